"""Spot checks of a full-size GPU context against the oracle (test
infrastructure only; used by tests/test_gpu_full_size.py and bench.py's
--workload parity leg).

The oracle cannot rebuild contexts of 10,000 rows and more inside a test, so
each checked estimator of a GPU-built context gets:

- the column K/V of sampled features, from the oracle's full N-row column
  stream of each feature (ora_context_columns, pinned bitwise against
  ora_build_context in test_oracle_model.py);
- the ICL K/V of sampled training rows at all twelve blocks, each block's from
  the GPU context's earlier blocks (teacher forcing, ora_context_rows), so no
  error compounds;
- the logits of sampled test rows, the oracle's cached prediction against the
  GPU-built context.

Each to |gpu - cpu| <= 1e-5 + 1e-4 |cpu|, with identical argmax for a
classifier's logits. Where a check misses that bar, the float64 restatement
(tests/reference_np.py) decides: at 200,000 training rows the reference's
FP32 CPU path itself strays from exact arithmetic by more than the bar (each
attention accumulates its output, and in exact math its softmax denominator,
over the 200,000 keys one key at a time, cpu.rs:963-969). For K/V, on the
first sampled feature and rows, the GPU's error against float64 must not
exceed the oracle's own. For logits, on every sampled test row, the GPU must
meet the strict bar against float64 itself and be no further from it than
the oracle; the argmax must still equal the oracle's.
"""

from __future__ import annotations

import json
import os
import time

import numpy as np


def spot_checks(task, weights, width, ctx, x, y, xt, logits, features=4, train_rows=16, test_rows=32,
                float64_rows=4, members=None, log=print, tests=None, more_logits=None) -> dict:
    """Report of the checks on estimators `members` (default 0 and B-1) of the
    GPU context `ctx` (a StaticExecutor) built from x [B,N,H], y [B,N], with
    GPU logits [B,Q,>=width] of xt [B,Q,H]; report["ok"] is the outcome.
    `tests` fixes the sampled test rows; `more_logits` maps a name to other
    GPU logits [B, len(tests), >=width] of those rows (another pass size), each
    checked like `logits` against the same oracle rows."""
    import oracle as O
    from reference_np import Model

    threads = min(16, os.cpu_count() or 1)
    O.set_threads(threads)
    oracle = O.OracleModel(task, weights, O.EXACT)
    exact = Model(task, weights)
    b, n, h = x.shape
    q = xt.shape[1]
    rng = np.random.default_rng(7)
    feats = np.sort(rng.choice(h, min(h, features), replace=False))
    rows = np.sort(rng.choice(n, min(n, train_rows), replace=False))
    tests = np.sort(rng.choice(q, min(q, test_rows), replace=False)) if tests is None else np.asarray(tests)
    f64_rows = rows[:float64_rows]

    def excess(gpu, cpu):
        gpu, cpu = np.asarray(gpu, np.float64), np.asarray(cpu, np.float64)
        return float((np.abs(gpu - cpu) - (1e-5 + 1e-4 * np.abs(cpu))).max()), float(np.abs(gpu - cpu).max())

    report = {k: {"max_abs_diff_vs_oracle": 0.0, "strict_ok": True} for k in ("column_kv", "icl_kv", "logits")}
    for k in ("column_kv", "icl_kv", "logits"):
        report[k]["float64"] = {"gpu_max_abs_err": 0.0, "oracle_max_abs_err": 0.0}
    report["logits"]["float64"]["gpu_strict_vs_float64"] = True

    def note(kind, got, want):
        ex, d = excess(got, want)
        r = report[kind]
        r["strict_ok"] &= ex <= 0
        r["max_abs_diff_vs_oracle"] = max(r["max_abs_diff_vs_oracle"], d)

    def note64(kind, gpu, cpu, ref):
        r = report[kind]["float64"]
        r["gpu_max_abs_err"] = max(r["gpu_max_abs_err"], float(np.abs(np.asarray(gpu, np.float64) - ref).max()))
        r["oracle_max_abs_err"] = max(r["oracle_max_abs_err"], float(np.abs(np.asarray(cpu, np.float64) - ref).max()))

    members = sorted({0, b - 1}) if members is None else list(members)
    argmax_ok = True
    for e in members:
        t0 = time.perf_counter()
        ck, cv, ik, iv = ctx.estimator_tensors(e)
        log(f"estimator {e}: context read from HBM in {time.perf_counter() - t0:.1f} s")
        t0 = time.perf_counter()
        kv = oracle.context_columns(x[e], y[e], feats)
        for blk in range(3):
            note("column_kv", ck[blk][4 + feats], kv[2 * blk])
            note("column_kv", cv[blk][4 + feats], kv[2 * blk + 1])
        keys, values = oracle.context_rows(x[e], y[e], rows, ck, cv, ik, iv)
        for blk in range(12):
            note("icl_kv", ik[blk][:, rows], keys[blk])
            note("icl_kv", iv[blk][:, rows], values[blk])
        cpu = oracle.predict_cached(([c[None] for c in ck], [c[None] for c in cv], [t[None] for t in ik],
                                     [t[None] for t in iv]), np.ascontiguousarray(xt[e:e + 1, tests]))[..., :width]
        gpu = logits[e:e + 1, tests, :width]
        note("logits", gpu, cpu)
        if task == "classifier":
            argmax_ok &= bool(np.array_equal(gpu.argmax(-1), cpu.argmax(-1)))
        for name, other in (more_logits or {}).items():
            got = other[e:e + 1, :, :width]
            ex_o, d_o = excess(got, cpu)
            r = report.setdefault(f"logits_{name}", {"max_abs_diff_vs_oracle": 0.0, "strict_ok": True})
            r["strict_ok"] &= ex_o <= 0
            r["max_abs_diff_vs_oracle"] = max(r["max_abs_diff_vs_oracle"], d_o)
            if task == "classifier":
                r["argmax_identical"] = r.get("argmax_identical", True) and bool(
                    np.array_equal(got.argmax(-1), cpu.argmax(-1)))
        log(f"estimator {e}: oracle checks in {time.perf_counter() - t0:.1f} s")
        if excess(gpu, cpu)[0] > 0:
            t0 = time.perf_counter()
            ref = exact.cached_logits(xt[e, tests].astype(np.float64), ck, cv, ik, iv)[None, :, :width]
            note64("logits", gpu, cpu, ref)
            report["logits"]["float64"]["gpu_strict_vs_float64"] &= excess(gpu, ref)[0] <= 0
            log(f"estimator {e}: float64 logits in {time.perf_counter() - t0:.1f} s")
        if not (report["column_kv"]["strict_ok"] and report["icl_kv"]["strict_ok"]):
            t0 = time.perf_counter()
            for blk, (k64, v64) in enumerate(exact.column_kv(x[e].astype(np.float64), y[e], int(feats[0]))):
                note64("column_kv", ck[blk][4 + feats[0]], kv[2 * blk][0], k64)
                note64("column_kv", cv[blk][4 + feats[0]], kv[2 * blk + 1][0], v64)
            ik64 = [a.astype(np.float64) for a in ik]
            iv64 = [a.astype(np.float64) for a in iv]
            for j, r in enumerate(f64_rows):
                k64, v64 = exact.row_kv(x[e, r].astype(np.float64), y[e, r], ck, cv, ik64, iv64)
                for blk in range(12):
                    note64("icl_kv", ik[blk][:, r], keys[blk][:, j], k64[blk])
                    note64("icl_kv", iv[blk][:, r], values[blk][:, j], v64[blk])
            del ik64, iv64
            log(f"estimator {e}: float64 checks in {time.perf_counter() - t0:.1f} s")
        del ck, cv, ik, iv
        log(f"estimator {e}: {json.dumps(report)}")
    ok = argmax_ok
    for k in ("column_kv", "icl_kv", "logits"):
        f = report[k]["float64"]
        report[k]["ok"] = report[k]["strict_ok"] or (f["gpu_max_abs_err"] <= f["oracle_max_abs_err"] and
                                                     f.get("gpu_strict_vs_float64", True))
        ok &= report[k]["ok"]
    report["logits"]["argmax_identical"] = argmax_ok
    report.update({"estimators": members, "features": feats.tolist(), "train_rows": rows.tolist(),
                   "float64_features": [int(feats[0])], "float64_train_rows": f64_rows.tolist(),
                   "test_rows": tests.tolist(), "oracle_threads": threads, "ok": bool(ok)})
    return report
