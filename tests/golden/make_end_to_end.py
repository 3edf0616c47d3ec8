"""Writes tests/golden/end_to_end.npz: the oracle's uncached forward
(Executor::predict_logits_inner, cpu.rs:997-1065, exact math) on two
10,000-row contexts that the oracle cannot rerun inside a GPU test (each takes
minutes of serial ICL attention on the host):

  clf10k   the 10,000-row, 100-feature classifier workload (20% log-normal
           columns, MLP labeller) at the random-init weights: logits of all
           1,024 test rows [1024, 10];
  cond10k  10,000 training rows x 20 features N(0, 1), 10 classes, 64 test
           rows, at the conditioned weights of tests/conditioned.py (sharpened
           attention): logits [64, 10].

Each entry keeps a SHA-256 of its inputs (weights, x, y, test rows) so the GPU
test can check that it regenerated the same ones. Run from the repository
root after building the oracle:

    python tests/golden/make_end_to_end.py [--stats]

--stats also prints the conditioned weights' attention statistics on the
1,024-row, 54-feature workload.
"""

from __future__ import annotations

import hashlib
import os
import sys
import time

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

import conditioned as C  # noqa: E402
import oracle as O  # noqa: E402
from ironicl_amd import synthetic as S  # noqa: E402
from ironicl_amd import tabicl  # noqa: E402

OUT = os.path.join(HERE, "end_to_end.npz")
COND_10K = S.Workload("cond-10k", "classifier", 1, 10_000, 20, 64, 10, 6)


def inputs_digest(weights, x, y, xt) -> str:
    h = hashlib.sha256(tabicl.weights_sha256("classifier", weights).encode())
    for a in (x, y, xt):
        h.update(np.ascontiguousarray(a, np.float32).tobytes())
    return h.hexdigest()


def cases():
    """(name, weights, x, y, xt) of each fixture, as the GPU test rebuilds them."""
    w = S.random_weights("classifier")
    x, y, xt, _ = S.workload_data(S.WORKLOADS["clf-10k"])
    yield "clf10k", w, x, y, xt
    x, y, xt, _ = S.workload_data(COND_10K)
    yield "cond10k", C.conditioned_weights(w), x, y, xt


def main() -> None:
    O.set_threads(os.cpu_count() or 8)
    out = {}
    for name, w, x, y, xt in cases():
        t = time.time()
        logits = O.OracleModel("classifier", w, O.EXACT).predict_uncached(x, y, xt)[0, :, :10]
        out[f"{name}_logits"] = np.ascontiguousarray(logits, np.float32)
        out[f"{name}_inputs_sha256"] = np.array(inputs_digest(w, x, y, xt))
        print(f"{name}: {logits.shape} in {time.time() - t:.0f} s", flush=True)
    np.savez(OUT, **out)
    print(f"wrote {OUT}")
    if "--stats" in sys.argv:
        w = S.random_weights("classifier")
        x, y, xt, _ = S.workload_data(S.WORKLOADS["clf-1k"])
        for label, weights in (("random-init", w), ("conditioned", C.conditioned_weights(w))):
            stats = C.attention_stats("classifier", weights, x[0], y[0], xt[0])
            print(label, {k: (round(a, 3), round(b, 3)) for k, (a, b) in stats.items()})


if __name__ == "__main__":
    main()
