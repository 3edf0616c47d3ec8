"""Whole-model checks of the oracle (CPU only): the official manifest, an
independent float64 restatement on tiny shapes, and the reference's model
invariants (tests/checkpoint_fixtures.rs:202-353; cpu.rs:5368-5411)."""

import numpy as np
import pytest

import oracle as O
from conftest import ROOT  # noqa: F401
from ironicl_amd import manifest as mf
from ironicl_amd import synthetic as S
from reference_np import Model


def reference_lcg_data(b, n, q, h, classes=3):
    """Data of built_context_matches_the_uncached_forward_pass
    (tests/checkpoint_fixtures.rs:216-233): an LCG in [-2, 2), class shifts per estimator."""
    state = 0x2545F491
    x = np.empty(b * (n + q) * h, np.float32)
    for i in range(x.size):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        x[i] = np.float32((state >> 8) / float(1 << 24) * 4.0 - 2.0)
    x = x.reshape(b, n + q, h)
    shifts = np.array([[(c + e) % classes for c in range(classes)] for e in range(b)], np.uint64)
    y = np.array([[shifts[e][row % classes] for row in range(n)] for e in range(b)], np.float32)
    return x[:, :n].copy(), y, x[:, n:].copy(), shifts


@pytest.mark.parametrize("task", [mf.CLASSIFIER, mf.REGRESSOR])
def test_manifest_matches_official_profile(task):
    names = mf.tensor_manifest(task)
    count, params, nbytes = mf.PROFILE[task]
    assert len(names) == count
    total = sum(int(np.prod(s)) for s in names.values())
    assert total == params and 4 * total == nbytes
    w = S.random_weights(task)
    assert sorted(w) == sorted(names)
    assert all(w[k].shape == names[k] for k in names)


def test_random_weights_are_seeded_and_bounded(clf_weights):
    again = S.random_weights("classifier")
    assert all(np.array_equal(clf_weights[k], again[k]) for k in clf_weights)
    w = clf_weights["icl_predictor.tf_icl.blocks.3.linear1.weight"]
    assert np.abs(w).max() <= 1 / np.sqrt(512) + 1e-7
    assert np.allclose(clf_weights["row_interactor.tf_row.rope.freqs"], 100000.0 ** (-np.arange(8) / 8))


@pytest.mark.parametrize("task", [mf.CLASSIFIER, mf.REGRESSOR])
def test_oracle_matches_float64_restatement(task, clf_weights, reg_weights):
    weights = clf_weights if task == mf.CLASSIFIER else reg_weights
    rng = np.random.default_rng(11)
    n, q, h = 48, 5, 4
    x = rng.normal(size=(n + q, h)).astype(np.float32)
    y = (np.arange(n) % 3).astype(np.float32) if task == mf.CLASSIFIER else rng.normal(size=n).astype(np.float32)
    ref_cols, ref_rows, ref_logits = Model(task, weights).forward(x.astype(np.float64), y.astype(np.float64), n)
    m = O.OracleModel(task, weights, O.EXACT)
    cols, rows = m.trace_uncached(x[None], y[None], n)
    cols[0, :, :4] = 0.0
    np.testing.assert_allclose(cols[0], ref_cols, atol=2e-5, rtol=1e-4)
    np.testing.assert_allclose(rows[0], ref_rows, atol=2e-5, rtol=1e-4)
    logits = m.predict_uncached(x[None, :n], y[None], x[None, n:])
    np.testing.assert_allclose(logits[0], ref_logits[n:], atol=1e-5, rtol=1e-4)
    ctx = m.build_context(x[None, :n], y[None])
    np.testing.assert_allclose(m.predict_cached(ctx, x[None, n:])[0], ref_logits[n:], atol=1e-5, rtol=1e-4)


@pytest.fixture(scope="module")
def lcg_case(clf_weights):
    b, n, q, h = 2, 240, 250, 5
    x, y, xt, shifts = reference_lcg_data(b, n, q, h)
    m = O.OracleModel("classifier", clf_weights, O.EXACT)
    O.set_threads(4)
    ctx = m.build_context(x, y)
    return m, x, y, xt, ctx


def test_cached_matches_uncached(lcg_case):
    m, x, y, xt, ctx = lcg_case
    cached = m.predict_cached(ctx, xt)
    uncached = m.predict_uncached(x, y, xt)
    assert np.abs(cached - uncached).max() <= 1e-4
    assert np.array_equal(cached.argmax(-1), uncached.argmax(-1))


def test_context_layout_reserved_streams_are_zero(lcg_case):
    _, x, _, _, (ck, cv, ik, iv) = lcg_case
    b, n, h = x.shape
    assert ck[0].shape == (b, h + 4, 8, 128, 16) and ik[0].shape == (b, 8, n, 64)
    for t in ck + cv:
        assert not t[:, :4].any() and t[:, 4:].any()


def test_threads_do_not_change_results(lcg_case):
    m, _, _, xt, ctx = lcg_case
    O.set_threads(1)
    serial = m.predict_cached(ctx, xt)
    O.set_threads(4)
    parallel = m.predict_cached(ctx, xt)
    assert np.array_equal(serial, parallel)


def test_training_row_permutation_invariance(lcg_case):
    m, x, y, xt, ctx = lcg_case
    perm = np.random.default_rng(2).permutation(x.shape[1])
    ctx_p = m.build_context(np.ascontiguousarray(x[:, perm]), np.ascontiguousarray(y[:, perm]))
    np.testing.assert_allclose(m.predict_cached(ctx_p, xt[:, :40]), m.predict_cached(ctx, xt[:, :40]), atol=2e-5)


def test_rows_are_independent_and_chunks_join_in_place(lcg_case):
    """large_cached_query_runs_in_chunks (tests/checkpoint_fixtures.rs:297-353)."""
    m, _, _, xt, ctx = lcg_case
    big = np.concatenate([xt] * 5, axis=1)[:, :1100]
    whole = m.predict_cached(ctx, big)
    part = m.predict_cached(ctx, big[:, 1000:1100])
    np.testing.assert_array_equal(whole[:, 1000:1100], part)
    np.testing.assert_array_equal(whole[:, :250], whole[:, 250:500])


def test_native_math_within_tolerance_of_exact(clf_weights, lcg_case):
    _, x, y, xt, ctx = lcg_case
    native = O.OracleModel("classifier", clf_weights, O.NATIVE)
    exact = lcg_case[0].predict_cached(ctx, xt[:, :50])
    approx = native.predict_cached(ctx, xt[:, :50])
    assert np.all(np.abs(approx - exact) <= 1e-5 + 1e-4 * np.abs(exact))


def test_missing_marker_rows_run_on_the_cpu_path(clf_weights):
    m = O.OracleModel("classifier", clf_weights, O.EXACT)
    x, y, xt, _ = reference_lcg_data(1, 64, 4, 5)
    xt[0, 1, :] = -100.0
    out = m.predict_uncached(x, y, xt)
    assert np.all(np.isfinite(out))


def test_invalid_labels_are_rejected(clf_weights):
    m = O.OracleModel("classifier", clf_weights, O.EXACT)
    x, _, _, _ = reference_lcg_data(1, 64, 1, 5)
    with pytest.raises(ValueError):
        m.build_context(x, np.full((1, 64), 10.0, np.float32))


def test_missing_tensor_is_reported(clf_weights):
    w = dict(clf_weights)
    del w["icl_predictor.ln.weight"]
    with pytest.raises(ValueError, match="icl_predictor.ln.weight"):
        O.OracleModel("classifier", w)


def test_spot_checks_reproduce_the_build(lcg_case):
    """The full-size spot checks (column K/V of chosen features, ICL K/V of chosen
    training rows by teacher forcing) give the build's own tensors bitwise."""
    m, x, y, _, (ck, cv, ik, iv) = lcg_case
    feats, rows = [0, 3, 4], [0, 17, 239, 100]
    for e in range(x.shape[0]):
        kv = m.context_columns(x[e], y[e], feats)
        for blk in range(3):
            np.testing.assert_array_equal(kv[2 * blk], ck[blk][e, 4 + np.array(feats)])
            np.testing.assert_array_equal(kv[2 * blk + 1], cv[blk][e, 4 + np.array(feats)])
        keys, values = m.context_rows(x[e], y[e], rows, [c[e] for c in ck], [c[e] for c in cv],
                                      [t[e] for t in ik], [t[e] for t in iv])
        for blk in range(12):
            np.testing.assert_array_equal(keys[blk], ik[blk][e][:, rows])
            np.testing.assert_array_equal(values[blk], iv[blk][e][:, rows])


def test_spot_checks_see_a_wrong_block(lcg_case):
    """A value changed in one block of the context shows in the checked rows'
    K/V of the next block only (teacher forcing), and a changed column cache
    in every ICL block."""
    m, x, y, _, (ck, cv, ik, iv) = lcg_case
    rows = [5, 6]
    bad_iv = [t[0].copy() for t in iv]
    bad_iv[4] *= 1.01
    keys, _ = m.context_rows(x[0], y[0], rows, [c[0] for c in ck], [c[0] for c in cv], [t[0] for t in ik], bad_iv)
    for blk in range(12):
        same = np.array_equal(keys[blk], ik[blk][0][:, rows])
        assert same == (blk <= 4), blk
    bad_cv = [c[0].copy() for c in cv]
    bad_cv[2][4 + 1] *= 1.01
    keys, _ = m.context_rows(x[0], y[0], rows, [c[0] for c in ck], bad_cv, [t[0] for t in ik], [t[0] for t in iv])
    assert not np.array_equal(keys[0], ik[0][0][:, rows])


def test_float64_spot_checks_match_the_oracle_build(lcg_case, clf_weights):
    """The float64 restatement's spot checks (column K/V of a feature, a
    training row's ICL K/V by teacher forcing) agree with the oracle's build."""
    from reference_np import Model

    _, x, y, _, (ck, cv, ik, iv) = lcg_case
    m = Model("classifier", clf_weights)
    for blk, (k, v) in enumerate(m.column_kv(x[1], y[1], 2)):
        np.testing.assert_allclose(k, ck[blk][1, 6], atol=2e-5, rtol=1e-4)
        np.testing.assert_allclose(v, cv[blk][1, 6], atol=2e-5, rtol=1e-4)
    keys, values = m.row_kv(x[1, 33], y[1, 33], [c[1] for c in ck], [c[1] for c in cv], [t[1] for t in ik],
                            [t[1] for t in iv])
    for blk in range(12):
        np.testing.assert_allclose(keys[blk], ik[blk][1][:, 33], atol=2e-5, rtol=1e-4)
        np.testing.assert_allclose(values[blk], iv[blk][1][:, 33], atol=2e-5, rtol=1e-4)


def test_float64_cached_prediction_matches_the_oracle(clf_weights):
    """reference_np's cached prediction (the float64 arbiter of the full-size
    logit checks) against the oracle's, on an oracle-built context."""
    rng = np.random.default_rng(12)
    n, q, h = 64, 6, 5
    x = rng.normal(size=(n + q, h)).astype(np.float32)
    y = (np.arange(n) % 3).astype(np.float32)
    m = O.OracleModel("classifier", clf_weights, O.EXACT)
    ck, cv, ik, iv = m.build_context(x[None, :n], y[None])
    want = m.predict_cached((ck, cv, ik, iv), x[None, n:])[0]
    got = Model("classifier", clf_weights).cached_logits(x[n:].astype(np.float64), [c[0] for c in ck],
                                                        [c[0] for c in cv], [t[0] for t in ik], [t[0] for t in iv])
    np.testing.assert_allclose(got, want, atol=1e-5, rtol=1e-4)
