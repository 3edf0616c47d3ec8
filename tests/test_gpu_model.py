"""Whole-model parity of the GPU path against the oracle, through the C ABI.

The parity bar: every logit / regression output within
|gpu - cpu| <= 1e-5 + 1e-4 |cpu| of the oracle's FP32 CPU path on identical
inputs and weights, with identical argmax."""

import numpy as np
import pytest

import oracle as O
from ironicl_amd import hip, hipmem
from ironicl_amd import synthetic as S
from ironicl_amd import tabicl
from test_oracle_model import reference_lcg_data

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-5, 1e-4


def assert_parity(gpu, cpu, what=""):
    gpu, cpu = np.asarray(gpu, np.float64), np.asarray(cpu, np.float64)
    err = np.abs(gpu - cpu) - (ATOL + RTOL * np.abs(cpu))
    worst = np.unravel_index(np.argmax(err), err.shape)
    assert err.max() <= 0, f"{what}: |gpu-cpu| {abs(gpu[worst] - cpu[worst]):.3e} at {worst} (cpu {cpu[worst]:.6f})"


@pytest.fixture(scope="module")
def device():
    return hip.Device(0)


@pytest.fixture(scope="module")
def clf(device, clf_weights):
    return tabicl.Executor("classifier", clf_weights, device)


@pytest.fixture(scope="module")
def clf_oracle(clf_weights):
    O.set_threads(16)
    return O.OracleModel("classifier", clf_weights, O.EXACT)


@pytest.fixture(scope="module")
def lcg(clf, clf_oracle):
    x, y, xt, shifts = reference_lcg_data(2, 240, 250, 5)
    ctx_cpu = clf_oracle.build_context(x, y)
    ctx_gpu = clf.build_context(x, y, class_permutations=shifts, download=True)
    return x, y, xt, shifts, ctx_cpu, ctx_gpu


def test_built_context_matches_oracle(lcg):
    x, y, xt, shifts, ctx_cpu, ctx_gpu = lcg
    ck, cv, ik, iv = ctx_gpu.context
    for blk in range(3):
        np.testing.assert_allclose(ck[blk][:, 4:], ctx_cpu[0][blk][:, 4:], atol=1e-4, rtol=1e-3)
        np.testing.assert_allclose(cv[blk][:, 4:], ctx_cpu[1][blk][:, 4:], atol=1e-4, rtol=1e-3)
    for blk in range(12):
        np.testing.assert_allclose(ik[blk], ctx_cpu[2][blk], atol=2e-4, rtol=1e-3, err_msg=f"icl {blk} keys")
        np.testing.assert_allclose(iv[blk], ctx_cpu[3][blk], atol=2e-4, rtol=1e-3, err_msg=f"icl {blk} values")


def test_cached_prediction_on_the_oracle_context(clf, clf_oracle, lcg):
    """The predictor alone: the oracle's context uploaded, GPU vs CPU predict."""
    x, y, xt, shifts, ctx_cpu, _ = lcg
    st = clf.load_context_tensors(ctx_cpu, x.shape, 3, shifts)
    gpu = st.predict_raw(xt).logits
    cpu = clf_oracle.predict_cached(ctx_cpu, xt)
    assert_parity(gpu, cpu, "predict on the oracle context")
    assert np.array_equal(gpu[..., :3].argmax(-1), cpu[..., :3].argmax(-1))


def test_built_context_prediction_matches_uncached_oracle(clf_oracle, lcg):
    """Build and predict on the GPU against the oracle's uncached forward."""
    x, y, xt, shifts, _, ctx_gpu = lcg
    gpu = ctx_gpu.predict_raw(xt).logits
    cpu = clf_oracle.predict_uncached(x, y, xt)
    assert_parity(gpu, cpu, "build + predict")
    assert np.array_equal(gpu[..., :3].argmax(-1), cpu[..., :3].argmax(-1))
    probs = ctx_gpu.predict_probabilities(xt)
    ref = O.aggregate(np.ascontiguousarray(cpu[..., :3]), shifts)
    np.testing.assert_allclose(probs, ref, atol=1e-5)


def test_pass_rows_and_device_path_do_not_change_results(lcg):
    *_, ctx_gpu = lcg
    xt = lcg[2]
    whole = ctx_gpu.predict_raw(xt).logits
    ctx_gpu.set_pass_rows(32)
    try:
        small = ctx_gpu.predict_raw(xt).logits
    finally:
        ctx_gpu.set_pass_rows(512)
    np.testing.assert_allclose(small, whole, atol=1e-6, rtol=1e-6)
    dx = hipmem.DeviceArray.from_host(xt)
    dl = hipmem.DeviceArray.from_host(np.zeros((2, xt.shape[1], 10), np.float32))
    hip.check(hip.lib().irx_predictor_predict_device(ctx_gpu.handle, dx.ptr, xt.shape[1], dl.ptr, None))
    np.testing.assert_array_equal(dl.to_host(), whole)


@pytest.mark.parametrize("rows", [1, 2, 4, 5, 8])
def test_passes_of_few_rows_match_the_oracle(clf, clf_oracle, lcg, rows):
    """Calls of 1-8 test rows over two estimators: passes of at most eight
    (estimator, row) pairs take the small-row products and LayerNorm + linear
    kernels, sixteen pairs the split-K products and 16-row MFMA tiles, and all
    of them the 16-row block tails. Checked against the oracle on its own
    context and against the 512-row passes."""
    x, y, xt, shifts, ctx_cpu, ctx_gpu = lcg
    few = np.ascontiguousarray(xt[:, :rows])
    st = clf.load_context_tensors(ctx_cpu, x.shape, 3, shifts)
    gpu = st.predict_raw(few).logits
    cpu = clf_oracle.predict_cached(ctx_cpu, few)
    assert_parity(gpu, cpu, f"{rows} rows on the oracle context")
    assert np.array_equal(gpu[..., :3].argmax(-1), cpu[..., :3].argmax(-1))
    whole = ctx_gpu.predict_raw(xt).logits
    np.testing.assert_allclose(ctx_gpu.predict_raw(few).logits, whole[:, :rows], atol=1e-6, rtol=1e-6)


def test_stream_counts_give_identical_results(lcg):
    *_, ctx_gpu = lcg
    xt = lcg[2]
    ctx_gpu.set_pass_rows(32)  # 250 rows: 8 passes rotating over the streams
    try:
        by_streams = {}
        for streams in (2, 1, 3, 4):
            ctx_gpu.set_streams(streams)
            by_streams[streams] = ctx_gpu.predict_raw(xt).logits
    finally:
        ctx_gpu.set_streams(2)
        ctx_gpu.set_pass_rows(512)
    for streams in (2, 3, 4):
        np.testing.assert_array_equal(by_streams[streams], by_streams[1])
    for bad in (0, 5):
        with pytest.raises(hip.HipError):
            ctx_gpu.set_streams(bad)


def test_graph_replays_match_launched_passes(lcg):
    """Passes replayed from HIP graphs give the logits of passes launched
    kernel by kernel, bitwise, with new rows on every replay (three inputs,
    twice round), at 512-, 64- and 32-row passes with a ragged last pass, on
    one and two streams."""
    *_, ctx = lcg
    xt = lcg[2]
    inputs = [np.ascontiguousarray(xt[:, a:a + 200]) for a in (0, 50, 25)]
    default = ctx.pass_rows()
    try:
        for rows in (512, 64, 32):
            ctx.set_pass_rows(rows)
            for streams in (1, 2):
                ctx.set_streams(streams)
                ctx.set_graphs(False)
                eager = [ctx.predict_raw(x).logits for x in inputs]
                ctx.set_graphs(True)
                for _ in range(2):
                    for x, want in zip(inputs, eager):
                        np.testing.assert_array_equal(ctx.predict_raw(x).logits, want)
    finally:
        ctx.set_graphs(True)
        ctx.set_streams(2)
        ctx.set_pass_rows(default)


def test_many_ragged_lengths_replay_safely(clf, lcg):
    """Serving calls of many lengths on two streams: a pass of more than 32
    rows computes a multiple of 32 rows, so the predictor keeps one graph per
    (stream, shape): 32 shapes up to 32 rows, then one per 32 rows. With
    3,072-row passes that is 2 x 127 shapes, past the 192 it keeps, so graphs
    are evicted while earlier passes of the same call may still run them.
    Every call matches kernel-by-kernel launches bitwise."""
    x, _, _, shifts, ctx_cpu, _ = lcg
    st = clf.load_context_tensors(ctx_cpu, x.shape, 3, shifts)
    rng = np.random.default_rng(5)
    xt = rng.uniform(-2, 2, size=(2, 2 * 3072, 5)).astype(np.float32)
    tails = list(range(1, 33)) + [32 * t - 5 for t in range(2, 97)]
    lengths = tails + [3072 + t for t in tails]
    st.set_pass_rows(3072)
    st.set_graphs(False)
    eager = {q: st.predict_raw(np.ascontiguousarray(xt[:, :q])).logits for q in lengths}
    st.set_graphs(True)
    for q in lengths + lengths[::-1]:
        np.testing.assert_array_equal(st.predict_raw(np.ascontiguousarray(xt[:, :q])).logits, eager[q],
                                      err_msg=f"{q} rows")


def test_predictor_fits_its_workspace_to_the_budget(clf, lcg, device):
    """A device limit with room for the caches and one stream's workspace at
    128-row passes, but not at 256, gives one stream of 128-row passes
    (Predictor::predict halves its run rows when memory runs out,
    predictor.rs:248-258) with the unconstrained predictor's results; without
    room for one 32-row pass the context does not fit (the CPU path's case)."""
    import ctypes

    x, _, xt, shifts, _, ctx_gpu = lcg
    b, n, h = x.shape
    shape = hip.Shape(b, h, n, clf.width)
    ws = lambda rows: hip.lib().irx_predict_workspace_bytes(device.handle, ctypes.byref(shape), hip.PRECISION_FP32,
                                                             rows)
    assert 0 < ws(32) < ws(128) < ws(256) < ws(512)
    cache = sum(t.nbytes for part in ctx_gpu.context for t in part)
    weights = hip.lib().irx_weights_bytes(clf.handle)
    budget = (cache + ws(128)) * 10 // 9 + 20
    assert budget // 10 * 9 < cache + ws(256)
    small = clf.load_context_tensors(ctx_gpu.context, (b, n, h), 3, shifts, device_limit=weights + budget)
    assert small.pass_rows() == 128
    full = clf.load_context_tensors(ctx_gpu.context, (b, n, h), 3, shifts)
    assert full.pass_rows() == 512
    assert_parity(small.predict_logits(xt).logits, full.predict_logits(xt).logits, "128-row passes")
    with pytest.raises(hip.HipError) as e:
        clf.load_context_tensors(ctx_gpu.context, (b, n, h), 3, shifts, device_limit=weights + cache + ws(32) // 2)
    assert e.value.status == hip.DOES_NOT_FIT


def test_kernel_timing_records_launches(lcg):
    *_, ctx_gpu = lcg
    hip.profile_enable(True)
    try:
        ctx_gpu.predict_raw(lcg[2])
        icl = hip.profile_read("icl_attention")
        gemm = hip.profile_read("gemm")
    finally:
        hip.profile_enable(False)
    assert icl["launches"] == 12 and icl["milliseconds"] > 0
    assert 0 < icl["busy_milliseconds"] <= icl["milliseconds"] * (1 + 1e-6)
    # 250 rows run as one pass of 256 (passes over 32 rows compute multiples of 32).
    assert icl["flops"] == pytest.approx(12 * 4.0 * 16 * 256 * 240 * 64)
    assert gemm["launches"] > 50 and gemm["flops"] > 0
    with pytest.raises(hip.HipError):
        hip.profile_read("nonsense")


def test_missing_marker_rows_are_flagged(lcg):
    *_, ctx_gpu = lcg
    xt = lcg[2][:, :40].copy()
    xt[1, 7, :] = -100.0   # every grouped triple of row 7 in estimator 1
    p = ctx_gpu.predict_raw(xt)
    assert p.cpu_rows == [7]
    assert np.all(np.isnan(p.logits[:, 7])) and np.all(np.isfinite(np.delete(p.logits, 7, axis=1)))
    # Probabilities of such a row would be NaN: refused, not returned.
    with pytest.raises(ValueError, match="all-missing marker"):
        ctx_gpu.predict_probabilities(xt)
    # Over several passes on two streams, in both estimators, and again after
    # a call without marked rows (the flags start from zero on every call).
    xt = lcg[2][:, :200].copy()
    xt[0, 3, :] = -100.0
    xt[1, 150, :] = -100.0
    xt[0, 199, :] = -100.0
    default = ctx_gpu.pass_rows()
    ctx_gpu.set_pass_rows(64)
    try:
        assert ctx_gpu.predict_raw(lcg[2][:, :200]).cpu_rows == []
        assert ctx_gpu.predict_raw(xt).cpu_rows == [3, 150, 199]
        assert ctx_gpu.predict_raw(lcg[2][:, :200]).cpu_rows == []
    finally:
        ctx_gpu.set_pass_rows(default)


def test_config_clf_1k_end_to_end(clf, clf_oracle):
    """1024 train rows x 54 features, 7 classes, 8 test rows."""
    w = S.WORKLOADS["clf-1k"]
    x, y, xt, meta = S.workload_data(w)
    st = clf.build_context(x, y)
    gpu = st.predict_logits(xt).logits
    cpu = clf_oracle.predict_uncached(x, y, xt)[..., :7]
    assert_parity(gpu, cpu, "clf-1k")
    assert np.array_equal(gpu.argmax(-1), cpu.argmax(-1))


def test_regressor_quantiles(device, reg_weights):
    w = S.WORKLOADS["reg-20k"]
    x, y, xt, meta = S.workload_data(w, train_rows=300, test_rows=40, features=7)
    ex = tabicl.Executor("regressor", reg_weights, device)
    st = ex.build_context(x, y)
    gpu = st.predict_logits(xt).logits
    m = O.OracleModel("regressor", reg_weights, O.EXACT)
    cpu = m.predict_uncached(x, y, xt)
    assert_parity(gpu, cpu, "regressor quantiles")
    alphas = [0.05, 0.5, 0.95]
    gm, gq = st.predict_regression(xt, alphas)
    cm, cq = O.regression_summary(cpu, alphas)
    assert_parity(gm, cm, "mean")
    assert_parity(gq, cq, "quantiles")
    # Summaries of the same decoded outputs: the GPU's are the oracle's to the bit.
    names = ("mean", "variance", "median", "quantiles", "raw_quantiles")
    got = st.predict_regression_outputs(xt, names, alphas)
    om, ov, oq, oraw = O.regression_outputs(gpu, list(alphas) + [0.5])
    for g, want in zip(got, (om, ov, oq[:, -1], oq[:, :3], oraw)):
        np.testing.assert_array_equal(g, want)


@pytest.mark.parametrize("task", ["classifier", "regressor"])
def test_device_label_embeddings_equal_the_host_ones(device, clf_weights, reg_weights, task):
    """Builds from targets (the device embeds them through its y_encoder
    weights) and from host-computed embeddings (the reference's BuildInputs)
    give the same context and logits, bit for bit: an 8-estimator classifier
    with class shifts and a regressor with real-valued targets."""
    weights = clf_weights if task == "classifier" else reg_weights
    ex = tabicl.Executor(task, weights, device)
    w = S.WORKLOADS["clf-200k" if task == "classifier" else "reg-20k"]
    x, y, xt, meta = S.workload_data(w, train_rows=700, test_rows=20, features=11)
    perms = meta.get("class_permutations")
    out = []
    for device_labels in (True, False):
        ex.device_labels = device_labels
        st = ex.build_context(x, y, class_permutations=perms, download=True)
        out.append((st.context, st.predict_logits(xt).logits))
    (ctx_d, lg_d), (ctx_h, lg_h) = out
    for part_d, part_h in zip(ctx_d, ctx_h):
        for a, b in zip(part_d, part_h):
            np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(lg_d, lg_h)


def test_ensemble_with_feature_permutations(clf, clf_oracle):
    w = S.WORKLOADS["clf-200k"]
    x, y, xt, meta = S.workload_data(w, train_rows=200, test_rows=30, features=9)
    x, y, xt = x[:3], y[:3], xt[:3]
    st = clf.build_context(x, y, class_permutations=meta["class_permutations"][:3])
    gpu = st.predict_logits(xt).logits
    cpu = clf_oracle.predict_uncached(x, y, xt)[..., :10]
    assert_parity(gpu, cpu, "3 estimators")


@pytest.mark.parametrize("features", [1, 2, 3])
def test_contexts_of_one_to_three_features(clf, clf_oracle, features):
    """Feature counts where the column inputs' (f + 1, f + 2, f + 4) mod H
    neighbours repeat or are the feature itself, and the row transformer sees
    5-7 tokens (cpu.rs:818-823 accepts any H >= 1): build and predict on the
    GPU against the oracle's uncached forward."""
    x, y, xt, shifts = reference_lcg_data(1, 128, 6, features)
    ctx = clf.build_context(x, y, class_permutations=shifts)
    gpu = ctx.predict_raw(xt).logits
    cpu = clf_oracle.predict_uncached(x, y, xt)
    assert_parity(gpu, cpu, f"{features} features")
    assert np.array_equal(gpu[..., :3].argmax(-1), cpu[..., :3].argmax(-1))


def test_rows_longer_than_the_staged_attention_takes(clf, clf_oracle):
    """600 features: the row transformer's sequences are 604 tokens, past the
    512 keys of the staged row attention, so its self-attention takes the
    long-range kernel with RoPE (four waves per 128-query chunk, key ranges
    merged), and the CLS block's four queries read 604 tokens."""
    x, y, xt, shifts = reference_lcg_data(1, 96, 5, 600)
    ctx = clf.build_context(x, y, class_permutations=shifts)
    gpu = ctx.predict_raw(xt).logits
    cpu = clf_oracle.predict_uncached(x, y, xt)
    assert_parity(gpu, cpu, "600 features")
    assert np.array_equal(gpu[..., :3].argmax(-1), cpu[..., :3].argmax(-1))


@pytest.mark.parametrize("classes", [2, 10])
def test_two_and_ten_classes(clf, clf_oracle, classes):
    """The fewest and the most classes the classifier takes (label
    embeddings, logits over `classes` of the 10 outputs, probability
    aggregation with per-estimator class shifts), two estimators: build and
    predict on the GPU against the oracle's uncached forward."""
    x, y, xt, shifts = reference_lcg_data(2, 160, 12, 6, classes=classes)
    ctx = clf.build_context(x, y, class_permutations=shifts)
    gpu = ctx.predict_raw(xt).logits
    cpu = clf_oracle.predict_uncached(x, y, xt)
    assert_parity(gpu, cpu, f"{classes} classes")
    assert np.array_equal(gpu[..., :classes].argmax(-1), cpu[..., :classes].argmax(-1))
    probs = ctx.predict_probabilities(xt)
    ref = O.aggregate(np.ascontiguousarray(cpu[..., :classes]), shifts)
    np.testing.assert_allclose(probs, ref, atol=1e-5)


def test_progress_hook_can_interrupt(clf):
    x, y, xt, _ = reference_lcg_data(2, 128, 8, 5)
    calls = []

    def hook(stage, done, total):
        calls.append((stage, done, total))
        if done == 1:
            raise RuntimeError("stop")

    with pytest.raises(hip.HipError) as e:
        clf.build_context(x, y, progress=hook)
    assert e.value.status == hip.INTERRUPTED
    assert calls[0] == (hip.STAGE_BUILD, 0, 2)


def test_build_rejects_missing_marker_and_tiny_contexts(clf):
    x, y, _, _ = reference_lcg_data(1, 128, 1, 5)
    x[0, 3, :] = -100.0
    with pytest.raises(hip.HipError) as e:
        clf.build_context(x, y)
    assert e.value.status == hip.UNSUPPORTED
    x, y, _, _ = reference_lcg_data(1, 32, 1, 5)
    with pytest.raises(hip.HipError) as e:
        clf.build_context(x, y)
    assert e.value.status == hip.DOES_NOT_FIT


def test_builds_reuse_the_devices_kept_workspace(clf, lcg):
    """A device keeps its last build's workspace for the next build. A context
    rebuilt after a larger build in between (whose data the kept workspace
    then holds) is bitwise the first one: no stage reads workspace memory it
    has not written."""
    x, y, xt, shifts, _, ctx_gpu = lcg
    first = ctx_gpu.predict_raw(xt).logits
    rng = np.random.default_rng(5)
    xb = rng.normal(size=(1, 700, 9)).astype(np.float32)
    yb = (np.arange(700) % 4).astype(np.float32)[None]
    big = clf.build_context(xb, yb)
    assert np.isfinite(big.predict_raw(xb[:, :16]).logits).all()
    del big
    again = clf.build_context(x, y, class_permutations=shifts, download=True)
    np.testing.assert_array_equal(again.predict_raw(xt).logits, first)
    for blk in range(12):
        np.testing.assert_array_equal(again.context[2][blk], ctx_gpu.context[2][blk])


@pytest.mark.parametrize("bad", [3.5, -1.0, 10.0, float("nan"), float("inf")])
def test_build_rejects_bad_classifier_targets_at_the_abi(clf, bad):
    """Targets handed straight to irx_build (past the Python checks) are
    checked as the reference checks labels (cpu.rs:4717-4740)."""
    rng = np.random.default_rng(2)
    x = rng.normal(size=(1, 80, 6)).astype(np.float32)
    y = (np.arange(80) % 3).astype(np.float32)[None]
    meta, xf, yf = clf._unhashed_metadata(x, y, None, None)
    y_bad = yf.copy()
    y_bad[0, 17] = bad
    with pytest.raises(hip.HipError) as e:
        clf._build(xf, y_bad, meta, False, None, 0)
    assert e.value.status == hip.INVALID_ARGUMENT


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), -float("inf")])
def test_build_rejects_non_finite_regression_targets_at_the_abi(device, reg_weights, bad):
    reg = tabicl.Executor("regressor", reg_weights, device)
    rng = np.random.default_rng(3)
    x = rng.normal(size=(1, 80, 6)).astype(np.float32)
    y = rng.normal(size=(1, 80)).astype(np.float32)
    meta, xf, yf = reg._unhashed_metadata(x, y, None, None)
    y_bad = yf.copy()
    y_bad[0, 5] = bad
    with pytest.raises(hip.HipError) as e:
        reg._build(xf, y_bad, meta, False, None, 0)
    assert e.value.status == hip.INVALID_ARGUMENT
