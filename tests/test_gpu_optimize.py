"""optimize="auto" on the GPU: an FP16 ICL cache read by split-FP16 attention
products. Its accuracy gate is the reference's for reduced-precision levels
(docs/experiments.md:406-423): against the "safe" (FP32) output on the same
context, at most 1e-2 absolute logit error, and labels flip only on
near-ties. The FP16 cache is checked against the FP32 one bitwise where the
two builds still agree (the first block's keys and values)."""

import numpy as np
import pytest

import oracle as O
from ironicl_amd import context_file as cf
from ironicl_amd import hip, tabicl
from test_oracle_model import reference_lcg_data

pytestmark = pytest.mark.gpu

AUTO_LOGIT_TOL = 1e-2


@pytest.fixture(scope="module")
def clf(clf_weights):
    return tabicl.Executor("classifier", clf_weights, hip.Device(0))


@pytest.fixture(scope="module")
def lcg(clf):
    x, y, xt, shifts = reference_lcg_data(2, 240, 250, 5)
    safe = clf.build_context(x, y, class_permutations=shifts, download=True)
    auto = clf.build_context(x, y, class_permutations=shifts, download=True, optimize="auto")
    return x, y, xt, shifts, safe, auto


def gate(auto, safe, what):
    err = np.abs(auto - safe)
    assert err.max() <= AUTO_LOGIT_TOL, f"{what}: max |auto - safe| {err.max():.3e}"
    top2 = np.sort(safe, axis=-1)[..., -2:]
    decided = (top2[..., 1] - top2[..., 0]) > 2 * AUTO_LOGIT_TOL
    assert np.array_equal(auto.argmax(-1)[decided], safe.argmax(-1)[decided]), f"{what}: a label flipped"


def test_auto_cache_is_the_fp16_cache(lcg):
    _, _, _, _, safe, auto = lcg
    ck, cv, ik, iv = safe.context
    ak, av, aik, aiv = auto.context
    for b in range(3):  # column caches stay FP32 and do not depend on the ICL stage
        np.testing.assert_array_equal(ak[b], ck[b])
        np.testing.assert_array_equal(av[b], cv[b])
    assert aik[0].dtype == np.float16
    np.testing.assert_array_equal(aik[0], ik[0].astype(np.float16))
    np.testing.assert_array_equal(aiv[0], iv[0].astype(np.float16))
    for b in range(1, 12):  # later blocks follow the FP16 attention of the blocks before
        np.testing.assert_allclose(aik[b].astype(np.float32), ik[b], atol=2e-2, rtol=2e-2)


def test_auto_predictions_pass_the_gate(lcg, clf_weights):
    x, y, xt, shifts, safe, auto = lcg
    s = safe.predict_raw(xt).logits[..., :3]
    a = auto.predict_raw(xt).logits[..., :3]
    gate(a, s, "auto vs safe")
    O.set_threads(16)
    oracle = O.OracleModel("classifier", clf_weights, O.EXACT)
    cpu = oracle.predict_uncached(x, y, xt)[..., :3]
    gate(a, cpu, "auto vs the oracle's FP32 uncached forward")
    pa, ps = auto.predict_probabilities(xt), safe.predict_probabilities(xt)
    assert np.abs(pa - ps).max() <= 1e-3


def test_auto_pass_sizes_and_small_passes(lcg):
    _, _, xt, _, _, auto = lcg
    whole = auto.predict_raw(xt).logits
    auto.set_pass_rows(32)
    try:
        chunked = auto.predict_raw(xt).logits
        one = auto.predict_raw(xt[:, :1]).logits
    finally:
        auto.set_pass_rows(512)
    np.testing.assert_allclose(chunked, whole, atol=1e-5, rtol=1e-5)
    np.testing.assert_allclose(one[:, 0], whole[:, 0], atol=1e-5, rtol=1e-5)


def test_auto_context_exports_as_fp16_and_reloads(clf, lcg, tmp_path):
    x, y, xt, shifts, safe, auto = lcg
    resident = clf.build_context(x, y, class_permutations=shifts, optimize="auto")
    path, host = tmp_path / "auto.irctx", tmp_path / "auto-host.irctx"
    resident.save_context(path)  # streamed out of HBM, unpacked from the cache layout
    auto.save_context(host)      # from the build's host download
    assert path.read_bytes() == host.read_bytes()
    ctx = cf.read(path)
    assert ctx.version == 2 and ctx.tensor("icl.0.key").dtype == np.float16
    assert ctx.tensor("column.0.key").dtype == np.float32
    assert ctx.metadata.context_sha256 != safe.metadata.context_sha256  # the identity covers optimize
    reloaded = clf.load_context(path)
    np.testing.assert_array_equal(reloaded.predict_raw(xt).logits, resident.predict_raw(xt).logits)
    with pytest.raises(cf.ContextError, match="optimize"):
        clf.load_context(path, optimize="safe")
    d = tmp_path / "cache"
    a = clf.build_context(x, y, class_permutations=shifts, optimize="auto", cache_dir=d)
    s = clf.build_context(x, y, class_permutations=shifts, cache_dir=d)
    assert len(cf.cache_info(d).entries) == 2
    hit = clf.build_context(x, y, class_permutations=shifts, optimize="auto", cache_dir=d)
    np.testing.assert_array_equal(hit.predict_raw(xt).logits, a.predict_raw(xt).logits)
    assert s.precision == hip.PRECISION_FP32 and hit.precision == hip.PRECISION_SPLIT


# ---- optimize="fast": FP8 E4M3 ICL cache, single FP16 products ----

FAST_LOGIT_TOL = 5e-2  # docs/experiments.md:414: fast within 5e-2 of safe


@pytest.fixture(scope="module")
def fast(clf, lcg):
    x, y, xt, shifts, safe, auto = lcg
    return clf.build_context(x, y, class_permutations=shifts, download=True, optimize="fast")


def test_fast_builds_the_auto_context(lcg, fast):
    """The reference builds "fast" as "auto" (cuda/build.rs:477-511): the
    context's FP16 tensors are the same; only the resident cache is FP8."""
    *_, auto = lcg
    for a, f in zip(auto.context, fast.context):
        for ta, tf in zip(a, f):
            np.testing.assert_array_equal(tf, ta)
    assert fast.precision == hip.PRECISION_HALF and fast.context[2][0].dtype == np.float16


def test_fast_predictions_pass_their_gate(lcg, fast, clf_weights):
    x, y, xt, shifts, safe, auto = lcg
    s = safe.predict_raw(xt).logits[..., :3]
    f = fast.predict_raw(xt).logits[..., :3]
    err = np.abs(f - s)
    assert err.max() <= FAST_LOGIT_TOL, err.max()
    top2 = np.sort(s, axis=-1)[..., -2:]
    decided = (top2[..., 1] - top2[..., 0]) > 2 * FAST_LOGIT_TOL
    assert np.array_equal(f.argmax(-1)[decided], s.argmax(-1)[decided])
    O.set_threads(16)
    cpu = O.OracleModel("classifier", clf_weights, O.EXACT).predict_uncached(x, y, xt)[..., :3]
    assert np.abs(f - cpu).max() <= FAST_LOGIT_TOL
    assert np.abs(fast.predict_probabilities(xt) - safe.predict_probabilities(xt)).max() <= 1e-2
    # FP8 is coarser than the FP16 cache: "fast" is no closer to safe than "auto".
    assert err.max() >= np.abs(auto.predict_raw(xt).logits[..., :3] - s).max()


def test_fast_pass_sizes_agree(lcg, fast):
    _, _, xt, _, _, _ = lcg
    whole = fast.predict_raw(xt).logits
    fast.set_pass_rows(32)
    try:
        chunked = fast.predict_raw(xt).logits
        one = fast.predict_raw(xt[:, :1]).logits
    finally:
        fast.set_pass_rows(512)
    assert np.abs(chunked - whole).max() <= 1e-2
    assert np.abs(one[:, 0] - whole[:, 0]).max() <= 1e-2


def test_fast_context_exports_as_fp16_and_reloads(clf, lcg, fast, tmp_path):
    x, y, xt, shifts, safe, auto = lcg
    resident = clf.build_context(x, y, class_permutations=shifts, optimize="fast")  # no download asked
    path, host = tmp_path / "fast.irctx", tmp_path / "fast-host.irctx"
    resident.save_context(path)  # the build's FP16 cache, kept in HBM beside the FP8 one
    fast.save_context(host)
    assert path.read_bytes() == host.read_bytes()
    ctx = cf.read(path)
    np.testing.assert_array_equal(ctx.tensor("icl.3.value"), auto.context[3][3])
    assert ctx.metadata.context_sha256 not in (auto.metadata.context_sha256, safe.metadata.context_sha256)
    reloaded = clf.load_context(path, optimize="fast")
    np.testing.assert_array_equal(reloaded.predict_raw(xt).logits, resident.predict_raw(xt).logits)
    assert reloaded.precision == hip.PRECISION_HALF
    with pytest.raises(hip.HipError) as e:  # made from host tensors: FP8 only on the device
        buf = np.zeros(4, np.float16)
        hip.check(hip.lib().irx_predictor_read_context(reloaded.handle, 6, 0, 4, buf.ctypes.data))
    assert e.value.status == hip.UNSUPPORTED
    again = tmp_path / "fast-again.irctx"
    reloaded.save_context(again)  # from the host tensors it was made from
    assert again.read_bytes() == path.read_bytes()
    with pytest.raises(cf.ContextError, match="optimize"):
        clf.load_context(path, optimize="safe")
    d = tmp_path / "cache"
    first = clf.build_context(x, y, class_permutations=shifts, optimize="fast", cache_dir=d)
    hit = clf.build_context(x, y, class_permutations=shifts, optimize="fast", cache_dir=d)
    assert len(cf.cache_info(d).entries) == 1 and hit.precision == hip.PRECISION_HALF
    np.testing.assert_array_equal(hit.predict_raw(xt).logits, first.predict_raw(xt).logits)
