"""Kernel families on the GPU through the C ABI harness, against float64
references (the reference's tests/cuda_products.rs:54-103 and
tests/cuda_attention.rs:58-118 at FP32)."""

import ctypes
import math

import numpy as np
import pytest

from ironicl_amd import hip

import fp8_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def device():
    return hip.Device(0)


def values(count: int, seed: int) -> np.ndarray:
    """tests/cuda_products.rs:9-24: a 64-bit LCG, unit = (state >> 40) / 2^24,
    value = (unit - 0.5) * 0.2."""
    out = np.empty(count, np.float32)
    state = seed
    mask = (1 << 64) - 1
    for i in range(count):
        state = (state * 6364136223846793005 + 1442695040888963407) & mask
        out[i] = np.float32(((state >> 40) / float(1 << 24) - 0.5) * 0.2)
    return out


def fast_values(count: int, seed: int, scale: float = 1.0) -> np.ndarray:
    return (np.random.default_rng(seed).uniform(-1.0, 1.0, count) * scale).astype(np.float32)


def gelu64(x):
    from scipy.special import erf
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


@pytest.mark.parametrize("m,n,k,n2", [(65, 64, 64, 64), (300, 512, 512, 10), (513, 1024, 512, 512),
                                      (128, 512, 1024, 512), (4096, 384, 128, 128), (7, 1024, 512, 999),
                                      (1, 512, 512, 512), (3, 128, 256, 128), (8, 1024, 512, 512),
                                      (17, 1024, 512, 999), (40, 512, 1024, 512), (64, 1024, 512, 512),
                                      (9, 512, 512, 512), (32, 1024, 1024, 512)])
def test_products_match_float64(device, m, n, k, n2):
    """Each product family: tiled GEMMs, split-K over four waves, the eight-wave
    split-K of 9-64 rows at K = 512 / 1,024 (ragged N = 999 included; the
    second product adds its input as residual when n2 == n), and the small-row
    products of at most eight rows."""
    gen = values if m * k < 300_000 else fast_values
    x = gen(m * k, 1)
    w1, b1 = gen(n * k, 2), gen(n, 3)
    w2, b2 = gen(n2 * n, 4), gen(n2, 5)
    first = np.zeros(m * n, np.float32)
    second = np.zeros(m * n2, np.float32)
    F = hip.fptr
    hip.check(hip.lib().irx_test_products(device.handle, F(x), F(w1), F(b1), F(w2), F(b2), m, n, k, n2,
                                          F(first), F(second)))
    y = gelu64(x.reshape(m, k).astype(np.float64) @ w1.reshape(n, k).T.astype(np.float64) + b1)
    z = y @ w2.reshape(n2, n).T.astype(np.float64) + b2
    if n2 == n:
        z = z + y

    def rel(got, want):
        return np.abs(got.reshape(want.shape) - want).max() / np.abs(want).max()

    assert rel(first, y) < 1e-5 and rel(second, z) < 1e-5, (rel(first, y), rel(second, z))


def test_large_products_with_a_split_last_round(device):
    """70,000 rows: 2,188 tiles of 128 x 128 fill whole rounds on 256 CUs up to
    row 65,536 (two rounds of four workgroups per CU, or four of two), so both
    products (GELU, then residual) run those rows as 128 x 128 tiles and the
    4,464 rows after them as 64 x 64 tiles. Rows on both sides of that
    boundary and the last rows against float64."""
    m, n, k = 70_000, 512, 512
    x = fast_values(m * k, 11)
    w1, b1 = fast_values(n * k, 12, 0.05), fast_values(n, 13)
    w2, b2 = fast_values(n * n, 14, 0.05), fast_values(n, 15)
    first = np.zeros(m * n, np.float32)
    second = np.zeros(m * n, np.float32)
    F = hip.fptr
    hip.check(hip.lib().irx_test_products(device.handle, F(x), F(w1), F(b1), F(w2), F(b2), m, n, k, n,
                                          F(first), F(second)))
    rows = np.r_[0:64, 65_472:65_600, m - 64:m]
    y = gelu64(x.reshape(m, k)[rows].astype(np.float64) @ w1.reshape(n, k).T.astype(np.float64) + b1)
    z = y @ w2.reshape(n, n).T.astype(np.float64) + b2 + y
    got1, got2 = first.reshape(m, n)[rows], second.reshape(m, n)[rows]
    assert np.abs(got1 - y).max() / np.abs(y).max() < 1e-5
    assert np.abs(got2 - z).max() / np.abs(z).max() < 1e-5


def attention64(q, k, v, scale):
    s = (q.astype(np.float64) @ k.astype(np.float64).T) * scale
    p = np.exp(s - s.max(-1, keepdims=True))
    return (p / p.sum(-1, keepdims=True)) @ v.astype(np.float64)


@pytest.mark.parametrize("rows", [1, 63, 64, 65, 2000, 10007])
def test_icl_attention_matches_float64(device, rows):
    pairs = 64
    k = fast_values(pairs * rows * 64, 2).reshape(pairs, rows, 64)
    v = fast_values(pairs * rows * 64, 3).reshape(pairs, rows, 64)
    for query_rows in (1, 5, 8, 16, 17, 32, 33, 64, 100):
        q = fast_values(pairs * query_rows * 64, 1, scale=3.0).reshape(pairs, query_rows, 64)
        out = np.zeros_like(q)
        F = hip.fptr
        hip.check(hip.lib().irx_test_icl_attention(device.handle, F(q), F(k), F(v), pairs, query_rows, rows,
                                                   F(out)))
        worst = 0.0
        for pair in (0, 17, 63):
            rows_sel = list(range(query_rows)) if query_rows <= 32 else sorted({0, query_rows // 2, query_rows - 1})
            want = attention64(q[pair, rows_sel], k[pair], v[pair], 0.125)
            worst = max(worst, np.abs(out[pair, rows_sel] - want).max())
        assert worst < 1e-5, (rows, query_rows, worst)


@pytest.fixture(scope="module")
def keys_50k():
    """K and V of one estimator's 8 heads over 50,000 cached rows, the
    benchmark's context size."""
    pairs, rows = 8, 50_000
    return (fast_values(pairs * rows * 64, 41).reshape(pairs, rows, 64),
            fast_values(pairs * rows * 64, 42).reshape(pairs, rows, 64))


@pytest.mark.parametrize("query_rows", [512, 1, 16, 17, 32])
@pytest.mark.parametrize("peaked", [False, True])
def test_icl_attention_at_the_benchmarks_launch_shapes(device, keys_50k, query_rows, peaked):
    """The headline's exact launches: 8 pairs (one estimator's heads) over
    50,000 keys, at 512 queries (the 512-row pass: 16 key ranges per query
    tile, merged) and at 1, 16, 17 and 32 queries (passes of at most 32 rows:
    the decode kernel over 64 key ranges, one or two query groups). Queries
    scaled by 3, or peaked: each query 40 times a key spread over the whole
    key range, so one key dominates and the running reference moves in the
    range that holds it."""
    k, v = keys_50k
    pairs, rows = k.shape[0], k.shape[1]
    if peaked:
        at = np.linspace(0, rows - 1, query_rows).astype(np.int64)
        q = np.ascontiguousarray(k[:, at] * np.float32(40.0))
    else:
        q = fast_values(pairs * query_rows * 64, 43, scale=3.0).reshape(pairs, query_rows, 64)
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_icl_attention(device.handle, F(q), F(k), F(v), pairs, query_rows, rows, F(out)))
    sel = sorted({0, 1, query_rows // 2, query_rows - 1}) if query_rows > 32 else list(range(query_rows))
    worst = 0.0
    for pair in (0, 3, 7):
        want = attention64(q[pair, sel], k[pair], v[pair], 0.125)
        worst = max(worst, np.abs(out[pair, sel] - want).max())
    assert worst < 1e-5, (query_rows, peaked, worst)


@pytest.mark.parametrize("query_rows,rows", [(8193, 9000), (20000, 20000), (50000, 50000)])
@pytest.mark.parametrize("peaked", [False, True])
def test_icl_attention_whole_rounds_and_split_tail(device, query_rows, rows, peaked):
    """Self-attention sized launches (the build's 20,000- and 50,000-row
    shapes, and 8,193 queries over 9,000 keys): the (query tile, pair) units
    that fill whole rounds of one workgroup per CU take every key, and the
    units left over are split over key ranges and merged (on 256 CUs: 32
    units in 8 ranges, 120 in 2, 8 in 16). Rows checked against float64 on
    both sides of the boundary between the two launches."""
    pairs = 8
    k = fast_values(pairs * rows * 64, 51).reshape(pairs, rows, 64)
    v = fast_values(pairs * rows * 64, 52).reshape(pairs, rows, 64)
    if peaked:
        at = np.linspace(0, rows - 1, query_rows).astype(np.int64)
        q = np.ascontiguousarray(k[:, at] * np.float32(40.0))
    else:
        q = fast_values(pairs * query_rows * 64, 53, scale=3.0).reshape(pairs, query_rows, 64)
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_icl_attention(device.handle, F(q), F(k), F(v), pairs, query_rows, rows, F(out)))
    qtiles = -(-query_rows // 256)
    units = qtiles * pairs
    first_tail = units // 256 * 256  # first unit past the whole rounds (256 CUs)
    # Three rows of the units at the boundary, one row of every tail unit and
    # of every 37th unit before it.
    check = {}
    for unit in {0, first_tail - 1, first_tail, units - 1}:
        pair, qt = divmod(unit, qtiles)
        check.setdefault(pair, set()).update({qt * 256, min(qt * 256 + 129, query_rows - 1),
                                              min(qt * 256 + 255, query_rows - 1)})
    for unit in list(range(0, first_tail, 37)) + list(range(first_tail, units)):
        pair, qt = divmod(unit, qtiles)
        check.setdefault(pair, set()).add(min(qt * 256 + (unit * 97) % 256, query_rows - 1))
    worst = 0.0
    for pair, sel in check.items():
        sel = sorted(sel)
        want = attention64(q[pair, sel], k[pair], v[pair], 0.125)
        worst = max(worst, np.abs(out[pair, sel] - want).max())
    assert worst < 1e-5, (query_rows, rows, peaked, worst)


@pytest.mark.parametrize("rows", [1, 63, 64, 65, 2000, 10007])
def test_icl_attention_split_fp16_matches_float64(device, rows):
    """Split-FP16 products over the FP16 cache (optimize="auto"): against
    float64 attention of the FP16-rounded keys and values, and against the
    unrounded ones within the cache's own rounding."""
    pairs = 16
    k = fast_values(pairs * rows * 64, 2).reshape(pairs, rows, 64)
    v = fast_values(pairs * rows * 64, 3).reshape(pairs, rows, 64)
    k16, v16 = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
    for query_rows in (1, 5, 16, 17, 32, 40, 64, 100, 300):
        q = fast_values(pairs * query_rows * 64, 1, scale=3.0).reshape(pairs, query_rows, 64)
        out = np.zeros_like(q)
        F = hip.fptr
        hip.check(hip.lib().irx_test_icl_attention_precision(device.handle, hip.PRECISION_SPLIT, F(q), F(k), F(v),
                                                             pairs, query_rows, rows, F(out)))
        worst16 = worst = 0.0
        for pair in (0, 7, 15):
            rows_sel = sorted({0, query_rows // 2, query_rows - 1})
            want16 = attention64(q[pair, rows_sel], k16[pair], v16[pair], 0.125)
            want = attention64(q[pair, rows_sel], k[pair], v[pair], 0.125)
            worst16 = max(worst16, np.abs(out[pair, rows_sel] - want16).max())
            worst = max(worst, np.abs(out[pair, rows_sel] - want).max())
        assert worst16 < 2e-5, (rows, query_rows, worst16)
        assert worst < 5e-3, (rows, query_rows, worst)


@pytest.mark.parametrize("rows", [1, 63, 64, 65, 1000])
def test_fp8_cache_encoding_matches_the_restatement(device, rows):
    """The FP8 cache block (optimize="fast") byte for byte: E4M3 keys, V^T
    tiles in the stored key order, zero padding, per-(pair, dim) scales."""
    pairs = 8
    rng = np.random.default_rng(rows)
    k = (rng.normal(size=(pairs, rows, 64)) * rng.uniform(0.01, 30, size=(1, 1, 64))).astype(np.float16)
    v = (rng.normal(size=(pairs, rows, 64)) * rng.uniform(0.01, 30, size=(1, 1, 64))).astype(np.float16)
    k[:, :, 5] = 0  # an all-zero dim: scale 1
    v[1, :, 7] = 2.0 ** -20  # subnormal FP16 values
    n_pad = (rows + 63) // 64 * 64
    block = np.zeros(2 * pairs * n_pad * 64 + 1024 * pairs, np.uint8)
    hip.check(hip.lib().irx_test_encode_icl8(device.handle, k.ctypes.data, v.ctypes.data, pairs, rows,
                                             block.ctypes.data))
    plane = pairs * n_pad * 64
    got_k = block[:plane].reshape(pairs, n_pad, 64)
    got_vt = block[plane:2 * plane].reshape(pairs, n_pad // 64, 64, 64)
    got_ks = block[2 * plane:2 * plane + 256 * pairs].view(np.float32).reshape(pairs, 64)
    got_vs = block[2 * plane + 256 * pairs:2 * plane + 512 * pairs].view(np.float32).reshape(pairs, 64)
    k8, vt, ks, vs = fp8_np.encode_block(k, v)
    np.testing.assert_array_equal(got_ks, ks)
    np.testing.assert_array_equal(got_vs, vs)
    np.testing.assert_array_equal(got_k, k8)
    np.testing.assert_array_equal(got_vt, vt)
    assert np.all(got_ks[:, 5] == 1.0)


@pytest.mark.parametrize("rows", [1, 63, 64, 65, 2000, 10007])
def test_icl_attention_fp8_matches_float64(device, rows):
    """Single FP16 products over the FP8 cache (optimize="fast"): against
    float64 attention of the dequantized keys and values (byte x scale), within
    the FP16 rounding of the scaled queries and of the probabilities."""
    pairs = 16
    k = fast_values(pairs * rows * 64, 2).reshape(pairs, rows, 64)
    v = fast_values(pairs * rows * 64, 3).reshape(pairs, rows, 64)
    k8, vt, ks, vs = fp8_np.encode_block(k.astype(np.float16), v.astype(np.float16))
    kd = fp8_np.e4m3_value(k8[:, :rows]) * ks[:, None, :]
    vq = np.zeros_like(k8)
    key = np.arange(64)
    pos = 16 * (key // 16) + fp8_np.stored_position(key % 16)
    vq.reshape(pairs, -1, 64, 64)[:] = vt[:, :, :, pos].transpose(0, 1, 3, 2)
    vd = fp8_np.e4m3_value(vq[:, :rows]) * vs[:, None, :]
    for query_rows in (1, 5, 16, 17, 32, 40, 64, 300):
        q = fast_values(pairs * query_rows * 64, 1, scale=3.0).reshape(pairs, query_rows, 64)
        out = np.zeros_like(q)
        F = hip.fptr
        hip.check(hip.lib().irx_test_icl_attention_precision(device.handle, hip.PRECISION_HALF, F(q), F(k), F(v),
                                                             pairs, query_rows, rows, F(out)))
        worst = 0.0
        for pair in (0, 7, 15):
            rows_sel = sorted({0, query_rows // 2, query_rows - 1})
            want = attention64(q[pair, rows_sel], kd[pair], vd[pair], 0.125)
            worst = max(worst, np.abs(out[pair, rows_sel] - want).max())
        assert worst < 5e-3, (rows, query_rows, worst)


@pytest.mark.parametrize("qr", [12, 40])
def test_icl_attention_split_fp16_peaked_scores(device, qr):
    """Large logits with the FP16 path's lower lazy limit: the reference is
    raised more often and the output stays exact to the cache's rounding."""
    pairs, rows = 8, 3000
    k = fast_values(pairs * rows * 64, 7).reshape(pairs, rows, 64)
    v = fast_values(pairs * rows * 64, 8).reshape(pairs, rows, 64)
    q = (k[:, 1234:1234 + qr] * 40.0).copy()
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_icl_attention_precision(device.handle, hip.PRECISION_SPLIT, F(q), F(k), F(v), pairs,
                                                         qr, rows, F(out)))
    k16, v16 = k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)
    for pair in (0, 5):
        want = attention64(q[pair], k16[pair], v16[pair], 0.125)
        assert np.abs(out[pair] - want).max() < 2e-5


@pytest.mark.parametrize("qr", [12, 30, 40])
def test_icl_attention_peaked_scores(device, qr):
    """Large logits: one key dominates; the online max must stay exact."""
    pairs, rows = 8, 3000
    k = fast_values(pairs * rows * 64, 7).reshape(pairs, rows, 64)
    v = fast_values(pairs * rows * 64, 8).reshape(pairs, rows, 64)
    q = (k[:, 1234:1234 + qr] * 40.0).copy()
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_icl_attention(device.handle, F(q), F(k), F(v), pairs, qr, rows, F(out)))
    for pair in (0, 5):
        want = attention64(q[pair], k[pair], v[pair], 0.125)
        assert np.abs(out[pair] - want).max() < 1e-5


def block_tail64(att, state, wo, bo, n2w, n2b, w1, b1, w2, b2):
    """cpu.rs:1555-1601 in float64: out-projection + residual, LN2, FFN + residual."""
    s1 = state.astype(np.float64) + (att.astype(np.float64) @ wo.astype(np.float64).T + bo)
    x = (s1 - s1.mean(1, keepdims=True)) / np.sqrt(s1.var(1, keepdims=True) + 1e-5) * n2w + n2b
    h = gelu64(x @ w1.astype(np.float64).T + b1)
    return s1 + (h @ w2.astype(np.float64).T + b2)


@pytest.mark.parametrize("rows,outputs", [(1, 128), (3, 384), (8, 256), (65, 384), (1000, 256), (16411, 384),
                                          (17000, 128)])
@pytest.mark.parametrize("fused", [0, 1])
def test_block_head_matches_float64(device, rows, outputs, fused):
    """LN1 + in_proj of a 128-wide block: the fused kernel, and the product
    with the LayerNorm in its prologue (small products) or before it."""
    x = fast_values(rows * 128, 21, 3.0) + 0.2
    lnw, lnb = fast_values(128, 22, 0.2) + 1.0, fast_values(128, 23, 0.1)
    w, b = fast_values(outputs * 128, 24, 0.09), fast_values(outputs, 25, 0.1)
    out = np.zeros(rows * outputs, np.float32)
    F = hip.fptr
    hip.check(hip.lib().irx_test_block_head(device.handle, fused, F(x), rows, F(lnw), F(lnb), F(w), F(b), outputs,
                                            F(out)))
    want = ln64(x.reshape(rows, 128), lnw, lnb) @ w.reshape(outputs, 128).T.astype(np.float64) + b
    np.testing.assert_allclose(out.reshape(rows, outputs), want, rtol=1e-4, atol=1e-5)


@pytest.mark.parametrize("rows", [1, 5, 17, 64, 65, 1000, 16411])
@pytest.mark.parametrize("fused", [0, 1, 2])
def test_block_tail_matches_float64(device, rows, fused):
    att = fast_values(rows * 128, 1, 2.0)
    state = fast_values(rows * 128, 2, 3.0)
    wo, bo = fast_values(128 * 128, 3, 0.09), fast_values(128, 4, 0.1)
    n2w, n2b = fast_values(128, 5, 0.2) + 1.0, fast_values(128, 6, 0.1)
    w1, b1 = fast_values(256 * 128, 7, 0.09), fast_values(256, 8, 0.1)
    w2, b2 = fast_values(128 * 256, 9, 0.06), fast_values(128, 10, 0.1)
    out = np.zeros_like(state)
    F = hip.fptr
    hip.check(hip.lib().irx_test_block_tail(device.handle, fused, F(att), F(state), rows, F(wo), F(bo), F(n2w),
                                            F(n2b), F(w1), F(b1), F(w2), F(b2), 1, F(out)))
    want = block_tail64(att.reshape(rows, 128), state.reshape(rows, 128), wo.reshape(128, 128), bo, n2w, n2b,
                        w1.reshape(256, 128), b1, w2.reshape(128, 256), b2)
    np.testing.assert_allclose(out.reshape(rows, 128), want, rtol=1e-4, atol=1e-5)
    assert np.abs(out.reshape(rows, 128) - want).max() < 2e-5


@pytest.mark.parametrize("rows", [1, 16, 33, 1000])
def test_block_tail_small_pass_form_equals_tail128(device, rows):
    """The 16-rows-per-workgroup tail takes every product in tail128's order:
    the same bits, on rows that are not a multiple of either's tile."""
    att = fast_values(rows * 128, 11, 2.0)
    state = fast_values(rows * 128, 12, 3.0)
    wo, bo = fast_values(128 * 128, 13, 0.09), fast_values(128, 14, 0.1)
    n2w, n2b = fast_values(128, 15, 0.2) + 1.0, fast_values(128, 16, 0.1)
    w1, b1 = fast_values(256 * 128, 17, 0.09), fast_values(256, 18, 0.1)
    w2, b2 = fast_values(128 * 256, 19, 0.06), fast_values(128, 20, 0.1)
    outs = []
    F = hip.fptr
    for fused in (1, 2):
        out = np.zeros_like(state)
        hip.check(hip.lib().irx_test_block_tail(device.handle, fused, F(att), F(state), rows, F(wo), F(bo), F(n2w),
                                                F(n2b), F(w1), F(b1), F(w2), F(b2), 1, F(out)))
        outs.append(out)
    np.testing.assert_array_equal(outs[0], outs[1])


def column_weights(seed):
    """LN1, the query rows of in_proj and the tail's weights of a cached column block."""
    shapes = {"lnw": (128,), "lnb": (128,), "wq": (128, 128), "bq": (128,), "wo": (128, 128), "bo": (128,),
              "n2w": (128,), "n2b": (128,), "w1": (256, 128), "b1": (256,), "w2": (128, 256), "b2": (128,)}
    scales = {"lnw": 0.2, "lnb": 0.1, "wq": 0.09, "bq": 0.1, "wo": 0.09, "bo": 0.1, "n2w": 0.2, "n2b": 0.1,
              "w1": 0.09, "b1": 0.1, "w2": 0.06, "b2": 0.1}
    out = {}
    for i, (name, shape) in enumerate(shapes.items()):
        out[name] = fast_values(int(np.prod(shape)), seed + i, scales[name]).reshape(shape)
    out["lnw"] = out["lnw"] + np.float32(1.0)
    out["n2w"] = out["n2w"] + np.float32(1.0)
    return out


def column_block64(state, k, v, wt):
    """cached_block (cpu.rs:2587-2850) in float64 for [cols, rows, 128] states
    against [cols, 8, 128, 16] cached inducing keys and values."""
    cols, rows = state.shape[:2]
    x = state.astype(np.float64).reshape(-1, 128)
    q = (ln64(x, wt["lnw"], wt["lnb"]) @ wt["wq"].T.astype(np.float64) + wt["bq"]).reshape(cols, rows, 128)
    att = np.zeros((cols, rows, 128))
    for h in range(8):
        s = np.matmul(q[..., 16 * h:16 * h + 16], np.swapaxes(k[:, h].astype(np.float64), 1, 2)) * 0.25
        s = np.exp(s - s.max(-1, keepdims=True))
        att[..., 16 * h:16 * h + 16] = np.matmul(s / s.sum(-1, keepdims=True), v[:, h].astype(np.float64))
    return block_tail64(att.reshape(-1, 128), x, wt["wo"], wt["bo"], wt["n2w"], wt["n2b"], wt["w1"], wt["b1"],
                        wt["w2"], wt["b2"]).reshape(cols, rows, 128)


def run_column_block(device, fused, state, k, v, wt):
    cols, rows = state.shape[:2]
    out = np.zeros_like(state)
    F = hip.fptr
    hip.check(hip.lib().irx_test_column_block(device.handle, fused, F(state), cols, rows, F(k), F(v), F(wt["lnw"]),
                                              F(wt["lnb"]), F(wt["wq"]), F(wt["bq"]), F(wt["wo"]), F(wt["bo"]),
                                              F(wt["n2w"]), F(wt["n2b"]), F(wt["w1"]), F(wt["b1"]), F(wt["w2"]),
                                              F(wt["b2"]), 1, F(out)))
    return out


def column_inputs(cols, rows, seed):
    state = fast_values(cols * rows * 128, seed, 3.0).reshape(cols, rows, 128)
    k = fast_values(cols * 8 * 128 * 16, seed + 1, 1.5).reshape(cols, 8, 128, 16)
    v = fast_values(cols * 8 * 128 * 16, seed + 2, 1.0).reshape(cols, 8, 128, 16)
    return state, k, v


@pytest.mark.parametrize("cols,rows", [(1, 1), (3, 17), (2, 100), (64, 512), (5, 3333)])
@pytest.mark.parametrize("fused", [0, 1, 2])
def test_column_block_matches_float64(device, cols, rows, fused):
    """A cached column block (LN1, query projection, 8-head attention to the
    column's 128 cached inducing K/V, tail), as one kernel (64-row tiles or
    the small-pass form) and as three launches, against float64; rows not a
    multiple of the kernels' 64 or 16."""
    state, k, v = column_inputs(cols, rows, 31)
    wt = column_weights(40)
    out = run_column_block(device, fused, state, k, v, wt)
    want = column_block64(state, k, v, wt)
    np.testing.assert_allclose(out, want, rtol=1e-4, atol=1e-5)
    assert np.abs(out - want).max() < 3e-5


@pytest.mark.parametrize("cols,rows", [(64, 512), (37, 1000), (3, 6000)])
def test_column_block_one_kernel_equals_three_launches(device, cols, rows):
    """From 16,384 states the three launches are head128, the 16-wide
    attention and tail128, whose arithmetic the one kernel repeats: the same
    bits (peaked scores included: keys scaled up so one dominates)."""
    state, k, v = column_inputs(cols, rows, 51)
    wt = column_weights(60)
    for kscale in (1.0, 12.0):
        kk = (k * np.float32(kscale)).astype(np.float32)
        one = run_column_block(device, 1, state, kk, v, wt)
        three = run_column_block(device, 0, state, kk, v, wt)
        np.testing.assert_array_equal(one, three)


@pytest.mark.parametrize("cols,rows", [(64, 1), (3, 17), (64, 32), (7, 300)])
def test_column_block_small_pass_form_equals_one_kernel(device, cols, rows):
    """The 16-rows-per-workgroup form repeats the one kernel's arithmetic:
    the same bits at every pass size (peaked scores included)."""
    state, k, v = column_inputs(cols, rows, 71)
    wt = column_weights(80)
    for kscale in (1.0, 12.0):
        kk = (k * np.float32(kscale)).astype(np.float32)
        np.testing.assert_array_equal(run_column_block(device, 2, state, kk, v, wt),
                                      run_column_block(device, 1, state, kk, v, wt))


def ln64(x, w, b):
    x = x.astype(np.float64)
    return (x - x.mean(1, keepdims=True)) / np.sqrt(x.var(1, keepdims=True) + 1e-5) * w + b


@pytest.mark.parametrize("m,n", [(1, 512), (2, 1024), (3, 1024), (8, 512), (9, 1024), (16, 512), (17, 1024),
                                 (512, 1024), (1000, 512)])
def test_ln_linear_gelu_matches_float64(device, m, n):
    """LN2 + FFN up (and the decoder's LN + first layer) in one kernel."""
    x = fast_values(m * 512, 1, 3.0) + 0.25
    lnw, lnb = fast_values(512, 2, 0.2) + 1.0, fast_values(512, 3, 0.1)
    w, b = fast_values(n * 512, 4, 0.05), fast_values(n, 5, 0.1)
    out = np.zeros(m * n, np.float32)
    F = hip.fptr
    hip.check(hip.lib().irx_test_ln_linear(device.handle, 1, F(x), m, 0, F(lnw), F(lnb), F(w), F(b), n,
                                           None, None, None, None, None, F(out)))
    want = gelu64(ln64(x.reshape(m, 512), lnw, lnb) @ w.reshape(n, 512).T.astype(np.float64) + b)
    np.testing.assert_allclose(out.reshape(m, n), want, rtol=1e-4, atol=2e-5)


@pytest.mark.parametrize("form,estimators,rows", [(2, 1, 1), (2, 1, 2), (2, 1, 5), (2, 8, 1), (2, 4, 2), (2, 3, 3),
                                                  (2, 1, 16), (2, 2, 8), (2, 3, 5), (2, 1, 32), (2, 4, 8), (2, 3, 11),
                                                  (2, 2, 250), (2, 3, 17), (3, 1, 1), (3, 3, 5), (3, 2, 250),
                                                  (3, 1, 2049), (3, 3, 1001)])
def test_ln_linear_qass_matches_float64(device, form, estimators, rows):
    """LN1 + Q projection + QASSMax (query MLP and gate per head), head-major:
    form 2 the prediction's fused kernel, form 3 the build's (LayerNorm, tiled
    projection, then the MLP and gate over the projected rows, whose waves each
    take a contiguous share of 16-row tasks; 3 x 1001 x 8 rows end mid-task)."""
    m = estimators * rows
    x = fast_values(m * 512, 6, 3.0) - 0.1
    lnw, lnb = fast_values(512, 7, 0.2) + 1.0, fast_values(512, 8, 0.1)
    w, b = fast_values(512 * 512, 9, 0.05), fast_values(512, 10, 0.1)
    m0w, m0b = fast_values(64 * 64, 11, 0.15), fast_values(64, 12, 0.1)
    m2w, m2b = fast_values(64 * 64, 13, 0.15), fast_values(64, 14, 0.1)
    base = fast_values(512, 15, 0.5) + 1.0
    out = np.zeros(m * 512, np.float32)
    F = hip.fptr
    hip.check(hip.lib().irx_test_ln_linear(device.handle, form, F(x), m, rows, F(lnw), F(lnb), F(w), F(b), 512,
                                           F(m0w), F(m0b), F(m2w), F(m2b), F(base), F(out)))
    q = ln64(x.reshape(m, 512), lnw, lnb) @ w.reshape(512, 512).T.astype(np.float64) + b
    q = q.reshape(estimators, rows, 8, 64).transpose(0, 2, 1, 3)  # head-major
    h = gelu64(q @ m0w.reshape(64, 64).T.astype(np.float64) + m0b)
    g = h @ m2w.reshape(64, 64).T.astype(np.float64) + m2b
    want = q * base.reshape(1, 8, 1, 64) * (1 + np.tanh(g))
    np.testing.assert_allclose(out.reshape(estimators, 8, rows, 64), want, rtol=1e-4, atol=2e-5)


def test_gelu_matches_float64(device):
    """The GELU every kernel computes (erfc from one fitted polynomial of log2
    erfc and one exponential) against float64 0.5 x (1 + erf(x / sqrt 2)) on a
    dense grid over [-12, 12], the fit's end at |x| = 4 sqrt 2, tiny and huge
    magnitudes: within 1.2e-7 (1 + |x|); +inf stays inf and NaN stays NaN."""
    from scipy.special import erf
    grid = np.linspace(-12.0, 12.0, 2_000_001)
    edge = 4.0 * math.sqrt(2.0) + np.linspace(-1e-4, 1e-4, 2001)
    extra = np.array([0.0, -0.0, 1e-30, -1e-30, 1e-7, -1e-7, 30.0, -30.0, 1e6, -1e6, 3.4e38, -3.4e38])
    x = np.concatenate([grid, edge, -edge, extra]).astype(np.float32)
    out = np.zeros_like(x)
    hip.check(hip.lib().irx_test_gelu(device.handle, hip.fptr(x), x.size, hip.fptr(out)))
    x64 = x.astype(np.float64)
    want = 0.5 * x64 * (1.0 + erf(x64 / math.sqrt(2.0)))
    err = np.abs(out.astype(np.float64) - want)
    assert (err <= 1.2e-7 * (1.0 + np.abs(x64))).all(), (x[err.argmax()], err.max())
    special = np.array([np.inf, np.nan], np.float32)
    got = np.zeros_like(special)
    hip.check(hip.lib().irx_test_gelu(device.handle, hip.fptr(special), 2, hip.fptr(got)))
    assert got[0] == np.inf and np.isnan(got[1])


@pytest.mark.parametrize("rows,width", [(1, 128), (333, 128), (1000, 512), (4, 512)])
def test_layer_norm_matches_float64(device, rows, width):
    x = fast_values(rows * width, 4, 3.0) + 0.5
    w, b = fast_values(width, 5, 0.1) + 1.0, fast_values(width, 6, 0.1)
    out = np.zeros_like(x)
    F = hip.fptr
    hip.check(hip.lib().irx_test_layer_norm(device.handle, F(x), F(w), F(b), rows, width, F(out)))
    x64 = x.reshape(rows, width).astype(np.float64)
    want = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5) * w + b
    assert np.abs(out.reshape(rows, width) - want).max() < 1e-5


@pytest.mark.parametrize("query_rows,rows", [(1, 1), (4, 68), (16, 16), (17, 33), (68, 68), (80, 127), (81, 100),
                                             (130, 128), (512, 128), (600, 50), (1000, 100), (128, 129),
                                             (128, 1000), (504, 504)])
def test_small_attention_matches_float64(device, query_rows, rows):
    heads = 8
    q = fast_values(heads * query_rows * 16, 1, 3.0).reshape(heads, query_rows, 16)
    k = fast_values(heads * rows * 16, 2).reshape(heads, rows, 16)
    v = fast_values(heads * rows * 16, 3).reshape(heads, rows, 16)
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_small_attention(device.handle, F(q), F(k), F(v), heads, query_rows, rows,
                                                 F(out)))
    for h in range(heads):
        assert np.abs(out[h] - attention64(q[h], k[h], v[h], 0.25)).max() < 1e-5


@pytest.mark.parametrize("query_rows,rows,qscale", [(128, 50000, 3.0), (4, 3000, 3.0), (20, 2049, 3.0),
                                                    (33, 777, 3.0), (300, 5000, 3.0), (128, 129, 40.0),
                                                    (64, 5000, 40.0), (1, 100000, 40.0)])
def test_small_attention_many_keys_matches_float64(device, query_rows, rows, qscale):
    """More than 128 keys (the inducing points over a column's train rows):
    every query-group width, key ranges split over workgroups and merged
    (8 heads leave most of the chip idle), ragged last blocks, and peaked
    scores that move the running reference many times."""
    heads = 8
    q = fast_values(heads * query_rows * 16, 4, qscale).reshape(heads, query_rows, 16)
    k = fast_values(heads * rows * 16, 5).reshape(heads, rows, 16)
    v = fast_values(heads * rows * 16, 6).reshape(heads, rows, 16)
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_small_attention(device.handle, F(q), F(k), F(v), heads, query_rows, rows,
                                                 F(out)))
    worst = max(np.abs(out[h] - attention64(q[h], k[h], v[h], 0.25)).max() for h in range(heads))
    assert worst < 1e-5, worst


@pytest.mark.parametrize("heads,query_rows,rows", [(1024, 68, 68), (512, 100, 128), (1024, 16, 80)])
def test_small_attention_many_items_matches_float64(device, heads, query_rows, rows):
    """As many (sequence, head) items as a 128-row pass has, where waves take
    several 16-query blocks each (few items give every block its own wave)."""
    q = fast_values(heads * query_rows * 16, 10, 3.0).reshape(heads, query_rows, 16)
    k = fast_values(heads * rows * 16, 11).reshape(heads, rows, 16)
    v = fast_values(heads * rows * 16, 12).reshape(heads, rows, 16)
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_small_attention(device.handle, F(q), F(k), F(v), heads, query_rows, rows,
                                                 F(out)))
    worst = max(np.abs(out[h] - attention64(q[h], k[h], v[h], 0.25)).max() for h in range(heads))
    assert worst < 1e-5, worst


def rope64(x, cos_t, sin_t):
    """x [rows, 16] at positions 0..rows-1: x[d] cos[t][d] + x[d ^ 8] sin[t][d]."""
    x = x.astype(np.float64)
    n = x.shape[0]
    return x * cos_t[:n] + x[:, np.arange(16) ^ 8] * sin_t[:n]


@pytest.mark.parametrize("query_rows,rows", [(68, 68), (130, 130), (20, 300), (128, 4000), (4, 133)])
def test_small_attention_rope_matches_float64(device, query_rows, rows):
    """The row transformer's attention with rotary embeddings, on the short
    (<= 128 keys) and long kernels. Tables as the row stage builds them: cos
    twice and [-sin, sin] of position x frequency."""
    heads = 8
    n = max(query_rows, rows)
    freqs = 1.0 / (10000.0 ** (np.arange(8) / 8.0))
    angle = np.arange(n)[:, None] * freqs[None, :]
    cos_t = np.concatenate([np.cos(angle), np.cos(angle)], 1).astype(np.float32)
    sin_t = np.concatenate([-np.sin(angle), np.sin(angle)], 1).astype(np.float32)
    q = fast_values(heads * query_rows * 16, 7, 3.0).reshape(heads, query_rows, 16)
    k = fast_values(heads * rows * 16, 8).reshape(heads, rows, 16)
    v = fast_values(heads * rows * 16, 9).reshape(heads, rows, 16)
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_small_attention_rope(device.handle, F(q), F(k), F(v), F(cos_t), F(sin_t), heads,
                                                      query_rows, rows, F(out)))
    worst = max(np.abs(out[h] - attention64(rope64(q[h], cos_t, sin_t), rope64(k[h], cos_t, sin_t), v[h],
                                            0.25)).max() for h in range(heads))
    assert worst < 1e-5, worst


def rope_tables(n):
    """The row stage's tables: cos twice and [-sin, sin] of position x
    100000^(-i/8) (docs/model.md:33)."""
    freqs = 1.0 / (100000.0 ** (np.arange(8) / 8.0))
    angle = np.arange(n)[:, None] * freqs[None, :]
    return (np.concatenate([np.cos(angle), np.cos(angle)], 1).astype(np.float32),
            np.concatenate([-np.sin(angle), np.sin(angle)], 1).astype(np.float32))


@pytest.mark.parametrize("seqs,query_rows,rows,rope,qscale", [
    (3, 58, 58, True, 3.0), (3, 68, 68, True, 3.0), (2, 104, 104, True, 3.0), (2, 204, 204, True, 3.0),
    (1, 504, 504, True, 3.0), (2, 17, 17, True, 3.0), (2, 32, 33, True, 3.0), (1, 600, 512, True, 3.0),
    (2, 1100, 128, False, 3.0), (4, 68, 68, True, 40.0), (2, 204, 204, True, 40.0), (1, 300, 257, False, 40.0)])
@pytest.mark.parametrize("method", [1, 2])
def test_small_attention_tokens_match_float64(device, seqs, query_rows, rows, rope, qscale, method):
    """Token-major sequences (a token's 8 heads adjacent, as the row
    transformer stores them) through the staged kernel (every key of an item
    in LDS once, query blocks over waves; method 2) and the per-wave and
    long-range kernels (method 1): the row transformer's lengths (H + 4 at
    54, 64, 100, 200 and 500 features), one- and two-block sequences, more
    query blocks than a workgroup holds at once, and peaked scores
    (qscale 40) that move the lazy softmax reference."""
    heads = 8
    q = fast_values(seqs * query_rows * heads * 16, 31, qscale).reshape(seqs, query_rows, heads, 16)
    k = fast_values(seqs * rows * heads * 16, 32).reshape(seqs, rows, heads, 16)
    v = fast_values(seqs * rows * heads * 16, 33).reshape(seqs, rows, heads, 16)
    cos_t, sin_t = rope_tables(max(query_rows, rows)) if rope else (None, None)
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_small_attention_tokens(device.handle, method, F(q), F(k), F(v),
                                                        F(cos_t) if rope else None, F(sin_t) if rope else None,
                                                        seqs, heads, query_rows, rows, F(out), 0, None))
    worst = 0.0
    for s_ in range(seqs):
        for h in (0, 3, 7):
            qq, kk = q[s_, :, h], k[s_, :, h]
            if rope:
                qq, kk = rope64(qq, cos_t, sin_t), rope64(kk, cos_t, sin_t)
            worst = max(worst, np.abs(out[s_, :, h] - attention64(qq, kk, v[s_, :, h], 0.25)).max())
    assert worst < 1e-5, worst


@pytest.mark.parametrize("qscale", [3.0, 40.0])
def test_rope_attention_past_512_tokens_matches_float64(device, qscale):
    """Rows of 604 tokens (600 features) are longer than the staged kernel
    takes: the row transformer's self-attention with RoPE then runs on the
    long-range kernel (method 0, as a build chooses)."""
    seqs, heads, tokens = 2, 8, 604
    q = fast_values(seqs * tokens * heads * 16, 34, qscale).reshape(seqs, tokens, heads, 16)
    k = fast_values(seqs * tokens * heads * 16, 35).reshape(seqs, tokens, heads, 16)
    v = fast_values(seqs * tokens * heads * 16, 36).reshape(seqs, tokens, heads, 16)
    cos_t, sin_t = rope_tables(tokens)
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_small_attention_tokens(device.handle, 0, F(q), F(k), F(v), F(cos_t), F(sin_t),
                                                        seqs, heads, tokens, tokens, F(out), 0, None))
    worst = 0.0
    for s_ in range(seqs):
        for h in (0, 5, 7):
            qq, kk = rope64(q[s_, :, h], cos_t, sin_t), rope64(k[s_, :, h], cos_t, sin_t)
            worst = max(worst, np.abs(out[s_, :, h] - attention64(qq, kk, v[s_, :, h], 0.25)).max())
    assert worst < 1e-5, worst


def test_staged_attention_rejects_what_it_cannot_take(device):
    z = np.zeros(16 * 8 * 600, np.float32)
    out = np.zeros_like(z)
    F = hip.fptr
    # 16 queries (one block) and 513 keys are both outside the staged kernel.
    assert hip.lib().irx_test_small_attention_tokens(device.handle, 2, F(z), F(z), F(z), None, None, 1, 8, 16, 16,
                                                     F(out), 0, None) == hip.INVALID_ARGUMENT
    assert hip.lib().irx_test_small_attention_tokens(device.handle, 2, F(z), F(z), F(z), None, None, 1, 1, 20, 513,
                                                     F(out), 0, None) == hip.INVALID_ARGUMENT
    assert hip.lib().irx_test_small_attention_tokens(device.handle, 3, F(z), F(z), F(z), None, None, 1, 1, 20, 20,
                                                     F(out), 0, None) == hip.INVALID_ARGUMENT


def test_harness_rejects_bad_shapes(device):
    z = np.zeros(64, np.float32)
    F = hip.fptr
    assert hip.lib().irx_test_icl_attention(device.handle, F(z), F(z), F(z), 3, 1, 1, F(z)) == hip.INVALID_ARGUMENT
    assert hip.lib().irx_test_products(device.handle, F(z), F(z), F(z), F(z), F(z), 1, 8, 8, 8, F(z),
                                       F(z)) == hip.INVALID_ARGUMENT
