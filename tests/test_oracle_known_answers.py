"""Pins the oracle's primitive kernels to the reference's own known answers
(tests/golden/known_answers.json, written from the reference's unit tests) and
to closed forms. CPU only."""

import json
import math
import os

import numpy as np
import pytest

import oracle as O
from conftest import lcg_values

KA = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def f32(v):
    return np.asarray(v, dtype=np.float32)


def test_affine_pytorch_layout():
    c = KA["affine"]
    out = O.affine(f32(c["input"]).reshape(c["rows"], c["in_dim"]),
                   f32(c["weight"]).reshape(c["out_dim"], c["in_dim"]), c["bias"])
    np.testing.assert_allclose(out.ravel(), c["expected"], atol=c["tolerance"])


def test_affine_without_bias_is_pure_product():
    w = f32([[1, 2], [3, 4]])
    out = O.affine(f32([[1, 1]]), w)
    np.testing.assert_array_equal(out, [[3, 7]])


def test_one_hot_linear_selects_columns():
    c = KA["one_hot_linear"]
    lib = O.lib()
    out = np.zeros(len(c["expected"]), np.float32)
    labels = f32(c["classes"])
    lib.ora_one_hot_linear(O.fp(labels), len(labels), O.fp(f32(c["weight"])), O.fp(f32(c["bias"])),
                           c["class_count"], c["out_dim"], O.fp(out))
    np.testing.assert_array_equal(out, c["expected"])


def test_layer_norm_epsilon_and_constant_row():
    c = KA["layer_norm"]
    out = O.layer_norm(f32([c["input"]]), c["weight"], c["bias"])
    np.testing.assert_allclose(out.ravel(), c["expected"], atol=c["tolerance"])
    out = O.layer_norm(f32([c["constant_input"]]), [1.0, 1.0])
    np.testing.assert_array_equal(out.ravel(), c["constant_expected"])


def test_layer_norm_matches_float64_on_model_widths():
    rng = np.random.default_rng(3)
    for width in (128, 512):
        x = f32(rng.normal(size=(7, width)) * 3 + 1)
        w, b = f32(rng.uniform(0.9, 1.1, width)), f32(rng.uniform(-0.1, 0.1, width))
        x64 = x.astype(np.float64)
        ref = (x64 - x64.mean(1, keepdims=True)) / np.sqrt(x64.var(1, keepdims=True) + 1e-5) * w + b
        np.testing.assert_allclose(O.layer_norm(x, w, b), ref, atol=2e-5)


@pytest.mark.parametrize("math_mode", [O.EXACT, O.NATIVE])
def test_gelu_known_values(math_mode):
    c = KA["gelu"]
    np.testing.assert_allclose(O.gelu(f32(c["input"]), math_mode), c["expected"], atol=c["tolerance"])


def test_native_approximations_within_reference_bounds():
    b = KA["native_bounds"]
    lo, hi, step = b["exp_domain"]
    xs = f32(np.arange(int(lo / step), int(hi / step) + 1) * step)
    lib = O.lib()
    worst = max(abs(lib.ora_fast_exp_negative(float(v)) - math.exp(float(v))) / math.exp(float(v)) for v in xs[::7])
    assert worst <= b["exp_relative"], worst
    lo, hi, step = b["gelu_domain"]
    xs = f32(np.arange(int(lo / step), int(hi / step) + 1) * step)
    exact, native = O.gelu(xs, O.EXACT), O.gelu(xs, O.NATIVE)
    assert np.abs(exact - native).max() <= b["gelu_abs"]


def test_rope_rotates_contiguous_halves():
    c = KA["rope"]
    x = f32(c["input"]).reshape(c["heads"], c["rows"], c["head_dim"])
    out = O.rope(x, f32(c["frequencies"]), c["position_offset"])
    np.testing.assert_allclose(out.ravel(), c["expected"], atol=c["tolerance"])


def test_qassmax_base_zero_at_one_source_and_monotone_at_two():
    c = KA["qassmax"]
    lib = O.lib()
    q = f32(c["queries"])
    args = [f32(c[k]) for k in ("base_first_weight", "base_first_bias", "base_second_weight", "base_second_bias",
                                  "query_first_weight", "query_first_bias", "query_second_weight",
                                  "query_second_bias")]
    for source, check in ((1, "zero"), (2, "monotone")):
        out = np.zeros(2, np.float32)
        lib.ora_qassmax(O.fp(q), c["heads"], c["rows"], c["head_dim"], source, c["hidden"],
                        *[O.fp(a) for a in args], O.fp(out))
        if check == "zero":
            np.testing.assert_array_equal(out, c["expected_at_one_source"])
        else:
            assert 0 < out[0] < out[1]


def test_attention_closed_form():
    c = KA["attention_closed_form"]
    q, k, v = f32(c["query"]).reshape(1, 1, 2), f32(c["key"]).reshape(1, 2, 2), f32(c["value"]).reshape(1, 2, 2)
    w = c["weight"]
    expected = [10 * w + 30 * (1 - w), 20 * w + 40 * (1 - w)]
    for out in (O.attention_materialized(q, k, v), O.attention(q, k, v), O.attention(q, k, v, O.NATIVE)):
        np.testing.assert_allclose(out.ravel(), expected, atol=c["tolerance"])


def test_online_attention_matches_materialized_across_tiles():
    state = 1
    for heads, qr, sr, hd, _qb, _kt in KA["online_attention_cases"]:
        q, state = lcg_values(heads * qr * hd, state)
        k, state = lcg_values(heads * sr * hd, state)
        v, state = lcg_values(heads * sr * hd, state)
        q, k, v = q.reshape(heads, qr, hd), k.reshape(heads, sr, hd), v.reshape(heads, sr, hd)
        expected = O.attention_materialized(q, k, v)
        np.testing.assert_allclose(O.attention(q, k, v), expected, atol=1e-5)
        np.testing.assert_allclose(O.attention(q, k, v, O.NATIVE), expected, atol=1e-4)
        # And against float64 (the materialized form itself is checked, not just retyped).
        s = np.einsum("hqd,hkd->hqk", q.astype(np.float64), k.astype(np.float64)) / math.sqrt(hd)
        p = np.exp(s - s.max(-1, keepdims=True))
        ref = np.einsum("hqk,hkd->hqd", p / p.sum(-1, keepdims=True), v.astype(np.float64))
        np.testing.assert_allclose(expected, ref, atol=1e-5)


def test_online_attention_long_sources_cross_tiles():
    rng = np.random.default_rng(5)
    for sr in (127, 128, 129, 1000):
        q, k, v = (f32(rng.normal(size=(2, 3, 64)) * 2), f32(rng.normal(size=(2, sr, 64))),
                   f32(rng.normal(size=(2, sr, 64))))
        np.testing.assert_allclose(O.attention(q, k, v), O.attention_materialized(q, k, v), atol=1e-5)


def test_uniform_and_peaked_scores():
    v = f32([1, 2, 3, 4]).reshape(1, 2, 2)
    for case in KA["uniform_peaked"]:
        q, k = f32(case["query"]).reshape(1, 1, 2), f32(case["key"]).reshape(1, 2, 2)
        np.testing.assert_allclose(O.attention(q, k, v), O.attention_materialized(q, k, v), atol=1e-5)
    np.testing.assert_allclose(O.attention(f32([0, 0]).reshape(1, 1, 2), f32([0, 0, 0, 0]).reshape(1, 2, 2), v).ravel(),
                               [2, 3], atol=1e-6)


def test_aggregation_closed_form():
    c = KA["aggregation"]
    logits = f32(c["logits"]).reshape(c["shape"])
    perms = np.array(c["permutations"], np.uint64).reshape(2, 3)
    members = np.array(c["members"], np.float64)

    def sm(x, t):
        e = np.exp(np.asarray(x, np.float64) / t)
        return e / e.sum()

    for t, avg in c["options"]:
        expected = sm(members.mean(0), t) if avg else (sm(members[0], t) + sm(members[1], t)) / 2
        np.testing.assert_allclose(O.aggregate(logits, perms, t, avg).ravel(), expected, atol=c["tolerance"])
    for t in c["invalid_temperatures"]:
        with pytest.raises(ValueError):
            O.aggregate(logits, perms, float(t), True)


def _levels(k):
    return (np.arange(1, k + 1, dtype=np.float64) / (k + 1)).astype(np.float32).astype(np.float64)


def test_quantile_linear_and_exponential_tails():
    c = KA["linear_quantiles"]
    k = c["k"]
    lv = _levels(k)
    assert abs(lv[0] - KA["quantile_levels"]["first"]) < 1e-7 and abs(lv[-1] - 0.999) < 1e-7
    assert abs(lv[499] - 0.5) < 1e-7
    row = f32(10 * lv - 5)[::-1].copy()
    mean, quant = O.regression_summary(row.reshape(1, 1, k), [0.5] + c["alphas"])
    assert abs(mean[0]) < c["tolerance"] and abs(quant[0, 0]) < c["tolerance"]
    np.testing.assert_allclose(quant[0, 1:], c["quantiles"], atol=c["tolerance"])
    t = KA["exponential_tail"]
    row = f32(np.log(lv))
    _, quant = O.regression_summary(np.stack([row, row]).reshape(2, 1, k), [t["alpha"]])
    assert abs(float(quant[0, 0]) - t["expected"]) < t["tolerance"]


def test_quantile_variance_raw_and_closed_forms():
    """quantiles.rs:224-251: the unbiased variance of Q(alpha) = 10 alpha - 5
    over the levels; sorted raw quantiles; float64 closed forms on random rows."""
    c = KA["linear_quantiles"]
    k = c["k"]
    lv = _levels(k)
    row = f32(10 * lv - 5)[::-1].copy()
    mean, var, quant, raw = O.regression_outputs(row.reshape(1, 1, k), [0.25, 0.5, 0.75])
    m = lv.sum() / k
    assert abs(float(var[0]) - (100 * (lv - m) ** 2).sum() / (k - 1)) < 1e-4
    np.testing.assert_array_equal(raw[0], np.sort(row))
    np.testing.assert_allclose(quant[0], [-2.5, 0.0, 2.5], atol=1e-5)
    x = np.random.default_rng(5).normal(size=(3, 4, 37)).astype(np.float32)
    mean, var, quant, raw = O.regression_outputs(x, [])
    s = np.sort(x.astype(np.float64), axis=-1)
    np.testing.assert_allclose(mean, s.mean(-1).mean(0), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(var, s.var(-1, ddof=1).mean(0), rtol=1e-5)
    np.testing.assert_allclose(raw, s.mean(0), rtol=1e-6, atol=1e-7)
    assert quant.shape == (4, 0)


def test_quantile_sort_follows_total_order():
    """f32::total_cmp: -NaN first, +NaN last. (Raw sums start at +0.0, as the
    reference's do, so both zeros come out as +0.0.)"""
    neg_nan = np.array([0xFFC00000], np.uint32).view(np.float32)[0]
    row = np.array([1.0, np.nan, -0.0, 0.0, -np.inf, neg_nan, 3.0, -2.0], np.float32)
    _, _, _, raw = O.regression_outputs(row.reshape(1, 1, -1), [])
    bits = raw[0].view(np.uint32)
    assert bits[0] == 0xFFC00000 and np.isneginf(raw[0, 1]) and raw[0, 2] == -2.0
    assert bits[3] == 0 and bits[4] == 0 and list(raw[0, 5:7]) == [1.0, 3.0] and np.isnan(raw[0, 7])
