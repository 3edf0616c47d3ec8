"""Regression summaries on the GPU (quantiles::summarize, quantiles.rs:80-213)
against the oracle's restatement, bit for bit: the kernel sorts in
f32::total_cmp order and repeats the reference's f64 operations in order, with
the logarithms taken on the host."""

import numpy as np
import pytest

import oracle as O
from ironicl_amd import hip, hipmem, tabicl

pytestmark = pytest.mark.gpu

NAMES = ("mean", "variance", "median", "quantiles", "raw_quantiles")


@pytest.fixture(scope="module")
def device():
    return hip.Device(0)


def levels(k):
    return (np.arange(1, k + 1, dtype=np.float64) / (k + 1)).astype(np.float32)


def summarize(device, decoded, alphas, names=NAMES):
    d = hipmem.DeviceArray.from_host(decoded)
    return tabicl.summarize_regression(device, d.ptr, decoded.shape, names, alphas)


def check(device, decoded, alphas):
    got = summarize(device, decoded, alphas)
    om, ov, oq, oraw = O.regression_outputs(decoded, list(alphas) + [0.5])
    for name, g, want in zip(NAMES, got, (om, ov, oq[:, -1], oq[:, :-1], oraw)):
        np.testing.assert_array_equal(g, want, err_msg=name)


@pytest.mark.parametrize("b,q,k", [(1, 5, 999), (3, 7, 999), (2, 3, 2), (1, 4, 5), (2, 2, 1000), (1, 2, 4096)])
def test_summary_matches_the_oracle_bitwise(device, b, q, k):
    rng = np.random.default_rng(b * 1000 + k)
    decoded = (rng.normal(size=(b, q, k)) * rng.uniform(0.1, 5.0, size=(b, q, 1))).astype(np.float32)
    lv = levels(k)
    alphas = [1e-4, 0.001, 0.05, 0.5, 0.95, 0.999, 0.9999, 0.0, 1.0, 1 / 3, float(lv[0]), float(lv[-1]),
              float(lv[k // 2])]
    check(device, decoded, alphas)


def test_summary_of_ties_signed_zeros_and_nan_rows(device):
    k = 999
    rng = np.random.default_rng(3)
    decoded = np.round(rng.normal(size=(2, 4, k)), 1).astype(np.float32)  # many ties
    decoded[0, 1, ::7] = -0.0
    decoded[1, 1, ::5] = 0.0
    decoded[0, 2, 10] = np.nan  # a NaN row, as the all-missing marker's
    decoded[:, 3] = np.float32(2.5)  # constant quantiles: zero variance, flat tails
    check(device, decoded, [0.01, 0.2, 0.5, 0.9, 0.99999])


def test_linear_quantiles_known_answers(device):
    """quantiles.rs:235-251 on the GPU."""
    k = 999
    lv = levels(k).astype(np.float64)
    row = (10 * lv - 5).astype(np.float32)[::-1].copy().reshape(1, 1, k)
    mean, var, median, quant, raw = summarize(device, row, [0.25, 0.75])
    assert abs(mean[0]) < 1e-5 and abs(median[0]) < 1e-5
    np.testing.assert_allclose(quant[0], [-2.5, 2.5], atol=1e-5)
    m = lv.sum() / k
    assert abs(float(var[0]) - (100 * (lv - m) ** 2).sum() / (k - 1)) < 1e-4
    np.testing.assert_array_equal(raw[0], np.sort(row[0, 0]))
    tail = np.log(levels(k).astype(np.float64)).astype(np.float32)
    (q,) = summarize(device, np.stack([tail, tail]).reshape(2, 1, k), [1e-4], ("quantiles",))
    assert abs(float(q[0, 0]) - np.log(1e-4)) < 1e-3


def test_summary_rejects_bad_requests(device):
    d = hipmem.DeviceArray.from_host(np.zeros((1, 2, 8), np.float32))
    lv = np.full(65, 0.5, np.float32)
    bad = [(1, 2, 1, None, 0), (1, 2, 4097, None, 0), (0, 2, 8, None, 0), (1, 2, 8, lv, 65),
           (1, 2, 8, np.array([np.nan], np.float32), 1)]
    for b, q, k, levels_, n in bad:
        st = hip.lib().irx_regression_summary(device.handle, d.ptr, b, q, k,
                                              hip.fptr(levels_) if levels_ is not None else None, n,
                                              None, None, None, None)
        assert st == hip.INVALID_ARGUMENT
    with pytest.raises(ValueError):
        tabicl.parse_regression_output("mode")
    with pytest.raises(ValueError):
        tabicl.parse_regression_output("quantiles", [float("nan")])
