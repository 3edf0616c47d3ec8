"""Parity at shapes whose tiles do not divide evenly, through the C ABI: a
three-estimator context of 12,345 training rows x 37 features (class shifts
and feature permutations per estimator, 300 test rows), checked on its first
and last estimator with the oracle's spot checks (column K/V of sampled
features from their whole column streams, ICL K/V of sampled training rows
by teacher forcing) and cached predictions; contexts of 1, 2 and 3 features
(the grouped triple (f+1, f+2, f+4) mod H repeats columns); the smallest
contexts the device builds (64 and 65 training rows). The bar is the north
star's: |gpu - cpu| <= 1e-5 + 1e-4 |cpu| with identical argmax."""

import numpy as np
import pytest

import oracle as O
from ironicl_amd import hip
from ironicl_amd import synthetic as S
from ironicl_amd import tabicl
from test_gpu_full_size import assert_parity, check_context, sample

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def device():
    return hip.Device(0)


@pytest.fixture(scope="module")
def clf(device, clf_weights):
    return tabicl.Executor("classifier", clf_weights, device)


@pytest.fixture(scope="module")
def oracle(clf_weights):
    O.set_threads(16)
    return O.OracleModel("classifier", clf_weights, O.EXACT)


def test_ragged_ensemble_spot_checks_and_predictions(clf, oracle):
    w = S.WORKLOADS["clf-200k"]
    x, y, xt, meta = S.workload_data(w, train_rows=12_345, test_rows=300, features=37)
    x, y, xt = x[:3], y[:3], xt[:3]
    st = clf.build_context(x, y, class_permutations=meta["class_permutations"][:3], download=True)
    gpu = st.predict_logits(xt).logits
    assert gpu.shape == (3, 300, 10)
    rows = sample(24, 300, 11)
    for e in (0, 2):
        ctx = tuple([t[e:e + 1] for t in part] for part in st.context)
        check_context(oracle, x[e:e + 1], y[e:e + 1], ctx, f"12345x37 estimator {e}", features=4, rows=12)
        cpu = oracle.predict_cached(ctx, np.ascontiguousarray(xt[e:e + 1, rows]))[..., :10]
        assert_parity(gpu[e:e + 1, rows], cpu, f"12345x37 estimator {e} logits")
        assert np.array_equal(gpu[e:e + 1, rows].argmax(-1), cpu.argmax(-1))


@pytest.mark.parametrize("features", [1, 2, 3])
def test_few_features(clf, oracle, features):
    rng = np.random.default_rng(features)
    x = rng.standard_normal((1, 700, features)).astype(np.float32)
    xt = rng.standard_normal((1, 40, features)).astype(np.float32)
    # Seven classes, each present (a linear labeller of one feature yields two).
    y = (np.argsort(rng.standard_normal(700)) % 7).astype(np.float32)[None]
    gpu = clf.build_context(x, y).predict_logits(xt).logits
    cpu = oracle.predict_uncached(x, y, xt)[..., :7]
    assert_parity(gpu, cpu, f"{features} features")
    assert np.array_equal(gpu.argmax(-1), cpu.argmax(-1))


@pytest.mark.parametrize("train_rows", [64, 65])
def test_smallest_contexts(clf, oracle, train_rows):
    w = S.WORKLOADS["clf-1k"]
    x, y, xt, _ = S.workload_data(w, train_rows=train_rows, test_rows=33, features=6)
    gpu = clf.build_context(x, y).predict_logits(xt).logits
    cpu = oracle.predict_uncached(x, y, xt)[..., :7]
    assert_parity(gpu, cpu, f"{train_rows} training rows")
    assert np.array_equal(gpu.argmax(-1), cpu.argmax(-1))
