"""TabICL preprocessing on the GPU through the C ABI: the f64 fit and
transform kernels against the reference's golden fixtures (SciPy /
scikit-learn Yeo-Johnson, TabICL 2.1.1's rows) and the f64 oracle, the
overflow fallback, and raw-X prediction of the fitted model against the
oracle pipeline (oracle preprocessing + the oracle model on the CPU)."""

import ctypes
import json
import os

import numpy as np
import pytest

import oracle as O
import preprocess_oracle as PO
from ironicl_amd import estimators, hip
from ironicl_amd import preprocess as pp
from ironicl_amd import tabicl
from ironicl_amd.fitted import FittedModel
from ironicl_amd.tabicl import aggregate_classifier_probabilities

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "preprocessing")
ATOL, RTOL = 1e-5, 1e-4


def fixture(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


@pytest.fixture(scope="module")
def device():
    return hip.Device(0)


def close(actual, expected, tol, what):
    assert abs(actual - expected) <= tol * (1 + abs(expected)), f"{what}: {actual} vs {expected}"


def gpu_power_fit(device, x):
    x = np.ascontiguousarray(x, dtype=np.float64)
    rows, cols = x.shape
    lms = np.zeros((3, cols))
    fitted = np.zeros((rows, cols))
    hip.check(hip.lib().irx_test_power_fit(device.handle, x.ctypes.data, rows, cols, lms.ctypes.data,
                                           fitted.ctypes.data))
    return lms, fitted


def test_power_fit_matches_scipy_and_scikit_learn(device):
    f = fixture("yeo_johnson.json")
    for case in f["normmax"]:
        x = np.array(case["x"], np.float64).reshape(-1, 1)
        lms, _ = gpu_power_fit(device, x)
        close(lms[0, 0], case["lambda"], 1e-7, f"{case['name']} lambda")
    for case in f["power_transformer"]:
        cols = case["columns"]
        x = np.array(case["x"], np.float64).reshape(-1, cols)
        lms, fitted = gpu_power_fit(device, x)
        expect = np.array(case["fit_transform"]).reshape(-1, cols)
        for c in range(cols):
            close(lms[0, c], case["lambdas"][c], 1e-7, "lambda")
            close(lms[1, c], case["mean"][c], 1e-7, "mean")
            close(lms[2, c], case["scale"][c], 1e-7, "scale")
        assert np.all(np.abs(fitted - expect) <= 1e-7 * (1 + np.abs(expect)))


OPTIONS = pp.PreprocessOptions(8, 42, ("none", "power"), 4.0)


def test_pipeline_matches_tabicl(device):
    f = fixture("preprocessing.json")
    x, q, case = np.array(f["training"]), np.array(f["query"]), f["cases"][0]
    p = pp.Preprocessor.fit(OPTIONS, x, f["labels"], device)
    assert p.group_methods == case["group_names"] and p.classes == case["classes_"]
    assert p.feature_mask.tolist() == case["feature_mask_"]
    assert p.member_groups == case["ensemble_groups_"]
    assert p.feature_permutations == case["feature_permutations_"]
    assert p.class_permutations == case["class_permutations_"]
    for data, key in ((x, "training_groups"), (q, "query_groups")):
        got = p.transform(data)
        for g, expected in enumerate(case[key]):
            e = np.array(expected)
            assert np.all(np.abs(got[g] - e) <= 2e-6 + 2e-6 * np.abs(e)), (key, g)
    members = p.member_rows(q)
    groups = p.transform(q)
    for b, (g, order) in enumerate(zip(p.member_groups, p.feature_permutations)):
        np.testing.assert_array_equal(members[b], groups[g][:, order])


def skewed_data(rows, seed):
    rng = np.random.default_rng(seed)
    cols = [rng.standard_normal(rows), np.exp(rng.standard_normal(rows) * 1.5),      # normal, log-normal
            -np.exp(rng.standard_normal(rows)), rng.standard_normal(rows) ** 3 * 5,  # negative, heavy tails
            np.full(rows, 3.25), rng.integers(0, 4, rows).astype(float),              # constant (dropped), ints
            np.where(rng.random(rows) < 0.5, 0.0, 1.0), rng.uniform(-1e3, 1e3, rows),  # two values, wide
            np.r_[rng.standard_normal(rows - 3), [40.0, -35.0, 60.0]]]                 # outliers
    return np.stack(cols, axis=1)


@pytest.mark.parametrize("rows", [50, 3000])
def test_fit_and_transform_match_the_oracle(device, rows):
    x = skewed_data(rows, rows)
    y = (np.arange(rows) % 3).astype(np.int64)
    p = pp.Preprocessor.fit(OPTIONS, x, y, device)
    kept = p.kept
    assert 4 not in kept
    want = PO.fit(x, kept, p.group_methods, 4.0)
    for g, method in enumerate(p.group_methods):
        count = 9 if method == "power" else 6
        got, exp = p.statistics[g, :count], want[g, :count]
        tol = np.full(count, 1e-10)
        if method == "power":
            tol[6:] = 1e-6  # lambda along fminbound's path; the power mean and scale follow it
            tol[4:6] = 1e-6
        assert np.all(np.abs(got - exp) <= tol[:, None] * (1 + np.abs(exp))), (method, got - exp)
    q = skewed_data(257, rows + 1)
    q[:, 4] = 1.0
    got = p.transform(q)
    for g, method in enumerate(p.group_methods):
        e = PO.transform_group(q, kept, method, p.statistics[g])
        assert np.all(np.abs(got[g] - e) <= 2e-6 + 2e-6 * np.abs(e)), method


def test_f32_input_is_its_f64_value(device):
    x = skewed_data(400, 5).astype(np.float32)
    y = np.arange(400) % 2
    a = pp.Preprocessor.fit(OPTIONS, x, y, device)
    b = pp.Preprocessor.fit(OPTIONS, x.astype(np.float64), y, device)
    np.testing.assert_array_equal(a.statistics, b.statistics)
    np.testing.assert_array_equal(a.member_rows(x[:30]), b.member_rows(x[:30].astype(np.float64)))


def overflow_preprocessor(device):
    st = np.array([0.0, 1.0, -1.0, 0.25, -1e30, 1e30, 200.0, 0.0, 1.0]).reshape(1, 9, 1)
    p = pp.Preprocessor(np.array([True]), ["power"], st, [0], [[0]], [[0, 1]], "int", [0, 1])
    p.attach(device)
    return p


def test_overflow_clips_the_whole_chunk(device):
    """preprocess.rs:866-884 on the GPU: 51^200 overflows, so its chunk is
    clipped to the training range, including 0.5, which alone would not be."""
    p = overflow_preprocessor(device)
    t = lambda v, chunk=None: p.transform(np.array(v, np.float64).reshape(-1, 1), chunk)[0, :, 0]
    batch = t([50.0, 0.5])
    np.testing.assert_array_equal(batch, t([0.25, 0.25]))
    assert t([0.5])[0] != batch[1]
    t([1e6])
    # Chunks of one row: only the overflowing row's chunk is clipped.
    per_row = t([50.0, 0.5], chunk=1)
    assert per_row[0] == batch[0] and per_row[1] == t([0.5])[0]
    oracle = PO.transform_group(np.array([[50.0], [0.5]]), [0], "power", p.statistics[0])
    np.testing.assert_allclose(batch, oracle[:, 0], rtol=1e-6)


def test_transform_errors(device):
    p = overflow_preprocessor(device)
    with pytest.raises(ValueError, match="finite"):
        p.transform(np.array([[np.nan]]))
    with pytest.raises(ValueError, match="features"):
        p.transform(np.zeros((2, 3)))
    with pytest.raises(ValueError, match="nonconstant"):
        pp.Preprocessor.fit(OPTIONS, np.ones((5, 3)), [0, 1, 0, 1, 0], device)
    with pytest.raises(ValueError, match="2..10 classes"):
        pp.Preprocessor.fit(OPTIONS, skewed_data(20, 1), [0] * 20, device)


# ---- the fitted model: raw X to probabilities ----

@pytest.fixture(scope="module")
def clf(device, clf_weights):
    return tabicl.Executor("classifier", clf_weights, device)


@pytest.fixture(scope="module")
def clf_oracle(clf_weights):
    O.set_threads(16)
    return O.OracleModel("classifier", clf_weights, O.EXACT)


def raw_classification(seed=3):
    rng = np.random.default_rng(seed)
    x = skewed_data(220, seed)
    score = x[:, 0] + 0.5 * np.log1p(x[:, 1]) - 0.2 * x[:, 3]
    y = np.array(["ant", "bee", "cat"])[np.digitize(score, np.quantile(score, [0.33, 0.66]))]
    xq = skewed_data(90, seed + 100)
    xq[:, 4] = rng.standard_normal(90)  # a training-constant column varies at prediction: still dropped
    return x, y, xq


def oracle_probabilities(p: pp.Preprocessor, model, x, y, xq):
    """The oracle pipeline: oracle statistics and transforms, member rows and
    targets as fitted.rs builds them, the oracle model's context and logits."""
    kept = p.kept
    stats = PO.fit(x, kept, p.group_methods, 4.0)

    def members(data):
        groups = [PO.transform_group(data, kept, m, stats[g]) for g, m in enumerate(p.group_methods)]
        return np.stack([groups[g][:, order] for g, order in zip(p.member_groups, p.feature_permutations)])

    codes = p.encode_labels(y)
    targets = np.stack([np.asarray(order, np.float32)[codes] for order in p.class_permutations])
    ctx = model.build_context(members(x), targets)
    logits = model.predict_cached(ctx, members(xq))[:, :, : len(p.classes)]
    return logits, aggregate_classifier_probabilities(logits, np.asarray(p.class_permutations), 0.9, True)


def test_raw_x_probabilities_match_the_oracle_pipeline(clf, clf_oracle):
    x, y, xq = raw_classification()
    fm = FittedModel.fit(clf, x, y, OPTIONS)
    gpu_logits = fm._logits(xq)[:, :, :3]
    cpu_logits, cpu_proba = oracle_probabilities(fm.preprocessor, clf_oracle, x, y, xq)
    err = np.abs(gpu_logits - cpu_logits) - (ATOL + RTOL * np.abs(cpu_logits))
    assert err.max() <= 0, np.abs(gpu_logits - cpu_logits).max()
    proba = fm.predict_proba(xq)
    np.testing.assert_allclose(proba, cpu_proba, atol=1e-5)
    assert np.array_equal(proba.argmax(1), cpu_proba.argmax(1))
    assert set(fm.predict(xq)) <= {"ant", "bee", "cat"}


def test_saved_fit_reloads_and_predicts_identically(clf):
    x, y, xq = raw_classification(4)
    fm = FittedModel.fit(clf, x, y, OPTIONS)
    want = fm.predict_proba(xq)
    irprep, ircntxt = fm.preprocessor_bytes(), fm.context_bytes()
    np.testing.assert_array_equal(FittedModel.load(clf, irprep, ircntxt).predict_proba(xq), want)
    np.testing.assert_array_equal(FittedModel.load(clf, irprep, training=(x, y)).predict_proba(xq), want)
    other = FittedModel.fit(clf, x, y, pp.PreprocessOptions(4, 42, ("none", "power"), 4.0))
    with pytest.raises(ValueError, match="does not match its preprocessing"):
        FittedModel.load(clf, irprep, other.context_bytes())


def test_estimators(clf, device, reg_weights):
    x, y, xq = raw_classification(5)
    est = estimators.TabICLClassifier(clf).fit(x, y)
    assert list(est.classes_) == ["ant", "bee", "cat"]
    np.testing.assert_allclose(est.predict_proba(xq).sum(1), 1.0, rtol=1e-5)
    assert est.predict(xq).shape == (90,)
    reg = tabicl.Executor("regressor", reg_weights, device)
    target = 100.0 + 20.0 * np.tanh(x[:, 0]) + 5.0 * x[:, 5]
    r = estimators.TabICLRegressor(reg, n_estimators=4).fit(x, target)
    mean = r.predict(xq)
    quantiles = r.predict(xq, "quantiles", alphas=[0.1, 0.9])
    assert mean.shape == (90,) and quantiles.shape == (90, 2)
    assert np.all(np.isfinite(mean))
    assert np.all(quantiles[:, 0] <= quantiles[:, 1] + 1e-4)
