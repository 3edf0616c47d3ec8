"""TabICL preprocessing on the CPU: the host logic (ensemble draws, labels,
mask, IRPREP) and the f64 oracle against the reference's golden fixtures,
copied as data into tests/golden/preprocessing/ from the reference's
tests/fixtures/: python_random.json (CPython 3.12 draws),
yeo_johnson.json (SciPy 1.18 yeojohnson_llf / yeojohnson_normmax,
scikit-learn 1.9 PowerTransformer) and preprocessing.json (TabICL 2.1.1's
preprocessed rows). The checks and tolerances follow the reference's own
tests (python_random.rs:107-160, yeo_johnson.rs:245-314,
preprocess.rs:760-957)."""

import json
import os
import random

import numpy as np
import pytest

import preprocess_oracle as PO
from ironicl_amd import preprocess as pp

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "preprocessing")


def fixture(name):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def ints(v):
    return [int(x) for x in v]


# ---- CPython's random, as the ensemble draws it ----

def test_draws_match_cpython():
    for case in fixture("python_random.json")["streams"]:
        rng = random.Random(int(case["seed"]))
        below = [rng._randbelow(n) for n in (1, 2, 3, 7, 8, 1000, 1 << 31, (1 << 32) + 1, (1 << 40) + 3, 1 << 63)]
        assert below == ints(case["randbelow"])
        assert [rng._randbelow(n) for n in (1, 2, 5, 100)] == ints(case["choice"])
        for n, expected in zip((0, 1, 2, 10, 100), case["shuffle"]):
            values = list(range(n))
            rng.shuffle(values)
            assert values == ints(expected)
        for (n, k), expected in zip(((1, 1), (6, 6), (50, 50), (1000, 3), (5000, 40)), case["sample"]):
            assert rng.sample(list(range(n)), k) == ints(expected)


def test_feature_shuffles_match_cpython():
    for case in fixture("python_random.json")["feature_shuffles"]:
        orders = pp.feature_orders(case["features"], case["estimators"], int(case["seed"]))
        assert len(orders) == case["count"]
        if "orders" in case:
            assert orders == [ints(o) for o in case["orders"]]
        else:
            state = 0xCBF29CE484222325
            for value in (v for o in orders for v in o):
                state = ((state ^ value) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
            assert f"{state:016x}" == case["digest"]


def literal_latin_square(features, seed):
    """TabICL's construction, O(H^3) (preprocess.rs:902-924)."""
    rng = random.Random(seed)
    indices = list(range(features))
    removed = []
    while len(indices) > 1:
        removed.append(indices.pop(rng._randbelow(len(indices))))
    square = [indices]
    for symbol in reversed(removed):
        square.append(list(square[0]))
        for i, row in enumerate(square):
            row.insert(i, symbol)
    rng.shuffle(square)
    transposed = [[row[c] for row in square] for c in range(features)]
    rng.shuffle(transposed)
    return transposed


def test_the_closed_form_is_the_square_tabicl_builds():
    for features in range(1, 40):
        for seed in (0, 1, 42, -3, 1 << 40):
            assert pp.feature_orders(features, 8, seed) == literal_latin_square(features, seed)


def test_one_member_keeps_the_feature_order_and_many_features_sample():
    assert pp.feature_orders(5, 1, 7) == [[0, 1, 2, 3, 4]]
    sampled = pp.feature_orders(4001, 3, 0)
    assert len(sampled) == 3 and sorted(sampled[2]) == list(range(4001))


# ---- the oracle against SciPy and scikit-learn ----

def close(actual, expected, tol, what):
    assert abs(actual - expected) <= tol * (1 + abs(expected)), f"{what}: {actual} vs {expected}"


def test_oracle_yeo_johnson_fit_matches_scipy():
    for case in fixture("yeo_johnson.json")["normmax"]:
        x = np.array(case["x"], dtype=np.float64)
        for at, expected in case["llf"]:
            close(PO.log_likelihood(x, at), expected, 1e-13, f"{case['name']} llf({at})")
        close(PO.normmax(x), case["lambda"], 1e-7, f"{case['name']} lambda")


def test_oracle_power_transformer_matches_scikit_learn():
    for case in fixture("yeo_johnson.json")["power_transformer"]:
        cols = case["columns"]
        x = np.array(case["x"], dtype=np.float64).reshape(-1, cols)
        q = np.array(case["query"], dtype=np.float64).reshape(-1, cols)
        fitted = np.array(case["fit_transform"]).reshape(-1, cols)
        transformed = np.array(case["transform"]).reshape(-1, cols)
        for c in range(cols):
            lam, mean, scale, values = PO.fit_power(x[:, c])
            close(lam, case["lambdas"][c], 1e-7, "lambda")
            close(mean, case["mean"][c], 1e-7, "mean")
            close(scale, case["scale"][c], 1e-7, "scale")
            for a, e in zip(values, fitted[:, c]):
                close(a, e, 1e-7, "fit_transform")
            for a, e in zip((PO.yeo_johnson(q[:, c], lam) - mean) / scale, transformed[:, c]):
                close(a, e, 1e-7, "transform")


# ---- the pipeline against TabICL 2.1.1 ----

OPTIONS = pp.PreprocessOptions(n_estimators=8, random_state=42, norm_methods=("none", "power"),
                               outlier_threshold=4.0)


def tabicl_case():
    f = fixture("preprocessing.json")
    return (np.array(f["training"], np.float64), np.array(f["query"], np.float64), f["labels"], f["cases"][0])


def test_host_ensemble_labels_and_mask_match_tabicl():
    x, _, labels, case = tabicl_case()
    kind, classes = pp.label_classes(labels)
    assert kind == "text" and classes == case["classes_"]
    assert pp.encode_labels(labels, kind, classes).tolist() == case["encoded_labels"]
    mask = np.any(x[1:] != x[0], axis=0)
    assert mask.tolist() == case["feature_mask_"]
    methods, groups, forders, corders = pp.ensemble(OPTIONS, int(mask.sum()), len(classes))
    assert methods == case["group_names"]
    assert groups == case["ensemble_groups_"]
    assert forders == case["feature_permutations_"]
    assert corders == case["class_permutations_"]


def test_oracle_rows_match_tabicl():
    x, q, labels, case = tabicl_case()
    kept = list(np.flatnonzero(np.any(x[1:] != x[0], axis=0)))
    stats = PO.fit(x, kept, case["group_names"], 4.0)
    for data, key in ((x, "training_groups"), (q, "query_groups")):
        for g, (method, expected) in enumerate(zip(case["group_names"], case[key])):
            got = PO.transform_group(data, kept, method, stats[g])
            e = np.array(expected, np.float64)
            assert np.all(np.abs(got - e) <= 2e-6 + 2e-6 * np.abs(e)), (key, g)


def test_oracle_overflow_clips_the_whole_batch():
    """preprocess.rs:866-884: 51^200 overflows, so the whole batch is clipped to
    the training range, including 0.5, which alone would not be."""
    st = np.array([0.0, 1.0, -1.0, 0.25, -1e30, 1e30, 200.0, 0.0, 1.0]).reshape(9, 1)
    t = lambda v: PO.transform_group(np.array(v).reshape(-1, 1), [0], "power", st)
    batch = t([50.0, 0.5])
    np.testing.assert_array_equal(batch, t([0.25, 0.25]))
    assert t([0.5])[0, 0] != batch[1, 0]
    t([1e6])  # clipped, so it no longer overflows


# ---- IRPREP ----

def fitted_preprocessor(regression=False):
    x, _, labels, case = tabicl_case()
    kept = list(np.flatnonzero(np.any(x[1:] != x[0], axis=0)))
    stats = PO.fit(x, kept, case["group_names"], 4.0)
    if regression:
        methods, groups, forders, corders = pp.ensemble(OPTIONS, len(kept), None)
        return pp.Preprocessor(np.array(case["feature_mask_"]), methods, stats, groups, forders, corders,
                               None, None, (1.5, 2.5))
    return pp.Preprocessor(np.array(case["feature_mask_"]), case["group_names"], stats, case["ensemble_groups_"],
                           case["feature_permutations_"], case["class_permutations_"], "text", case["classes_"])


def same(a: pp.Preprocessor, b: pp.Preprocessor):
    assert a.feature_mask.tolist() == b.feature_mask.tolist() and a.group_methods == b.group_methods
    np.testing.assert_array_equal(a.statistics, b.statistics)
    assert (a.member_groups, a.feature_permutations, a.class_permutations) == \
        (b.member_groups, b.feature_permutations, b.class_permutations)
    assert (a.label_kind, a.classes, a.target_scale) == (b.label_kind, b.classes, b.target_scale)


@pytest.mark.parametrize("regression", [False, True])
def test_irprep_round_trip(regression):
    p = fitted_preprocessor(regression)
    sha = bytes([7]) * 32
    data = pp.encode_irprep(p, sha)
    got_sha, q = pp.decode_irprep(data)
    assert got_sha == sha
    same(p, q)
    assert pp.encode_irprep(q, sha) == data


@pytest.mark.parametrize("kind,classes", [("int", [-3, 0, 7]), ("float", [-0.5, 2.0]), ("bool", [False, True])])
def test_irprep_label_kinds(kind, classes):
    p = fitted_preprocessor()
    c = len(classes)
    p.label_kind, p.classes = kind, classes
    p.class_permutations = [[(i - s) % c for i in range(c)] for s in range(len(p.member_groups))]
    got = pp.decode_irprep(pp.encode_irprep(p, bytes(32)))[1]
    assert got.label_kind == kind and got.classes == classes


def test_irprep_rejects_corruption():
    data = bytearray(pp.encode_irprep(fitted_preprocessor(), bytes([7]) * 32))
    bad = bytearray(data)
    bad[20] ^= 1
    with pytest.raises(ValueError, match="checksum"):
        pp.decode_irprep(bytes(bad))
    import hashlib

    def resign(b):
        b[-32:] = hashlib.sha256(bytes(b[:-32])).digest()
        return bytes(b)

    bad = bytearray(data)
    bad[8] = 2  # version
    with pytest.raises(ValueError, match="version"):
        pp.decode_irprep(resign(bad))
    bad = bytearray(data[:-32]) + b"\0" + bytes(32)
    with pytest.raises(ValueError, match="trailing"):
        pp.decode_irprep(resign(bad))
    bad = bytearray(data)
    bad[8 + 4 + 32 + 8] = 5  # the first feature-mask flag
    with pytest.raises(ValueError, match="invalid flag"):
        pp.decode_irprep(resign(bad))


def test_options_and_labels_are_validated():
    with pytest.raises(ValueError):
        pp.PreprocessOptions(n_estimators=0).validate()
    with pytest.raises(ValueError):
        pp.PreprocessOptions(norm_methods=("none", "none")).validate()
    with pytest.raises(ValueError):
        pp.PreprocessOptions(outlier_threshold=float("inf")).validate()
    with pytest.raises(ValueError, match="did not"):
        pp.encode_labels(["a", "z"], "text", ["a", "b"])
    with pytest.raises(ValueError, match="different label type"):
        pp.encode_labels([1, 2], "text", ["a", "b"])
