"""The oracle's whole-model composition against closed forms (CPU only).

At the degenerate weights of tests/closed_forms.py every attention's softmax
is a formula of its sources alone, so the forward is a short float64 NumPy
computation written from the model's definition, independent of the oracle's
code and of tests/reference_np.py. The oracle's uncached forward
(cpu.rs:997-1065) and its build + cached prediction (cpu.rs:873-960,
2111-2850) must equal it within the parity bar, for the classifier and the
regressor; each plausible mistake listed in closed_forms.MUTATIONS moves the
closed form's logits far past that bar, so none of them could pass."""

import numpy as np
import pytest

import closed_forms as CF
import oracle as O
from ironicl_amd import synthetic as S

ATOL, RTOL = 1e-5, 1e-4
N, H, Q = 96, 6, 12


def within_bar(got, want, what):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    err = np.abs(got - want) - (ATOL + RTOL * np.abs(want))
    assert err.max() <= 0, f"{what}: max |diff| {np.abs(got - want).max():.3e}"


def case(task, seed=3):
    """One estimator: N training rows x H features, Q test rows, labels
    covering classes 0..3 (classifier) or continuous targets (regressor)."""
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(N + Q, H)).astype(np.float32)
    if task == "classifier":
        y = (np.arange(N) * 7 % 4).astype(np.float32)
    else:
        y = rng.normal(size=N).astype(np.float32)
    return x[:N], y, x[N:]


def family(name, weights):
    return CF.uniform_weights(weights) if name == "uniform" else CF.constant_query_weights(weights, N)


@pytest.fixture(scope="module")
def weights():
    return {"classifier": S.random_weights("classifier"), "regressor": S.random_weights("regressor")}


@pytest.mark.parametrize("task", ["classifier", "regressor"])
@pytest.mark.parametrize("name", ["uniform", "constant_query"])
def test_oracle_equals_the_closed_form(weights, task, name):
    w = family(name, weights[task])
    x, y, xt = case(task)
    want = CF.ClosedForm(task, w).forward(x.astype(np.float64), y.astype(np.float64), xt)
    O.set_threads(4)
    m = O.OracleModel(task, w, O.EXACT)
    uncached = m.predict_uncached(x[None], y[None], xt[None])[0]
    within_bar(uncached, want, f"{task} {name} uncached")
    cached = m.predict_cached(m.build_context(x[None], y[None]), xt[None])[0]
    within_bar(cached, want, f"{task} {name} build + cached")
    native = O.OracleModel(task, w, O.NATIVE).predict_uncached(x[None], y[None], xt[None])[0]
    within_bar(native, want, f"{task} {name} native math")


@pytest.mark.parametrize("task", ["classifier"])
def test_closed_forms_are_not_flat(weights, task):
    """The two families differ from each other and from the model at its own
    weights: the constant queries' softmaxes are not uniform."""
    x, y, xt = case(task)
    u = CF.ClosedForm(task, family("uniform", weights[task])).forward(x, y, xt)
    c = CF.ClosedForm(task, family("constant_query", weights[task])).forward(x, y, xt)
    assert np.abs(u).max() > 0.1 and np.abs(c - u).max() > 0.05


@pytest.fixture(scope="module")
def right_forwards(weights):
    x, y, xt = case("classifier")
    out = {}
    for name in ("uniform", "constant_query"):
        w = family(name, weights["classifier"])
        out[name] = (w, CF.ClosedForm("classifier", w).forward(x, y, xt))
    return out


@pytest.mark.parametrize("mutation", sorted(CF.MUTATIONS))
def test_each_planted_mistake_fails_the_bar(right_forwards, mutation):
    """A mistake that either family's closed form cannot tell from the right
    forward would pass these checks unseen; every one listed must move some
    logit by more than 100 times the parity bar."""
    x, y, xt = case("classifier")
    moved = 0.0
    for name, (w, right) in right_forwards.items():
        wrong = CF.ClosedForm("classifier", w, mutation).forward(x, y, xt)
        moved = max(moved, np.abs(wrong - right).max())
    assert moved > 100 * (ATOL + RTOL), f"{CF.MUTATIONS[mutation]}: logits move by only {moved:.2e}"
