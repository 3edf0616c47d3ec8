"""The GPU path against closed forms and against the oracle at sharpened
attention, through the C ABI.

- Closed forms (tests/closed_forms.py): at the uniform and constant-query
  weight families every softmax is a formula of its sources, and the whole
  forward is a few float64 NumPy lines per stage written from the model's
  definition. The GPU build + cached prediction must equal it at the parity
  bar, for the classifier and the regressor, two estimators, a 40-row pass
  (the wide attention kernel) and a 12-row pass (the decode kernel). The
  oracle meets the same closed forms (test_oracle_closed_forms.py), and each
  plausible mistake listed there moves the logits far past the bar.
- Conditioned weights (tests/conditioned.py): the random-init model with every
  attention's query and key rows scaled so the softmaxes are sharp (median
  effective source count 0.1-0.2 of the sources) but not saturated. The GPU
  build + prediction against the oracle's uncached forward, end to end: on the
  1,024-row, 54-feature workload live, and on a 10,000-row, 20-feature context
  against the oracle logits committed in tests/golden/end_to_end.npz (written
  by tests/golden/make_end_to_end.py).
- The 10,000-row, 100-feature workload at the random-init weights, end to end
  against that fixture's oracle logits of all 1,024 test rows.

The bar: |gpu - want| <= 1e-5 + 1e-4 |want|, with identical argmax against
the oracle."""

import os
import sys

import numpy as np
import pytest

import closed_forms as CF
import conditioned as C
import oracle as O
from conftest import ROOT
from ironicl_amd import hip
from ironicl_amd import synthetic as S
from ironicl_amd import tabicl

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-5, 1e-4
N, H, Q = 96, 6, 40
FIXTURE = os.path.join(ROOT, "tests", "golden", "end_to_end.npz")


def assert_parity(gpu, want, what=""):
    gpu, want = np.asarray(gpu, np.float64), np.asarray(want, np.float64)
    err = np.abs(gpu - want) - (ATOL + RTOL * np.abs(want))
    worst = np.unravel_index(np.argmax(err), err.shape)
    assert err.max() <= 0, f"{what}: |gpu-want| {abs(gpu[worst] - want[worst]):.3e} at {worst}"


@pytest.fixture(scope="module")
def device():
    return hip.Device(0)


def two_estimators(task):
    """x [2, N, H], y [2, N], xt [2, Q, H]: different rows per estimator."""
    xs, ys, xts = [], [], []
    for e in range(2):
        rng = np.random.default_rng(30 + e)
        x = rng.normal(size=(N + Q, H)).astype(np.float32)
        if task == "classifier":
            y = ((np.arange(N) * 7 + e) % 4).astype(np.float32)
        else:
            y = rng.normal(size=N).astype(np.float32)
        xs.append(x[:N]), ys.append(y), xts.append(x[N:])
    return np.stack(xs), np.stack(ys), np.stack(xts)


@pytest.mark.parametrize("task", ["classifier", "regressor"])
@pytest.mark.parametrize("name", ["uniform", "constant_query"])
def test_gpu_equals_the_closed_form(device, clf_weights, reg_weights, task, name):
    base = clf_weights if task == "classifier" else reg_weights
    w = CF.uniform_weights(base) if name == "uniform" else CF.constant_query_weights(base, N)
    x, y, xt = two_estimators(task)
    print(f"closed form {name} {task}: B=2, N={N}, H={H}, Q={Q}", flush=True)
    ctx = tabicl.Executor(task, w, device).build_context(x, y)
    gpu = ctx.predict_raw(xt).logits
    decode = ctx.predict_raw(np.ascontiguousarray(xt[:, :12])).logits
    for e in range(2):
        want = CF.ClosedForm(task, w).forward(x[e].astype(np.float64), y[e].astype(np.float64), xt[e])
        assert_parity(gpu[e], want, f"{task} {name} estimator {e}, 40-row pass")
        assert_parity(decode[e], want[:12], f"{task} {name} estimator {e}, 12-row pass")


def test_conditioned_weights_end_to_end_1k(device, clf_weights):
    """1,024 training rows x 54 features, 7 classes, 8 test rows: one pass of
    eight rows, then calls of one and three rows (the small-pass kernels'
    one- and four-row forms) on peaked softmaxes."""
    w = C.conditioned_weights(clf_weights)
    x, y, xt, _ = S.workload_data(S.WORKLOADS["clf-1k"])
    print("conditioned weights, 1,024 x 54", flush=True)
    ctx = tabicl.Executor("classifier", w, device).build_context(x, y)
    gpu = ctx.predict_logits(xt).logits
    O.set_threads(16)
    cpu = O.OracleModel("classifier", w, O.EXACT).predict_uncached(x, y, xt)[..., :7]
    assert_parity(gpu, cpu, "conditioned clf-1k")
    assert np.array_equal(gpu.argmax(-1), cpu.argmax(-1))
    for rows in (slice(0, 1), slice(1, 4)):
        part = ctx.predict_logits(np.ascontiguousarray(xt[:, rows])).logits
        assert_parity(part, cpu[:, rows], f"conditioned clf-1k, rows {rows.start}-{rows.stop - 1}")


@pytest.fixture(scope="module")
def fixture():
    sys.path.insert(0, os.path.join(ROOT, "tests", "golden"))
    import make_end_to_end as E  # the inputs the fixture was made from

    with np.load(FIXTURE, allow_pickle=False) as f:
        data = {k: f[k] for k in f.files}
    return E, data


@pytest.mark.parametrize("name", ["clf10k", "cond10k"])
def test_10k_end_to_end_against_the_oracle_fixture(device, fixture, name):
    """The oracle's uncached forward, run where there is time for it (minutes
    of serial ICL attention), against the GPU's build + prediction of the same
    inputs, regenerated here and checked against the fixture's digest."""
    E, data = fixture
    (_, w, x, y, xt), = [c for c in E.cases() if c[0] == name]
    assert E.inputs_digest(w, x, y, xt) == str(data[f"{name}_inputs_sha256"]), "inputs differ from the fixture's"
    print(f"end to end {name}: {x.shape} -> {xt.shape[1]} test rows", flush=True)
    gpu = tabicl.Executor("classifier", w, device).build_context(x, y).predict_logits(xt).logits[0]
    cpu = data[f"{name}_logits"]
    classes = int(y.max()) + 1
    assert_parity(gpu[:, :classes], cpu[:, :classes], f"{name} logits")
    assert np.array_equal(gpu[:, :classes].argmax(-1), cpu[:, :classes].argmax(-1))
