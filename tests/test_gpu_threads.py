"""The boundary's thread-safety contract, driven from host threads.

The reference's Predictor serializes calls with an internal Mutex and is
shared across threads (src/models/tabicl_v2/cuda/predictor.rs:104,234);
different predictors, and builds, may run at the same time. ctypes releases
the GIL for the duration of each C ABI call, so Python threads here call
irx_predictor_predict and irx_build concurrently. Every concurrent result must
be bitwise the sequential one."""

import threading

import numpy as np
import pytest

from ironicl_amd import hip
from ironicl_amd import tabicl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def clf(clf_weights):
    return tabicl.Executor("classifier", clf_weights, hip.Device(0))


def data(seed, n, h, q, classes=4):
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(1, n, h)).astype(np.float32)
    y = (rng.permutation(n) % classes).astype(np.float32)[None]
    xt = rng.normal(size=(1, q, h)).astype(np.float32)
    return x, y, xt


def run_threads(*targets):
    """Runs each callable on its own thread, released together; re-raises the
    first failure."""
    start = threading.Barrier(len(targets))
    errors = []

    def wrap(fn):
        def go():
            try:
                start.wait()
                fn()
            except BaseException as e:  # noqa: BLE001 - reported below
                errors.append(e)
        return go

    threads = [threading.Thread(target=wrap(t)) for t in targets]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in threads), "a thread did not finish"
    if errors:
        raise errors[0]


def test_two_threads_share_one_predictor(clf):
    """Calls of different sizes (one 600-row call is two passes) from two
    threads on one predictor serialize and give the sequential logits."""
    x, y, xt = data(1, 400, 7, 600)
    ctx = clf.build_context(x, y)
    calls = [xt[:, :7], xt, xt[:, 100:133], xt[:, :1], xt[:, 50:562]]
    want = [ctx.predict_raw(c).logits for c in calls]
    got = {0: [], 1: []}

    def worker(k):
        def go():
            for rep in range(3):
                order = range(len(calls)) if (k + rep) % 2 == 0 else reversed(range(len(calls)))
                for i in order:
                    got[k].append((i, ctx.predict_raw(calls[i]).logits))
        return go

    run_threads(worker(0), worker(1))
    for k in (0, 1):
        assert len(got[k]) == 3 * len(calls)
        for i, logits in got[k]:
            np.testing.assert_array_equal(logits, want[i])


def test_two_predictors_predict_concurrently(clf):
    """Two contexts of one device, each predicted from its own thread."""
    xa, ya, qa = data(2, 300, 5, 700)
    xb, yb, qb = data(3, 520, 11, 90)
    a, b = clf.build_context(xa, ya), clf.build_context(xb, yb)
    want_a, want_b = a.predict_raw(qa).logits, b.predict_raw(qb).logits
    out = {"a": [], "b": []}

    def on(ctx, q, key):
        def go():
            for _ in range(4):
                out[key].append(ctx.predict_raw(q).logits)
        return go

    run_threads(on(a, qa, "a"), on(b, qb, "b"))
    for logits in out["a"]:
        np.testing.assert_array_equal(logits, want_a)
    for logits in out["b"]:
        np.testing.assert_array_equal(logits, want_b)


def test_builds_and_predictions_run_concurrently(clf):
    """Two builds at once (one borrows the device's kept workspace, the other
    allocates its own) beside predictions on a third context."""
    xa, ya, qa = data(4, 350, 6, 40)
    xb, yb, qb = data(5, 610, 9, 40)
    xc, yc, qc = data(6, 260, 4, 300)
    want_a = clf.build_context(xa, ya).predict_raw(qa).logits
    want_b = clf.build_context(xb, yb).predict_raw(qb).logits
    c = clf.build_context(xc, yc)
    want_c = c.predict_raw(qc).logits
    got = {}

    def build(key, x, y, q):
        def go():
            for r in range(2):
                got[(key, r)] = clf.build_context(x, y).predict_raw(q).logits
        return go

    def predict():
        for r in range(6):
            got[("c", r)] = c.predict_raw(qc).logits

    run_threads(build("a", xa, ya, qa), build("b", xb, yb, qb), predict)
    for r in range(2):
        np.testing.assert_array_equal(got[("a", r)], want_a)
        np.testing.assert_array_equal(got[("b", r)], want_b)
    for r in range(6):
        np.testing.assert_array_equal(got[("c", r)], want_c)
