"""The `run` path (src/main.rs:197-223) on the GPU: an IRMODEL artifact with
an IRQUERY bundle and the IRCNTXT context it was made for (cached), or with an
IRINPUT bundle (uncached), to logits that print and write as IRLOGITS."""

import numpy as np
import pytest

import oracle as O
from ironicl_amd import bundles, hip
from ironicl_amd import model_file as M
from ironicl_amd import run as R
from ironicl_amd import tabicl
from test_oracle_model import reference_lcg_data

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def artifacts(tmp_path_factory, clf_weights):
    d = tmp_path_factory.mktemp("run")
    model = d / "classifier.irmodel"
    M.write_model(model, "classifier", clf_weights)
    device = hip.Device(0)
    ex = tabicl.Executor.from_model_file(model, device)
    x, y, xt, shifts = reference_lcg_data(2, 240, 37, 5)
    ctx = ex.build_context(x, y, class_permutations=shifts)
    ctx.save_context(d / "context.irctx")
    query = bundles.StaticQueryBundle.new(ctx.metadata.model_sha256, ctx.metadata.context_sha256, xt)
    query.write(d / "query.irquery")
    return d, model, device, ctx, x, y, xt


def test_query_bundle_against_its_context(artifacts):
    d, model, device, ctx, x, y, xt = artifacts
    want = ctx.predict_logits(xt).logits
    got = R.run(model, d / "query.irquery", context=d / "context.irctx", logits_out=d / "out.irlogits",
                device=device)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(bundles.read_logits(d / "out.irlogits"), want)
    text = R.format_logits(got).splitlines()
    assert text[0] == f"shape: 2 37 {want.shape[2]}" and text[1].startswith("logits[0,0]: ")
    assert float(text[1].split()[1]) == pytest.approx(float(want[0, 0, 0]), rel=1e-8)
    probs = R.run(model, d / "query.irquery", context=d / "context.irctx", probabilities=True, device=device)
    np.testing.assert_array_equal(probs, ctx.predict_probabilities(xt))
    assert np.allclose(probs.sum(-1), 1.0, atol=1e-6)


def test_query_bundle_for_another_context_is_refused(artifacts):
    d, model, device, ctx, x, y, xt = artifacts
    other = bundles.StaticQueryBundle.new(ctx.metadata.model_sha256, bytes(31) + b"\1", xt)
    with pytest.raises(ValueError, match="identity"):
        ctx.predict_bundle(other)
    np.testing.assert_array_equal(ctx.predict_bundle(bundles.StaticQueryBundle.read(d / "query.irquery")).logits,
                                  ctx.predict_logits(xt).logits)


def test_input_bundle_uncached_against_the_oracle(artifacts, clf_weights):
    """IRINPUT: each estimator's first N of T rows train, the rest are
    predicted; against the oracle's uncached forward at the parity bar."""
    d, model, device, ctx, x, y, xt = artifacts
    n = 240
    bundle = bundles.InputBundle.new(2, n + 37, 5, n, np.concatenate([x, xt], axis=1), y)
    bundle.write(d / "input.irinput")
    got = R.run(model, d / "input.irinput", logits_out=d / "uncached.irlogits", device=device)
    assert got.shape[:2] == (2, 37)
    O.set_threads(8)
    cpu = O.OracleModel("classifier", clf_weights, O.EXACT).predict_uncached(x, y, xt)[..., :got.shape[2]]
    err = np.abs(got - cpu) - (1e-5 + 1e-4 * np.abs(cpu))
    assert err.max() <= 0, np.abs(got - cpu).max()
    assert np.array_equal(got.argmax(-1), cpu.argmax(-1))
    np.testing.assert_array_equal(bundles.read_logits(d / "uncached.irlogits"), got)
