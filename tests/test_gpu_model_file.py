"""Weights from an IRMODEL artifact through irx_weights_upload: a context
built and predicted from the file-loaded model equals, bit for bit, the one
from the same weights held in memory, for the classifier and the regressor;
the artifact's source SHA-256 is the model identity the context carries."""

import numpy as np
import pytest

from ironicl_amd import hip
from ironicl_amd import manifest as mf
from ironicl_amd import model_file as M
from ironicl_amd import tabicl
from test_oracle_model import reference_lcg_data

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("task", ["classifier", "regressor"])
def test_file_loaded_weights_predict_bitwise_as_in_memory(tmp_path, clf_weights, reg_weights, task):
    weights = clf_weights if task == "classifier" else reg_weights
    path = tmp_path / f"{task}.irmodel"
    M.write_model(path, task, weights)
    device = hip.Device(0)
    from_file = tabicl.Executor.from_model_file(path, device)
    in_memory = tabicl.Executor(task, weights, device)
    assert from_file.task == task and from_file.artifact.profile != M.PROFILE_UNKNOWN
    assert from_file.source_sha256 == M.official_sha256(task).hex()
    x, y, xt, shifts = reference_lcg_data(2, 240, 64, 5)
    if task == "regressor":
        y = np.ascontiguousarray(np.sin(np.arange(y.size, dtype=np.float32)).reshape(y.shape))
        shifts = None
    print(f"IRMODEL {task}: build 2 x 240 x 5, predict 64 rows", flush=True)
    a = from_file.build_context(x, y, class_permutations=shifts)
    b = in_memory.build_context(x, y, class_permutations=shifts)
    np.testing.assert_array_equal(a.predict_raw(xt).logits, b.predict_raw(xt).logits)
    assert a.metadata.model_sha256.hex() == M.official_sha256(task).hex()
    assert a.metadata.shape == b.metadata.shape
    assert hip.lib().irx_weights_bytes(from_file.handle) == hip.lib().irx_weights_bytes(in_memory.handle)
    assert len(mf.tensor_manifest(task)) == from_file.artifact.tensor_count
