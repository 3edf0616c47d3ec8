"""IRMODEL v1 (ironicl_amd/model_file.py) against the reference's format rules
(src/format/model.rs): its own tests (model.rs:948-1072) restated, the header
and directory laid out field by field, and the random-init weights written
as an executable artifact of the official profile."""

import hashlib
import struct

import numpy as np
import pytest

from ironicl_amd import manifest as mf
from ironicl_amd import model_file as M
from ironicl_amd import synthetic as S

CONFIG = (10, 999, 128, 3, 3, 4, 12)


def fixture_model():
    """The reference's fixture (model.rs:1050-1072): two zero tensors, listed out of order."""
    return bytes([1] * 32), CONFIG, [M.Tensor("b.bias", M.F32, (2,), bytes(8)),
                                     M.Tensor("a.weight", M.F32, (2, 2), bytes(16))]


def test_round_trip_and_corruption(tmp_path):
    path = tmp_path / "model.irmodel"
    written = M.write(path, M.encode(*fixture_model()))
    assert written == M.inspect(path)
    assert (written.tensor_count, written.parameter_count, written.tensor_bytes) == (2, 6, 24)
    assert written.profile == M.PROFILE_UNKNOWN and written.dtype_counts == {"f32": 2}
    data = bytearray(path.read_bytes())
    data[M.HEADER_BYTES] ^= 1
    path.write_bytes(bytes(data))
    with pytest.raises(M.ModelFileError, match="checksum"):
        M.inspect(path)
    assert [p.name for p in tmp_path.iterdir()] == ["model.irmodel"]  # no temporary left behind


def test_parsed_ranges_include_the_payload_offset():
    data = M.encode(*fixture_model())
    parsed = M.parse(data)
    _, dims, (a, b) = parsed.tensors["a.weight"]
    assert dims == (2, 2) and data[a:b] == bytes(16) and a >= M.HEADER_BYTES


def test_layout_field_by_field():
    data = M.encode(*fixture_model())
    assert data[:8] == b"IRMODEL\0"
    version, kind = struct.unpack_from("<II", data, 8)
    assert (version, kind) == (1, 1)
    assert data[16:48] == bytes([1] * 32)
    count, params, nbytes = struct.unpack_from("<IQQ", data, 48)
    assert (count, params, nbytes) == (2, 6, 24)
    assert struct.unpack_from("<7Q", data, 68) == CONFIG
    dir_len, pay_len, reserved = struct.unpack_from("<QQI", data, 124)
    assert reserved == 0 and 124 + 20 == M.HEADER_BYTES
    # Directory: names in bytewise order, each payload 64-byte aligned.
    pos = M.HEADER_BYTES
    entries = []
    for _ in range(2):
        name_len, rank, dtype, zero, offset, length = struct.unpack_from("<IHBBQQ", data, pos)
        pos += 24
        dims = struct.unpack_from(f"<{rank}Q", data, pos)
        pos += 8 * rank
        entries.append((data[pos:pos + name_len].decode(), dtype, zero, offset, length, dims))
        pos += name_len
    assert pos == M.HEADER_BYTES + dir_len
    assert entries == [("a.weight", 5, 0, 0, 16, (2, 2)), ("b.bias", 5, 0, 64, 8, (2,))]
    payload = (M.HEADER_BYTES + dir_len + 63) // 64 * 64
    assert data[M.HEADER_BYTES + dir_len:payload] == bytes(payload - M.HEADER_BYTES - dir_len)
    assert payload + pay_len + 32 == len(data) and pay_len == 72
    assert data[-32:] == hashlib.sha256(data[:-32]).digest()


def test_encoder_and_parser_reject_what_the_reference_rejects():
    sha, config, tensors = fixture_model()
    with pytest.raises(M.ModelFileError, match="hash is empty"):
        M.encode(bytes(32), config, tensors)
    with pytest.raises(M.ModelFileError, match="greater than zero"):
        M.encode(sha, (10, 0, 128, 3, 3, 4, 12), tensors)
    with pytest.raises(M.ModelFileError, match="duplicate"):
        M.encode(sha, config, tensors + [M.Tensor("a.weight", M.F32, (1,), bytes(4))])
    with pytest.raises(M.ModelFileError, match="bytes; expected"):
        M.encode(sha, config, [M.Tensor("a", M.F32, (3,), bytes(8))])

    good = M.encode(sha, config, tensors)

    def resealed(mutate):
        b = bytearray(good[:-32])
        mutate(b)
        return bytes(b) + hashlib.sha256(b).digest()

    cases = {
        "magic": lambda b: b.__setitem__(0, ord("X")),
        "version": lambda b: struct.pack_into("<I", b, 8, 2),
        "kind": lambda b: struct.pack_into("<I", b, 12, 2),
        "reserved bytes": lambda b: struct.pack_into("<I", b, 140, 1),
        "aggregate": lambda b: struct.pack_into("<Q", b, 52, 7),
        "reserved byte": lambda b: b.__setitem__(M.HEADER_BYTES + 7, 1),
        "dtype": lambda b: b.__setitem__(M.HEADER_BYTES + 6, 9),
        "offset or length": lambda b: struct.pack_into("<Q", b, M.HEADER_BYTES + 8, 3),
    }
    for what, mutate in cases.items():
        with pytest.raises(M.ModelFileError):
            M.parse(resealed(mutate))
    with pytest.raises(M.ModelFileError, match="truncated"):
        M.parse(good[:100])


def test_manifests_have_all_official_tensors():
    c, r = mf.tensor_manifest(mf.CLASSIFIER), mf.tensor_manifest(mf.REGRESSOR)
    assert len(c) == 391 and c["icl_predictor.tf_icl.blocks.11.linear2.weight"] == (512, 1024)
    assert c["row_interactor.tf_row.rope.freqs"] == (8,)
    assert len(r) == 347 and r["icl_predictor.decoder.2.weight"] == (999, 1024)
    assert r["col_embedder.y_encoder.weight"] == (128, 1)
    assert "icl_predictor.ln.bias" not in r and "row_interactor.tf_row.blocks.0.norm1.bias" not in r


@pytest.fixture(scope="module")
def classifier_file(tmp_path_factory):
    w = S.random_weights("classifier")
    path = tmp_path_factory.mktemp("models") / "classifier.irmodel"
    summary = M.write_model(path, "classifier", w)
    return w, path, summary


def test_random_init_classifier_is_an_official_profile(classifier_file):
    w, path, summary = classifier_file
    assert summary.profile == M.PROFILE_CLASSIFIER
    assert summary.source_sha256 == mf.CLASSIFIER_SHA256.hex()
    assert (summary.tensor_count, summary.parameter_count, summary.tensor_bytes) == (391, 27_552_258, 110_209_032)
    assert summary.config == CONFIG
    artifact = M.load(path)
    assert artifact.task == "classifier" and sorted(artifact.tensors) == sorted(w)
    for name, arr in w.items():
        assert artifact.tensors[name].dtype == np.float32
        np.testing.assert_array_equal(artifact.tensors[name], arr)


def test_random_init_regressor_loads_with_zero_layer_norm_biases(tmp_path):
    w = S.random_weights("regressor")
    path = tmp_path / "regressor.irmodel"
    summary = M.write_model(path, "regressor", w)
    assert summary.profile == M.PROFILE_REGRESSOR
    assert (summary.tensor_count, summary.parameter_count, summary.tensor_bytes) == (347, 28_544_991, 114_179_964)
    artifact = M.load(path)
    assert artifact.task == "regressor"
    assert not artifact.tensors["icl_predictor.ln.bias"].any()
    assert artifact.tensors["row_interactor.tf_row.blocks.2.norm2.bias"].shape == (128,)
    np.testing.assert_array_equal(artifact.tensors["icl_predictor.decoder.2.weight"],
                                  w["icl_predictor.decoder.2.weight"])


def test_only_official_models_execute(classifier_file, tmp_path):
    w, _, _ = classifier_file
    custom = M.encode_model("classifier", w, source_sha256=bytes([7] * 32))
    assert M.parse(custom).summary.profile == M.PROFILE_UNKNOWN
    with pytest.raises(M.ModelFileError, match="official TabICLv2"):
        M.from_bytes(custom)
    # A released hash on the other task's tensors is no profile either.
    wrong = M.encode_model("classifier", w, source_sha256=mf.REGRESSOR_SHA256)
    with pytest.raises(M.ModelFileError, match="official TabICLv2"):
        M.from_bytes(wrong)


def test_manifest_rejects_wrong_shape_unexpected_tensor_and_dtype(classifier_file):
    w, _, _ = classifier_file
    tensors = M.model_tensors("classifier", w)
    first = tensors[0]
    sha, config = mf.CLASSIFIER_SHA256, M.release_config("classifier")

    def parsed(ts):
        return M.parse(M.encode(sha, config, ts))

    # Same counts and bytes as the profile, so only the manifest check can refuse them.
    reshaped = [M.Tensor(first.name, M.F32, tuple(reversed(first.dims)) + (1,), first.data)] + tensors[1:]
    with pytest.raises(M.ModelFileError, match="shape"):
        M.validate_executable(parsed(reshaped))
    renamed = [M.Tensor("aaa.unexpected", M.F32, first.dims, first.data)] + tensors[1:]
    with pytest.raises(M.ModelFileError, match="unexpected"):
        M.validate_executable(parsed(renamed))
    with pytest.raises(M.ModelFileError, match="configuration"):
        M.validate_executable(M.parse(M.encode(sha, (10, 998, 128, 3, 3, 4, 12), tensors)))
