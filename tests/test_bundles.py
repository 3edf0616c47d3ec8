"""IRINPUT / IRQUERY / IRLOGITS readers and writers (ironicl_amd/bundles.py):
the reference's own format tests restated (src/format/query_bundle.rs:155-206,
src/format/input_bundle.rs:449-495), the layouts pinned by bytes packed here
independently from the documented fields (docs/validation.md:168-179), and the
reader's rejections."""

import hashlib
import struct

import numpy as np
import pytest

from ironicl_amd import bundles as B


def seal(body: bytes) -> bytes:
    return body + hashlib.sha256(body).digest()


def query_fixture() -> bytes:
    """query_bundle.rs:158-173: B=1, Q=2, H=3, identities [1;32] / [2;32], x = 1..6."""
    body = b"IRQUERY\0" + struct.pack("<II", 1, 1) + bytes([1] * 32) + bytes([2] * 32)
    body += b"".join(struct.pack("<Q", v) for v in (1, 2, 3, 6))
    body += b"".join(struct.pack("<f", v) for v in (1.0, 2.0, 3.0, 4.0, 5.0, 6.0))
    return seal(body)


def test_decodes_checked_query():
    q = B.StaticQueryBundle.from_bytes(query_fixture())
    assert q.x.shape == (1, 2, 3)
    assert q.model_sha256 == bytes([1] * 32) and q.context_sha256 == bytes([2] * 32)
    np.testing.assert_array_equal(q.x.ravel(), np.arange(1, 7, dtype=np.float32))
    assert q.to_bytes() == query_fixture()


def test_rejects_corrupt_and_non_finite_queries():
    corrupt = bytearray(query_fixture())
    corrupt[112] ^= 1
    with pytest.raises(B.BundleError, match="checksum"):
        B.StaticQueryBundle.from_bytes(bytes(corrupt))
    nonfinite = bytearray(query_fixture()[:-32])
    nonfinite[112:116] = struct.pack("<f", float("nan"))
    with pytest.raises(B.BundleError, match="non-finite"):
        B.StaticQueryBundle.from_bytes(seal(bytes(nonfinite)))


@pytest.mark.parametrize("edit,match", [
    (lambda b: b[:8].__class__(b"IRQUERX\0") + b[8:], "magic"),
    (lambda b: b[:8] + struct.pack("<I", 2) + b[12:], "version or kind"),
    (lambda b: b[:16] + bytes(32) + b[48:], "identity is empty"),
    (lambda b: b[:80] + struct.pack("<Q", 0) + b[88:], "resource limits"),
    (lambda b: b[:104] + struct.pack("<Q", 7) + b[112:], "do not match"),
])
def test_query_header_rejections(edit, match):
    body = edit(query_fixture()[:-32])
    with pytest.raises(B.BundleError, match=match):
        B.StaticQueryBundle.from_bytes(seal(body))


def input_fixture() -> B.InputBundle:
    """input_bundle.rs:452-454: B=2, T=3, H=2, N=2, zero X, labels 0, 9, 1, 8."""
    return B.InputBundle.new(2, 3, 2, 2, np.zeros(12, np.float32), [0.0, 9.0, 1.0, 8.0])


def test_input_round_trip_is_deterministic():
    bundle = input_fixture()
    data = bundle.to_bytes()
    assert data == bundle.to_bytes()
    back = B.InputBundle.from_bytes(data)
    np.testing.assert_array_equal(back.x, bundle.x)
    np.testing.assert_array_equal(back.y_train, bundle.y_train)
    assert back.shape == (2, 3, 2, 2)
    # The documented layout, packed independently: an 80-byte header, X, y, SHA-256.
    head = b"IRINPUT\0" + struct.pack("<II8Q", 1, 1, 2, 3, 2, 2, 12, 4, 48, 16)
    want = seal(head + bytes(48) + struct.pack("<4f", 0.0, 9.0, 1.0, 8.0))
    assert data == want and len(head) == 80
    assert bundle.sha256() == hashlib.sha256(want[:-32]).hexdigest()


def test_input_rejects_corruption_and_truncation():
    corrupt = bytearray(input_fixture().to_bytes())
    corrupt[80] ^= 1
    with pytest.raises(B.BundleError):
        B.InputBundle.from_bytes(bytes(corrupt))
    data = input_fixture().to_bytes()
    with pytest.raises(B.BundleError):
        B.InputBundle.from_bytes(data[:-1])


def test_input_rejects_invalid_shapes_and_noninteger_labels():
    with pytest.raises(B.BundleError, match="T > N"):
        B.InputBundle.new(1, 2, 1, 2, np.zeros(2, np.float32), np.zeros(2, np.float32))
    with pytest.raises(B.BundleError, match="0..=9"):
        B.InputBundle.new(1, 2, 1, 1, np.zeros(2, np.float32), [1.5])
    with pytest.raises(B.BundleError, match="0..=9"):
        B.InputBundle.new(1, 2, 1, 1, np.zeros(2, np.float32), [10.0])
    with pytest.raises(B.BundleError, match="non-finite"):
        B.InputBundle.new(1, 2, 1, 1, [0.0, float("inf")], [1.0])
    malformed = bytearray(input_fixture().to_bytes()[:-32])
    malformed[24:32] = struct.pack("<Q", 2)  # T = 2 = N
    with pytest.raises(B.BundleError):
        B.InputBundle.from_bytes(seal(bytes(malformed)))
    malformed = bytearray(input_fixture().to_bytes()[:-32])
    malformed[48:56] = struct.pack("<Q", 11)  # X element count
    with pytest.raises(B.BundleError, match="element counts"):
        B.InputBundle.from_bytes(seal(bytes(malformed)))


def test_query_requests_reject_shape_and_non_finite_values():
    """QueryRequest::new (input_bundle.rs:489-494), as StaticQueryBundle.new."""
    B.StaticQueryBundle.new(bytes([1] * 32), bytes([2] * 32), np.zeros((1, 2, 3), np.float32))
    with pytest.raises(B.BundleError):
        B.StaticQueryBundle.new(bytes([1] * 32), bytes([2] * 32), np.zeros((2, 3), np.float32))
    x = np.zeros((1, 2, 3), np.float32)
    x[0, 1, 2] = np.nan
    with pytest.raises(B.BundleError, match="non-finite"):
        B.StaticQueryBundle.new(bytes([1] * 32), bytes([2] * 32), x)


def test_logits_layout_and_round_trip(tmp_path):
    logits = np.arange(2 * 3 * 4, dtype=np.float32).reshape(2, 3, 4) / 7
    data = B.encode_logits(logits)
    head = b"IRLOGITS" + struct.pack("<II4Q", 1, 1, 2, 3, 4, 24)
    assert len(head) == 48 and data == seal(head + logits.astype("<f4").tobytes())
    np.testing.assert_array_equal(B.decode_logits(data), logits)
    path = tmp_path / "x.irlogits"
    B.write_logits(path, logits)
    np.testing.assert_array_equal(B.read_logits(path), logits)
    with pytest.raises(B.BundleError, match="checksum"):
        B.decode_logits(data[:-1] + bytes([data[-1] ^ 1]))
    with pytest.raises(B.BundleError, match="metadata"):
        B.decode_logits(seal(head[:40] + struct.pack("<Q", 23) + logits.tobytes()))
    with pytest.raises(B.BundleError, match="length"):
        B.decode_logits(seal(head + logits.tobytes()[:-4]))


def test_files_round_trip(tmp_path):
    q = B.StaticQueryBundle.from_bytes(query_fixture())
    q.write(tmp_path / "q.irquery")
    assert (tmp_path / "q.irquery").read_bytes() == query_fixture()
    back = B.StaticQueryBundle.read(tmp_path / "q.irquery")
    np.testing.assert_array_equal(back.x, q.x)
    i = input_fixture()
    i.write(tmp_path / "i.irinput")
    assert B.InputBundle.read(tmp_path / "i.irinput").to_bytes() == i.to_bytes()
