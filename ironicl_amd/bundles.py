"""The harness's request and result files: IRINPUT v1 classifier inputs,
IRQUERY v1 static-context queries and IRLOGITS v1 logits.

Byte layouts are the reference's, so files move between the two unchanged
(the interface is kept alike for that reason): all little-endian, FP32
row-major tensors, a SHA-256 trailer over every preceding byte.

    IRINPUT  (src/format/input_bundle.rs:14-26, 78-206)
        b"IRINPUT\\0" | version u32 = 1 | kind u32 = 1
        B, T, H, N, X elements, y elements, X bytes, y bytes   8 x u64
        X [B, T, H] | y_train [B, N] (labels 0..9) | SHA-256
    IRQUERY  (src/format/query_bundle.rs:11-110)
        b"IRQUERY\\0" | version u32 = 1 | kind u32 = 1
        model SHA-256 (32) | context SHA-256 (32)
        B, Q, H, X elements                                    4 x u64
        X [B, Q, H] | SHA-256
    IRLOGITS (docs/validation.md:174-179)
        b"IRLOGITS" | version u32 = 1 | kind u32 = 1
        B, test rows, classes, elements                        4 x u64
        logits [B, test rows, classes] | SHA-256

Readers check what the reference's readers check, in its order, with its
resource limits (512 MiB per file, B <= 4,096, rows <= 1,000,000,
H <= 65,536), and raise BundleError.
"""

from __future__ import annotations

import hashlib
import os
import struct
import tempfile
from dataclasses import dataclass

import numpy as np

INPUT_MAGIC, QUERY_MAGIC, LOGITS_MAGIC = b"IRINPUT\0", b"IRQUERY\0", b"IRLOGITS"
VERSION = KIND = 1
CHECKSUM_BYTES = 32
MAX_BUNDLE_BYTES = 512 * 1024 * 1024
MAX_ENSEMBLE_COUNT = 4096
MAX_ROWS = 1_000_000
MAX_FEATURE_COUNT = 65_536
_INPUT_HEADER = struct.Struct("<8sII8Q")   # 80 bytes
_QUERY_HEADER = struct.Struct("<8sII32s32s4Q")  # 112 bytes
_LOGITS_HEADER = struct.Struct("<8sII4Q")  # 48 bytes


class BundleError(ValueError):
    """A malformed, corrupt or invalid bundle (Error::InputBundle)."""


def _sealed(body: bytes) -> bytes:
    return body + hashlib.sha256(body).digest()


def _checked(data: bytes, header_bytes: int, what: str) -> None:
    if len(data) < header_bytes + CHECKSUM_BYTES:
        raise BundleError(f"{what} is truncated")
    if len(data) > MAX_BUNDLE_BYTES:
        raise BundleError(f"{what} exceeds the resource limit")
    if hashlib.sha256(data[:-CHECKSUM_BYTES]).digest() != data[-CHECKSUM_BYTES:]:
        raise BundleError(f"{what} checksum does not match")


def _read_file(path, what: str) -> bytes:
    try:
        size = os.path.getsize(path)
        if size > MAX_BUNDLE_BYTES:
            raise BundleError(f"{what} exceeds the resource limit")
        with open(path, "rb") as f:
            return f.read(MAX_BUNDLE_BYTES + 1)
    except OSError as e:
        raise BundleError(f"{what}: {e}") from None


def _write_file(path, data: bytes) -> None:
    """Writes atomically: a private temporary file next to `path`, synced and renamed."""
    directory = os.path.dirname(os.path.abspath(path))
    fd, tmp = tempfile.mkstemp(prefix=".bundle-", dir=directory)
    try:
        with os.fdopen(fd, "wb") as f:
            f.write(data)
            f.flush()
            os.fsync(f.fileno())
        os.replace(tmp, path)
    except BaseException:
        try:
            os.unlink(tmp)
        except OSError:
            pass
        raise


def _f32(values, shape) -> np.ndarray:
    a = np.ascontiguousarray(values, dtype=np.float32)
    if a.size != int(np.prod(shape)):
        raise BundleError("tensor lengths do not match dimensions")
    return a.reshape(shape)


@dataclass(eq=False)
class InputBundle:
    """Preprocessed classifier tensors of one request: x [B, T, H] whose first
    N rows per estimator are the training rows, y_train [B, N] (InputBundle,
    input_bundle.rs:28-75)."""

    x: np.ndarray
    y_train: np.ndarray

    @classmethod
    def new(cls, ensemble_count: int, total_rows: int, feature_count: int, training_rows: int, x,
            y_train) -> "InputBundle":
        b, t, h, n = ensemble_count, total_rows, feature_count, training_rows
        if (not 0 < b <= MAX_ENSEMBLE_COUNT or not 0 < t <= MAX_ROWS or not 0 < h <= MAX_FEATURE_COUNT
                or not 0 < n <= MAX_ROWS or t <= n):
            raise BundleError(f"invalid dimensions B={b}, T={t}, H={h}, N={n}; require B, H, N > 0, T > N, "
                              "and resource limits")
        x, y = _f32(x, (b, t, h)), _f32(y_train, (b, n))
        if _INPUT_HEADER.size + 4 * (x.size + y.size) + CHECKSUM_BYTES > MAX_BUNDLE_BYTES:
            raise BundleError("bundle exceeds the resource limit")
        if not np.isfinite(x).all():
            raise BundleError("X contains a non-finite value")
        if not (np.isfinite(y) & (y >= 0) & (y <= 9) & (y == np.floor(y))).all():
            raise BundleError("y_train labels must be finite integer-valued FP32 values in 0..=9")
        return cls(x, y)

    @property
    def shape(self) -> tuple[int, int, int, int]:
        b, t, h = self.x.shape
        return b, t, h, self.y_train.shape[1]

    def to_bytes(self) -> bytes:
        b, t, h, n = self.shape
        head = _INPUT_HEADER.pack(INPUT_MAGIC, VERSION, KIND, b, t, h, n, self.x.size, self.y_train.size,
                                  4 * self.x.size, 4 * self.y_train.size)
        return _sealed(head + self.x.astype("<f4").tobytes() + self.y_train.astype("<f4").tobytes())

    @classmethod
    def from_bytes(cls, data: bytes) -> "InputBundle":
        _checked(data, _INPUT_HEADER.size, "bundle")
        magic, version, kind, b, t, h, n, xe, ye, xb, yb = _INPUT_HEADER.unpack_from(data)
        if magic != INPUT_MAGIC:
            raise BundleError("bundle magic does not match")
        if version != VERSION:
            raise BundleError(f"bundle version {version} is unsupported; expected {VERSION}")
        if kind != KIND:
            raise BundleError("bundle kind is not a classifier input")
        if (not 0 < b <= MAX_ENSEMBLE_COUNT or not 0 < t <= MAX_ROWS or not 0 < h <= MAX_FEATURE_COUNT
                or not 0 < n <= MAX_ROWS or t <= n):
            raise BundleError(f"invalid dimensions B={b}, T={t}, H={h}, N={n}; require B, H, N > 0, T > N, "
                              "and resource limits")
        if xe != b * t * h or ye != b * n:
            raise BundleError("declared tensor element counts do not match dimensions")
        if xb != 4 * xe or yb != 4 * ye:
            raise BundleError("declared tensor byte lengths do not match element counts")
        if len(data) != _INPUT_HEADER.size + xb + yb + CHECKSUM_BYTES:
            raise BundleError("bundle section lengths do not match whole-file length")
        x = np.frombuffer(data, "<f4", xe, _INPUT_HEADER.size)
        y = np.frombuffer(data, "<f4", ye, _INPUT_HEADER.size + xb)
        return cls.new(b, t, h, n, x, y)

    @classmethod
    def read(cls, path) -> "InputBundle":
        return cls.from_bytes(_read_file(path, "bundle"))

    def write(self, path) -> None:
        _write_file(path, self.to_bytes())

    def sha256(self) -> str:
        """Lowercase hex SHA-256 of the encoded bundle (its trailer)."""
        return self.to_bytes()[-CHECKSUM_BYTES:].hex()


@dataclass(eq=False)
class StaticQueryBundle:
    """Preprocessed queries x [B, Q, H] for one exact static context, with the
    model and context identities they require (StaticQueryBundle,
    query_bundle.rs:23-147)."""

    model_sha256: bytes
    context_sha256: bytes
    x: np.ndarray

    @classmethod
    def new(cls, model_sha256: bytes, context_sha256: bytes, x) -> "StaticQueryBundle":
        x = np.ascontiguousarray(x, dtype=np.float32)
        if len(model_sha256) != 32 or len(context_sha256) != 32:
            raise BundleError("static query: identities are 32-byte SHA-256 digests")
        if model_sha256 == bytes(32) or context_sha256 == bytes(32):
            raise BundleError("static query: query bundle identity is empty")
        if x.ndim != 3:
            raise BundleError("static query: queries must be [B, Q, H]")
        b, q, h = x.shape
        if not 0 < b <= MAX_ENSEMBLE_COUNT or not 0 < q <= MAX_ROWS or not 0 < h <= MAX_FEATURE_COUNT:
            raise BundleError("static query: query bundle dimensions are outside the resource limits")
        if not np.isfinite(x).all():
            raise BundleError("static query: query bundle contains a non-finite value")
        return cls(bytes(model_sha256), bytes(context_sha256), x)

    def to_bytes(self) -> bytes:
        b, q, h = self.x.shape
        head = _QUERY_HEADER.pack(QUERY_MAGIC, VERSION, KIND, self.model_sha256, self.context_sha256, b, q, h,
                                  self.x.size)
        return _sealed(head + self.x.astype("<f4").tobytes())

    @classmethod
    def from_bytes(cls, data: bytes) -> "StaticQueryBundle":
        if len(data) < _QUERY_HEADER.size + CHECKSUM_BYTES or len(data) > MAX_BUNDLE_BYTES:
            raise BundleError("static query: query bundle length is outside the resource limit")
        if hashlib.sha256(data[:-CHECKSUM_BYTES]).digest() != data[-CHECKSUM_BYTES:]:
            raise BundleError("static query: query bundle checksum does not match")
        magic, version, kind, model, context, b, q, h, elements = _QUERY_HEADER.unpack_from(data)
        if magic != QUERY_MAGIC:
            raise BundleError("static query: query bundle magic does not match")
        if version != VERSION or kind != KIND:
            raise BundleError("static query: query bundle version or kind is unsupported")
        if model == bytes(32) or context == bytes(32):
            raise BundleError("static query: query bundle identity is empty")
        if not 0 < b <= MAX_ENSEMBLE_COUNT or not 0 < q <= MAX_ROWS or not 0 < h <= MAX_FEATURE_COUNT:
            raise BundleError("static query: query bundle dimensions are outside the resource limits")
        if elements != b * q * h or len(data) != _QUERY_HEADER.size + 4 * b * q * h + CHECKSUM_BYTES:
            raise BundleError("static query: query bundle dimensions and length do not match")
        x = np.frombuffer(data, "<f4", elements, _QUERY_HEADER.size).reshape(b, q, h)
        if not np.isfinite(x).all():
            raise BundleError("static query: query bundle contains a non-finite value")
        return cls(model, context, np.array(x, np.float32))

    @classmethod
    def read(cls, path) -> "StaticQueryBundle":
        data = _read_file(path, "static query: query bundle")
        return cls.from_bytes(data)

    def write(self, path) -> None:
        _write_file(path, self.to_bytes())


def encode_logits(logits) -> bytes:
    """IRLOGITS v1 bytes of logits [B, test rows, classes]."""
    a = np.ascontiguousarray(logits, dtype=np.float32)
    if a.ndim != 3 or 0 in a.shape:
        raise BundleError("logits must be a nonempty [B, test rows, classes] tensor")
    if _LOGITS_HEADER.size + 4 * a.size + CHECKSUM_BYTES > MAX_BUNDLE_BYTES:
        raise BundleError("logits exceed the resource limit")
    b, q, c = a.shape
    return _sealed(_LOGITS_HEADER.pack(LOGITS_MAGIC, VERSION, KIND, b, q, c, a.size) + a.astype("<f4").tobytes())


def decode_logits(data: bytes) -> np.ndarray:
    """Logits [B, test rows, classes] of IRLOGITS v1 bytes, checked as the
    reference's comparison tool reads them (tools/compare_cached_logits.py:20-29)."""
    if len(data) < _LOGITS_HEADER.size + CHECKSUM_BYTES or \
            hashlib.sha256(data[:-CHECKSUM_BYTES]).digest() != data[-CHECKSUM_BYTES:]:
        raise BundleError("invalid IRLOGITS checksum")
    magic, version, kind, b, q, c, count = _LOGITS_HEADER.unpack_from(data)
    if (magic, version, kind) != (LOGITS_MAGIC, VERSION, KIND) or count != b * q * c:
        raise BundleError("invalid IRLOGITS metadata")
    if len(data) != _LOGITS_HEADER.size + 4 * count + CHECKSUM_BYTES:
        raise BundleError("invalid IRLOGITS length")
    return np.frombuffer(data, "<f4", count, _LOGITS_HEADER.size).reshape(b, q, c).astype(np.float32)


def write_logits(path, logits) -> None:
    _write_file(path, encode_logits(logits))


def read_logits(path) -> np.ndarray:
    return decode_logits(_read_file(path, "IRLOGITS"))
