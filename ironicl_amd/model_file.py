"""IRMODEL v1: the reference's portable model artifact, read and written
unchanged (src/format/model.rs:19-30, 381-483 encode, 486-714 parse,
869-885 profiles; common rules in src/format/mod.rs:1-26).

Kept alike on purpose: it is the on-disk interchange format the backend's
weights come from (the reference's own artifacts must load unchanged), so an
artifact written here loads in the reference and one the reference writes loads
here.

Layout, little-endian:

    header (144 bytes)
        magic "IRMODEL\\0" | u32 version = 1 | u32 kind = 1
        source checkpoint SHA-256 (32) | u32 tensor count
        u64 parameter count | u64 tensor bytes
        u64 x 7 config: max_classes (10 | 0), num_quantiles, embed_dim,
                        column_blocks, row_blocks, row_cls_tokens, icl_blocks
        u64 directory length | u64 payload length | u32 0
    directory, one entry per tensor in bytewise name order:
        u32 name length | u16 rank | u8 dtype id | u8 0
        u64 payload offset (a multiple of 64) | u64 byte length
        u64 x rank dimensions | name (UTF-8)
    zero padding to 64 | payload (each tensor 64-byte aligned)
    SHA-256 of every preceding byte

An executable model is one of the two official profiles: the official source
SHA-256, task, tensor count, parameter count and tensor bytes, the release
configuration and the exact FP32 manifest (model.rs:240-250, 839-867). The
regressor's bias-free LayerNorms load with zero biases (model.rs:273-280).
"""

from __future__ import annotations

import hashlib
import mmap
import os
import struct
import tempfile
import time
from dataclasses import dataclass, field

import numpy as np

from . import manifest as mf

MAGIC = b"IRMODEL\0"
VERSION = 1
KIND = 1
HEADER_BYTES = 144
CHECKSUM_BYTES = 32
ALIGNMENT = 64
MAX_ARTIFACT_BYTES = 512 << 20
MAX_DIRECTORY_BYTES = 4 << 20
MAX_TENSOR_COUNT = 4096
MAX_TENSOR_RANK = 16
MAX_TENSOR_NAME_BYTES = 4096
MAX_TENSOR_BYTES = 64 << 20
MAX_TOTAL_TENSOR_BYTES = 256 << 20

# dtype id -> (name, bytes per element, NumPy little-endian type) (model.rs:110-156).
DTYPES = {1: ("u8", 1, "u1"), 2: ("i64", 8, "<i8"), 3: ("bf16", 2, "<u2"), 4: ("f16", 2, "<f2"),
          5: ("f32", 4, "<f4"), 6: ("f64", 8, "<f8")}
F32 = 5

PROFILE_CLASSIFIER = "TabICLv2 classifier"
PROFILE_REGRESSOR = "TabICLv2 regressor"
PROFILE_UNKNOWN = "unknown/custom"

_HEADER = struct.Struct("<8sII32sIQQ7QQQI")
_ENTRY = struct.Struct("<IHBBQQ")
assert _HEADER.size == HEADER_BYTES


class ModelFileError(ValueError):
    """An artifact that is malformed, corrupt or not an executable model (Error::Artifact)."""


@dataclass
class Tensor:
    name: str
    dtype: int
    dims: tuple[int, ...]
    data: bytes | memoryview | np.ndarray


@dataclass
class Summary:
    """ModelArtifactSummary (model.rs:175-185)."""
    source_sha256: str
    profile: str
    tensor_count: int
    parameter_count: int
    tensor_bytes: int
    dtype_counts: dict[str, int]
    config: tuple[int, ...]

    def task(self) -> str | None:
        return None if not self.config else (mf.REGRESSOR if self.config[0] == 0 else mf.CLASSIFIER)


@dataclass
class Parsed:
    summary: Summary
    # name -> (dtype id, dims, absolute byte range in the artifact)
    tensors: dict[str, tuple[int, tuple[int, ...], tuple[int, int]]] = field(default_factory=dict)


def release_config(task: str) -> tuple[int, ...]:
    """The official configuration (validate_config, model.rs:820-836)."""
    return (mf.MAX_CLASSES if task == mf.CLASSIFIER else 0, mf.NUM_QUANTILES, mf.COLUMN_DIM, mf.COLUMN_BLOCKS,
            mf.ROW_BLOCKS, mf.RESERVED, mf.ICL_BLOCKS)


def official_sha256(task: str) -> bytes:
    return mf.CLASSIFIER_SHA256 if task == mf.CLASSIFIER else mf.REGRESSOR_SHA256


def _elements(name: str, dims) -> int:
    n = 1
    for d in dims:
        n *= int(d)
        if n >= 1 << 64:
            raise ModelFileError(f"tensor '{name}' element count overflows u64")
    return n


def _align(n: int) -> int:
    return (n + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT


def encode(source_sha256: bytes, config: tuple[int, ...], tensors: list[Tensor]) -> bytes:
    """The artifact bytes (encode_model_artifact, model.rs:381-483)."""
    if len(config) != 7 or any(v <= 0 for v in config[1:]):
        raise ModelFileError("model configuration dimensions must be greater than zero")
    if len(source_sha256) != 32 or source_sha256 == bytes(32):
        raise ModelFileError("source checkpoint hash is empty")
    if not 1 <= len(tensors) <= MAX_TENSOR_COUNT:
        raise ModelFileError(f"model has {len(tensors)} tensors; expected 1..={MAX_TENSOR_COUNT}")
    directory = bytearray()
    payload = bytearray()
    params = total = 0
    seen = set()
    for t in sorted(tensors, key=lambda t: t.name.encode()):
        name = t.name.encode()
        if not 0 < len(name) <= MAX_TENSOR_NAME_BYTES:
            raise ModelFileError(f"invalid tensor name '{t.name}'")
        if len(t.dims) > MAX_TENSOR_RANK:
            raise ModelFileError(f"tensor '{t.name}' rank {len(t.dims)} exceeds {MAX_TENSOR_RANK}")
        if t.dtype not in DTYPES:
            raise ModelFileError(f"unsupported tensor dtype ID {t.dtype}")
        data = memoryview(np.ascontiguousarray(t.data) if isinstance(t.data, np.ndarray) else t.data).cast("B")
        elements = _elements(t.name, t.dims)
        expected = elements * DTYPES[t.dtype][1]
        if len(data) != expected or len(data) > MAX_TENSOR_BYTES:
            raise ModelFileError(f"tensor '{t.name}' is {len(data)} bytes; expected {expected} with limit "
                                 f"{MAX_TENSOR_BYTES}")
        if name in seen:
            raise ModelFileError(f"duplicate tensor name '{t.name}'")
        seen.add(name)
        payload.extend(bytes(_align(len(payload)) - len(payload)))
        directory += _ENTRY.pack(len(name), len(t.dims), t.dtype, 0, len(payload), len(data))
        directory += struct.pack(f"<{len(t.dims)}Q", *t.dims) + name
        payload += data
        params += elements
        total += len(data)
    if total > MAX_TOTAL_TENSOR_BYTES:
        raise ModelFileError(f"model tensors are {total} bytes; limit is {MAX_TOTAL_TENSOR_BYTES}")
    if len(directory) > MAX_DIRECTORY_BYTES:
        raise ModelFileError("model tensor directory is too large")
    out = bytearray(_HEADER.pack(MAGIC, VERSION, KIND, source_sha256, len(tensors), params, total, *config,
                                 len(directory), len(payload), 0))
    out += directory
    out += bytes(_align(len(out)) - len(out))
    out += payload
    out += hashlib.sha256(out).digest()
    if len(out) > MAX_ARTIFACT_BYTES:
        raise ModelFileError(f"artifact is {len(out)} bytes; limit is {MAX_ARTIFACT_BYTES}")
    return bytes(out)


def _profile(sha: bytes, task: str | None, count: int, params: int, nbytes: int) -> str:
    """identify_profile (model.rs:869-885)."""
    for t, name in ((mf.CLASSIFIER, PROFILE_CLASSIFIER), (mf.REGRESSOR, PROFILE_REGRESSOR)):
        if sha == official_sha256(t) and task == t and (count, params, nbytes) == mf.PROFILE[t]:
            return name
    return PROFILE_UNKNOWN


def parse(data) -> Parsed:
    """Verify an artifact and describe it (parse_model_artifact_bytes,
    model.rs:486-714): checksum, header, section offsets, zero padding, the
    directory's sorted unique names, sizes and non-overlapping ranges, and
    the declared totals."""
    buf = memoryview(data).cast("B")
    size = len(buf)
    if size < HEADER_BYTES + CHECKSUM_BYTES:
        raise ModelFileError("artifact is truncated")
    if size > MAX_ARTIFACT_BYTES:
        raise ModelFileError(f"artifact is {size} bytes; limit is {MAX_ARTIFACT_BYTES}")
    end = size - CHECKSUM_BYTES
    if hashlib.sha256(buf[:end]).digest() != bytes(buf[end:]):
        raise ModelFileError("artifact checksum does not match")
    (magic, version, kind, sha, count, params, nbytes, *rest) = _HEADER.unpack_from(buf, 0)
    config, dir_len, pay_len, reserved = tuple(rest[:7]), rest[7], rest[8], rest[9]
    if magic != MAGIC:
        raise ModelFileError("model artifact magic does not match")
    if version != VERSION:
        raise ModelFileError(f"model artifact version {version} is unsupported; expected {VERSION}")
    if kind != KIND:
        raise ModelFileError(f"artifact kind {kind} is not a portable model")
    if sha == bytes(32):
        raise ModelFileError("source checkpoint hash is empty")
    if not 1 <= count <= MAX_TENSOR_COUNT:
        raise ModelFileError(f"artifact has {count} tensors; expected 1..={MAX_TENSOR_COUNT}")
    if any(v == 0 for v in config[1:]):
        raise ModelFileError("model configuration dimensions must be greater than zero")
    if reserved != 0:
        raise ModelFileError("artifact header reserved bytes are invalid")
    if dir_len > MAX_DIRECTORY_BYTES or pay_len > MAX_TOTAL_TENSOR_BYTES + 64 * 4096:
        raise ModelFileError("artifact section length exceeds its limit")
    dir_end = HEADER_BYTES + dir_len
    pay_start = _align(dir_end)
    if pay_start + pay_len != end:
        raise ModelFileError("artifact section offsets are inconsistent")
    if any(buf[dir_end:pay_start]):
        raise ModelFileError("artifact alignment padding is not zero")
    out = Parsed(Summary(sha.hex(), PROFILE_UNKNOWN, count, 0, 0, {}, config))
    pos, prev, ranges, total_params, total_bytes = HEADER_BYTES, None, [], 0, 0
    for _ in range(count):
        if pos + _ENTRY.size > dir_end:
            raise ModelFileError("tensor directory is truncated")
        name_len, rank, dtype, zero, offset, length = _ENTRY.unpack_from(buf, pos)
        pos += _ENTRY.size
        if not 0 < name_len <= MAX_TENSOR_NAME_BYTES:
            raise ModelFileError(f"invalid tensor name length {name_len}")
        if rank > MAX_TENSOR_RANK:
            raise ModelFileError(f"tensor rank {rank} exceeds {MAX_TENSOR_RANK}")
        if dtype not in DTYPES:
            raise ModelFileError(f"unsupported tensor dtype ID {dtype}")
        if zero != 0:
            raise ModelFileError("tensor directory reserved byte is not zero")
        if length > MAX_TENSOR_BYTES or offset % ALIGNMENT:
            raise ModelFileError("tensor payload offset or length is invalid")
        if pos + 8 * rank + name_len > dir_end:
            raise ModelFileError("tensor directory is truncated")
        dims = struct.unpack_from(f"<{rank}Q", buf, pos)
        pos += 8 * rank
        raw = bytes(buf[pos:pos + name_len])
        pos += name_len
        try:
            name = raw.decode("utf-8")
        except UnicodeDecodeError as e:
            raise ModelFileError(f"tensor name is not UTF-8: {e}") from None
        if prev is not None and prev >= raw:
            raise ModelFileError("tensor names are not unique and sorted")
        prev = raw
        elements = _elements(name, dims)
        if elements * DTYPES[dtype][1] != length:
            raise ModelFileError(f"tensor '{name}' is {length} bytes; expected {elements * DTYPES[dtype][1]}")
        if offset + length > pay_len:
            raise ModelFileError(f"tensor '{name}' exceeds the payload section")
        ranges.append((offset, offset + length))
        out.tensors[name] = (dtype, tuple(dims), (pay_start + offset, pay_start + offset + length))
        total_params += elements
        total_bytes += length
        tag = DTYPES[dtype][0]
        out.summary.dtype_counts[tag] = out.summary.dtype_counts.get(tag, 0) + 1
    if pos != dir_end:
        raise ModelFileError("tensor directory has trailing bytes")
    ranges.sort()
    if any(a[1] > b[0] for a, b in zip(ranges, ranges[1:])):
        raise ModelFileError("tensor payload ranges overlap")
    if total_params != params or total_bytes != nbytes:
        raise ModelFileError("artifact aggregate tensor metadata does not match")
    out.summary.parameter_count, out.summary.tensor_bytes = total_params, total_bytes
    out.summary.profile = _profile(sha, out.summary.task(), count, total_params, total_bytes)
    return out


def validate_executable(parsed: Parsed) -> str:
    """The task of an official model, or ModelFileError (ModelArtifact::from_bytes,
    validate_config and validate_manifest, model.rs:240-250, 777-836)."""
    s = parsed.summary
    if s.profile == PROFILE_CLASSIFIER:
        task = mf.CLASSIFIER
    elif s.profile == PROFILE_REGRESSOR:
        task = mf.REGRESSOR
    else:
        raise ModelFileError("executable model must be an official TabICLv2 classifier or regressor")
    if s.config != release_config(task):
        raise ModelFileError(f"official {task} configuration is {list(s.config)}; expected "
                             f"{list(release_config(task))}")
    expected = mf.tensor_manifest(task)
    if len(parsed.tensors) != len(expected):
        raise ModelFileError(f"official {task} has {len(parsed.tensors)} tensors; expected {len(expected)}")
    for name, (dtype, dims, _) in parsed.tensors.items():
        if name not in expected:
            raise ModelFileError(f"unexpected official {task} tensor '{name}'")
        if dtype != F32:
            raise ModelFileError(f"official {task} tensor '{name}' has dtype {DTYPES[dtype][0]}; expected f32")
        if tuple(dims) != tuple(expected[name]):
            raise ModelFileError(f"official {task} tensor '{name}' has shape {list(dims)}; expected "
                                 f"{list(expected[name])}")
    return task


@dataclass
class ModelArtifact:
    """An executable official model (ModelArtifact, model.rs:205-320): its
    summary, task and FP32 tensors by official name. The tensors are views of
    the artifact's bytes (kept alive here), not copies; the regressor's
    LayerNorm biases are zero arrays."""
    summary: Summary
    task: str
    tensors: dict[str, np.ndarray]
    _keep: object = None

    @property
    def source_sha256(self) -> str:
        return self.summary.source_sha256


def from_bytes(data) -> ModelArtifact:
    parsed = parse(data)
    task = validate_executable(parsed)
    buf = memoryview(data).cast("B")
    tensors = {}
    for name, (_, dims, (a, b)) in parsed.tensors.items():
        tensors[name] = np.frombuffer(buf[a:b], dtype="<f4").reshape(dims)
    if task == mf.REGRESSOR:
        for name, dims in mf.tensor_manifest(mf.CLASSIFIER).items():
            if name not in tensors and mf._is_ln_bias(name):
                tensors[name] = np.zeros(dims, np.float32)
    return ModelArtifact(parsed.summary, task, tensors, data)


def load(path) -> ModelArtifact:
    """Read, verify and prepare an official model artifact (ModelArtifact::load);
    the file is mapped read-only."""
    with open(path, "rb") as f:
        size = os.fstat(f.fileno()).st_size
        if size > MAX_ARTIFACT_BYTES:
            raise ModelFileError(f"artifact is {size} bytes; limit is {MAX_ARTIFACT_BYTES}")
        if size == 0:
            raise ModelFileError("artifact is truncated")
        mapped = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    return from_bytes(mapped)


def inspect(path) -> Summary:
    """Verify an artifact and return its summary (inspect_model_artifact)."""
    with open(path, "rb") as f:
        return parse(f.read()).summary


def model_tensors(task: str, weights: dict[str, np.ndarray]) -> list[Tensor]:
    """The manifest's FP32 tensors of `weights` (the regressor's has no LayerNorm biases)."""
    out = []
    for name, dims in mf.tensor_manifest(task).items():
        arr = np.ascontiguousarray(weights[name], dtype="<f4")
        if arr.shape != tuple(dims):
            raise ModelFileError(f"tensor '{name}' has shape {list(arr.shape)}; expected {list(dims)}")
        out.append(Tensor(name, F32, tuple(dims), arr))
    return out


def encode_model(task: str, weights: dict[str, np.ndarray], source_sha256: bytes | None = None) -> bytes:
    """An official-profile artifact of `weights`: the release configuration, the
    manifest's tensors and (by default) the official source SHA-256 of `task`."""
    sha = official_sha256(task) if source_sha256 is None else source_sha256
    return encode(sha, release_config(task), model_tensors(task, weights))


def write(path, data: bytes) -> Summary:
    """Write artifact bytes atomically: a new temporary file beside `path`,
    synced and verified, renamed into place, then the directory synced
    (write_model_artifact, model.rs:343-379). A failed write leaves nothing."""
    expected = parse(data).summary
    path = os.fspath(path)
    parent = os.path.dirname(path) or "."
    os.makedirs(parent, exist_ok=True)
    fd, tmp = tempfile.mkstemp(prefix=f".{os.path.basename(path)}.tmp-{os.getpid()}-{time.time_ns()}-",
                               dir=parent)
    try:
        with os.fdopen(fd, "wb") as f:
            f.write(data)
            f.flush()
            os.fsync(f.fileno())
        if inspect(tmp) != expected:
            raise ModelFileError("temporary artifact verification changed metadata")
        os.replace(tmp, path)
        dfd = os.open(parent, os.O_RDONLY)
        try:
            os.fsync(dfd)
        finally:
            os.close(dfd)
    except BaseException:
        try:
            os.unlink(tmp)
        except OSError:
            pass
        raise
    return inspect(path)


def write_model(path, task: str, weights: dict[str, np.ndarray], source_sha256: bytes | None = None) -> Summary:
    return write(path, encode_model(task, weights, source_sha256))
