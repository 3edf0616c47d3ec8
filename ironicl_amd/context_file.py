"""IRCNTXT static-context artifacts and the context cache, for contexts built
on (or uploaded to) the GPU.

The byte layout is the reference's IRCNTXT container, version 1 (all FP32)
or version 2 (tagged FP32 / FP16 tensors, as the reference writes GPU-built
optimize="auto" contexts) (src/format/static_context.rs:820-987), so a file
written here loads in the reference and a file the reference writes loads here:

    header (164 bytes, little-endian)
        magic b"IRCNTXT\\0" | version u32 | kind u32 = 1
        model SHA-256 (32) | context SHA-256 (32)
        B, N, H, classes                      4 x u64
        architecture 3, 12, 8, 16, 64         5 x u32
        tensor count, class-permutation count, feature-permutation count  3 x u32
        directory bytes u64 | payload bytes u64 | reserved u32 = 0
    permutations: class [B, C] then feature [B, H], u64, estimator-major
    directory, one entry per tensor in bytewise name order:
        name bytes u32 | rank u16 | dtype tag u16 (0 in version 1)
        payload offset u64 | byte length u64 | dims rank x u64 | name
    zero padding to a 64-byte boundary
    payload: each tensor at a 64-byte-aligned offset, zero padding between
    SHA-256 of every preceding byte

Writing streams the payload (from host arrays or straight out of HBM through
`irx_predictor_read_context`) into a private temporary file next to the
destination while hashing it, syncs it and renames it into place, so a reader
never sees a partial file (static_context.rs:1005-1027). Reading maps the file,
verifies the digest and every header, directory and value rule the reference
checks (static_context.rs:551-818, 1099-1219), and hands out zero-copy views.
"""

from __future__ import annotations

import hashlib
import mmap
import os
import struct
import tempfile
import time
from dataclasses import dataclass, field
from datetime import datetime, timedelta
from pathlib import Path
from typing import Callable, Iterable

import numpy as np

from . import manifest as mf

MAGIC = b"IRCNTXT\0"
VERSION_FP32 = 1           # every tensor FP32, zero dtype tags
VERSION_TAGGED = 2         # explicit dtype per tensor (FP32 / BF16 / FP16); written for FP16 ICL caches
VERSION_PACKED_KEYS = 3    # source-tile, dimension-major ICL K
KIND = 1
HEADER_BYTES = 164
CHECKSUM_BYTES = 32
ALIGNMENT = 64
ARCHITECTURE = (3, 12, 8, 16, 64)  # column blocks, ICL blocks, heads, column and ICL head dims

# Resource limits (static_context.rs:31-43).
MAX_ARTIFACT_BYTES = 48 << 30
MAX_DIRECTORY_BYTES = 4 << 20
MAX_TENSOR_COUNT = 4096
MAX_TENSOR_RANK = 16
MAX_TENSOR_NAME_BYTES = 4096
MAX_TENSOR_BYTES = 4 << 30
MAX_TOTAL_TENSOR_BYTES = 48 << 30
MAX_ENSEMBLE_COUNT = 4096
MAX_TRAINING_ROWS = 1_000_000
MAX_FEATURE_COUNT = 65_536
MAX_CLASS_COUNT = 4096

# Context identity (cpu.rs:841-858): the prefix, and the Ironicl version it
# covers (Cargo.toml:3).
IDENTITY_PREFIX = b"ironicl-context-v2\0"
IRONICL_VERSION = "0.1.0"
OPTIMIZE_LEVELS = ("safe", "auto", "fast")

SUFFIX = ".irctx"
STALE_TEMPORARY_SECONDS = 3600

_HEAD = struct.Struct("<8sII32s32sQQQQ5IIIIQQI")
assert _HEAD.size == HEADER_BYTES
_ENTRY = struct.Struct("<IHHQQ")

# A tensor's values, `count` floats from element `start`, as a float32 array.
TensorSource = Callable[[str, int, int], np.ndarray]


class ContextError(ValueError):
    """An invalid, unsupported or mismatched static context (Error::Artifact)."""

    def __init__(self, message: str):
        super().__init__(f"static context: {message}")


@dataclass
class Metadata:
    """What identifies and describes one static context (StaticContextMetadata,
    static_context.rs:56-74). Permutations are flat, estimator-major u64."""

    model_sha256: bytes
    context_sha256: bytes
    ensemble_count: int
    training_rows: int
    feature_count: int
    class_count: int
    class_permutations: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint64))
    feature_permutations: np.ndarray = field(default_factory=lambda: np.zeros(0, np.uint64))

    def __post_init__(self):
        self.class_permutations = np.ascontiguousarray(self.class_permutations, dtype=np.uint64).reshape(-1)
        self.feature_permutations = np.ascontiguousarray(self.feature_permutations, dtype=np.uint64).reshape(-1)

    def __eq__(self, other) -> bool:
        if not isinstance(other, Metadata):
            return NotImplemented
        return (self.model_sha256 == other.model_sha256 and self.context_sha256 == other.context_sha256
                and (self.ensemble_count, self.training_rows, self.feature_count, self.class_count)
                == (other.ensemble_count, other.training_rows, other.feature_count, other.class_count)
                and np.array_equal(self.class_permutations, other.class_permutations)
                and np.array_equal(self.feature_permutations, other.feature_permutations))

    @property
    def shape(self) -> tuple[int, int, int]:
        return self.ensemble_count, self.training_rows, self.feature_count


def context_tensor_specs(b: int, n: int, h: int, icl_dtype=np.float32) -> list[tuple[str, tuple[int, ...], np.dtype]]:
    """The 30 cache tensors of a context in the reference's order
    (context_tensors, cpu.rs:4106-4123): column blocks then ICL blocks, each
    key then value, with their storage (the column tensors are always FP32;
    the ICL ones FP32, or FP16 for an optimize="auto" context, cpu.rs:4038-4044).
    This is also the tensor index `irx_predictor_read_context` takes."""
    specs = []
    for block in range(mf.COLUMN_BLOCKS):
        shape = (b, h + mf.RESERVED, mf.HEADS, mf.INDUCING, mf.COLUMN_DIM // mf.HEADS)
        specs += [(f"column.{block}.key", shape, np.dtype(np.float32)),
                  (f"column.{block}.value", shape, np.dtype(np.float32))]
    for block in range(mf.ICL_BLOCKS):
        shape = (b, mf.HEADS, n, mf.ICL_DIM // mf.HEADS)
        specs += [(f"icl.{block}.key", shape, np.dtype(icl_dtype)), (f"icl.{block}.value", shape, np.dtype(icl_dtype))]
    return specs


def context_identity(source_sha256: str, optimize: str, x: np.ndarray, y_train: np.ndarray,
                     class_permutations: np.ndarray, feature_permutations: np.ndarray,
                     version: str = IRONICL_VERSION) -> bytes:
    """The context's cache identity (cpu.rs:841-858): SHA-256 over the prefix,
    the Ironicl version, the model's source-checkpoint hash (hex text) and the
    optimize level, each NUL-terminated, then B, N, H as u64 and the raw bytes
    of x [B, N, H] f32, y_train [B, N] f32 and the u64 permutations."""
    if optimize not in OPTIMIZE_LEVELS:
        raise ValueError(f"optimize must be one of {OPTIMIZE_LEVELS}, not {optimize!r}")
    x = np.ascontiguousarray(x, dtype="<f4")
    y_train = np.ascontiguousarray(y_train, dtype="<f4")
    if x.ndim != 3:
        raise ValueError("x must be [B, N, H]")
    digest = hashlib.sha256(IDENTITY_PREFIX)
    for part in (version, source_sha256, optimize):
        digest.update(part.encode() + b"\0")
    digest.update(struct.pack("<3Q", *x.shape))
    for arr in (x, y_train, np.ascontiguousarray(class_permutations, dtype="<u8"),
                np.ascontiguousarray(feature_permutations, dtype="<u8")):
        digest.update(memoryview(arr).cast("B"))
    return digest.digest()


def _align(value: int) -> int:
    return (value + ALIGNMENT - 1) // ALIGNMENT * ALIGNMENT


def _check_permutations(values: np.ndarray, b: int, width: int, what: str) -> None:
    if values.size != b * width:
        raise ContextError(f"{what} permutation count does not match estimator metadata")
    if width:
        rows = values.reshape(b, width)
        if (rows >= width).any() or not (np.sort(rows, axis=1) == np.arange(width, dtype=np.uint64)).all():
            raise ContextError(f"{what} permutation is invalid")


def validate_metadata(meta: Metadata) -> None:
    """validate_metadata (static_context.rs:1099-1127)."""
    if len(meta.model_sha256) != 32 or len(meta.context_sha256) != 32:
        raise ContextError("SHA-256 identities must be 32 bytes")
    if meta.model_sha256 == bytes(32) or meta.context_sha256 == bytes(32):
        raise ContextError("static context SHA-256 identity is empty")
    if not (0 < meta.ensemble_count <= MAX_ENSEMBLE_COUNT and 0 < meta.training_rows <= MAX_TRAINING_ROWS
            and 0 < meta.feature_count <= MAX_FEATURE_COUNT and 0 <= meta.class_count <= MAX_CLASS_COUNT):
        raise ContextError("static context dimensions are outside the resource limits")
    _check_permutations(meta.class_permutations, meta.ensemble_count, meta.class_count, "class")
    _check_permutations(meta.feature_permutations, meta.ensemble_count, meta.feature_count, "feature")


@dataclass
class _Entry:
    name: str
    shape: tuple[int, ...]
    offset: int        # within the payload
    nbytes: int
    dtype: np.dtype = np.dtype(np.float32)


# StorageDType's on-disk tags in tagged versions (src/config.rs:79-86).
_TAGS = {np.dtype(np.float32): 1, np.dtype(np.float16): 3}


def _spec(s):
    """(name, shape) or (name, shape, dtype), FP32 by default."""
    name, shape = str(s[0]), tuple(int(d) for d in s[1])
    dtype = np.dtype(s[2]) if len(s) > 2 else np.dtype(np.float32)
    if dtype not in _TAGS:
        raise ContextError(f"tensor '{name}' storage {dtype} is not supported (FP32 or FP16)")
    return name, shape, dtype


def _layout(meta: Metadata, specs: Iterable[tuple[str, tuple[int, ...]]]) -> tuple[bytes, list[_Entry], int]:
    """The bytes before the payload (header, permutations, directory,
    padding), the tensors in file order with their payload offsets, and the
    whole encoded length (static_context.rs:876-987)."""
    validate_metadata(meta)
    specs = sorted((_spec(s) for s in specs), key=lambda t: t[0].encode())
    if not specs or len(specs) > MAX_TENSOR_COUNT:
        raise ContextError("static context section exceeds the resource limit")
    # Version 1 when every tensor is FP32; version 2 tags each tensor's storage.
    version = VERSION_FP32 if all(d == np.float32 for _, _, d in specs) else VERSION_TAGGED
    directory = bytearray()
    entries = []
    payload = 0
    previous = None
    for name, shape, dtype in specs:
        raw = name.encode()
        if previous is not None and raw <= previous:
            raise ContextError("static context tensor names are not unique and sorted")
        previous = raw
        if not raw or len(raw) > MAX_TENSOR_NAME_BYTES or not shape or len(shape) > MAX_TENSOR_RANK:
            raise ContextError("static context tensor name or rank is invalid")
        if min(shape) <= 0:
            raise ContextError("static context tensor dimension is zero")
        nbytes = dtype.itemsize * int(np.prod(shape, dtype=np.uint64))
        if nbytes > MAX_TENSOR_BYTES:
            raise ContextError(f"static context tensor '{name}' exceeds the resource limit")
        offset = _align(payload)
        payload = offset + nbytes
        tag = 0 if version == VERSION_FP32 else _TAGS[dtype]
        directory += _ENTRY.pack(len(raw), len(shape), tag, offset, nbytes)
        directory += struct.pack(f"<{len(shape)}Q", *shape) + raw
        entries.append(_Entry(name, shape, offset, nbytes, dtype))
    if len(directory) > MAX_DIRECTORY_BYTES or payload > MAX_TOTAL_TENSOR_BYTES:
        raise ContextError("static context section exceeds the resource limit")
    head = bytearray(_HEAD.pack(
        MAGIC, version, KIND, meta.model_sha256, meta.context_sha256,
        meta.ensemble_count, meta.training_rows, meta.feature_count, meta.class_count, *ARCHITECTURE,
        len(entries), meta.class_permutations.size, meta.feature_permutations.size,
        len(directory), payload, 0))
    head += meta.class_permutations.astype("<u8").tobytes() + meta.feature_permutations.astype("<u8").tobytes()
    head += directory
    head += bytes(_align(len(head)) - len(head))
    total = len(head) + payload + CHECKSUM_BYTES
    if total > MAX_ARTIFACT_BYTES:
        raise ContextError("static context exceeds the resource limit")
    return bytes(head), entries, total


def encoded_len(meta: Metadata, specs) -> int:
    return _layout(meta, specs)[2]


def encode(meta: Metadata, specs, source: TensorSource, sink, chunk_floats: int = 1 << 24) -> None:
    """Write the artifact to the binary file-like `sink` in one pass, hashing
    as it goes (StaticContextArtifact::encode, static_context.rs:842-874).
    `source` returns each tensor's values in its storage type. Values must be
    finite, as a stored context's are (validate_tensor, static_context.rs:1167-1176)."""
    head, entries, _ = _layout(meta, specs)
    digest = hashlib.sha256()

    def put(data) -> None:
        digest.update(data)
        sink.write(data)

    put(head)
    written = 0
    for e in entries:
        if e.offset > written:
            put(bytes(e.offset - written))
        count = e.nbytes // e.dtype.itemsize
        for start in range(0, count, chunk_floats):
            n = min(chunk_floats, count - start)
            chunk = np.ascontiguousarray(source(e.name, start, n), dtype=e.dtype.newbyteorder("<")).reshape(-1)
            if chunk.size != n:
                raise ContextError(f"tensor '{e.name}' source returned {chunk.size} values, expected {n}")
            if not np.isfinite(chunk).all():
                raise ContextError(f"static context tensor '{e.name}' has a non-finite value")
            put(memoryview(chunk).cast("B"))
        written = e.offset + e.nbytes
    sink.write(digest.digest())


def to_bytes(meta: Metadata, tensors: dict[str, np.ndarray]) -> bytes:
    """The whole artifact in memory (StaticContextArtifact::to_bytes)."""
    import io

    specs = [(name, np.shape(arr), np.float16 if np.asarray(arr).dtype == np.float16 else np.float32)
             for name, arr in tensors.items()]
    flat = {name: np.ascontiguousarray(arr).reshape(-1) for name, arr in tensors.items()}
    out = io.BytesIO()
    encode(meta, specs, lambda name, start, n: flat[name][start:start + n], out)
    return out.getvalue()


def write(path, meta: Metadata, specs, source: TensorSource, chunk_floats: int = 1 << 24) -> None:
    """Encode into a new owner-only temporary file beside `path`, sync it and
    rename it into place; on any failure the temporary file is removed
    (StaticContextArtifact::write, static_context.rs:1005-1027)."""
    path = Path(path)
    directory = path.parent if str(path.parent) else Path(".")
    fd, tmp = tempfile.mkstemp(prefix=".ironicl-", suffix=".tmp", dir=directory)
    try:
        with os.fdopen(fd, "wb", buffering=1 << 22) as f:
            encode(meta, specs, source, f, chunk_floats)
            f.flush()
            os.fsync(f.fileno())
        os.replace(tmp, path)
    except BaseException:
        try:
            os.unlink(tmp)
        except OSError:
            pass
        raise


class ContextFile:
    """A verified IRCNTXT artifact with zero-copy FP32 tensor views over its
    bytes (StaticContextArtifact)."""

    def __init__(self, buffer, version: int, metadata: Metadata, tensors: dict[str, np.ndarray]):
        self._buffer = buffer
        self.version = version
        self.metadata = metadata
        self._tensors = tensors

    @property
    def names(self) -> list[str]:
        return list(self._tensors)

    def tensor(self, name: str) -> np.ndarray | None:
        return self._tensors.get(name)

    def host_tensors(self):
        """(column keys, column values, ICL keys, ICL values), the upload
        layout of `irx_context_tensors`."""
        t = self._tensors
        return ([t[f"column.{i}.key"] for i in range(mf.COLUMN_BLOCKS)],
                [t[f"column.{i}.value"] for i in range(mf.COLUMN_BLOCKS)],
                [t[f"icl.{i}.key"] for i in range(mf.ICL_BLOCKS)],
                [t[f"icl.{i}.value"] for i in range(mf.ICL_BLOCKS)])


def _parse(buf) -> ContextFile:
    """Verify and index an artifact held in `buf` (bytes or a read-only
    mapping): StaticContextArtifact::from_mapping (static_context.rs:551-818).
    FP32 and FP16 tensors load (an FP16 ICL cache is what optimize="auto"
    predicts from); BF16 tensors and packed keys (version 3) are refused: no
    predictor here reads them (the reference's CUDA path leaves such contexts
    on its CPU, cpu.rs:1862-1870)."""
    view = memoryview(buf)
    length = len(view)
    if not HEADER_BYTES + CHECKSUM_BYTES <= length <= MAX_ARTIFACT_BYTES:
        raise ContextError("static context length is outside the resource limit")
    body = length - CHECKSUM_BYTES
    digest = hashlib.sha256()
    for start in range(0, body, 1 << 26):
        digest.update(view[start:min(body, start + (1 << 26))])
    if digest.digest() != bytes(view[body:]):
        raise ContextError("static context checksum does not match")
    (magic, version, kind, model_sha, context_sha, b, n, h, classes, a0, a1, a2, a3, a4,
     tensor_count, class_count_perm, feature_count_perm, dir_len, payload_len, reserved) = _HEAD.unpack_from(view, 0)
    if magic != MAGIC:
        raise ContextError("static context magic does not match")
    if version not in (VERSION_FP32, VERSION_TAGGED, VERSION_PACKED_KEYS):
        raise ContextError(f"static context version {version} is unsupported")
    if kind != KIND:
        raise ContextError("artifact kind is not a static context")
    if (a0, a1, a2, a3, a4) != ARCHITECTURE:
        raise ContextError("static context architecture metadata is unsupported")
    if reserved != 0:
        raise ContextError("static context header reserved bytes are invalid")
    if not 0 < tensor_count <= MAX_TENSOR_COUNT or dir_len > MAX_DIRECTORY_BYTES or payload_len > MAX_TOTAL_TENSOR_BYTES:
        raise ContextError("static context section exceeds the resource limit")
    if class_count_perm != b * classes or feature_count_perm != b * h:
        raise ContextError("static context permutation lengths do not match metadata")
    perms_end = HEADER_BYTES + 8 * (class_count_perm + feature_count_perm)
    dir_end = perms_end + dir_len
    payload_start = _align(dir_end)
    if payload_start + payload_len != body or dir_end > payload_start:
        raise ContextError("static context section offsets are inconsistent")
    if any(view[dir_end:payload_start]):
        raise ContextError("static context alignment padding is not zero")
    perms = np.frombuffer(view, dtype="<u8", count=class_count_perm + feature_count_perm, offset=HEADER_BYTES)
    meta = Metadata(bytes(model_sha), bytes(context_sha), b, n, h, classes,
                    perms[:class_count_perm].copy(), perms[class_count_perm:].copy())
    validate_metadata(meta)
    if version == VERSION_PACKED_KEYS:
        raise ContextError("contexts with packed ICL keys (version 3) are not supported by the FP32 GPU backend")

    tensors: dict[str, np.ndarray] = {}
    ranges = []
    pos, previous, total = perms_end, None, 0
    for _ in range(tensor_count):
        if pos + _ENTRY.size > dir_end:
            raise ContextError("static context tensor directory is truncated")
        name_len, rank, tag, offset, nbytes = _ENTRY.unpack_from(view, pos)
        pos += _ENTRY.size
        if not 0 < name_len <= MAX_TENSOR_NAME_BYTES or not 0 < rank <= MAX_TENSOR_RANK:
            raise ContextError("static context tensor directory entry is invalid")
        if version == VERSION_FP32 and tag != 0:
            raise ContextError("static context tensor directory entry is invalid")
        if offset % ALIGNMENT or nbytes > MAX_TENSOR_BYTES:
            raise ContextError("static context tensor offset or length is invalid")
        if pos + 8 * rank + name_len > dir_end:
            raise ContextError("static context tensor directory is truncated")
        dims = struct.unpack_from(f"<{rank}Q", view, pos)
        pos += 8 * rank
        raw = bytes(view[pos:pos + name_len])
        pos += name_len
        try:
            name = raw.decode("utf-8")
        except UnicodeDecodeError:
            raise ContextError("static context tensor name is not UTF-8") from None
        if previous is not None and previous >= raw:
            raise ContextError("static context tensor names are not unique and sorted")
        previous = raw
        if 0 in dims:
            raise ContextError("static context tensor dimension is zero")
        elements = 1
        for d in dims:
            elements *= d
        # Version 2 tags: the reference's on-disk StorageDType numbering. FP32
        # and FP16 feed this backend; BF16 does not.
        if version == VERSION_FP32:
            dtype = np.dtype("<f4")
        elif tag == _FP32_TAG:
            dtype = np.dtype("<f4")
        elif tag == _F16_TAG:
            dtype = np.dtype("<f2")
        elif tag == 2:
            raise ContextError(f"tensor '{name}' is BF16, which this backend does not read")
        else:
            raise ContextError("static context tensor directory entry is invalid")
        if nbytes != dtype.itemsize * elements:
            raise ContextError(f"static context tensor '{name}' byte length does not match its shape")
        if offset + nbytes > payload_len:
            raise ContextError(f"static context tensor '{name}' exceeds the payload section")
        total += nbytes
        ranges.append((offset, offset + nbytes))
        values = np.frombuffer(view, dtype=dtype, count=elements, offset=payload_start + offset)
        if not np.isfinite(values).all():
            raise ContextError("static context tensor contains a non-finite value")
        tensors[name] = values.reshape(dims)
    if pos != dir_end:
        raise ContextError("static context tensor directory has trailing bytes")
    ranges.sort()
    if any(a[1] > b_[0] for a, b_ in zip(ranges, ranges[1:])) or total > MAX_TOTAL_TENSOR_BYTES:
        raise ContextError("static context tensor payload ranges are invalid")
    return ContextFile(buf, version, meta, tensors)


# StorageDType's on-disk tags for FP32 and FP16 in tagged versions (src/config.rs:79-86).
_FP32_TAG = 1
_F16_TAG = 3


def from_bytes(data: bytes) -> ContextFile:
    """StaticContextArtifact::from_bytes."""
    return _parse(bytes(data))


def read(path) -> ContextFile:
    """Map the file read-only and verify it (StaticContextArtifact::read_mapped_prefault)."""
    with open(path, "rb") as f:
        size = os.fstat(f.fileno()).st_size
        if not HEADER_BYTES + CHECKSUM_BYTES <= size <= MAX_ARTIFACT_BYTES:
            raise ContextError("static context length is outside the resource limit")
        mapping = mmap.mmap(f.fileno(), 0, access=mmap.ACCESS_READ)
    return _parse(mapping)


def read_cached(path, expected: Metadata) -> ContextFile | None:
    """The verified artifact at `path` when it describes exactly `expected`;
    None when it is missing, unreadable, invalid or another context
    (read_cached, static_context.rs:1029-1035)."""
    try:
        context = read(path)
    except (OSError, ValueError):
        return None
    return context if context.metadata == expected else None


def validate_for_model(context: ContextFile, source_sha256: str, task: str) -> None:
    """validate_static_context (cpu.rs:3953-3964) with the serving contract
    (:4125-4143): the model hash, the class count the task allows, and every
    cache tensor present with its logical shape."""
    meta = context.metadata
    if meta.model_sha256.hex() != source_sha256:
        raise ContextError("static context model SHA-256 does not match model artifact")
    if task == mf.CLASSIFIER and not 2 <= meta.class_count <= mf.MAX_CLASSES:
        raise ContextError(f"static context class count {meta.class_count} is unsupported; expected 2..=10")
    if task == mf.REGRESSOR and meta.class_count != 0:
        raise ContextError(f"static context class count {meta.class_count} is unsupported; expected 0")
    for name, shape, _ in context_tensor_specs(*meta.shape):
        t = context.tensor(name)
        if t is None:
            raise ContextError(f"static context cache tensor '{name}' is missing")
        if tuple(t.shape) != shape:
            raise ContextError(f"static context cache tensor '{name}' has shape {list(t.shape)}; "
                               f"expected {list(shape)}")


# ---- the cache directory (python/ironicl/cache.py) ----

def resolve_cache_dir(cache_dir) -> Path | None:
    """None/True: IRONICL_CACHE_DIR or <XDG cache>/ironicl/contexts; False:
    no cache; otherwise the path itself (_cache_dir, cache.py:20-34)."""
    if cache_dir is False:
        return None
    if cache_dir is None or cache_dir is True:
        override = os.environ.get("IRONICL_CACHE_DIR")
        if override:
            return Path(override)
        root = Path(os.environ.get("XDG_CACHE_HOME") or Path.home() / ".cache")
        return root / "ironicl" / "contexts"
    return Path(cache_dir)


def cache_path(directory: Path, meta: Metadata) -> Path:
    """<directory>/<context SHA-256 hex>.irctx (cpu.rs:650-653)."""
    return Path(directory) / f"{meta.context_sha256.hex()}{SUFFIX}"


@dataclass(frozen=True)
class CacheEntry:
    path: Path
    size_bytes: int
    last_used: datetime


@dataclass(frozen=True)
class CacheInfo:
    directory: Path
    entries: tuple[CacheEntry, ...]

    @property
    def size_bytes(self) -> int:
        return sum(e.size_bytes for e in self.entries)

    def __str__(self) -> str:
        lines = [f"{self.directory}: {len(self.entries)} contexts, {self.size_bytes / 2**30:.2f} GiB"]
        lines += [f"  {e.size_bytes / 2**30:>7.2f} GiB  last used {e.last_used:%Y-%m-%d %H:%M}  {e.path.name}"
                  for e in self.entries]
        return "\n".join(lines)


def cache_info(cache_dir=None) -> CacheInfo:
    """Cached contexts, most recently used first (cache_info, cache.py:65-78)."""
    directory = resolve_cache_dir(True if cache_dir is None else cache_dir)
    if directory is None:
        raise ValueError("cache_dir=False disables caching; pass None or a directory")
    entries = []
    for path in directory.glob(f"*{SUFFIX}") if directory.is_dir() else ():
        try:
            st = path.stat()
        except OSError:
            continue
        entries.append(CacheEntry(path, st.st_size, datetime.fromtimestamp(st.st_mtime)))
    entries.sort(key=lambda e: e.last_used, reverse=True)
    return CacheInfo(directory, tuple(entries))


def parse_size(text: str) -> int:
    """A size in bytes, or with a K, M, G or T suffix (binary, optionally
    followed by B or iB), such as 512M or 16GiB (parse_bytes, src/memory.rs:107-150)."""
    lower = text.strip().lower()
    number = lower[:-2] if lower.endswith("ib") else lower[:-1] if lower.endswith("b") else lower
    shift = 10 * ("kmgt".index(number[-1]) + 1) if number and number[-1] in "kmgt" else 0
    digits = number[:-1] if shift else number
    if (shift == 0 and lower.endswith("ib")) or not digits or any(c not in "0123456789." for c in digits):
        raise ValueError("expected a positive size in bytes, or with a K, M, G, or T suffix such as 512M or 16G")
    try:
        value = float(digits) if "." in digits else int(digits)
    except ValueError:
        raise ValueError(f"invalid size {text!r}") from None
    return int(value * (1 << shift))


def clear_cache(cache_dir=None, *, older_than: timedelta | datetime | None = None,
                max_size: int | str | None = None) -> CacheInfo:
    """Remove cached contexts and return what was removed (clear_cache,
    cache.py:81-125): all of them by default; `older_than` removes those last
    used before it, then `max_size` removes the least recently used until the
    rest fit. Temporary files of interrupted writes older than an hour go too."""
    info = cache_info(cache_dir)
    keep = list(info.entries)
    if older_than is None and max_size is None:
        keep = []
    if older_than is not None:
        cutoff = datetime.now() - older_than if isinstance(older_than, timedelta) else older_than
        if cutoff.tzinfo is not None:
            cutoff = cutoff.astimezone().replace(tzinfo=None)
        keep = [e for e in keep if e.last_used >= cutoff]
    if max_size is not None:
        limit = parse_size(max_size) if isinstance(max_size, str) else max_size
        if isinstance(limit, bool) or not isinstance(limit, int) or limit < 0:
            raise ValueError(f"max_size must be a number of bytes or a size such as '10G', not {max_size!r}")
        while keep and sum(e.size_bytes for e in keep) > limit:
            keep.pop()
    removed = []
    for e in info.entries:
        if e not in keep:
            try:
                e.path.unlink()
                removed.append(e)
            except OSError:
                pass
    for path in info.directory.glob(".ironicl-*.tmp") if info.directory.is_dir() else ():
        try:
            if time.time() - path.stat().st_mtime > STALE_TEMPORARY_SECONDS:
                path.unlink()
        except OSError:
            pass
    return CacheInfo(info.directory, tuple(removed))
