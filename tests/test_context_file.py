"""IRCNTXT container and context cache on the CPU (no GPU): the byte layout
field by field, round trips, the rejections and cache behaviour the
reference's own tests check (src/format/static_context.rs:1243-1515,
tests/test_cache.py), and the context identity."""

import hashlib
import os
import struct
import threading
import time
from datetime import timedelta
from pathlib import Path

import numpy as np
import pytest

from ironicl_amd import context_file as cf


def fixture_metadata(**changes):
    """The reference's test fixture (static_context.rs:1247-1262)."""
    fields = dict(model_sha256=bytes([1]) * 32, context_sha256=bytes([2]) * 32, ensemble_count=2,
                  training_rows=3, feature_count=2, class_count=3,
                  class_permutations=[2, 0, 1, 1, 2, 0], feature_permutations=[1, 0, 0, 1])
    fields.update(changes)
    return cf.Metadata(**fields)


def fixture_tensors():
    return {"column.k.0": np.full((2, 8, 3, 16), 1.0, np.float32),
            "icl.v.0": np.full((2, 8, 3, 64), 2.0, np.float32)}


def encode_fixture(meta=None, tensors=None):
    return cf.to_bytes(meta or fixture_metadata(), tensors or fixture_tensors())


def resign(data: bytearray) -> bytes:
    data[-32:] = hashlib.sha256(bytes(data[:-32])).digest()
    return bytes(data)


def test_layout_field_by_field():
    """Every field at the offset the format defines (static_context.rs:876-987)."""
    data = encode_fixture()
    u32 = lambda o: struct.unpack_from("<I", data, o)[0]
    u64 = lambda o: struct.unpack_from("<Q", data, o)[0]
    assert data[:8] == b"IRCNTXT\0"
    assert u32(8) == 1 and u32(12) == 1                      # version 1 (all FP32), kind 1
    assert data[16:48] == bytes([1]) * 32 and data[48:80] == bytes([2]) * 32
    assert [u64(80 + 8 * i) for i in range(4)] == [2, 3, 2, 3]  # B, N, H, classes
    assert [u32(112 + 4 * i) for i in range(5)] == [3, 12, 8, 16, 64]
    assert (u32(132), u32(136), u32(140)) == (2, 6, 4)       # tensors, class and feature permutation counts
    dir_len, payload_len = u64(144), u64(152)
    assert u32(160) == 0                                     # reserved
    perms = struct.unpack_from("<10Q", data, 164)
    assert perms == (2, 0, 1, 1, 2, 0, 1, 0, 0, 1)
    pos = 164 + 80
    # Directory: column.k.0 then icl.v.0 (bytewise order), 64-byte-aligned offsets.
    entries = []
    for _ in range(2):
        name_len, rank, tag, offset, nbytes = struct.unpack_from("<IHHQQ", data, pos)
        dims = struct.unpack_from(f"<{rank}Q", data, pos + 24)
        name = data[pos + 24 + 8 * rank: pos + 24 + 8 * rank + name_len].decode()
        pos += 24 + 8 * rank + name_len
        entries.append((name, dims, tag, offset, nbytes))
    assert pos - (164 + 80) == dir_len
    assert entries == [("column.k.0", (2, 8, 3, 16), 0, 0, 3072), ("icl.v.0", (2, 8, 3, 64), 0, 3072, 12288)]
    payload_start = (pos + 63) // 64 * 64
    assert data[pos:payload_start] == bytes(payload_start - pos)
    assert payload_len == 3072 + 12288
    assert len(data) == payload_start + payload_len + 32
    col = np.frombuffer(data, "<f4", 768, payload_start)
    icl = np.frombuffer(data, "<f4", 3072, payload_start + 3072)
    assert (col == 1.0).all() and (icl == 2.0).all()
    assert data[-32:] == hashlib.sha256(data[:-32]).digest()


def test_padding_between_tensors_is_zero_and_aligned():
    tensors = {"a": np.arange(3, dtype=np.float32), "b": np.arange(5, dtype=np.float32) + 1}
    data = cf.to_bytes(fixture_metadata(), tensors)
    ctx = cf.from_bytes(data)
    np.testing.assert_array_equal(ctx.tensor("b"), tensors["b"])
    head_len = len(data) - 32 - struct.unpack_from("<Q", data, 152)[0]
    assert head_len % 64 == 0
    # "a" is 12 bytes at offset 0, "b" starts at 64: 52 zero bytes between.
    assert data[head_len + 12: head_len + 64] == bytes(52)


def test_round_trip_is_deterministic(tmp_path):
    data = encode_fixture()
    assert data == encode_fixture()
    ctx = cf.from_bytes(data)
    assert ctx.metadata == fixture_metadata() and ctx.version == 1
    assert np.float32(ctx.tensor("icl.v.0").reshape(-1)[0]).tobytes() == np.float32(2.0).tobytes()
    path = tmp_path / "context.irctx"
    path.write_bytes(data)
    mapped = cf.read(path)
    assert mapped.metadata == ctx.metadata
    assert cf.to_bytes(mapped.metadata, {n: mapped.tensor(n) for n in mapped.names}) == data


def test_regression_context_without_classes_round_trips(tmp_path):
    meta = fixture_metadata(class_count=0, class_permutations=[])
    data = encode_fixture(meta)
    assert cf.from_bytes(data).metadata == meta
    path = tmp_path / "context.irctx"
    path.write_bytes(data)
    assert cf.read(path).metadata == meta


def test_rejects_corruption_and_invalid_values():
    corrupt = bytearray(encode_fixture())
    corrupt[cf.HEADER_BYTES] ^= 1
    with pytest.raises(cf.ContextError, match="checksum"):
        cf.from_bytes(bytes(corrupt))
    # Re-signed, the flipped class permutation is caught by validation.
    with pytest.raises(cf.ContextError, match="class permutation is invalid"):
        cf.from_bytes(resign(corrupt))
    with pytest.raises(cf.ContextError, match="non-finite"):
        cf.to_bytes(fixture_metadata(), {"bad": np.array([np.nan, 1.0], np.float32)})
    # A non-finite value written by another encoder is refused on load.
    data = bytearray(encode_fixture())
    start = len(data) - 32 - 12288 - 3072
    data[start:start + 4] = np.float32(np.inf).tobytes()
    with pytest.raises(cf.ContextError, match="non-finite"):
        cf.from_bytes(resign(data))


def test_rejects_resource_and_directory_metadata():
    data = bytearray(encode_fixture())
    struct.pack_into("<I", data, 8 + 4 + 4 + 32 + 32 + 32 + 20, 0)  # tensor count 0
    with pytest.raises(cf.ContextError):
        cf.from_bytes(resign(data))
    with pytest.raises(cf.ContextError, match="resource limits"):
        cf.to_bytes(fixture_metadata(feature_count=cf.MAX_FEATURE_COUNT + 1,
                                     feature_permutations=[0] * (2 * (cf.MAX_FEATURE_COUNT + 1))),
                    {"x": np.zeros(1, np.float32)})


@pytest.mark.parametrize("offset,value,message", [
    (0, b"IRCNTXX\0", "magic"),
    (8, struct.pack("<I", 4), "version 4 is unsupported"),
    (12, struct.pack("<I", 2), "kind"),
    (112, struct.pack("<I", 4), "architecture"),
    (160, struct.pack("<I", 1), "reserved"),
    (136, struct.pack("<I", 5), "permutation lengths"),
    (144, struct.pack("<Q", 1 << 23), "resource limit"),
])
def test_rejects_header_fields(offset, value, message):
    data = bytearray(encode_fixture())
    data[offset:offset + len(value)] = value
    with pytest.raises(cf.ContextError, match=message):
        cf.from_bytes(resign(data))


def test_rejects_directory_errors():
    base = encode_fixture()
    first = 164 + 80
    # Nonzero dtype tag in version 1.
    data = bytearray(base)
    struct.pack_into("<H", data, first + 6, 1)
    with pytest.raises(cf.ContextError, match="directory entry is invalid"):
        cf.from_bytes(resign(data))
    # Misaligned payload offset of the second tensor.
    second = first + 24 + 4 * 8 + len("column.k.0")
    data = bytearray(base)
    struct.pack_into("<Q", data, second + 8, 3072 + 4)
    with pytest.raises(cf.ContextError, match="offset or length"):
        cf.from_bytes(resign(data))
    # Byte length that does not match the shape.
    data = bytearray(base)
    struct.pack_into("<Q", data, second + 16, 12288 - 4)
    with pytest.raises(cf.ContextError, match="does not match its shape"):
        cf.from_bytes(resign(data))
    # Names out of order ("icl.v.0" renamed to "a.v.0...", same length).
    data = bytearray(base)
    name_at = second + 24 + 4 * 8
    data[name_at:name_at + 7] = b"a.v.0.x"
    with pytest.raises(cf.ContextError, match="sorted"):
        cf.from_bytes(resign(data))
    # Nonzero alignment padding before the payload.
    data = bytearray(base)
    pad_at = second + 24 + 4 * 8 + len("icl.v.0")
    data[pad_at] = 1
    with pytest.raises(cf.ContextError, match="padding"):
        cf.from_bytes(resign(data))
    # Truncated file.
    with pytest.raises(cf.ContextError):
        cf.from_bytes(base[:100])


def test_rejects_reduced_precision_and_packed_versions():
    data = bytearray(encode_fixture())
    struct.pack_into("<I", data, 8, 3)
    with pytest.raises(cf.ContextError, match="packed ICL keys"):
        cf.from_bytes(resign(data))
    # Version 2 with the FP32 tag (1) loads; a BF16 tag (2) is refused.
    data = bytearray(encode_fixture())
    struct.pack_into("<I", data, 8, 2)
    first = 164 + 80
    second = first + 24 + 4 * 8 + len("column.k.0")
    struct.pack_into("<H", data, first + 6, 1)
    struct.pack_into("<H", data, second + 6, 1)
    assert cf.from_bytes(resign(data)).version == 2
    struct.pack_into("<H", data, second + 6, 2)
    with pytest.raises(cf.ContextError, match="BF16"):
        cf.from_bytes(resign(data))


def test_fp16_tensors_round_trip_as_version_2():
    """An optimize="auto" context: FP16 ICL tensors, FP32 column tensors,
    written as version 2 with per-tensor tags (FP32 1, FP16 3; src/config.rs:79-86)."""
    rng = np.random.default_rng(0)
    tensors = {"column.k.0": rng.standard_normal((2, 8, 3, 16)).astype(np.float32),
               "icl.v.0": rng.standard_normal((2, 8, 3, 64)).astype(np.float16)}
    data = cf.to_bytes(fixture_metadata(), tensors)
    assert struct.unpack_from("<I", data, 8)[0] == 2
    first = 164 + 80
    second = first + 24 + 4 * 8 + len("column.k.0")
    assert struct.unpack_from("<H", data, first + 6)[0] == 1 and struct.unpack_from("<H", data, second + 6)[0] == 3
    assert struct.unpack_from("<Q", data, second + 16)[0] == 2 * 3072
    ctx = cf.from_bytes(data)
    assert ctx.version == 2 and ctx.tensor("icl.v.0").dtype == np.float16
    np.testing.assert_array_equal(ctx.tensor("icl.v.0"), tensors["icl.v.0"])
    np.testing.assert_array_equal(ctx.tensor("column.k.0"), tensors["column.k.0"])
    assert cf.to_bytes(ctx.metadata, {n: ctx.tensor(n) for n in ctx.names}) == data
    bad = dict(tensors)
    bad["icl.v.0"] = bad["icl.v.0"].copy()
    bad["icl.v.0"][0, 0, 0, 0] = np.float16(np.inf)
    with pytest.raises(cf.ContextError, match="non-finite"):
        cf.to_bytes(fixture_metadata(), bad)


def test_cached_read_accepts_only_the_expected_context(tmp_path):
    meta, tensors = fixture_metadata(), fixture_tensors()
    path = tmp_path / "context.irctx"
    assert cf.read_cached(path, meta) is None
    cf.write(path, meta, [(n, t.shape) for n, t in tensors.items()],
             lambda n, s, c: tensors[n].reshape(-1)[s:s + c])
    got = cf.read_cached(path, meta)
    assert got is not None and got.metadata == meta
    assert cf.read_cached(path, fixture_metadata(context_sha256=bytes([3]) * 32)) is None
    data = path.read_bytes()
    path.write_bytes(data[: len(data) // 2])
    assert cf.read_cached(path, meta) is None


def test_streamed_write_matches_in_memory_encoding(tmp_path):
    meta, tensors = fixture_metadata(), fixture_tensors()
    path = tmp_path / "context.irctx"
    specs = [(n, t.shape) for n, t in tensors.items()]
    cf.write(path, meta, specs, lambda n, s, c: tensors[n].reshape(-1)[s:s + c], chunk_floats=100)
    assert path.read_bytes() == encode_fixture()
    assert cf.encoded_len(meta, specs) == len(encode_fixture())


def test_concurrent_writes_leave_one_private_context(tmp_path):
    meta, tensors = fixture_metadata(), fixture_tensors()
    path = tmp_path / "context.irctx"
    specs = [(n, t.shape) for n, t in tensors.items()]
    threads = [threading.Thread(target=cf.write, args=(path, meta, specs,
                                                       lambda n, s, c: tensors[n].reshape(-1)[s:s + c]))
               for _ in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert path.read_bytes() == encode_fixture()
    assert list(tmp_path.glob("*.tmp")) == []
    if os.name == "posix":
        assert path.stat().st_mode & 0o777 == 0o600


def test_failed_write_removes_its_temporary_file(tmp_path):
    path = tmp_path / "context.irctx"
    path.mkdir()
    (path / "kept").write_bytes(b"kept")
    tensors = fixture_tensors()
    with pytest.raises(OSError):
        cf.write(path, fixture_metadata(), [(n, t.shape) for n, t in tensors.items()],
                 lambda n, s, c: tensors[n].reshape(-1)[s:s + c])
    assert list(tmp_path.glob("*.tmp")) == []
    assert (path / "kept").read_bytes() == b"kept"

    def failing(name, start, count):
        raise RuntimeError("device read failed")

    with pytest.raises(RuntimeError):
        cf.write(tmp_path / "other.irctx", fixture_metadata(), [("a", (4,))], failing)
    assert list(tmp_path.glob("*.tmp")) == [] and not (tmp_path / "other.irctx").exists()


def test_context_tensor_specs_follow_the_reference_order():
    specs = [s[:2] for s in cf.context_tensor_specs(2, 100, 7)]
    assert len(specs) == 30
    assert specs[0] == ("column.0.key", (2, 11, 8, 128, 16)) and specs[5] == ("column.2.value", (2, 11, 8, 128, 16))
    assert specs[6] == ("icl.0.key", (2, 8, 100, 64)) and specs[29] == ("icl.11.value", (2, 8, 100, 64))
    f16 = cf.context_tensor_specs(1, 5, 2, np.float16)
    assert {s[2] for s in f16[:6]} == {np.dtype(np.float32)} and {s[2] for s in f16[6:]} == {np.dtype(np.float16)}
    # File order is bytewise: icl.1.* < icl.10.* < icl.11.* < icl.2.*
    meta = fixture_metadata(training_rows=1, feature_count=1, ensemble_count=1, class_permutations=[0, 1, 2],
                            feature_permutations=[0])
    head, entries, _ = cf._layout(meta, cf.context_tensor_specs(1, 1, 1))
    names = [e.name for e in entries]
    assert names.index("icl.1.value") + 1 == names.index("icl.10.key")
    assert names.index("icl.11.value") + 1 == names.index("icl.2.key")


def test_identity_covers_every_input():
    """context_metadata's identity (cpu.rs:841-858) changes with each input it
    covers and with nothing else."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((1, 5, 3)).astype(np.float32)
    y = np.array([[0, 1, 0, 1, 1]], np.float32)
    cp, fp = np.array([0, 1], np.uint64), np.array([0, 1, 2], np.uint64)
    src = "ab" * 32
    base = cf.context_identity(src, "safe", x, y, cp, fp)
    assert base == cf.context_identity(src, "safe", x.copy(), y.copy(), cp.copy(), fp.copy())
    x2 = x.copy()
    x2[0, 4, 2] = np.nextafter(x2[0, 4, 2], np.float32(9))
    variants = [cf.context_identity("cd" * 32, "safe", x, y, cp, fp), cf.context_identity(src, "auto", x, y, cp, fp),
                cf.context_identity(src, "safe", x2, y, cp, fp),
                cf.context_identity(src, "safe", x, np.array([[1, 1, 0, 1, 1]], np.float32), cp, fp),
                cf.context_identity(src, "safe", x, y, cp[::-1].copy(), fp),
                cf.context_identity(src, "safe", x, y, cp, np.array([2, 1, 0], np.uint64)),
                cf.context_identity(src, "safe", x, y, cp, fp, version="0.1.1"),
                cf.context_identity(src, "safe", x.reshape(1, 3, 5), y[:, :3], cp, np.arange(5, dtype=np.uint64))]
    assert len({base, *variants}) == len(variants) + 1
    # The digest is SHA-256 over the documented byte stream.
    stream = (b"ironicl-context-v2\0" + b"0.1.0\0" + src.encode() + b"\0" + b"safe\0" + struct.pack("<3Q", 1, 5, 3)
              + x.tobytes() + y.tobytes() + cp.astype("<u8").tobytes() + fp.astype("<u8").tobytes())
    assert base == hashlib.sha256(stream).digest()


# ---- the cache directory (tests/test_cache.py) ----

DAY = 24 * 3600


@pytest.fixture
def cache(tmp_path):
    now = time.time()
    for name, size, age in (("a", 10, 3), ("b", 20, 2), ("c", 30, 1)):
        p = tmp_path / f"{name}.irctx"
        p.write_bytes(b"x" * size)
        os.utime(p, (now - age * DAY, now - age * DAY))
    stale = tmp_path / ".ironicl-1-1.tmp"
    stale.write_bytes(b"x")
    os.utime(stale, (now - 7200, now - 7200))
    writing = tmp_path / ".ironicl-1-2.tmp"
    writing.write_bytes(b"x")
    return tmp_path, stale, writing


def names(info):
    return [e.path.stem for e in info.entries]


def test_info_lists_contexts_most_recently_used_first(cache):
    d, _, _ = cache
    info = cf.cache_info(d)
    assert names(info) == ["c", "b", "a"] and info.size_bytes == 60 and "3 contexts" in str(info)
    assert cf.cache_info(d / "missing").entries == ()
    with pytest.raises(ValueError):
        cf.cache_info(False)


def test_older_than_and_max_size(cache):
    d, _, _ = cache
    assert names(cf.clear_cache(d, older_than=timedelta(days=1.5))) == ["b", "a"]
    assert names(cf.cache_info(d)) == ["c"]


def test_max_size_removes_the_least_recently_used(cache):
    d, _, _ = cache
    assert cf.clear_cache(d, max_size="1K").entries == ()
    assert names(cf.clear_cache(d, max_size=35)) == ["b", "a"]
    with pytest.raises(ValueError):
        cf.clear_cache(d, max_size=-1)


def test_clear_removes_everything_and_stale_temporary_files(cache):
    d, stale, writing = cache
    assert cf.clear_cache(d).size_bytes == 60
    assert cf.cache_info(d).entries == ()
    assert not stale.exists() and writing.exists()


def test_cache_dir_resolution(monkeypatch, tmp_path):
    assert cf.resolve_cache_dir(False) is None
    assert cf.resolve_cache_dir(tmp_path) == tmp_path
    monkeypatch.setenv("IRONICL_CACHE_DIR", str(tmp_path / "o"))
    assert cf.resolve_cache_dir(None) == tmp_path / "o" and cf.resolve_cache_dir(True) == tmp_path / "o"
    monkeypatch.delenv("IRONICL_CACHE_DIR")
    monkeypatch.setenv("XDG_CACHE_HOME", str(tmp_path / "x"))
    assert cf.resolve_cache_dir(None) == tmp_path / "x" / "ironicl" / "contexts"


def test_parse_size():
    assert cf.parse_size("512M") == 512 << 20 and cf.parse_size("16GiB") == 16 << 30
    assert cf.parse_size("1.5k") == 1536 and cf.parse_size("100") == 100 and cf.parse_size("2tb") == 2 << 40
    for bad in ("", "G", "16iB", "-1", "1e3", "inf"):
        with pytest.raises(ValueError):
            cf.parse_size(bad)
