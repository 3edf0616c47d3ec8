"""IRCNTXT export and import of GPU-built contexts, and the context cache,
through the C ABI on the GPU: a context streamed out of HBM is byte-identical
to the same context downloaded at build time, a reloaded context predicts
bitwise like the one built in place, and cache_dir hits, misses and rebuilds
as Executor::build_context does (cpu.rs:640-672, tests/test_cache.py)."""

import io
import os
import shutil

import numpy as np
import pytest

from ironicl_amd import context_file as cf
from ironicl_amd import hip
from ironicl_amd import tabicl

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def clf(clf_weights):
    return tabicl.Executor("classifier", clf_weights, hip.Device(0))


@pytest.fixture(scope="module")
def data():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 300, 5)).astype(np.float32)
    y = (rng.standard_normal((2, 300)) > 0).astype(np.float32) + (x[:, :, 0] > 1)
    xt = rng.standard_normal((2, 40, 5)).astype(np.float32)
    perms = np.array([[0, 1, 2], [2, 0, 1]], np.uint64)
    return x, y, xt, perms


def test_export_from_hbm_matches_download_and_reloads(clf, data, tmp_path):
    x, y, xt, perms = data
    resident = clf.build_context(x, y, class_permutations=perms)
    assert resident.context is None  # nothing on the host: export streams from HBM
    downloaded = clf.build_context(x, y, class_permutations=perms, download=True)
    a, b = tmp_path / "hbm.irctx", tmp_path / "host.irctx"
    resident.save_context(a)
    downloaded.save_context(b)
    assert a.read_bytes() == b.read_bytes()
    assert resident.context_encoded_len() == a.stat().st_size

    ctx = cf.read(a)
    assert ctx.metadata == resident.metadata
    ck, cv, ik, iv = downloaded.context
    for i in range(3):
        np.testing.assert_array_equal(ctx.tensor(f"column.{i}.key"), ck[i])
        np.testing.assert_array_equal(ctx.tensor(f"column.{i}.value"), cv[i])
    for i in range(12):
        np.testing.assert_array_equal(ctx.tensor(f"icl.{i}.key"), ik[i])
        np.testing.assert_array_equal(ctx.tensor(f"icl.{i}.value"), iv[i])

    reloaded = clf.load_context(a)
    want = resident.predict_raw(xt).logits
    np.testing.assert_array_equal(reloaded.predict_raw(xt).logits, want)
    np.testing.assert_array_equal(reloaded.predict_probabilities(xt), resident.predict_probabilities(xt))
    # Re-export of the reloaded context (host views of the mapping) is byte-stable.
    c = tmp_path / "again.irctx"
    reloaded.save_context(c)
    assert c.read_bytes() == a.read_bytes()

    sink = io.BytesIO()
    resident.encode_context(sink)
    assert sink.getvalue() == a.read_bytes()
    np.testing.assert_array_equal(clf.load_context_bytes(sink.getvalue()).predict_raw(xt).logits, want)


def test_load_rejects_another_models_context(clf, clf_weights, data, tmp_path):
    x, y, _, perms = data
    path = tmp_path / "c.irctx"
    clf.build_context(x, y, class_permutations=perms).save_context(path)
    other = tabicl.Executor("classifier", clf_weights, clf.device, source_sha256="ab" * 32)
    with pytest.raises(cf.ContextError, match="model SHA-256"):
        other.load_context(path)


def test_cache_dir_hit_miss_and_rebuild(clf, data, tmp_path):
    x, y, xt, perms = data
    d = tmp_path / "cache"
    calls = []
    built = clf.build_context(x, y, class_permutations=perms, cache_dir=d, progress=lambda *a: calls.append(a))
    assert calls, "a miss builds"
    (entry,) = cf.cache_info(d).entries
    assert entry.path == cf.cache_path(d, built.metadata)
    if os.name == "posix":
        assert entry.path.stat().st_mode & 0o777 == 0o600
    want = built.predict_raw(xt).logits

    day = 24 * 3600
    os.utime(entry.path, (entry.path.stat().st_atime - day, entry.path.stat().st_mtime - day))
    old = cf.cache_info(d).entries[0].last_used
    calls.clear()
    hit = clf.build_context(x, y, class_permutations=perms, cache_dir=d, progress=lambda *a: calls.append(a))
    assert not calls, "a hit loads the file without building"
    assert cf.cache_info(d).entries[0].last_used > old
    np.testing.assert_array_equal(hit.predict_raw(xt).logits, want)

    # Other labels: another identity, another entry.
    y2 = y.copy()
    y2[0, 0] = 2 - y2[0, 0]
    other = clf.build_context(x, y2, class_permutations=perms, cache_dir=d)
    assert len(cf.cache_info(d).entries) == 2
    # A valid context of other data stored under this context's name is rebuilt.
    shutil.copyfile(cf.cache_path(d, other.metadata), entry.path)
    calls.clear()
    rebuilt = clf.build_context(x, y, class_permutations=perms, cache_dir=d, progress=lambda *a: calls.append(a))
    assert calls
    np.testing.assert_array_equal(rebuilt.predict_raw(xt).logits, want)
    assert cf.read(entry.path).metadata == built.metadata


def test_unwritable_cache_does_not_fail_the_build(clf, data, tmp_path):
    if os.name != "posix" or os.geteuid() == 0:
        pytest.skip("needs POSIX permissions as a non-root user")
    x, y, xt, perms = data
    d = tmp_path / "ro"
    d.mkdir()
    d.chmod(0o500)
    try:
        st = clf.build_context(x, y, class_permutations=perms, cache_dir=d)
        assert cf.cache_info(d).entries == ()
        np.testing.assert_array_equal(st.predict_raw(xt).logits,
                                      clf.build_context(x, y, class_permutations=perms).predict_raw(xt).logits)
    finally:
        d.chmod(0o700)
