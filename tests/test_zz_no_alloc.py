"""The no-allocation ICL attention (irx_icl_attention_noalloc) against the
allocating kernel harness (irx_test_icl_attention) on the same device: two
calls in a row, the second smaller, each bitwise equal; and a shape whose
split-K partials exceed the library's scratch array refused before any work.
Collected last: its entry point shares one scratch array per device."""

import numpy as np
import pytest

from ironicl_amd import hip, hipmem

pytestmark = pytest.mark.gpu


def values(count, seed, scale=1.0):
    return (np.random.default_rng(seed).standard_normal(count) * scale).astype(np.float32)


@pytest.fixture(scope="module")
def device():
    return hip.Device(0)


def harness(device, q, k, v):
    pairs, query_rows, _ = q.shape
    out = np.zeros_like(q)
    F = hip.fptr
    hip.check(hip.lib().irx_test_icl_attention(device.handle, F(q), F(k), F(v), pairs, query_rows, k.shape[1],
                                               F(out)))
    return out


def no_alloc(device, q, k, v):
    """Token rows [pairs / 8, query_rows, 512] back to [pairs, query_rows, 64]."""
    pairs, query_rows, _ = q.shape
    dq, dk, dv = (hipmem.DeviceArray.from_host(a) for a in (q, k, v))
    dout = hipmem.DeviceArray((pairs // 8, query_rows, 512))
    hip.check(hip.lib().irx_icl_attention_noalloc(device.handle, dq.ptr, dk.ptr, dv.ptr, pairs, query_rows,
                                                  k.shape[1], dout.ptr, None))
    hipmem.synchronize()
    tokens = dout.to_host().reshape(pairs // 8, query_rows, 8, 64)
    return np.ascontiguousarray(tokens.transpose(0, 2, 1, 3).reshape(pairs, query_rows, 64))


@pytest.mark.parametrize("shapes", [((16, 512, 5000), (8, 17, 3000)), ((8, 64, 20000), (8, 1, 700))])
def test_no_alloc_attention_matches_the_harness(device, shapes):
    for call, (pairs, query_rows, rows) in enumerate(shapes):
        print(f"no-alloc attention call {call}: pairs {pairs}, queries {query_rows}, keys {rows}", flush=True)
        q = values(pairs * query_rows * 64, 10 * call + 1, 3.0).reshape(pairs, query_rows, 64)
        k = values(pairs * rows * 64, 10 * call + 2).reshape(pairs, rows, 64)
        v = values(pairs * rows * 64, 10 * call + 3).reshape(pairs, rows, 64)
        want = harness(device, q, k, v)
        got = no_alloc(device, q, k, v)
        np.testing.assert_array_equal(got, want, err_msg=f"call {call}")


def test_no_alloc_attention_refuses_what_its_scratch_cannot_hold(device):
    """8 pairs x 8,448 queries x 4,096 keys splits its keys 8 ways: 8 x 8 x
    8,448 x 65 partial floats (140 MB), past the 64 MiB scratch. Refused on the
    host; the buffers are real and sized for the shape all the same."""
    pairs, query_rows, rows = 8, 8448, 4096
    q = hipmem.DeviceArray.from_host(np.zeros((pairs, query_rows, 64), np.float32))
    kv = hipmem.DeviceArray.from_host(np.zeros((pairs, rows, 64), np.float32))
    out = hipmem.DeviceArray((pairs // 8, query_rows, 512))
    status = hip.lib().irx_icl_attention_noalloc(device.handle, q.ptr, kv.ptr, kv.ptr, pairs, query_rows, rows,
                                                 out.ptr, None)
    assert status == hip.INVALID_ARGUMENT
    assert b"no-allocation entry point holds" in hip.lib().irx_last_error()
    assert hip.lib().irx_icl_attention_noalloc(device.handle, None, kv.ptr, kv.ptr, 8, 1, 1, out.ptr,
                                               None) == hip.INVALID_ARGUMENT
