"""The no-allocation ICL attention (irx_icl_attention_noalloc) against the
allocating kernel harness (irx_test_icl_attention) on the same device: two
calls in a row, the second smaller, each bitwise equal; the shape with the
largest split-K partials the split plan makes on 256 CUs; and invalid calls
refused before any work. Collected last: its entry point shares one scratch
array per device."""

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


def test_no_alloc_attention_at_the_largest_partials(device):
    """The split plan's partials are largest just below one round of
    (query tile, pair) units: 8 pairs x 7,936 queries (248 units on 256 CUs)
    split 2 ways over 4,096 keys, 2 x 8 x 7,936 x 65 floats (33 MB), inside
    the 64 MiB scratch. (At a full round or more, whole rounds run unsplit and
    only the units left over are split, into at most one round: at most 17
    MB.) Bitwise the harness's result."""
    pairs, query_rows, rows = 8, 7936, 4096
    print(f"no-alloc attention: pairs {pairs}, queries {query_rows}, keys {rows}", flush=True)
    q = values(pairs * query_rows * 64, 31, 3.0).reshape(pairs, query_rows, 64)
    k = values(pairs * rows * 64, 32).reshape(pairs, rows, 64)
    v = values(pairs * rows * 64, 33).reshape(pairs, rows, 64)
    np.testing.assert_array_equal(no_alloc(device, q, k, v), harness(device, q, k, v))


def test_no_alloc_attention_refuses_invalid_calls(device):
    """A null operand and an out-of-range shape are refused on the host with
    IRX_INVALID_ARGUMENT, before any work."""
    kv = hipmem.DeviceArray.from_host(np.zeros((8, 16, 64), np.float32))
    out = hipmem.DeviceArray((1, 16, 512))
    assert hip.lib().irx_icl_attention_noalloc(device.handle, None, kv.ptr, kv.ptr, 8, 1, 1, out.ptr,
                                               None) == hip.INVALID_ARGUMENT
    assert hip.lib().irx_icl_attention_noalloc(device.handle, kv.ptr, kv.ptr, kv.ptr, 8, 1 << 25, 16, out.ptr,
                                               None) == hip.INVALID_ARGUMENT
    assert b"out of range" in hip.lib().irx_last_error()
