"""NumPy restatement of the FP8 ICL cache of optimize="fast" for the tests.

E4M3 here is OCP's (bias 7, no infinities, 0x7f/0xff NaN, largest 448), as
the reference encodes it (src/kernels/cuda/ops/fp8.rs:30-62): round to the
nearest, ties to an even mantissa, saturate at +-448. Scales are per (pair,
dim), peak / 448 or 1 (kernels.rs:828-845); values are encoded as
e4m3(value / scale) (kernels.rs:847-875)."""

import numpy as np


def e4m3(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    bits = x.view(np.uint32)
    sign = ((bits >> 24) & 0x80).astype(np.uint32)
    mag = np.fmin(np.abs(x), np.float32(448.0)).astype(np.float32)
    steps = ((mag * np.float32(512.0) + np.float32(8388608.0)) - np.float32(8388608.0)).astype(np.uint32)
    mb = mag.view(np.uint32)
    exponent = ((mb >> 23) & 0xFF).astype(np.int64) - 127
    mantissa = ((mb >> 20) & 7).astype(np.int64)
    rest = mb & 0xFFFFF
    mantissa += (rest > 0x80000) | ((rest == 0x80000) & (mantissa & 1 == 1))
    carry = mantissa == 8
    mantissa[carry] = 0
    exponent[carry] += 1
    sat = (exponent > 8) | ((exponent == 8) & (mantissa == 7))
    normal = sign | (((exponent + 7) << 3) | mantissa).astype(np.uint32)
    out = np.where(mag < np.float32(1 / 64), sign | steps, np.where(sat, sign | 0x7E, normal))
    return out.astype(np.uint8)


def e4m3_value(code) -> np.ndarray:
    """Decode E4M3 bytes (NaN for 0x7f / 0xff)."""
    c = np.asarray(code, dtype=np.int64)
    s, e, m = c >> 7, (c >> 3) & 15, c & 7
    v = np.where(e == 0, m * 2.0 ** -9, (1 + m / 8) * 2.0 ** (e - 7))
    v = np.where((e == 15) & (m == 7), np.nan, v)
    return np.where(s == 1, -v, v)


def scales(values16: np.ndarray) -> np.ndarray:
    """[pairs, rows, 64] FP16 -> scales [pairs, 64]."""
    peak = np.abs(values16.astype(np.float32)).max(axis=1)
    return np.where(peak > 0, peak / np.float32(448.0), np.float32(1.0)).astype(np.float32)


def stored_position(key):
    """Position of key (mod 16) in a group of the V^T tile: 0..3, 8..11, 4..7, 12..15."""
    return (key & 3) | ((key & 4) << 1) | ((key & 8) >> 1)


def encode_block(k16: np.ndarray, v16: np.ndarray):
    """FP16 K, V [pairs, rows, 64] -> (K bytes [pairs, Np, 64], V^T bytes
    [pairs, Np / 64, 64, 64], key scales, value scales)."""
    pairs, rows, _ = k16.shape
    n_pad = (rows + 63) // 64 * 64
    ks, vs = scales(k16), scales(v16)
    k8 = np.zeros((pairs, n_pad, 64), np.uint8)
    k8[:, :rows] = e4m3(k16.astype(np.float32) / ks[:, None, :])
    vq = np.zeros((pairs, n_pad, 64), np.uint8)
    vq[:, :rows] = e4m3(v16.astype(np.float32) / vs[:, None, :])
    vt = np.zeros((pairs, n_pad // 64, 64, 64), np.uint8)
    key = np.arange(64)
    pos = 16 * (key // 16) + stored_position(key % 16)
    tiles = vq.reshape(pairs, n_pad // 64, 64, 64)  # [pair, tile, key, dim]
    vt[:, :, :, pos] = tiles.transpose(0, 1, 3, 2)
    return k8, vt, ks, vs
