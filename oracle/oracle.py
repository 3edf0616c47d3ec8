"""ctypes wrapper of the oracle (libtabicl_oracle.so).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg load this as the checker / CPU baseline. The product path
(ironicl_amd) never imports it.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtabicl_oracle.so")

EXACT, NATIVE = 0, 1
CLASSIFIER, REGRESSOR = 0, 1

_F = ctypes.POINTER(ctypes.c_float)
_LOOKUP = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p, ctypes.c_char_p,
                           ctypes.POINTER(_F), ctypes.POINTER(ctypes.c_size_t))
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sz, vp, cp = ctypes.c_size_t, ctypes.c_void_p, ctypes.c_char_p
        PF = ctypes.POINTER(_F)
        L.ora_model_new.restype = vp
        L.ora_model_new.argtypes = [ctypes.c_int, _LOOKUP, vp, ctypes.c_int, cp, sz]
        L.ora_model_free.argtypes = [vp]
        L.ora_model_width.restype = sz
        L.ora_model_width.argtypes = [vp]
        L.ora_set_threads.argtypes = [ctypes.c_int]
        L.ora_get_threads.restype = ctypes.c_int
        L.ora_build_context.argtypes = [vp, sz, sz, sz, _F, _F, PF, PF, PF, PF, cp, sz]
        L.ora_predict_cached.argtypes = [vp, sz, sz, sz, sz, _F, PF, PF, PF, PF, _F, cp, sz]
        L.ora_predict_uncached.argtypes = [vp, sz, sz, sz, sz, _F, _F, _F, cp, sz]
        L.ora_trace_uncached.argtypes = [vp, sz, sz, sz, sz, _F, _F, _F, _F, cp, sz]
        PS = ctypes.POINTER(sz)
        L.ora_context_columns.argtypes = [vp, sz, sz, _F, _F, PS, sz, PF, cp, sz]
        L.ora_context_rows.argtypes = [vp, sz, sz, _F, _F, PS, sz, PF, PF, PF, PF, PF, PF, cp, sz]
        L.ora_affine.argtypes = [_F, sz, sz, _F, _F, sz, _F]
        L.ora_layer_norm.argtypes = [_F, sz, sz, _F, _F, _F]
        L.ora_gelu.argtypes = [ctypes.c_int, _F, sz, _F]
        L.ora_fast_exp_negative.restype = ctypes.c_float
        L.ora_fast_exp_negative.argtypes = [ctypes.c_float]
        L.ora_bounded_exp.restype = ctypes.c_float
        L.ora_bounded_exp.argtypes = [ctypes.c_float]
        L.ora_one_hot_linear.argtypes = [_F, sz, _F, _F, sz, sz, _F]
        L.ora_rope.argtypes = [_F, sz, sz, sz, _F, sz, _F]
        L.ora_qassmax.argtypes = [_F, sz, sz, sz, sz, sz] + [_F] * 9
        L.ora_attention.argtypes = [ctypes.c_int, _F, sz, _F, _F, sz, sz, sz, _F]
        L.ora_attention.restype = ctypes.c_int
        L.ora_attention_materialized.argtypes = [_F, sz, _F, _F, sz, sz, sz, _F]
        L.ora_aggregate.argtypes = [_F, sz, sz, sz, ctypes.POINTER(ctypes.c_uint64), ctypes.c_float,
                                    ctypes.c_int, _F]
        L.ora_aggregate.restype = ctypes.c_int
        L.ora_regression_summary.argtypes = [_F, sz, sz, sz, _F, sz, _F, _F]
        L.ora_regression_summary.restype = ctypes.c_int
        L.ora_regression_outputs.argtypes = [_F, sz, sz, sz, _F, sz, _F, _F, _F, _F]
        L.ora_regression_outputs.restype = ctypes.c_int
        _lib = L
    return _lib


def fp(a: np.ndarray | None):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_F)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def ptr_array(arrays):
    arr = (_F * len(arrays))()
    for i, a in enumerate(arrays):
        arr[i] = fp(a)
    return arr


def set_threads(n: int) -> None:
    lib().ora_set_threads(int(n))


class OracleModel:
    """The reference's Executor/StaticExecutor restated on the CPU."""

    def __init__(self, task: str, weights: dict[str, np.ndarray], math: int = EXACT):
        self.task = task
        self._weights = {k: f32(v) for k, v in weights.items()}

        @_LOOKUP
        def lookup(_user, name, data, length):
            arr = self._weights.get(name.decode())
            if arr is None:
                return 1
            data[0] = arr.ctypes.data_as(_F)
            length[0] = arr.size
            return 0

        err = ctypes.create_string_buffer(512)
        t = CLASSIFIER if task == "classifier" else REGRESSOR
        self._handle = lib().ora_model_new(t, lookup, None, math, err, 512)
        if not self._handle:
            raise ValueError(err.value.decode())
        self.width = lib().ora_model_width(self._handle)

    def __del__(self):
        h = getattr(self, "_handle", None)
        if h and _lib is not None:
            _lib.ora_model_free(h)
            self._handle = None

    def build_context(self, x: np.ndarray, y: np.ndarray):
        """x [B,N,H], y [B,N] -> (column_keys[3], column_values[3], icl_keys[12], icl_values[12])."""
        b, n, h = x.shape
        x, y = f32(x), f32(y)
        ck = [np.zeros((b, h + 4, 8, 128, 16), np.float32) for _ in range(3)]
        cv = [np.zeros_like(ck[0]) for _ in range(3)]
        ik = [np.zeros((b, 8, n, 64), np.float32) for _ in range(12)]
        iv = [np.zeros_like(ik[0]) for _ in range(12)]
        err = ctypes.create_string_buffer(512)
        st = lib().ora_build_context(self._handle, b, n, h, fp(x), fp(y), ptr_array(ck), ptr_array(cv),
                                     ptr_array(ik), ptr_array(iv), err, 512)
        if st:
            raise ValueError(err.value.decode())
        return ck, cv, ik, iv

    def predict_cached(self, context, x: np.ndarray) -> np.ndarray:
        ck, cv, ik, iv = context
        b, q, h = x.shape
        n = ik[0].shape[2]
        x = f32(x)
        out = np.zeros((b, q, self.width), np.float32)
        err = ctypes.create_string_buffer(512)
        st = lib().ora_predict_cached(self._handle, b, n, h, q, fp(x), ptr_array(ck), ptr_array(cv),
                                      ptr_array(ik), ptr_array(iv), fp(out), err, 512)
        if st:
            raise ValueError(err.value.decode())
        return out

    def predict_uncached(self, x_train, y, x_test) -> np.ndarray:
        b, n, h = x_train.shape
        q = x_test.shape[1]
        x = f32(np.concatenate([x_train, x_test], axis=1))
        out = np.zeros((b, q, self.width), np.float32)
        err = ctypes.create_string_buffer(512)
        st = lib().ora_predict_uncached(self._handle, b, n + q, n, h, fp(x), fp(f32(y)), fp(out), err, 512)
        if st:
            raise ValueError(err.value.decode())
        return out

    def context_columns(self, x: np.ndarray, y: np.ndarray, features) -> list[np.ndarray]:
        """One estimator (x [N,H], y [N]): the six column K/V tensors [nf,8,128,16]
        (key, value per block) of the listed features, from the full N-row column
        stream as build_context computes them."""
        n, h = x.shape
        feats = np.ascontiguousarray(features, dtype=np.uintp)
        kv = [np.zeros((len(feats), 8, 128, 16), np.float32) for _ in range(6)]
        err = ctypes.create_string_buffer(512)
        x, y = f32(x), f32(y)
        st = lib().ora_context_columns(self._handle, n, h, fp(x), fp(y),
                                       feats.ctypes.data_as(ctypes.POINTER(ctypes.c_size_t)), len(feats),
                                       ptr_array(kv), err, 512)
        if st:
            raise ValueError(err.value.decode())
        return kv

    def context_rows(self, x: np.ndarray, y: np.ndarray, rows, ck, cv, ik, iv):
        """One estimator (x [N,H], y [N], column K/V [H+4,8,128,16] x 3, ICL K/V
        [8,N,64] x 12 of a built context): the ICL keys and values [8,nr,64] of the
        listed training rows at every block, each block's computed from the given
        context's earlier blocks (teacher forcing)."""
        n, h = x.shape
        idx = np.ascontiguousarray(rows, dtype=np.uintp)
        keys = [np.zeros((8, len(idx), 64), np.float32) for _ in range(12)]
        values = [np.zeros_like(keys[0]) for _ in range(12)]
        err = ctypes.create_string_buffer(512)
        # Contiguous float32 views kept alive for the call.
        x, y = f32(x), f32(y)
        ck, cv, ik, iv = ([f32(a) for a in t] for t in (ck, cv, ik, iv))
        st = lib().ora_context_rows(self._handle, n, h, fp(x), fp(y),
                                    idx.ctypes.data_as(ctypes.POINTER(ctypes.c_size_t)), len(idx),
                                    ptr_array(ck), ptr_array(cv), ptr_array(ik), ptr_array(iv),
                                    ptr_array(keys), ptr_array(values), err, 512)
        if st:
            raise ValueError(err.value.decode())
        return keys, values

    def trace_uncached(self, x_all, y, n):
        b, t, h = x_all.shape
        cols = np.zeros((b, t, h + 4, 128), np.float32)
        rows = np.zeros((b, t, 512), np.float32)
        err = ctypes.create_string_buffer(512)
        st = lib().ora_trace_uncached(self._handle, b, t, n, h, fp(f32(x_all)), fp(f32(y)), fp(cols),
                                      fp(rows), err, 512)
        if st:
            raise ValueError(err.value.decode())
        return cols, rows


def affine(x, w, b=None):
    x, w = f32(x), f32(w)
    rows, k = x.shape
    out = np.zeros((rows, w.shape[0]), np.float32)
    lib().ora_affine(fp(x), rows, k, fp(w), fp(f32(b)) if b is not None else None, w.shape[0], fp(out))
    return out


def layer_norm(x, w, b=None):
    x = f32(x)
    out = np.zeros_like(x)
    lib().ora_layer_norm(fp(x), x.shape[0], x.shape[1], fp(f32(w)), fp(f32(b)) if b is not None else None,
                         fp(out))
    return out


def gelu(x, math=EXACT):
    x = f32(x)
    out = np.zeros_like(x)
    lib().ora_gelu(math, fp(x), x.size, fp(out))
    return out


def rope(x, freqs, offset=0):
    x = f32(x)
    heads, rows, hd = x.shape
    out = np.zeros_like(x)
    lib().ora_rope(fp(x), heads, rows, hd, fp(f32(freqs)), offset, fp(out))
    return out


def attention(q, k, v, math=EXACT):
    q, k, v = f32(q), f32(k), f32(v)
    heads, qr, hd = q.shape
    out = np.zeros_like(q)
    st = lib().ora_attention(math, fp(q), qr, fp(k), fp(v), k.shape[1], heads, hd, fp(out))
    if st:
        raise ValueError("softmax normalization is not finite")
    return out


def attention_materialized(q, k, v):
    q, k, v = f32(q), f32(k), f32(v)
    heads, qr, hd = q.shape
    out = np.zeros_like(q)
    lib().ora_attention_materialized(fp(q), qr, fp(k), fp(v), k.shape[1], heads, hd, fp(out))
    return out


def aggregate(logits, perms, temperature=0.9, average_logits=True):
    logits = f32(logits)
    b, q, c = logits.shape
    perms = np.ascontiguousarray(perms, dtype=np.uint64)
    out = np.zeros((q, c), np.float32)
    st = lib().ora_aggregate(fp(logits), b, q, c, perms.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64)),
                             temperature, int(average_logits), fp(out))
    if st:
        raise ValueError("invalid aggregation")
    return out


def regression_outputs(logits, alphas):
    """(mean [Q], variance [Q], icdf at alphas [Q, A], sorted quantiles [Q, K]),
    each averaged over the B estimators of logits [B, Q, K]."""
    logits = f32(logits)
    b, q, k = logits.shape
    alphas = f32(alphas)
    mean, var = np.zeros(q, np.float32), np.zeros(q, np.float32)
    quant = np.zeros((q, len(alphas)), np.float32)
    raw = np.zeros((q, k), np.float32)
    st = lib().ora_regression_outputs(fp(logits), b, q, k, fp(alphas), len(alphas), fp(mean), fp(var), fp(quant),
                                      fp(raw))
    if st:
        raise ValueError("regression needs at least two quantiles")
    return mean, var, quant, raw


def regression_summary(logits, alphas):
    logits = f32(logits)
    b, q, k = logits.shape
    alphas = f32(alphas)
    mean = np.zeros(q, np.float32)
    quant = np.zeros((q, len(alphas)), np.float32)
    st = lib().ora_regression_summary(fp(logits), b, q, k, fp(alphas), len(alphas), fp(mean), fp(quant))
    if st:
        raise ValueError("regression needs at least two quantiles")
    return mean, quant
