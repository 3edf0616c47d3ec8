"""An independent float64 NumPy restatement of the TabICLv2 uncached forward
(src/models/tabicl_v2/cpu.rs:997-1333), vectorized over rows and heads. It
cross-checks the C oracle on tiny shapes; test infrastructure only."""

from __future__ import annotations

import math

import numpy as np
from scipy.special import erf


def gelu(x):
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def layer_norm(x, w, b):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    y = (x - m) / np.sqrt(v + 1e-5) * w
    return y + b if b is not None else y


class Model:
    def __init__(self, task: str, weights: dict[str, np.ndarray]):
        self.task = task
        self.w = {k: np.asarray(v, dtype=np.float64) for k, v in weights.items()}

    def t(self, name):
        return self.w.get(name)

    def rope(self, x, positions):
        """x [..., heads, rows, hd]; non-interleaved halves (reference.rs:433-475)."""
        f = self.t("row_interactor.tf_row.rope.freqs")
        hd = x.shape[-1]
        half = hd // 2
        ang = positions[:, None] * f[None, :half]
        c, s = np.cos(ang), np.sin(ang)
        left, right = x[..., :half], x[..., half:]
        return np.concatenate([left * c - right * s, right * c + left * s], axis=-1)

    def source(self, prefix, kv, rope=False):
        """LN1 and the K/V projections of the source rows, head-major
        [..., 8, src, hd] each (source_heads, cpu.rs:1356-1416)."""
        t = self.t
        d = kv.shape[-1]
        hd = d // 8
        w, b = t(f"{prefix}.attn.in_proj_weight"), t(f"{prefix}.attn.in_proj_bias")
        kn = layer_norm(kv, t(f"{prefix}.norm1.weight"), t(f"{prefix}.norm1.bias"))
        heads = lambda a: np.swapaxes(a.reshape(*a.shape[:-1], 8, hd), -2, -3)
        Kh, Vh = heads(kn @ w[d:2 * d].T + b[d:2 * d]), heads(kn @ w[2 * d:].T + b[2 * d:])
        if rope:
            Kh = self.rope(Kh, np.arange(Kh.shape[-2], dtype=np.float64))
        return Kh, Vh

    def attend(self, prefix, q, Kh, Vh, qass_source=None, rope=False):
        """Pre-norm MAB of queries q [..., rows, d] against head-major keys and
        values (attend / cached_block, cpu.rs:1475-1602, 2587-2850)."""
        t = self.t
        d = q.shape[-1]
        hd = d // 8
        w, b = t(f"{prefix}.attn.in_proj_weight"), t(f"{prefix}.attn.in_proj_bias")
        qn = layer_norm(q, t(f"{prefix}.norm1.weight"), t(f"{prefix}.norm1.bias"))
        Qh = np.swapaxes((qn @ w[:d].T + b[:d]).reshape(*q.shape[:-1], 8, hd), -2, -3)
        if qass_source is not None:
            s = lambda part: t(f"{prefix}.attn.ssmax_layer.{part}")
            hidden = gelu(s("base_mlp.0.weight")[:, 0] * math.log(max(qass_source, 1)) + s("base_mlp.0.bias"))
            base = (s("base_mlp.2.weight") @ hidden + s("base_mlp.2.bias")).reshape(8, 1, hd)
            g = gelu(Qh @ s("query_mlp.0.weight").T + s("query_mlp.0.bias")) @ s("query_mlp.2.weight").T
            g = g + s("query_mlp.2.bias")
            Qh = Qh * base * (1.0 + np.tanh(g))
        if rope:
            Qh = self.rope(Qh, np.arange(Qh.shape[-2], dtype=np.float64))
        S = Qh @ np.swapaxes(Kh, -1, -2) / math.sqrt(hd)
        P = np.exp(S - S.max(-1, keepdims=True))
        P /= P.sum(-1, keepdims=True)
        O = np.swapaxes(P @ Vh, -2, -3)
        O = O.reshape(*O.shape[:-2], d)
        r = q + O @ t(f"{prefix}.attn.out_proj.weight").T + t(f"{prefix}.attn.out_proj.bias")
        f = layer_norm(r, t(f"{prefix}.norm2.weight"), t(f"{prefix}.norm2.bias"))
        f = gelu(f @ t(f"{prefix}.linear1.weight").T + t(f"{prefix}.linear1.bias"))
        return r + f @ t(f"{prefix}.linear2.weight").T + t(f"{prefix}.linear2.bias")

    def block(self, prefix, q, kv, qass_source=None, rope=False):
        """Pre-norm MAB: q [..., rows, d], kv [..., src, d] (attend, cpu.rs:1475-1602)."""
        return self.attend(prefix, q, *self.source(prefix, kv, rope), qass_source=qass_source, rope=rope)

    def column_input(self, x, f):
        """Grouped features (f+1, f+2, f+4) mod H through the 3 -> 128 input affine."""
        H = x.shape[-1]
        g = x[..., [(f + 1) % H, (f + 2) % H, (f + 4) % H]].astype(np.float64)
        e = g @ self.t("col_embedder.in_linear.weight").T + self.t("col_embedder.in_linear.bias")
        e[np.all(g == -100.0, axis=-1)] = -100.0
        return e

    def column_kv(self, x, y, f):
        """Training rows x [N, H], y [N]: feature f's multihead_attn2 keys and
        values [8, 128, 16] per column block, from its whole column stream."""
        n = x.shape[0]
        e = self.column_input(x, f) + self.target("col_embedder", y)
        out = []
        for blk in range(3):
            p = f"col_embedder.tf_col.blocks.{blk}"
            hidden = self.block(f"{p}.multihead_attn1", self.t(f"{p}.ind_vectors"), e, qass_source=n)
            Kh, Vh = self.source(f"{p}.multihead_attn2", hidden)
            out.append((Kh, Vh))
            e = self.attend(f"{p}.multihead_attn2", e, Kh, Vh)
        return out

    def row_kv(self, xr, yr, ck, cv, ik, iv):
        """One training row (xr [H], label yr) against a built context (column
        K/V [3][H+4,8,128,16], ICL K/V [12][8,N,64]): its ICL keys and values
        [8, 64] at every block, each block's from the context's earlier blocks."""
        t = self.t
        H, n = xr.shape[0], ik[0].shape[1]
        y = np.array([yr], dtype=np.float64)
        ycol = self.target("col_embedder", y)
        seq = np.zeros((H + 4, 128))
        seq[:4] = t("row_interactor.cls_tokens")
        for f in range(H):
            e = self.column_input(xr[None], f) + ycol
            for blk in range(3):
                p = f"col_embedder.tf_col.blocks.{blk}.multihead_attn2"
                e = self.attend(p, e, np.asarray(ck[blk][4 + f], np.float64), np.asarray(cv[blk][4 + f], np.float64))
            seq[4 + f] = e[0]
        for blk in range(2):
            seq = self.block(f"row_interactor.tf_row.blocks.{blk}", seq, seq, rope=True)
        final = self.block("row_interactor.tf_row.blocks.2", seq[:4], seq, rope=True)
        row = layer_norm(final, t("row_interactor.out_ln.weight"), t("row_interactor.out_ln.bias")).reshape(1, 512)
        row = row + self.target("icl_predictor", y)
        keys, values = [], []
        for blk in range(12):
            p = f"icl_predictor.tf_icl.blocks.{blk}"
            Kh, Vh = self.source(p, row)
            keys.append(Kh[:, 0])
            values.append(Vh[:, 0])
            if blk < 11:
                row = self.attend(p, row, np.asarray(ik[blk], np.float64), np.asarray(iv[blk], np.float64),
                                  qass_source=n)
        return keys, values

    def cached_logits(self, xq, ck, cv, ik, iv):
        """Test rows xq [Q, H] against a built context (column K/V
        [3][H+4,8,128,16], ICL K/V [12][8,N,64]), cached prediction in float64
        (StaticExecutor::predict_chunk, cpu.rs:2200-2273): decoder outputs [Q, width]."""
        t = self.t
        q, h = xq.shape
        n = ik[0].shape[1]
        seq = np.zeros((q, h + 4, 128))
        seq[:, :4] = t("row_interactor.cls_tokens")
        for f in range(h):
            e = self.column_input(xq, f)
            for blk in range(3):
                p = f"col_embedder.tf_col.blocks.{blk}.multihead_attn2"
                e = self.attend(p, e, np.asarray(ck[blk][4 + f], np.float64), np.asarray(cv[blk][4 + f], np.float64))
            seq[:, 4 + f] = e
        for blk in range(2):
            seq = self.block(f"row_interactor.tf_row.blocks.{blk}", seq, seq, rope=True)
        final = self.block("row_interactor.tf_row.blocks.2", seq[:, :4], seq, rope=True)
        rows = layer_norm(final, t("row_interactor.out_ln.weight"), t("row_interactor.out_ln.bias")).reshape(q, 512)
        for blk in range(12):
            rows = self.attend(f"icl_predictor.tf_icl.blocks.{blk}", rows, np.asarray(ik[blk], np.float64),
                               np.asarray(iv[blk], np.float64), qass_source=n)
        hid = gelu(layer_norm(rows, t("icl_predictor.ln.weight"), t("icl_predictor.ln.bias")) @
                   t("icl_predictor.decoder.0.weight").T + t("icl_predictor.decoder.0.bias"))
        return hid @ t("icl_predictor.decoder.2.weight").T + t("icl_predictor.decoder.2.bias")

    def target(self, prefix, y):
        w, b = self.t(f"{prefix}.y_encoder.weight"), self.t(f"{prefix}.y_encoder.bias")
        if self.task == "classifier":
            return w[:, y.astype(np.int64)].T + b
        return y[:, None] * w[:, 0] + b

    def forward(self, x, y, n):
        """x [T, H] (training rows first), y [N]; returns (columns [T,H+4,128],
        rows [T,512], logits [T,width])."""
        t = self.t
        T, H = x.shape
        cls = t("row_interactor.cls_tokens")
        cols = np.zeros((T, H + 4, 128))
        ycol = self.target("col_embedder", y)
        for f in range(H):
            g = x[:, [(f + 1) % H, (f + 2) % H, (f + 4) % H]]
            e = g @ t("col_embedder.in_linear.weight").T + t("col_embedder.in_linear.bias")
            e[np.all(g == -100.0, axis=1)] = -100.0
            e[:n] += ycol
            for blk in range(3):
                if np.all(e == -100.0):
                    continue
                p = f"col_embedder.tf_col.blocks.{blk}"
                hidden = self.block(f"{p}.multihead_attn1", t(f"{p}.ind_vectors"), e[:n], qass_source=n)
                e = self.block(f"{p}.multihead_attn2", e, hidden)
            cols[:, 4 + f] = e
        seq = cols.copy()
        seq[:, :4] = cls
        for blk in range(2):
            p = f"row_interactor.tf_row.blocks.{blk}"
            seq = self.block(p, seq, seq, rope=True)
        final = self.block("row_interactor.tf_row.blocks.2", seq[:, :4], seq, rope=True)
        rows = layer_norm(final, t("row_interactor.out_ln.weight"), t("row_interactor.out_ln.bias")).reshape(T, 512)
        cols[:, :4] = 0.0
        reps = rows.copy()
        rows[:n] += self.target("icl_predictor", y)
        for blk in range(12):
            rows = self.block(f"icl_predictor.tf_icl.blocks.{blk}", rows, rows[:n], qass_source=n)
        h = layer_norm(rows, t("icl_predictor.ln.weight"), t("icl_predictor.ln.bias"))
        h = gelu(h @ t("icl_predictor.decoder.0.weight").T + t("icl_predictor.decoder.0.bias"))
        logits = h @ t("icl_predictor.decoder.2.weight").T + t("icl_predictor.decoder.2.bias")
        return cols, reps, logits
