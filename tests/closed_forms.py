"""Closed forms of the TabICLv2 forward at degenerate weights (test
infrastructure only).

Each weight family makes every attention's queries independent of the query
row, so its softmax is a formula of the sources alone, and the whole forward
reduces to a few float64 NumPy lines per stage, written here from the model's
definition (docs/model.md:14-47; the stage order of cpu.rs:1132-1333):

  - ``uniform_weights``: every attention's query projection (in_proj rows
    0..d, weights and biases) is zero. Every score is 0, every softmax is
    uniform, and each attention returns the mean of its sources' values. The
    logits then depend on which rows are each attention's sources (the N
    training rows for attn1 and the ICL blocks, the 128 inducing points for
    attn2, the H + 4 tokens of a row), where the labels are added (training
    rows only), which tokens are the CLS tokens that block 2 reads, and the
    residual / feed-forward / decoder chain.
  - ``constant_query_weights``: the query projection's weights are zero and its
    biases are not, so every query is its bias b_q, through QASSMax where the
    block has it. Scores are b_q . k_j / sqrt(head_dim): a softmax over the
    sources' keys, the same for every query row, except in the row
    transformer, where RoPE rotates the query by its position i and the key by
    its position j. This fixes the attention scales (1/4, 1/8), RoPE's
    positions, pairing and signs, the order of the tokens, and QASSMax's gate
    and base scale; the base MLP's first layer is made steep in ln(N) so that
    a base computed for N + 1 sources instead of N moves the logits far past
    the parity bar.

``forward`` computes the closed-form logits of one estimator for either family.
``ClosedForm(..., mutation=...)`` plants one plausible mistake in the closed
form (``MUTATIONS``), so a test can show that each moves the logits far past
the parity bar, i.e. that the checks would catch it. Nothing here calls the
oracle or the backend.
"""

from __future__ import annotations

import math

import numpy as np
from scipy.special import erf

HEADS = 8

COLUMN_ATTN = [f"col_embedder.tf_col.blocks.{b}.multihead_attn{i}" for b in range(3) for i in (1, 2)]
ROW_BLOCKS = [f"row_interactor.tf_row.blocks.{b}" for b in range(3)]
ICL_BLOCKS = [f"icl_predictor.tf_icl.blocks.{b}" for b in range(12)]
QASS_BLOCKS = [f"col_embedder.tf_col.blocks.{b}.multihead_attn1" for b in range(3)] + ICL_BLOCKS


def _dim(prefix: str) -> int:
    return 512 if prefix.startswith("icl_predictor") else 128


def uniform_weights(weights: dict) -> dict:
    """Every attention's query rows of in_proj (weight and bias) set to zero."""
    w = {k: np.array(v, np.float32, copy=True) for k, v in weights.items()}
    for p in COLUMN_ATTN + ROW_BLOCKS + ICL_BLOCKS:
        d = _dim(p)
        w[f"{p}.attn.in_proj_weight"][:d] = 0.0
        w[f"{p}.attn.in_proj_bias"][:d] = 0.0
    return w


def constant_query_weights(weights: dict, train_rows: int, seed: int = 7) -> dict:
    """Query weights zero and query biases drawn so the softmaxes are neither
    flat nor saturated; each QASSMax base MLP's first layer steep in
    ln(train_rows): w1 = 40, b1 = -40 ln(train_rows) + U(-1, 1), so that ln(N)
    and ln(N + 1) differ by 40 / N in its input.

    At random-init weights the rows' ICL representations differ little, so the
    ICL keys' weights are scaled by 16 too. On the tests' 96-row case the
    median effective source count (1 / sum p^2 over the sources) is then about
    half the sources in the inducing points' attention and the ICL blocks and
    0.8-0.85 of them in attn2 and the row blocks, with the largest probability
    0.24-0.45 (not saturated)."""
    rng = np.random.default_rng(seed)
    w = {k: np.array(v, np.float32, copy=True) for k, v in weights.items()}
    for p in COLUMN_ATTN + ROW_BLOCKS + ICL_BLOCKS:
        d = _dim(p)
        hd = d // HEADS
        scale = 24.0 if p.endswith("attn1") else 8.0 if d == 512 else 2.0
        w[f"{p}.attn.in_proj_weight"][:d] = 0.0
        w[f"{p}.attn.in_proj_bias"][:d] = rng.normal(0.0, scale * hd ** 0.25 / math.sqrt(hd), d).astype(np.float32)
        if d == 512:
            w[f"{p}.attn.in_proj_weight"][d:2 * d] *= 16.0
    log_n = math.log(train_rows)
    for p in QASS_BLOCKS:
        s = f"{p}.attn.ssmax_layer"
        w[f"{s}.base_mlp.0.weight"][:] = 40.0
        w[f"{s}.base_mlp.0.bias"][:] = (-40.0 * log_n + rng.uniform(-1.0, 1.0, 64)).astype(np.float32)
    return w


def gelu(x):
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def layer_norm(x, w, b):
    m = x.mean(-1, keepdims=True)
    v = ((x - m) ** 2).mean(-1, keepdims=True)
    return (x - m) / np.sqrt(v + 1e-5) * w + (0.0 if b is None else b)


# Plausible mistakes, each planted in the closed form by ClosedForm(mutation=...).
MUTATIONS = {
    "icl_sources_all_rows": "ICL blocks attend to every row, test rows included",
    "attn1_sources_all_rows": "the inducing points attend to every row, test rows included",
    "labels_on_all_rows": "label embeddings added to the test rows too",
    "grouping_f123": "feature f reads (f+1, f+2, f+3) mod H",
    "cls_last": "the CLS tokens after the feature tokens",
    "qass_sources_plus_one": "QASSMax base scale for N + 1 sources",
    "rope_sin_sign": "RoPE rotating the other way",
    "rope_query_off_by_one": "RoPE queries at positions 1..L, keys at 0..L-1",
    "row_scale_eighth": "row attention scaled by 1/8",
    "icl_scale_quarter": "ICL attention scaled by 1/4 instead of 1/8",
}


class ClosedForm:
    """The forward of one estimator at ``uniform_weights`` or
    ``constant_query_weights`` (which one is read from the weights)."""

    def __init__(self, task: str, weights: dict, mutation: str | None = None):
        assert mutation is None or mutation in MUTATIONS, mutation
        self.task = task
        self.mutation = mutation
        self.w = {k: np.asarray(v, np.float64) for k, v in weights.items()}
        self.uniform = not np.any(self.w[f"{ICL_BLOCKS[0]}.attn.in_proj_bias"][:512])

    def t(self, name):
        return self.w.get(name)

    def rotate(self, x, position):
        """x [..., 8 heads, 16]: dims d and d + 8 of each head turned by
        position * freq[d] (x[d] cos - x[d+8] sin, x[d+8] cos + x[d] sin)."""
        angle = position * self.t("row_interactor.tf_row.rope.freqs")
        c, s = np.cos(angle), np.sin(angle)
        if self.mutation == "rope_sin_sign":
            s = -s
        lo, hi = x[..., :8], x[..., 8:]
        return np.concatenate([lo * c - hi * s, hi * c + lo * s], axis=-1)

    def query(self, prefix, sources):
        """The constant query of a block, heads [8, hd], through QASSMax for
        `sources` keys where the block has it."""
        d = _dim(prefix)
        hd = d // HEADS
        q = self.t(f"{prefix}.attn.in_proj_bias")[:d].reshape(HEADS, hd)
        if prefix in QASS_BLOCKS:
            if self.mutation == "qass_sources_plus_one":
                sources += 1
            s = lambda part: self.t(f"{prefix}.attn.ssmax_layer.{part}")
            base = s("base_mlp.2.weight") @ gelu(s("base_mlp.0.weight")[:, 0] * math.log(sources) +
                                                 s("base_mlp.0.bias")) + s("base_mlp.2.bias")
            gate = gelu(q @ s("query_mlp.0.weight").T + s("query_mlp.0.bias")) @ s("query_mlp.2.weight").T
            q = q * base.reshape(HEADS, hd) * (1.0 + np.tanh(gate + s("query_mlp.2.bias")))
        return q

    def attention(self, prefix, sources, q_rows, rope=False):
        """[q_rows, d]: each query row's attention over the source rows."""
        d = _dim(prefix)
        hd = d // HEADS
        w, b = self.t(f"{prefix}.attn.in_proj_weight"), self.t(f"{prefix}.attn.in_proj_bias")
        normed = layer_norm(sources, self.t(f"{prefix}.norm1.weight"), self.t(f"{prefix}.norm1.bias"))
        v = (normed @ w[2 * d:].T + b[2 * d:]).reshape(-1, HEADS, hd)           # [S, 8, hd]
        if self.uniform:
            return np.broadcast_to(v.mean(0).reshape(d), (q_rows, d))
        k = (normed @ w[d:2 * d].T + b[d:2 * d]).reshape(-1, HEADS, hd)          # [S, 8, hd]
        q = self.query(prefix, sources.shape[0])                                 # [8, hd]
        if rope:
            k = np.stack([self.rotate(k[j], j) for j in range(k.shape[0])])
            shift = 1 if self.mutation == "rope_query_off_by_one" else 0
            qs = np.stack([self.rotate(q, i + shift) for i in range(q_rows)])    # [q_rows, 8, hd]
        else:
            qs = np.broadcast_to(q, (q_rows, HEADS, hd))
        scale = 1.0 / math.sqrt(hd)
        if (self.mutation == "row_scale_eighth" and rope) or (self.mutation == "icl_scale_quarter" and d == 512):
            scale = 0.125 if rope else 0.25
        scores = np.einsum("qhd,shd->hqs", qs, k) * scale
        p = np.exp(scores - scores.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        return np.einsum("hqs,shd->qhd", p, v).reshape(q_rows, d)

    def block(self, prefix, q, sources, rope=False):
        """Pre-norm block: q + out_proj(attention), then + FFN(LN2(.))."""
        t = self.t
        att = self.attention(prefix, sources, q.shape[0], rope)
        r = q + att @ t(f"{prefix}.attn.out_proj.weight").T + t(f"{prefix}.attn.out_proj.bias")
        h = gelu(layer_norm(r, t(f"{prefix}.norm2.weight"), t(f"{prefix}.norm2.bias")) @
                 t(f"{prefix}.linear1.weight").T + t(f"{prefix}.linear1.bias"))
        return r + h @ t(f"{prefix}.linear2.weight").T + t(f"{prefix}.linear2.bias")

    def label(self, prefix, y):
        w, b = self.t(f"{prefix}.y_encoder.weight"), self.t(f"{prefix}.y_encoder.bias")
        if self.task == "classifier":
            return w[:, y.astype(np.int64)].T + b
        return y[:, None] * w[:, 0] + b

    def forward(self, x_train, y, x_test):
        """Decoder outputs [Q, width] of x_test [Q, H] against x_train [N, H],
        labels y [N]."""
        t = self.t
        n, h = x_train.shape
        x = np.concatenate([x_train, x_test]).astype(np.float64)
        rows = x.shape[0]
        # Column stage: feature f reads features (f+1, f+2, f+4) mod H.
        m = self.mutation
        labelled = rows if m == "labels_on_all_rows" else n
        y_all = np.concatenate([y, y[: rows - n]]) if m == "labels_on_all_rows" else y
        columns = np.zeros((rows, h, 128))
        for f in range(h):
            g = x[:, [(f + 1) % h, (f + 2) % h, (f + (3 if m == "grouping_f123" else 4)) % h]]
            e = g @ t("col_embedder.in_linear.weight").T + t("col_embedder.in_linear.bias")
            e[:labelled] += self.label("col_embedder", y_all)
            for b in range(3):
                p = f"col_embedder.tf_col.blocks.{b}"
                src = e if m == "attn1_sources_all_rows" else e[:n]
                hidden = self.block(f"{p}.multihead_attn1", t(f"{p}.ind_vectors"), src)
                e = self.block(f"{p}.multihead_attn2", e, hidden)
            columns[:, f] = e
        # Row stage: [CLS0..3, column 0..H-1], two full blocks, then the CLS tokens.
        reps = np.zeros((rows, 512))
        for r in range(rows):
            if m == "cls_last":
                seq = np.concatenate([columns[r], t("row_interactor.cls_tokens")])
            else:
                seq = np.concatenate([t("row_interactor.cls_tokens"), columns[r]])
            for b in range(2):
                seq = self.block(ROW_BLOCKS[b], seq, seq, rope=True)
            cls = self.block(ROW_BLOCKS[2], seq[-4:] if m == "cls_last" else seq[:4], seq, rope=True)
            reps[r] = layer_norm(cls, t("row_interactor.out_ln.weight"), t("row_interactor.out_ln.bias")).reshape(512)
        # ICL: labels on the training rows, every row attends to the training rows.
        reps[:labelled] += self.label("icl_predictor", y_all)
        for p in ICL_BLOCKS:
            reps = self.block(p, reps, reps if m == "icl_sources_all_rows" else reps[:n])
        out = gelu(layer_norm(reps[n:], t("icl_predictor.ln.weight"), t("icl_predictor.ln.bias")) @
                   t("icl_predictor.decoder.0.weight").T + t("icl_predictor.decoder.0.bias"))
        return out @ t("icl_predictor.decoder.2.weight").T + t("icl_predictor.decoder.2.bias")
