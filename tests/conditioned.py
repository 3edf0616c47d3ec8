"""Conditioned weights: the random-init model with sharpened attention (test
infrastructure only).

At the configurations' random-init weights every softmax is nearly uniform
(median effective source count above 0.9 of the sources, largest probability
0.002 in the ICL blocks at 1,024 training rows), so logit parity there says
little about the score path. ``conditioned_weights`` scales the query and key
rows of every attention's in_proj (weights and biases) by a factor per family,
which scales its scores by the factor squared, to bring the median effective
source count (1 / sum p^2) to a tenth to a fifth of the sources without
saturating. ``attention_stats`` measures that on a float64 forward.
"""

from __future__ import annotations

import math

import numpy as np

# Query/key scale per attention family: the inducing points' attention over
# the training rows (attn1), the rows' attention to the inducing points
# (attn2), the row transformer, the ICL blocks.
SCALES = {"attn1": 2.5, "attn2": 2.3, "row": 2.4, "icl": 4.5}


def family(name: str) -> str:
    if "multihead_attn1" in name:
        return "attn1"
    if "multihead_attn2" in name:
        return "attn2"
    return "row" if name.startswith("row_interactor") else "icl"


def conditioned_weights(weights: dict, scales: dict = SCALES) -> dict:
    w = {k: np.array(v, np.float32, copy=True) for k, v in weights.items()}
    for name, value in w.items():
        if name.endswith("attn.in_proj_weight") or name.endswith("attn.in_proj_bias"):
            d = value.shape[0] // 3
            value[: 2 * d] *= np.float32(scales[family(name)])
    return w


def attention_stats(task: str, weights: dict, x_train, y, x_test) -> dict:
    """{family: (median of the per-query median effective source fraction,
    largest probability)} over one float64 uncached forward (the restatement
    in reference_np.py, with its attention instrumented)."""
    import reference_np as R

    seen: dict[str, list] = {}
    attend = R.Model.attend

    def recording(self, prefix, q, Kh, Vh, qass_source=None, rope=False):
        t = self.t
        d = q.shape[-1]
        hd = d // 8
        wq, bq = t(f"{prefix}.attn.in_proj_weight")[:d], t(f"{prefix}.attn.in_proj_bias")[:d]
        qn = R.layer_norm(q, t(f"{prefix}.norm1.weight"), t(f"{prefix}.norm1.bias"))
        Qh = np.swapaxes((qn @ wq.T + bq).reshape(*q.shape[:-1], 8, hd), -2, -3)
        if qass_source is not None:
            s = lambda part: t(f"{prefix}.attn.ssmax_layer.{part}")
            hidden = R.gelu(s("base_mlp.0.weight")[:, 0] * math.log(max(qass_source, 1)) + s("base_mlp.0.bias"))
            base = (s("base_mlp.2.weight") @ hidden + s("base_mlp.2.bias")).reshape(8, 1, hd)
            g = R.gelu(Qh @ s("query_mlp.0.weight").T + s("query_mlp.0.bias")) @ s("query_mlp.2.weight").T
            Qh = Qh * base * (1.0 + np.tanh(g + s("query_mlp.2.bias")))
        if rope:
            Qh = self.rope(Qh, np.arange(Qh.shape[-2], dtype=np.float64))
        scores = Qh @ np.swapaxes(Kh, -1, -2) / math.sqrt(hd)
        p = np.exp(scores - scores.max(-1, keepdims=True))
        p /= p.sum(-1, keepdims=True)
        neff = 1.0 / (p ** 2).sum(-1) / p.shape[-1]
        seen.setdefault(family(prefix), []).append((float(np.median(neff)), float(p.max())))
        return attend(self, prefix, q, Kh, Vh, qass_source, rope)

    R.Model.attend = recording
    try:
        n = x_train.shape[0]
        x = np.concatenate([x_train, x_test]).astype(np.float64)
        R.Model(task, weights).forward(x, np.asarray(y, np.float64), n)
    finally:
        R.Model.attend = attend
    return {k: (float(np.median([a for a, _ in v])), float(max(b for _, b in v))) for k, v in seen.items()}
