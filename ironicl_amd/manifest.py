"""The official TabICLv2 tensor manifest and architecture constants.

Restates ``tensor_manifest`` / ``insert_attention_manifest``
(src/format/model.rs:772-867) and the constants of
src/models/tabicl_v2/cpu.rs:40-54. The regressor encodes a scalar target,
decodes 999 quantiles and has no LayerNorm biases; its loader fills those with
zeros (src/format/model.rs:273-280).
"""

from __future__ import annotations

CLASSIFIER = "classifier"
REGRESSOR = "regressor"

COLUMN_DIM = 128
ICL_DIM = 512
HEADS = 8
INDUCING = 128
COLUMN_BLOCKS = 3
ROW_BLOCKS = 3
ICL_BLOCKS = 12
RESERVED = 4
FFN_HIDDEN = 1024
MAX_CLASSES = 10
NUM_QUANTILES = 999

# Source-checkpoint SHA-256 of the two official models (src/format/model.rs:31-38).
CLASSIFIER_SHA256 = bytes.fromhex(
    "bdc7dbd5e4ff21f8f0456fcf90c6b7cdf72dbea960f2d05b19bec19f9b3d4ed0")
REGRESSOR_SHA256 = bytes.fromhex(
    "0db9cb538f114e79026bf08f45f41ad8dd7ad2de2aaca9a5ca8cd3bd9748ae7a")
# (tensor count, parameter count, tensor bytes) per profile (model.rs:869-885).
PROFILE = {
    CLASSIFIER: (391, 27_552_258, 110_209_032),
    REGRESSOR: (347, 28_544_991, 114_179_964),
}


def _is_ln_bias(name: str) -> bool:
    return name.endswith("norm1.bias") or name.endswith("norm2.bias") or name.endswith("ln.bias")


def _attention(out: dict, prefix: str, dim: int, ssmax: bool) -> None:
    attn = f"{prefix}.attn"
    out[f"{attn}.in_proj_bias"] = (3 * dim,)
    out[f"{attn}.in_proj_weight"] = (3 * dim, dim)
    out[f"{attn}.out_proj.bias"] = (dim,)
    out[f"{attn}.out_proj.weight"] = (dim, dim)
    if ssmax:
        qd = dim // 8
        for layer, dims in (("base_mlp.0", (64, 1)), ("base_mlp.2", (dim, 64)),
                            ("query_mlp.0", (64, qd)), ("query_mlp.2", (qd, 64))):
            out[f"{attn}.ssmax_layer.{layer}.bias"] = (dims[0],)
            out[f"{attn}.ssmax_layer.{layer}.weight"] = dims
    out[f"{prefix}.linear1.bias"] = (2 * dim,)
    out[f"{prefix}.linear1.weight"] = (2 * dim, dim)
    out[f"{prefix}.linear2.bias"] = (dim,)
    out[f"{prefix}.linear2.weight"] = (dim, 2 * dim)
    out[f"{prefix}.norm1.bias"] = (dim,)
    out[f"{prefix}.norm1.weight"] = (dim,)
    out[f"{prefix}.norm2.bias"] = (dim,)
    out[f"{prefix}.norm2.weight"] = (dim,)


def tensor_manifest(task: str) -> dict[str, tuple[int, ...]]:
    """Official tensor names and shapes, sorted by name (model.rs:772-836)."""
    targets, outputs = (10, 10) if task == CLASSIFIER else (1, 999)
    t: dict[str, tuple[int, ...]] = {}
    t["col_embedder.in_linear.bias"] = (128,)
    t["col_embedder.in_linear.weight"] = (128, 3)
    t["col_embedder.y_encoder.bias"] = (128,)
    t["col_embedder.y_encoder.weight"] = (128, targets)
    for b in range(COLUMN_BLOCKS):
        p = f"col_embedder.tf_col.blocks.{b}"
        t[f"{p}.ind_vectors"] = (128, 128)
        _attention(t, f"{p}.multihead_attn1", 128, True)
        _attention(t, f"{p}.multihead_attn2", 128, False)
    t["icl_predictor.decoder.0.bias"] = (1024,)
    t["icl_predictor.decoder.0.weight"] = (1024, 512)
    t["icl_predictor.decoder.2.bias"] = (outputs,)
    t["icl_predictor.decoder.2.weight"] = (outputs, 1024)
    t["icl_predictor.ln.bias"] = (512,)
    t["icl_predictor.ln.weight"] = (512,)
    t["icl_predictor.y_encoder.bias"] = (512,)
    t["icl_predictor.y_encoder.weight"] = (512, targets)
    for b in range(ICL_BLOCKS):
        _attention(t, f"icl_predictor.tf_icl.blocks.{b}", 512, True)
    t["row_interactor.cls_tokens"] = (4, 128)
    t["row_interactor.out_ln.bias"] = (128,)
    t["row_interactor.out_ln.weight"] = (128,)
    t["row_interactor.tf_row.rope.freqs"] = (8,)
    for b in range(ROW_BLOCKS):
        _attention(t, f"row_interactor.tf_row.blocks.{b}", 128, False)
    if task == REGRESSOR:
        t = {k: v for k, v in t.items() if not _is_ln_bias(k)}
    return dict(sorted(t.items()))


def decoder_width(task: str) -> int:
    return MAX_CLASSES if task == CLASSIFIER else NUM_QUANTILES
