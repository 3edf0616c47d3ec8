"""Writes known_answers.json: the reference's own known-answer vectors for the
hot path's primitive kernels, as data (inputs and expected outputs), each
with the reference test it comes from. Run: python tests/golden/make_known_answers.py
"""

import json
import math
import os

HERE = os.path.dirname(os.path.abspath(__file__))

cases = {
    # affine_matches_pytorch_output_by_input_weight_layout (src/kernels/reference.rs:1643-1651)
    "affine": {"input": [1.0, 2.0, -1.0, 3.0], "rows": 2, "in_dim": 2,
               "weight": [2.0, -1.0, 0.5, 1.0, 3.0, -2.0], "bias": [0.5, -1.0, 2.0], "out_dim": 3,
               "expected": [0.5, 1.5, 1.0, -4.5, 1.5, -7.0], "tolerance": 1e-5},
    # transposed_input3_affine_matches_standard_layout (reference.rs:1653-1671): inputs only,
    # the expectation is the standard affine of the same data.
    "affine_input3": {"input": [1.0, 2.0, -1.0, 3.0, -2.0, 0.5],
                      "weight": [2.0, -1.0, 0.5, 1.0, 3.0, -2.0, -0.5, 0.25, 4.0, 2.5, -3.0, 1.5],
                      "bias": [0.5, -1.0, 2.0, -0.25]},
    # one_hot_linear_selects_weight_columns_and_adds_bias (reference.rs:1682-1694)
    "one_hot_linear": {"classes": [2, 0], "weight": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0], "bias": [10.0, 20.0],
                       "class_count": 3, "out_dim": 2, "expected": [13.0, 26.0, 11.0, 24.0]},
    # layer_norm_uses_epsilon_and_optional_bias (reference.rs:1696-1705)
    "layer_norm": {"input": [1.0, 3.0], "weight": [2.0, 3.0], "bias": [1.0, -1.0],
                   "expected": [1.0 - 2.0 / math.sqrt(1.0 + 1e-5), -1.0 + 3.0 / math.sqrt(1.0 + 1e-5)],
                   "constant_input": [4.0, 4.0], "constant_expected": [0.0, 0.0], "tolerance": 1e-5},
    # gelu_tracks_erf_form (reference.rs:1707-1712)
    "gelu": {"input": [-1.0, 0.0, 1.0], "expected": [-0.15865526, 0.0, 0.8413447], "tolerance": 1e-5},
    # packed_qkv_splits_pytorch_packed_projection (reference.rs:1722-1746)
    "packed_qkv": {"input": [2.0, 3.0], "weight": [1.0, 0.0, 0.0, 1.0, 1.0, 1.0, 2.0, 0.0, 0.0, 2.0, 1.0, -1.0],
                   "bias": [0.0, 1.0, 2.0, 3.0, 4.0, 5.0], "query": [2.0, 4.0], "key": [7.0, 7.0],
                   "value": [10.0, 4.0]},
    # head_layout_round_trip_preserves_tokens (reference.rs:1748-1758)
    "head_layout": {"tokens": [1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0, 8.0], "rows": 2, "dim": 4, "heads": 2,
                    "heads_layout": [1.0, 2.0, 5.0, 6.0, 3.0, 4.0, 7.0, 8.0]},
    # qassmax_applies_base_scale_and_query_modulation (reference.rs:1760-1807)
    "qassmax": {"queries": [1.0, 2.0], "heads": 1, "rows": 1, "head_dim": 2, "hidden": 1,
                "base_first_weight": [1.0], "base_first_bias": [0.0], "base_second_weight": [2.0, 3.0],
                "base_second_bias": [0.0, 0.0], "query_first_weight": [1.0, 0.0], "query_first_bias": [0.0],
                "query_second_weight": [1.0, 0.0], "query_second_bias": [0.0, 0.0],
                "expected_at_one_source": [0.0, 0.0], "two_sources": "0 < out[0] < out[1]"},
    # non_interleaved_rope_rotates_contiguous_halves (reference.rs:1809-1824)
    "rope": {"input": [1.0, 2.0, 3.0, 4.0], "heads": 1, "rows": 1, "head_dim": 4,
             "frequencies": [math.pi / 2, 0.0], "position_offset": 1, "expected": [-3.0, 2.0, 1.0, 4.0],
             "tolerance": 1e-5},
    # attention_materializes_stable_scaled_dot_product (reference.rs:1826-1848)
    "attention_closed_form": {"query": [1.0, 0.0], "key": [1.0, 0.0, 0.0, 1.0], "value": [10.0, 20.0, 30.0, 40.0],
                              "source_rows": 2, "head_dim": 2,
                              "weight": math.exp(1 / math.sqrt(2)) / (math.exp(1 / math.sqrt(2)) + 1.0),
                              "tolerance": 1e-5},
    # tiled_online_attention_matches_materialized_across_tiles_and_scores (reference.rs:1850-1985):
    # (heads, query_rows, source_rows, head_dim, query_block_rows, key_tile_rows), LCG data.
    "online_attention_cases": [[1, 1, 1, 1, 1, 1], [2, 3, 5, 2, 3, 3], [3, 9, 17, 4, 7, 7],
                               [2, 10, 129, 8, 8, 128]],
    # tiled_online_attention_matches_uniform_and_peaked_scores (reference.rs:2061-2106)
    "uniform_peaked": [{"query": [0.0, 0.0], "key": [0.0, 0.0, 0.0, 0.0]},
                       {"query": [100.0, 0.0], "key": [1.0, 0.0, 0.0, 0.0]}],
    # probabilities_reverse_class_permutations_and_follow_aggregation_options (cpu.rs:5421-5473)
    "aggregation": {"logits": [1.0, 2.0, 3.0, 4.0, 8.0, 6.0], "shape": [2, 1, 3], "permutations": [2, 0, 1, 1, 2, 0],
                    "members": [[3.0, 1.0, 2.0], [8.0, 6.0, 4.0]],
                    "options": [[0.9, True], [0.5, True], [0.9, False], [2.0, False]],
                    "invalid_temperatures": [0.0, -1.0, "nan", "inf"], "tolerance": 1e-6},
    # quantiles.rs:224-275
    "quantile_levels": {"k": 999, "first": 0.001, "middle_index": 499, "middle": 0.5, "last": 0.999,
                        "tolerance": 1e-7},
    "linear_quantiles": {"k": 999, "formula": "10*alpha - 5 at each level, reversed", "mean": 0.0, "median": 0.0,
                         "alphas": [0.25, 0.75], "quantiles": [-2.5, 2.5], "tolerance": 1e-5},
    "exponential_tail": {"k": 999, "formula": "ln(alpha) at each level, two equal estimators", "alpha": 0.0001,
                         "expected": math.log(0.0001), "tolerance": 1e-3},
    # src/kernels/cpu/tests.rs:606-649: native approximations against libm.
    "native_bounds": {"exp_relative": 5e-6, "exp_domain": [-80.0, 0.0, 0.001], "erf_abs": 6e-7, "gelu_abs": 1e-6,
                      "gelu_domain": [-10.0, 10.0, 0.001]},
}

if __name__ == "__main__":
    with open(os.path.join(HERE, "known_answers.json"), "w") as f:
        json.dump(cases, f, indent=1)
        f.write("\n")
