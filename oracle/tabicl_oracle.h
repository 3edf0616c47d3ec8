/*
 * CPU restatement of Ironicl's FP32 TabICLv2 forward pass (the oracle).
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker for the HIP backend
 * in ironicl_amd/, and the CPU baseline that bench.py times beside it. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it. The product path never links or calls it.
 *
 * It restates, in plain C, the reference's scalar FP32 CPU path:
 *   - src/kernels/reference.rs:83-475   (affine, one-hot linear, LayerNorm,
 *                                         GELU, QASSMax, RoPE)
 *   - src/kernels/reference.rs:563-1024 (tiled / source-major online attention)
 *   - src/models/tabicl_v2/cpu.rs:873-1333   (Executor: build and uncached forward)
 *   - src/models/tabicl_v2/cpu.rs:2111-2850  (StaticExecutor: cached prediction)
 *   - src/models/tabicl_v2/cpu.rs:3768-3932  (QASS base scale, static QASS,
 *                                              probability aggregation)
 *   - src/models/tabicl_v2/quantiles.rs:80-213 (regression summaries)
 *
 * Two math modes follow the reference's two builds:
 *   ORA_MATH_EXACT  - libm erff/expf/tanhf (the `exact-math` feature),
 *   ORA_MATH_NATIVE - the AVX-512 host default: Abramowitz-Stegun GELU with
 *                     bounded_exp (src/kernels/cpu/ops/pointwise.rs:49-96) and
 *                     the degree-7 softmax exp (src/kernels/cpu/arch/x86_64.rs:40-51).
 *
 * Thread partitioning follows the reference (features and rows on workers,
 * ICL self-attention serial per estimator in the build, head-parallel cached
 * attention in prediction): src/models/tabicl_v2/cpu.rs:1101,1212,2401-2435,
 * 3014-3048, 3064-3104, 4439-4525.
 */
#ifndef TABICL_ORACLE_H
#define TABICL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORA_MATH_EXACT = 0, ORA_MATH_NATIVE = 1 };
enum { ORA_CLASSIFIER = 0, ORA_REGRESSOR = 1 };

/* Returns 0 and sets *data and *len for a tensor by its official checkpoint name,
 * non-zero when the model has no such tensor. */
typedef int (*ora_lookup)(void *user, const char *name, const float **data, size_t *len);

typedef struct ora_model ora_model;

/* Copies every official tensor (src/format/model.rs:772-867). Returns NULL and
 * writes a message into err on a missing or wrong-sized tensor. The regressor's
 * bias-free LayerNorms get zero biases (src/format/model.rs:273-280). */
ora_model *ora_model_new(int task, ora_lookup lookup, void *user, int math, char *err, size_t errlen);
void ora_model_free(ora_model *model);
size_t ora_model_width(const ora_model *model);
void ora_set_threads(int threads);
int ora_get_threads(void);

/* Build: Executor::build_tensors_cpu (cpu.rs:873-960). x [B,N,H], y [B,N].
 * Outputs are caller-allocated: column_keys[3]/column_values[3] of
 * [B,H+4,8,128,16] (reserved streams written as zeros) and icl_keys[12] /
 * icl_values[12] of [B,8,N,64]. Returns 0 on success. */
int ora_build_context(const ora_model *model, size_t b, size_t n, size_t h, const float *x,
                      const float *y, float *const *column_keys, float *const *column_values,
                      float *const *icl_keys, float *const *icl_values, char *err, size_t errlen);

/* Spot checks of one estimator's built context at full size (x [N,H], y [N]).
 * ora_context_columns: the column K/V of the listed features, as
 * ora_build_context computes them; kv[2*block], kv[2*block+1] are [nf,8,128,16].
 * ora_context_rows: the ICL K/V of the listed training rows, each block's from
 * the given context's earlier blocks (teacher forcing); ck/cv [H+4,8,128,16],
 * ik/iv [8,N,64] of that estimator; keys/values out 12 x [8,nr,64]. */
int ora_context_columns(const ora_model *model, size_t n, size_t h, const float *x, const float *y,
                        const size_t *features, size_t nf, float *const *kv, char *err, size_t errlen);
int ora_context_rows(const ora_model *model, size_t n, size_t h, const float *x, const float *y,
                     const size_t *rows, size_t nr, const float *const *ck, const float *const *cv,
                     const float *const *ik, const float *const *iv, float *const *keys,
                     float *const *values, char *err, size_t errlen);

/* Cached prediction: StaticExecutor::predict_chunk per estimator
 * (cpu.rs:2200-2273), over 1024-row chunks (cpu.rs:2111-2153).
 * x [B,Q,H]; logits [B,Q,width] (every decoder output). */
int ora_predict_cached(const ora_model *model, size_t b, size_t n, size_t h, size_t q,
                       const float *x, const float *const *column_keys,
                       const float *const *column_values, const float *const *icl_keys,
                       const float *const *icl_values, float *logits, char *err, size_t errlen);

/* Uncached forward: Executor::predict_logits_inner (cpu.rs:997-1065). x
 * [B,T,H] with the N training rows first; y [B,N]; logits [B,T-N,width]. */
int ora_predict_uncached(const ora_model *model, size_t b, size_t t, size_t n, size_t h,
                         const float *x, const float *y, float *logits, char *err, size_t errlen);

/* Row representations [B,T,512] and column embeddings [B,T,H+4,128] of the
 * uncached forward (the ForwardTrace stages, cpu.rs:227-258); either may be NULL. */
int ora_trace_uncached(const ora_model *model, size_t b, size_t t, size_t n, size_t h,
                       const float *x, const float *y, float *columns, float *rows, char *err,
                       size_t errlen);

/* ---- Primitive kernels, exported for known-answer tests ---- */
void ora_affine(const float *input, size_t rows, size_t in_dim, const float *weight,
                const float *bias, size_t out_dim, float *output);
void ora_layer_norm(const float *input, size_t rows, size_t width, const float *weight,
                    const float *bias, float *output);
void ora_gelu(int math, const float *input, size_t len, float *output);
float ora_fast_exp_negative(float value);
float ora_bounded_exp(float value);
void ora_one_hot_linear(const float *labels, size_t rows, const float *weight, const float *bias,
                        size_t classes, size_t out_dim, float *output);
void ora_rope(const float *input, size_t heads, size_t rows, size_t head_dim,
              const float *freqs, size_t position_offset, float *output);
/* qassmax_f32 (reference.rs:335-430): queries [heads,rows,head_dim]. */
void ora_qassmax(const float *queries, size_t heads, size_t rows, size_t head_dim,
                 size_t source_len, size_t hidden, const float *bm0_w, const float *bm0_b,
                 const float *bm2_w, const float *bm2_b, const float *qm0_w, const float *qm0_b,
                 const float *qm2_w, const float *qm2_b, float *output);
/* Online attention (source-major, reference.rs:792-1024), [heads,rows,head_dim]. */
int ora_attention(int math, const float *query, size_t query_rows, const float *key,
                  const float *value, size_t source_rows, size_t heads, size_t head_dim,
                  float *output);
/* Materialized attention (reference.rs:482-540). */
int ora_attention_materialized(const float *query, size_t query_rows, const float *key,
                               const float *value, size_t source_rows, size_t heads,
                               size_t head_dim, float *output);
/* aggregate_classifier_probabilities (cpu.rs:3873-3932). */
int ora_aggregate(const float *logits, size_t b, size_t q, size_t classes,
                  const uint64_t *class_permutations, float temperature, int average_logits,
                  float *probabilities);
/* quantiles::summarize for one [rows,999] block of one estimator set: mean and
 * quantiles at alphas (quantiles.rs:80-213). logits [B,Q,999]. */
int ora_regression_summary(const float *logits, size_t b, size_t q, size_t width,
                           const float *alphas, size_t n_alphas, float *mean, float *quantiles);
/* The same with every output of quantiles::summarize (any may be null): mean
 * [Q], unbiased variance [Q], inverse CDF at alphas [Q, n_alphas] and the
 * sorted quantiles [Q, width], each averaged over B. Sorting follows
 * f32::total_cmp; f64 arithmetic is not contracted into fused multiply-adds. */
int ora_regression_outputs(const float *logits, size_t b, size_t q, size_t width, const float *alphas,
                           size_t n_alphas, float *mean, float *variance, float *quantiles, float *raw);

#ifdef __cplusplus
}
#endif
#endif
