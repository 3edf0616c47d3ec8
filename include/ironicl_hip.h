/*
 * ironicl_hip.h - C ABI of the MI355X (gfx950) TabICLv2 FP32 forward backend.
 *
 * The library, libironicl_hip.so, replaces Ironicl's CUDA backend at its
 * plugin point: the `Device` enum (src/models/tabicl_v2/mod.rs:15-41) and the
 * `cuda` module surface (src/models/tabicl_v2/cuda/mod.rs:47-52). A thin Rust
 * FFI crate wraps these entry points into a `rocm` module with the same
 * surface.
 *
 * Conventions
 *   - Every entry point returns an irx_status. On failure the calling thread's
 *     irx_last_error() holds a message. Nothing panics or aborts across the ABI.
 *   - Host buffers passed in are borrowed for the duration of the call; output
 *     buffers are allocated by the caller.
 *   - All tensors are FP32, row-major, in the reference's logical layouts.
 *   - Weights are reference counted and shared by every predictor of a model.
 *   - Calls on one predictor serialize (an internal mutex); different
 *     predictors may run concurrently, each on its own HIP stream.
 */
#ifndef IRONICL_HIP_H
#define IRONICL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define IRX_ABI_VERSION 1

/* Result codes. The Rust wrapper maps them onto `Error` like gpu_error /
 * out_of_memory (src/kernels/cuda/mod.rs:61-68): DEVICE_ERROR and
 * OUT_OF_MEMORY become Error::UnsupportedBackend("ROCm: ..."),
 * INVALID_ARGUMENT becomes Error::InvalidArgument, INTERRUPTED carries the
 * progress hook's error (src/progress.rs:29-72). */
typedef enum irx_status {
    IRX_OK = 0,
    IRX_NO_DEVICE = 1,        /* no usable GPU, or IRONICL_NO_ROCM is set: Device::new() -> None */
    IRX_OUT_OF_MEMORY = 2,
    IRX_INVALID_ARGUMENT = 3, /* shape or pointer mismatch */
    IRX_DEVICE_ERROR = 4,     /* a HIP call failed */
    IRX_INTERRUPTED = 5,      /* the progress hook returned non-zero */
    IRX_DOES_NOT_FIT = 6,     /* the context does not fit the device: the caller falls back to the CPU */
    IRX_NOT_FINITE = 7,       /* a cached key or value is not finite (cuda/build.rs:340-350) */
    IRX_UNSUPPORTED = 8       /* e.g. a grouped all-missing (-100) triple in build inputs */
} irx_status;

/* Precision of the products (Precision in src/models/tabicl_v2/cuda/mod.rs:71-105).
 * FP32: optimize="safe", FP32 everywhere, the ICL cache in FP32.
 * SPLIT: optimize="auto": the ICL cache in FP16 (cpu.rs:4038-4044) and the ICL
 * attention's products on FP16 MFMA with queries and probabilities split into
 * high and low FP16 parts; other products in FP32.
 * HALF: optimize="fast": built as SPLIT (the context keeps FP16 K/V), then the
 * resident ICL cache is FP8 E4M3 with a scale per (estimator, head, dim)
 * (cuda/cache.rs:60-275) and the ICL attention's products take FP16 queries
 * and probabilities, one FP16 product each; other products in FP32. */
typedef enum irx_precision {
    IRX_PRECISION_FP32 = 0,
    IRX_PRECISION_SPLIT = 1,
    IRX_PRECISION_HALF = 2
} irx_precision;

typedef enum irx_task { IRX_TASK_CLASSIFIER = 0, IRX_TASK_REGRESSOR = 1 } irx_task;

/* Progress stages (src/progress.rs: Stage::Build, Stage::Predict). */
typedef enum irx_stage { IRX_STAGE_BUILD = 0, IRX_STAGE_PREDICT = 1 } irx_stage;

/* Estimators B, features H, training rows N, decoder outputs per row
 * (workspace::Shape, src/models/tabicl_v2/cuda/workspace.rs:25). */
typedef struct irx_shape {
    size_t ensembles;
    size_t features;
    size_t rows;
    size_t outputs;
} irx_shape;

typedef struct irx_device irx_device;
typedef struct irx_weights irx_weights;
typedef struct irx_built_cache irx_built_cache;
typedef struct irx_predictor irx_predictor;

/* Looks up an official tensor by checkpoint name (src/format/model.rs:772-867):
 * returns 0 and a borrowed view valid for the duration of the call, non-zero
 * when absent. Replaces the `|name| self.tensor(name)` closure passed to
 * ModelWeights::new (src/models/tabicl_v2/cuda/weights.rs:299). */
typedef int (*irx_tensor_lookup)(void *user, const char *name, const float **data, size_t *len);

/* Progress hook (src/progress.rs:29-72): called on the calling thread between
 * groups and passes; a non-zero return stops the work with IRX_INTERRUPTED. */
typedef int (*irx_progress_fn)(void *user, int stage, size_t done, size_t total);

/* The ICL keys and values of one block on the host, `[B, 8, N, 64]` each
 * (IclSource::block, src/models/tabicl_v2/cuda/cache.rs:61-64). */
typedef int (*irx_icl_source)(void *user, size_t block, const float **keys, const float **values);

/* Message of the last failure on this thread; never NULL. */
const char *irx_last_error(void);
int irx_abi_version(void);

/* ---- Device: Device::new / free_memory (src/kernels/cuda/mod.rs:116-209) ---- */

/* Opens GPU `ordinal`. IRX_NO_DEVICE when there is none or IRONICL_NO_ROCM is
 * set (the CPU path then runs); an error only when a device exists but fails. */
int irx_device_open(int ordinal, irx_device **out);
void irx_device_close(irx_device *device);
int irx_device_free_memory(irx_device *device, size_t *bytes);
/* Number of compute units (for launch sizing by callers and tests). */
int irx_device_compute_units(irx_device *device, int *units);

/* ---- Weights: ModelWeights::new / budget (src/models/tabicl_v2/cuda/weights.rs:286-342) ---- */

/* Uploads every official tensor once. The regressor's absent LayerNorm biases
 * are zero-filled (src/format/model.rs:273-280). The device stays open while
 * any weights hold it. */
int irx_weights_upload(irx_device *device, int task, irx_tensor_lookup lookup, void *user,
                       irx_weights **out);
void irx_weights_retain(irx_weights *weights);
void irx_weights_release(irx_weights *weights);
size_t irx_weights_bytes(const irx_weights *weights);
/* Free device memory, capped by device_limit minus the weights (0 = no limit). */
int irx_weights_budget(const irx_weights *weights, uint64_t device_limit, size_t *budget);

/* ---- Build: fits / build (src/models/tabicl_v2/cuda/build.rs:42-212) ---- */

/* Bytes per cached ICL key or value at `precision` (context_bytes, build.rs:92-97). */
size_t irx_context_bytes(int precision);
/* Device bytes of one stream's prediction workspace on `device` for passes of
 * `pass_rows` rows (0 for an invalid shape; the attention's split plan, and so
 * its partials, follow the device's compute units). A predictor holds one per
 * stream beside its caches; irx_predictor_new fits them into the budget by
 * taking one stream, then halving the passes (Predictor::predict's
 * out-of-memory fallback, predictor.rs:248-258). No counterpart in the
 * reference. */
size_t irx_predict_workspace_bytes(irx_device *device, const irx_shape *shape, int precision, size_t pass_rows);
/* Whether a context of `shape` builds on the device within `budget` bytes
 * (fits, build.rs:158-160), planned for the calling thread's current device. */
int irx_build_fits(size_t budget, int precision, const irx_shape *shape);

/* BuildInputs (build.rs:42-63). */
typedef struct irx_build_inputs {
    irx_shape shape;
    const float *x;                    /* [B, N, H] preprocessed training rows */
    const float *column_labels;        /* [B, N, 128] column-stage label embeddings */
    const float *icl_labels;           /* [B, N, 512] ICL label embeddings */
    const float *inducing_queries[3];  /* per column block: norm1, q-proj and QASSMax of the inducing points, [128, 128] */
    const float *base_scales[12];      /* per ICL block: QASSMax base scale for N sources, [512] */
    const float *rope_frequencies;     /* [8] */
    const float *cls_tokens;           /* [4, 128] */
    size_t budget;                     /* device bytes the build may use */
    irx_progress_fn progress;          /* may be NULL */
    void *progress_user;
    /* No counterpart in the reference's BuildInputs: [B, N] targets (a
     * classifier's class indices 0..9 as floats, a regressor's targets), or
     * NULL. When column_labels and icl_labels are both NULL, the device
     * computes those embeddings from the targets through the uploaded
     * y_encoder weights, bitwise as target_embeddings (cpu.rs:1658-1680) does
     * on the host, instead of receiving 640 floats per training row. */
    const float *targets;
} irx_build_inputs;

/* BuildOutputs (build.rs:66-74), host buffers owned by the caller. A NULL
 * pointer skips that tensor's download (the context then lives in HBM only,
 * through `keep`). The reserved CLS streams of the column tensors are left as
 * they are. */
typedef struct irx_build_outputs {
    float *column_keys[3];   /* [B, H+4, 8, 128, 16] */
    float *column_values[3];
    float *icl_keys[12];     /* [B, 8, N, 64]; FP16 bits (2 bytes each) at IRX_PRECISION_SPLIT and HALF */
    float *icl_values[12];
} irx_build_outputs;

/* Builds a context: the training rows' pass through the column ISAB, the row
 * transformer and the ICL self-attention, keeping every block's K/V. With
 * keep != NULL the ICL and column K/V stay resident in HBM and *keep owns them
 * until passed to irx_predictor_new or irx_built_cache_free (BuiltCache,
 * src/models/tabicl_v2/cuda/cache.rs:137). */
int irx_build(irx_weights *weights, int precision, const irx_build_inputs *inputs,
              irx_build_outputs *outputs, irx_built_cache **keep);
void irx_built_cache_free(irx_built_cache *cache);

/* ---- Predictor (src/models/tabicl_v2/cuda/predictor.rs:57-271) ---- */

/* ContextTensors (predictor.rs:57-72). */
typedef struct irx_context_tensors {
    irx_shape shape;
    const float *column_keys[3];    /* [B, H+4, 8, 128, 16]; may be NULL when adopting a built cache */
    const float *column_values[3];
    irx_icl_source icl;             /* may be NULL when adopting a built cache; at IRX_PRECISION_SPLIT
                                     * and HALF its blocks are FP16 bits [B, 8, N, 64] */
    void *icl_user;
    const float *base_scales[12];   /* [512] each */
    const float *rope_frequencies;  /* [8] */
    const float *cls_tokens;        /* [4, 128] */
    size_t budget;
} irx_context_tensors;

/* Uploads the context's caches, or adopts `adopt` (ownership transfers, also
 * on failure). IRX_DOES_NOT_FIT when the context cannot stay on the device:
 * the caller predicts on the CPU (Predictor::new -> None). */
int irx_predictor_new(irx_weights *weights, int precision, const irx_context_tensors *context,
                      irx_built_cache *adopt, irx_predictor **out);
void irx_predictor_free(irx_predictor *predictor);
/* Whether the ICL cache streams from the host (always 0: on a 288 GB MI355X
 * the cache stays resident). */
int irx_predictor_streamed(const irx_predictor *predictor);
/* Query rows per pass. */
size_t irx_predictor_pass_rows(const irx_predictor *predictor);
/* Sets the query rows per pass (a multiple of 32, at least 32). */
int irx_predictor_set_pass_rows(irx_predictor *predictor, size_t rows);
/* Streams (1 to 4) the passes of a prediction rotate over: more than one lets
 * one pass's short launches overlap another pass's work (2 is the default); 1
 * runs every pass in order on one stream. Each stream has its own workspace.
 * Results are identical either way. No counterpart in the reference (its
 * predictor runs passes in order, predictor.rs:224-271). */
int irx_predictor_set_streams(irx_predictor *predictor, int streams);
/* Whether prediction passes replay HIP graphs (1, the default; the environment
 * variable IRONICL_NO_GRAPHS=1 makes 0 the default) or launch their kernels one
 * by one (0). A graph is captured per stream and pass size on first use; each
 * replay reads the pass's rows from a copy in the stream's workspace. Passes
 * launch one by one while kernel timing (irx_profile_enable) is on. Results are
 * identical either way. No counterpart in the reference. */
int irx_predictor_set_graphs(irx_predictor *predictor, int enable);
/* Copies floats [offset, offset + floats) of one resident context tensor to
 * host memory, after every pass issued before the call. `tensor` indexes the
 * reference's context tensor order (context_tensors, cpu.rs:4106-4123):
 * 0..5 = column.{0..2}.{key,value} [B, H+4, 8, 128, 16], 6..29 =
 * icl.{0..11}.{key,value} [B, 8, N, 64]. It is what exporting a GPU-built
 * context to IRCNTXT needs (StaticExecutor::save_context, cpu.rs:1716-1742;
 * the reference's CUDA build always writes the tensors to host pages,
 * cpu.rs:744-805, where this backend keeps them in HBM until asked). Values
 * are FP32 (4 bytes), except the ICL tensors of an IRX_PRECISION_SPLIT
 * predictor, which are FP16 bits (2 bytes), as its context stores them. An
 * IRX_PRECISION_HALF predictor reads them as FP16 too when it adopted a build
 * (which keeps its FP16 cache beside the FP8 one); one made from context
 * tensors holds them only as FP8 and returns IRX_UNSUPPORTED (its caller has
 * the FP16 tensors). */
int irx_predictor_read_context(irx_predictor *predictor, size_t tensor, size_t offset, size_t floats,
                               void *dst);

/* Predictor::predict (predictor.rs:224-271): x [B, Q, H] on the host, logits
 * [B, Q, outputs] on the host. cpu_rows, when not NULL, gets Q flags: 1 for a
 * row with a grouped all-missing (-100) triple, which the caller predicts on
 * the CPU (its logits are left unspecified). */
int irx_predictor_predict(irx_predictor *predictor, const float *x, size_t q, float *logits,
                          uint8_t *cpu_rows, irx_progress_fn progress, void *progress_user);
/* The same with x and logits already in device memory (HBM-resident inputs).
 * Returns when the logits are written. */
int irx_predictor_predict_device(irx_predictor *predictor, const float *x_device, size_t q,
                                 float *logits_device, uint8_t *cpu_rows);

/* ---- Kernel timing (opt-in). No counterpart in the reference, whose
 * profile.rs (src/profile.rs:5-146) times CPU phases: this records HIP events
 * on the stream each kernel family launches on, with each launch's
 * algorithmic FLOPs and minimal HBM bytes, for roofline measurement. ---- */

/* ---- TabICL preprocessing on the GPU (f64) ----
 * Fitting every kept feature at once replaces fit_feature
 * (src/models/tabicl_v2/preprocess.rs:259-296, run per feature on CPU
 * threads there); transforming replaces Normalization::transform and
 * Preprocessor::ensemble_rows (:223-254, :588-613), writing each member's
 * FP32 rows where the predictor reads them. The ensemble draws, labels and
 * the IRPREP bytes stay host code. */

/* x [rows, columns] on the host, f32 (x_f64 = 0) or f64; kept: increasing
 * indices of the kept columns; methods[groups]: 0 none, 1 power, unique.
 * statistics [groups, 9, kept_count] f64 receives, per group and kept feature,
 * mean, scale, minimum, maximum, lower, upper, then (power groups) lambda,
 * mean, scale (Normalization::statistics order; none groups leave the last
 * three 0). Errors as fit_feature's. */
int irx_preprocess_fit(irx_device *device, const void *x, int x_f64, size_t rows, size_t columns,
                       const uint32_t *kept, size_t kept_count, const int *methods, size_t groups,
                       double outlier_threshold, double *statistics);

typedef struct irx_preprocessor irx_preprocessor;
/* A fitted preprocessor resident on the device: statistics as
 * irx_preprocess_fit returns them, member_groups[members] and
 * feature_orders[members, kept_count] (each a permutation of 0..kept_count). */
int irx_preprocessor_new(irx_device *device, size_t columns, const uint32_t *kept, size_t kept_count,
                         const int *methods, size_t groups, const double *statistics, size_t members,
                         const uint32_t *member_groups, const uint32_t *feature_orders, irx_preprocessor **out);
void irx_preprocessor_free(irx_preprocessor *preprocessor);
/* x [rows, columns] on the host. With members_out, out receives each member's
 * rows [members, rows, kept_count] (the predictor's x); otherwise each
 * group's rows [groups, rows, kept_count]. out is device memory when
 * out_on_device. A group whose power transform overflows within a chunk of
 * chunk_rows rows is recomputed for that chunk clipped to the training range
 * (the reference predicts in chunks of 8,192 rows, fitted.rs:13; training
 * rows are one chunk). */
int irx_preprocessor_transform(irx_preprocessor *preprocessor, const void *x, int x_f64, size_t rows,
                               size_t chunk_rows, int members_out, float *out, int out_on_device);

typedef struct irx_kernel_stats {
    uint64_t launches;
    double milliseconds; /* summed kernel durations */
    double flops;        /* algorithmic FLOPs of those launches */
    double bytes;        /* minimal HBM bytes: operands read once, results written once */
    double busy_milliseconds; /* union of the launch intervals (launches on the
                               * predictor's two streams may overlap) */
} irx_kernel_stats;

/* Kernel families, as bits of irx_profile_enable's mask. */
#define IRX_PROFILE_GEMM (1u << 0)
#define IRX_PROFILE_ICL_ATTENTION (1u << 1)
#define IRX_PROFILE_ICL_MERGE (1u << 2)
#define IRX_PROFILE_SMALL_ATTENTION (1u << 3)
#define IRX_PROFILE_LAYER_NORM (1u << 4)
#define IRX_PROFILE_GLUE (1u << 5)
#define IRX_PROFILE_ALL 0xffffffffu

/* Records the families in `families` (0 stops recording); a non-zero mask
 * clears the totals first. Recording adds two events per recorded launch. */
int irx_profile_enable(unsigned families);
/* Totals of one kernel family: "gemm", "icl_attention", "icl_merge",
 * "small_attention", "layer_norm" or "glue". Waits for recorded launches. */
int irx_profile_read(const char *family, irx_kernel_stats *out);

/* ---- Regression summary on the GPU ---- */

/* Regression outputs of a regressor's decoded quantiles, on the device
 * (quantiles::summarize, src/models/tabicl_v2/quantiles.rs:80-213, which the
 * reference runs on the host). decoded: device [ensembles, rows, quantiles]
 * (2 <= quantiles <= 4096), e.g. irx_predictor_predict_device's output of a
 * regressor. Per row, each estimator's quantiles are sorted and summarized in
 * f64, then averaged over the estimators and rounded to f32, into device
 * outputs (any may be null): mean [rows]; variance [rows] (unbiased);
 * at_levels [rows, n_levels], the inverse CDF at each of the host array
 * `levels` (finite, at most 64; 0.5 gives the median); raw [rows, quantiles],
 * the sorted quantiles. Synchronous. */
int irx_regression_summary(irx_device *device, const float *decoded, size_t ensembles, size_t rows,
                           size_t quantiles, const float *levels, size_t n_levels, float *mean,
                           float *variance, float *at_levels, float *raw);

/* ---- Kernel harness (cuda/testing.rs:27-207): one kernel family on host data ---- */

/* softmax(q k^T / 8) v for `pairs` (estimator, head) pairs: q [pairs, query_rows, 64],
 * k and v [pairs, rows, 64]; out [pairs, query_rows, 64]. */
int irx_test_icl_attention(irx_device *device, const float *q, const float *k, const float *v,
                           size_t pairs, size_t query_rows, size_t rows, float *out);
/* The FP32 attention of irx_test_icl_attention on device buffers, allocating
 * nothing. No counterpart in the reference: it is for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops).
 * q [pairs, query_rows, 64], k and v [pairs, rows, 64] and out are device
 * memory, 16-byte aligned; out receives token rows [pairs / 8, query_rows,
 * 512] (head h of estimator b at columns 64 h .. 64 h + 63 of row b,
 * query). The kernels' split-K partials live in a 64 MiB scratch array that
 * the library holds on each device from irx_device_open until the process
 * ends; a shape whose partials exceed it is refused with
 * IRX_INVALID_ARGUMENT (the split plan keeps them under 34 MB on a 256-CU
 * MI355X, so there none is). The work is enqueued on `stream` (a hipStream_t, or
 * NULL for the null stream) and the call returns without waiting. Every call
 * on one device shares its scratch array: calls whose work overlaps on one
 * device (on different streams, or from different threads) race. Results are
 * bitwise those of irx_test_icl_attention on the same device. */
int irx_icl_attention_noalloc(irx_device *device, const float *q, const float *k, const float *v, size_t pairs,
                              size_t query_rows, size_t rows, float *out, void *stream);
/* The same at `precision`: SPLIT packs k and v into the FP16 cache first;
 * HALF rounds them to FP16 and encodes the FP8 cache from those. */
int irx_test_icl_attention_precision(irx_device *device, int precision, const float *q, const float *k,
                                     const float *v, size_t pairs, size_t query_rows, size_t rows, float *out);
/* The FP8 cache block (IRX_PRECISION_HALF) of FP16 keys and values [pairs,
 * rows, 64] (FP16 bits), as the predictor holds it: K [pairs, Np, 64] E4M3
 * bytes (Np = rows rounded up to 64, zero rows after `rows`), V^T [pairs, Np /
 * 64, 64 dims, 64 keys] bytes (keys of each group of 16 in the order 0..3,
 * 8..11, 4..7, 12..15), key scales [pairs, 64] and value scales [pairs, 64]
 * (FP32), then [2, pairs, 64] words of the encoder's own. `block` receives
 * 2 * pairs * Np * 64 + 1024 * pairs bytes. */
int irx_test_encode_icl8(irx_device *device, const uint16_t *k, const uint16_t *v, size_t pairs, size_t rows,
                         void *block);
/* first = gelu(x w1^T + b1); second = first w2^T + b2 (+ first when width2 == width).
 * x [rows, depth], w1 [width, depth], w2 [width2, width]. */
int irx_test_products(irx_device *device, const float *x, const float *w1, const float *b1,
                      const float *w2, const float *b2, size_t rows, size_t width, size_t depth,
                      size_t width2, float *first, float *second);
/* The pre-attention head of a 128-wide block on `rows` rows: out [rows,
 * outputs] = LN1(x) w^T + b, LN1 with lnw / lnb, w [outputs, 128] (outputs
 * 128, 256 or 384: the column blocks' queries, the CLS block's keys and
 * values, the row blocks' Q/K/V). fused = 1 runs the one-kernel head, 0 a
 * LayerNorm and a product. */
int irx_test_block_head(irx_device *device, int fused, const float *x, size_t rows, const float *lnw,
                        const float *lnb, const float *w, const float *b, size_t outputs, float *out);
/* The post-attention half of a 128-wide block (cpu.rs:1555-1601) on `rows`
 * rows: s1 = state + (att wo^T + bo); out = s1 + (gelu(LN2(s1) w1^T + b1) w2^T + b2),
 * LN2 with n2w / n2b. fused = 1 runs the one-kernel tail, 2 its
 * small-pass form (16 rows per workgroup), 0 the separate products and
 * LayerNorm. wo [128,128], w1 [256,128], w2 [128,256]. With
 * repeats > 1 the tail is applied again repeats - 1 times after `out` is
 * read (for timing with irx_profile_read). */
int irx_test_block_tail(irx_device *device, int fused, const float *att, const float *state, size_t rows,
                        const float *wo, const float *bo, const float *n2w, const float *n2b,
                        const float *w1, const float *b1, const float *w2, const float *b2,
                        size_t repeats, float *out);
/* A cached column block (multihead_attn2 of a column ISAB block and its
 * feed-forward half, cpu.rs:2587-2850; the reference's column_block_f32,
 * kernels.rs:1342) on `cols` columns of `rows` rows, state [cols, rows, 128]
 * updated into out: LN1 (lnw / lnb), q = LN1(state) wq^T + bq (wq [128, 128]),
 * attention of 8 heads of 16 (scale 1/4) to the column's cached inducing keys
 * and values k, v [cols, 8, 128, 16], then the tail of irx_test_block_tail
 * (same weights). fused = 1 runs the one-kernel block, 2 its small-pass form
 * (16 rows per workgroup), 0 the head, 16-wide attention and tail launches.
 * repeats as irx_test_block_tail. */
int irx_test_column_block(irx_device *device, int fused, const float *state, size_t cols, size_t rows,
                          const float *k, const float *v, const float *lnw, const float *lnb, const float *wq,
                          const float *bq, const float *wo, const float *bo, const float *n2w, const float *n2b,
                          const float *w1, const float *b1, const float *w2, const float *b2, size_t repeats,
                          float *out);
/* LayerNorm fused into a 512-wide product, x [m, 512], w [n, 512]:
 * epilogue 1 (GELU): out [m, n] = gelu(LN(x) w^T + b); epilogue 2 (QASS, the
 * ICL query path, n = 512): q = LN(x) w^T + b, then per head
 * q * base[head] * (1 + tanh(gelu(q qm0w^T + qm0b) qm2w^T + qm2b)), into out
 * head-major [m / rows, 8, rows, 64] (StaticExecutor::qass, cpu.rs:3798-3853);
 * epilogue 3: the same result as the build computes it for many query rows
 * (LayerNorm, a tiled head-major Q projection, then the QASS MLP and gate
 * over the projected rows). */
int irx_test_ln_linear(irx_device *device, int epilogue, const float *x, size_t m, size_t rows,
                       const float *lnw, const float *lnb, const float *w, const float *b, size_t n,
                       const float *qm0w, const float *qm0b, const float *qm2w, const float *qm2b,
                       const float *base, float *out);
/* GELU, 0.5 x (1 + erf(x / sqrt 2)), of count floats as every kernel here
 * computes it (src/kernels/reference.rs:52-54). */
int irx_test_gelu(irx_device *device, const float *x, size_t count, float *out);
/* LayerNorm over width (128 or 512), eps 1e-5. */
int irx_test_layer_norm(irx_device *device, const float *x, const float *weight, const float *bias,
                        size_t rows, size_t width, float *out);
/* A plain device-to-device copy of `floats` floats by a one-float4-per-thread
 * kernel: the known-size reference for HBM traffic counters. */
int irx_test_copy(irx_device *device, size_t floats);
/* The Yeo-Johnson PowerTransformer fit alone (yeo_johnson.rs fit_power) on
 * each column of x [rows, columns] f64 as given: lambda_mean_scale [3, columns]
 * and, when not NULL, the fitted standardized values [rows, columns]. */
int irx_test_power_fit(irx_device *device, const double *x, size_t rows, size_t columns, double *lambda_mean_scale,
                       double *fitted);
/* 16-wide-head attention: q [heads, query_rows, 16], k and v [heads, rows, 16];
 * more than 128 keys take the long-range kernel, with its key ranges split
 * over workgroups when the heads do not fill the chip. */
int irx_test_small_attention(irx_device *device, const float *q, const float *k, const float *v,
                             size_t heads, size_t query_rows, size_t rows, float *out);
/* The same with rotary position embedding of queries and keys (the row
 * transformer's, rope_non_interleaved_f32, reference.rs:433-475): dim d of
 * the token at position t becomes x[d] cos[t][d] + x[d ^ 8] sin[t][d], with
 * tables [max(query_rows, rows), 16] (sin signed). */
int irx_test_small_attention_rope(irx_device *device, const float *q, const float *k, const float *v,
                                  const float *rope_cos, const float *rope_sin, size_t heads, size_t query_rows,
                                  size_t rows, float *out);
/* Token-major sequences q [seqs, query_rows, heads, 16], k and v [seqs, rows,
 * heads, 16] (a token's heads adjacent, as in the row transformer), RoPE
 * tables as above or null, through the kernel `method` picks: 0 the
 * library's choice, 1 the per-wave and long-range kernels, 2 the staged
 * kernel (every key of an item in LDS once; more than 16 queries, at most 512
 * keys). With reps > 0 the launch is then repeated reps times on the null
 * stream and *ms_per_launch receives the mean launch time from HIP events. */
int irx_test_small_attention_tokens(irx_device *device, int method, const float *q, const float *k, const float *v,
                                    const float *rope_cos, const float *rope_sin, size_t seqs, size_t heads,
                                    size_t query_rows, size_t rows, float *out, int reps, float *ms_per_launch);

#ifdef __cplusplus
}
#endif
#endif
