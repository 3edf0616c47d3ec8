// Shared definitions of the gfx950 TabICLv2 backend: model constants, error
// plumbing, wave64 reductions and the launchers every translation unit uses.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <string>
#include <vector>

namespace irx {

// Architecture constants (src/models/tabicl_v2/cpu.rs:40-54).
constexpr int kColumnDim = 128;
constexpr int kIclDim = 512;
constexpr int kHeads = 8;
constexpr int kInducing = 128;
constexpr int kColumnBlocks = 3;
constexpr int kRowBlocks = 3;
constexpr int kIclBlocks = 12;
constexpr int kReserved = 4;
constexpr int kFfnHidden = 1024;
constexpr int kColumnHead = kColumnDim / kHeads;  // 16
constexpr int kIclHead = kIclDim / kHeads;         // 64
// One column's cached inducing K (or V): 8 heads x 128 points x 16 dims.
constexpr int kColumnCache = kHeads * kInducing * kColumnHead;
// Softmaxes run in the exp2 domain: scores are scaled by log2(e).
constexpr float kLog2e = 1.44269504088896340736f;

// A failed HIP call or argument check. The C ABI turns it into a status code
// and the thread's last-error message.
struct Failure {
    int status;
    std::string message;
};

[[noreturn]] void fail(int status, const std::string &message);
void check_hip(hipError_t err, const char *what);

#define IRX_HIP(call) ::irx::check_hip((call), #call)

// ---- device helpers ----

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int offset = 32; offset >= 1; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int offset = 32; offset >= 1; offset >>= 1) v = fmaxf(v, __shfl_xor(v, offset, 64));
    return v;
}

// GELU, 0.5 x (1 + erf(x / sqrt 2)) (src/kernels/reference.rs:52-54), with
// 1 + erf(x / sqrt 2) = 2 - erfc(t) for x >= 0 and erfc(t) for x < 0, t =
// |x| / sqrt 2, and erfc(t) = 2^P(t) from one polynomial P(t) = t Q(t) of
// degree 10 on [0, 4], fitted by weighted least squares (Lawson iterations)
// to log2 erfc(t) so that the absolute error of erfc is near-minimax; past
// t = 4, erfc(t) < 1.6e-8 is taken as 0. Against float64 GELU the result is
// within 1.2e-7 (1 + |x|) over the whole line (the rounding of 0.5 x (2 - e)
// included; irx_test_gelu), with one exponential, ten FMAs and no branch
// where the device library's erff took about 35 instructions over two
// divergent branches. P'(0) = -2 / (sqrt(pi) ln 2) as erfc requires.
__device__ __forceinline__ float gelu_erf(float x) {
    const float tr = fabsf(x) * 0.70710678118654752440f;
    const float t = fminf(tr, 4.0f);
    float p = -1.9093147e-06f;
    p = fmaf(p, t, 3.273919e-05f);
    p = fmaf(p, t, -0.00024974978f);
    p = fmaf(p, t, 0.0010867005f);
    p = fmaf(p, t, -0.0026190714f);
    p = fmaf(p, t, 0.00038220972f);
    p = fmaf(p, t, 0.027573992f);
    p = fmaf(p, t, -0.1482662f);
    p = fmaf(p, t, -0.9184484f);
    p = fmaf(p, t, -1.627907f);
    float e = __builtin_amdgcn_exp2f(p * t);  // erfc(t)
    e = tr < 4.0f ? e : 0.0f;
    return 0.5f * x * (x < 0.0f ? e : 2.0f - e);
}

inline unsigned ceil_div(size_t a, size_t b) { return static_cast<unsigned>((a + b - 1) / b); }

// ---- opt-in kernel timing (irx_profile_enable / irx_profile_read) ----

enum KernelFamily { kFamGemm, kFamIcl, kFamIclMerge, kFamSmall, kFamNorm, kFamGlue, kFamCount };

// Records HIP events around one launch on `stream` while profiling is on,
// with the launch's algorithmic FLOPs and minimal HBM bytes.
class KernelTimer {
  public:
    KernelTimer(KernelFamily family, hipStream_t stream, double flops, double bytes);
    ~KernelTimer();
    KernelTimer(const KernelTimer &) = delete;
    KernelTimer &operator=(const KernelTimer &) = delete;

  private:
    KernelFamily family_;
    hipStream_t stream_;
    double flops_, bytes_;
    hipEvent_t start_ = nullptr, stop_ = nullptr;
};

// ---- launchers (defined in the kernel translation units) ----

// Where a product writes element (m, n): segments of `col_seg` columns go to
// head-major planes, rows to groups. A plain row-major [M, N] output is
// col_seg = N, heads = 1, rows_per_group >= M, strides 0, ldc = row stride.
struct OutMap {
    int col_seg;
    int heads;
    long long plane_stride;
    long long head_stride;
    int rows_per_group;
    long long group_stride;
    long long ldc;
    static OutMap row_major(int n, long long ldc) { return {n, 1, 0, 0, 1 << 30, 0, ldc}; }
    // [heads, rows, hd] head-major (and a second plane after `plane_stride`
    // for columns past heads * hd, e.g. keys then values).
    static OutMap head_major(int hd, int heads, long long rows, long long plane_stride) {
        return {hd, heads, plane_stride, rows * hd, 1 << 30, 0, hd};
    }
};

enum Epilogue : int {
    kEpiNone = 0,
    kEpiGelu = 1,      // gelu(acc + bias)
    kEpiResidual = 2,  // acc + bias + residual[m, n]
};

struct GemmArgs {
    const float *a;         // [M, K], row stride lda
    long long lda;
    const float *w;         // [N, K] row-major (PyTorch Linear layout)
    const float *bias;      // [N] or null
    const float *residual;  // [M, N] row-major with stride ldr, or null
    long long ldr;
    float *c;
    OutMap out;
    int m, n, k;
    int epilogue;
    // Optional LayerNorm of A's rows taken in the product's prologue (K = 128,
    // products for which gemm_fuses_ln holds): ln_w [128], ln_b [128] or null.
    const float *ln_w, *ln_b;
};

// C = epilogue(A W^T + bias) on FP32 MFMA. K must be a multiple of 64.
void gemm(const GemmArgs &args, hipStream_t stream);
// Whether gemm takes a LayerNorm prologue (GemmArgs::ln_w) for an
// m x n product with K = 128 and plain row-major output.
bool gemm_fuses_ln(long long m, int n);

// Post-attention half of a 128-wide block in one kernel (cpu.rs:1555-1601):
// s1 = state + (att Wo^T + bo); state = s1 + (gelu(LN2(s1) W1^T + b1) W2^T + b2).
// `pack` holds Wo [128,128], W1 [256,128] and W2 [128,256] as packed by
// tail128_pack (host code, kTail128PackFloats floats).
constexpr size_t kTail128PackFloats = 10 * 8192;
struct Tail128 {
    const float *att;  // [m, 128], row stride lda
    long long lda;
    float *state;      // [m, 128], row stride ldx, updated in place
    long long ldx;
    const float *pack;
    const float *bo, *n2w, *n2b, *b1, *b2;  // all [128] or [256]; bias-free LayerNorms pass zeros
    long long m;
};
void tail128_pack(const float *wo, const float *w1, const float *w2, float *out);
// rows16: the small-pass form (16 rows per workgroup, bitwise the same results).
void tail128(const Tail128 &t, hipStream_t stream, bool rows16 = false);

// Pre-attention head of a 128-wide block in one kernel: out = LN1(x) W^T + b
// for nb = 8, 16 or 24 blocks of 16 outputs (W [16 nb, 128], packed by
// head128_pack into head128_pack_floats(16 nb) floats).
struct Head128 {
    const float *x;  // [m, 128], row stride ldx
    long long ldx;
    const float *lnw, *lnb;  // [128]
    const float *pack;
    const float *b;          // [16 nb]
    float *out;              // [m, 16 nb], row stride ldo
    long long ldo;
    long long m;
    int nb;
};
size_t head128_pack_floats(int outputs);
void head128_pack(const float *w, int outputs, float *out);
void head128(const Head128 &h, hipStream_t stream);

// A cached column block in one kernel (multihead_attn2 of a column ISAB block
// with its feed-forward half, cached_block, cpu.rs:2587-2850; the reference's
// one-launch column_block_f32, kernels.rs:1342): for the states x of `cols`
// columns of `rows` rows,
//   q = LN1(x) Wq^T + bq, att = softmax(q K^T / 4) V per head of 16 against
//   the column's 128 cached inducing keys and values,
// then the tail128 chain on (att, x). Bitwise the results of head128 (8
// blocks), the 16-wide attention and tail128 run in turn.
struct ColumnBlock {
    float *state;  // [cols, rows, 128], updated in place
    long long rows;
    int cols;
    // Column c's keys [8][128][16] at k + (c / group) * group_stride + (c % group) * kColumnCache (values at v + ...).
    const float *k, *v;
    int group;
    long long group_stride;
    const float *lnw, *lnb;  // LN1 [128]
    const float *qpack;      // head128_pack of in_proj rows 0..127
    const float *qb;         // their bias [128]
    const float *pack;       // tail128_pack of the block
    const float *bo, *n2w, *n2b, *b1, *b2;
};
// rows16: the small-pass form (16 rows of a column per workgroup, the same bits).
void column_block(const ColumnBlock &c, hipStream_t stream, bool rows16 = false);

// Regression outputs of decoded quantiles [b, q, k] (k <= 4096) on the device
// (quantiles::summarize, quantiles.rs:80-213): per query row, averaged over
// the b estimators, the mean, the unbiased variance, the inverse CDF at each
// level and the sorted quantiles; null outputs are skipped. regression_tables
// (host) prepares the tail fit's log levels and each level's case of the
// inverse CDF.
constexpr int kRegressionMaxLevels = 64;
struct RegressionLevel {
    int kind;     // 0 left tail, 1 right tail, 2 the last quantile, 3 between quantiles
    int segment;  // kind 3: the lower quantile's index
    double value; // kind 0 / 1: the difference of log levels; kind 3: the interpolation weight
};
struct RegressionSummary {
    const float *decoded;
    int b, q, k;
    int tail;               // quantiles in each tail fit
    const double *tail_x;   // [2 * tail]: ln of the left levels, then of one minus the right ones
    int levels;
    const RegressionLevel *level;  // [levels]
    float *mean, *variance;        // [q]
    float *at_levels;              // [q, levels]
    float *raw;                    // [q, k]
};
void regression_tables(const float *alphas, int n_alphas, int k, int *tail, std::vector<double> &tail_x,
                       std::vector<RegressionLevel> &levels);
void regression_summary(const RegressionSummary &s, hipStream_t stream);

// epilogue(LN(x) W^T + b) over 512-wide rows x [m, 512] (W [n, 512]), the
// LayerNorm in the product's prologue: kLnGelu writes gelu() row-major [m, n];
// kLnQass (n = 512) runs each head's QASS query MLP and gate and writes
// head-major [m / rows, 8, rows, 64]. For prediction-sized m.
enum LnEpilogue : int { kLnGelu = 1, kLnQass = 2 };
struct LnLinear {
    const float *x;
    long long ldx;
    const float *lnw, *lnb;  // [512]; bias-free LayerNorms pass zeros
    const float *w, *b;      // [n, 512], [n]
    float *out;
    long long ldo;           // kLnGelu: output row stride
    int m, n;
    const float *qm0w, *qm0b, *qm2w, *qm2b;  // kLnQass: [64, 64], [64] each
    const float *base;                       // kLnQass: [8, 64]
    int rows;                                // kLnQass: rows per estimator
};
void ln_linear512(const LnLinear &a, int epilogue, hipStream_t stream);

// The QASS query MLP and gate over already projected head-major query rows q
// [m, 64] (m = estimators x 8 heads x rows): out = q * base[head] * (1 +
// tanh(gelu(q Wm0^T + bm0) Wm2^T + bm2)), head = (row / rows) % 8
// (qassmax_f32, reference.rs:417-428), with kLnQass's arithmetic. For the
// build's N-row queries.
struct QassRows {
    const float *q;                  // [m, 64]
    const float *w0, *b0, *w2, *b2;  // [64, 64], [64] each
    const float *base;               // [8, 64]
    float *out;                      // [m, 64]
    long long m;
    int rows;                        // rows per (estimator, head)
    int compute_units;
};
void qass_rows(const QassRows &a, hipStream_t stream);

// LayerNorm over `width` (128 or 512), eps 1e-5, two passes (reference.rs:223-252).
void layer_norm(const float *x, long long ldx, const float *weight, const float *bias, float *y,
                long long ldy, long long rows, int width, hipStream_t stream);

// Attention of 16-wide heads with online softmax. Element (seq, head, row, d)
// of Q is at q + qoff(seq) + row * q_row + head * q_head + d, where qoff(seq) =
// (seq / group) * q_group + (seq % group) * q_seq; likewise K, V, O.
struct SmallAttention {
    const float *q, *k, *v;
    float *o;
    long long q_seq, q_group, q_row, q_head;
    long long k_seq, k_group, k_row, k_head;
    long long v_seq, v_group, v_row, v_head;
    long long o_seq, o_group, o_row, o_head;
    int group;           // sequences per group (>= 1)
    int seqs, heads;
    int q_rows, kv_rows;
    float scale;         // 1/sqrt(16)
    const float *rope_cos, *rope_sin;  // [positions, 16] tables or null
    // More than 128 keys: room for key ranges split over workgroups (null: no
    // split); small_attention_partial_floats gives the size that allows them.
    float *partial;
    long long partial_floats;
    // 0 chooses the kernel; 1 keeps the per-wave / long kernels; 2 forces the
    // staged kernel (every key in LDS once per item) where it applies.
    int method;
};
void small_attention(const SmallAttention &args, hipStream_t stream);
long long small_attention_partial_floats(const SmallAttention &args);

// ICL attention of 64-wide heads: Q [pairs, q_rows, 64] (head-major, q_stride
// between pairs), K and V [pairs, kv_rows, 64]; the output goes to tokens
// [b * q_rows + row, head * 64 + d] with pair = b * 8 + head, row stride ldo.
// Split-K partials use `partial` (floats) when splits > 1.
struct IclAttention {
    const float *q;
    long long q_pair_stride;
    const float *k, *v;
    long long kv_pair_stride;
    float *o;
    long long ldo;
    int pairs, q_rows, kv_rows;
    float *partial;       // [splits, pairs, q_rows_padded, 65] or null
    size_t partial_floats;
    int compute_units;
    // The FP16 cache (split-FP16 products) instead of k / v: K [pairs, Np, 64]
    // and tile-transposed V [pairs, Np / 64, 64, 64], Np = kv_rows rounded up to 64.
    const unsigned short *k16, *v16;
    // Or the FP8 cache: K [pairs, Np, 64] and V^T tiles as the FP16 one, E4M3
    // bytes, with the values' scales [pairs, 64] (value = byte * scale).
    const unsigned char *k8, *v8;
    const float *kscale, *vscale;
};
// Splits the ICL attention would use, and the partial floats it needs.
// Floats of the split partials icl_attention needs for this shape (0: none).
size_t icl_attention_partial_floats(int pairs, int q_rows, int kv_rows, int compute_units, bool f16 = false);
void icl_attention(const IclAttention &args, hipStream_t stream);
// Halves of one FP16 cache plane (K or V) for `pairs` x `rows` keys.
inline size_t icl16_plane(long long pairs, long long rows) { return (size_t)pairs * ((rows + 63) / 64 * 64) * 64; }
// One ICL block's FP8 cache (IRX_PRECISION_HALF), in one allocation: K
// [pairs, Np, 64] and V^T tiles [pairs, Np / 64, 64, 64] as E4M3 bytes, then
// the key and value scales [pairs, 64] and the encoder's peak words [2, pairs, 64].
inline size_t icl8_plane(long long pairs, long long rows) { return (size_t)pairs * ((rows + 63) / 64 * 64) * 64; }
inline size_t icl8_block_bytes(long long pairs, long long rows) {
    return 2 * icl8_plane(pairs, rows) + 4 * (size_t)pairs * 64 * 4;
}
struct Icl8Block {
    unsigned char *k, *v;
    float *kscale, *vscale;
    unsigned *kpeak, *vpeak;
};
Icl8Block icl8_block(void *base, long long pairs, long long rows);
// FP16 K and V [pairs, rows, 64] (logical layout, FP16 bits) into the FP8
// block at `block`; values that are not finite in FP16 are counted into `bad`.
void encode_icl8(const unsigned short *k, const unsigned short *v, long long rows, int pairs, void *block,
                 unsigned *bad, hipStream_t stream);
// K and V [pairs, rows, 64] (FP32, or FP16 bits when src_f16) into the FP16
// cache layout; adds the count of values not finite in FP16 to *bad.
void pack_icl16(const void *k, const void *v, bool src_f16, long long rows, int pairs, unsigned short *k16,
                unsigned short *v16, unsigned *bad, hipStream_t stream);
// The FP16 cache back to logical FP16 K and V [pairs, rows, 64].
void unpack_icl16(const unsigned short *k16, const unsigned short *v16, long long rows, int pairs,
                  unsigned short *k, unsigned short *v, hipStream_t stream);

// TabICL preprocessing (preprocess.hip), in f64. Fit: statistics of every
// kept feature, [groups, 9, kept_count] (mean, scale, minimum, maximum,
// lower, upper, then lambda, mean, scale of the power transform), and a
// status per feature (0 ok, 1 non-finite statistics, 2 Yeo-Johnson bounds
// not finite, 3 power transform not finite). Features go `batch` at a time
// through `scratch` (batch x 3 x rows doubles).
struct PreprocessFit {
    const void *x;  // [rows, columns], f32 or f64 (x_f64)
    int x_f64;
    long long rows, columns;
    const unsigned *kept;
    int kept_count;
    int groups;
    int methods[2];  // 0 none, 1 power
    double threshold;
    double *scratch;
    int batch;
    double *stats;
    int *status;
    int raw;         // power fit on the values as given (a test of the Yeo-Johnson fit alone)
    double *fitted;  // raw mode: fitted values [kept_count, rows], or null
};
void preprocess_fit(const PreprocessFit &args, hipStream_t stream);

// Transform: every group's FP32 rows [groups, rows, kept_count]. `redo`
// (null on the first pass) marks the (chunk, group) pairs to recompute with
// clipping after `overflow` flagged them.
struct PreprocessTransform {
    const void *x;
    int x_f64;
    long long rows, columns;
    const unsigned *kept;
    int kept_count;
    int groups;
    int methods[2];
    const double *stats;
    long long chunk_rows;
    const int *redo;
    int *overflow;
    int *nonfinite;
    float *out;
};
void preprocess_transform(const PreprocessTransform &args, hipStream_t stream);
// Members' rows [members, rows, features] from the group rows and each
// member's group and feature order.
void preprocess_gather(const float *group_rows, long long rows, int features, int members,
                       const unsigned *member_groups, const unsigned *orders, float *out, hipStream_t stream);

// Glue kernels (glue.hip).
void column_input(const float *x, long long x_estimator_stride, int b, int rows, int h, const float *in_w, const float *in_b,
                  const float *labels, float *state, uint8_t *missing_rows, hipStream_t stream);
void build_rows(const float *state, int b, int rows, int h, const float *cls, float *seq,
                hipStream_t stream);
void gather_cls(const float *seq, long long seqs, int len, float *cls, hipStream_t stream);
void add_inplace(float *y, const float *x, long long count, hipStream_t stream);
// y = gelu_erf(x) elementwise (every kernel's GELU; for tests).
void gelu_apply(const float *x, float *y, long long count, hipStream_t stream);
// Label embeddings [n, width] of targets [n] from a y_encoder's weight [width,
// classes] and bias [width]: column `class` + bias (classifier), or target *
// weight + bias (regressor, classes = 1).
void label_embeddings(const float *targets, long long n, const float *w, const float *b, int classes, int width,
                      bool classifier, float *out, hipStream_t stream);
void repeat_rows(const float *src, long long src_floats, long long copies, float *dst,
                 hipStream_t stream);
void count_nonfinite(const float *x, long long count, unsigned *counter, hipStream_t stream);
void fill_zero(float *x, long long count, hipStream_t stream);
void copy_floats(const float *src, float *dst, long long count, hipStream_t stream);

}  // namespace irx
