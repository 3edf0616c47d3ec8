/*
 * CPU restatement of Ironicl's FP32 TabICLv2 forward pass: the oracle.
 *
 * TEST INFRASTRUCTURE ONLY (see tabicl_oracle.h): the checker of the HIP
 * backend and the CPU baseline bench.py times beside it. Never part of the
 * product path.
 *
 * Each function cites the reference file:line it restates.
 */
#include "tabicl_oracle.h"

#include <immintrin.h>
#include <math.h>
#include <omp.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define D 128      /* column / row embedding width, cpu.rs:40 */
#define E 512      /* ICL width, cpu.rs:41 */
#define HEADS 8    /* cpu.rs:42 */
#define M 128      /* inducing points, cpu.rs:43 */
#define COLB 3     /* column blocks, cpu.rs:44 */
#define ICLB 12    /* ICL blocks, cpu.rs:45 */
#define RES 4      /* CLS streams, cpu.rs:47 */
#define KEY_TILE 128 /* ATTENTION_KEY_TILE_ROWS, cpu.rs:49 */
#define CHUNK 1024 /* QUERY_CHUNK_ROWS, cpu.rs:54 */
#define LN_EPS 1e-5f /* reference.rs:14 */

static int g_threads = 1;

void ora_set_threads(int threads) { g_threads = threads > 0 ? threads : 1; }
int ora_get_threads(void) { return g_threads; }

static void set_err(char *err, size_t errlen, const char *fmt, ...) {
    if (!err || !errlen) return;
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(err, errlen, fmt, ap);
    va_end(ap);
}

static void *xcalloc(size_t count, size_t size) {
    void *p = calloc(count ? count : 1, size);
    if (!p) {
        fprintf(stderr, "oracle: out of memory (%zu x %zu)\n", count, size);
        abort();
    }
    return p;
}

/* ------------------------------------------------------------------ */
/* Elementwise math                                                    */
/* ------------------------------------------------------------------ */

/* Rust never contracts a * b + c into a fused multiply-add, so this file is
 * built with -ffp-contract=off and every fused operation of the reference
 * (mul_add, _mm512_fmadd_ps / _mm512_fnmadd_ps) is an explicit fmaf. Rust's
 * f32::round() rounds halves away from zero (roundf); the AVX-512 kernels'
 * _mm512_cvt_roundps_epi32 with _MM_FROUND_TO_NEAREST_INT rounds them to
 * even (rintf under the default rounding mode). */
#define ORA_LOG2E 1.44269504088896340736f
#define ORA_LN2 0.693147180559945309417f

/* bounded_exp: src/kernels/cpu/ops/pointwise.rs:49-74. */
float ora_bounded_exp(float value) {
    float v = value < -40.0f ? -40.0f : (value > 20.0f ? 20.0f : value);
    int exponent = (int)roundf(v * ORA_LOG2E);
    float r = fmaf((float)(-exponent), ORA_LN2, v);
    float p = fmaf(r, 1.0f / 5040.0f, 1.0f / 720.0f);
    p = fmaf(r, p, 1.0f / 120.0f);
    p = fmaf(r, p, 1.0f / 24.0f);
    p = fmaf(r, p, 1.0f / 6.0f);
    p = fmaf(r, p, 0.5f);
    p = fmaf(r, p, 1.0f);
    p = fmaf(r, p, 1.0f);
    union { unsigned u; float f; } pw;
    pw.u = (unsigned)(exponent + 127) << 23;
    return p * pw.f;
}

static inline float exp_polynomial(float r) {
    float p = 1.0f / 5040.0f;
    const float c[7] = {1.0f / 720.0f, 1.0f / 120.0f, 1.0f / 24.0f, 1.0f / 6.0f, 0.5f, 1.0f, 1.0f};
    for (int i = 0; i < 7; ++i) p = fmaf(p, r, c[i]);
    return p;
}

static inline float pow2i(int exponent) {
    union { unsigned u; float f; } pw;
    pw.u = (unsigned)(exponent + 127) << 23;
    return pw.f;
}

/* fast_exp_negative, the scalar form: src/kernels/cpu/arch/x86_64.rs:40-51
 * (half away from zero; exponent * LN_2 rounded before the subtraction). */
float ora_fast_exp_negative(float value) {
    float v = value < -87.0f ? -87.0f : value;
    int exponent = (int)roundf(v * ORA_LOG2E);
    float r = v - (float)exponent * ORA_LN2;
    return exp_polynomial(r) * pow2i(exponent);
}

/* One lane of the AVX-512 exp in softmax_exp_sum_avx512 and gelu_avx512
 * (x86_64.rs:610-660, 1394-1441): ties to even, the remainder one fnmadd. */
static inline float vector_exp_negative(float value) {
    float v = value < -87.0f ? -87.0f : value;
    int exponent = (int)rintf(v * ORA_LOG2E);
    float r = fmaf(-(float)exponent, ORA_LN2, v);
    return exp_polynomial(r) * pow2i(exponent);
}

/* fast_erf: pointwise.rs:76-91 (Abramowitz-Stegun 7.1.26). */
static float fast_erf(float value) {
    float mag = fabsf(value);
    float sgn = value < 0.0f ? -1.0f : 1.0f;
    if (mag >= 6.0f) return sgn;
    if (mag < 1e-4f) return value * 1.12837916709551257390f;
    float t = 1.0f / fmaf(0.3275911f, mag, 1.0f);
    float p = fmaf(1.0614054f, t, -1.4531521f);
    p = fmaf(p, t, 1.4214138f);
    p = fmaf(p, t, -0.28449672f);
    p = fmaf(p, t, 0.2548296f) * t;
    return sgn * (1.0f - p * ora_bounded_exp(-mag * mag));
}

/* gelu (reference.rs:52-54) and fast_gelu (pointwise.rs:93-96). */
static inline float gelu_exact(float x) { return 0.5f * x * (1.0f + erff(x / 1.41421356237309504880f)); }
static inline float gelu_native(float x) { return 0.5f * x * (1.0f + fast_erf(x / 1.41421356237309504880f)); }

/* One lane of gelu_avx512 (x86_64.rs:1394-1441): its own erf, with the
 * vector exp clamped at -87 rather than bounded_exp. */
static inline float gelu_vector(float x) {
    float scaled = x * 0.707106781186547524401f;
    float mag = fmaxf(scaled, 0.0f - scaled);
    float t = 1.0f / fmaf(0.3275911f, mag, 1.0f);
    float p = 1.0614054f;
    const float c[4] = {-1.4531521f, 1.4214138f, -0.28449672f, 0.2548296f};
    for (int i = 0; i < 4; ++i) p = fmaf(p, t, c[i]);
    p = p * t;
    float e = vector_exp_negative(0.0f - mag * mag);
    float erf = fmaf(-p, e, 1.0f);
    if (scaled < 0.0f) erf = 0.0f - erf;
    if (mag < 1e-4f) erf = scaled * 1.12837916709551257390f;
    if (mag >= 6.0f) erf = scaled < 0.0f ? -1.0f : 1.0f;
    return 0.5f * x * (1.0f + erf);
}

/* gelu_f32 (reference.rs:256-266): native math is gelu_avx512 over whole
 * groups of 16 and fast_gelu on the rest (x86_64.rs:1347-1441). */
void ora_gelu(int math, const float *input, size_t len, float *output) {
    if (math == ORA_MATH_NATIVE) {
        size_t body = len / 16 * 16;
        for (size_t i = 0; i < body; ++i) output[i] = gelu_vector(input[i]);
        for (size_t i = body; i < len; ++i) output[i] = gelu_native(input[i]);
    } else {
        for (size_t i = 0; i < len; ++i) output[i] = gelu_exact(input[i]);
    }
}

/* The softmax numerators of one score row against its maximum, in place,
 * added into *denominator. Native: softmax_exp_sum_avx512
 * (x86_64.rs:610-660): 16 lane sums over whole groups of 16, reduced
 * pairwise, then the scalar fast_exp_negative of the rest added in order, the
 * total added once. Exact (the exact-math feature): libm expf, each numerator
 * added to the denominator in order (reference.rs:963-969). */
static void softmax_numerators(int math, float *scores, size_t n, float maximum, float *denominator) {
    if (math != ORA_MATH_NATIVE) {
        for (size_t i = 0; i < n; ++i) *denominator += (scores[i] = expf(scores[i] - maximum));
        return;
    }
    /* vector_exp_negative on 16 lanes at once: the same clamp, ties-to-even
     * exponent, fused remainder, polynomial and exponent bits per lane. */
    const __m512 vmax = _mm512_set1_ps(maximum), lo = _mm512_set1_ps(-87.0f);
    const __m512 log2e = _mm512_set1_ps(ORA_LOG2E), ln2 = _mm512_set1_ps(ORA_LN2);
    const float coef[7] = {1.0f / 720.0f, 1.0f / 120.0f, 1.0f / 24.0f, 1.0f / 6.0f, 0.5f, 1.0f, 1.0f};
    __m512 acc = _mm512_setzero_ps();
    size_t body = n / 16 * 16;
    for (size_t i = 0; i < body; i += 16) {
        const __m512 v = _mm512_max_ps(_mm512_sub_ps(_mm512_loadu_ps(scores + i), vmax), lo);
        const __m512 e = _mm512_roundscale_ps(_mm512_mul_ps(v, log2e), _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
        const __m512 r = _mm512_fnmadd_ps(e, ln2, v);
        __m512 poly = _mm512_set1_ps(1.0f / 5040.0f);
        for (int c = 0; c < 7; ++c) poly = _mm512_fmadd_ps(poly, r, _mm512_set1_ps(coef[c]));
        const __m512i bits = _mm512_slli_epi32(_mm512_add_epi32(_mm512_cvtps_epi32(e), _mm512_set1_epi32(127)), 23);
        const __m512 num = _mm512_mul_ps(poly, _mm512_castsi512_ps(bits));
        _mm512_storeu_ps(scores + i, num);
        acc = _mm512_add_ps(acc, num);
    }
    float lanes[16];
    _mm512_storeu_ps(lanes, acc);
    for (int w = 8; w >= 1; w >>= 1)
        for (int l = 0; l < w; ++l) lanes[l] += lanes[l + w];
    float total = lanes[0];
    for (size_t i = body; i < n; ++i) total += (scores[i] = ora_fast_exp_negative(scores[i] - maximum));
    *denominator += total;
}

/* ------------------------------------------------------------------ */
/* Dense kernels                                                       */
/* ------------------------------------------------------------------ */

/* 16-lane partial sums, the way the AVX-512 kernels reduce; any summation
 * order is within the parity tolerance. */
static inline float dot16(const float *a, const float *b, size_t n) {
    float acc[16] = {0};
    size_t k = 0;
    for (; k + 16 <= n; k += 16)
        for (int l = 0; l < 16; ++l) acc[l] = fmaf(a[k + l], b[k + l], acc[l]);
    float tail = 0.0f;
    for (; k < n; ++k) tail = fmaf(a[k], b[k], tail);
    for (int w = 8; w >= 1; w >>= 1)
        for (int l = 0; l < w; ++l) acc[l] += acc[l + w];
    return acc[0] + tail;
}

/* dot16's lane reduction on a vector: lanes l and l + 8, then l + 4, l + 2,
 * l + 1, the same additions in the same order. */
static inline float reduce16(__m512 acc) {
    const __m256 s8 = _mm256_add_ps(_mm512_castps512_ps256(acc), _mm512_extractf32x8_ps(acc, 1));
    const __m128 s4 = _mm_add_ps(_mm256_castps256_ps128(s8), _mm256_extractf128_ps(s8, 1));
    const __m128 s2 = _mm_add_ps(s4, _mm_movehl_ps(s4, s4));
    return _mm_cvtss_f32(_mm_add_ss(s2, _mm_shuffle_ps(s2, s2, 1)));
}

/* affine_f32: reference.rs:83-120. weight [out,in] (PyTorch layout).
 * Register-blocked as affine_avx512 runs it (x86_64.rs:1639-1780): four input
 * rows by four outputs share each 16-wide load; every output is still dot16's
 * arithmetic (16 lane chains over the input, reduced pairwise, then the tail,
 * then the bias), so the blocking changes no bit. */
void ora_affine(const float *input, size_t rows, size_t in_dim, const float *weight,
                const float *bias, size_t out_dim, float *output) {
    const size_t body = in_dim / 16 * 16;
    size_t r = 0;
    for (; r + 4 <= rows && body; r += 4) {
        const float *x0 = input + r * in_dim;
        size_t o = 0;
        for (; o + 4 <= out_dim; o += 4) {
            __m512 acc[4][4];
            for (int i = 0; i < 4; ++i)
                for (int c = 0; c < 4; ++c) acc[i][c] = _mm512_setzero_ps();
            for (size_t k = 0; k < body; k += 16) {
                __m512 w[4];
                for (int c = 0; c < 4; ++c) w[c] = _mm512_loadu_ps(weight + (o + c) * in_dim + k);
                for (int i = 0; i < 4; ++i) {
                    const __m512 xv = _mm512_loadu_ps(x0 + i * in_dim + k);
                    for (int c = 0; c < 4; ++c) acc[i][c] = _mm512_fmadd_ps(w[c], xv, acc[i][c]);
                }
            }
            for (int i = 0; i < 4; ++i)
                for (int c = 0; c < 4; ++c) {
                    const float *wr = weight + (o + c) * in_dim, *xr = x0 + i * in_dim;
                    float tail = 0.0f;
                    for (size_t k = body; k < in_dim; ++k) tail = fmaf(wr[k], xr[k], tail);
                    output[(r + i) * out_dim + o + c] = (bias ? bias[o + c] : 0.0f) + (reduce16(acc[i][c]) + tail);
                }
        }
        for (; o < out_dim; ++o)
            for (int i = 0; i < 4; ++i)
                output[(r + i) * out_dim + o] =
                    (bias ? bias[o] : 0.0f) + dot16(weight + o * in_dim, x0 + i * in_dim, in_dim);
    }
    for (; r < rows; ++r) {
        const float *x = input + r * in_dim;
        float *y = output + r * out_dim;
        for (size_t o = 0; o < out_dim; ++o)
            y[o] = (bias ? bias[o] : 0.0f) + dot16(weight + o * in_dim, x, in_dim);
    }
}

/* parallel_affine: rows split over workers (cpu.rs:3014-3048). */
static void affine_par(int workers, const float *input, size_t rows, size_t in_dim,
                       const float *weight, const float *bias, size_t out_dim, float *output) {
    if (workers <= 1 || rows < 16) {
        ora_affine(input, rows, in_dim, weight, bias, out_dim, output);
        return;
    }
    size_t per = (rows + (size_t)workers - 1) / (size_t)workers;
#pragma omp parallel for num_threads(workers) schedule(static, 1)
    for (int w = 0; w < workers; ++w) {
        size_t start = (size_t)w * per;
        if (start >= rows) continue;
        size_t len = rows - start < per ? rows - start : per;
        ora_affine(input + start * in_dim, len, in_dim, weight, bias, out_dim, output + start * out_dim);
    }
}

/* layer_norm_f32: reference.rs:223-252 / layer_norm_avx512 x86_64.rs:1470-1520. */
void ora_layer_norm(const float *input, size_t rows, size_t width, const float *weight,
                    const float *bias, float *output) {
    for (size_t r = 0; r < rows; ++r) {
        const float *x = input + r * width;
        float *y = output + r * width;
        /* Lanes of 16 as the AVX-512 kernel sums, then the tail of a width
         * that is not a multiple of 16 (the scalar path's order). */
        size_t body = width / 16 * 16;
        float acc[16] = {0};
        for (size_t c = 0; c < body; c += 16)
            for (int l = 0; l < 16; ++l) acc[l] += x[c + l];
        for (int w = 8; w >= 1; w >>= 1)
            for (int l = 0; l < w; ++l) acc[l] += acc[l + w];
        for (size_t c = body; c < width; ++c) acc[0] += x[c];
        float mean = acc[0] / (float)width;
        float sq[16] = {0};
        for (size_t c = 0; c < body; c += 16)
            for (int l = 0; l < 16; ++l) {
                float d = x[c + l] - mean;
                sq[l] = fmaf(d, d, sq[l]);
            }
        for (int w = 8; w >= 1; w >>= 1)
            for (int l = 0; l < w; ++l) sq[l] += sq[l + w];
        for (size_t c = body; c < width; ++c) sq[0] = fmaf(x[c] - mean, x[c] - mean, sq[0]);
        float scale = 1.0f / sqrtf(sq[0] / (float)width + LN_EPS);
        for (size_t c = 0; c < width; ++c)
            y[c] = (x[c] - mean) * scale * weight[c] + (bias ? bias[c] : 0.0f);
    }
}

/* one_hot_linear_f32: reference.rs:190-220. Labels are class indices stored as f32. */
void ora_one_hot_linear(const float *labels, size_t rows, const float *weight, const float *bias,
                        size_t classes, size_t out_dim, float *output) {
    for (size_t r = 0; r < rows; ++r) {
        size_t c = (size_t)labels[r];
        for (size_t o = 0; o < out_dim; ++o) output[r * out_dim + o] = weight[o * classes + c] + bias[o];
    }
}

/* rope_non_interleaved_f32: reference.rs:433-475. */
void ora_rope(const float *input, size_t heads, size_t rows, size_t head_dim, const float *freqs,
              size_t position_offset, float *output) {
    size_t half = head_dim / 2;
    for (size_t row = 0; row < rows; ++row) {
        float position = (float)(position_offset + row);
        for (size_t d = 0; d < half; ++d) {
            float angle = position * freqs[d];
            float s = sinf(angle), c = cosf(angle);
            for (size_t h = 0; h < heads; ++h) {
                size_t off = (h * rows + row) * head_dim;
                float left = input[off + d], right = input[off + half + d];
                output[off + d] = left * c - right * s;
                output[off + half + d] = right * c + left * s;
            }
        }
    }
}

/* tokens_to_heads / heads_to_tokens: cpu.rs:5007-5019, 5123-5135. */
static void tokens_to_heads(const float *in, size_t rows, size_t dim, float *out) {
    size_t hd = dim / HEADS;
    for (size_t r = 0; r < rows; ++r)
        for (size_t h = 0; h < HEADS; ++h) memcpy(out + (h * rows + r) * hd, in + r * dim + h * hd, hd * 4);
}
static void heads_to_tokens(const float *in, size_t rows, size_t dim, float *out) {
    size_t hd = dim / HEADS;
    for (size_t r = 0; r < rows; ++r)
        for (size_t h = 0; h < HEADS; ++h) memcpy(out + r * dim + h * hd, in + (h * rows + r) * hd, hd * 4);
}

/* ------------------------------------------------------------------ */
/* Attention                                                           */
/* ------------------------------------------------------------------ */

/* Source-major online attention for `heads` heads, as the reference's x86-64
 * path runs it (source_major_online_attention_with_backend_f32,
 * reference.rs:792-1024, with the AVX-512 tiles of x86_64.rs): key tiles of
 * 128 outermost; per head, the tile's keys packed dimension-major and padded
 * to 16 sources; per block of 16 query rows, the score tile with one lane per
 * source (each score a sequential fused chain over the dimensions, times the
 * scale: attention_score_packed_key_padded_tile_avx512, x86_64.rs:866-915);
 * per row the running maximum, the rescale by exp(old - new) and the
 * numerators' sum; then the value tile, one fused multiply-add per source in
 * order (attention_value_tile_fma). */
#define QUERY_BLOCK 16 /* ATTENTION_QUERY_BLOCK_ROWS, cpu.rs:48 */
static int attention_heads(int math, const float *query, size_t query_rows, const float *key,
                           const float *value, size_t source_rows, size_t heads, size_t head_dim,
                           float *output) {
    const float scale = 1.0f / sqrtf((float)head_dim);
    const size_t packed_tile = (KEY_TILE + 15) / 16 * 16;
    float *packed = xcalloc(packed_tile * head_dim, sizeof(float));
    float *scores = xcalloc(QUERY_BLOCK * KEY_TILE, sizeof(float));
    float *qd = xcalloc(QUERY_BLOCK * head_dim, sizeof(float));
    float *maximum = xcalloc(heads * query_rows, sizeof(float));
    float *denominator = xcalloc(heads * query_rows, sizeof(float));
    int status = 0;
    for (size_t i = 0; i < heads * query_rows; ++i) maximum[i] = -INFINITY;
    memset(output, 0, heads * query_rows * head_dim * sizeof(float));
    for (size_t s0 = 0; s0 < source_rows && !status; s0 += KEY_TILE) {
        const size_t ns = source_rows - s0 < KEY_TILE ? source_rows - s0 : KEY_TILE;
        const size_t ps = (ns + 15) / 16 * 16;
        for (size_t h = 0; h < heads && !status; ++h) {
            const float *kt = key + (h * source_rows + s0) * head_dim;
            const float *vt = value + (h * source_rows + s0) * head_dim;
            memset(packed, 0, ps * head_dim * sizeof(float));
            for (size_t d = 0; d < head_dim; ++d)
                for (size_t s = 0; s < ns; ++s) packed[d * ps + s] = kt[s * head_dim + d];
            for (size_t q0 = 0; q0 < query_rows && !status; q0 += QUERY_BLOCK) {
                const size_t rows = query_rows - q0 < QUERY_BLOCK ? query_rows - q0 : QUERY_BLOCK;
                const float *qt = query + (h * query_rows + q0) * head_dim;
                /* The block's queries dimension-major, zero rows past `rows`,
                 * so the tile loop has constant bounds (one register per row). */
                for (size_t d = 0; d < head_dim; ++d)
                    for (size_t r = 0; r < QUERY_BLOCK; ++r) qd[d * QUERY_BLOCK + r] = r < rows ? qt[r * head_dim + d] : 0.0f;
                /* One 16-source score vector per query row, in registers: each
                 * lane a fused chain over the dimensions, then times the scale. */
                const __m512 vscale = _mm512_set1_ps(scale);
                for (size_t s = 0; s < ps; s += 16) {
                    __m512 acc[QUERY_BLOCK];
                    for (int r = 0; r < QUERY_BLOCK; ++r) acc[r] = _mm512_setzero_ps();
                    for (size_t d = 0; d < head_dim; ++d) {
                        const __m512 kd = _mm512_loadu_ps(packed + d * ps + s);
                        const float *qv = qd + d * QUERY_BLOCK;
                        for (int r = 0; r < QUERY_BLOCK; ++r) acc[r] = _mm512_fmadd_ps(kd, _mm512_set1_ps(qv[r]), acc[r]);
                    }
                    const size_t lanes = ns - s < 16 ? ns - s : 16;
                    const __mmask16 keep = (__mmask16)((1u << lanes) - 1u);
                    for (size_t r = 0; r < rows; ++r)
                        _mm512_mask_storeu_ps(scores + r * ns + s, keep, _mm512_mul_ps(acc[r], vscale));
                }
                for (size_t r = 0; r < rows; ++r) {
                    float *sc = scores + r * ns;
                    const size_t state = h * query_rows + q0 + r;
                    /* The tile's maximum (and whether any score is NaN), 16 at a time. */
                    __m512 vmax = _mm512_set1_ps(-INFINITY);
                    __mmask16 nan = 0;
                    size_t s = 0;
                    for (; s + 16 <= ns; s += 16) {
                        const __m512 x = _mm512_loadu_ps(sc + s);
                        nan |= _mm512_cmp_ps_mask(x, x, _CMP_UNORD_Q);
                        vmax = _mm512_max_ps(vmax, x);
                    }
                    float tile_max = _mm512_reduce_max_ps(vmax);
                    if (nan) status = -1;
                    for (; s < ns; ++s) {
                        if (sc[s] != sc[s]) status = -1;
                        if (sc[s] > tile_max) tile_max = sc[s];
                    }
                    float mx = maximum[state] > tile_max ? maximum[state] : tile_max;
                    if (status || (isinf(mx) && mx > 0)) { status = -1; break; }
                    if (mx == -INFINITY) continue;
                    float *o = output + state * head_dim;
                    if (denominator[state] != 0.0f) {
                        const float old = expf(maximum[state] - mx);
                        for (size_t d = 0; d < head_dim; ++d) o[d] *= old;
                        denominator[state] *= old;
                    }
                    softmax_numerators(math, sc, ns, mx, &denominator[state]);
                    maximum[state] = mx;
                }
                if (status) break;
                /* The value tile: per output element one fused multiply-add per
                 * source, in source order. Four rows at a time share each value
                 * row's loads, their 64-dim outputs held in registers. */
                size_t r = 0;
                if (head_dim == 64) {
                    for (; r + 4 <= rows; r += 4) {
                        float *o = output + (h * query_rows + q0 + r) * 64;
                        __m512 acc[4][4];
                        for (int i = 0; i < 4; ++i)
                            for (int c = 0; c < 4; ++c) acc[i][c] = _mm512_loadu_ps(o + i * 64 + 16 * c);
                        const float *w0 = scores + r * ns;
                        for (size_t s = 0; s < ns; ++s) {
                            const float *v = vt + s * 64;
                            const __m512 v0 = _mm512_loadu_ps(v), v1 = _mm512_loadu_ps(v + 16);
                            const __m512 v2 = _mm512_loadu_ps(v + 32), v3 = _mm512_loadu_ps(v + 48);
                            for (int i = 0; i < 4; ++i) {
                                const __m512 ws = _mm512_set1_ps(w0[i * ns + s]);
                                acc[i][0] = _mm512_fmadd_ps(ws, v0, acc[i][0]);
                                acc[i][1] = _mm512_fmadd_ps(ws, v1, acc[i][1]);
                                acc[i][2] = _mm512_fmadd_ps(ws, v2, acc[i][2]);
                                acc[i][3] = _mm512_fmadd_ps(ws, v3, acc[i][3]);
                            }
                        }
                        for (int i = 0; i < 4; ++i)
                            for (int c = 0; c < 4; ++c) _mm512_storeu_ps(o + i * 64 + 16 * c, acc[i][c]);
                    }
                }
                if (head_dim == 16 && r < rows) {
                    /* 16-wide heads: the block's rows in one register each. */
                    __m512 acc[QUERY_BLOCK];
                    float *o = output + (h * query_rows + q0) * 16;
                    for (size_t i = r; i < rows; ++i) acc[i] = _mm512_loadu_ps(o + i * 16);
                    for (size_t s = 0; s < ns; ++s) {
                        const __m512 v = _mm512_loadu_ps(vt + s * 16);
                        for (size_t i = r; i < rows; ++i)
                            acc[i] = _mm512_fmadd_ps(_mm512_set1_ps(scores[i * ns + s]), v, acc[i]);
                    }
                    for (size_t i = r; i < rows; ++i) _mm512_storeu_ps(o + i * 16, acc[i]);
                    r = rows;
                }
                for (; r < rows; ++r) {
                    float *o = output + (h * query_rows + q0 + r) * head_dim;
                    const float *w = scores + r * ns;
                    for (size_t s = 0; s < ns; ++s) {
                        const float *v = vt + s * head_dim;
                        for (size_t d = 0; d < head_dim; ++d) o[d] = fmaf(w[s], v[d], o[d]);
                    }
                }
            }
        }
    }
    for (size_t i = 0; i < heads * query_rows && !status; ++i) {
        const float den = denominator[i];
        if (!isfinite(den) || den == 0.0f) { status = -1; break; }
        for (size_t d = 0; d < head_dim; ++d) output[i * head_dim + d] /= den;
    }
    free(packed);
    free(scores);
    free(qd);
    free(maximum);
    free(denominator);
    return status;
}

int ora_attention(int math, const float *query, size_t query_rows, const float *key,
                  const float *value, size_t source_rows, size_t heads, size_t head_dim,
                  float *output) {
    if (!query_rows || !source_rows || !heads || !head_dim) return -1;
    return attention_heads(math, query, query_rows, key, value, source_rows, heads, head_dim, output);
}

/* Head-parallel cached attention: parallel_cached_attention, cpu.rs:4439-4525. */
static int attention_par(int math, int workers, const float *query, size_t query_rows,
                         const float *key, const float *value, size_t source_rows, size_t head_dim,
                         float *output) {
    int w = workers < HEADS ? workers : HEADS;
    if (w <= 1)
        return attention_heads(math, query, query_rows, key, value, source_rows, HEADS, head_dim, output);
    int per = (HEADS + w - 1) / w;
    int status = 0;
#pragma omp parallel for num_threads(w) schedule(static, 1) reduction(| : status)
    for (int t = 0; t < w; ++t) {
        int start = t * per;
        if (start >= HEADS) continue;
        int nh = HEADS - start < per ? HEADS - start : per;
        size_t qe = query_rows * head_dim, se = source_rows * head_dim;
        status |= attention_heads(math, query + start * qe, query_rows, key + start * se,
                                  value + start * se, source_rows, (size_t)nh, head_dim,
                                  output + start * qe) != 0;
    }
    return status ? -1 : 0;
}

/* scaled_dot_product_attention_f32: reference.rs:482-540, and softmax_f32. */
int ora_attention_materialized(const float *query, size_t query_rows, const float *key,
                               const float *value, size_t source_rows, size_t heads,
                               size_t head_dim, float *output) {
    float scale = 1.0f / sqrtf((float)head_dim);
    float *scores = xcalloc(source_rows, sizeof(float));
    for (size_t h = 0; h < heads; ++h)
        for (size_t r = 0; r < query_rows; ++r) {
            const float *q = query + (h * query_rows + r) * head_dim;
            float mx = -INFINITY;
            for (size_t s = 0; s < source_rows; ++s) {
                float acc = 0.0f;
                for (size_t d = 0; d < head_dim; ++d) acc = fmaf(q[d], key[(h * source_rows + s) * head_dim + d], acc);
                scores[s] = acc * scale;
                if (scores[s] > mx) mx = scores[s];
            }
            float sum = 0.0f;
            for (size_t s = 0; s < source_rows; ++s) sum += (scores[s] = expf(scores[s] - mx));
            for (size_t s = 0; s < source_rows; ++s) scores[s] /= sum;
            float *o = output + (h * query_rows + r) * head_dim;
            for (size_t d = 0; d < head_dim; ++d) o[d] = 0.0f;
            for (size_t s = 0; s < source_rows; ++s)
                for (size_t d = 0; d < head_dim; ++d)
                    o[d] = fmaf(scores[s], value[(h * source_rows + s) * head_dim + d], o[d]);
        }
    free(scores);
    return 0;
}

/* ------------------------------------------------------------------ */
/* Model weights                                                       */
/* ------------------------------------------------------------------ */

typedef struct {
    size_t dim;
    const float *n1w, *n1b, *n2w, *n2b;
    const float *in_w, *in_b, *out_w, *out_b;
    const float *l1w, *l1b, *l2w, *l2b;
    int qass;
    const float *bm0w, *bm0b, *bm2w, *bm2b, *qm0w, *qm0b, *qm2w, *qm2b;
} blk_t;

struct ora_model {
    int task, math;
    size_t width, targets;
    const float *in_w, *in_b, *col_yw, *col_yb;
    const float *ind[COLB];
    blk_t col1[COLB], col2[COLB], row[3], icl[ICLB];
    const float *cls, *out_ln_w, *out_ln_b, *freqs;
    const float *icl_yw, *icl_yb, *ln_w, *ln_b, *dec0_w, *dec0_b, *dec2_w, *dec2_b;
    float *arena;
    size_t arena_used, arena_cap;
};

typedef struct {
    ora_model *m;
    ora_lookup lookup;
    void *user;
    char *err;
    size_t errlen;
    int failed;
} loader_t;

static const float *take(loader_t *L, const char *name, size_t expected, int zero_if_missing) {
    if (L->failed) return NULL;
    const float *data = NULL;
    size_t len = 0;
    int missing = L->lookup(L->user, name, &data, &len);
    if (missing) {
        if (!zero_if_missing) {
            set_err(L->err, L->errlen, "model tensor '%s' is missing", name);
            L->failed = 1;
            return NULL;
        }
        data = NULL;
        len = expected;
    }
    if (len != expected) {
        set_err(L->err, L->errlen, "model tensor '%s' has %zu values; expected %zu", name, len, expected);
        L->failed = 1;
        return NULL;
    }
    ora_model *m = L->m;
    if (m->arena_used + expected > m->arena_cap) {
        set_err(L->err, L->errlen, "oracle weight arena overflow at '%s'", name);
        L->failed = 1;
        return NULL;
    }
    float *dst = m->arena + m->arena_used;
    if (data) memcpy(dst, data, expected * sizeof(float));
    else memset(dst, 0, expected * sizeof(float));
    m->arena_used += expected;
    return dst;
}

static void load_block(loader_t *L, blk_t *b, const char *prefix, size_t dim, int qass) {
    char name[256];
    int zero_bias = L->m->task == ORA_REGRESSOR; /* model.rs:273-280 */
    b->dim = dim;
    b->qass = qass;
#define T(field, suffix, len, z) (snprintf(name, sizeof name, "%s%s", prefix, suffix), b->field = take(L, name, len, z))
    T(in_w, ".attn.in_proj_weight", 3 * dim * dim, 0);
    T(in_b, ".attn.in_proj_bias", 3 * dim, 0);
    T(out_w, ".attn.out_proj.weight", dim * dim, 0);
    T(out_b, ".attn.out_proj.bias", dim, 0);
    T(l1w, ".linear1.weight", 2 * dim * dim, 0);
    T(l1b, ".linear1.bias", 2 * dim, 0);
    T(l2w, ".linear2.weight", 2 * dim * dim, 0);
    T(l2b, ".linear2.bias", dim, 0);
    T(n1w, ".norm1.weight", dim, 0);
    T(n1b, ".norm1.bias", dim, zero_bias);
    T(n2w, ".norm2.weight", dim, 0);
    T(n2b, ".norm2.bias", dim, zero_bias);
    if (qass) {
        size_t hd = dim / HEADS;
        T(bm0w, ".attn.ssmax_layer.base_mlp.0.weight", 64, 0);
        T(bm0b, ".attn.ssmax_layer.base_mlp.0.bias", 64, 0);
        T(bm2w, ".attn.ssmax_layer.base_mlp.2.weight", dim * 64, 0);
        T(bm2b, ".attn.ssmax_layer.base_mlp.2.bias", dim, 0);
        T(qm0w, ".attn.ssmax_layer.query_mlp.0.weight", 64 * hd, 0);
        T(qm0b, ".attn.ssmax_layer.query_mlp.0.bias", 64, 0);
        T(qm2w, ".attn.ssmax_layer.query_mlp.2.weight", hd * 64, 0);
        T(qm2b, ".attn.ssmax_layer.query_mlp.2.bias", hd, 0);
    }
#undef T
}

ora_model *ora_model_new(int task, ora_lookup lookup, void *user, int math, char *err, size_t errlen) {
    ora_model *m = xcalloc(1, sizeof *m);
    m->task = task;
    m->math = math;
    m->targets = task == ORA_CLASSIFIER ? 10 : 1;
    m->width = task == ORA_CLASSIFIER ? 10 : 999;
    m->arena_cap = 30u * 1000u * 1000u; /* > 28.6 M parameters */
    m->arena = xcalloc(m->arena_cap, sizeof(float));
    loader_t L = {m, lookup, user, err, errlen, 0};
    int zb = task == ORA_REGRESSOR;
    char name[256];
    m->in_w = take(&L, "col_embedder.in_linear.weight", D * 3, 0);
    m->in_b = take(&L, "col_embedder.in_linear.bias", D, 0);
    m->col_yw = take(&L, "col_embedder.y_encoder.weight", D * m->targets, 0);
    m->col_yb = take(&L, "col_embedder.y_encoder.bias", D, 0);
    for (int b = 0; b < COLB; ++b) {
        snprintf(name, sizeof name, "col_embedder.tf_col.blocks.%d.ind_vectors", b);
        m->ind[b] = take(&L, name, M * D, 0);
        snprintf(name, sizeof name, "col_embedder.tf_col.blocks.%d.multihead_attn1", b);
        load_block(&L, &m->col1[b], name, D, 1);
        snprintf(name, sizeof name, "col_embedder.tf_col.blocks.%d.multihead_attn2", b);
        load_block(&L, &m->col2[b], name, D, 0);
    }
    for (int b = 0; b < 3; ++b) {
        snprintf(name, sizeof name, "row_interactor.tf_row.blocks.%d", b);
        load_block(&L, &m->row[b], name, D, 0);
    }
    m->cls = take(&L, "row_interactor.cls_tokens", RES * D, 0);
    m->out_ln_w = take(&L, "row_interactor.out_ln.weight", D, 0);
    m->out_ln_b = take(&L, "row_interactor.out_ln.bias", D, zb);
    m->freqs = take(&L, "row_interactor.tf_row.rope.freqs", 8, 0);
    for (int b = 0; b < ICLB; ++b) {
        snprintf(name, sizeof name, "icl_predictor.tf_icl.blocks.%d", b);
        load_block(&L, &m->icl[b], name, E, 1);
    }
    m->icl_yw = take(&L, "icl_predictor.y_encoder.weight", E * m->targets, 0);
    m->icl_yb = take(&L, "icl_predictor.y_encoder.bias", E, 0);
    m->ln_w = take(&L, "icl_predictor.ln.weight", E, 0);
    m->ln_b = take(&L, "icl_predictor.ln.bias", E, zb);
    m->dec0_w = take(&L, "icl_predictor.decoder.0.weight", 1024 * E, 0);
    m->dec0_b = take(&L, "icl_predictor.decoder.0.bias", 1024, 0);
    m->dec2_w = take(&L, "icl_predictor.decoder.2.weight", m->width * 1024, 0);
    m->dec2_b = take(&L, "icl_predictor.decoder.2.bias", m->width, 0);
    if (L.failed) {
        ora_model_free(m);
        return NULL;
    }
    return m;
}

void ora_model_free(ora_model *m) {
    if (!m) return;
    free(m->arena);
    free(m);
}

size_t ora_model_width(const ora_model *m) { return m->width; }

/* ------------------------------------------------------------------ */
/* QASSMax                                                             */
/* ------------------------------------------------------------------ */

/* qass_base_scale: cpu.rs:3768-3791 (exact GELU, ln(max(source,1))). */
static void qass_base(const blk_t *b, size_t source, float *scale) {
    float log_source = logf((float)(source > 1 ? source : 1));
    float hidden[64];
    for (int i = 0; i < 64; ++i) hidden[i] = gelu_exact(fmaf(b->bm0w[i], log_source, b->bm0b[i]));
    ora_affine(hidden, 1, 64, b->bm2w, b->bm2b, b->dim, scale);
}

/* The query gate q * base * (1 + tanh(MLP_q(q))), over [heads, rows, hd]:
 * Executor path qassmax_f32 (reference.rs:396-428, exact GELU) and
 * StaticExecutor::qass (cpu.rs:3798-3853, GELU per the math mode). */
static void qass_gate(const blk_t *b, int gelu_math, int workers, const float *base, float *qh,
                      size_t rows) {
    size_t hd = b->dim / HEADS, qr = HEADS * rows;
    float *hidden = xcalloc(qr * 64, sizeof(float));
    float *gate = xcalloc(qr * hd, sizeof(float));
    affine_par(workers, qh, qr, hd, b->qm0w, b->qm0b, 64, hidden);
    ora_gelu(gelu_math, hidden, qr * 64, hidden);
    affine_par(workers, hidden, qr, 64, b->qm2w, b->qm2b, hd, gate);
    for (size_t h = 0; h < HEADS; ++h)
        for (size_t r = 0; r < rows; ++r)
            for (size_t d = 0; d < hd; ++d) {
                size_t i = (h * rows + r) * hd + d;
                qh[i] = qh[i] * base[h * hd + d] * (1.0f + tanhf(gate[i]));
            }
    free(hidden);
    free(gate);
}

void ora_qassmax(const float *queries, size_t heads, size_t rows, size_t head_dim,
                 size_t source_len, size_t hidden, const float *bm0_w, const float *bm0_b,
                 const float *bm2_w, const float *bm2_b, const float *qm0_w, const float *qm0_b,
                 const float *qm2_w, const float *qm2_b, float *output) {
    size_t embed = heads * head_dim, qr = heads * rows;
    float log_source = logf((float)(source_len > 1 ? source_len : 1));
    float *bh = xcalloc(hidden, sizeof(float));
    float *base = xcalloc(embed, sizeof(float));
    float *qh = xcalloc(qr * hidden, sizeof(float));
    for (size_t i = 0; i < hidden; ++i) bh[i] = gelu_exact(fmaf(bm0_w[i], log_source, bm0_b[i]));
    ora_affine(bh, 1, hidden, bm2_w, bm2_b, embed, base);
    ora_affine(queries, qr, head_dim, qm0_w, qm0_b, hidden, qh);
    for (size_t i = 0; i < qr * hidden; ++i) qh[i] = gelu_exact(qh[i]);
    ora_affine(qh, qr, hidden, qm2_w, qm2_b, head_dim, output);
    for (size_t h = 0; h < heads; ++h)
        for (size_t r = 0; r < rows; ++r)
            for (size_t d = 0; d < head_dim; ++d) {
                size_t i = (h * rows + r) * head_dim + d;
                output[i] = queries[i] * base[h * head_dim + d] * (1.0f + tanhf(output[i]));
            }
    free(bh);
    free(base);
    free(qh);
}

/* ------------------------------------------------------------------ */
/* Transformer block                                                   */
/* ------------------------------------------------------------------ */

/* source_heads: cpu.rs:1356-1416. LN1 then the K and V projections, head
 * major; RoPE on the keys for the row stage. Outputs [8, rows, hd] each. */
static void source_heads(const ora_model *m, const blk_t *b, const float *src, size_t rows, int rope,
                         int workers, float *kh, float *vh) {
    size_t d = b->dim;
    float *norm = xcalloc(rows * d, sizeof(float));
    float *proj = xcalloc(rows * d, sizeof(float));
    ora_layer_norm(src, rows, d, b->n1w, b->n1b, norm);
    affine_par(workers, norm, rows, d, b->in_w + d * d, b->in_b + d, d, proj);
    tokens_to_heads(proj, rows, d, kh);
    if (rope) {
        memcpy(proj, kh, rows * d * 4);
        ora_rope(proj, HEADS, rows, d / HEADS, m->freqs, 0, kh);
    }
    affine_par(workers, norm, rows, d, b->in_w + 2 * d * d, b->in_b + 2 * d, d, proj);
    tokens_to_heads(proj, rows, d, vh);
    free(norm);
    free(proj);
}

typedef struct {
    const float *qass_base; /* NULL without QASS; else [dim] base scale */
    int qass_gelu;          /* GELU math of the QASS query MLP */
    int rope;
    int workers;            /* affine / head workers (cached path) */
} attend_opts;

/* attend (cpu.rs:1475-1602) and cached_block (cpu.rs:2587-2850): LN1 + Q
 * projection (+QASS, +RoPE), attention, out-projection + residual, then the
 * residual feed-forward block. out may alias nothing; q is [q_rows, dim]. */
static int attend(const ora_model *m, const blk_t *b, const float *q, size_t q_rows, const float *kh,
                  const float *vh, size_t source_rows, const attend_opts *o, float *out) {
    size_t d = b->dim, hd = d / HEADS;
    float *t0 = xcalloc(q_rows * 2 * d, sizeof(float));
    float *t1 = xcalloc(q_rows * 2 * d, sizeof(float));
    int st = 0;
    ora_layer_norm(q, q_rows, d, b->n1w, b->n1b, t0);
    affine_par(o->workers, t0, q_rows, d, b->in_w, b->in_b, d, t1);
    tokens_to_heads(t1, q_rows, d, t0); /* t0 = query heads */
    if (o->qass_base) qass_gate(b, o->qass_gelu, o->workers, o->qass_base, t0, q_rows);
    if (o->rope) {
        memcpy(t1, t0, q_rows * d * 4);
        ora_rope(t1, HEADS, q_rows, hd, m->freqs, 0, t0);
    }
    st = attention_par(m->math, o->workers, t0, q_rows, kh, vh, source_rows, hd, t1);
    if (st) goto done;
    heads_to_tokens(t1, q_rows, d, t0);
    affine_par(o->workers, t0, q_rows, d, b->out_w, b->out_b, d, t1);
    for (size_t i = 0; i < q_rows * d; ++i) out[i] = q[i] + t1[i];
    ora_layer_norm(out, q_rows, d, b->n2w, b->n2b, t0);
    affine_par(o->workers, t0, q_rows, d, b->l1w, b->l1b, 2 * d, t1);
    ora_gelu(m->math, t1, q_rows * 2 * d, t1);
    affine_par(o->workers, t1, q_rows, 2 * d, b->l2w, b->l2b, d, t0);
    for (size_t i = 0; i < q_rows * d; ++i) out[i] += t0[i];
done:
    free(t0);
    free(t1);
    return st;
}

/* ------------------------------------------------------------------ */
/* Stages                                                              */
/* ------------------------------------------------------------------ */

/* target_embeddings: cpu.rs:1658-1680. */
static void target_embeddings(const ora_model *m, const float *w, const float *bias, const float *y,
                              size_t n, size_t width, float *out) {
    if (m->task == ORA_CLASSIFIER) {
        ora_one_hot_linear(y, n, w, bias, 10, width, out);
    } else {
        for (size_t r = 0; r < n; ++r)
            for (size_t o = 0; o < width; ++o) out[r * width + o] = y[r] * w[o] + bias[o];
    }
}

/* Grouped features (f+1, f+2, f+4) mod H and the 3->128 input affine, with the
 * all-missing marker: cpu.rs:1144-1157 and 2461-2473. */
static void column_input(const ora_model *m, const float *x, size_t t, size_t h, size_t f, float *emb) {
    static const size_t offs[3] = {1, 2, 4};
    for (size_t r = 0; r < t; ++r) {
        float s[3];
        for (int p = 0; p < 3; ++p) s[p] = x[r * h + (f + offs[p]) % h];
        float *e = emb + r * D;
        for (size_t c = 0; c < D; ++c) {
            float v = fmaf(m->in_w[c * 3 + 0], s[0], m->in_b[c]);
            v = fmaf(m->in_w[c * 3 + 1], s[1], v);
            e[c] = fmaf(m->in_w[c * 3 + 2], s[2], v);
        }
        if (s[0] == -100.0f && s[1] == -100.0f && s[2] == -100.0f)
            for (size_t c = 0; c < D; ++c) e[c] = -100.0f;
    }
}

/* Executor::column_stream + isab (cpu.rs:1132-1207): one feature over t rows,
 * the first n of them training rows. With kv != NULL, writes the three
 * multihead_attn2 K/V [8,128,16] (kv[2*block], kv[2*block+1]). Returns
 * non-zero for an all-missing column that a context cannot hold. */
static int column_stream(const ora_model *m, const float *x, const float *ycol, size_t t, size_t h,
                         size_t n, size_t f, int workers, float *emb, float **kv) {
    column_input(m, x, t, h, f, emb);
    for (size_t r = 0; r < n; ++r)
        for (size_t c = 0; c < D; ++c) emb[r * D + c] += ycol[r * D + c];
    float *kh = xcalloc((n > M ? n : M) * D, sizeof(float));
    float *vh = xcalloc((n > M ? n : M) * D, sizeof(float));
    float *hidden = xcalloc(M * D, sizeof(float));
    float *next = xcalloc(t * D, sizeof(float));
    float base[D];
    int st = 0;
    for (int blk = 0; blk < COLB && !st; ++blk) {
        int all_missing = 1;
        for (size_t i = 0; i < t * D && all_missing; ++i) all_missing = emb[i] == -100.0f;
        if (all_missing) { /* isab shortcut, cpu.rs:1187-1189 */
            if (kv) st = -2;
            continue;
        }
        /* multihead_attn1: inducing points attend to the n training rows, with QASS. */
        source_heads(m, &m->col1[blk], emb, n, 0, workers, kh, vh);
        qass_base(&m->col1[blk], n, base);
        attend_opts o1 = {base, ORA_MATH_EXACT, 0, workers};
        st = attend(m, &m->col1[blk], m->ind[blk], M, kh, vh, n, &o1, hidden);
        if (st) break;
        /* multihead_attn2: all t rows attend to the inducing state. */
        source_heads(m, &m->col2[blk], hidden, M, 0, workers, kh, vh);
        if (kv) {
            memcpy(kv[2 * blk], kh, M * D * 4);
            memcpy(kv[2 * blk + 1], vh, M * D * 4);
        }
        attend_opts o2 = {NULL, ORA_MATH_EXACT, 0, workers};
        st = attend(m, &m->col2[blk], emb, t, kh, vh, M, &o2, next);
        memcpy(emb, next, t * D * 4);
    }
    free(kh);
    free(vh);
    free(hidden);
    free(next);
    return st;
}

/* Executor::row_embedding (cpu.rs:1226-1266) and its StaticExecutor twin
 * (cpu.rs:3106-3144): CLS tokens replace the reserved streams, blocks 0 and 1
 * self-attend over L tokens with RoPE, block 2 lets the CLS tokens attend,
 * then out_ln of the four CLS tokens is the [512] row representation. */
static int row_embedding(const ora_model *m, const float *seq_in, size_t streams, float *out512) {
    size_t L = streams;
    float *seq = xcalloc(L * D, sizeof(float));
    float *nxt = xcalloc(L * D, sizeof(float));
    float *kh = xcalloc(L * D, sizeof(float));
    float *vh = xcalloc(L * D, sizeof(float));
    float cls_out[RES * D];
    int st = 0;
    memcpy(seq, seq_in, L * D * 4);
    memcpy(seq, m->cls, RES * D * 4);
    attend_opts o = {NULL, ORA_MATH_EXACT, 1, 1};
    for (int blk = 0; blk < 2 && !st; ++blk) {
        source_heads(m, &m->row[blk], seq, L, 1, 1, kh, vh);
        st = attend(m, &m->row[blk], seq, L, kh, vh, L, &o, nxt);
        memcpy(seq, nxt, L * D * 4);
    }
    if (!st) {
        source_heads(m, &m->row[2], seq, L, 1, 1, kh, vh);
        st = attend(m, &m->row[2], seq, RES, kh, vh, L, &o, cls_out);
    }
    if (!st) ora_layer_norm(cls_out, RES, D, m->out_ln_w, m->out_ln_b, out512);
    free(seq);
    free(nxt);
    free(kh);
    free(vh);
    return st;
}

/* row_embeddings: rows split over workers (cpu.rs:1209-1224, 3064-3104). */
static int row_embeddings(const ora_model *m, const float *columns, size_t t, size_t streams,
                          int workers, float *rows) {
    int st = 0;
#pragma omp parallel for num_threads(workers) schedule(static) reduction(| : st)
    for (size_t r = 0; r < t; ++r)
        st |= row_embedding(m, columns + r * streams * D, streams, rows + r * E) != 0;
    return st ? -1 : 0;
}

/* Decoder: cpu.rs:1297-1333 and 2543-2580. */
static void decoder(const ora_model *m, const float *rows, size_t t, int workers, float *logits) {
    float *norm = xcalloc(t * E, sizeof(float));
    float *hidden = xcalloc(t * 1024, sizeof(float));
    ora_layer_norm(rows, t, E, m->ln_w, m->ln_b, norm);
    affine_par(workers, norm, t, E, m->dec0_w, m->dec0_b, 1024, hidden);
    ora_gelu(m->math, hidden, t * 1024, hidden);
    affine_par(workers, hidden, t, 1024, m->dec2_w, m->dec2_b, m->width, logits);
    free(norm);
    free(hidden);
}

/* Executor::column_embeddings (cpu.rs:1073-1121): features on workers. */
static int column_embeddings(const ora_model *m, const float *x, const float *y, size_t t, size_t h,
                             size_t n, int workers, float *columns, float *const *feature_kv) {
    size_t streams = h + RES;
    float *ycol = xcalloc(n * D, sizeof(float));
    target_embeddings(m, m->col_yw, m->col_yb, y, n, D, ycol);
    for (size_t r = 0; r < t; ++r) memcpy(columns + r * streams * D, m->cls, RES * D * 4);
    int st = 0;
#pragma omp parallel for num_threads(workers) schedule(static) reduction(| : st)
    for (size_t f = 0; f < h; ++f) {
        float *emb = xcalloc(t * D, sizeof(float));
        float *kv[6];
        for (int i = 0; i < 6; ++i) kv[i] = feature_kv ? feature_kv[i] + f * M * D : NULL;
        st |= column_stream(m, x, ycol, t, h, n, f, 1, emb, feature_kv ? kv : NULL) != 0;
        for (size_t r = 0; r < t; ++r) memcpy(columns + (r * streams + RES + f) * D, emb + r * D, D * 4);
        free(emb);
    }
    free(ycol);
    return st ? -1 : 0;
}

/* Executor::icl_rows (cpu.rs:1270-1295): labels into the training rows, then
 * twelve blocks whose K/V come from the training rows only. Serial, as the
 * reference builds one estimator's ICL stage on one thread. */
static int icl_rows(const ora_model *m, float *rows, const float *y, size_t t, size_t n,
                    float *const *keys, float *const *values) {
    float *yicl = xcalloc(n * E, sizeof(float));
    target_embeddings(m, m->icl_yw, m->icl_yb, y, n, E, yicl);
    for (size_t i = 0; i < n * E; ++i) rows[i] += yicl[i];
    free(yicl);
    float *kh = keys ? NULL : xcalloc(n * E, sizeof(float));
    float *vh = values ? NULL : xcalloc(n * E, sizeof(float));
    float *next = xcalloc(t * E, sizeof(float));
    float base[E];
    int st = 0;
    for (int blk = 0; blk < ICLB && !st; ++blk) {
        float *k = keys ? keys[blk] : kh, *v = values ? values[blk] : vh;
        source_heads(m, &m->icl[blk], rows, n, 0, 1, k, v);
        qass_base(&m->icl[blk], n, base);
        attend_opts o = {base, ORA_MATH_EXACT, 0, 1};
        st = attend(m, &m->icl[blk], rows, t, k, v, n, &o, next);
        memcpy(rows, next, t * E * 4);
    }
    free(kh);
    free(vh);
    free(next);
    return st;
}

static int validate_shapes(const ora_model *m, size_t b, size_t n, size_t h, const float *y,
                           char *err, size_t errlen) {
    if (!b || !n || !h) {
        set_err(err, errlen, "context needs nonempty x[B, N, H] and y_train[B, N]");
        return -1;
    }
    if (m->task == ORA_CLASSIFIER) {
        for (size_t i = 0; i < b * n; ++i) {
            float v = y[i];
            if (!(v >= 0.0f && v <= 9.0f && v == floorf(v))) {
                set_err(err, errlen, "labels must be integers in 0..=9");
                return -1;
            }
        }
    } else {
        for (size_t i = 0; i < b * n; ++i)
            if (!isfinite(y[i])) {
                set_err(err, errlen, "regression targets must be finite");
                return -1;
            }
    }
    return 0;
}

int ora_build_context(const ora_model *m, size_t b, size_t n, size_t h, const float *x, const float *y,
                      float *const *column_keys, float *const *column_values, float *const *icl_keys,
                      float *const *icl_values, char *err, size_t errlen) {
    if (validate_shapes(m, b, n, h, y, err, errlen)) return -1;
    size_t streams = h + RES, stream_el = (size_t)M * D;
    int workers = g_threads;
    for (size_t e = 0; e < b; ++e) {
        const float *xe = x + e * n * h, *ye = y + e * n;
        float *columns = xcalloc(n * streams * D, sizeof(float));
        float *fkv[6];
        for (int i = 0; i < 6; ++i) fkv[i] = xcalloc(h * stream_el, sizeof(float));
        int st = column_embeddings(m, xe, ye, n, h, n, workers, columns, fkv);
        if (st) {
            set_err(err, errlen, st == -2 ? "a static context for an all-missing feature column"
                                          : "softmax normalization is not finite");
            for (int i = 0; i < 6; ++i) free(fkv[i]);
            free(columns);
            return -1;
        }
        for (int blk = 0; blk < COLB; ++blk) {
            float *ck = column_keys[blk] + e * streams * stream_el;
            float *cv = column_values[blk] + e * streams * stream_el;
            memset(ck, 0, RES * stream_el * 4); /* reserved streams, cpu.rs:936-938 */
            memset(cv, 0, RES * stream_el * 4);
            memcpy(ck + RES * stream_el, fkv[2 * blk], h * stream_el * 4);
            memcpy(cv + RES * stream_el, fkv[2 * blk + 1], h * stream_el * 4);
        }
        for (int i = 0; i < 6; ++i) free(fkv[i]);
        float *rows = xcalloc(n * E, sizeof(float));
        st = row_embeddings(m, columns, n, streams, workers, rows);
        free(columns);
        float *ik[ICLB], *iv[ICLB];
        for (int blk = 0; blk < ICLB; ++blk) {
            ik[blk] = icl_keys[blk] + e * HEADS * n * (E / HEADS);
            iv[blk] = icl_values[blk] + e * HEADS * n * (E / HEADS);
        }
        if (!st) st = icl_rows(m, rows, ye, n, n, ik, iv);
        free(rows);
        if (st) {
            set_err(err, errlen, "softmax normalization is not finite");
            return -1;
        }
    }
    return 0;
}

/* Spot check of one estimator's column tensors at full size: the three
 * multihead_attn2 K/V pairs [8,128,16] of the listed features, each from the
 * whole N-row column stream (column_stream + isab, cpu.rs:1132-1207) exactly
 * as ora_build_context computes them. kv[2*block] / kv[2*block+1] are
 * [nf, 8*128*16]. Features run on the oracle's threads. */
int ora_context_columns(const ora_model *m, size_t n, size_t h, const float *x, const float *y,
                        const size_t *features, size_t nf, float *const *kv, char *err, size_t errlen) {
    if (validate_shapes(m, 1, n, h, y, err, errlen)) return -1;
    for (size_t i = 0; i < nf; ++i)
        if (features[i] >= h) {
            set_err(err, errlen, "feature index out of range");
            return -1;
        }
    size_t stream_el = (size_t)M * D;
    float *ycol = xcalloc(n * D, sizeof(float));
    target_embeddings(m, m->col_yw, m->col_yb, y, n, D, ycol);
    int st = 0;
    /* Fewer features than threads: one feature at a time, its products and
     * attention on every thread (rows and heads split; each value is computed
     * as on one thread). */
    int outer = nf < (size_t)g_threads ? 1 : g_threads, inner = outer == 1 ? g_threads : 1;
#pragma omp parallel for num_threads(outer) schedule(dynamic) reduction(| : st)
    for (size_t i = 0; i < nf; ++i) {
        float *emb = xcalloc(n * D, sizeof(float));
        float *out[6];
        for (int j = 0; j < 6; ++j) out[j] = kv[j] + i * stream_el;
        st |= column_stream(m, x, ycol, n, h, n, features[i], inner, emb, out) != 0;
        free(emb);
    }
    free(ycol);
    if (st) set_err(err, errlen, "column stream failed (all-missing column or non-finite softmax)");
    return st ? -1 : 0;
}

/* Spot check of one estimator's ICL tensors at full size, by teacher forcing:
 * for each listed training row, its column embeddings against the context's
 * column K/V with its column label added (the attn2 half of isab,
 * cpu.rs:1180-1207), its row representation (cpu.rs:1226-1266), its ICL label
 * (cpu.rs:1270-1277), then per ICL block its K/V (LN1 + projections,
 * cpu.rs:1356-1416) and its attention over the context's K/V of all N
 * training rows of that block (cpu.rs:1278-1295). Each row's K/V at block b
 * thus depends on the context only through blocks < b, so every block is
 * checked against the same inputs the build used. ck/cv: [H+4,8,128,16]
 * (one estimator); ik/iv: [8,N,64]; keys/values out: 12 x [8, nr, 64].
 * Rows run on the oracle's threads, the row representation as in the build. */
int ora_context_rows(const ora_model *m, size_t n, size_t h, const float *x, const float *y,
                     const size_t *rows, size_t nr, const float *const *ck, const float *const *cv,
                     const float *const *ik, const float *const *iv, float *const *keys,
                     float *const *values, char *err, size_t errlen) {
    if (validate_shapes(m, 1, n, h, y, err, errlen)) return -1;
    for (size_t i = 0; i < nr; ++i)
        if (rows[i] >= n) {
            set_err(err, errlen, "row index out of range");
            return -1;
        }
    size_t streams = h + RES, stream_el = (size_t)M * D, hd = E / HEADS;
    float (*bases)[E] = xcalloc(ICLB, sizeof *bases);
    for (int blk = 0; blk < ICLB; ++blk) qass_base(&m->icl[blk], n, bases[blk]);
    int st = 0;
#pragma omp parallel for num_threads(g_threads) schedule(dynamic) reduction(| : st)
    for (size_t i = 0; i < nr; ++i) {
        size_t r = rows[i];
        float ycol[D], yicl[E], emb[D], next[D], row[E], rnext[E], kh[E], vh[E];
        float *columns = xcalloc(streams * D, sizeof(float));
        memcpy(columns, m->cls, RES * D * 4);
        target_embeddings(m, m->col_yw, m->col_yb, y + r, 1, D, ycol);
        target_embeddings(m, m->icl_yw, m->icl_yb, y + r, 1, E, yicl);
        int rs = 0;
        for (size_t f = 0; f < h && !rs; ++f) {
            column_input(m, x + r * h, 1, h, f, emb);
            for (size_t c = 0; c < D; ++c) emb[c] += ycol[c];
            for (int blk = 0; blk < COLB && !rs; ++blk) {
                attend_opts o2 = {NULL, ORA_MATH_EXACT, 0, 1};
                rs = attend(m, &m->col2[blk], emb, 1, ck[blk] + (RES + f) * stream_el,
                            cv[blk] + (RES + f) * stream_el, M, &o2, next);
                memcpy(emb, next, D * 4);
            }
            memcpy(columns + (RES + f) * D, emb, D * 4);
        }
        if (!rs) rs = row_embedding(m, columns, streams, row);
        free(columns);
        for (size_t c = 0; c < E; ++c) row[c] += yicl[c];
        for (int blk = 0; blk < ICLB && !rs; ++blk) {
            source_heads(m, &m->icl[blk], row, 1, 0, 1, kh, vh);
            for (size_t hh = 0; hh < HEADS; ++hh) {
                memcpy(keys[blk] + (hh * nr + i) * hd, kh + hh * hd, hd * 4);
                memcpy(values[blk] + (hh * nr + i) * hd, vh + hh * hd, hd * 4);
            }
            if (blk + 1 == ICLB) break;
            attend_opts o = {bases[blk], ORA_MATH_EXACT, 0, 1};
            rs = attend(m, &m->icl[blk], row, 1, ik[blk], iv[blk], n, &o, rnext);
            memcpy(row, rnext, E * 4);
        }
        st |= rs != 0;
    }
    free(bases);
    if (st) set_err(err, errlen, "softmax normalization is not finite");
    return st ? -1 : 0;
}

static int forward_uncached(const ora_model *m, size_t b, size_t t, size_t n, size_t h, const float *x,
                            const float *y, float *logits, float *trace_columns, float *trace_rows,
                            char *err, size_t errlen) {
    if (validate_shapes(m, b, n, h, y, err, errlen)) return -1;
    if (t < n) {
        set_err(err, errlen, "total rows are fewer than training rows");
        return -1;
    }
    size_t streams = h + RES, test = t - n;
    int workers = g_threads;
    for (size_t e = 0; e < b; ++e) {
        const float *xe = x + e * t * h, *ye = y + e * n;
        float *columns = xcalloc(t * streams * D, sizeof(float));
        int st = column_embeddings(m, xe, ye, t, h, n, workers, columns, NULL);
        float *rows = xcalloc(t * E, sizeof(float));
        if (!st) st = row_embeddings(m, columns, t, streams, workers, rows);
        if (trace_columns) memcpy(trace_columns + e * t * streams * D, columns, t * streams * D * 4);
        if (trace_rows) memcpy(trace_rows + e * t * E, rows, t * E * 4);
        free(columns);
        if (!st) st = icl_rows(m, rows, ye, t, n, NULL, NULL);
        if (!st && logits) {
            float *dec = xcalloc(t * m->width, sizeof(float));
            decoder(m, rows, t, 1, dec);
            memcpy(logits + e * test * m->width, dec + n * m->width, test * m->width * 4);
            free(dec);
        }
        free(rows);
        if (st) {
            set_err(err, errlen, "softmax normalization is not finite");
            return -1;
        }
    }
    return 0;
}

int ora_predict_uncached(const ora_model *m, size_t b, size_t t, size_t n, size_t h, const float *x,
                         const float *y, float *logits, char *err, size_t errlen) {
    return forward_uncached(m, b, t, n, h, x, y, logits, NULL, NULL, err, errlen);
}

int ora_trace_uncached(const ora_model *m, size_t b, size_t t, size_t n, size_t h, const float *x,
                       const float *y, float *columns, float *rows, char *err, size_t errlen) {
    return forward_uncached(m, b, t, n, h, x, y, NULL, columns, rows, err, errlen);
}

/* StaticExecutor::predict_estimator (cpu.rs:2259-2273) for one chunk of q rows. */
static int predict_chunk(const ora_model *m, size_t n, size_t h, size_t q, const float *x,
                         const float *const *ck, const float *const *cv, const float *const *ik,
                         const float *const *iv, const float (*bases)[E], float *logits) {
    size_t streams = h + RES, stream_el = (size_t)M * D;
    int workers = g_threads;
    float *columns = xcalloc(q * streams * D, sizeof(float));
    for (size_t r = 0; r < q; ++r) memcpy(columns + r * streams * D, m->cls, RES * D * 4);
    int st = 0;
    /* cached_column_embeddings: features on workers (cpu.rs:2388-2443). */
    int fw = workers < (int)h ? workers : (int)h;
#pragma omp parallel for num_threads(fw) schedule(static) reduction(| : st)
    for (size_t f = 0; f < h; ++f) {
        float *emb = xcalloc(q * D, sizeof(float));
        float *next = xcalloc(q * D, sizeof(float));
        column_input(m, x, q, h, f, emb);
        for (int blk = 0; blk < COLB; ++blk) {
            const float *k = ck[blk] + (RES + f) * stream_el, *v = cv[blk] + (RES + f) * stream_el;
            attend_opts o = {NULL, m->math, 0, 1};
            st |= attend(m, &m->col2[blk], emb, q, k, v, M, &o, next) != 0;
            memcpy(emb, next, q * D * 4);
        }
        for (size_t r = 0; r < q; ++r) memcpy(columns + (r * streams + RES + f) * D, emb + r * D, D * 4);
        free(emb);
        free(next);
    }
    float *rows = xcalloc(q * E, sizeof(float));
    if (!st) st = row_embeddings(m, columns, q, streams, workers, rows);
    free(columns);
    float *next = xcalloc(q * E, sizeof(float));
    for (int blk = 0; blk < ICLB && !st; ++blk) {
        attend_opts o = {bases[blk], m->math, 0, workers};
        st = attend(m, &m->icl[blk], rows, q, ik[blk], iv[blk], n, &o, next);
        memcpy(rows, next, q * E * 4);
    }
    if (!st) decoder(m, rows, q, workers, logits);
    free(rows);
    free(next);
    return st;
}

int ora_predict_cached(const ora_model *m, size_t b, size_t n, size_t h, size_t q, const float *x,
                       const float *const *column_keys, const float *const *column_values,
                       const float *const *icl_keys, const float *const *icl_values, float *logits,
                       char *err, size_t errlen) {
    if (!b || !n || !h) {
        set_err(err, errlen, "empty context shape");
        return -1;
    }
    if (!q) return 0;
    size_t streams = h + RES, stream_el = (size_t)M * D, icl_el = (size_t)n * E;
    float (*bases)[E] = xcalloc(ICLB, sizeof *bases);
    for (int blk = 0; blk < ICLB; ++blk) qass_base(&m->icl[blk], n, bases[blk]); /* cpu.rs:588-599 */
    int st = 0;
    for (size_t e = 0; e < b && !st; ++e) {
        const float *ck[COLB], *cv[COLB], *ik[ICLB], *iv[ICLB];
        for (int blk = 0; blk < COLB; ++blk) {
            ck[blk] = column_keys[blk] + e * streams * stream_el;
            cv[blk] = column_values[blk] + e * streams * stream_el;
        }
        for (int blk = 0; blk < ICLB; ++blk) {
            ik[blk] = icl_keys[blk] + e * icl_el;
            iv[blk] = icl_values[blk] + e * icl_el;
        }
        for (size_t s = 0; s < q && !st; s += CHUNK) {
            size_t len = q - s < CHUNK ? q - s : CHUNK;
            st = predict_chunk(m, n, h, len, x + (e * q + s) * h, ck, cv, ik, iv,
                               (const float(*)[E])bases, logits + (e * q + s) * m->width);
        }
    }
    free(bases);
    if (st) set_err(err, errlen, "softmax normalization is not finite");
    return st ? -1 : 0;
}

/* ------------------------------------------------------------------ */
/* Host post-processing                                                */
/* ------------------------------------------------------------------ */

static void softmax_t(float *v, size_t n, float temperature) {
    float mx = -INFINITY;
    for (size_t i = 0; i < n; ++i) if (v[i] / temperature > mx) mx = v[i] / temperature;
    float den = 0.0f;
    for (size_t i = 0; i < n; ++i) den += (v[i] = expf(v[i] / temperature - mx));
    for (size_t i = 0; i < n; ++i) v[i] /= den;
}

/* aggregate_classifier_probabilities: cpu.rs:3873-3932. */
int ora_aggregate(const float *logits, size_t b, size_t q, size_t classes, const uint64_t *perm,
                  float temperature, int average_logits, float *out) {
    if (!isfinite(temperature) || temperature <= 0.0f || classes > 10) return -1;
    float member[10];
    float scale = 1.0f / (float)b;
    memset(out, 0, q * classes * 4);
    for (size_t e = 0; e < b; ++e)
        for (size_t r = 0; r < q; ++r) {
            for (size_t c = 0; c < classes; ++c)
                member[c] = logits[(e * q + r) * classes + (size_t)perm[e * classes + c]];
            if (!average_logits) softmax_t(member, classes, temperature);
            for (size_t c = 0; c < classes; ++c) out[r * classes + c] += member[c] * scale;
        }
    for (size_t r = 0; r < q; ++r) {
        float *row = out + r * classes;
        if (average_logits) softmax_t(row, classes, temperature);
        float sum = 0.0f;
        for (size_t c = 0; c < classes; ++c) sum += row[c];
        for (size_t c = 0; c < classes; ++c) row[c] /= sum;
    }
    return 0;
}

/* f32::total_cmp: integer keys ordered -NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN. */
static unsigned total_key(float v) {
    unsigned u;
    memcpy(&u, &v, 4);
    return (u & 0x80000000u) ? ~u : u | 0x80000000u;
}
static int cmp_total(const void *a, const void *b) {
    unsigned x = total_key(*(const float *)a), y = total_key(*(const float *)b);
    return (x > y) - (x < y);
}

/* The reference's f64 arithmetic is plain Rust: no multiply-add contraction. */
#define ORA_NO_CONTRACT __attribute__((optimize("fp-contract=off")))

/* tail_slope: quantiles.rs:202-213. */
ORA_NO_CONTRACT static double tail_slope(const float *q, const double *x, size_t n) {
    double xm = 0, qm = 0;
    for (size_t i = 0; i < n; ++i) xm += x[i], qm += q[i];
    xm /= (double)n;
    qm /= (double)n;
    double cov = 0, var = 0;
    for (size_t i = 0; i < n; ++i) {
        cov += ((double)q[i] - qm) * (x[i] - xm);
        var += (x[i] - xm) * (x[i] - xm);
    }
    double v = var / (double)n;
    return (cov / (double)n) / (v > 1e-6 ? v : 1e-6);
}

/* f64::clamp of |beta| to [0.01, 100]; NaN stays NaN. */
static double clamp_beta(double beta) {
    double m = fabs(beta);
    return m != m ? m : (m < 0.01 ? 0.01 : (m > 100.0 ? 100.0 : m));
}

/* quantiles::summarize (quantiles.rs:80-213): per estimator and row, sort the
 * decoded quantiles (total order), then the mean, the unbiased variance, the
 * inverse CDF at each alpha (exponential tails fitted to the outermost
 * quantiles) and the sorted values; each averaged over B. Outputs may be null. */
ORA_NO_CONTRACT int ora_regression_outputs(const float *logits, size_t b, size_t q, size_t k, const float *alphas,
                                           size_t n_alphas, float *mean_out, float *var_out, float *quant_out,
                                           float *raw_out) {
    if (k < 2 || b < 1) return -1;
    const double TOL = 1e-6;
    double *levels = xcalloc(k, sizeof(double));
    for (size_t i = 0; i < k; ++i) levels[i] = (double)(float)((double)(i + 1) / (double)(k + 1));
    double *msum = xcalloc(q, sizeof(double)), *vsum = xcalloc(q, sizeof(double));
    double *qsum = xcalloc(q * (n_alphas ? n_alphas : 1), sizeof(double));
    double *rsum = raw_out ? xcalloc(q * k, sizeof(double)) : NULL;
    float *sorted = xcalloc(k, sizeof(float));
    size_t tk = k / 4 < 20 ? k / 4 : 20;
    if (tk < 1) tk = 1;
    double *xl = xcalloc(tk, sizeof(double)), *xr = xcalloc(tk, sizeof(double));
    for (size_t i = 0; i < tk; ++i) {
        xl[i] = log(levels[i] > TOL ? levels[i] : TOL);
        double om = 1.0 - levels[k - tk + i];
        xr[i] = log(om > TOL ? om : TOL);
    }
    for (size_t e = 0; e < b; ++e)
        for (size_t r = 0; r < q; ++r) {
            memcpy(sorted, logits + (e * q + r) * k, k * 4);
            qsort(sorted, k, sizeof(float), cmp_total);
            double m = 0;
            for (size_t i = 0; i < k; ++i) m += sorted[i];
            const double mean = m / (double)k;
            msum[r] += mean;
            double sq = 0;
            for (size_t i = 0; i < k; ++i) {
                double d = (double)sorted[i] - mean;
                sq += d * d;
            }
            vsum[r] += sq / (double)(k - 1);
            if (rsum)
                for (size_t i = 0; i < k; ++i) rsum[r * k + i] += (double)sorted[i];
            double bl = clamp_beta(tail_slope(sorted, xl, tk)), br = clamp_beta(-tail_slope(sorted + k - tk, xr, tk));
            for (size_t a = 0; a < n_alphas; ++a) {
                double alpha = alphas[a], al = levels[0], ar = levels[k - 1];
                double ql = sorted[0], qr = sorted[k - 1], v;
                if (alpha < al) {
                    v = ql + bl * (log(alpha > TOL ? alpha : TOL) - log(al > TOL ? al : TOL));
                } else if (alpha > ar) {
                    double omr = 1.0 - (ar < 1.0 - TOL ? ar : 1.0 - TOL);
                    double om = 1.0 - alpha;
                    v = qr - br * (log(om > TOL ? om : TOL) - log(omr));
                } else if (alpha >= ar) {
                    v = qr;
                } else {
                    size_t lo = 0, hi = k - 1; /* partition_point over levels[..k-1] of level <= alpha */
                    while (lo < hi) {
                        size_t mid = (lo + hi) / 2;
                        if (levels[mid] <= alpha) lo = mid + 1; else hi = mid;
                    }
                    size_t seg = lo ? lo - 1 : 0;
                    double l0 = levels[seg], l1 = levels[seg + 1];
                    double span = l1 - l0 > TOL ? l1 - l0 : TOL;
                    double t = (alpha - l0) / span;
                    t = t < 0 ? 0 : (t > 1 ? 1 : t);
                    v = (double)sorted[seg] + t * ((double)sorted[seg + 1] - (double)sorted[seg]);
                }
                qsum[r * n_alphas + a] += v;
            }
        }
    for (size_t r = 0; r < q; ++r) {
        if (mean_out) mean_out[r] = (float)(msum[r] / (double)b);
        if (var_out) var_out[r] = (float)(vsum[r] / (double)b);
        for (size_t a = 0; a < n_alphas; ++a)
            if (quant_out) quant_out[r * n_alphas + a] = (float)(qsum[r * n_alphas + a] / (double)b);
        if (rsum)
            for (size_t i = 0; i < k; ++i) raw_out[r * k + i] = (float)(rsum[r * k + i] / (double)b);
    }
    free(levels);
    free(msum);
    free(vsum);
    free(qsum);
    free(rsum);
    free(sorted);
    free(xl);
    free(xr);
    return 0;
}

int ora_regression_summary(const float *logits, size_t b, size_t q, size_t k, const float *alphas,
                           size_t n_alphas, float *mean_out, float *quant_out) {
    return ora_regression_outputs(logits, b, q, k, alphas, n_alphas, mean_out, NULL, quant_out, NULL);
}
