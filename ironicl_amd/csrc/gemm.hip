// FP32 products on gfx950 matrix cores: C = epilogue(A W^T + bias).
//
// Every dense layer of the model (the role of linear64 / linear_reduce in the
// reference's CUDA backend, src/kernels/cuda/kernels.rs:290-470) runs here.
// A is [M, K] activations, W is [N, K] in PyTorch Linear layout, so both
// operands are K-contiguous.
//
// Two kernels, both on v_mfma_f32_32x32x2f32: tiled (BM x BN per workgroup,
// 32-deep K steps through double-buffered LDS, one barrier per step, the next
// step's global loads in flight during the MFMAs; LDS rows padded to 36
// floats so a half-wave's 16-byte reads hit distinct banks) for products with
// many tiles, and split-K (a 32 x 32 tile per workgroup, K split over its four
// waves, LDS reduction) for the small ones of a prediction pass.
//
// Workgroups walk tiles XCD by XCD: the dispatcher sends workgroup i to XCD
// i % 8, so tile (i % 8) * per_xcd + i / 8 gives each XCD one contiguous band
// of M, whose A rows then stay in that XCD's L2 for all N tiles.
#include "common.hpp"

#include <atomic>

namespace irx {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 32;
// Workgroups per CU of the 128 x 128 tiles with 32-deep K steps (73.7 KB of
// LDS) and with 16-deep ones (40 KB, 128 registers).
constexpr long long kDeepPerCu = 2, kShallowPerCu = 4;

__device__ __forceinline__ long long col_offset(const OutMap &o, int n) {
    int seg = n / o.col_seg;
    int within = n - seg * o.col_seg;
    int plane = seg / o.heads;
    int head = seg - plane * o.heads;
    return plane * o.plane_stride + head * o.head_stride + within;
}

// LayerNorm of one 128-wide row by a half-wave, lane c4 holding columns
// 4 c4 .. 4 c4 + 3 (layer_norm_f32, reference.rs:223-252: two-pass mean and
// variance, eps 1e-5), in the arithmetic of the standalone 128-wide LayerNorm.
__device__ __forceinline__ f32x4 layer_norm128_lanes(f32x4 v, const float *w, const float *b, int c4) {
    auto half_wave_sum = [](float x) {
#pragma unroll
        for (int offset = 16; offset >= 1; offset >>= 1) x += __shfl_xor(x, offset, 64);
        return x;
    };
    const float mean = half_wave_sum((v[0] + v[1]) + (v[2] + v[3])) / 128.0f;
    const f32x4 d = v - mean;
    float sq = d[0] * d[0];
    sq = fmaf(d[1], d[1], sq);
    sq = fmaf(d[2], d[2], sq);
    sq = fmaf(d[3], d[3], sq);
    const float rstd = 1.0f / sqrtf(half_wave_sum(sq) / 128.0f + 1e-5f);
    f32x4 o = d * rstd * *reinterpret_cast<const f32x4 *>(w + 4 * c4);
    if (b) o += *reinterpret_cast<const f32x4 *>(b + 4 * c4);
    return o;
}

// Epilogue of one accumulator value at (row, col): bias, then GELU or
// residual, then the output map. EPI and GROUPED are compile-time so
// each instantiation is straight-line code.
template <int EPI, bool GROUPED>
__device__ __forceinline__ void store_out(const GemmArgs &p, int row, int col, long long coff, float bias,
                                          float acc) {
    float v = acc + bias;
    if constexpr (EPI == kEpiGelu) v = gelu_erf(v);
    if constexpr (EPI == kEpiResidual) v += p.residual[(long long)row * p.ldr + col];
    long long roff;
    if constexpr (GROUPED) {
        int g = row / p.out.rows_per_group;
        roff = g * p.out.group_stride + (long long)(row - g * p.out.rows_per_group) * p.out.ldc;
    } else {
        roff = (long long)row * p.out.ldc;
    }
    p.c[roff + coff] = v;
}

// The 16 accumulator rows row0 + (r&3) + 8*(r>>2) of one column of a plain
// row-major output: one lane pointer per block, per-row offsets that are the
// same for every lane (scalar), and no row bounds checks when the tile's rows
// all exist.
template <int EPI>
__device__ __forceinline__ void store_rows(const GemmArgs &p, int row0, int col, long long coff, float bias,
                                           const f32x16 &acc, bool full_rows) {
    const long long ldc = p.out.ldc;
    float *dst = p.c + (long long)row0 * ldc + coff;
    const float *res = nullptr;
    if constexpr (EPI == kEpiResidual) res = p.residual + (long long)row0 * p.ldr + col;
    auto one = [&](int r) {
        const int dr = (r & 3) + 8 * (r >> 2);
        float v = acc[r] + bias;
        if constexpr (EPI == kEpiGelu) v = gelu_erf(v);
        if constexpr (EPI == kEpiResidual) v += res[dr * p.ldr];
        dst[dr * ldc] = v;
    };
    if (full_rows) {
        if constexpr (EPI == kEpiResidual) {
            // The residual may be the output itself (an in-place update), so
            // the compiler cannot move a residual load above an earlier store:
            // load all 16 first (each lane reads only the elements it writes),
            // or every load's latency is paid in turn.
            float rv[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) rv[r] = res[((r & 3) + 8 * (r >> 2)) * p.ldr];
#pragma unroll
            for (int r = 0; r < 16; ++r) dst[((r & 3) + 8 * (r >> 2)) * ldc] = acc[r] + bias + rv[r];
            return;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) one(r);
    } else {
#pragma unroll
        for (int r = 0; r < 16; ++r)
            if (row0 + (r & 3) + 8 * (r >> 2) < p.m) one(r);
    }
}

// Large products: a BM x BN tile per 256-thread workgroup (2 x 2 waves of
// (BM/2) x (BN/2)), K in 32-deep steps through double-buffered LDS. Within a
// step lanes 0-31 feed k = 0..15 and lanes 32-63 k = 16..31, one k from each
// half per MFMA, so a lane reads its 16 operands as four 16-byte LDS loads.
template <int BM, int BN, int EPI, bool GROUPED, int BK = kBK>
__global__ __launch_bounds__(256, BK == 16 ? 3 : 2) void gemm_kernel(GemmArgs p, int tiles_m, int tiles_n, int per_xcd) {
    constexpr int MI = BM / 64, NI = BN / 64;
    constexpr int STRIDE = BK + 4, KQ = BK / 8;  // LDS row floats; 16-byte operand loads per lane and block
    constexpr int A_LOADS = BM * BK / 4 / 256, B_LOADS = BN * BK / 4 / 256;
    __shared__ __attribute__((aligned(16))) float As[2][BM * STRIDE];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN * STRIDE];

    const int bid = blockIdx.x;
    const int tile = (bid % 8) * per_xcd + bid / 8;
    if (tile >= tiles_m * tiles_n) return;
    const int tm = tile / tiles_n, tn = tile - (tile / tiles_n) * tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, r32 = lane & 31;

    // Global loads: thread t covers float4 (row = idx / 8, k4 = idx % 8), idx = t + 256 i.
    const float *a_src[A_LOADS];
    int a_lds[A_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        int idx = tid + 256 * i, row = idx / (BK / 4), k4 = idx % (BK / 4);
        a_src[i] = p.a + (long long)min(m0 + row, p.m - 1) * p.lda + k4 * 4;
        a_lds[i] = row * STRIDE + k4 * 4;
    }
    const float *b_src[B_LOADS];
    int b_lds[B_LOADS];
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
        int idx = tid + 256 * i, row = idx / (BK / 4), k4 = idx % (BK / 4);
        b_src[i] = p.w + (long long)min(n0 + row, p.n - 1) * p.k + k4 * 4;
        b_lds[i] = row * STRIDE + k4 * 4;
    }
    f32x4 a_reg[A_LOADS], b_reg[B_LOADS];
    auto load_tile = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) a_reg[i] = *reinterpret_cast<const f32x4 *>(a_src[i] + k0);
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) b_reg[i] = *reinterpret_cast<const f32x4 *>(b_src[i] + k0);
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i) *reinterpret_cast<f32x4 *>(&As[buf][a_lds[i]]) = a_reg[i];
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i) *reinterpret_cast<f32x4 *>(&Bs[buf][b_lds[i]]) = b_reg[i];
    };

    f32x16 acc[MI][NI];
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int ktiles = p.k / BK;
    load_tile(0);
    store_tile(0);
    __syncthreads();
    const int a_row = (wm * (BM / 2) + r32) * STRIDE + (BK / 2) * half;
    const int b_row = (wn * (BN / 2) + r32) * STRIDE + (BK / 2) * half;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) load_tile((kt + 1) * BK);
        f32x4 af[MI][KQ], bf[NI][KQ];
#pragma unroll
        for (int i = 0; i < MI; ++i)
#pragma unroll
            for (int c = 0; c < KQ; ++c)
                af[i][c] = *reinterpret_cast<const f32x4 *>(&As[buf][a_row + i * 32 * STRIDE + 4 * c]);
#pragma unroll
        for (int j = 0; j < NI; ++j)
#pragma unroll
            for (int c = 0; c < KQ; ++c)
                bf[j][c] = *reinterpret_cast<const f32x4 *>(&Bs[buf][b_row + j * 32 * STRIDE + 4 * c]);
#pragma unroll
        for (int t = 0; t < 4 * KQ; ++t)
#pragma unroll
            for (int i = 0; i < MI; ++i)
#pragma unroll
                for (int j = 0; j < NI; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(af[i][t >> 2][t & 3],
                                                                     bf[j][t >> 2][t & 3], acc[i][j], 0, 0, 0);
        if (more) store_tile(buf ^ 1);
        __syncthreads();
    }

    // Epilogue. Lane (r32, half) holds column r32 and rows half*4 + (r&3) + 8*(r>>2).
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int col = n0 + wn * (BN / 2) + j * 32 + r32;
        if (col >= p.n) continue;
        const long long coff = col_offset(p.out, col);
        const float bias = p.bias ? p.bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const int row0 = m0 + wm * (BM / 2) + i * 32 + half * 4;
            if constexpr (!GROUPED) {
                store_rows<EPI>(p, row0, col, coff, bias, acc[i][j], m0 + BM <= p.m);
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = row0 + (r & 3) + 8 * (r >> 2);
                    if (row < p.m) store_out<EPI, GROUPED>(p, row, col, coff, bias, acc[i][j][r]);
                }
            }
        }
    }
}

// Small products (few output tiles): a 32 x 32 tile per workgroup whose four
// waves each take a quarter of K, reading their operands straight from L2 in
// MFMA order (one 16-deep step ahead), then reduce through LDS; each wave
// finishes four of the sixteen accumulator registers.
// LN: A's rows are LayerNormed first (K = 128), the tile's 32 rows staged in
// LDS by the workgroup's eight half-waves, and the A operands read from there.
template <int EPI, bool GROUPED, bool LN = false>
__global__ __launch_bounds__(256) void gemm_splitk_kernel(GemmArgs p, int tiles_m, int tiles_n, int per_xcd) {
    constexpr int kLnStride = 132;
    __shared__ float red[4][16][64];
    __shared__ __attribute__((aligned(16))) float xs[LN ? 32 * kLnStride : 4];
    const int bid = blockIdx.x;
    const int tile = (bid % 8) * per_xcd + bid / 8;
    if (tile >= tiles_m * tiles_n) return;
    const int tm = tile / tiles_n, tn = tile - (tile / tiles_n) * tiles_n;
    const int m0 = tm * 32, n0 = tn * 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int half = lane >> 5, r32 = lane & 31;
    const int kq = p.k / 4;
    const float *a = p.a + (long long)min(m0 + r32, p.m - 1) * p.lda + wave * kq + 8 * half;
    const float *b = p.w + (long long)min(n0 + r32, p.n - 1) * p.k + wave * kq + 8 * half;
    const int a_lds = r32 * kLnStride + wave * kq + 8 * half;
    auto load_a = [&](int off) {
        if constexpr (LN)
            return *reinterpret_cast<const f32x4 *>(&xs[a_lds + off]);
        else
            return *reinterpret_cast<const f32x4 *>(a + off);
    };

    f32x4 b0 = *reinterpret_cast<const f32x4 *>(b), b1 = *reinterpret_cast<const f32x4 *>(b + 4);
    if constexpr (LN) {
        const int hw = tid >> 5;
#pragma unroll
        for (int pass = 0; pass < 4; ++pass) {
            const int r = 8 * pass + hw;
            const f32x4 v = *reinterpret_cast<const f32x4 *>(p.a + (long long)min(m0 + r, p.m - 1) * p.lda + 4 * r32);
            *reinterpret_cast<f32x4 *>(&xs[r * kLnStride + 4 * r32]) = layer_norm128_lanes(v, p.ln_w, p.ln_b, r32);
        }
        __syncthreads();
    }
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    f32x4 a0 = load_a(0), a1 = load_a(4);
    const int steps = kq / 16;
    for (int s = 0; s < steps; ++s) {
        f32x4 na0 = a0, na1 = a1, nb0 = b0, nb1 = b1;
        if (s + 1 < steps) {
            const int off = 16 * (s + 1);
            na0 = load_a(off);
            na1 = load_a(off + 4);
            nb0 = *reinterpret_cast<const f32x4 *>(b + off);
            nb1 = *reinterpret_cast<const f32x4 *>(b + off + 4);
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a0[t], b0[t], acc, 0, 0, 0);
#pragma unroll
        for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a1[t], b1[t], acc, 0, 0, 0);
        a0 = na0, a1 = na1, b0 = nb0, b1 = nb1;
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();
    const int col = n0 + r32;
    if (col >= p.n) return;
    const long long coff = col_offset(p.out, col);
    const float bias = p.bias ? p.bias[col] : 0.f;
    // This wave finishes registers 4 wave .. 4 wave + 3: rows half*4 + rr + 8 wave.
    const int row0 = m0 + half * 4 + 8 * wave;
    f32x16 v16;
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
        const int r = wave * 4 + rr;
        v16[rr] = red[0][r][lane] + red[1][r][lane] + red[2][r][lane] + red[3][r][lane];
    }
    if constexpr (!GROUPED) {
        const long long ldc = p.out.ldc;
        float *dst = p.c + (long long)row0 * ldc + coff;
        const float *res = nullptr;
        if constexpr (EPI == kEpiResidual) res = p.residual + (long long)row0 * p.ldr + col;
        auto one = [&](int rr) {
            float v = v16[rr] + bias;
            if constexpr (EPI == kEpiGelu) v = gelu_erf(v);
            if constexpr (EPI == kEpiResidual) v += res[rr * p.ldr];
            dst[rr * ldc] = v;
        };
        if (m0 + 32 <= p.m) {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr) one(rr);
        } else {
#pragma unroll
            for (int rr = 0; rr < 4; ++rr)
                if (row0 + rr < p.m) one(rr);
        }
    } else {
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
            const int row = row0 + rr;
            if (row < p.m) store_out<EPI, GROUPED>(p, row, col, coff, bias, v16[rr]);
        }
    }
}

// Small products with K = 512 or 1,024 and a few dozen rows (the 512-wide
// out-projection and FFN down of passes of 9-64 rows): the split-K tile over
// eight waves, each taking an eighth of K with all of its operand loads
// issued before the first product, so a tile costs one memory round trip
// rather than one per 16-deep step (the four-wave kernel's 8-16 dependent
// steps). Each wave finishes two of the
// sixteen accumulator registers: rows (2w % 4) + 8 (w / 2) + 4 half + rr.
template <int EPI, bool GROUPED, int KW>  // KW: K per wave
__global__ __launch_bounds__(512) void gemm_splitk8_kernel(GemmArgs p, int tiles_m, int tiles_n, int per_xcd) {
    constexpr int S = KW / 16;
    __shared__ float red[8][16][64];
    const int bid = blockIdx.x;
    const int tile = (bid % 8) * per_xcd + bid / 8;
    if (tile >= tiles_m * tiles_n) return;
    const int tm = tile / tiles_n, tn = tile - (tile / tiles_n) * tiles_n;
    const int m0 = tm * 32, n0 = tn * 32;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int half = lane >> 5, r32 = lane & 31;
    const float *a = p.a + (long long)min(m0 + r32, p.m - 1) * p.lda + wave * KW + 8 * half;
    const float *b = p.w + (long long)min(n0 + r32, p.n - 1) * p.k + wave * KW + 8 * half;
    f32x4 av[S][2], bv[S][2];
#pragma unroll
    for (int st = 0; st < S; ++st) {
        av[st][0] = *reinterpret_cast<const f32x4 *>(a + 16 * st);
        av[st][1] = *reinterpret_cast<const f32x4 *>(a + 16 * st + 4);
        bv[st][0] = *reinterpret_cast<const f32x4 *>(b + 16 * st);
        bv[st][1] = *reinterpret_cast<const f32x4 *>(b + 16 * st + 4);
    }
    // Left to itself the compiler would sink each load down to its product.
    __builtin_amdgcn_sched_barrier(0);
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
#pragma unroll
    for (int st = 0; st < S; ++st)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int t = 0; t < 4; ++t) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av[st][h][t], bv[st][h][t], acc, 0, 0, 0);
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();
    const int col = n0 + r32;
    if (col >= p.n) return;
    const long long coff = col_offset(p.out, col);
    const float bias = p.bias ? p.bias[col] : 0.f;
    const int row0 = m0 + (2 * wave) % 4 + 8 * (wave / 2) + 4 * half;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
        const int r = 2 * wave + rr;
        float v = red[0][r][lane];
#pragma unroll
        for (int w = 1; w < 8; ++w) v += red[w][r][lane];
        if (row0 + rr < p.m) store_out<EPI, GROUPED>(p, row0 + rr, col, coff, bias, v);
    }
}

// Products of at most eight rows (passes of 1-8 rows: the ICL blocks'
// out-projection and FFN down, the decoder's last layer). A workgroup stages
// the rows in LDS once; each of its waves' four 16-lane groups takes one
// output column, lane i of a group the floats 64j + 4i .. 64j + 4i + 3 of K
// (so the group's weight loads and LDS reads are contiguous 256-byte runs),
// with every weight load of the wave in flight before the products; the
// group's 16 partial sums are reduced by shuffles and lane m writes row m.
// At one row a launch is one round trip for its weights instead of
// split-K's eight dependent steps.
// LN (K = 128): row m is LayerNormed by half-wave m as it is staged.
template <int M, int EPI, int KPL, bool LN = false>  // KPL: K / 16 floats per lane
__global__ __launch_bounds__(256) void gemm_rows_kernel(GemmArgs p) {
    constexpr int K = 16 * KPL;
    static_assert(!LN || (K == 128 && M <= 8), "the LayerNorm prologue stages at most eight 128-wide rows");
    __shared__ __attribute__((aligned(16))) float xs[M * K];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int grp = lane >> 4, i = lane & 15;
    const int col = blockIdx.x * 16 + wave * 4 + grp;
    const float *wr = p.w + (long long)min(col, p.n - 1) * K + 4 * i;
    f32x4 w[KPL / 4];
#pragma unroll
    for (int j = 0; j < KPL / 4; ++j) w[j] = *reinterpret_cast<const f32x4 *>(wr + 64 * j);
    if constexpr (LN) {
        const int m = tid >> 5, c4 = tid & 31;
        if (m < M) {
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (m < p.m)
                v = layer_norm128_lanes(*reinterpret_cast<const f32x4 *>(p.a + (long long)m * p.lda + 4 * c4),
                                        p.ln_w, p.ln_b, c4);
            *reinterpret_cast<f32x4 *>(&xs[m * K + 4 * c4]) = v;
        }
    } else {
        for (int idx = tid; idx < M * K / 4; idx += 256) {
            const int m = idx / (K / 4), k4 = idx - m * (K / 4);
            f32x4 v = {0.f, 0.f, 0.f, 0.f};
            if (m < p.m) v = *reinterpret_cast<const f32x4 *>(p.a + (long long)m * p.lda + 4 * k4);
            *reinterpret_cast<f32x4 *>(&xs[m * K + 4 * k4]) = v;
        }
    }
    __syncthreads();
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < KPL / 4; ++j) {
            const f32x4 xv = *reinterpret_cast<const f32x4 *>(&xs[m * K + 64 * j + 4 * i]);
#pragma unroll
            for (int e = 0; e < 4; ++e) a = fmaf(xv[e], w[j][e], a);
        }
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) a += __shfl_xor(a, off, 16);
        acc[m] = a;
    }
    if (col >= p.n) return;
    const long long coff = col_offset(p.out, col);
    const float bias = p.bias ? p.bias[col] : 0.f;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        if (m == i && m < p.m) {
            float v = acc[m] + bias;
            if constexpr (EPI == kEpiGelu) v = gelu_erf(v);
            if constexpr (EPI == kEpiResidual) v += p.residual[(long long)m * p.ldr + col];
            p.c[(long long)m * p.out.ldc + coff] = v;
        }
    }
}

// Compute units of the current device, looked up once per device ordinal.
int device_compute_units() {
    constexpr int kMaxDevices = 64;
    static std::atomic<int> cached[kMaxDevices] = {};
    int ordinal = 0;
    if (hipGetDevice(&ordinal) != hipSuccess || ordinal < 0 || ordinal >= kMaxDevices) {
        (void)hipGetLastError();
        return 256;
    }
    int cus = cached[ordinal].load(std::memory_order_relaxed);
    if (cus > 0) return cus;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, ordinal) != hipSuccess || cus <= 0) {
        (void)hipGetLastError();
        return 256;
    }
    cached[ordinal].store(cus, std::memory_order_relaxed);
    return cus;
}

struct Flops {
    double flops, bytes;
};

Flops work(const GemmArgs &args) {
    const double m = args.m, n = args.n, k = args.k;
    const double resid = args.epilogue == kEpiResidual ? m * n : 0.0;
    return {2.0 * m * n * k, 4.0 * (m * k + n * k + m * n + resid)};
}

// Kernel of one epilogue kind and output map.
template <template <int, bool> class K>
void dispatch_epilogue(const GemmArgs &args, dim3 grid, hipStream_t stream, int tiles_m, int tiles_n, int per_xcd,
                       int threads = 256) {
    const bool grouped = args.out.rows_per_group < args.m;
    const Flops f = work(args);
    KernelTimer timer(kFamGemm, stream, f.flops, f.bytes);
#define IRX_GEMM_CASE(E)                                                                                         \
    if (args.epilogue == E) {                                                                                    \
        if (grouped)                                                                                             \
            hipLaunchKernelGGL((K<E, true>::kernel), grid, dim3(threads), 0, stream, args, tiles_m, tiles_n, per_xcd); \
        else                                                                                                     \
            hipLaunchKernelGGL((K<E, false>::kernel), grid, dim3(threads), 0, stream, args, tiles_m, tiles_n, per_xcd); \
        IRX_HIP(hipGetLastError());                                                                              \
        return;                                                                                                  \
    }
    IRX_GEMM_CASE(kEpiNone)
    IRX_GEMM_CASE(kEpiGelu)
    IRX_GEMM_CASE(kEpiResidual)
#undef IRX_GEMM_CASE
    fail(3, "gemm: unknown epilogue");
}

template <int BM, int BN, int BK>
struct Tiled {
    template <int E, bool G>
    struct K {
        static constexpr auto kernel = gemm_kernel<BM, BN, E, G, BK>;
    };
};

template <int E, bool G>
struct SplitK {
    static constexpr auto kernel = gemm_splitk_kernel<E, G>;
};

template <int E, bool G>
struct SplitKLn {
    static constexpr auto kernel = gemm_splitk_kernel<E, G, true>;
};

// Rows up to which K = 512 and 1,024 products take the eight-wave split-K:
// passes of a few dozen rows gain (16-row pass 1.29 -> 1.27 ms), but beside
// the other stream's attention a 512-row pass's 512-thread, 150-register
// workgroups cost more than they save (the two-stream step 43.8 -> 46.5 ms).
constexpr int kSplitK8Rows = 64;

template <int KW>
struct SplitK8 {
    template <int E, bool G>
    struct K {
        static constexpr auto kernel = gemm_splitk8_kernel<E, G, KW>;
    };
};

template <int BM, int BN, int BK = kBK>
void launch(const GemmArgs &args, hipStream_t stream) {
    int tiles_m = (int)ceil_div(args.m, BM), tiles_n = (int)ceil_div(args.n, BN);
    int per_xcd = (tiles_m * tiles_n + 7) / 8;
    dispatch_epilogue<Tiled<BM, BN, BK>::template K>(args, dim3(per_xcd * 8), stream, tiles_m, tiles_n, per_xcd);
}

// gemm_rows_kernel for m <= 8 rows and K = 128, 256, 512 or 1,024 (plain
// epilogues, ungrouped rows); false when the shape is not one of those.
bool launch_rows(const GemmArgs &args, hipStream_t stream) {
    if (args.m > 8 || args.out.rows_per_group < args.m) return false;
    const int m = args.m <= 1 ? 1 : args.m <= 2 ? 2 : args.m <= 4 ? 4 : 8;
    const dim3 grid(ceil_div(args.n, 16)), block(256);
    bool launched = false;
    auto go = [&]<int M, int KPL>() {
        if (m != M || args.k != 16 * KPL) return;
        const Flops f = work(args);
        KernelTimer timer(kFamGemm, stream, f.flops, f.bytes);
        if constexpr (KPL == 8) {
            if (args.ln_w) {
                if (args.epilogue == kEpiNone)
                    hipLaunchKernelGGL((gemm_rows_kernel<M, kEpiNone, 8, true>), grid, block, 0, stream, args);
                else if (args.epilogue == kEpiGelu)
                    hipLaunchKernelGGL((gemm_rows_kernel<M, kEpiGelu, 8, true>), grid, block, 0, stream, args);
                else
                    hipLaunchKernelGGL((gemm_rows_kernel<M, kEpiResidual, 8, true>), grid, block, 0, stream, args);
                IRX_HIP(hipGetLastError());
                launched = true;
                return;
            }
        }
        if (args.epilogue == kEpiNone)
            hipLaunchKernelGGL((gemm_rows_kernel<M, kEpiNone, KPL>), grid, block, 0, stream, args);
        else if (args.epilogue == kEpiGelu)
            hipLaunchKernelGGL((gemm_rows_kernel<M, kEpiGelu, KPL>), grid, block, 0, stream, args);
        else
            hipLaunchKernelGGL((gemm_rows_kernel<M, kEpiResidual, KPL>), grid, block, 0, stream, args);
        IRX_HIP(hipGetLastError());
        launched = true;
    };
    auto each_k = [&]<int M>() {
        go.template operator()<M, 8>();
        go.template operator()<M, 16>();
        go.template operator()<M, 32>();
        go.template operator()<M, 64>();
    };
    each_k.template operator()<1>();
    each_k.template operator()<2>();
    each_k.template operator()<4>();
    each_k.template operator()<8>();
    return launched;
}

void launch_splitk(const GemmArgs &args, hipStream_t stream) {
    int tiles_m = (int)ceil_div(args.m, 32), tiles_n = (int)ceil_div(args.n, 32);
    int per_xcd = (tiles_m * tiles_n + 7) / 8;
    if (args.ln_w)
        dispatch_epilogue<SplitKLn>(args, dim3(per_xcd * 8), stream, tiles_m, tiles_n, per_xcd);
    else if (args.m <= kSplitK8Rows && args.k == 512)
        dispatch_epilogue<SplitK8<64>::template K>(args, dim3(per_xcd * 8), stream, tiles_m, tiles_n, per_xcd, 512);
    else if (args.m <= kSplitK8Rows && args.k == 1024)
        dispatch_epilogue<SplitK8<128>::template K>(args, dim3(per_xcd * 8), stream, tiles_m, tiles_n, per_xcd, 512);
    else
        dispatch_epilogue<SplitK>(args, dim3(per_xcd * 8), stream, tiles_m, tiles_n, per_xcd);
}

// Products with fewer than 256 tiles of 64 x 64 take split-K or, at up to
// eight rows, the small-row kernel.
bool small_product(long long m, long long n) { return ceil_div(m, 64) * ceil_div(n, 64) < 256; }

}  // namespace

bool gemm_fuses_ln(long long m, int n) { return m > 0 && n > 0 && small_product(m, n); }

void gemm(const GemmArgs &args, hipStream_t stream) {
    if (args.m <= 0 || args.n <= 0) return;
    if (args.ln_w && (args.k != 128 || !gemm_fuses_ln(args.m, args.n) || args.out.rows_per_group < args.m ||
                      (reinterpret_cast<uintptr_t>(args.ln_w) & 15) ||
                      (reinterpret_cast<uintptr_t>(args.ln_b) & 15)))
        fail(3, "gemm: a LayerNorm prologue needs K = 128, a small product and plain rows");
    if (args.k <= 0 || args.k % 64 != 0 || args.lda % 4 != 0 ||
        (reinterpret_cast<uintptr_t>(args.a) & 15) || (reinterpret_cast<uintptr_t>(args.w) & 15))
        fail(3, "gemm: K must be a positive multiple of 64 with 16-byte aligned rows");
    if (args.epilogue == kEpiResidual && !args.residual)
        fail(3, "gemm: residual epilogue without a residual");
    // Products with few 64 x 64 tiles split K over a workgroup's waves; those
    // with four or more 128 x 128 tiles per CU take them (GELU ones, whose
    // epilogue is long, from two per CU), the rest 64 x 64 (measured on the
    // prediction pass's products).
    const long long big_tiles = (long long)ceil_div(args.m, 128) * ceil_div(args.n, 128);
    if (small_product(args.m, args.n)) {
        if (!launch_rows(args, stream)) launch_splitk(args, stream);
    } else if (big_tiles >= 1024 || (args.epilogue == kEpiGelu && big_tiles >= 512)) {
        // 128 x 128 tiles: 16-deep K steps (40 KB of LDS, 128 registers: four
        // workgroups per CU) when there are at least two such rounds of
        // tiles, else 32-deep steps at two per CU (the 50,000-row build's
        // products: N = 1,024 and 1,536 take the first, N = 512 the second,
        // whose 1,564 tiles are 1.5 rounds of four per CU). When the last
        // round would be mostly empty (at N = 512: 3.05 rounds of two per CU)
        // the whole rounds take the first rows and the rows left over run as
        // 64 x 64 tiles, a quarter of the work each, spread over the chip.
        const long long cus = device_compute_units();
        const bool deep = big_tiles < 2 * kShallowPerCu * cus;
        const long long slots = (deep ? kDeepPerCu : kShallowPerCu) * cus;
        const long long tiles_n = ceil_div(args.n, 128);
        const long long main_tm = big_tiles / slots * slots / tiles_n;
        const bool plain_rows = args.out.rows_per_group >= args.m;
        auto big = [&](const GemmArgs &a) {
            if (deep)
                launch<128, 128, 32>(a, stream);
            else
                launch<128, 128, 16>(a, stream);
        };
        if (plain_rows && big_tiles % slots < slots / 2 && main_tm > 0 && main_tm * 128 < args.m) {
            GemmArgs head = args, rest = args;
            const long long rows = main_tm * 128;
            head.m = (int)rows;
            rest.m = args.m - (int)rows;
            rest.a = args.a + rows * args.lda;
            rest.c = args.c + rows * args.out.ldc;
            if (args.residual) rest.residual = args.residual + rows * args.ldr;
            big(head);
            launch<64, 64>(rest, stream);
        } else {
            big(args);
        }
    } else {
        launch<64, 64>(args, stream);
    }
}

}  // namespace irx
