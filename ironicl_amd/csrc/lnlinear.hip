// LayerNorm fused into the product that reads it, for 512-wide rows.
//
// y = epilogue(LN(x) W^T + b) over x [m, 512], with the LayerNorm of cpu.rs's
// blocks (two-pass mean and variance, eps 1e-5, reference.rs:223-252) taken
// in the product's prologue, and two epilogues:
//   kLnGelu  gelu(y) into a row-major [m, n] output (LN2 + the FFN's first
//            layer, cpu.rs:1585-1595; the decoder's, cpu.rs:2543-2580);
//   kLnQass  the ICL query path, one 64-wide head per workgroup (n = 512):
//            q = y, then the QASS query MLP per head, h = gelu(q Wm0^T + bm0),
//            g = h Wm2^T + bm2, and the gate q * base[head] * (1 + tanh(g)),
//            stored head-major [b, 8, rows, 64] (StaticExecutor::qass,
//            cpu.rs:3798-3853; qassmax_f32, reference.rs:417-428).
// It replaces, per ICL block of a prediction pass, LayerNorm + Q projection +
// two QASS products (four launches), and LayerNorm + FFN up (two launches).
// Passes of at most eight rows take ln_rows512_kernel instead.
//
// A workgroup of four waves computes 16 rows x 64 columns; wave w reduces over
// K = 128 w .. 128 w + 127 on v_mfma_f32_16x16x4f32 with the product
// transposed (D = W x^T: lane (m, g) = (lane % 16, lane / 16) holds row m's
// columns 16 b + 4 g + r in register r of block b). Each wave loads its rows'
// quarter of x in that layout, the row statistics are summed over the four
// waves through LDS, and the partial products are summed there too.
#include "common.hpp"

#include <algorithm>

namespace irx {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kRows = 16;

__device__ __forceinline__ f32x4 mfma(float a, float b, const f32x4 &acc) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, acc, 0, 0, 0);
}

// Sum of a[0..W-1] as a pairwise tree ((a0 + a1) + (a2 + a3)) + ...
template <int W, typename F>
__device__ __forceinline__ auto tree_sum(F a) {
    if constexpr (W == 4)
        return (a(0) + a(1)) + (a(2) + a(3));
    else
        return ((a(0) + a(1)) + (a(2) + a(3))) + ((a(4) + a(5)) + (a(6) + a(7)));
}

// OB: 16-column output blocks per workgroup (4, or 2 for the GELU form of
// passes of at most 32 rows, which then spread over twice the workgroups).
// W: waves, each taking 512 / W of K (8 for the QASS form of passes of at
// most 32 rows: half the products and weight loads per wave; waves 4-7 then
// only pass the barriers of the epilogue).
template <int EPI, int OB = 4, int W = 4>
__global__ __launch_bounds__(64 * W) void ln_linear512_kernel(LnLinear p) {
    static_assert(OB == 4 || (OB == 2 && EPI == kLnGelu), "QASS needs a whole 64-wide head per workgroup");
    static_assert(W == 4 || W == 8, "four or eight waves");
    constexpr int KB = 32 / W;  // 16-wide k-blocks per wave
    __shared__ float red[2][W][kRows];
    __shared__ __attribute__((aligned(16))) float part[W][kRows][68];
    __shared__ __attribute__((aligned(16))) float tile[2][kRows][68];  // QASS: q, then the hidden layer
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int m16 = lane & 15, g = lane >> 4;
    const long long row0 = (long long)blockIdx.x * kRows;
    const int col0 = 16 * OB * blockIdx.y;
    const long long row = row0 + m16;
    const long long r = row < p.m ? row : p.m - 1;
    const int k0 = 16 * KB * w;

    // x[row][k0 + 16 kb + 4 g + e], and every weight fragment of this wave's
    // quarter up front (columns col0 + 16 ob + lane % 16): the loads' latency
    // is paid once, under the LayerNorm.
    f32x4 x[KB], wf[KB][OB];
    const float *xr = p.x + r * p.ldx + k0 + 4 * g;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) x[kb] = *reinterpret_cast<const f32x4 *>(xr + 16 * kb);
    const float *wr = p.w + (long long)(col0 + m16) * 512 + k0 + 4 * g;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int ob = 0; ob < OB; ++ob) wf[kb][ob] = *reinterpret_cast<const f32x4 *>(wr + ob * 16 * 512 + 16 * kb);
    float s = 0.f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) s += (x[kb][0] + x[kb][1]) + (x[kb][2] + x[kb][3]);
    s += __shfl_xor(s, 16, 64);
    s += __shfl_xor(s, 32, 64);
    if (g == 0) red[0][w][m16] = s;
    __syncthreads();
    const float mean = tree_sum<W>([&](int i) { return red[0][i][m16]; }) / 512.f;
    float sq = 0.f;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float d = x[kb][e] - mean;
            sq = fmaf(d, d, sq);
        }
    sq += __shfl_xor(sq, 16, 64);
    sq += __shfl_xor(sq, 32, 64);
    if (g == 0) red[1][w][m16] = sq;
    __syncthreads();
    const float var = tree_sum<W>([&](int i) { return red[1][i][m16]; }) / 512.f;
    const float rstd = 1.0f / sqrtf(var + 1e-5f);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
        const f32x4 lw = *reinterpret_cast<const f32x4 *>(p.lnw + k0 + 16 * kb + 4 * g);
        const f32x4 lb = *reinterpret_cast<const f32x4 *>(p.lnb + k0 + 16 * kb + 4 * g);
#pragma unroll
        for (int e = 0; e < 4; ++e) x[kb][e] = (x[kb][e] - mean) * rstd * lw[e] + lb[e];
    }

    // This wave's quarter of the product: columns col0 + 16 ob + n, n = lane % 16.
    f32x4 acc[OB];
#pragma unroll
    for (int ob = 0; ob < OB; ++ob) acc[ob] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
            for (int ob = 0; ob < OB; ++ob) acc[ob] = mfma(wf[kb][ob][e], x[kb][e], acc[ob]);
#pragma unroll
    for (int ob = 0; ob < OB; ++ob)
        *reinterpret_cast<f32x4 *>(&part[w][m16][16 * ob + 4 * g]) = acc[ob];
    __syncthreads();

    // Threads 0-255 finish row t / 16, columns 4 (t % 16) .. +3.
    const int om = (tid >> 4) & (kRows - 1), oc = 4 * (tid & 15);
    const bool finisher = tid < 16 * kRows;
    const long long orow = row0 + om;
    if (oc >= 16 * OB) return;  // OB = 2: only the GELU form, which has no barrier after this
    f32x4 v = tree_sum<W>([&](int i) { return *reinterpret_cast<const f32x4 *>(&part[i][om][oc]); });
    v += *reinterpret_cast<const f32x4 *>(p.b + col0 + oc);
    if constexpr (EPI == kLnGelu) {
        if (finisher && orow < p.m) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = gelu_erf(v[e]);
            *reinterpret_cast<f32x4 *>(p.out + orow * p.ldo + col0 + oc) = v;
        }
    } else {
        // The head's query tile, then its MLP: wave w < 4 computes columns
        // 16 w .. 16 w + 15 of each layer from the whole previous tile (with
        // eight waves, waves 4-7 only pass the barriers).
        const bool mlp = w < 4;
        const int wq = w & 3;
        f32x4 mw[2][4];
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            mw[0][kb] = *reinterpret_cast<const f32x4 *>(p.qm0w + (16 * wq + m16) * 64 + 16 * kb + 4 * g);
            mw[1][kb] = *reinterpret_cast<const f32x4 *>(p.qm2w + (16 * wq + m16) * 64 + 16 * kb + 4 * g);
        }
        if (finisher) *reinterpret_cast<f32x4 *>(&tile[0][om][oc]) = v;
        __syncthreads();
        auto layer = [&](const f32x4 *wt, const float *bias, int src) {
            f32x4 a = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kb = 0; kb < 4; ++kb) {
                const f32x4 xf = *reinterpret_cast<const f32x4 *>(&tile[src][m16][16 * kb + 4 * g]);
#pragma unroll
                for (int e = 0; e < 4; ++e) a = mfma(wt[kb][e], xf[e], a);
            }
            return a + *reinterpret_cast<const f32x4 *>(bias + 16 * wq + 4 * g);
        };
        if (mlp) {
            f32x4 h = layer(mw[0], p.qm0b, 0);
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = gelu_erf(h[e]);
            *reinterpret_cast<f32x4 *>(&tile[1][m16][16 * wq + 4 * g]) = h;
        }
        __syncthreads();
        if (mlp && row < p.m) {
            const f32x4 gm = layer(mw[1], p.qm2b, 1);
            const int head = blockIdx.y, col = 16 * wq + 4 * g;
            const f32x4 q = *reinterpret_cast<const f32x4 *>(&tile[0][m16][col]);
            const f32x4 base = *reinterpret_cast<const f32x4 *>(p.base + head * 64 + col);
            f32x4 o;
#pragma unroll
            for (int e = 0; e < 4; ++e) o[e] = q[e] * base[e] * (1.0f + tanhf(gm[e]));
            const long long b = row / p.rows, rr = row - b * p.rows;
            *reinterpret_cast<f32x4 *>(p.out + (((b * kHeads + head) * p.rows + rr) * 64) + col) = o;
        }
    }
}

// Passes of at most eight rows (M = 1, 2, 4 or 8 after rounding up). The
// 16-row MFMA tiles above would spend 128 serial MFMAs per wave on one or two
// real rows; here every weight load is issued first, the rows' LayerNorms
// are taken under those loads (row r by wave r % waves, two-pass statistics
// over a wave's 64 lanes) and staged in LDS, and each 16-lane group owns one
// output column: lane i multiplies K floats 64 j + 4 i .. 64 j + 4 i + 3 and
// the group's partial sums are reduced by shuffles. kLnGelu: 16 columns per
// 256-thread workgroup, lane m of a group writes row m. kLnQass: a
// 1,024-thread workgroup per head, whose 64 groups then take the head's
// query MLP the same way (one column of h, then of g, per group, K = 64 over
// the group's lanes) through LDS.
template <int M, int EPI>
__global__ __launch_bounds__(EPI == kLnQass ? 1024 : 256) void ln_rows512_kernel(LnLinear p) {
    constexpr int kThreads = EPI == kLnQass ? 1024 : 256, kCols = kThreads / 16, kWaves = kThreads / 64;
    __shared__ __attribute__((aligned(16))) float xs[M * 512];
    __shared__ __attribute__((aligned(16))) float qh[EPI == kLnQass ? 2 : 1][M][64];  // QASS: q, then h
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int i = lane & 15, c = tid >> 4;
    const int col = blockIdx.x * kCols + c;

    const float *wr = p.w + (long long)min(col, p.n - 1) * 512 + 4 * i;
    f32x4 w[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) w[j] = *reinterpret_cast<const f32x4 *>(wr + 64 * j);
    f32x4 m0w, m2w;
    if constexpr (EPI == kLnQass) {
        m0w = *reinterpret_cast<const f32x4 *>(p.qm0w + c * 64 + 4 * i);
        m2w = *reinterpret_cast<const f32x4 *>(p.qm2w + c * 64 + 4 * i);
    }

    for (int r = wave; r < M; r += kWaves) {
        f32x4 *dst = reinterpret_cast<f32x4 *>(&xs[r * 512]);
        if (r >= p.m) {
            dst[lane] = f32x4{0.f, 0.f, 0.f, 0.f};
            dst[64 + lane] = f32x4{0.f, 0.f, 0.f, 0.f};
            continue;
        }
        const float *xr = p.x + (long long)r * p.ldx;
        f32x4 v[2] = {*reinterpret_cast<const f32x4 *>(xr + 4 * lane),
                      *reinterpret_cast<const f32x4 *>(xr + 256 + 4 * lane)};
        float s = ((v[0][0] + v[0][1]) + (v[0][2] + v[0][3])) + ((v[1][0] + v[1][1]) + (v[1][2] + v[1][3]));
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) s += __shfl_xor(s, off, 64);
        const float mean = s / 512.f;
        float sq = 0.f;
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float d = v[h][e] - mean;
                sq = fmaf(d, d, sq);
            }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) sq += __shfl_xor(sq, off, 64);
        const float rstd = 1.0f / sqrtf(sq / 512.f + 1e-5f);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const f32x4 lw = *reinterpret_cast<const f32x4 *>(p.lnw + 256 * h + 4 * lane);
            const f32x4 lb = *reinterpret_cast<const f32x4 *>(p.lnb + 256 * h + 4 * lane);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[h][e] = (v[h][e] - mean) * rstd * lw[e] + lb[e];
            dst[64 * h + lane] = v[h];
        }
    }
    __syncthreads();

    // acc[m]: row m of this group's column, identical in all 16 lanes.
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float a = 0.f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const f32x4 xv = *reinterpret_cast<const f32x4 *>(&xs[m * 512 + 64 * j + 4 * i]);
#pragma unroll
            for (int e = 0; e < 4; ++e) a = fmaf(xv[e], w[j][e], a);
        }
#pragma unroll
        for (int off = 8; off >= 1; off >>= 1) a += __shfl_xor(a, off, 16);
        acc[m] = a;
    }
    if constexpr (EPI == kLnGelu) {
        if (col >= p.n) return;
        const float bias = p.b[col];
#pragma unroll
        for (int m = 0; m < M; ++m)
            if (m == i && m < p.m) p.out[(long long)m * p.ldo + col] = gelu_erf(acc[m] + bias);
    } else {
        // One head per workgroup (n = 512): column c of the head is col.
        const int head = blockIdx.x;
        const float bias = p.b[col];
#pragma unroll
        for (int m = 0; m < M; ++m)
            if (m == i) qh[0][m][c] = acc[m] + bias;
        __syncthreads();
        auto mlp = [&](const f32x4 &wt, int src, int m) {
            const f32x4 xv = *reinterpret_cast<const f32x4 *>(&qh[src][m][4 * i]);
            float a = 0.f;
#pragma unroll
            for (int e = 0; e < 4; ++e) a = fmaf(xv[e], wt[e], a);
#pragma unroll
            for (int off = 8; off >= 1; off >>= 1) a += __shfl_xor(a, off, 16);
            return a;
        };
        float hv[M];
#pragma unroll
        for (int m = 0; m < M; ++m) hv[m] = gelu_erf(mlp(m0w, 0, m) + p.qm0b[c]);
#pragma unroll
        for (int m = 0; m < M; ++m)
            if (m == i) qh[1][m][c] = hv[m];
        __syncthreads();
        const float base = p.base[head * 64 + c];
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const float g = mlp(m2w, 1, m) + p.qm2b[c];
            if (m == i && m < p.m) {
                const int b = m / p.rows, rr = m - b * p.rows;
                p.out[(((long long)b * kHeads + head) * p.rows + rr) * 64 + c] = qh[0][m][c] * base * (1.0f + tanhf(g));
            }
        }
    }
}

// The QASS query MLP and gate over head-major query rows that are already
// projected (the build's N-row queries, whose Q projection is a tiled
// product): out = q * base[head] * (1 + tanh(gelu(q Wm0^T + bm0) Wm2^T +
// bm2)). Each wave holds both 64 x 64 weights in its registers as A-operand
// fragments (w[ob][kb] = W[16 ob + m][16 kb + 4 g .. +3]) and takes a
// contiguous share of the 16-row tasks, loading the next task's rows while
// it computes one. Rows are the B operand in the layout of the kLnQass
// epilogue above (lane (m, g) holds row m's columns 16 b + 4 g + r in
// register r of block b), which is also the layout the products return, so
// the hidden layer goes from the first product to the second in registers.
// Every output takes its sixteen products in that epilogue's order, then
// the same bias, GELU, tanh and gate arithmetic: the two paths agree bit for
// bit on the same queries.
__global__ __launch_bounds__(256, 2) void qass_rows_kernel(QassRows p, long long tasks) {
    const int lane = threadIdx.x & 63, m16 = lane & 15, g = lane >> 4;
    const long long waves = (long long)gridDim.x * 4;
    const long long wave = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    const long long t_begin = wave * tasks / waves, t_end = (wave + 1) * tasks / waves;
    if (t_begin >= t_end) return;

    f32x4 w0[4][4], w2[4][4];
#pragma unroll
    for (int ob = 0; ob < 4; ++ob)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) {
            w0[ob][kb] = *reinterpret_cast<const f32x4 *>(p.w0 + (16 * ob + m16) * 64 + 16 * kb + 4 * g);
            w2[ob][kb] = *reinterpret_cast<const f32x4 *>(p.w2 + (16 * ob + m16) * 64 + 16 * kb + 4 * g);
        }
    auto load = [&](long long t, f32x4 *x) {
        const long long row = min(16 * t + m16, p.m - 1);
        const float *src = p.q + row * 64 + 4 * g;
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) x[kb] = *reinterpret_cast<const f32x4 *>(src + 16 * kb);
    };
    f32x4 x[4], xn[4];
    load(t_begin, x);
    for (long long t = t_begin; t < t_end; ++t) {
        if (t + 1 < t_end) load(t + 1, xn);
        // Four independent accumulators, each summed over (kb, e) in order.
        f32x4 h[4];
#pragma unroll
        for (int ob = 0; ob < 4; ++ob) h[ob] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int ob = 0; ob < 4; ++ob) h[ob] = mfma(w0[ob][kb][e], x[kb][e], h[ob]);
#pragma unroll
        for (int ob = 0; ob < 4; ++ob) {
            h[ob] += *reinterpret_cast<const f32x4 *>(p.b0 + 16 * ob + 4 * g);
#pragma unroll
            for (int e = 0; e < 4; ++e) h[ob][e] = gelu_erf(h[ob][e]);
        }
        f32x4 a[4];
#pragma unroll
        for (int ob = 0; ob < 4; ++ob) a[ob] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
            for (int e = 0; e < 4; ++e)
#pragma unroll
                for (int ob = 0; ob < 4; ++ob) a[ob] = mfma(w2[ob][kb][e], h[kb][e], a[ob]);
        const long long row = 16 * t + m16;
        const int head = (int)((row / p.rows) % kHeads);
        if (row < p.m) {
            float *dst = p.out + row * 64 + 4 * g;
#pragma unroll
            for (int ob = 0; ob < 4; ++ob) {
                const f32x4 gm = a[ob] + *reinterpret_cast<const f32x4 *>(p.b2 + 16 * ob + 4 * g);
                const f32x4 base = *reinterpret_cast<const f32x4 *>(p.base + head * 64 + 16 * ob + 4 * g);
                f32x4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) o[e] = x[ob][e] * base[e] * (1.0f + tanhf(gm[e]));
                *reinterpret_cast<f32x4 *>(dst + 16 * ob) = o;
            }
        }
#pragma unroll
        for (int kb = 0; kb < 4; ++kb) x[kb] = xn[kb];
    }
}

template <int EPI>
void launch_rows(const LnLinear &a, hipStream_t stream) {
    const dim3 grid(EPI == kLnQass ? kHeads : a.n / 16), block(EPI == kLnQass ? 1024 : 256);
    if (a.m <= 1)
        hipLaunchKernelGGL((ln_rows512_kernel<1, EPI>), grid, block, 0, stream, a);
    else if (a.m <= 2)
        hipLaunchKernelGGL((ln_rows512_kernel<2, EPI>), grid, block, 0, stream, a);
    else if (a.m <= 4)
        hipLaunchKernelGGL((ln_rows512_kernel<4, EPI>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((ln_rows512_kernel<8, EPI>), grid, block, 0, stream, a);
}

}  // namespace

void ln_linear512(const LnLinear &a, int epilogue, hipStream_t stream) {
    if (a.m <= 0) return;
    if (a.n <= 0 || a.n % 64 || (epilogue == kLnQass && (a.n != 512 || a.rows <= 0)) ||
        (epilogue != kLnQass && epilogue != kLnGelu))
        fail(3, "ln_linear512: unsupported shape");
    if ((a.ldx & 3) || (a.ldo & 3) || (reinterpret_cast<uintptr_t>(a.x) & 15) ||
        (reinterpret_cast<uintptr_t>(a.w) & 15) || (reinterpret_cast<uintptr_t>(a.out) & 15))
        fail(3, "ln_linear512: rows must be 16-byte aligned");
    const double m = a.m, n = a.n;
    const double flops = 2.0 * m * n * 512 + (epilogue == kLnQass ? 2.0 * 2.0 * m * 8 * 64 * 64 : 0.0);
    KernelTimer timer(kFamGemm, stream, flops, 4.0 * (m * 512 + n * 512 + m * n));
    const dim3 grid((unsigned)ceil_div((size_t)a.m, kRows), (unsigned)(a.n / 64));
    if (a.m <= 8) {
        if (epilogue == kLnQass)
            launch_rows<kLnQass>(a, stream);
        else
            launch_rows<kLnGelu>(a, stream);
    } else if (epilogue == kLnQass && a.m <= 32) {
        hipLaunchKernelGGL((ln_linear512_kernel<kLnQass, 4, 8>), grid, dim3(512), 0, stream, a);
    } else if (epilogue == kLnQass) {
        hipLaunchKernelGGL(ln_linear512_kernel<kLnQass>, grid, dim3(256), 0, stream, a);
    } else if (a.m <= 32) {
        const dim3 narrow((unsigned)ceil_div((size_t)a.m, kRows), (unsigned)(a.n / 32));
        hipLaunchKernelGGL((ln_linear512_kernel<kLnGelu, 2>), narrow, dim3(256), 0, stream, a);
    } else {
        hipLaunchKernelGGL(ln_linear512_kernel<kLnGelu>, grid, dim3(256), 0, stream, a);
    }
    IRX_HIP(hipGetLastError());
}

void qass_rows(const QassRows &a, hipStream_t stream) {
    if (a.m <= 0) return;
    if (a.rows <= 0) fail(3, "qass_rows: rows per head must be positive");
    if ((reinterpret_cast<uintptr_t>(a.q) & 15) || (reinterpret_cast<uintptr_t>(a.out) & 15) ||
        (reinterpret_cast<uintptr_t>(a.w0) & 15) || (reinterpret_cast<uintptr_t>(a.w2) & 15) ||
        (reinterpret_cast<uintptr_t>(a.b0) & 15) || (reinterpret_cast<uintptr_t>(a.b2) & 15) ||
        (reinterpret_cast<uintptr_t>(a.base) & 15))
        fail(3, "qass_rows: operands must be 16-byte aligned");
    const long long tasks = (long long)ceil_div((size_t)a.m, 16);
    // Two workgroups of four waves per CU, each wave a contiguous share of the tasks.
    const long long groups = std::min<long long>(ceil_div((size_t)tasks, 4), 2LL * std::max(1, a.compute_units));
    const double m = (double)a.m;
    KernelTimer timer(kFamGemm, stream, 2.0 * 2.0 * m * 64 * 64, 4.0 * (2.0 * m * 64 + 2.0 * 64 * 64));
    hipLaunchKernelGGL(qass_rows_kernel, dim3((unsigned)groups), dim3(256), 0, stream, a, tasks);
    IRX_HIP(hipGetLastError());
}

}  // namespace irx
