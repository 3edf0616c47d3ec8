// FP32 products on gfx950 matrix cores: C = epilogue(A W^T + bias).
//
// Every dense layer of the model (the role of linear64 / linear_reduce in the
// reference's CUDA backend, src/kernels/cuda/kernels.rs:290-470) runs here.
// A is [M, K] activations, W is [N, K] in PyTorch Linear layout, so both
// operands are K-contiguous.
//
// Tiling: a 256-thread workgroup (4 waves, 2 x 2) owns a BM x BN tile; each
// wave a (BM/2) x (BN/2) block of 32 x 32 v_mfma_f32_32x32x2f32 tiles. K runs
// in 16-deep steps through double-buffered LDS, one barrier per step, with
// the next step's global loads in flight during the current step's MFMAs.
// Within a 16-deep step, lanes 0-31 feed k = 0..7 and lanes 32-63 feed
// k = 8..15 (one MFMA consumes one k from each half), so every lane reads
// its eight operands as two 16-byte LDS loads; rows are padded to 20 floats
// so a half-wave's 16-byte reads hit distinct banks.
//
// Workgroups walk tiles XCD by XCD: the dispatcher sends workgroup i to XCD
// i % 8, so tile (i % 8) * per_xcd + i / 8 gives each XCD one contiguous band
// of M, whose A rows then stay in that XCD's L2 for all N tiles.
#include "common.hpp"

namespace irx {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kBK = 16;
constexpr int kLdsStride = 20;

__device__ __forceinline__ long long col_offset(const OutMap &o, int n) {
    int seg = n / o.col_seg;
    int within = n - seg * o.col_seg;
    int plane = seg / o.heads;
    int head = seg - plane * o.heads;
    return plane * o.plane_stride + head * o.head_stride + within;
}

template <int BM, int BN>
__global__ __launch_bounds__(256) void gemm_kernel(GemmArgs p, int tiles_m, int tiles_n, int per_xcd) {
    constexpr int MI = BM / 64, NI = BN / 64;
    constexpr int A_LOADS = BM / 64, B_LOADS = BN / 64;
    __shared__ __attribute__((aligned(16))) float As[2][BM * kLdsStride];
    __shared__ __attribute__((aligned(16))) float Bs[2][BN * kLdsStride];

    const int bid = blockIdx.x;
    const int tile = (bid % 8) * per_xcd + bid / 8;
    if (tile >= tiles_m * tiles_n) return;
    const int tm = tile / tiles_n, tn = tile - (tile / tiles_n) * tiles_n;
    const int m0 = tm * BM, n0 = tn * BN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int half = lane >> 5, r32 = lane & 31;

    // Global loads: thread t covers float4 (row = idx / 4, k4 = idx % 4), idx = t + 256 i.
    const float *a_src[A_LOADS];
    bool a_ok[A_LOADS];
    int a_lds[A_LOADS];
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
        int idx = tid + 256 * i, row = idx >> 2, k4 = idx & 3;
        int grow = m0 + row;
        a_ok[i] = grow < p.m;
        a_src[i] = p.a + (long long)(a_ok[i] ? grow : 0) * p.lda + k4 * 4;
        a_lds[i] = row * kLdsStride + k4 * 4;
    }
    const float *b_src[B_LOADS];
    bool b_ok[B_LOADS];
    int b_lds[B_LOADS];
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
        int idx = tid + 256 * i, row = idx >> 2, k4 = idx & 3;
        int gcol = n0 + row;
        b_ok[i] = gcol < p.n;
        b_src[i] = p.w + (long long)(b_ok[i] ? gcol : 0) * p.k + k4 * 4;
        b_lds[i] = row * kLdsStride + k4 * 4;
    }
    const f32x4 zero4 = {0.f, 0.f, 0.f, 0.f};
    f32x4 a_reg[A_LOADS], b_reg[B_LOADS];
    auto load_tile = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_LOADS; ++i)
            a_reg[i] = a_ok[i] ? *reinterpret_cast<const f32x4 *>(a_src[i] + k0) : zero4;
#pragma unroll
        for (int i = 0; i < B_LOADS; ++i)
            b_reg[i] = b_ok[i] ? *reinterpret_cast<const f32x4 *>(b_src[i] + k0) : zero4;
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

    const int ktiles = p.k / kBK;
    load_tile(0);
    store_tile(0);
    __syncthreads();
    const int a_row = (wm * (BM / 2) + r32) * kLdsStride + 8 * half;
    const int b_row = (wn * (BN / 2) + r32) * kLdsStride + 8 * half;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        const bool more = kt + 1 < ktiles;
        if (more) load_tile((kt + 1) * kBK);
        f32x4 af[MI][2], bf[NI][2];
#pragma unroll
        for (int i = 0; i < MI; ++i) {
            const float *s = &As[buf][a_row + i * 32 * kLdsStride];
            af[i][0] = *reinterpret_cast<const f32x4 *>(s);
            af[i][1] = *reinterpret_cast<const f32x4 *>(s + 4);
        }
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const float *s = &Bs[buf][b_row + j * 32 * kLdsStride];
            bf[j][0] = *reinterpret_cast<const f32x4 *>(s);
            bf[j][1] = *reinterpret_cast<const f32x4 *>(s + 4);
        }
#pragma unroll
        for (int t = 0; t < 8; ++t)
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
    const bool grouped = p.out.rows_per_group < p.m;
#pragma unroll
    for (int j = 0; j < NI; ++j) {
        const int col = n0 + wn * (BN / 2) + j * 32 + r32;
        if (col >= p.n) continue;
        const long long coff = col_offset(p.out, col);
        const float bias = p.bias ? p.bias[col] : 0.f;
#pragma unroll
        for (int i = 0; i < MI; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * (BM / 2) + i * 32 + half * 4 + (r & 3) + 8 * (r >> 2);
                if (row >= p.m) continue;
                float v = acc[i][j][r] + bias;
                if (p.epilogue & kEpiGelu) v = gelu_erf(v);
                if (p.epilogue & kEpiResidual) v += p.residual[(long long)row * p.ldr + col];
                if (p.epilogue & kEpiQass) {
                    const int head = (row / p.qass_rows) % kHeads;
                    v = p.residual[(long long)row * p.ldr + col] * p.qass_base[head * p.n + col] *
                        (1.0f + tanhf(v));
                }
                long long roff;
                if (grouped) {
                    int g = row / p.out.rows_per_group;
                    roff = g * p.out.group_stride + (long long)(row - g * p.out.rows_per_group) * p.out.ldc;
                } else {
                    roff = (long long)row * p.out.ldc;
                }
                p.c[roff + coff] = v;
            }
        }
    }
}

template <int BM, int BN>
void launch(const GemmArgs &args, hipStream_t stream) {
    int tiles_m = (int)ceil_div(args.m, BM), tiles_n = (int)ceil_div(args.n, BN);
    int tiles = tiles_m * tiles_n;
    int per_xcd = (tiles + 7) / 8;
    const double m = args.m, n = args.n, k = args.k;
    const double resid = (args.epilogue & (kEpiResidual | kEpiQass)) ? m * n : 0.0;
    KernelTimer timer(kFamGemm, stream, 2.0 * m * n * k, 4.0 * (m * k + n * k + m * n + resid));
    hipLaunchKernelGGL((gemm_kernel<BM, BN>), dim3(per_xcd * 8), dim3(256), 0, stream, args, tiles_m, tiles_n,
                       per_xcd);
    IRX_HIP(hipGetLastError());
}

}  // namespace

void gemm(const GemmArgs &args, hipStream_t stream) {
    if (args.m <= 0 || args.n <= 0) return;
    if (args.k <= 0 || args.k % kBK != 0 || args.lda % 4 != 0 ||
        (reinterpret_cast<uintptr_t>(args.a) & 15) || (reinterpret_cast<uintptr_t>(args.w) & 15))
        fail(3, "gemm: K must be a positive multiple of 16 with 16-byte aligned rows");
    if ((args.epilogue & (kEpiResidual | kEpiQass)) && !args.residual)
        fail(3, "gemm: residual epilogue without a residual");
    // Large products take 128 x 128 tiles; ones that would leave the 256 CUs
    // idle take 64 x 64.
    long long big_tiles = (long long)ceil_div(args.m, 128) * ceil_div(args.n, 128);
    if (big_tiles >= 512)
        launch<128, 128>(args, stream);
    else
        launch<64, 64>(args, stream);
}

}  // namespace irx
