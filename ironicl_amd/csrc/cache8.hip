// The FP8 ICL cache of optimize="fast" (IRX_PRECISION_HALF): E4M3 keys and
// values with one scale per (pair, dim).
//
// The reference encodes each block's FP16 keys and values on the device
// (fp8_peaks / fp8_scales / fp8_encode, src/kernels/cuda/kernels.rs:795-875;
// encode_fp8 in cuda/cache.rs): the scale of a (pair, dim) maps its largest
// magnitude over the rows to E4M3's largest, 448 (1 when all are zero), and a
// value is stored as e4m3(value / scale), rounded to the nearest (ties to
// even) and saturated at +-448 (src/kernels/cuda/ops/fp8.rs:30-62). Here:
//   icl8_peaks_kernel   max |value| per (pair, dim), one workgroup per
//                       (256-row chunk, pair), folded into the block's peak
//                       words with atomicMax on the non-negative float bits;
//                       counts values that are not finite;
//   icl8_encode_kernel  one workgroup per (pair, 64-key tile): K rows as
//                       [pairs, Np, 64] bytes, V^T tiles [pairs, Np / 64, 64
//                       dims, 64 keys] in the FP16 cache's stored key order
//                       (0..3, 8..11, 4..7, 12..15 in each group of 16), zero
//                       past the rows; the first tile also writes the scales.
#include "common.hpp"

namespace irx {
namespace {

typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float half_bits_to_float(unsigned short h) { return (float)__builtin_bit_cast(_Float16, h); }

// E4M3 (OCP: bias 7, no infinities, 0x7f NaN) of x, nearest even, saturated at +-448.
__device__ __forceinline__ unsigned e4m3(float x) {
    const unsigned sign = (__float_as_uint(x) >> 24) & 0x80u;
    const float mag = fminf(fabsf(x), 448.0f);
    if (mag < 0.015625f) {
        // Below 2^-6 the representable values are the multiples of 2^-9:
        // adding and removing 2^23 rounds mag * 512 to the nearest even integer.
        const float steps = (mag * 512.0f + 8388608.0f) - 8388608.0f;
        return sign | (unsigned)steps;
    }
    const unsigned bits = __float_as_uint(mag);
    int exponent = (int)((bits >> 23) & 0xffu) - 127;
    unsigned mantissa = (bits >> 20) & 7u;
    const unsigned rest = bits & 0xfffffu;
    if (rest > 0x80000u || (rest == 0x80000u && (mantissa & 1u))) ++mantissa;
    if (mantissa == 8u) mantissa = 0u, ++exponent;
    // 448 is exponent 8, mantissa 6; exponent 8 with mantissa 7 is NaN.
    if (exponent > 8 || (exponent == 8 && mantissa == 7u)) return sign | 0x7eu;
    return sign | ((unsigned)(exponent + 7) << 3) | mantissa;
}

__device__ __forceinline__ float scale_of(unsigned peak_bits) {
    const float peak = __uint_as_float(peak_bits);
    return peak > 0.0f ? peak / 448.0f : 1.0f;
}

__global__ __launch_bounds__(256) void icl8_peaks_kernel(const unsigned short *k, const unsigned short *v,
                                                         long long rows, unsigned *kpeak, unsigned *vpeak,
                                                         unsigned *bad) {
    __shared__ float red[2][4][64];
    const int tid = threadIdx.x, dim = tid & 63, part = tid >> 6;
    const int pair = blockIdx.y;
    const long long r0 = (long long)blockIdx.x * 256, r1 = min(rows, r0 + 256);
    float km = 0.0f, vm = 0.0f;
    unsigned nonfinite = 0;
    for (long long r = r0 + part; r < r1; r += 4) {
        const long long at = ((long long)pair * rows + r) * 64 + dim;
        const float a = fabsf(half_bits_to_float(k[at])), b = fabsf(half_bits_to_float(v[at]));
        nonfinite += !(a <= 65504.0f) + !(b <= 65504.0f);
        km = fmaxf(km, a), vm = fmaxf(vm, b);
    }
    red[0][part][dim] = km, red[1][part][dim] = vm;
    if (nonfinite) atomicAdd(bad, nonfinite);
    __syncthreads();
    if (tid < 64) {
        float a = red[0][0][tid], b = red[1][0][tid];
#pragma unroll
        for (int i = 1; i < 4; ++i) a = fmaxf(a, red[0][i][tid]), b = fmaxf(b, red[1][i][tid]);
        atomicMax(kpeak + pair * 64 + tid, __float_as_uint(a));
        atomicMax(vpeak + pair * 64 + tid, __float_as_uint(b));
    }
}

__global__ __launch_bounds__(256) void icl8_encode_kernel(const unsigned short *k, const unsigned short *v,
                                                          long long rows, long long n_pad, const unsigned *kpeak,
                                                          const unsigned *vpeak, unsigned char *k8,
                                                          unsigned char *v8, float *kscale, float *vscale) {
    const int tid = threadIdx.x, tile = blockIdx.x, pair = blockIdx.y;
    const long long tile_row = (long long)tile * 64;
    // Keys: thread t encodes dims 16 (t % 4) .. +15 of key t / 4.
    {
        const int key = tid >> 2, d0 = 16 * (tid & 3);
        const long long row = tile_row + key;
        unsigned word[4] = {0u, 0u, 0u, 0u};
        if (row < rows) {
            const unsigned short *src = k + ((long long)pair * rows + row) * 64 + d0;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const float x = half_bits_to_float(src[i]) / scale_of(kpeak[pair * 64 + d0 + i]);
                word[i >> 2] |= e4m3(x) << (8 * (i & 3));
            }
        }
        *reinterpret_cast<u32x4 *>(k8 + ((long long)pair * n_pad + row) * 64 + d0) =
            u32x4{word[0], word[1], word[2], word[3]};
    }
    // Values: thread t encodes keys 16 (t % 4) .. +15 of dim t / 4, each at its stored position.
    {
        const int dim = tid >> 2, grp = tid & 3;
        const float scale = scale_of(vpeak[pair * 64 + dim]);
        unsigned word[4] = {0u, 0u, 0u, 0u};
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const long long row = tile_row + 16 * grp + i;
            if (row < rows) {
                const float x = half_bits_to_float(v[((long long)pair * rows + row) * 64 + dim]) / scale;
                const int pos = (i & 3) | ((i & 4) << 1) | ((i & 8) >> 1);
                word[pos >> 2] |= e4m3(x) << (8 * (pos & 3));
            }
        }
        *reinterpret_cast<u32x4 *>(v8 + ((long long)pair * n_pad + tile_row) * 64 + dim * 64 + 16 * grp) =
            u32x4{word[0], word[1], word[2], word[3]};
    }
    if (tile == 0 && tid < 64) {
        kscale[pair * 64 + tid] = scale_of(kpeak[pair * 64 + tid]);
        vscale[pair * 64 + tid] = scale_of(vpeak[pair * 64 + tid]);
    }
}

}  // namespace

Icl8Block icl8_block(void *base, long long pairs, long long rows) {
    Icl8Block b;
    const size_t plane = icl8_plane(pairs, rows);
    unsigned char *p = static_cast<unsigned char *>(base);
    b.k = p, b.v = p + plane;
    float *f = reinterpret_cast<float *>(p + 2 * plane);
    b.kscale = f, b.vscale = f + pairs * 64;
    b.kpeak = reinterpret_cast<unsigned *>(f + 2 * pairs * 64);
    b.vpeak = b.kpeak + pairs * 64;
    return b;
}

void encode_icl8(const unsigned short *k, const unsigned short *v, long long rows, int pairs, void *block,
                 unsigned *bad, hipStream_t stream) {
    if (rows <= 0 || pairs <= 0) return;
    const Icl8Block b = icl8_block(block, pairs, rows);
    const long long n_pad = (rows + 63) / 64 * 64;
    fill_zero(reinterpret_cast<float *>(b.kpeak), 2LL * pairs * 64, stream);
    {
        KernelTimer timer(kFamGlue, stream, 0.0, 2.0 * 2.0 * pairs * rows * 64);
        hipLaunchKernelGGL(icl8_peaks_kernel, dim3((unsigned)ceil_div(rows, 256), (unsigned)pairs), dim3(256), 0,
                           stream, k, v, rows, b.kpeak, b.vpeak, bad);
        IRX_HIP(hipGetLastError());
    }
    KernelTimer timer(kFamGlue, stream, 0.0, 2.0 * 2.0 * pairs * rows * 64 + 2.0 * pairs * n_pad * 64);
    hipLaunchKernelGGL(icl8_encode_kernel, dim3((unsigned)(n_pad / 64), (unsigned)pairs), dim3(256), 0, stream, k, v,
                       rows, n_pad, b.kpeak, b.vpeak, b.k, b.v, b.kscale, b.vscale);
    IRX_HIP(hipGetLastError());
}

}  // namespace irx
