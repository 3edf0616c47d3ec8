// LayerNorm and the bandwidth-bound glue of the forward pass.
//
// LayerNorm (src/kernels/reference.rs:223-252): one wave per row, two passes
// over registers (mean, then centred variance), eps 1e-5, population
// variance. Glue kernels restate the data movement of the reference's CUDA
// backend (column_input, build_rows, gather_cls, repeat, add_labels;
// src/kernels/cuda/kernels.rs:475-718) in this backend's layouts:
//   column states   [B*H, rows, 128]   (column c = b*H + f)
//   row sequences   [B*rows, H+4, 128] (4 CLS tokens, then the features)
#include "common.hpp"

namespace irx {
namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float half_wave_sum(float v) {
#pragma unroll
    for (int offset = 16; offset >= 1; offset >>= 1) v += __shfl_xor(v, offset, 64);
    return v;
}

// 128-wide rows (layer_norm_f32, reference.rs:223-252: two-pass mean and
// variance, eps 1e-5): 32 lanes per row, each moving 16 bytes, two rows per
// wave and eight per workgroup, so every load and store instruction of a wave
// covers 1 KB of contiguous rows. Shuffles stay within a row's half-wave.
__global__ __launch_bounds__(256) void layer_norm128_kernel(const float *x, long long ldx, const float *w,
                                                            const float *b, float *y, long long ldy, long long rows) {
    const long long row = (long long)blockIdx.x * 8 + (threadIdx.x >> 5);
    if (row >= rows) return;  // a whole half-wave: its shuffles never read the other half
    const int c = (threadIdx.x & 31) * 4;
    const f32x4 v = *reinterpret_cast<const f32x4 *>(x + row * ldx + c);
    const float mean = half_wave_sum((v[0] + v[1]) + (v[2] + v[3])) / 128.0f;
    const f32x4 d = v - mean;
    float sq = d[0] * d[0];
    sq = fmaf(d[1], d[1], sq);
    sq = fmaf(d[2], d[2], sq);
    sq = fmaf(d[3], d[3], sq);
    const float rstd = 1.0f / sqrtf(half_wave_sum(sq) / 128.0f + 1e-5f);
    const f32x4 g = *reinterpret_cast<const f32x4 *>(w + c);
    f32x4 o = d * rstd * g;
    if (b) o += *reinterpret_cast<const f32x4 *>(b + c);
    *reinterpret_cast<f32x4 *>(y + row * ldy + c) = o;
}

// 512-wide rows (layer_norm_f32, reference.rs:223-252: two-pass mean and
// variance, eps 1e-5): one wave takes two rows, each lane eight values of
// each, with all four 16-byte loads issued before the two rows' reduction
// chains run side by side; eight rows per workgroup.
__global__ __launch_bounds__(256) void layer_norm512_kernel(const float *x, long long ldx, const float *w,
                                                            const float *b, float *y, long long ldy, long long rows) {
    const long long r0 = ((long long)blockIdx.x * 4 + (threadIdx.x >> 6)) * 2;
    if (r0 >= rows) return;
    const bool two = r0 + 1 < rows;
    const int c = (threadIdx.x & 63) * 8;
    f32x4 v[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const float *xr = x + (r0 + (two ? i : 0)) * ldx + c;
        v[i][0] = *reinterpret_cast<const f32x4 *>(xr);
        v[i][1] = *reinterpret_cast<const f32x4 *>(xr + 4);
    }
    float s[2], mean[2], sq[2], rstd[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) s[i] = ((v[i][0][0] + v[i][0][1]) + (v[i][0][2] + v[i][0][3])) +
                                       ((v[i][1][0] + v[i][1][1]) + (v[i][1][2] + v[i][1][3]));
#pragma unroll
    for (int offset = 32; offset >= 1; offset >>= 1)
#pragma unroll
        for (int i = 0; i < 2; ++i) s[i] += __shfl_xor(s[i], offset, 64);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        mean[i] = s[i] / 512.0f;
        v[i][0] -= mean[i];
        v[i][1] -= mean[i];
        float q = v[i][0][0] * v[i][0][0];
        q = fmaf(v[i][0][1], v[i][0][1], q);
        q = fmaf(v[i][0][2], v[i][0][2], q);
        q = fmaf(v[i][0][3], v[i][0][3], q);
        q = fmaf(v[i][1][0], v[i][1][0], q);
        q = fmaf(v[i][1][1], v[i][1][1], q);
        q = fmaf(v[i][1][2], v[i][1][2], q);
        sq[i] = fmaf(v[i][1][3], v[i][1][3], q);
    }
#pragma unroll
    for (int offset = 32; offset >= 1; offset >>= 1)
#pragma unroll
        for (int i = 0; i < 2; ++i) sq[i] += __shfl_xor(sq[i], offset, 64);
    const f32x4 g0 = *reinterpret_cast<const f32x4 *>(w + c), g1 = *reinterpret_cast<const f32x4 *>(w + c + 4);
    f32x4 b0 = {0.f, 0.f, 0.f, 0.f}, b1 = b0;
    if (b) b0 = *reinterpret_cast<const f32x4 *>(b + c), b1 = *reinterpret_cast<const f32x4 *>(b + c + 4);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        if (i == 1 && !two) break;
        rstd[i] = 1.0f / sqrtf(sq[i] / 512.0f + 1e-5f);
        float *yr = y + (r0 + i) * ldy + c;
        *reinterpret_cast<f32x4 *>(yr) = v[i][0] * rstd[i] * g0 + b0;
        *reinterpret_cast<f32x4 *>(yr + 4) = v[i][1] * rstd[i] * g1 + b1;
    }
}

// Grouped features (f+1, f+2, f+4) mod H through the 3 -> 128 input affine
// (cpu.rs:1144-1157, 2461-2473), the -100 all-missing marker, and the
// column-stage label embeddings of training rows. One thread per four channels
// of an (estimator, feature, row); the launcher keeps b * h * rows below 2^32
// so the index arithmetic is 32-bit.
__global__ __launch_bounds__(256) void column_input_kernel(const float *x, long long xs, int b, int rows, int h,
                                                           const float *in_w, const float *in_b,
                                                           const float *labels, float *state,
                                                           uint8_t *missing) {
    const long long total4 = (long long)b * h * rows * (kColumnDim / 4);
    const unsigned urows = (unsigned)rows, uh = (unsigned)h;
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total4; i += (long long)gridDim.x * 256) {
        const int ch = (int)(i & (kColumnDim / 4 - 1)) * 4;
        const unsigned cr = (unsigned)(i / (kColumnDim / 4));
        const unsigned r = cr % urows, c = cr / urows;
        const unsigned e = c / uh, f = c - e * uh;
        const float *xr = x + (long long)e * xs + (long long)r * h;
        const float s0 = xr[(f + 1) % uh], s1 = xr[(f + 2) % uh], s2 = xr[(f + 4) % uh];
        // in_w [128, 3]: the 12 weights of channels ch..ch+3 are contiguous.
        const f32x4 wa = *reinterpret_cast<const f32x4 *>(in_w + ch * 3);
        const f32x4 wb = *reinterpret_cast<const f32x4 *>(in_w + ch * 3 + 4);
        const f32x4 wc = *reinterpret_cast<const f32x4 *>(in_w + ch * 3 + 8);
        const float w[12] = {wa[0], wa[1], wa[2], wa[3], wb[0], wb[1], wb[2], wb[3], wc[0], wc[1], wc[2], wc[3]};
        const f32x4 bias = *reinterpret_cast<const f32x4 *>(in_b + ch);
        f32x4 v;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float t = fmaf(w[3 * j + 0], s0, bias[j]);
            t = fmaf(w[3 * j + 1], s1, t);
            v[j] = fmaf(w[3 * j + 2], s2, t);
        }
        if (s0 == -100.0f && s1 == -100.0f && s2 == -100.0f) {
            v = f32x4{-100.0f, -100.0f, -100.0f, -100.0f};
            if (missing && ch == 0) missing[r] = 1;  // row r holds the marker in some estimator
        }
        if (labels) v += *reinterpret_cast<const f32x4 *>(labels + ((long long)e * rows + r) * kColumnDim + ch);
        *reinterpret_cast<f32x4 *>(state + (long long)cr * kColumnDim + ch) = v;
    }
}

// Row sequences: the 4 CLS tokens, then feature f's column state
// (cpu.rs:1226-1231). One thread per four channels of a token; the launcher
// keeps b * rows * (h + 4) below 2^32.
__global__ __launch_bounds__(256) void build_rows_kernel(const float *state, int b, int rows, int h,
                                                         const float *cls, float *seq) {
    const unsigned len = (unsigned)h + kReserved, urows = (unsigned)rows;
    const long long total4 = (long long)b * rows * len * (kColumnDim / 4);
    for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < total4; i += (long long)gridDim.x * 256) {
        const int ch = (int)(i & (kColumnDim / 4 - 1)) * 4;
        const unsigned st = (unsigned)(i / (kColumnDim / 4));
        const unsigned t = st % len, s = st / len;
        const unsigned r = s % urows, e = s / urows;
        const f32x4 v = t < kReserved
                            ? *reinterpret_cast<const f32x4 *>(cls + t * kColumnDim + ch)
                            : *reinterpret_cast<const f32x4 *>(
                                  state + (((long long)e * h + (t - kReserved)) * rows + r) * kColumnDim + ch);
        *reinterpret_cast<f32x4 *>(seq + (long long)st * kColumnDim + ch) = v;
    }
}

__global__ __launch_bounds__(256) void gather_cls_kernel(const float *seq, long long seqs, int len, float *cls) {
    const long long total = seqs * kReserved * kColumnDim;
    for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (long long)gridDim.x * 256) {
        const long long s = idx / (kReserved * kColumnDim);
        const int within = (int)(idx - s * (kReserved * kColumnDim));
        cls[idx] = seq[s * len * kColumnDim + within];
    }
}

// Label embeddings [n, width] from targets [n] (target_embeddings,
// cpu.rs:1658-1680): a classifier's row takes column `class` of w [width,
// classes] plus the bias, one FP32 sum; a regressor's is target * w[:, 0] +
// bias with both roundings (never a fused multiply-add), as the reference's
// loop computes it. Classes outside 0 .. classes - 1 are clamped (the host
// validates labels first).
__global__ __launch_bounds__(256) void label_embedding_kernel(const float *targets, long long n, const float *w,
                                                              const float *b, int classes, int width,
                                                              bool classifier, float *out) {
    const long long count = n * width;
    for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < count; idx += (long long)gridDim.x * 256) {
        const long long row = idx / width;
        const int c = (int)(idx - row * width);
        const float t = targets[row];
        float v;
        if (classifier) {
            const int k = min(max((int)t, 0), classes - 1);
            v = __fadd_rn(w[(long long)c * classes + k], b[c]);
        } else {
            v = __fadd_rn(__fmul_rn(t, w[c]), b[c]);
        }
        out[idx] = v;
    }
}

__global__ __launch_bounds__(256) void gelu_kernel(const float *x, float *y, long long count) {
    for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < count; idx += (long long)gridDim.x * 256)
        y[idx] = gelu_erf(x[idx]);
}

__global__ __launch_bounds__(256) void add_kernel(float *y, const float *x, long long count) {
    for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < count; idx += (long long)gridDim.x * 256)
        y[idx] += x[idx];
}

__global__ __launch_bounds__(256) void repeat_kernel(const float *src, long long src_floats, long long copies,
                                                     float *dst) {
    const long long total = src_floats * copies;
    for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < total; idx += (long long)gridDim.x * 256)
        dst[idx] = src[idx % src_floats];
}

__global__ __launch_bounds__(256) void nonfinite_kernel(const float *x, long long count, unsigned *counter) {
    bool bad = false;
    for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < count; idx += (long long)gridDim.x * 256)
        bad |= !isfinite(x[idx]);
    if (__any(bad) && (threadIdx.x & 63) == 0) atomicAdd(counter, 1u);
}

// A plain copy, one float4 per thread: the reference point that scales the
// HBM traffic counters of the other kernels.
__global__ __launch_bounds__(256) void copy_kernel(const float *src, float *dst, long long count4) {
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx < count4) reinterpret_cast<f32x4 *>(dst)[idx] = reinterpret_cast<const f32x4 *>(src)[idx];
}

__global__ __launch_bounds__(256) void zero_kernel(float *x, long long count) {
    for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < count; idx += (long long)gridDim.x * 256)
        x[idx] = 0.f;
}

// Blocks of 256 threads for a 1D element loop of `total` items: the kernels
// stride over the grid, so a launch stays far below the 2^32 work-items a
// dispatch can hold (one estimator's column states at 200,000 rows x 500
// features are 12.8G floats).
dim3 grid_1d(long long total) {
    constexpr long long kMaxBlocks = 1 << 20;
    return dim3((unsigned)std::min<long long>((total + 255) / 256, kMaxBlocks));
}

}  // namespace

void layer_norm(const float *x, long long ldx, const float *weight, const float *bias, float *y, long long ldy,
                long long rows, int width, hipStream_t stream) {
    if (rows <= 0) return;
    if ((reinterpret_cast<uintptr_t>(x) & 15) || (reinterpret_cast<uintptr_t>(y) & 15) || (ldx & 3) || (ldy & 3))
        fail(3, "layer norm operands must be 16-byte aligned");
    KernelTimer timer(kFamNorm, stream, 8.0 * rows * width, 8.0 * rows * width);
    if (width == 128)
        hipLaunchKernelGGL(layer_norm128_kernel, dim3(ceil_div(rows, 8)), dim3(256), 0, stream, x, ldx, weight, bias,
                           y, ldy, rows);
    else if (width == 512)
        hipLaunchKernelGGL(layer_norm512_kernel, dim3(ceil_div(rows, 8)), dim3(256), 0, stream, x, ldx, weight,
                           bias, y, ldy, rows);
    else
        fail(3, "layer norm width must be 128 or 512");
    IRX_HIP(hipGetLastError());
}

void column_input(const float *x, long long x_estimator_stride, int b, int rows, int h, const float *in_w,
                  const float *in_b, const float *labels, float *state, uint8_t *missing_rows, hipStream_t stream) {
    long long total = (long long)b * h * rows * kColumnDim;
    if (total <= 0) return;
    if ((long long)b * h * rows >= (1LL << 32)) fail(3, "column input: more than 2^32 columns x rows");
    if ((reinterpret_cast<uintptr_t>(state) | reinterpret_cast<uintptr_t>(labels) | reinterpret_cast<uintptr_t>(in_w) |
         reinterpret_cast<uintptr_t>(in_b)) & 15)
        fail(3, "column input: operands must be 16-byte aligned");
    KernelTimer timer(kFamGlue, stream, 0.0, 4.0 * total + 4.0 * b * rows * h);
    hipLaunchKernelGGL(column_input_kernel, grid_1d(total / 4), dim3(256), 0, stream, x, x_estimator_stride, b, rows, h, in_w,
                       in_b, labels, state, missing_rows);
    IRX_HIP(hipGetLastError());
}

void build_rows(const float *state, int b, int rows, int h, const float *cls, float *seq, hipStream_t stream) {
    long long total = (long long)b * rows * (h + kReserved) * kColumnDim;
    if (total <= 0) return;
    if ((long long)b * rows * (h + kReserved) >= (1LL << 32)) fail(3, "row sequences: more than 2^32 tokens");
    if ((reinterpret_cast<uintptr_t>(state) | reinterpret_cast<uintptr_t>(cls) | reinterpret_cast<uintptr_t>(seq)) & 15)
        fail(3, "row sequences: operands must be 16-byte aligned");
    KernelTimer timer(kFamGlue, stream, 0.0, 8.0 * total);
    hipLaunchKernelGGL(build_rows_kernel, grid_1d(total / 4), dim3(256), 0, stream, state, b, rows, h, cls,
                       seq);
    IRX_HIP(hipGetLastError());
}

void gather_cls(const float *seq, long long seqs, int len, float *cls, hipStream_t stream) {
    long long total = seqs * kReserved * kColumnDim;
    if (total <= 0) return;
    KernelTimer timer(kFamGlue, stream, 0.0, 8.0 * total);
    hipLaunchKernelGGL(gather_cls_kernel, grid_1d(total), dim3(256), 0, stream, seq, seqs, len, cls);
    IRX_HIP(hipGetLastError());
}

void label_embeddings(const float *targets, long long n, const float *w, const float *b, int classes, int width,
                      bool classifier, float *out, hipStream_t stream) {
    if (n <= 0) return;
    const long long count = n * width;
    KernelTimer timer(kFamGlue, stream, 0.0, 4.0 * (n + count));
    hipLaunchKernelGGL(label_embedding_kernel, grid_1d(count), dim3(256), 0, stream, targets, n, w, b, classes, width,
                       classifier, out);
    IRX_HIP(hipGetLastError());
}

void gelu_apply(const float *x, float *y, long long count, hipStream_t stream) {
    if (count <= 0) return;
    hipLaunchKernelGGL(gelu_kernel, grid_1d(count), dim3(256), 0, stream, x, y, count);
    IRX_HIP(hipGetLastError());
}

void add_inplace(float *y, const float *x, long long count, hipStream_t stream) {
    if (count <= 0) return;
    KernelTimer timer(kFamGlue, stream, 0.0, 12.0 * count);
    hipLaunchKernelGGL(add_kernel, grid_1d(count), dim3(256), 0, stream, y, x, count);
    IRX_HIP(hipGetLastError());
}

void repeat_rows(const float *src, long long src_floats, long long copies, float *dst, hipStream_t stream) {
    long long total = src_floats * copies;
    if (total <= 0) return;
    KernelTimer timer(kFamGlue, stream, 0.0, 4.0 * total + 4.0 * src_floats);
    hipLaunchKernelGGL(repeat_kernel, grid_1d(total), dim3(256), 0, stream, src, src_floats, copies,
                       dst);
    IRX_HIP(hipGetLastError());
}

void count_nonfinite(const float *x, long long count, unsigned *counter, hipStream_t stream) {
    if (count <= 0) return;
    KernelTimer timer(kFamGlue, stream, 0.0, 4.0 * count);
    hipLaunchKernelGGL(nonfinite_kernel, grid_1d(count), dim3(256), 0, stream, x, count, counter);
    IRX_HIP(hipGetLastError());
}

void copy_floats(const float *src, float *dst, long long count, hipStream_t stream) {
    if (count <= 0) return;
    if (count % 4 || (reinterpret_cast<uintptr_t>(src) & 15) || (reinterpret_cast<uintptr_t>(dst) & 15))
        fail(3, "copy: count must be a multiple of 4 floats with 16-byte aligned buffers");
    KernelTimer timer(kFamGlue, stream, 0.0, 8.0 * count);
    hipLaunchKernelGGL(copy_kernel, dim3(ceil_div(count / 4, 256)), dim3(256), 0, stream, src, dst, count / 4);
    IRX_HIP(hipGetLastError());
}

void fill_zero(float *x, long long count, hipStream_t stream) {
    if (count <= 0) return;
    KernelTimer timer(kFamGlue, stream, 0.0, 4.0 * count);
    hipLaunchKernelGGL(zero_kernel, grid_1d(count), dim3(256), 0, stream, x, count);
    IRX_HIP(hipGetLastError());
}

}  // namespace irx
