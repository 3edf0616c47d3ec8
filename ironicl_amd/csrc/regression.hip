// Regression outputs from the regressor's decoded quantiles, on the device.
//
// quantiles::summarize (src/models/tabicl_v2/quantiles.rs:80-213): per query
// row and estimator, sort the K decoded quantiles (f32::total_cmp order),
// then in f64 the mean, the unbiased variance, the inverse CDF at each level
// (linear between quantiles, exponential tails fitted to the outermost 20)
// and the sorted values themselves, each averaged over the estimators and
// rounded to f32.
//
// One workgroup per query row. The sort is a bitonic network over order-
// preserving integer keys in LDS; the statistics then run in one lane in the
// reference's own order of f64 operations, with no contraction into fused
// multiply-adds, and every logarithm they need comes precomputed from the
// host (glibc log, as the reference's f64::ln), so the results are the
// reference's to the bit.
#include "common.hpp"

#include <algorithm>
#include <cmath>
#include <vector>

#pragma clang fp contract(off)

namespace irx {
namespace {

constexpr int kSortMax = 4096;

// f32 bits -> unsigned key with the order of f32::total_cmp (-NaN < -inf <
// ... < -0 < +0 < ... < +inf < +NaN).
__device__ __forceinline__ unsigned order_key(unsigned bits) {
    return (bits & 0x80000000u) ? ~bits : bits | 0x80000000u;
}
__device__ __forceinline__ float key_value(unsigned key) {
    return __uint_as_float((key & 0x80000000u) ? key & 0x7FFFFFFFu : ~key);
}

__global__ __launch_bounds__(256) void regression_summary_kernel(RegressionSummary p) {
    __shared__ unsigned keys[kSortMax];
    __shared__ double acc[2 + kRegressionMaxLevels];
    const int tid = threadIdx.x;
    const int row = blockIdx.x;
    const int k = p.k;
    int span = 2;
    while (span < k) span <<= 1;
    if (tid < 2 + kRegressionMaxLevels) acc[tid] = 0.0;
    double raw[kSortMax / 256];
#pragma unroll
    for (int m = 0; m < kSortMax / 256; ++m) raw[m] = 0.0;

    for (int e = 0; e < p.b; ++e) {
        const float *src = p.decoded + ((long long)e * p.q + row) * k;
        for (int i = tid; i < span; i += 256) keys[i] = i < k ? order_key(__float_as_uint(src[i])) : 0xFFFFFFFFu;
        __syncthreads();
        for (int size = 2; size <= span; size <<= 1)
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                for (int i = tid; i < span / 2; i += 256) {
                    const int a = 2 * i - (i & (stride - 1)), b = a + stride;
                    const unsigned ka = keys[a], kb = keys[b];
                    if ((ka > kb) == ((a & size) == 0)) keys[a] = kb, keys[b] = ka;
                }
                __syncthreads();
            }
#pragma unroll
        for (int m = 0; m < kSortMax / 256; ++m) {
            const int i = tid + 256 * m;
            if (i < k) raw[m] = raw[m] + (double)key_value(keys[i]);
        }
        if (tid == 0) {
            auto q = [&](int i) { return (double)key_value(keys[i]); };
            const double n = (double)k;
            double sum = 0.0;
            for (int i = 0; i < k; ++i) sum = sum + q(i);
            const double mean = sum / n;
            acc[0] = acc[0] + mean;
            double squares = 0.0;
            for (int i = 0; i < k; ++i) {
                const double d = q(i) - mean;
                squares = squares + d * d;
            }
            acc[1] = acc[1] + squares / (double)(k - 1);
            // Least-squares slopes of the outermost tk quantiles against the
            // host's log levels (tail_slope).
            const int tk = p.tail;
            auto slope = [&](int first, const double *x) {
                const double nt = (double)tk;
                double xs = 0.0, qs = 0.0;
                for (int i = 0; i < tk; ++i) xs = xs + x[i];
                for (int i = 0; i < tk; ++i) qs = qs + q(first + i);
                const double xm = xs / nt, qm = qs / nt;
                double cov = 0.0, var = 0.0;
                for (int i = 0; i < tk; ++i) {
                    const double dx = x[i] - xm;
                    cov = cov + (q(first + i) - qm) * dx;
                    var = var + dx * dx;
                }
                return (cov / nt) / fmax(var / nt, 1e-6);
            };
            // f64::clamp of |beta| to [0.01, 100]; NaN stays NaN.
            auto clamp = [](double beta) {
                const double m = fabs(beta);
                return m != m ? m : (m < 0.01 ? 0.01 : (m > 100.0 ? 100.0 : m));
            };
            const double bl = clamp(slope(0, p.tail_x)), br = clamp(-slope(k - tk, p.tail_x + tk));
            const double ql = q(0), qr = q(k - 1);
            for (int a = 0; a < p.levels; ++a) {
                const RegressionLevel &lv = p.level[a];
                double v;
                if (lv.kind == 0) {
                    v = ql + bl * lv.value;
                } else if (lv.kind == 1) {
                    v = qr - br * lv.value;
                } else if (lv.kind == 2) {
                    v = qr;
                } else {
                    const double lo = q(lv.segment), hi = q(lv.segment + 1);
                    v = lo + lv.value * (hi - lo);
                }
                acc[2 + a] = acc[2 + a] + v;
            }
        }
        __syncthreads();
    }

    const double nb = (double)p.b;
    if (tid == 0) {
        if (p.mean) p.mean[row] = (float)(acc[0] / nb);
        if (p.variance) p.variance[row] = (float)(acc[1] / nb);
    }
    if (p.at_levels && tid < p.levels) p.at_levels[(long long)row * p.levels + tid] = (float)(acc[2 + tid] / nb);
    if (p.raw) {
#pragma unroll
        for (int m = 0; m < kSortMax / 256; ++m) {
            const int i = tid + 256 * m;
            if (i < k) p.raw[(long long)row * k + i] = (float)(raw[m] / nb);
        }
    }
}

}  // namespace

void regression_tables(const float *alphas, int n_alphas, int k, int *tail, std::vector<double> &tail_x,
                       std::vector<RegressionLevel> &levels) {
    // levels(k) = linspace(0, 1, k + 2)[1:-1] through f32 (quantiles.rs:134-139).
    const double tol = 1e-6;
    std::vector<double> lv(k);
    for (int i = 0; i < k; ++i) lv[i] = (double)(float)((double)(i + 1) / (double)(k + 1));
    const int tk = std::max(1, std::min(20, k / 4));
    *tail = tk;
    tail_x.assign(2 * tk, 0.0);
    for (int i = 0; i < tk; ++i) {
        tail_x[i] = std::log(std::max(lv[i], tol));
        tail_x[tk + i] = std::log(std::max(1.0 - lv[k - tk + i], tol));
    }
    // Distribution::icdf (quantiles.rs:176-201) up to the row's quantiles.
    levels.assign(n_alphas, RegressionLevel{});
    const double al = lv[0], ar = lv[k - 1];
    for (int j = 0; j < n_alphas; ++j) {
        const double a = (double)alphas[j];
        RegressionLevel &r = levels[j];
        if (a < al) {
            r.kind = 0, r.value = std::log(std::max(a, tol)) - std::log(std::max(al, tol));
        } else if (a > ar) {
            const double one_minus_r = 1.0 - std::min(ar, 1.0 - tol);
            r.kind = 1, r.value = std::log(std::max(1.0 - a, tol)) - std::log(one_minus_r);
        } else if (a >= ar) {
            r.kind = 2;
        } else {
            // The last segment whose lower level is at most a (partition_point over levels[..k-1]).
            const int point = (int)(std::upper_bound(lv.begin(), lv.end() - 1, a) - lv.begin());
            const int seg = std::max(point - 1, 0);
            const double lo = lv[seg], hi = lv[seg + 1];
            double t = (a - lo) / std::max(hi - lo, tol);
            t = t < 0.0 ? 0.0 : (t > 1.0 ? 1.0 : t);
            r.kind = 3, r.segment = seg, r.value = t;
        }
    }
}

void regression_summary(const RegressionSummary &s, hipStream_t stream) {
    if (s.q <= 0) return;
    if (s.b < 1 || s.k < 2 || s.k > kSortMax || s.levels < 0 || s.levels > kRegressionMaxLevels || s.tail < 1 ||
        2 * s.tail > s.k || !s.decoded || !s.tail_x || (s.levels && !s.level))
        fail(3, "regression summary: unsupported shape");
    KernelTimer timer(kFamGlue, stream, 0.0, 4.0 * s.b * s.q * s.k);
    hipLaunchKernelGGL(regression_summary_kernel, dim3((unsigned)s.q), dim3(256), 0, stream, s);
    IRX_HIP(hipGetLastError());
}

}  // namespace irx
