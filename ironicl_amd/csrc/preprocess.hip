// TabICL's numeric preprocessing on the GPU, in f64: fitting every kept
// feature's statistics at once, and transforming raw rows into each ensemble
// member's FP32 rows in HBM.
//
// Fit (fit_feature, src/models/tabicl_v2/preprocess.rs:259-296): one
// workgroup per kept feature. It standardizes and clips the column
// (scale.rs standard_clip / clip_standardized) into a column-major f64
// scratch, takes its range, then per normalization group the two-pass
// outlier bounds (scale.rs outlier_bounds) and, for "power", scikit-learn's
// Yeo-Johnson PowerTransformer: SciPy's yeojohnson_normmax, whose
// bounded-Brent search (fminbound) runs on every thread of the workgroup in
// lockstep while each log-likelihood evaluation is a workgroup reduction over
// the N rows (yeo_johnson.rs:55-216). Sums are workgroup trees rather than
// the reference's serial loops, so statistics agree to rounding, not bitwise.
//
// Transform (Normalization::transform, preprocess.rs:223-254, and
// ensemble_rows, :588-613): one thread per (row, kept feature) and group,
// then a gather of each member's feature order. A group whose power
// transform overflows anywhere in a chunk of rows is redone for that whole
// chunk with values clipped to the training range, as TabICL's fallback does.
#include <algorithm>

#include "common.hpp"

namespace irx {
namespace {

constexpr int kFitThreads = 512;
constexpr int kFitWaves = kFitThreads / 64;
constexpr double kEps = 2.220446049250313080847e-16;       // f64 machine epsilon
constexpr double kMinPositive = 2.2250738585072013831e-308;  // smallest normal f64
constexpr double kMax = 1.7976931348623157081e308;

__device__ double block_sum(double v, double *lds) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    __syncthreads();  // the previous reduction's readers are done with lds
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
#pragma unroll
    for (int w = 0; w < kFitWaves; ++w) t += lds[w];
    return t;
}

__device__ double block_max(double v, double *lds) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = fmax(v, __shfl_xor(v, off, 64));
    __syncthreads();
    if ((threadIdx.x & 63) == 0) lds[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = -INFINITY;
#pragma unroll
    for (int w = 0; w < kFitWaves; ++w) t = fmax(t, lds[w]);
    return t;
}

__device__ double block_min(double v, double *lds) { return -block_max(-v, lds); }

// SciPy's _yeojohnson_transform of one value (yeo_johnson.rs:21-33).
__device__ __forceinline__ double yeo_johnson(double x, double lambda) {
    if (x >= 0.0) {
        if (fabs(lambda) < kEps) return log1p(x);
        return expm1(lambda * log1p(x)) / lambda;
    }
    if (fabs(lambda - 2.0) > kEps) return -expm1((2.0 - lambda) * log1p(-x)) / (2.0 - lambda);
    return -log1p(-x);
}

// scale.rs is_constant: StandardScaler's test for a zero variance.
__device__ __forceinline__ bool is_constant(double variance, double mean, long long rows) {
    const double n = (double)rows;
    const double bound = n * mean * kEps;
    return variance <= n * kEps * variance + bound * bound;
}

// clamp_outlier (scale.rs): soft bounds that grow with log1p of the value.
__device__ __forceinline__ double clamp_outlier(double value, double lower, double upper) {
    const double low = fmax(value, lower - log1p(fabs(value)));
    return fmin(low, upper + log1p(fabs(low)));
}

struct FitArgs {
    const void *x;
    int x_f64;
    long long rows, columns;
    const unsigned *kept;  // kept column of each fitted feature
    int features;          // features in this launch
    int feature0;          // index of the first within all kept features
    int kept_count;
    int groups;
    int methods[2];        // 0 none, 1 power
    double threshold;
    double *scratch;       // [features, 3, rows]
    double *stats;         // [groups, 9, kept_count]
    int *status;           // [kept_count]
    int raw;               // fit the power transform on the values as given (no standardization)
    double *fitted;        // raw mode: the fitted, standardized power transform [kept_count, rows], or null
};

enum FitStatus { kFitOk = 0, kFitNonFinite = 1, kFitBounds = 2, kFitPowerNonFinite = 3 };

// One kept feature per workgroup; every scalar below is computed identically
// by all threads (reductions are broadcast), so control flow is uniform.
__global__ __launch_bounds__(kFitThreads) void preprocess_fit_kernel(FitArgs a) {
    __shared__ double lds[kFitWaves];
    const int f = blockIdx.x;
    if (f >= a.features) return;
    const int k = a.feature0 + f;
    const long long n = a.rows;
    const long long col = a.kept[k];
    double *s = a.scratch + (long long)f * 3 * n;  // standardized values
    double *lg = s + n;                            // log1p(|s|) for the power fit
    double *w = lg + n;                            // power-transformed values
    const int t0 = threadIdx.x;
    auto xv = [&](long long r) -> double {
        return a.x_f64 ? static_cast<const double *>(a.x)[r * a.columns + col]
                       : (double)static_cast<const float *>(a.x)[r * a.columns + col];
    };

    // standard_clip: mean and population variance, scale = std + 1e-6.
    double acc = 0.0;
    for (long long r = t0; r < n; r += kFitThreads) acc += xv(r);
    const double mean = block_sum(acc, lds) / (double)n;
    acc = 0.0;
    for (long long r = t0; r < n; r += kFitThreads) {
        const double d = xv(r) - mean;
        acc += d * d;
    }
    const double scale = sqrt(block_sum(acc, lds) / (double)n) + 1e-6;
    double lo = INFINITY, hi = -INFINITY;
    for (long long r = t0; r < n; r += kFitThreads) {
        const double v = a.raw ? xv(r) : fmin(fmax((xv(r) - mean) / scale, -100.0), 100.0);
        s[r] = v;
        lo = fmin(lo, v), hi = fmax(hi, v);
    }
    const double minimum = block_min(lo, lds), maximum = block_max(hi, lds);
    __syncthreads();  // s is complete

    // mean and variance (ddof) of v[r] over the rows where keep(v) holds.
    auto moments = [&](auto value, auto keep, int ddof, double &m, double &var, double &count) {
        double c = 0.0, sum = 0.0;
        for (long long r = t0; r < n; r += kFitThreads) {
            const double v = value(r);
            if (keep(v)) c += 1.0, sum += v;
        }
        count = block_sum(c, lds);
        m = block_sum(sum, lds) / count;
        double sq = 0.0;
        for (long long r = t0; r < n; r += kFitThreads) {
            const double v = value(r);
            if (keep(v)) sq += (v - m) * (v - m);
        }
        var = block_sum(sq, lds) / (count - (double)ddof);
    };
    auto all = [](double) { return true; };
    // Two-pass outlier bounds of v (scale.rs outlier_bounds).
    auto outlier_bounds = [&](const double *v, double &lower, double &upper) {
        auto at = [&](long long r) { return v[r]; };
        double m, var, count;
        lower = upper = NAN;
        if (n < 2) return;
        moments(at, all, 1, m, var, count);
        double spread = a.threshold * fmax(sqrt(var), 1e-6);
        const double l0 = m - spread, u0 = m + spread;
        moments(at, [&](double x) { return x >= l0 && x <= u0; }, 1, m, var, count);
        if (count < 2.0) return;
        spread = a.threshold * fmax(sqrt(var), 1e-6);
        lower = m - spread, upper = m + spread;
    };

    int status = kFitOk;
    for (int g = 0; g < a.groups; ++g) {
        double lower, upper, lambda = 0.0, pmean = 0.0, pscale = 0.0;
        const bool power = a.methods[g] == 1;
        if (!power) {
            outlier_bounds(s, lower, upper);
        } else {
            // fit_power on the standardized values (yeo_johnson.rs:219-243).
            double m0, var0, cnt;
            moments([&](long long r) { return s[r]; }, all, 0, m0, var0, cnt);
            bool transform = false;
            lambda = 1.0;
            if (!is_constant(var0, m0, n)) {
                transform = true;
                // yeojohnson_normmax (yeo_johnson.rs:170-208).
                double big = 0.0, neg = 0.0, nonneg = 0.0, nonzero = 0.0, jac = 0.0;
                for (long long r = t0; r < n; r += kFitThreads) {
                    const double v = s[r];
                    big = fmax(big, fabs(v));
                    neg += v < 0.0 ? 1.0 : 0.0;
                    nonneg += v >= 0.0 ? 1.0 : 0.0;
                    nonzero += v != 0.0 ? 1.0 : 0.0;
                    const double sg = signbit(v) ? -1.0 : 1.0;
                    jac += sg * log1p(fabs(v));
                }
                big = block_max(big, lds);
                neg = block_sum(neg, lds);
                nonneg = block_sum(nonneg, lds);
                nonzero = block_sum(nonzero, lds);
                jac = block_sum(jac, lds);
                if (nonzero == 0.0) {
                    lambda = 1.0;
                } else {
                    const double log1p_max_x = log1p(20.0 * big);
                    const double log_eps = log(kEps);
                    const double log_tiny = (log(kMinPositive) - log_eps) / 2.0;
                    const double log_max = (log(kMax) + log_eps) / 2.0;
                    double lb = log_tiny / log1p_max_x, ub = log_max / log1p_max_x;
                    const bool all_neg = neg == (double)n, all_nonneg = nonneg == (double)n;
                    if (all_neg) {
                        const double l = 2.0 - ub, u = 2.0 - lb;
                        lb = l, ub = u;
                    } else if (!all_nonneg) {
                        const double l = fmax(lb, 2.0 - ub), u = fmin(ub, 2.0 - lb);
                        lb = l, ub = u;
                    }
                    if (!(isfinite(lb) && isfinite(ub)) || lb > ub) {
                        status = kFitBounds;
                        break;
                    }
                    const int mode = all_nonneg ? 1 : (all_neg ? 2 : 0);
                    if (mode) {
                        for (long long r = t0; r < n; r += kFitThreads) lg[r] = log1p(fabs(s[r]));
                        __syncthreads();
                    }
                    // -log-likelihood (yeo_johnson.rs:39-67), inf for an infinite one.
                    auto nll = [&](double lam) -> double {
                        double lv;
                        if (mode) {
                            const double p = mode == 1 ? lam : 2.0 - lam;
                            double mm, vv, cc;
                            if (fabs(p) < kEps) {
                                moments([&](long long r) { return lg[r]; }, all, 0, mm, vv, cc);
                                lv = log(vv);
                            } else {
                                double hiv = -INFINITY;
                                for (long long r = t0; r < n; r += kFitThreads) hiv = fmax(hiv, p * lg[r]);
                                const double largest = block_max(hiv, lds);
                                moments([&](long long r) { return exp(p * lg[r] - largest); }, all, 0, mm, vv, cc);
                                lv = log(vv) + 2.0 * largest - 2.0 * log(fabs(p));
                            }
                        } else {
                            double mm, vv, cc;
                            moments([&](long long r) { return yeo_johnson(s[r], lam); }, all, 0, mm, vv, cc);
                            lv = log(vv);
                        }
                        const double llf = -(double)n / 2.0 * lv + (lam - 1.0) * jac;
                        return isinf(llf) ? INFINITY : -llf;
                    };
                    // fminbound (yeo_johnson.rs:74-163), SciPy's bounded Brent search.
                    const double xatol = 1.48e-8;
                    const int maxfun = 500;
                    const double sqrt_eps = sqrt(2.2e-16);
                    const double golden_mean = 0.5 * (3.0 - sqrt(5.0));
                    auto step_sign = [](double v) { return v < 0.0 ? -1.0 : 1.0; };
                    double A = lb, B = ub;
                    double fulc = A + golden_mean * (B - A);
                    double nfc = fulc, xf = fulc, rat = 0.0, e = 0.0;
                    double fx = nll(xf);
                    int calls = 1;
                    double ffulc = fx, fnfc = fx;
                    double xm = 0.5 * (A + B);
                    double tol1 = sqrt_eps * fabs(xf) + xatol / 3.0, tol2 = 2.0 * tol1;
                    while (fabs(xf - xm) > (tol2 - 0.5 * (B - A))) {
                        bool golden = true;
                        if (fabs(e) > tol1) {
                            golden = false;
                            double r = (xf - nfc) * (fx - ffulc);
                            double q = (xf - fulc) * (fx - fnfc);
                            double p = (xf - fulc) * q - (xf - nfc) * r;
                            q = 2.0 * (q - r);
                            if (q > 0.0) p = -p;
                            q = fabs(q);
                            r = e;
                            e = rat;
                            if (fabs(p) < fabs(0.5 * q * r) && p > q * (A - xf) && p < q * (B - xf)) {
                                rat = p / q;
                                const double xn = xf + rat;
                                if ((xn - A) < tol2 || (B - xn) < tol2) rat = tol1 * step_sign(xm - xf);
                            } else {
                                golden = true;
                            }
                        }
                        if (golden) {
                            e = xf >= xm ? A - xf : B - xf;
                            rat = golden_mean * e;
                        }
                        const double xn = xf + step_sign(rat) * fmax(fabs(rat), tol1);
                        const double fu = nll(xn);
                        ++calls;
                        if (fu <= fx) {
                            if (xn >= xf) A = xf;
                            else B = xf;
                            fulc = nfc, ffulc = fnfc;
                            nfc = xf, fnfc = fx;
                            xf = xn, fx = fu;
                        } else {
                            if (xn < xf) A = xn;
                            else B = xn;
                            if (fu <= fnfc || nfc == xf) {
                                fulc = nfc, ffulc = fnfc;
                                nfc = xn, fnfc = fu;
                            } else if (fu <= ffulc || fulc == xf || fulc == nfc) {
                                fulc = xn, ffulc = fu;
                            }
                        }
                        xm = 0.5 * (A + B);
                        tol1 = sqrt_eps * fabs(xf) + xatol / 3.0;
                        tol2 = 2.0 * tol1;
                        if (calls >= maxfun) break;
                    }
                    lambda = xf;
                }
            }
            // The transformed values (a constant column keeps its values),
            // then StandardScaler (scale.rs standard_scaler).
            double bad = 0.0, sum = 0.0;
            for (long long r = t0; r < n; r += kFitThreads) {
                const double v = transform ? yeo_johnson(s[r], lambda) : s[r];
                w[r] = v;
                bad += isfinite(v) ? 0.0 : 1.0;
                sum += v;
            }
            if (block_sum(bad, lds) != 0.0) {
                status = kFitPowerNonFinite;
                break;
            }
            pmean = block_sum(sum, lds) / (double)n;
            double corr = 0.0, sq = 0.0;
            for (long long r = t0; r < n; r += kFitThreads) {
                const double d = w[r] - pmean;
                corr += d, sq += d * d;
            }
            corr = block_sum(corr, lds);
            sq = block_sum(sq, lds);
            const double var = (sq - corr * corr / (double)n) / (double)n;
            pscale = is_constant(var, pmean, n) ? 1.0 : sqrt(var);
            for (long long r = t0; r < n; r += kFitThreads) {
                w[r] = (w[r] - pmean) / pscale;
                if (a.fitted) a.fitted[(long long)k * n + r] = w[r];
            }
            __syncthreads();
            outlier_bounds(w, lower, upper);
        }
        const double st[9] = {mean, scale, minimum, maximum, lower, upper, lambda, pmean, pscale};
        const int count = power ? 9 : 6;
        bool finite = true;
        for (int i = 0; i < count; ++i) finite = finite && isfinite(st[i]);
        if (!finite) {
            status = kFitNonFinite;
            break;
        }
        if (t0 == 0)
            for (int i = 0; i < 9; ++i) a.stats[((long long)g * 9 + i) * a.kept_count + k] = i < count ? st[i] : 0.0;
    }
    if (t0 == 0) a.status[k] = status;
}

struct TransformArgs {
    const void *x;
    int x_f64;
    long long rows, columns;
    const unsigned *kept;
    int kept_count;
    int groups;
    int methods[2];
    const double *stats;   // [groups, 9, kept_count]
    long long chunk_rows;
    const int *redo;       // [chunks, groups]: clip and recompute; null on the first pass
    int *overflow;         // [chunks, groups]
    int *nonfinite;        // [1]
    float *out;            // [groups, rows, kept_count]
};

// One thread per (row, kept feature) of every group: Normalization::value.
__global__ __launch_bounds__(256) void preprocess_transform_kernel(TransformArgs a) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long per_group = a.rows * a.kept_count;
    if (i >= per_group * a.groups) return;
    const int g = (int)(i / per_group);
    const long long rk = i - g * per_group;
    const long long row = rk / a.kept_count;
    const int k = (int)(rk - row * a.kept_count);
    const long long chunk = row / a.chunk_rows;
    const bool clip = a.redo != nullptr;
    if (clip && !a.redo[chunk * a.groups + g]) return;
    const long long src = row * a.columns + a.kept[k];
    const double x = a.x_f64 ? static_cast<const double *>(a.x)[src] : (double)static_cast<const float *>(a.x)[src];
    auto stat = [&](int s) { return a.stats[((long long)g * 9 + s) * a.kept_count + k]; };
    double v = fmin(fmax((x - stat(0)) / stat(1), -100.0), 100.0);
    if (a.methods[g] == 1) {
        if (clip) v = fmin(fmax(v, stat(2)), stat(3));
        v = yeo_johnson(v, stat(6));
        if (!isfinite(v)) {
            a.overflow[chunk * a.groups + g] = 1;
            return;
        }
        v = (v - stat(7)) / stat(8);
    }
    const float out = (float)clamp_outlier(v, stat(4), stat(5));
    if (!isfinite(out)) a.nonfinite[0] = 1;
    a.out[i] = out;
}

// Each member's rows in its feature order: out[b, row, j] = groups[group(b), row, order(b)[j]].
__global__ __launch_bounds__(256) void preprocess_gather_kernel(const float *group_rows, long long rows, int features,
                                                                int members, const unsigned *member_groups,
                                                                const unsigned *orders, float *out) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long per_member = rows * features;
    if (i >= per_member * members) return;
    const int b = (int)(i / per_member);
    const long long rj = i - b * per_member;
    const long long row = rj / features;
    const int j = (int)(rj - row * features);
    out[i] = group_rows[((long long)member_groups[b] * rows + row) * features + orders[(long long)b * features + j]];
}

}  // namespace

void preprocess_fit(const PreprocessFit &p, hipStream_t stream) {
    if (p.rows < 1 || p.kept_count < 1 || p.groups < 1 || p.groups > 2) fail(3, "preprocessing fit: invalid shape");
    FitArgs a{};
    a.x = p.x, a.x_f64 = p.x_f64, a.rows = p.rows, a.columns = p.columns, a.kept = p.kept;
    a.kept_count = p.kept_count, a.groups = p.groups, a.threshold = p.threshold;
    a.methods[0] = p.methods[0], a.methods[1] = p.groups > 1 ? p.methods[1] : 0;
    a.stats = p.stats, a.status = p.status, a.raw = p.raw, a.fitted = p.fitted;
    for (int f0 = 0; f0 < p.kept_count; f0 += p.batch) {
        a.feature0 = f0;
        a.features = std::min(p.batch, p.kept_count - f0);
        a.scratch = p.scratch;
        hipLaunchKernelGGL(preprocess_fit_kernel, dim3(a.features), dim3(kFitThreads), 0, stream, a);
        IRX_HIP(hipGetLastError());
    }
}

void preprocess_transform(const PreprocessTransform &p, hipStream_t stream) {
    TransformArgs a{};
    a.x = p.x, a.x_f64 = p.x_f64, a.rows = p.rows, a.columns = p.columns, a.kept = p.kept;
    a.kept_count = p.kept_count, a.groups = p.groups, a.stats = p.stats, a.chunk_rows = p.chunk_rows;
    a.methods[0] = p.methods[0], a.methods[1] = p.groups > 1 ? p.methods[1] : 0;
    a.redo = p.redo, a.overflow = p.overflow, a.nonfinite = p.nonfinite, a.out = p.out;
    const long long total = p.rows * p.kept_count * p.groups;
    if (total <= 0) return;
    hipLaunchKernelGGL(preprocess_transform_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, stream, a);
    IRX_HIP(hipGetLastError());
}

void preprocess_gather(const float *group_rows, long long rows, int features, int members,
                       const unsigned *member_groups, const unsigned *orders, float *out, hipStream_t stream) {
    const long long total = rows * features * members;
    if (total <= 0) return;
    hipLaunchKernelGGL(preprocess_gather_kernel, dim3(ceil_div(total, 256)), dim3(256), 0, stream, group_rows, rows,
                       features, members, member_groups, orders, out);
    IRX_HIP(hipGetLastError());
}

}  // namespace irx
