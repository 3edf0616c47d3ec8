"""Oracle for TabICL's numeric preprocessing: a NumPy float64 restatement of
the reference's fit and transform, for tests only.

TEST INFRASTRUCTURE. Only tests/ may import this module, as the checker of
the GPU preprocessing (ironicl_amd/csrc/preprocess.hip); nothing in the
product calls it.

It follows, function by function:
- scale.rs (src/preprocess/scale.rs): mean_variance, is_constant,
  standard_scaler, standard_clip, clip_standardized, outlier_bounds,
  clamp_outlier;
- yeo_johnson.rs (src/preprocess/yeo_johnson.rs:21-243): yeo_johnson,
  log_variance_of_powers, log_likelihood, fminbound, normmax, fit_power;
- preprocess.rs (src/models/tabicl_v2/preprocess.rs:223-296): fit_feature,
  Normalization::value / transform (with the overflow fallback).

Pinned by the reference's golden fixtures (tests/golden/preprocessing/, from
the reference's tests/fixtures/): SciPy 1.18's yeojohnson_llf and
yeojohnson_normmax, scikit-learn 1.9's PowerTransformer, and TabICL 2.1.1's
preprocessed training and query rows. Sums are NumPy's (pairwise), not the
reference's serial loops, so results agree to rounding.
"""

from __future__ import annotations

import math

import numpy as np

EPS = np.finfo(np.float64).eps


def mean_variance(v: np.ndarray, ddof: int) -> tuple[float, float]:
    m = float(np.sum(v) / len(v))
    return m, float(np.sum((v - m) * (v - m)) / (len(v) - ddof))


def is_constant(variance: float, mean: float, rows: int) -> bool:
    n = float(rows)
    bound = n * mean * EPS
    return variance <= n * EPS * variance + bound * bound


def standard_scaler(v: np.ndarray) -> tuple[float, float]:
    n = float(len(v))
    mean = float(np.sum(v) / n)
    d = v - mean
    correction, squares = float(np.sum(d)), float(np.sum(d * d))
    variance = (squares - correction * correction / n) / n
    return mean, (1.0 if is_constant(variance, mean, len(v)) else math.sqrt(variance))


def standard_clip(v: np.ndarray) -> tuple[float, float]:
    m, var = mean_variance(v, 0)
    return m, math.sqrt(var) + 1e-6


def clip_standardized(v, mean, scale):
    return np.clip((v - mean) / scale, -100.0, 100.0)


def outlier_bounds(v: np.ndarray, threshold: float) -> tuple[float, float]:
    def bounds(values):
        if len(values) < 2:
            return math.nan, math.nan
        c, var = mean_variance(values, 1)
        spread = threshold * max(math.sqrt(var), 1e-6)
        return c - spread, c + spread

    lo, hi = bounds(v)
    return bounds(v[(v >= lo) & (v <= hi)])


def clamp_outlier(v, lower, upper):
    low = np.maximum(v, lower - np.log1p(np.abs(v)))
    return np.minimum(low, upper + np.log1p(np.abs(low)))


def yeo_johnson(x, lam: float):
    x = np.asarray(x, dtype=np.float64)
    out = np.empty_like(x)
    pos = x >= 0
    if abs(lam) < EPS:
        out[pos] = np.log1p(x[pos])
    else:
        out[pos] = np.expm1(lam * np.log1p(x[pos])) / lam
    if abs(lam - 2.0) > EPS:
        out[~pos] = -np.expm1((2.0 - lam) * np.log1p(-x[~pos])) / (2.0 - lam)
    else:
        out[~pos] = -np.log1p(-x[~pos])
    return out


def _log_variance_of_powers(logs: np.ndarray, power: float) -> float:
    if abs(power) < EPS:
        return math.log(mean_variance(logs, 0)[1])
    largest = float(np.max(power * logs))
    shifted = np.exp(power * logs - largest)
    return math.log(mean_variance(shifted, 0)[1]) + 2.0 * largest - 2.0 * math.log(abs(power))


def log_likelihood(data: np.ndarray, lam: float) -> float:
    with np.errstate(all="ignore"):
        if np.all(data >= 0):
            lv = _log_variance_of_powers(np.log1p(data), lam)
        elif np.all(data < 0):
            lv = _log_variance_of_powers(np.log1p(-data), 2.0 - lam)
        else:
            lv = math.log(mean_variance(yeo_johnson(data, lam), 0)[1])
        jacobian = float(np.sum(np.sign(data) * np.log1p(np.abs(data))))
        return -len(data) / 2.0 * lv + (lam - 1.0) * jacobian


def fminbound(f, a: float, b: float, xatol: float = 1.48e-8, maxfun: int = 500) -> float:
    """SciPy's bounded Brent search (yeo_johnson.rs:74-163)."""
    sqrt_eps = math.sqrt(2.2e-16)
    golden_mean = 0.5 * (3.0 - math.sqrt(5.0))
    sign = lambda v: -1.0 if v < 0 else 1.0
    fulc = a + golden_mean * (b - a)
    nfc = xf = fulc
    rat = e = 0.0
    fx = f(xf)
    calls = 1
    ffulc = fnfc = fx
    xm = 0.5 * (a + b)
    tol1 = sqrt_eps * abs(xf) + xatol / 3.0
    tol2 = 2.0 * tol1
    while abs(xf - xm) > (tol2 - 0.5 * (b - a)):
        golden = True
        if abs(e) > tol1:
            golden = False
            r = (xf - nfc) * (fx - ffulc)
            q = (xf - fulc) * (fx - fnfc)
            p = (xf - fulc) * q - (xf - nfc) * r
            q = 2.0 * (q - r)
            if q > 0.0:
                p = -p
            q = abs(q)
            r = e
            e = rat
            if abs(p) < abs(0.5 * q * r) and p > q * (a - xf) and p < q * (b - xf):
                rat = p / q
                x = xf + rat
                if (x - a) < tol2 or (b - x) < tol2:
                    rat = tol1 * sign(xm - xf)
            else:
                golden = True
        if golden:
            e = a - xf if xf >= xm else b - xf
            rat = golden_mean * e
        x = xf + sign(rat) * max(abs(rat), tol1)
        fu = f(x)
        calls += 1
        if fu <= fx:
            if x >= xf:
                a = xf
            else:
                b = xf
            fulc, ffulc = nfc, fnfc
            nfc, fnfc = xf, fx
            xf, fx = x, fu
        else:
            if x < xf:
                a = x
            else:
                b = x
            if fu <= fnfc or nfc == xf:
                fulc, ffulc = nfc, fnfc
                nfc, fnfc = x, fu
            elif fu <= ffulc or fulc == xf or fulc == nfc:
                fulc, ffulc = x, fu
        xm = 0.5 * (a + b)
        tol1 = sqrt_eps * abs(xf) + xatol / 3.0
        tol2 = 2.0 * tol1
        if calls >= maxfun:
            break
    return xf


def normmax(x: np.ndarray) -> float:
    """yeojohnson_normmax (yeo_johnson.rs:170-208)."""
    if np.all(x == 0.0):
        return 1.0
    largest = float(np.max(np.abs(x)))
    log1p_max_x = math.log1p(20.0 * largest)
    log_eps = math.log(EPS)
    log_tiny = (math.log(np.finfo(np.float64).tiny) - log_eps) / 2.0
    log_max = (math.log(np.finfo(np.float64).max) + log_eps) / 2.0
    lower, upper = log_tiny / log1p_max_x, log_max / log1p_max_x
    if np.all(x < 0):
        lower, upper = 2.0 - upper, 2.0 - lower
    elif np.any(x < 0):
        lower, upper = max(lower, 2.0 - upper), min(upper, 2.0 - lower)
    if not (math.isfinite(lower) and math.isfinite(upper)) or lower > upper:
        raise ValueError("Yeo-Johnson bounds are not finite")

    def nll(lam):
        v = log_likelihood(x, lam)
        return math.inf if math.isinf(v) else -v

    return fminbound(nll, lower, upper)


def fit_power(values: np.ndarray) -> tuple[float, float, float, np.ndarray]:
    """fit_power (yeo_johnson.rs:219-243): lambda, mean, scale and the fitted values."""
    m, var = mean_variance(values, 0)
    if is_constant(var, m, len(values)):
        lam, out = 1.0, values.copy()
    else:
        lam = normmax(values)
        out = yeo_johnson(values, lam)
    if not np.all(np.isfinite(out)):
        raise ValueError("the power transform of the training data is not finite")
    mean, scale = standard_scaler(out)
    return lam, mean, scale, (out - mean) / scale


def fit_feature(values: np.ndarray, methods: list[str], threshold: float) -> list[np.ndarray]:
    """fit_feature (preprocess.rs:259-296): per method the 6 (none) or 9
    (power) statistics."""
    mean, scale = standard_clip(values)
    s = clip_standardized(values, mean, scale)
    minimum, maximum = float(np.min(s)), float(np.max(s))
    out = []
    for method in methods:
        if method == "none":
            lower, upper = outlier_bounds(s, threshold)
            st = [mean, scale, minimum, maximum, lower, upper]
        else:
            lam, pm, ps, fitted = fit_power(s)
            lower, upper = outlier_bounds(fitted, threshold)
            st = [mean, scale, minimum, maximum, lower, upper, lam, pm, ps]
        if not all(math.isfinite(v) for v in st):
            raise ValueError("Training data produced non-finite preprocessing statistics")
        out.append(np.array(st))
    return out


def fit(x: np.ndarray, kept: list[int], methods: list[str], threshold: float) -> np.ndarray:
    """Statistics [groups, 9, kept] of every kept column (power slots 0 for none)."""
    x = np.asarray(x, dtype=np.float64)
    stats = np.zeros((len(methods), 9, len(kept)))
    for k, col in enumerate(kept):
        for g, st in enumerate(fit_feature(x[:, col], methods, threshold)):
            stats[g, : len(st), k] = st
    return stats


def transform_group(x: np.ndarray, kept: list[int], method: str, stats: np.ndarray) -> np.ndarray:
    """Normalization::transform (preprocess.rs:223-254) of one group, one batch:
    FP32 [rows, kept], redone clipped to the training range when the power
    transform overflows anywhere in the batch."""
    v0 = np.asarray(x, dtype=np.float64)[:, kept]
    mean, scale, minimum, maximum, lower, upper, lam, pm, ps = stats

    def fill(clip: bool):
        v = clip_standardized(v0, mean, scale)
        if method == "power":
            if clip:
                v = np.minimum(np.maximum(v, minimum), maximum)
            with np.errstate(all="ignore"):
                cols = [yeo_johnson(v[:, k], lam[k]) for k in range(v.shape[1])]
            v = np.stack(cols, axis=1) if cols else v
            if not np.all(np.isfinite(v)):
                return None
            v = (v - pm) / ps
        return clamp_outlier(v, lower, upper).astype(np.float32)

    out = fill(False)
    if out is None:
        out = fill(True)
    if out is None:
        raise ValueError("the power transform overflows even within the training range")
    if not np.all(np.isfinite(out)):
        raise ValueError("Preprocessing produced non-finite FP32 values")
    return out
