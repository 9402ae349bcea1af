"""Shared numeric helpers for the tests (ulp distances, seeded inputs)."""
import numpy as np


def f32_ulp_dist(a, b):
    """Distance in float32 ulps between two float32 arrays (NaN == NaN is 0,
    NaN vs number is huge).  Uses the monotone integer mapping of IEEE bits."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    ia = np.where(ia < 0, -(ia & 0x7FFFFFFF), ia)
    ib = np.where(ib < 0, -(ib & 0x7FFFFFFF), ib)
    d = np.abs(ia - ib)
    na, nb = np.isnan(a), np.isnan(b)
    d = np.where(na & nb, 0, d)
    d = np.where(na ^ nb, 1 << 40, d)
    return d


def bf16_ulp_dist(a_bits, b_bits):
    """Distance in bfloat16 ulps between two uint16 bit-pattern arrays."""
    ia = np.asarray(a_bits, np.uint16).astype(np.int64)
    ib = np.asarray(b_bits, np.uint16).astype(np.int64)
    ia = np.where(ia >= 0x8000, -(ia & 0x7FFF), ia)
    ib = np.where(ib >= 0x8000, -(ib & 0x7FFF), ib)
    return np.abs(ia - ib)


def ulp_vs_exact(got_f32, exact_f64):
    """Error of float32 results against exact double values, in ulps of the
    correctly rounded result (subnormal ulp below the normal range)."""
    got = np.asarray(got_f32, np.float64)
    ex = np.asarray(exact_f64, np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        r = ex.astype(np.float32).astype(np.float64)
        _, e = np.frexp(np.where(np.isfinite(r), np.abs(r), np.float64(3.4e38)))
        ulp = np.ldexp(1.0, np.maximum(e - 24, -149))
        err = np.abs(got - ex) / ulp
    both_inf = np.isinf(got) & np.isinf(r) & (got == r)
    err = np.where(both_inf, 0.0, err)
    err = np.where(np.isnan(got) & np.isnan(ex), 0.0, err)
    return err


def sample_f32(n, seed, lo=-30.0, hi=30.0):
    """Random float32 values: uniform in [lo, hi] plus log-spread magnitudes."""
    rng = np.random.default_rng(seed)
    u = rng.uniform(lo, hi, n // 2).astype(np.float32)
    mag = np.exp(rng.uniform(np.log(1e-30), np.log(max(abs(lo), abs(hi))), n - n // 2))
    s = rng.choice([-1.0, 1.0], n - n // 2)
    v = (s * mag).astype(np.float32)
    v = v[(v >= lo) & (v <= hi)]
    return np.concatenate([u, v])


def f32_ulp(v):
    """ulp of float32 values of magnitude |v| (2^-149 at and below the
    subnormal range)."""
    a = np.abs(np.asarray(v, np.float64))
    e = np.frexp(np.where(np.isfinite(a), a, 3.4e38))[1]
    return np.where(a == 0, 2.0 ** -149, np.ldexp(1.0, np.maximum(e - 24, -149)))
