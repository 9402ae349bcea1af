"""gelu parity: the oracle (and through the bit-exact GPU tests, the device)
evaluates the reference's formula, and agrees with upstream aten CPU on the
configs' own seeded inputs at the 2-ulp bar except where a stated, derived
bound explains the gap.

The reference computes gelu in float32 as (upstream GeluKernel.cu, CPU
Gelu.h:34-41 and 61-65)
    'none':  (x * 0.5) * (1 + erf(x * M_SQRT1_2))
    'tanh':  (0.5 * x) * (1 + tanh(kBeta * (x + kKappa * x^3))),
             x^3 = (x * x) * x, x + kKappa * x^3 one fused multiply-add.
For x << 0 both cancel in 1 + erf / 1 + tanh: a one-ulp difference in the
rounded erf or tanh value reaches the output as 0.5 |x| ulp(E), many output
ulps.  That, and nothing else, is what the exemptions below allow.

Inputs: c1 is BASELINE configs[0] (seed 0, randn(4096, 4096) float32, the
first tensor drawn).  c2 is configs[1] (seed 0, x = randn(64, 2048, 4096)
bfloat16, then bias = randn(4096) * 0.02); its gelu input y = x + bias is
taken for the first [2048, 4096] slice of x (torch's CPU randn yields the
same prefix whatever the tensor size; the bias needs the whole draw)."""
import ctypes
import math
import os
import subprocess

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from scipy import special

import oracle as O
from helpers import f32_ulp, f32_ulp_dist, ulp_vs_exact

F32 = np.float32
ALPHA = F32(0.70710678118654752440)  # (float)M_SQRT1_2
BETA = F32(0.7978845608028654)       # (float)(M_SQRT2 * M_2_SQRTPI * 0.5)
KAPPA = F32(0.044715)


@pytest.fixture(scope="module")
def c1():
    g = torch.Generator().manual_seed(0)
    return torch.randn(4096, 4096, generator=g)


@pytest.fixture(scope="module")
def c2_slice():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 2048, 4096, dtype=torch.bfloat16, generator=g)
    bias = torch.randn(4096, generator=g) * 0.02
    y = x[0] + bias  # bf16 + f32 -> f32, as the c2 add
    del x
    assert y.dtype == torch.float32
    return y


def _fma32(a, b, c):
    """float32 fused multiply-add: the product of two float32 values is exact
    in float64 and the sum is rounded there, then once more to float32
    (double rounding can only matter at exact float32 midpoints)."""
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(F32)


def _gelu_cr(x, approx):
    """The reference formula in float32 with erf / tanh correctly rounded
    (float64 libm rounded once)."""
    x = np.asarray(x, F32)
    if approx == "none":
        e = special.erf((x * ALPHA).astype(np.float64)).astype(F32)
        return (x * F32(0.5)) * (F32(1) + e)
    inner = BETA * _fma32(KAPPA, (x * x) * x, x)
    t = np.tanh(inner.astype(np.float64)).astype(F32)
    return (F32(0.5) * x) * (F32(1) + t)


@pytest.mark.parametrize("approx, op", [("none", O.GELU), ("tanh", O.GELU_TANH)])
def test_oracle_is_the_reference_formula(c1, approx, op):
    """Bit-exact with the reference formula evaluated with correctly rounded
    erf / tanh, except where the oracle's erf / tanh (within 0.978 / 0.5031
    ulp, exhaustively) is not the correctly rounded value; there the two
    differ by one ulp of E, and the gap is that ulp carried through
    (x/2)(1 + E), plus at most one ulp of the rounded 1 + E."""
    x = c1.numpy().ravel()
    got = O.unary(op, x)
    ref = _gelu_cr(x, approx)
    if approx == "none":
        z = x * ALPHA
        e_or, e_cr = O.unary(O.ERF, z), special.erf(z.astype(np.float64)).astype(F32)
    else:
        inner = BETA * _fma32(KAPPA, (x * x) * x, x)
        e_or, e_cr = O.unary(O.TANH, inner), np.tanh(inner.astype(np.float64)).astype(F32)
    off = e_or != e_cr
    # measured on c1: erf 5.82 % (1.46 % over all binary32 inputs; c1's
    # arguments sit where the mid range's rounding is closest), tanh 0.056 %
    # (0.008 % over all inputs)
    assert off.mean() < (0.065 if approx == "none" else 1e-3)
    assert np.all(np.abs(e_or[off].astype(np.float64) - e_cr[off]) <= f32_ulp(e_cr[off]))
    assert np.array_equal(got[~off], ref[~off])
    gap = np.abs(got[off].astype(np.float64) - ref[off])
    e = e_cr[off].astype(np.float64)
    step = f32_ulp(e) + f32_ulp(1.0 + e)
    assert np.all(gap <= 1.5 * f32_ulp(ref[off]) + 0.5 * np.abs(x[off]) * step)


def _check_tanh_vs_cpu(x_t, op=O.GELU_TANH):
    """CPU: Gelu.h:43-51 with Sleef_tanhf16_u10 (within 1.0 ulp;
    vec512_float.h:516); the oracle's tanh is within 0.5031 ulp, so the two
    rounded tanh values T differ by at most one ulp(T).  Exempt: an element
    more than 2 ulp from the CPU whose gap is at most 2 ulp + 0.5 |x| ulp(T).
    op GELU_TANH_FAST_ALT: the other value the device's forward may return
    where tanh's quotient is within 2^-44 of a rounding boundary (there the
    exact tanh is within 0.5 + 2^-20 ulp of either neighbour, so the same
    bound holds)."""
    x = x_t.numpy().ravel()
    cpu = F.gelu(x_t, approximate="tanh").numpy().ravel()
    got = O.unary(op, x)
    d = f32_ulp_dist(got, cpu)
    far = d > 2
    inner = BETA * _fma32(KAPPA, (x * x) * x, x)
    T = O.unary(O.TANH, inner)
    bound = 2 * f32_ulp(cpu) + 0.5 * np.abs(x.astype(np.float64)) * f32_ulp(T)
    gap = np.abs(got.astype(np.float64) - cpu)
    assert np.all(gap[far] <= bound[far])
    return far.mean()


def _check_none_vs_cpu(x_t, got=None):
    """CPU: float32 gelu 'none' dispatches to oneDNN's eltwise gelu_erf
    (upstream Activation.cpp gelu_out_cpu, use_mkldnn); it, too, rounds an erf
    value and adds 1, and is itself more than 2 ulp from the exact function
    on about 7 % of N(0, 1) inputs (measured here, against float64).

    Two ranges, two checks:
    * x >= -1, where 1 + erf(x / sqrt2) >= 0.31 does not cancel: the oracle is
      within 2.7 ulp of the exact x Phi(x) (measured on c1: 2.64), and an
      element more than 2 ulp from the CPU is exempt only where the CPU is
      itself at least 0.9 ulp from the exact value (measured: every one of
      c1's 3 633 such elements; the closest is 0.908 ulp).
    * x < -1: the derived cancellation bound.  z = fl(x M_SQRT1_2) is within
      1.28 2^-24 relative of x / sqrt2 (rounding plus the float32 constant),
      which moves erf by at most (2/sqrt(pi)) |z| e^-z^2 1.28 2^-24; E rounds
      erf(z) within 0.978 ulp(E); 1 + E and the two products add at most
      1.5 ulp(y); the whole is carried through 0.5 |x| (1 + E).
    Returns the share of elements more than 2 ulp from the CPU."""
    x = x_t.numpy().ravel()
    cpu = F.gelu(x_t).numpy().ravel()
    if got is None:
        got = O.unary(O.GELU, x)
    xd = x.astype(np.float64)
    exact = 0.5 * xd * special.erfc(-xd / math.sqrt(2.0))
    far = f32_ulp_dist(got, cpu) > 2
    hi = x >= -1
    ours_ulp = ulp_vs_exact(got[hi], exact[hi])
    assert ours_ulp.max() <= 2.7, float(ours_ulp.max())
    cpu_ulp = ulp_vs_exact(cpu[hi], exact[hi])
    assert np.all(cpu_ulp[far[hi]] >= 0.9), int((cpu_ulp[far[hi]] < 0.9).sum())
    lo = ~hi
    z = (x[lo] * ALPHA).astype(np.float64)
    E = special.erf(z)
    ours = 0.5 * np.abs(xd[lo]) * (0.978 * f32_ulp(E) + 1.45 * 2.0 ** -24 * np.abs(z) * np.exp(-z * z)) \
        + 1.5 * f32_ulp(exact[lo])
    assert np.all(np.abs(got[lo] - exact[lo]) <= ours)
    return far.mean()


@pytest.mark.parametrize("op", [O.GELU_TANH, O.GELU_TANH_FAST_ALT])
def test_gelu_tanh_vs_cpu_c1(c1, op):
    assert _check_tanh_vs_cpu(c1, op) <= 1e-4  # measured 0.0046 %


@pytest.mark.parametrize("op", [O.GELU_TANH, O.GELU_TANH_FAST_ALT])
def test_gelu_tanh_vs_cpu_c2(c2_slice, op):
    assert _check_tanh_vs_cpu(c2_slice, op) <= 1e-4


def test_gelu_tanh_fast_alt_is_rare(c1, c2_slice):
    """The device forward's other neighbour occurs where tanh's quotient lies
    within 2^-44 of a binary32 rounding boundary: about 2^-19.5 of the
    elements (c1: 2^24 elements, c2's slice 2^23)."""
    for t in (c1, c2_slice):
        x = t.numpy().ravel()
        ref, alt = O.unary(O.GELU_TANH, x), O.unary(O.GELU_TANH_FAST_ALT, x)
        n = int((ref != alt).sum())
        assert 0 < n <= 64, n


def test_gelu_none_vs_cpu_c1(c1):
    # measured 5.93 % (5.77 % for the formula with a correctly rounded erf):
    # the formula's float32 cancellation for x < -1 on both sides
    assert _check_none_vs_cpu(c1) <= 0.065


@pytest.mark.parametrize("k", [2, -2, 4, -4])
def test_gelu_none_check_detects_a_changed_erf(c1, k, tmp_path):
    """The checks above fail for an oracle whose erf is off by k 2^-24
    relative (one ulp of erf values in [1/2, 1) per 2^-24, a one-ulp change
    at k = 2 for values in [1, 2)): a separate build of the oracle with
    OR_ERF_SCALE = 1 + k 2^-24."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    so = str(tmp_path / "liboracle_erf.so")
    subprocess.run(["gcc", "-O2", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-std=c11",
                    "-shared", f"-DOR_ERF_SCALE=(1.0f+({k})*0x1p-24f)", "-o", so,
                    os.path.join(root, "oracle", "oracle.c"), "-lm"], check=True)
    lib = ctypes.CDLL(so)
    x = np.ascontiguousarray(c1.numpy().ravel())
    got = np.empty_like(x)
    lib.or_unary_f32(ctypes.c_int(O.GELU), x.ctypes.data_as(ctypes.c_void_p), got.ctypes.data_as(ctypes.c_void_p),
                     ctypes.c_int64(x.size))
    assert not np.array_equal(got, O.unary(O.GELU, x))
    with pytest.raises(AssertionError):
        _check_none_vs_cpu(c1, got)


def test_gelu_opt_in_forms_are_accurate():
    """The opt-in forms avoid the cancellation: gelu_logerfc within 1.6 ulp of
    x Phi(x) for x >= 0 and 9 ulp down to -2; gelu_tanh_logistic within
    3 (1 + |v|) ulp of x / (1 + e^v), v = -2 b (x + k x^3) rounded in float32."""
    x = np.random.default_rng(3).standard_normal(1 << 20).astype(F32) * 2
    xd = x.astype(np.float64)
    from helpers import ulp_vs_exact
    err = ulp_vs_exact(O.unary(O.GELU_LOGERFC, x), xd * special.ndtr(xd))
    assert err[x >= 0].max() <= 1.6 and err[(x < 0) & (x > -2)].max() <= 9.0
    v = -2 * math.sqrt(2 / math.pi) * (xd + 0.044715 * xd ** 3)
    ex = xd / (1 + np.exp(v))
    keep = np.abs(ex) > 1e-30
    err = ulp_vs_exact(O.unary(O.GELU_TANH_LOGISTIC, x)[keep], ex[keep])
    assert np.all(err <= 3.0 * (1.0 + np.abs(v[keep])))
