"""Pins the oracle's float32 primitives (oracle/oracle_math.h) against
double-precision math: erf and tanh exhaustively over every binary32 input
(tests/cpp/exhaustive_math.c), the others on random dense samples, edge
values and identities.

The same polynomials run on the device (csrc/kernels/devmath.h), so these
bounds are also the accuracy of the device primitives."""
import math
import os
import subprocess

import numpy as np
import pytest
from scipy import special

import oracle as O
from helpers import sample_f32, ulp_vs_exact

EDGES = np.array([0.0, -0.0, 1e-45, -1e-45, 1e-38, 1.17549435e-38, 0.5, 1.0, 2.0, 88.7, 88.72283, 89.0,
                  -87.3, -103.9, -104.0, 3.925, 0.921875, 0.55, 9.01, 20.0, -20.0, np.inf, -np.inf, np.nan],
                 np.float32)


@pytest.mark.parametrize(
    "op, ref, bound, lo, hi",
    [
        (O.EXP, np.exp, 1.01, -104.0, 89.0),
        (O.LOG, np.log, 0.94, 1e-30, 1e30),
        (O.ERF, special.erf, 0.978, -6.0, 6.0),
        (O.TANH, np.tanh, 0.5032, -12.0, 12.0),
    ],
)
def test_primitive_accuracy(op, ref, bound, lo, hi):
    if op == O.LOG:
        rng = np.random.default_rng(1)
        x = np.exp(rng.uniform(np.log(1e-44), np.log(3e38), 1 << 21)).astype(np.float32)
        x = np.concatenate([x, rng.uniform(0.5, 2.0, 1 << 20).astype(np.float32)])
    else:
        x = sample_f32(1 << 21, seed=op, lo=lo, hi=hi)
    got = O.unary(op, x)
    with np.errstate(all="ignore"):
        exact = ref(x.astype(np.float64))
    err = ulp_vs_exact(got, exact)
    assert err.max() <= bound, (op, float(x[np.argmax(err)]), float(err.max()))


def test_erf_tanh_exhaustive(tmp_path):
    """Every non-negative binary32 input below saturation (erf |x| < 4, tanh
    |x| < 10), the saturated range and the odd symmetry on a stride: erf
    within 0.978 ulp (1.455 % of results not correctly rounded), tanh within
    0.5031 ulp (0.008 % not correctly rounded)."""
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = tmp_path / "exhaustive_math"
    subprocess.run(["gcc", "-O2", "-march=x86-64-v3", "-ffp-contract=off", "-fno-fast-math", "-fopenmp",
                    "-std=c11", "-I", os.path.join(root, "oracle"), os.path.join(root, "tests", "cpp", "exhaustive_math.c"),
                    "-o", str(exe), "-lm"], check=True)
    r = subprocess.run([str(exe), "0.978", "0.5031"], capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = r.stdout.split("\n")
    assert lines[0].startswith("OK erf") and lines[1].startswith("OK tanh"), r.stdout
    notcr = float(lines[0].split("notcr=")[1].split()[0])
    assert notcr < 0.0146


def test_expm1_log1p_accuracy_and_edges():
    """expm1 reuses the exp reduction and polynomial; log1p adds the exact
    rounding error of 1 + z back.  Both within 2 ulp of double precision."""
    x = np.concatenate([sample_f32(1 << 21, seed=31, lo=-110.0, hi=89.0),
                        sample_f32(1 << 20, seed=32, lo=-1.0, hi=1.0),
                        np.float32([1e-30, -1e-30, 1e-8, -1e-8, 0.3466, -0.3466, 17.0, 24.0, 88.7])])
    with np.errstate(all="ignore"):
        ex = np.expm1(x.astype(np.float64))
    fin = np.isfinite(ex) & (np.abs(ex) < 3.4e38)
    assert ulp_vs_exact(O.unary(O.EXPM1, x)[fin], ex[fin]).max() <= 1.5
    z = np.concatenate([np.exp(np.random.default_rng(33).uniform(np.log(1e-38), np.log(3e38), 1 << 20)),
                        np.random.default_rng(34).uniform(-0.999999, 1.0, 1 << 20),
                        [1e-45, -1e-45, 6e-8, -6e-8, 1.0, -0.5, -0.75]]).astype(np.float32)
    assert ulp_vs_exact(O.unary(O.LOG1P, z), np.log1p(z.astype(np.float64))).max() <= 2.0
    # specials: expm1(0) = 0 and the tiny-argument identity, log1p(-1) = -inf, log1p(< -1) = nan
    e = O.unary(O.EXPM1, np.float32([0.0, -0.0, 1e-30, -200.0, np.inf, -np.inf, np.nan]))
    assert e[0] == 0.0 and e[2] == np.float32(1e-30) and e[3] == -1.0 and e[4] == np.inf and e[5] == -1.0
    assert np.isnan(e[6])
    l = O.unary(O.LOG1P, np.float32([0.0, 1e-30, -1.0, -2.0, np.inf, np.nan]))
    assert l[0] == 0.0 and l[1] == np.float32(1e-30) and l[2] == -np.inf and np.isnan(l[3]) and l[4] == np.inf
    assert np.isnan(l[5])


def test_gelu_tails():
    """Beyond |x| = 5.6 erf(x / sqrt2) rounds to +-1: gelu is x or -0 there,
    as upstream's; inf and NaN propagate."""
    for op in (O.GELU, O.GELU_TANH):
        tail = O.unary(op, np.float32([-6.0, -20.0, 6.0, 20.0, np.inf, np.nan]))
        assert tail[0] == 0.0 and np.signbit(tail[0]) and tail[1] == 0.0 and np.signbit(tail[1])
        assert tail[2] == 6.0 and tail[3] == 20.0 and tail[4] == np.inf and np.isnan(tail[5])


def test_primitive_edges():
    x = EDGES
    with np.errstate(all="ignore"):
        for op, ref in [(O.EXP, np.exp), (O.TANH, np.tanh), (O.ERF, special.erf)]:
            got = O.unary(op, x)
            ex = ref(x.astype(np.float64))
            np.testing.assert_array_equal(np.isnan(got), np.isnan(ex))
            fin = ~np.isnan(ex)
            assert ulp_vs_exact(got[fin], ex[fin]).max() <= 1.5
    # log specials: log(0) = -inf, log(<0) = nan, log(inf) = inf, log(1) = 0
    got = O.unary(O.LOG, np.array([0.0, -0.0, -1.0, np.inf, 1.0, np.nan], np.float32))
    assert got[0] == -np.inf and got[1] == -np.inf and np.isnan(got[2]) and got[3] == np.inf
    assert got[4] == 0.0 and np.isnan(got[5])
    # exp(0) == 1 exactly (the BCE-with-logits restatement relies on it)
    assert O.unary(O.EXP, np.array([0.0, -0.0], np.float32)).tolist() == [1.0, 1.0]


def test_activation_identities():
    x = np.linspace(-8, 8, 200001, dtype=np.float32)
    # odd functions
    np.testing.assert_array_equal(O.unary(O.ERF, -x), -O.unary(O.ERF, x))
    np.testing.assert_array_equal(O.unary(O.TANH, -x), -O.unary(O.TANH, x))
    # silu(x) - silu(-x) = x and gelu(x) - gelu(-x) = x, up to float rounding
    for op in (O.SILU, O.GELU, O.GELU_TANH):
        d = O.unary(op, x).astype(np.float64) - O.unary(op, -x).astype(np.float64)
        np.testing.assert_allclose(d, x, rtol=4e-7, atol=1e-7)
    # fixed points
    z = np.zeros(1, np.float32)
    assert O.unary(O.SIGMOID, z)[0] == 0.5
    for op in (O.GELU, O.GELU_TANH, O.SILU, O.TANH, O.ERF):
        assert O.unary(op, z)[0] == 0.0


@pytest.mark.parametrize("op, exact", [
    (O.SILU, lambda x: x / (1 + np.exp(-x))),
    (O.SIGMOID, lambda x: 1 / (1 + np.exp(-x))),
])
def test_activation_vs_exact(op, exact):
    """silu / sigmoid: within 3 ulp of the exact function wherever the exact
    value is at least 1e-30 in magnitude."""
    x = np.random.default_rng(7).standard_normal(1 << 20).astype(np.float32) * 3
    got = O.unary(op, x)
    ex = exact(x.astype(np.float64))
    keep = np.abs(ex) > 1e-30
    assert ulp_vs_exact(got[keep], ex[keep]).max() <= 3.0


def test_gelu_none_error_is_the_reference_formula_conditioning():
    """gelu 'none' evaluates the reference formula x*0.5*(1+erf(x/sqrt2)) in
    float32; its error against the exact function is bounded by the erf
    rounding scaled by |0.5 x|: |err| <= 2 ulp(y) + |0.5 x| * 2^-23."""
    x = np.random.default_rng(3).standard_normal(1 << 20).astype(np.float32) * 2
    got = O.unary(O.GELU, x).astype(np.float64)
    xd = x.astype(np.float64)
    ex = 0.5 * xd * special.erfc(-xd / math.sqrt(2))
    ulp = np.ldexp(1.0, np.maximum(np.frexp(np.abs(ex))[1] - 24, -149))
    assert np.all(np.abs(got - ex) <= 2 * ulp + np.abs(0.5 * xd) * 2.0 ** -23)


def test_quotient_by_a_constant_from_a_binary64_reciprocal():
    """The fused AdamW kernel rounds sqrt(v) / c (c = bias_correction2_sqrt, a
    per-tensor float32 constant in [2^-60, 1]) from the binary64 product
    sqrt(v) * RN64(1 / c).  Within 2^-52 of the exact quotient, that rounds
    to the IEEE float32 quotient for every float32 dividend: checked here on
    whole binades of dividends (every float32 in [1, 2) and [2^-70, 2^-69))
    for c of AdamW's first ten steps (beta2 = 0.999), and 2^20 random
    dividends over the whole normal range for c of steps 1..2000 (every 37th;
    beta2 = 0.999, 0.95) and 32 random c in [2^-60, 1]."""
    lo = np.arange(0x3F800000, 0x40000000, dtype=np.uint32).view(np.float32)
    tiny = np.arange(0x1C800000, 0x1D000000, dtype=np.uint32).view(np.float32)
    rng = np.random.default_rng(7)
    wide = np.exp2(rng.uniform(-125, 125, 1 << 20)).astype(np.float32)

    def check(c, s):
        c = np.float32(c)
        assert 2.0 ** -60 <= c <= 1.0
        got = (s.astype(np.float64) * (1.0 / np.float64(c))).astype(np.float32)
        want = s / c  # IEEE float32 division
        assert np.array_equal(got, want), (float(c), int((got != want).sum()))

    for step in range(1, 11):
        c = math.sqrt(1.0 - 0.999 ** step)
        check(c, lo)
        check(c, tiny)
    cs = [math.sqrt(1.0 - b ** k) for b in (0.999, 0.95) for k in range(1, 2001, 37)]
    cs += list(np.exp2(rng.uniform(-60, 0, 32)))
    for c in cs:
        check(c, wide)
