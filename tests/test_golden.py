"""The oracle against the committed golden vectors (tests/golden/, written by
tests/golden/make_golden.py from the upstream aten CPU kernels)."""
import os

import numpy as np
import pytest

from scipy import special

import oracle as O
from helpers import f32_ulp, f32_ulp_dist

G = np.load(os.path.join(os.path.dirname(__file__), "golden", "golden_cpu_aten.npz"))


def test_binary_exact():
    a, b = G["a"], G["b"]
    assert np.array_equal(O.binary(O.ADD, a, b), G["add"])
    assert np.array_equal(O.binary(O.ADD, a, b, 2.5), G["add_alpha"])
    assert np.array_equal(O.binary(O.MUL, a, b), G["mul"])
    assert np.array_equal(O.binary(O.DIV, a, b), G["div"])
    assert np.array_equal(O.binary(O.DIV_FLOOR, a, b), G["div_floor"])


def test_activations():
    a = G["a"]
    for op, key in [(O.SILU, "silu"), (O.SIGMOID, "sigmoid"), (O.TANH, "tanh")]:
        assert f32_ulp_dist(O.unary(op, a), G[key]).max() <= 2, key
    # gelu: 2 ulp, except where the float32 cancellation of 1 + erf / 1 + tanh
    # carries a one-ulp difference of the rounded erf / tanh value into the
    # output (the attribution of tests/test_gelu_parity.py: for 'tanh' one
    # ulp of T = tanh(inner), for 'none' our derived bound plus the CPU's own
    # distance from the exact function)
    x = a.astype(np.float64)
    ref = G["gelu_tanh"]
    got = O.unary(O.GELU_TANH, a)
    inner = np.float32(0.7978845608028654) * ((np.float32(0.044715) * ((a * a) * a)).astype(np.float64) + x).astype(np.float32)
    far = f32_ulp_dist(got, ref) > 2
    bound = 2 * f32_ulp(ref) + 0.5 * np.abs(x) * f32_ulp(O.unary(O.TANH, inner))
    assert far.mean() <= 1e-3 and np.all(np.abs(got - ref.astype(np.float64))[far] <= bound[far])
    ref = G["gelu"]
    got = O.unary(O.GELU, a)
    exact = 0.5 * x * special.erfc(-x / np.sqrt(2.0))
    z = x * np.float32(0.70710678118654752440)
    ours = 0.5 * np.abs(x) * (0.978 * f32_ulp(special.erf(z)) + 1.45 * 2.0 ** -24 * np.abs(z) * np.exp(-z * z)) \
        + 1.5 * f32_ulp(exact)
    far = f32_ulp_dist(got, ref) > 2
    gap = np.abs(got - ref.astype(np.float64))
    assert far.mean() <= 0.08 and np.all(gap[far] <= ours[far] + np.abs(ref - exact)[far])


def test_log_softmax_and_cross_entropy():
    x = G["lsm_x"]
    np.testing.assert_allclose(O.log_softmax(x), G["lsm"], rtol=1e-5, atol=1e-5)
    lp = O.log_softmax(x)
    t = G["ce_t"]
    out, tw = O.nll_loss(lp, t, None, "mean", -100)
    np.testing.assert_allclose(out, G["ce"], rtol=1e-5)
    gn = O.nll_loss_backward(np.ones(1, np.float32), t, x.shape[0], x.shape[1], tw, None, "mean", -100)
    np.testing.assert_allclose(O.log_softmax_backward(gn, lp), G["ce_grad"], rtol=1e-5, atol=1e-8)


@pytest.mark.parametrize("red", ["none", "mean", "sum"])
def test_losses(red):
    x, t, tb, pw = G["loss_x"], G["loss_t"], G["loss_tb"], G["loss_pw"]
    np.testing.assert_allclose(O.loss(O.MSE, x, t, reduction=red), G[f"mse_{red}"], rtol=1e-5)
    np.testing.assert_allclose(O.loss(O.SMOOTH_L1, x, t, reduction=red, beta=1.0), G[f"sl1_{red}"], rtol=1e-5,
                               atol=1e-7)
    np.testing.assert_allclose(O.loss(O.BCE_LOGITS, x, tb, pw, reduction=red), G[f"bce_{red}"], rtol=1e-5)


def test_adamw_ten_steps():
    p = G["adam_p0"].copy()
    g = G["adam_g"].copy()
    m, v = np.zeros_like(p), np.zeros_like(p)
    for s in range(1, 11):
        O.adamw_step(p, g, m, v, float(s), 1e-4, 0.9, 0.999, 0.01, 1e-8)
    np.testing.assert_allclose(p, G["adam_p10"], rtol=1e-5, atol=1e-9)
