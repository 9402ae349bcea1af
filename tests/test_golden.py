"""The oracle against the committed golden vectors (tests/golden/, written by
tests/golden/make_golden.py from the upstream aten CPU kernels)."""
import os

import numpy as np
import pytest

import oracle as O
from helpers import f32_ulp_dist

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
    xa = np.abs(a.astype(np.float64))
    for op, key, slope in [(O.GELU, "gelu", 0.5e-6), (O.GELU_TANH, "gelu_tanh", 2.0 ** -24)]:
        ref = G[key].astype(np.float64)
        ulp = np.ldexp(1.0, np.maximum(np.frexp(np.abs(ref))[1] - 24, -149))
        assert np.all(np.abs(O.unary(op, a) - ref) <= 2 * ulp + slope * xa), key


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
