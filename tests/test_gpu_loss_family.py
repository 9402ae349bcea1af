"""The losses beside the path's mse / smooth_l1 / BCE-with-logits on the
supa device -- huber, binary_cross_entropy on probabilities, l1 (abs / sgn),
kl_div (xlogy) -- forward and backward, no CPU fallback, against upstream's
CPU kernels: the elementwise gradients bit for bit in float32 (the same op
sequence), terms with a logarithm within a few ulps (the device log is this
build's own, within 1 ulp of exact), reductions within rtol 1e-5 (float32) /
1e-2 (bf16)."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import f32_ulp_dist

pytestmark = pytest.mark.gpu


def seeded(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g) * scale


def tol(dtype):
    return dict(rtol=1e-5, atol=1e-6) if dtype == torch.float32 else dict(rtol=1e-2, atol=1e-2)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
@pytest.mark.parametrize("delta", [1.0, 0.3])
def test_huber(delta, reduction, dtype, no_fallback):
    x, t = seeded((257, 129), 90).to(dtype), seeded((257, 129), 91).to(dtype)
    dx = x.to("supa").requires_grad_()
    xc = x.clone().requires_grad_()
    got = F.huber_loss(dx, t.to("supa"), reduction=reduction, delta=delta)
    want = F.huber_loss(xc, t, reduction=reduction, delta=delta)
    if reduction == "none" and dtype == torch.float32:
        assert torch.equal(got.detach().cpu(), want.detach())
    else:
        torch.testing.assert_close(got.detach().cpu(), want.detach(), **tol(dtype))
    g = seeded(got.shape, 92).to(dtype)
    got.backward(g.to("supa"))
    want.backward(g)
    torch.testing.assert_close(dx.grad.cpu(), xc.grad, **tol(dtype))
    if dtype == torch.float32:
        # upstream's device kernel, in float32: (-norm g) delta, (norm g) delta, (norm x) g
        # (its vectorised CPU kernel forms norm (x / delta) g delta instead)
        xd = (x - t).numpy()
        gn = np.broadcast_to(g.numpy(), xd.shape).astype(np.float32)
        norm = np.float32(1.0 / x.numel()) if reduction == "mean" else np.float32(1.0)
        dl = np.float32(delta)
        ref = np.where(xd < -dl, ((-norm) * gn) * dl, np.where(xd > dl, (norm * gn) * dl, (norm * xd) * gn))
        assert np.array_equal(dx.grad.cpu().numpy(), ref.astype(np.float32))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
@pytest.mark.parametrize("weighted", [False, True])
def test_binary_cross_entropy(weighted, reduction, dtype, no_fallback):
    p = torch.sigmoid(seeded((300, 77), 93, 3.0)).to(dtype)
    p.view(-1)[:4] = torch.tensor([0.0, 1.0, 1e-30, 0.5]).to(dtype)  # the -100 clamp and the 1e-12 floor
    t = torch.rand(300, 77, generator=torch.Generator().manual_seed(94)).to(dtype)
    w = torch.rand(300, 77, generator=torch.Generator().manual_seed(95)).to(dtype) if weighted else None
    dp = p.to("supa").requires_grad_()
    pc = p.clone().requires_grad_()
    got = F.binary_cross_entropy(dp, t.to("supa"), weight=None if w is None else w.to("supa"), reduction=reduction)
    want = F.binary_cross_entropy(pc, t, weight=w, reduction=reduction)
    if reduction == "none" and dtype == torch.float32:
        assert f32_ulp_dist(got.detach().cpu().numpy(), want.detach().numpy()).max() <= 4
    else:
        torch.testing.assert_close(got.detach().cpu(), want.detach(), **tol(dtype))
    g = seeded(got.shape, 96).to(dtype)
    got.backward(g.to("supa"))
    want.backward(g)
    if dtype == torch.float32:
        assert torch.equal(dp.grad.cpu(), pc.grad)
    else:
        torch.testing.assert_close(dp.grad.cpu(), pc.grad, **tol(dtype))


def test_xlogy_and_kl_div(no_fallback):
    x = seeded((400, 50), 97).abs()
    y = seeded((400, 50), 98).abs()
    x.view(-1)[:3] = torch.tensor([0.0, 0.0, 2.0])
    y.view(-1)[:3] = torch.tensor([0.0, float("nan"), float("nan")])
    got = torch.xlogy(x.to("supa"), y.to("supa")).cpu().numpy()
    want = torch.xlogy(x, y).numpy()
    assert f32_ulp_dist(got, want).max() <= 2
    assert got[0, 0] == 0.0 and np.isnan(got[0, 1]) and np.isnan(got[0, 2])
    assert f32_ulp_dist(torch.xlogy(x.to("supa"), 3.0).cpu().numpy(), torch.xlogy(x, 3.0).numpy()).max() <= 2
    assert f32_ulp_dist(torch.xlogy(2.0, y.to("supa")).cpu().numpy(), torch.xlogy(2.0, y).numpy()).max() <= 2
    logits = seeded((64, 100), 99)
    target = F.softmax(seeded((64, 100), 100), -1)
    for log_target in (False, True):
        tt = target.log() if log_target else target
        dl = logits.to("supa").requires_grad_()
        lc = logits.clone().requires_grad_()
        got = F.kl_div(F.log_softmax(dl, -1), tt.to("supa"), reduction="batchmean", log_target=log_target)
        want = F.kl_div(F.log_softmax(lc, -1), tt, reduction="batchmean", log_target=log_target)
        torch.testing.assert_close(got.detach().cpu(), want.detach(), rtol=1e-5, atol=1e-6)
        got.backward()
        want.backward()
        torch.testing.assert_close(dl.grad.cpu(), lc.grad, rtol=1e-4, atol=1e-7)


@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
def test_l1_loss(reduction, no_fallback):
    x, t = seeded((513, 33), 101), seeded((513, 33), 102)
    x.view(-1)[0] = t.view(-1)[0]  # zero difference: sgn 0
    dx = x.to("supa").requires_grad_()
    xc = x.clone().requires_grad_()
    got = F.l1_loss(dx, t.to("supa"), reduction=reduction)
    want = F.l1_loss(xc, t, reduction=reduction)
    torch.testing.assert_close(got.detach().cpu(), want.detach(), rtol=1e-5, atol=1e-6)
    got.sum().backward()
    want.sum().backward()
    assert torch.equal(dx.grad.cpu(), xc.grad)


_LOSS16 = {"mse": lambda a, b, red, beta: F.mse_loss(a, b, reduction=red),
           "smooth_l1": lambda a, b, red, beta: F.smooth_l1_loss(a, b, reduction=red, beta=beta),
           "huber": lambda a, b, red, beta: F.huber_loss(a, b, reduction=red, delta=beta)}


@pytest.mark.parametrize("beta", [1.0, 0.3])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", ["mse", "smooth_l1", "huber"])
def test_loss_16bit_bit_exact(name, dtype, beta, no_fallback):
    """mse / smooth_l1 / huber on bf16 and f16 operands against the oracle's
    16-bit rule (upstream's device kernels compute in scalar_t: the difference
    is rounded to the type, and so is every operation of the gradient):
    per-element forward and every gradient bit for bit, the fused sum / mean
    within one ulp of the type (float32 summation order)."""
    if name == "mse" and beta != 1.0:
        pytest.skip("mse has no beta")
    tname = "bf16" if dtype == torch.bfloat16 else "f16"
    g = torch.Generator().manual_seed(140)
    shape = (257, 129)
    x = ((torch.rand(shape, generator=g) * 2 - 1) * 1.25).to(dtype)
    t = ((torch.rand(shape, generator=g) * 2 - 1) * 1.25).to(dtype)
    gr = torch.rand(shape, generator=g).to(dtype)
    xf, tf, gf = x.float().numpy(), t.float().numpy(), gr.float().numpy()
    fn = _LOSS16[name]
    got = fn(x.to("supa"), t.to("supa"), "none", beta).cpu().float().numpy()
    assert np.array_equal(got, O.loss_16(name, xf, tf, tname, "none", beta))
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    for red in ("mean", "sum"):
        got = float(fn(x.to("supa"), t.to("supa"), red, beta))
        want = float(O.loss_16(name, xf, tf, tname, red, beta))
        assert abs(got - want) <= ulp * abs(want), (red, got, want)
    for red in ("none", "mean", "sum"):
        dx = x.to("supa").requires_grad_()
        y = fn(dx, t.to("supa"), red, beta)
        y.backward(gr.to("supa") if red == "none" else None)
        want = O.loss_backward_16(name, gf if red == "none" else 1.0, xf, tf, tname, red, beta)
        assert np.array_equal(dx.grad.cpu().float().numpy(), want), red


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_xlog1py(dtype, no_fallback):
    """special.xlog1py (Tensor, Tensor / Scalar forms, out=) against the
    oracle bit for bit, its special cases included."""
    name = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]
    x = seeded((333, 65), 103).to(dtype)
    y = (seeded((333, 65), 104).abs() * 3 - 0.9).to(dtype)
    x.view(-1)[:4] = torch.tensor([0.0, 0.0, 2.0, 1.5]).to(dtype)
    y.view(-1)[:4] = torch.tensor([-1.0, float("nan"), float("nan"), -1.0]).to(dtype)
    xf, yf = x.float().numpy(), y.float().numpy()
    got = torch.special.xlog1py(x.to("supa"), y.to("supa")).cpu().float().numpy()
    assert np.array_equal(got, O.xlog1py(xf, yf, name), equal_nan=True)
    got = torch.special.xlog1py(x.to("supa"), 0.5).cpu().float().numpy()
    assert np.array_equal(got, O.xlog1py(xf, np.float32(0.5), name), equal_nan=True)
    got = torch.special.xlog1py(2.0, y.to("supa")).cpu().float().numpy()
    assert np.array_equal(got, O.xlog1py(np.float32(2.0), yf, name), equal_nan=True)
    out = torch.empty(0, dtype=dtype, device="supa")
    torch.special.xlog1py(x.to("supa"), y.to("supa"), out=out)
    assert np.array_equal(out.cpu().float().numpy(), O.xlog1py(xf, yf, name), equal_nan=True)
