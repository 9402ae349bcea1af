"""The reference's test/test_loss.py, case for case: nll_loss forward,
backward and weighted backward over every (shape, target, reduction) of its
params list (including (1000, 200000), (200000, 1000) and the 4-d
(2, 19, 512, 1024) -> nll_loss2d), its br200 lists, and cross_entropy
forward and backward over its cross-entropy lists, with its tolerances
(GetAccumulationRtolAtol, test_loss.py:133-146) and its comparison (the CPU
result, computed in float32 and cast to the input dtype for the gradients,
against the supa result).

The reference's forward tests draw float32 inputs whatever the dtype
parameter says (test_loss.py:152-169, 237-248), so those run once per case
here.  Inputs are seeded N(0, 1) (its torch.randn / create_random_tensor) and
targets uniform over the classes (its random_(C))."""
import math

import numpy as np
import pytest
import torch
import torch.nn as nn

pytestmark = pytest.mark.gpu

SUPA = "supa"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
RTOL = {torch.float32: 1.3e-6, torch.bfloat16: 1.6e-2, torch.float16: 1e-3}
ATOL = {torch.float32: 1e-5, torch.bfloat16: 1e-5, torch.float16: 1e-5}
PARAMS = [
    ((15, 5), (15,), "mean"), ((16, 1000), (16,), "mean"), ((16, 1000), (16,), "sum"),
    ((16, 1000), (16,), "none"), ((8732, 81), (8732,), "sum"), ((8732, 81), (8732,), "none"),
    ((1000, 200000), (1000,), "mean"), ((200000, 1000), (200000,), "mean"), ((200000, 1000), (200000,), "sum"),
    ((200000, 1000), (200000,), "none"), ((2, 19, 512, 1024), (2, 512, 1024), "none"),
]
NLL_BR200 = [((15, 5), (15,), torch.float32, "none"), ((512, 1024), (512,), torch.float32, "none")]
CE_PARAMS = [((1, 1000), (1,), "mean"), ((16, 1000), (16,), "mean"), ((16, 1000), (16,), "sum"),
             ((16, 1000), (16,), "none")]
CE_BR200 = [((1, 6), (1,), torch.float32, "none"), ((512, 1024), (512,), torch.float32, "none"),
            ((512, 1024), (512,), torch.float32, "sum"), ((512, 1024), (512,), torch.float32, "mean")]

_inputs = {}


def _x(shape):
    """The float32 N(0, 1) input of a shape, drawn once per shape (the long
    shapes hold 2e8 elements)."""
    if shape not in _inputs:
        g = torch.Generator().manual_seed(hash(shape) % (2 ** 31))
        _inputs[shape] = torch.randn(shape, generator=g)
    return _inputs[shape]


def _target(shape, C):
    g = torch.Generator().manual_seed((hash(shape) + C) % (2 ** 31))
    return torch.empty(shape, dtype=torch.long).random_(C, generator=g)


def _accumulation_tol(count, dtype):
    """test_loss.py:133-146: (atol, rtol)."""
    k1 = 4.0 if count <= 32 else 4.0 * (math.log2(count) - 4.0)
    if dtype == torch.bfloat16:
        return 0.001, 0.016
    return k1 * 1e-5, k1 * 1.3e-6


def ref_allclose(golden, compare, rtol, atol):
    golden, compare = golden.detach().cpu(), compare.detach().cpu()
    if golden.dtype == compare.dtype == torch.bfloat16:
        torch.testing.assert_close(compare, golden, rtol=rtol, atol=atol)
    else:
        np.testing.assert_allclose(golden.numpy(), compare.numpy(), rtol, atol)


@pytest.mark.parametrize("shape, tshape, reduce", PARAMS)
def test_nll_loss_forward(shape, tshape, reduce, no_fallback):
    """test_loss.py:149-169 (float32 input for every dtype parameter there)."""
    x = _x(shape)
    t = _target(tshape, shape[1])
    loss = nn.NLLLoss(reduction=reduce)
    ts = t.to(SUPA)
    y_cpu, y_supa = loss(x, t), loss(x.to(SUPA), ts)
    atol, rtol = _accumulation_tol(shape[0], torch.float32)
    if reduce == "none":
        atol, rtol = 1e-2, 1.3e-3
    ref_allclose(y_cpu, y_supa, rtol, atol)
    assert torch.equal(ts.cpu(), t)  # the target is not changed by the loss


def _nll_backward(shape, tshape, dtype, reduce, weighted):
    """test_loss.py:171-195 and 203-227: the CPU's float32 gradient cast to
    dtype against the supa gradient computed in dtype."""
    C = shape[1]
    xc = _x(shape).detach().to(dtype).requires_grad_(True)  # a fresh leaf, not the cached tensor
    xs = xc.detach().to(SUPA).requires_grad_(True)
    t = _target(tshape, C)
    w = torch.ones(C, dtype=dtype) if weighted else None
    loss = nn.NLLLoss(weight=w, reduction=reduce).float()
    y_cpu = loss(xc.float(), t)
    g_cpu = torch.ones_like(y_cpu, dtype=dtype)
    y_cpu.backward(g_cpu.float())
    loss_supa = loss.to(dtype).to(SUPA)
    ts = t.to(SUPA)
    y_supa = loss_supa(xs, ts)
    y_supa.backward(g_cpu.to(dtype).to(SUPA))
    atol, rtol = _accumulation_tol(shape[0], dtype)
    if reduce == "none":
        atol, rtol = 1e-5, 1.3e-6
    ref_allclose(xc.grad.to(dtype), xs.grad, rtol, atol)
    assert torch.equal(ts.cpu(), t)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape, tshape, reduce", PARAMS)
def test_nll_loss_backward(shape, tshape, reduce, dtype, no_fallback):
    _nll_backward(shape, tshape, dtype, reduce, weighted=False)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape, tshape, reduce", PARAMS)
def test_nll_loss_backward_weight(shape, tshape, reduce, dtype, no_fallback):
    _nll_backward(shape, tshape, dtype, reduce, weighted=True)


@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("shape, tshape, dtype, reduce", NLL_BR200)
def test_nll_loss_br200(shape, tshape, dtype, reduce, weighted, no_fallback):
    """test_loss.py:197-235."""
    _nll_backward(shape, tshape, dtype, reduce, weighted)


def _ce_forward(shape, tshape, reduce):
    x = _x(shape)
    t = _target(tshape, shape[1])
    loss = nn.CrossEntropyLoss(reduction=reduce)
    y_cpu, y_supa = loss(x, t), loss(x.to(SUPA), t.to(SUPA))
    ref_allclose(y_cpu, y_supa, RTOL[torch.float32], ATOL[torch.float32])


def _ce_backward(shape, tshape, dtype, reduce):
    xc = _x(shape).detach().to(dtype).requires_grad_(True)  # a fresh leaf, not the cached tensor
    xs = xc.detach().to(SUPA).requires_grad_(True)
    t = _target(tshape, shape[1])
    loss = nn.CrossEntropyLoss(reduction=reduce).float()
    y_cpu = loss(xc.float(), t)
    g_cpu = torch.ones_like(y_cpu, dtype=dtype)
    y_cpu.backward(g_cpu.float())
    y_supa = loss.to(dtype).to(SUPA)(xs, t.to(SUPA))
    y_supa.backward(g_cpu.to(SUPA))
    if dtype == torch.float32 or reduce == "mean":
        ref_allclose(xc.grad.to(dtype), xs.grad, RTOL[dtype], ATOL[dtype])
        return
    # bf16 / f16 with unit gradients: the decomposition (the reference
    # device's too) rounds log_softmax's output y to the dtype, which moves
    # exp(y) by up to |y| u relative (u: half an ulp, relative), past the
    # reference's rtol once p exceeds a few 1e-3.  So: within one ulp of the
    # device decomposition's arithmetic (upstream's softmax backward: float
    # math on the rounded y, rounded once; the CPU's reduced-precision kernels
    # round in between and are no yardstick here), and the float32 result
    # within the reference tolerance plus that rounding.
    x32 = xc.detach().float()
    y = torch.log_softmax(xs.detach(), 1).cpu().float()  # the forward output the backward reads
    gn = torch.zeros_like(y)
    gn[torch.arange(y.shape[0]), t] = -1.0
    emu = (gn - torch.exp(y) * gn.sum(1, keepdim=True)).to(dtype).float()
    got = xs.grad.cpu().float()
    mant = 7 if dtype == torch.bfloat16 else 10
    ulp = torch.exp2(torch.floor(torch.log2(emu.abs().clamp_min(2.0 ** -60))) - mant)
    assert bool(((got - emu).abs() <= ulp).all())
    u = 2.0 ** -(mant + 1)
    g32 = xc.grad.float()
    bound = ATOL[dtype] + RTOL[dtype] * got.abs() + torch.softmax(x32, 1) * torch.expm1(torch.log_softmax(x32, 1).abs() * u) \
        + g32.abs() * u
    assert bool(((got - g32).abs() <= bound).all())


@pytest.mark.parametrize("shape, tshape, reduce", CE_PARAMS)
def test_cross_entropy_forward(shape, tshape, reduce, no_fallback):
    """test_loss.py:237-255 (float32 input for every dtype parameter there)."""
    _ce_forward(shape, tshape, reduce)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape, tshape, reduce", CE_PARAMS)
def test_cross_entropy_backward(shape, tshape, reduce, dtype, no_fallback):
    """test_loss.py:258-283."""
    _ce_backward(shape, tshape, dtype, reduce)


@pytest.mark.parametrize("shape, tshape, dtype, reduce", CE_BR200)
def test_cross_entropy_br200(shape, tshape, dtype, reduce, no_fallback):
    """test_loss.py:250-256 and 280-283."""
    _ce_forward(shape, tshape, reduce)
    _ce_backward(shape, tshape, dtype, reduce)
