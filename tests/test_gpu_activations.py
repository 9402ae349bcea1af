"""The parameterised activations (leaky_relu, hardtanh / relu6, elu / selu /
celu, softplus, hardswish, hardsigmoid, mish, logsigmoid, threshold and
relu's backward) and expm1 / log1p on the supa device: forward and autograd
backward bit-exact against the oracle's float32 arithmetic (bf16: that
result rounded once), with the CPU fallback disabled."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O

pytestmark = pytest.mark.gpu

CASES = [  # (name, torch forward, oracle act, params, flag for the backward)
    ("leaky_relu", lambda t: F.leaky_relu(t, 0.02), O.ACT_LEAKY_RELU, (0.02, 0.0, 0.0)),
    ("elu", F.elu, O.ACT_ELU, (1.0, 1.0, 1.0)),
    ("selu", torch.selu, O.ACT_ELU, (1.6732632423543772, 1.0507009873554805, 1.0)),
    ("celu", lambda t: F.celu(t, 0.7), O.ACT_ELU, (0.7, 1.0, 1.0 / 0.7)),
    ("softplus", F.softplus, O.ACT_SOFTPLUS, (1.0, 20.0, 0.0)),
    ("softplus_b2", lambda t: F.softplus(t, 2.0, 5.0), O.ACT_SOFTPLUS, (2.0, 5.0, 0.0)),
    ("hardswish", F.hardswish, O.ACT_HARDSWISH, (0.0, 0.0, 0.0)),
    ("hardsigmoid", F.hardsigmoid, O.ACT_HARDSIGMOID, (0.0, 0.0, 0.0)),
    ("mish", F.mish, O.ACT_MISH, (0.0, 0.0, 0.0)),
    ("logsigmoid", F.logsigmoid, O.ACT_LOG_SIGMOID, (0.0, 0.0, 0.0)),
]


def data(shape, seed, scale, dtype):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(shape, generator=g) * scale).to(dtype)
    x.view(-1)[:6] = torch.tensor([0.0, -3.0, 3.0, 20.0, -20.0, 1e-30]).to(dtype)
    return x


def want(arr, dtype):
    return torch.from_numpy(arr).to(dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name,fn,act,ps", CASES, ids=[c[0] for c in CASES])
def test_activation_forward_backward(name, fn, act, ps, dtype, no_fallback):
    x = data((513, 1031), 50, 6.0, dtype)
    g = data((513, 1031), 51, 1.0, dtype)
    dx = x.to("supa").requires_grad_()
    y = fn(dx)
    y.backward(g.to("supa"))
    xf, gf = x.float().numpy(), g.float().numpy()
    assert torch.equal(y.detach().cpu(), want(O.activation(act, xf, *ps), dtype)), name
    assert torch.equal(dx.grad.cpu(), want(O.activation_backward(act, gf, xf, *ps, 0), dtype)), name


def test_inplace_forms_and_relu_family(no_fallback):
    x = data((300, 77), 52, 4.0, torch.float32)
    g = data((300, 77), 53, 1.0, torch.float32)
    xf, gf = x.numpy(), g.numpy()
    # elu in place: its backward reads the output (is_result)
    a = x.to("supa").requires_grad_()
    b = a * 1.0
    F.elu(b, alpha=0.5, inplace=True).backward(g.to("supa"))
    y = O.activation(O.ACT_ELU, xf, 0.5, 1.0, 1.0)
    assert torch.equal(b.detach().cpu(), torch.from_numpy(y))
    assert torch.equal(a.grad.cpu(), torch.from_numpy(O.activation_backward(O.ACT_ELU, gf, y, 0.5, 1.0, 1.0, 1)))
    # relu: backward is threshold_backward(grad, result, 0)
    a = x.to("supa").requires_grad_()
    F.relu(a).backward(g.to("supa"))
    assert torch.equal(a.grad.cpu(), torch.from_numpy(np.where(xf > 0, gf, 0.0).astype(np.float32)))
    # relu6 = hardtanh(0, 6): clamp forward, hardtanh_backward
    a = x.to("supa").requires_grad_()
    r6 = F.relu6(a)
    r6.backward(g.to("supa"))
    assert torch.equal(r6.detach().cpu(), torch.clamp(x, 0, 6))
    assert torch.equal(a.grad.cpu(), torch.from_numpy(O.activation_backward(O.ACT_HARDTANH, gf, xf, 0.0, 6.0, 0.0)))
    # threshold forward / in place; leaky_relu / hardswish / hardsigmoid / mish in place
    assert torch.equal(F.threshold(x.to("supa"), 0.5, -2.0).cpu(),
                       torch.from_numpy(O.activation(O.ACT_THRESHOLD, xf, 0.5, -2.0)))
    for f_, act, ps in ((lambda t: F.leaky_relu_(t, 0.1), O.ACT_LEAKY_RELU, (0.1, 0, 0)),
                        (lambda t: F.hardswish(t, inplace=True), O.ACT_HARDSWISH, (0, 0, 0)),
                        (lambda t: F.hardsigmoid(t, inplace=True), O.ACT_HARDSIGMOID, (0, 0, 0)),
                        (lambda t: F.mish(t, inplace=True), O.ACT_MISH, (0, 0, 0))):
        t = x.to("supa")
        f_(t)
        assert torch.equal(t.cpu(), torch.from_numpy(O.activation(act, xf, *ps)))
    # integer threshold
    xi = torch.randint(-5, 5, (1000,))
    assert torch.equal(F.threshold(xi.to("supa"), 1, 7).cpu(), F.threshold(xi, 1, 7))


def test_expm1_log1p_and_foreach(no_fallback):
    x = data((4099,), 54, 5.0, torch.float32)
    z = x.abs() - 0.5
    dx, dz = x.to("supa"), z.to("supa")
    assert torch.equal(torch.expm1(dx).cpu(), torch.from_numpy(O.unary(O.EXPM1, x.numpy())))
    assert torch.equal(torch.log1p(dz).cpu(), torch.from_numpy(O.unary(O.LOG1P, z.numpy())))
    outs = torch._foreach_expm1([dx, dx[:100]])
    assert torch.equal(outs[1].cpu(), torch.from_numpy(O.unary(O.EXPM1, x[:100].numpy())))
    zs = [dz.clone(), dz[7:].clone()]
    torch._foreach_log1p_(zs)
    assert torch.equal(zs[1].cpu(), torch.from_numpy(O.unary(O.LOG1P, z[7:].numpy())))


def _dname(dtype):
    return {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]


@pytest.mark.parametrize("lam", [0.5, 0.3])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_shrink_forward_backward(dtype, lam, no_fallback):
    """hardshrink / softshrink and their backward against the oracle bit for
    bit (lambda in the storage type), including +-lambda, 0 and NaN inputs,
    and a non-contiguous input."""
    name = _dname(dtype)
    x = data((517, 129), 60, 1.0, dtype)
    lt = torch.tensor(lam).to(dtype).item()
    x.view(-1)[6:11] = torch.tensor([lt, -lt, float("nan"), 2 * lt, -0.0]).to(dtype)
    g = data((517, 129), 61, 1.0, dtype)
    for kind, fn in (("hardshrink", F.hardshrink), ("softshrink", F.softshrink)):
        for view in (lambda t: t, lambda t: t.t()):
            xs = view(x.to("supa")).detach().requires_grad_()
            y = fn(xs, lam)
            xf = view(x).float().numpy()
            assert np.array_equal(y.detach().cpu().float().numpy(), O.shrink(kind, xf, lam, name),
                                  equal_nan=True), kind
            y.backward(view(g.to("supa")))
            assert np.array_equal(xs.grad.cpu().float().numpy(),
                                  O.shrink_backward(view(g).float().numpy(), xf, lam, name)), kind
    with pytest.raises(RuntimeError, match="lambda must be greater or equal to 0"):
        F.softshrink(x.to("supa"), -0.5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("dim", [-1, 0, 1])
def test_glu_forward_backward(dim, dtype, no_fallback):
    """glu along each dim of a 3-d input (the halves are strided views) and
    its backward, against the oracle bit for bit; an odd halving dim is an
    error."""
    name = _dname(dtype)
    x = data((34, 18, 66), 62, 2.0, dtype)
    h = x.shape[dim] // 2
    xs = x.to("supa").requires_grad_()
    y = F.glu(xs, dim)
    a = x.narrow(dim, 0, h).float().numpy()
    b = x.narrow(dim, h, h).float().numpy()
    assert np.array_equal(y.detach().cpu().float().numpy(), O.glu(a, b, name))
    g = data(tuple(y.shape), 63, 1.0, dtype)
    y.backward(g.to("supa"))
    ga, gb = O.glu_backward(a, b, g.float().numpy(), name)
    got = xs.grad.cpu()
    assert np.array_equal(got.narrow(dim, 0, h).float().numpy(), ga)
    assert np.array_equal(got.narrow(dim, h, h).float().numpy(), gb)
    with pytest.raises(RuntimeError, match="Halving dimension must be even"):
        F.glu(torch.zeros(3, 5, device="supa", dtype=dtype), -1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape, nw", [((16,), 1), ((64, 33), 33), ((8, 6, 5, 7), 6), ((8, 6, 5, 7), 1)])
def test_prelu_forward_backward(shape, nw, dtype, no_fallback):
    """nn.PReLU: the forward and the input gradient against the oracle bit
    for bit; the weight gradient (the elementwise x g, summed by autograd to
    the weight's shape on the device) within the sum's float32 rounding."""
    name = _dname(dtype)
    x = data(shape, 64, 1.0, dtype)
    w = (torch.randn(nw, generator=torch.Generator().manual_seed(65)) * 0.3).abs().to(dtype)
    g = data(shape, 66, 1.0, dtype)
    xs = x.to("supa").requires_grad_()
    ws = w.to("supa").requires_grad_()
    y = F.prelu(xs, ws)
    wshape = [1] * len(shape)
    if nw > 1:
        wshape[1] = nw
    wf = w.float().numpy().reshape(wshape)
    assert np.array_equal(y.detach().cpu().float().numpy(), O.prelu(x.float().numpy(), wf, name))
    y.backward(g.to("supa"))
    gi, gw = O.prelu_backward(x.float().numpy(), wf, g.float().numpy(), name)
    assert np.array_equal(xs.grad.cpu().float().numpy(), gi)
    red = tuple(i for i in range(len(shape)) if i != 1 or nw == 1)
    want_w = gw.astype(np.float64).sum(axis=red).reshape(nw)
    tol = 1e-5 if dtype == torch.float32 else (2e-2 if dtype == torch.bfloat16 else 2e-3)
    np.testing.assert_allclose(ws.grad.cpu().float().numpy(), want_w, rtol=tol, atol=tol * np.abs(gw).sum() / nw)


def test_new_ops_on_empty_and_scalar_inputs(no_fallback):
    """Empty tensors through hardshrink / softshrink / glu / prelu and their
    backwards, special.xlog1py, scatter_ and _fused_sgd_ (an empty tensor in
    its list): empty results of the right shape, no launch
    errors; a 0-dim scatter_ target takes its one element."""
    e = torch.empty(0, 6, device="supa", requires_grad=True)
    for y in (F.hardshrink(e), F.softshrink(e), F.glu(e, -1), F.prelu(e, torch.ones(6, device="supa"))):
        assert y.shape[0] == 0
        y.sum().backward()
    assert torch.special.xlog1py(torch.empty(0, device="supa"), torch.empty(0, device="supa")).numel() == 0
    t = torch.zeros(3, device="supa")
    t.scatter_(0, torch.empty(0, dtype=torch.long, device="supa"), 1.0)
    assert torch.equal(t.cpu(), torch.zeros(3))
    z = torch.zeros((), device="supa")
    z.scatter_(0, torch.zeros((), dtype=torch.long, device="supa"), 2.5)
    assert float(z) == 2.5
    # (an all-empty list has no tensor to dispatch on, here as on any backend)
    p = [torch.empty(0, device="supa"), torch.ones(5, device="supa")]
    g = [torch.empty(0, device="supa"), torch.ones(5, device="supa")]
    torch._fused_sgd_(p, g, [], weight_decay=0.0, momentum=0.0, lr=0.5, dampening=0.0, nesterov=False,
                      maximize=False, is_first_step=False)
    assert torch.equal(p[1].cpu(), torch.full((5,), 0.5))
