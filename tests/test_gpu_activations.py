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
