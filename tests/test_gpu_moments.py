"""var / std / var_mean / std_mean with a correction on the supa device,
each row against the float64 oracle (rtol 1e-5 for float32 and float64
results at these sizes, 1e-2 for a bfloat16 result) and the layout against
upstream's CPU kernels: one dim, several dims, every element, keepdim, long
rows that take two launches, the degrees-of-freedom edge cases and the
backward of a hand-written LayerNorm."""
import math
import warnings

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

RTOL = {torch.float32: 1e-5, torch.float64: 1e-5, torch.bfloat16: 1e-2, torch.float16: 1e-3}


def rows_of(x, dims):
    keep = [d for d in range(x.dim()) if d not in dims]
    inner = int(np.prod([x.shape[d] for d in dims]))
    return x.double().permute(keep + list(dims)).reshape(-1, inner), [x.shape[d] for d in keep]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("correction", [0, 1, 2.5])
def test_var_std_mean_over_dims(dtype, correction, no_fallback):
    g = torch.Generator().manual_seed(31 + int(correction * 2))
    x = (torch.randn(5, 41, 131, generator=g) * 2 + 3).to(dtype)
    dx = x.to("supa")
    rtol = RTOL[dtype]
    for dim, keepdim in [(-1, False), (0, True), ((0, 2), False), (None, False), ((2, 1, 0), True)]:
        dims = tuple(range(3)) if dim is None else ((dim,) if isinstance(dim, int) else dim)
        dims = tuple(sorted(d % 3 for d in dims))
        rows, oshape = rows_of(x, dims)
        ref = [O.moments(r.numpy(), correction) for r in rows]
        rv = np.array([v for v, _ in ref]).reshape(oshape)
        rm = np.array([m for _, m in ref]).reshape(oshape)
        v = torch.var(dx, dim=dim, correction=correction, keepdim=keepdim)
        s = torch.std(dx, dim=dim, correction=correction, keepdim=keepdim)
        v2, m2 = torch.var_mean(dx, dim=dim, correction=correction, keepdim=keepdim)
        s2, m3 = torch.std_mean(dx, dim=dim, correction=correction, keepdim=keepdim)
        want = torch.var(x.double(), dim=dim, correction=correction, keepdim=keepdim)
        for t in (v, s, v2, m2, s2, m3):
            assert t.dtype == dtype and t.shape == want.shape
        np.testing.assert_allclose(v.double().cpu().reshape(rv.shape).numpy(), rv, rtol=rtol)
        np.testing.assert_allclose(s.double().cpu().reshape(rv.shape).numpy(), np.sqrt(rv), rtol=rtol)
        np.testing.assert_allclose(m2.double().cpu().reshape(rm.shape).numpy(), rm, rtol=rtol)
        assert torch.equal(v2.cpu(), v.cpu()) and torch.equal(s2.cpu(), s.cpu()) and torch.equal(m2.cpu(), m3.cpu())
        torch.testing.assert_close(v.double().cpu(), want, rtol=rtol, atol=0)


def test_var_long_rows_two_launches(no_fallback):
    """Rows over 65536 elements (few of them) merge per-chunk Welford
    triples in a second launch; a large mean over a small spread checks that
    the merge keeps the deviation form (a sum of squares would cancel)."""
    g = torch.Generator().manual_seed(57)
    x = torch.randn(3, 300007, generator=g) * 0.01 + 1000.0
    dx = x.to("supa")
    v, m = torch.var_mean(dx, dim=1)
    ref = [O.moments(r.numpy(), 1) for r in x.double()]
    np.testing.assert_allclose(v.double().cpu().numpy(), [a for a, _ in ref], rtol=1e-5)
    np.testing.assert_allclose(m.double().cpu().numpy(), [b for _, b in ref], rtol=1e-6)
    whole = torch.var(dx).item()
    assert whole == pytest.approx(O.moments(x.double().numpy(), 1)[0], rel=1e-5)


def test_var_edges(no_fallback):
    x = torch.randn(4, 3)
    dx = x.to("supa")
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        got = torch.var(dx, dim=1, correction=5).cpu()  # n <= correction: M2 / 0
        assert torch.equal(got, torch.var(x, dim=1, correction=5))
        one = torch.var(torch.tensor([2.0], device="supa")).item()  # 0 / 0
        assert math.isnan(one)
        e = torch.var_mean(torch.empty(0, 3, device="supa"), dim=0)
        assert all(torch.isnan(t.cpu()).all() for t in e) and e[0].shape == (3,)
    assert torch.var(torch.empty(0, 3, device="supa"), dim=1).shape == (0,)
    assert torch.std(torch.tensor(5.0, device="supa"), correction=0).item() == 0.0
    y = torch.randn(6, 9)
    y[2, 4] = float("nan")
    got = torch.std(y.to("supa"), dim=1).cpu()
    assert torch.isnan(got[2]) and not torch.isnan(got[[0, 1, 3, 4, 5]]).any()
    out = torch.empty(9, device="supa")
    torch.var(y[[0, 1]].to("supa"), dim=0, out=out)
    torch.testing.assert_close(out.cpu(), torch.var(y[[0, 1]], dim=0), rtol=1e-5, atol=0)
    torch.testing.assert_close(torch.var(dx, unbiased=False).cpu(), torch.var(x, unbiased=False), rtol=1e-5, atol=0)


def test_layernorm_written_out_forward_backward(no_fallback):
    """(x - mean) / sqrt(var + eps) over the last dim, and its backward,
    all on native kernels; against the float64 CPU result."""
    g = torch.Generator().manual_seed(64)
    x = torch.randn(16, 257, generator=g) * 3 + 1
    dx = x.to("supa").requires_grad_()
    m = dx.mean(-1, keepdim=True)
    v = dx.var(-1, unbiased=False, keepdim=True)
    y = (dx - m) / torch.sqrt(v + 1e-5)
    w = torch.linspace(0, 1, 257)
    (y * y * w.to("supa")).sum().backward()
    xr = x.double().requires_grad_()
    yr = (xr - xr.mean(-1, keepdim=True)) / torch.sqrt(xr.var(-1, unbiased=False, keepdim=True) + 1e-5)
    (yr * yr * w.double()).sum().backward()
    torch.testing.assert_close(y.detach().double().cpu(), yr.detach(), rtol=1e-4, atol=1e-4)
    torch.testing.assert_close(dx.grad.double().cpu(), xr.grad, rtol=1e-3, atol=1e-3)


def test_integer_input_takes_the_counted_fallback(supa):
    supa.supa.reset_fallback_counts()
    with pytest.raises(RuntimeError, match="floating point"):
        torch.var(torch.tensor([1, 2, 3, 4, 5]).to("supa"))
    assert supa.supa.fallback_counts().get("aten::var.correction", 0) == 1
