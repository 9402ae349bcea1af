"""The reference's own test shapes, on the supa device against the oracle:

* /root/reference/test/test_loss.py:20-34 -- nll_loss forward and backward on
  (15, 5), (16, 1000), (8732, 81), (1000, 200000) (rows longer than the
  register-resident row kernels hold), (200000, 1000) (many short rows) and
  the 4-D (2, 19, 512, 1024) case (nll_loss2d), with the reductions listed
  there, in float32, bfloat16 and float16 (the test's dtypes); and the
  cross-entropy that feeds them (log_softmax forward + backward through the
  streaming row kernels) at the two long shapes;
* /root/reference/test/test_binary_mul_kernel.py:96-139 -- the contiguous
  mixed-dtype (131072, 128) product both ways round, and the 11 bf16 x
  float32 broadcast shapes of its perf table, bit-exact (IEEE products of
  exactly widened values);
* /root/reference/test/test_copy_permute_3d_fastpath.py:49-139 -- copy_ and
  .contiguous() of a permute(0, 2, 1) stride layout built with as_strided on
  (4, 8, 16) and (3, 5, 7) in bfloat16 / float16, the float32 permute, a
  non-permute stride (100, 10, 1) and the contiguous identity, all bit-exact
  (rtol = atol = 0 there too); plus two shapes large enough for this build's
  tiled transposes.

Inputs are seeded N(0, 1) like the reference's create_random_tensor; targets
uniform over the classes (the reference's random_(C)).  Tolerances: the
path's -- nll 'none' and every backward bit-exact against the oracle on the
same dtype-rounded inputs; reductions rtol 1e-5 float32 / 1e-2 bfloat16 /
2e-3 float16."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import bf16_ulp_dist

pytestmark = pytest.mark.gpu

TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 2e-3}
NLL_CASES = [
    ((15, 5), "mean"), ((16, 1000), "mean"), ((16, 1000), "sum"), ((16, 1000), "none"),
    ((8732, 81), "sum"), ((8732, 81), "none"), ((1000, 200000), "mean"),
    ((200000, 1000), "mean"), ((200000, 1000), "sum"), ((200000, 1000), "none"),
]


def _seeded(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g).to(dtype)


def _round(x, dtype):
    if dtype == torch.bfloat16:
        return O.round_bf16(x)
    if dtype == torch.float16:
        return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)
    return np.asarray(x, np.float32)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape, reduction", NLL_CASES)
def test_nll_loss_reference_shapes(shape, reduction, dtype, no_fallback):
    n, c = shape
    x = _seeded(shape, 200 + n % 97, dtype)
    g = torch.Generator().manual_seed(300 + c % 89)
    t = torch.randint(0, c, (n,), generator=g)
    dx = x.to("supa").requires_grad_()
    loss = F.nll_loss(dx, t.to("supa"), reduction=reduction)
    xf = x.float().numpy()
    ref, tw = O.nll_loss(xf, t.numpy(), None, reduction)
    if reduction == "none":
        assert np.array_equal(loss.detach().float().cpu().numpy(), _round(ref, dtype))
        go = _seeded((n,), 7, dtype)
    else:
        assert abs(loss.float().item() - float(ref)) <= TOL[dtype] * abs(float(ref)) + 1e-6
        go = torch.tensor(1.0, dtype=dtype)
    loss.backward(go.to("supa"))
    twv = float(_round(tw, dtype)) if reduction == "mean" else float(tw)
    gi = O.nll_loss_backward(go.float().numpy(), t.numpy(), n, c, twv, None, reduction,
                             bf16=dtype == torch.bfloat16)
    got = dx.grad.float().cpu().numpy()
    if dtype == torch.float16:
        # -g / total_weight rounded once to half
        np.testing.assert_allclose(got, _round(gi, dtype), rtol=2e-3, atol=0)
    else:
        assert np.array_equal(got, _round(gi, dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(1000, 200000), (200000, 1000)])
def test_cross_entropy_reference_long_shapes(shape, dtype, no_fallback):
    """log_softmax + nll_loss forward and backward (the reference's bf16
    decomposition): the streaming row kernels at 200000 columns, and 200000
    rows of 1000."""
    n, c = shape
    x = _seeded(shape, 41, dtype)
    g = torch.Generator().manual_seed(42)
    t = torch.randint(0, c, (n,), generator=g)
    t[torch.randperm(n, generator=g)[: max(1, n // 20)]] = -100
    dx = x.to("supa").requires_grad_()
    lsm = F.log_softmax(dx, dim=1)
    lsm.retain_grad()
    loss = F.nll_loss(lsm, t.to("supa"), ignore_index=-100)
    loss.backward()
    ref_lp = O.log_softmax(x.float().numpy())
    y = lsm.detach().float().cpu().numpy()
    if dtype == torch.float32:
        np.testing.assert_allclose(y, ref_lp, rtol=1e-5, atol=1e-5)
    else:
        assert bf16_ulp_dist(lsm.detach().cpu().view(torch.int16).numpy().view(np.uint16),
                             O.f32_to_bf16(ref_lp)).max() <= 1
    out, tw = O.nll_loss(y, t.numpy(), None, "mean", -100)
    assert abs(loss.float().item() - float(out)) <= TOL[dtype] * abs(float(out))
    gl = lsm.grad.float().cpu().numpy()
    gin = O.log_softmax_backward(gl, y)
    if dtype == torch.float32:
        np.testing.assert_allclose(dx.grad.cpu().numpy(), gin, rtol=1e-5, atol=1e-9)
    else:
        assert bf16_ulp_dist(dx.grad.cpu().view(torch.int16).numpy().view(np.uint16), O.f32_to_bf16(gin)).max() <= 1


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_nll_loss2d_reference_shape(dtype, no_fallback):
    """(2, 19, 512, 1024) with targets (2, 512, 1024), reduction 'none'."""
    shape = (2, 19, 512, 1024)
    x = _seeded(shape, 51, dtype)
    g = torch.Generator().manual_seed(52)
    t = torch.randint(0, 19, (2, 512, 1024), generator=g)
    dx = x.to("supa").requires_grad_()
    loss = F.nll_loss(dx, t.to("supa"), reduction="none")
    ref, _ = O.nll_loss2d(x.float().numpy(), t.numpy(), None, "none")
    assert np.array_equal(loss.detach().float().cpu().numpy(), _round(ref, dtype))
    go = _seeded((2, 512, 1024), 53, dtype)
    loss.backward(go.to("supa"))
    gi = O.nll_loss2d_backward(go.float().numpy(), t.numpy(), shape, 0.0, None, "none",
                               bf16=dtype == torch.bfloat16)
    assert np.array_equal(dx.grad.float().cpu().numpy(), _round(gi, dtype))


@pytest.mark.parametrize("lhs, rhs", [(torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16)])
def test_mul_contiguous_mixed_dtype_reference_shape(lhs, rhs, no_fallback):
    a = _seeded((131072, 128), 61, lhs)
    b = _seeded((131072, 128), 62, rhs)
    c = a.to("supa") * b.to("supa")
    assert c.dtype == torch.float32
    assert np.array_equal(c.cpu().numpy(), O.binary(O.MUL, a.float().numpy(), b.float().numpy()))
    assert torch.equal(c.cpu(), a * b)


@pytest.mark.parametrize("shape, shape1", [
    ((1, 2048, 24, 64), (1, 2048, 1, 64)), ((1, 1024, 5120), (1, 1, 5120)),
    ((594, 4096), (594, 1)), ((601, 4096), (601, 1)), ((620, 4096), (620, 1)), ((635, 4096), (635, 1)),
    ((647, 4096), (647, 1)), ((656, 4096), (656, 1)), ((663, 4096), (663, 1)), ((670, 4096), (670, 1)),
    ((679, 4096), (679, 1)),
])
def test_mul_bf16_float_broadcast_reference_shapes(shape, shape1, no_fallback):
    a = _seeded(shape, 71, torch.bfloat16)
    b = _seeded(shape1, 72, torch.float32)
    c = a.to("supa") * b.to("supa")
    assert c.dtype == torch.float32
    want = a * b
    assert torch.equal(c.cpu(), want)
    assert np.array_equal(c.cpu().numpy(), O.binary(O.MUL, a.float().numpy(), b.numpy()))


def _contiguous_strides(shape):
    strides, acc = [0] * len(shape), 1
    for i in range(len(shape) - 1, -1, -1):
        strides[i] = acc
        acc *= shape[i]
    return strides


def _strided_pair(shape, stride, dtype, seed):
    """A (cpu, supa) pair of as_strided views of the same seeded storage."""
    base = _seeded((int(np.prod(shape)) + 1024,), seed, dtype)
    return torch.as_strided(base, shape, stride), torch.as_strided(base.to("supa"), shape, stride)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(4, 8, 16), (3, 5, 7), (4, 64, 256), (2, 208, 1040)])
def test_copy_permute_021(shape, dtype, no_fallback):
    """test_copy_permute_3d_fastpath.py:49-83: the permute(0, 2, 1) layout
    (strides (b c, 1, b)) copied into a contiguous layout, and .contiguous()."""
    a, b, c = shape
    src_cpu, src_dev = _strided_pair(shape, (b * c, 1, b), dtype, 80)
    dst_cpu, dst_dev = _strided_pair(shape, _contiguous_strides(shape), dtype, 81)
    torch.ops.aten.copy_(dst_cpu, src_cpu)
    torch.ops.aten.copy_(dst_dev, src_dev)
    assert torch.equal(dst_dev.cpu(), dst_cpu)
    assert torch.equal(src_dev.contiguous().cpu(), src_cpu.contiguous())


@pytest.mark.parametrize("case", ["float32_permute", "non_permute_stride", "identity"])
def test_copy_permute_021_bypass_cases(case, no_fallback):
    """test_copy_permute_3d_fastpath.py:85-139: layouts the reference's
    bf16 / f16 permute fast path must not take, still copied exactly."""
    shape = (4, 8, 16)
    dtype = torch.float32 if case == "float32_permute" else torch.bfloat16
    src_stride = {"float32_permute": (8 * 16, 1, 8), "non_permute_stride": (100, 10, 1),
                  "identity": tuple(_contiguous_strides(shape))}[case]
    src_cpu, src_dev = _strided_pair(shape, src_stride, dtype, 82)
    dst_cpu, dst_dev = _strided_pair(shape, _contiguous_strides(shape), dtype, 83)
    torch.ops.aten.copy_(dst_cpu, src_cpu)
    torch.ops.aten.copy_(dst_dev, src_dev)
    assert torch.equal(dst_dev.cpu(), dst_cpu)
