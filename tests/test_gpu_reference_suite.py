"""The reference's own kernel tests for the ops on this path, case for case,
with their shapes, dtypes, tolerances and comparison (CPU result against the
supa result):

* test_activation_gelu_kernel.py, test_activation_silu_kernel.py (forward and
  backward; gelu 'tanh' added beside the reference's default 'none');
* test_add.py (add / sub: Tensor, one-element broadcast, in place, Scalar, and
  the as_strided [1, 1024, 512] case), test_binary_div_true_kernel.py;
* test_fill_kernel.py (zeros / ones / full and their _like, new_, out= forms);
* test_softmax.py, test_persistent_softmax.py (softmax / log_softmax forward
  and backward over the last dim);
* test_reduce_sum_prod_kernel.py's shapes and keepdim cases for sum, and
  test_reduce_ops.py's mean cases;
* test_foreach_binary_op_list.py (with its clip_grad_norm_ case),
  test_foreach_binary_op_scalar.py, test_foreach_binary_op_scalar_list.py,
  test_foreach_binary_op_scalar_tensor.py, test_foreach_ternary_op.py
  (lerp), test_foreach_unary_op.py (the ops outside this build's native set
  through the counted CPU fallback), test_foreach_pointwise_op.py,
  test_foreach_reduce_op.py (with its accumulation-count tolerance);
* test_fused_adam_w_kernel.py (5 steps of AdamW(fused=True) on a
  cross-entropy loss against the CPU's unfused AdamW);
* test_amp_kernels.py (its known-answer _amp_update_scale_ sequence).

The reference draws unseeded inputs (create_random_tensor: N(0, 1) by
default); these draw seeded ones from the same distributions.  Where it picks
a random norm order, fixed orders over the same range stand in.  Comparison
as its assert_allclose (torch_supa/testing/common_utils.py:151-168):
torch.testing.assert_close for bfloat16, numpy's assert_allclose (CPU result
first) otherwise."""
import math

import numpy as np
import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

SUPA = "supa"  # a string: the device name exists once torch_supa is imported
RTOL = {torch.float32: 1.3e-6, torch.bfloat16: 1.6e-2, torch.float16: 1e-3}
ATOL = {torch.float32: 1e-5, torch.bfloat16: 1e-5, torch.float16: 1e-5}
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
BR200 = [(16,), (1024, 512), (1023, 511), (1025, 513), (1028, 2135)]
BR200_T = [(16,), (512, 1024), (1023, 511), (1025, 513), (1028, 2135)]
FOREACH_SHAPES = [(32,), (512, 1024), (1023, 511), (1025, 513), (1028, 2135)]

_seed = [1000]


def rand(shape, dtype, mode="norm", lo=-5, hi=5):
    """create_random_tensor's draws, seeded: N(0, 1), uniform(lo, hi), or
    integers in [lo, hi) (random bools for torch.bool)."""
    _seed[0] += 1
    g = torch.Generator().manual_seed(_seed[0])
    if dtype == torch.bool:
        return torch.randint(0, 2, shape, generator=g).bool()
    if not dtype.is_floating_point:
        return torch.randint(lo, hi, shape, generator=g).to(dtype)
    x = torch.randn(shape, generator=g) if mode == "norm" else torch.rand(shape, generator=g) * (hi - lo) + lo
    return x.to(dtype)


def pair(shape, dtype, requires_grad=False, **kw):
    c = rand(shape, dtype, **kw)
    s = c.to(SUPA)
    if requires_grad:
        c.requires_grad_(True)
        s.requires_grad_(True)
    return c, s


def ref_allclose(golden, compare, rtol, atol, equal_nan=False):
    golden, compare = golden.detach().cpu(), compare.detach().cpu()
    if golden.dtype == compare.dtype == torch.bfloat16:
        torch.testing.assert_close(compare, golden, rtol=rtol, atol=atol, equal_nan=equal_nan)
    else:
        np.testing.assert_allclose(golden.numpy(), compare.numpy(), rtol, atol, equal_nan)


# ------------------------------------------------------------ activations
@pytest.mark.parametrize("approximate", ["none", "tanh"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", BR200)
def test_gelu_forward_backward(shape, dtype, approximate, no_fallback):
    """test_activation_gelu_kernel.py:37-69."""
    xc, xs = pair(shape, dtype, requires_grad=True)
    gc, gs = pair(shape, dtype)
    m = nn.GELU(approximate=approximate)
    yc, ys = m(xc), m(xs)
    ref_allclose(yc, ys, RTOL[dtype], ATOL[dtype])
    yc.backward(gc)
    ys.backward(gs)
    ref_allclose(xc.grad, xs.grad, RTOL[dtype], ATOL[dtype])


@pytest.mark.parametrize("requires_grad", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", BR200)
def test_silu(shape, dtype, requires_grad, no_fallback):
    """test_activation_silu_kernel.py:38-61."""
    xc, xs = pair(shape, dtype, requires_grad=requires_grad)
    yc, ys = F.silu(xc, False), F.silu(xs, False)
    if not requires_grad:
        ref_allclose(yc, ys, RTOL[dtype], ATOL[dtype])
    else:
        gc, gs = pair(shape, dtype)
        yc.backward(gc)
        ys.backward(gs)
        ref_allclose(xc.grad, xs.grad, RTOL[dtype], ATOL[dtype])


# ------------------------------------------------------------ add / sub / div
@pytest.mark.parametrize("op", ["add", "sub"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", BR200)
def test_add_sub_forms(shape, dtype, op, no_fallback):
    """test_add.py:31-140: Tensor, one-element broadcast, in place, Scalar."""
    fn, fn_ = (torch.add, "add_") if op == "add" else (torch.sub, "sub_")
    ac, as_ = pair(shape, dtype)
    bc, bs = pair(shape, dtype)
    ref_allclose(fn(ac, bc), fn(as_, bs), RTOL[dtype], ATOL[dtype])
    b1 = rand([1], dtype)
    ref_allclose(fn(ac, b1), fn(as_, b1.to(SUPA)), RTOL[dtype], ATOL[dtype])
    ref_allclose(fn(ac, 3.0), fn(as_, 3.0), RTOL[dtype], ATOL[dtype])
    getattr(ac, fn_)(bc)
    getattr(as_, fn_)(bs)
    ref_allclose(ac, as_, RTOL[dtype], ATOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_add_strided(dtype, no_fallback):
    """test_add.py:79-92: a transposed and a plain as_strided view, alpha=1."""
    ac, as_ = pair([1, 1024, 512], dtype)
    bc, bs = pair([1, 1024, 512], dtype)
    ac, as_ = (torch.as_strided(t, [1, 1024, 512], [524288, 1, 1024]) for t in (ac, as_))
    bc, bs = (torch.as_strided(t, [1, 1024, 512], [524288, 512, 1]) for t in (bc, bs))
    ref_allclose(torch.add(ac, bc, alpha=1), torch.add(as_, bs, alpha=1), RTOL[dtype], ATOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", BR200)
def test_div_true(shape, dtype, no_fallback):
    """test_binary_div_true_kernel.py:23-90: a / b, rounding_mode=None, and
    the backward of both inputs."""
    ac, as_ = pair(shape, dtype, requires_grad=True)
    bc, bs = pair(shape, dtype, requires_grad=True)
    ref_allclose(ac / bc, as_ / bs, RTOL[dtype], ATOL[dtype], equal_nan=True)
    oc, os_ = torch.div(ac, bc, rounding_mode=None), torch.div(as_, bs, rounding_mode=None)
    ref_allclose(oc, os_, RTOL[dtype], ATOL[dtype], equal_nan=True)
    gc, gs = pair(oc.shape, dtype)
    oc.backward(gc)
    os_.backward(gs)
    ref_allclose(ac.grad, as_.grad, RTOL[dtype], ATOL[dtype], equal_nan=True)
    ref_allclose(bc.grad, bs.grad, RTOL[dtype], ATOL[dtype], equal_nan=True)


# ------------------------------------------------------------ fill
FILL_SHAPES = [(2, 8), (512, 1024), (1025, 513), (1023, 511), (1028, 2135), (32, 155, 155)]
FILL_DTYPES = [torch.float32, torch.uint8, torch.int8, torch.int32, torch.float16, torch.bfloat16]


@pytest.mark.parametrize("dtype", FILL_DTYPES)
@pytest.mark.parametrize("shape", FILL_SHAPES)
def test_zeros_ones_forms(shape, dtype, no_fallback):
    """test_fill_kernel.py:40-101, exact: zeros / ones, _like, zero_, new_zeros,
    out=."""
    eq = lambda c, s: ref_allclose(c, s, 0, 0)  # noqa: E731
    eq(torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype, device=SUPA))
    eq(torch.ones(shape, dtype=dtype), torch.ones(shape, dtype=dtype, device=SUPA))
    xc, xs = pair(shape, dtype, lo=0)
    eq(torch.zeros_like(xc), torch.zeros_like(xs))
    eq(torch.ones_like(xc), torch.ones_like(xs))
    bc, bs = pair([1, 3, 224, 224], dtype, lo=0)
    eq(bc.new_zeros(shape), bs.new_zeros(shape))
    torch.zeros(shape, out=xc)
    torch.zeros(shape, out=xs)
    eq(xc, xs)
    torch.ones(shape, out=xc)
    torch.ones(shape, out=xs)
    eq(xc, xs)
    xc, xs = pair(shape, dtype, lo=0)
    xc.zero_()
    xs.zero_()
    eq(xc, xs)


@pytest.mark.parametrize("value", [0.5, 1.0, 1000.0])
@pytest.mark.parametrize("shape", FILL_SHAPES)
def test_full_forms(shape, value, no_fallback):
    """test_fill_kernel.py:103-152, exact: full, full_like, new_full, out=."""
    eq = lambda c, s: ref_allclose(c, s, 0, 0)  # noqa: E731
    eq(torch.full(shape, value, dtype=torch.float32), torch.full(shape, value, dtype=torch.float32, device=SUPA))
    xc, xs = pair(shape, torch.float32)
    eq(torch.full_like(xc, value, dtype=torch.float32), torch.full_like(xs, value, dtype=torch.float32))
    bc, bs = pair([1, 3, 224, 224], torch.float32)
    eq(bc.new_full(shape, value, dtype=torch.float32), bs.new_full(shape, value, dtype=torch.float32))
    torch.full(shape, value, out=xc, dtype=torch.float32)
    torch.full(shape, value, out=xs, dtype=torch.float32)
    eq(xc, xs)


# ------------------------------------------------------------ softmax
@pytest.mark.parametrize("fn", [F.softmax, F.log_softmax])
@pytest.mark.parametrize("shape", BR200_T)
def test_softmax_log_softmax_f32(shape, fn, no_fallback):
    """test_softmax.py:24-127 (float32): forward and backward over dim -1."""
    dt = torch.float32
    xc, xs = pair(shape, dt, requires_grad=True)
    gc, gs = pair(shape, dt)
    yc, ys = fn(xc, -1), fn(xs, -1)
    ref_allclose(yc, ys, RTOL[dt], ATOL[dt], equal_nan=True)
    yc.backward(gc)
    ys.backward(gs)
    ref_allclose(xc.grad, xs.grad, RTOL[dt], ATOL[dt], equal_nan=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", BR200_T)
def test_persistent_softmax(shape, dtype, no_fallback):
    """test_persistent_softmax.py:22-72: softmax forward and backward, bf16
    with atol 1e-3."""
    atol = {torch.float32: 1e-5, torch.bfloat16: 1e-3}[dtype]
    xc, xs = pair(shape, dtype, requires_grad=True)
    gc, gs = pair(shape, dtype)
    yc, ys = F.softmax(xc, -1), F.softmax(xs, -1)
    ref_allclose(yc, ys, RTOL[dtype], atol, equal_nan=True)
    yc.backward(gc)
    ys.backward(gs)
    ref_allclose(xc.grad, xs.grad, RTOL[dtype], atol, equal_nan=True)


# ------------------------------------------------------------ sum
@pytest.mark.parametrize("dtype", DTYPES + [torch.bool])
@pytest.mark.parametrize("keepdim", [True, False])
@pytest.mark.parametrize("shape", BR200)
def test_sum_last_dim(shape, keepdim, dtype, no_fallback):
    """test_reduce_sum_prod_kernel.py:25-46's cases (dim -1, keepdim both
    ways; a bool input sums to int64, checked by dtype there) for sum, at the
    reference's reduction tolerance for float32 (test_reduce_ops.py:119, rtol
    1e-5 / atol 5e-5: a sum's rounding depends on its order) and its
    elementwise one for the 16-bit types."""
    xc, xs = pair(shape, dtype)
    yc, ys = torch.sum(xc, -1, keepdim), torch.sum(xs, -1, keepdim)
    assert yc.dtype == ys.dtype and yc.shape == ys.shape
    if dtype == torch.bool:
        assert torch.equal(yc, ys.cpu())
    elif dtype == torch.float32:
        ref_allclose(yc, ys, 1e-5, 5e-5)
    else:
        ref_allclose(yc, ys, RTOL[dtype], ATOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("keepdim", [True, False])
@pytest.mark.parametrize("shape, dim", [((2, 8), -1), ((512, 1024), -1), ((), []), ((1,), [])])
def test_mean(shape, dim, keepdim, dtype, no_fallback):
    """test_reduce_ops.py TestMean (test_mean, test_mean_br200,
    test_mean_special): atol 5e-5, rtol 1e-5 for every dtype."""
    xc, xs = pair(shape, dtype)
    ref_allclose(torch.mean(xc, dim, keepdim), torch.mean(xs, dim, keepdim), 1e-5, 5e-5)


# ------------------------------------------------------------ foreach
FE_BINARY_LIST = ["_foreach_add", "_foreach_sub", "_foreach_mul", "_foreach_div", "_foreach_clamp_max",
                  "_foreach_clamp_min", "_foreach_pow"]


@pytest.mark.parametrize("func", FE_BINARY_LIST)
@pytest.mark.parametrize("shape", FOREACH_SHAPES)
def test_foreach_binary_list(shape, func, no_fallback):
    """test_foreach_binary_op_list.py:30-58 (float32): f(list, list)."""
    dt = torch.float32
    c = [rand(shape, dt), rand(shape, dt)]
    s = [t.to(SUPA) for t in c]
    fn = getattr(torch, func)
    for rc, rs in zip(fn(c, c), fn(s, s)):
        ref_allclose(rc, rs, RTOL[dt], ATOL[dt], equal_nan=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("func", FE_BINARY_LIST[:6])
@pytest.mark.parametrize("shape", FOREACH_SHAPES)
def test_foreach_binary_scalar(shape, func, dtype, no_fallback):
    """test_foreach_binary_op_scalar.py:31-60: f(list, 2.0)."""
    c = [rand(shape, dtype), rand(shape, dtype)]
    s = [t.to(SUPA) for t in c]
    fn = getattr(torch, func)
    for rc, rs in zip(fn(c, 2.0), fn(s, 2.0)):
        ref_allclose(rc, rs, RTOL[dtype], ATOL[dtype], equal_nan=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", FOREACH_SHAPES)
def test_foreach_pow_scalar_base(shape, dtype, no_fallback):
    """test_foreach_binary_op_scalar.py:62-80: _foreach_pow(2.0, list)."""
    c = [rand(shape, dtype), rand(shape, dtype)]
    s = [t.to(SUPA) for t in c]
    for rc, rs in zip(torch._foreach_pow(2.0, c), torch._foreach_pow(2.0, s)):
        ref_allclose(rc, rs, RTOL[dtype], ATOL[dtype], equal_nan=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("input_type", ["scalar", "tensor", "scalar_list"])
@pytest.mark.parametrize("func", ["_foreach_addcmul", "_foreach_addcdiv"])
@pytest.mark.parametrize("shape", FOREACH_SHAPES)
def test_foreach_pointwise(shape, func, input_type, dtype, no_fallback):
    """test_foreach_pointwise_op.py:29-66: addcmul / addcdiv with a scalar, a
    CPU tensor of scalars (passed to both calls, as there) or a scalar list."""
    t1, t2, t3 = rand(shape, dtype), rand(shape, dtype), rand(shape, dtype)
    c1, c2, c3 = [t1, t1], [t2, t2], [t3, t3]
    s1, s2, s3 = ([t.to(SUPA) for t in lst] for lst in (c1, c2, c3))
    value = {"scalar": 2.0, "tensor": rand([2], dtype), "scalar_list": [2, 2]}[input_type]
    fn = getattr(torch, func)
    for rc, rs in zip(fn(c1, c2, c3, value), fn(s1, s2, s3, value)):
        ref_allclose(rc, rs, RTOL[dtype], ATOL[dtype], equal_nan=True)


def _accumulation_tol(count, dtype):
    """test_foreach_reduce_op.py:27-38 (GetAccumulationRtolAtol)."""
    k1 = 4.0 if count <= 32 else 4.0 * (math.log2(count) - 4.0)
    if dtype in (torch.bfloat16, torch.float16):
        return 0.001, 0.016
    return k1 * 1e-5, k1 * 1.3e-6


@pytest.mark.parametrize("ord", [1, 2, 3, 7, 50])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", [(32,), (1, 50), (512, 512), (1022, 500), (1023, 511), (1025, 513)])
def test_foreach_norm(shape, dtype, ord, no_fallback):
    """test_foreach_reduce_op.py:40-60: _foreach_norm at an order in [1, 50]."""
    c = [rand(shape, dtype), rand(shape, dtype)]
    s = [t.to(SUPA) for t in c]
    atol, rtol = _accumulation_tol(c[0].numel(), dtype)
    for rc, rs in zip(torch._foreach_norm(c, ord), torch._foreach_norm(s, ord)):
        ref_allclose(rc, rs, rtol, atol, equal_nan=True)


def test_clip_grad_norm(no_fallback):
    """test_foreach_binary_op_list.py:60-116: clip_grad_norm_ of five
    parameters with arange gradients, max_norm 10."""
    shapes = [(64, 100), (64, 100), (64,), (32,), (3, 32, 3, 3)]
    grads = [torch.arange(1.0, 6401).view(64, 100), torch.arange(1.0, 6401).view(64, 100),
             torch.arange(1.0, 65).view(64), torch.arange(1.0, 33).view(32), torch.arange(1.0, 865).view(3, 32, 3, 3)]
    pc = [rand(s, torch.float32) for s in shapes]
    ps = [p.to(SUPA) for p in pc]
    for p, q, g in zip(pc, ps, grads):
        p._grad = g.clone()
        q._grad = g.to(SUPA)
    nc = torch.nn.utils.clip_grad_norm_(pc, 10.0)
    ns = torch.nn.utils.clip_grad_norm_(ps, 10.0)
    for p, q in zip(pc, ps):
        ref_allclose(p.grad, q.grad, 1e-5, 5e-5, equal_nan=True)
    ref_allclose(nc, ns, 1e-5, 5e-5, equal_nan=True)


# ------------------------------------------------------------ optimizer / AMP
@pytest.mark.parametrize("shape", [(1, 100), (512, 1024), (1025, 513), (1023, 511), (1028, 2135)])
def test_fused_adamw_on_cross_entropy(shape, no_fallback):
    """test_fused_adam_w_kernel.py:21-78: weights uniform in [-1, 1] used as
    logits of a cross-entropy loss, 5 steps of AdamW(lr 1e-2, wd 0.01),
    fused=True on the device against the CPU's unfused AdamW, rtol 1e-2,
    atol 1e-3 after every step."""
    wc = rand(shape, torch.float32, mode="uniform", lo=-1, hi=1)
    ws = wc.to(SUPA)
    g = torch.Generator().manual_seed(_seed[0] + 7)
    target = torch.randint(0, shape[1], (shape[0],), generator=g)
    wc.requires_grad_(True)
    ws.requires_grad_(True)
    crit = nn.CrossEntropyLoss()
    oc = torch.optim.AdamW(params=[wc], lr=1e-2, weight_decay=0.01, fused=False)
    os_ = torch.optim.AdamW(params=[ws], lr=1e-2, weight_decay=0.01, fused=True)
    ts = target.to(SUPA)
    for _ in range(5):
        crit(wc, target).backward()
        oc.step()
        wc.grad.detach_()
        wc.grad.zero_()
        crit(ws, ts).backward()
        os_.step()
        ws.grad.detach_()
        ws.grad.zero_()
        ref_allclose(wc, ws, 1e-2, 1e-3, equal_nan=True)


def test_amp_update_scale_known_answers(no_fallback):
    """test_amp_kernels.py:14-75: growth 2, backoff 0.25, interval 2: two clean
    steps (tracker 1, then 0 with the scale 4 -> 8), then an overflow (scale
    8 -> 2, tracker 0)."""
    scale = torch.full((1,), 4.0, dtype=torch.float32, device=SUPA)
    tracker = torch.full((1,), 0.0, dtype=torch.int32, device=SUPA)
    found_inf = torch.full((1,), 0.0, dtype=torch.float, device=SUPA)
    torch._amp_update_scale_(scale, tracker, found_inf, 2.0, 0.25, 2)
    assert tracker.item() == 1 and scale.item() == 4.0
    torch._amp_update_scale_(scale, tracker, found_inf, 2.0, 0.25, 2)
    assert tracker.item() == 0 and scale.item() == 8.0
    found_inf.fill_(1.0)
    torch._amp_update_scale_(scale, tracker, found_inf, 2.0, 0.25, 2)
    assert tracker.item() == 0 and scale.item() == 2.0


# ------------------------------------------------------------ foreach, continued
def _scalar(v, dtype, device):
    return torch.tensor(v, dtype=dtype).to(device)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("func", FE_BINARY_LIST[:6])
@pytest.mark.parametrize("shape", FOREACH_SHAPES)
def test_foreach_binary_scalar_list(shape, func, dtype, no_fallback):
    """test_foreach_binary_op_scalar_list.py:47-72: f(list, [2, 3]) with the
    scalars as 0-dim tensors of the dtype (on each call's device)."""
    c = [rand(shape, dtype), rand(shape, dtype)]
    s = [t.to(SUPA) for t in c]
    fn = getattr(torch, func)
    rc = fn(c, [_scalar(2.0, dtype, "cpu"), _scalar(3.0, dtype, "cpu")])
    rs = fn(s, [_scalar(2.0, dtype, SUPA), _scalar(3.0, dtype, SUPA)])
    for a, b in zip(rc, rs):
        ref_allclose(a, b, RTOL[dtype], ATOL[dtype], equal_nan=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", FOREACH_SHAPES)
def test_foreach_pow_scalar_list(shape, dtype, no_fallback):
    """test_foreach_binary_op_scalar_list.py:74-96: _foreach_pow(list, [2, 3])."""
    c = [rand(shape, dtype), rand(shape, dtype)]
    s = [t.to(SUPA) for t in c]
    rc = torch._foreach_pow(c, [_scalar(2.0, dtype, "cpu"), _scalar(3.0, dtype, "cpu")])
    rs = torch._foreach_pow(s, [_scalar(2.0, dtype, SUPA), _scalar(3.0, dtype, SUPA)])
    for a, b in zip(rc, rs):
        ref_allclose(a, b, RTOL[dtype], ATOL[dtype], equal_nan=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("func", FE_BINARY_LIST[:6])
@pytest.mark.parametrize("shape", FOREACH_SHAPES)
def test_foreach_binary_scalar_tensor(shape, func, dtype, no_fallback):
    """test_foreach_binary_op_scalar_tensor.py:48-68: f(list, 0-dim tensor 2)."""
    c = [rand(shape, dtype), rand(shape, dtype)]
    s = [t.to(SUPA) for t in c]
    fn = getattr(torch, func)
    for a, b in zip(fn(c, _scalar(2.0, dtype, "cpu")), fn(s, _scalar(2.0, dtype, SUPA))):
        ref_allclose(a, b, RTOL[dtype], ATOL[dtype], equal_nan=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", FOREACH_SHAPES)
def test_foreach_pow_scalar_tensor_base(shape, dtype, no_fallback):
    """test_foreach_binary_op_scalar_tensor.py:70-90: _foreach_pow(0-dim 2, list)."""
    c = [rand(shape, dtype), rand(shape, dtype)]
    s = [t.to(SUPA) for t in c]
    rc = torch._foreach_pow(_scalar(2.0, dtype, "cpu"), c)
    rs = torch._foreach_pow(_scalar(2.0, dtype, SUPA), s)
    for a, b in zip(rc, rs):
        ref_allclose(a, b, RTOL[dtype], ATOL[dtype], equal_nan=True)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", FOREACH_SHAPES)
def test_foreach_lerp_lists(shape, dtype, no_fallback):
    """test_foreach_ternary_op.py:39-60: _foreach_lerp(list, list, weights)."""
    t1, t2, t3 = rand(shape, dtype), rand(shape, dtype), rand(shape, dtype)
    c1, c2, c3 = [t1, t1], [t2, t2], [t3, t3]
    s1, s2, s3 = ([t.to(SUPA) for t in lst] for lst in (c1, c2, c3))
    for a, b in zip(torch._foreach_lerp(c1, c2, c3), torch._foreach_lerp(s1, s2, s3)):
        ref_allclose(a, b, RTOL[dtype], ATOL[dtype], equal_nan=True)


FE_UNARY_NATIVE = ["_foreach_abs", "_foreach_ceil", "_foreach_erf", "_foreach_exp", "_foreach_expm1",
                   "_foreach_floor", "_foreach_log1p", "_foreach_log", "_foreach_neg", "_foreach_reciprocal",
                   "_foreach_round", "_foreach_sigmoid", "_foreach_sign", "_foreach_sqrt", "_foreach_tanh",
                   "_foreach_trunc", "_foreach_zero_"]
FE_UNARY_FALLBACK = ["_foreach_acos", "_foreach_asin", "_foreach_atan", "_foreach_cos", "_foreach_cosh",
                     "_foreach_erfc", "_foreach_frac", "_foreach_log10", "_foreach_log2", "_foreach_sin",
                     "_foreach_sinh", "_foreach_tan"]


def _foreach_unary(shape, func, dtype):
    c = [rand(shape, dtype), rand(shape, dtype)]
    s = [t.to(SUPA) for t in c]
    fn = getattr(torch, func)
    rc, rs = fn(c), fn(s)
    if func == "_foreach_zero_":  # in place, returns None
        rc, rs = c, s
    for a, b in zip(rc, rs):
        ref_allclose(a, b, RTOL[dtype], ATOL[dtype], equal_nan=True)


# the reference compares float32 and float16 only (its bf16 and lgamma cases
# run the op without a comparison, test_foreach_unary_op.py:74-95)
@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("func", FE_UNARY_NATIVE)
@pytest.mark.parametrize("shape", FOREACH_SHAPES)
def test_foreach_unary_native(shape, func, dtype, no_fallback):
    """test_foreach_unary_op.py, the ops this build runs on the device."""
    _foreach_unary(shape, func, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("func", FE_UNARY_FALLBACK)
def test_foreach_unary_outside_the_path(func, dtype, supa):
    """test_foreach_unary_op.py, the ops outside this build's native set: they
    run through the counted CPU fallback (the reference's own fallback,
    VariableFallbackKernel.cpp:44-64, does the same for its missing ops) and
    still match."""
    torch.supa.set_cpu_fallback_enabled(True)
    before = dict(torch.supa.fallback_counts())
    _foreach_unary((1023, 511), func, dtype)
    assert sum(dict(torch.supa.fallback_counts()).values()) > sum(before.values())
