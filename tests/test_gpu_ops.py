"""Parity through the PyTorch dispatcher: aten ops on ``supa`` tensors land on
this library's PrivateUse1 kernels (the CPU fallback is disabled and must stay
unused) and match the oracle -- bit-exact for IEEE add/mul/div and for the
float32 activations (same arithmetic), within the path's tolerances for
reductions and losses.  The BASELINE configs run at full size where the
oracle finishes in seconds, and through size-independent properties
otherwise."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import bf16_ulp_dist

pytestmark = pytest.mark.gpu

SHAPES = [(16,), (1024, 512), (1023, 511), (1025, 513), (1028, 2135)]


def seeded(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def dev(t):
    return t.to("supa")


# ------------------------------------------------------------ c1 config
def test_c1_full_size_bit_exact(no_fallback):
    g = torch.Generator().manual_seed(0)
    a = torch.randn(4096, 4096, generator=g)
    b = torch.randn(4096, 4096, generator=g)
    da, db = dev(a), dev(b)
    an, bn = a.numpy(), b.numpy()
    assert np.array_equal(torch.add(da, db, alpha=1).cpu().numpy(), O.binary(O.ADD, an, bn))
    assert np.array_equal(torch.mul(da, db).cpu().numpy(), O.binary(O.MUL, an, bn))
    # the same results as the upstream CPU kernels (the config's reference outputs)
    assert torch.equal(torch.add(da, db).cpu(), a + b)
    assert torch.equal(torch.mul(da, db).cpu(), a * b)
    assert np.array_equal(F.gelu(da).cpu().numpy(), O.unary(O.GELU, an))
    assert np.array_equal(F.silu(da).cpu().numpy(), O.unary(O.SILU, an))


# ------------------------------------------------------------ elementwise
@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_binary_ladder(shape, dtype, no_fallback):
    a, b = seeded(shape, 1, dtype=dtype), seeded(shape, 2, dtype=dtype)
    da, db = dev(a), dev(b)
    for fn in (torch.add, torch.sub, torch.mul, torch.div):
        got = fn(da, db).cpu()
        assert got.dtype == dtype
        assert torch.equal(got, fn(a, b)), fn


@pytest.mark.parametrize("shape", SHAPES)
def test_activations_ladder_bit_exact(shape, no_fallback):
    x = seeded(shape, 3, 3.0)
    dx = dev(x)
    xn = x.numpy()
    for fn, op in [(F.gelu, O.GELU), (lambda t: F.gelu(t, approximate="tanh"), O.GELU_TANH), (F.silu, O.SILU),
                   (torch.sigmoid, O.SIGMOID), (torch.tanh, O.TANH), (torch.exp, O.EXP), (torch.erf, O.ERF),
                   (torch.reciprocal, O.RECIPROCAL), (torch.abs, O.ABS), (lambda t: torch.sqrt(t.abs()), O.SQRT)]:
        if op == O.SQRT:
            assert np.array_equal(fn(dx).cpu().numpy(), O.unary(op, np.abs(xn)))
            continue
        if op == O.GELU_TANH:
            assert O.gelu_tanh_forward_equal(fn(dx).cpu().numpy(), xn)
            continue
        assert np.array_equal(fn(dx).cpu().numpy(), O.unary(op, xn))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_opt_in_accurate_gelu_forms(dtype, no_fallback):
    """torch.supa.set_accurate_gelu_enabled(True) selects the cancellation-free
    forms for both approximations, forward (x - (x/2) erfc(|x|/sqrt2) through
    log erfc; x / (1 + e^{-2u})) and backward: bit-exact against the oracle's
    GELU_LOGERFC / GELU_TANH_LOGISTIC in float32, and those rounded once to
    bfloat16 for bf16 tensors.  The switch is restored afterwards."""
    x = seeded((1000, 257), 60, 3.0)
    dy = seeded((1000, 257), 61)
    if dtype == torch.bfloat16:
        x, dy = x.to(dtype), dy.to(dtype)
    xn, dyn = x.float().numpy(), dy.float().numpy()
    was = torch.supa.accurate_gelu_enabled()
    try:
        torch.supa.set_accurate_gelu_enabled(True)
        for approx, op in [("none", O.GELU_LOGERFC), ("tanh", O.GELU_TANH_LOGISTIC)]:
            y = F.gelu(dev(x), approximate=approx).cpu().float().numpy()
            gx = torch.ops.aten.gelu_backward(dev(dy), dev(x), approximate=approx).cpu().float().numpy()
            want_y, want_gx = O.unary(op, xn), O.unary_backward(op, dyn, xn)
            if dtype == torch.bfloat16:
                want_y, want_gx = O.round_bf16(want_y), O.round_bf16(want_gx)
            assert np.array_equal(y, want_y), approx
            assert np.array_equal(gx, want_gx), approx
    finally:
        torch.supa.set_accurate_gelu_enabled(was)
    assert torch.supa.accurate_gelu_enabled() == was


def test_activation_backward_through_autograd(no_fallback):
    x = seeded((1000, 257), 4, 3.0)
    dy = seeded((1000, 257), 5)
    for fn, op, use_out in [(F.gelu, O.GELU, False), (lambda t: F.gelu(t, approximate="tanh"), O.GELU_TANH, False),
                            (F.silu, O.SILU, False), (torch.sigmoid, O.SIGMOID, True), (torch.tanh, O.TANH, True)]:
        dx = dev(x).requires_grad_()
        y = fn(dx)
        y.backward(dev(dy))
        inp = y.detach().cpu().numpy() if use_out else x.numpy()
        assert np.array_equal(dx.grad.cpu().numpy(), O.unary_backward(op, dy.numpy(), inp))


def test_broadcast_scalar_inplace_out(no_fallback):
    a = seeded((64, 128), 6)
    b = seeded((128,), 7)
    c = seeded((64, 1), 8)
    da, db, dc = dev(a), dev(b), dev(c)
    assert torch.equal((da + db).cpu(), a + b)
    assert torch.equal((da * dc).cpu(), a * c)
    assert torch.equal((da - 2.5).cpu(), a - 2.5)
    assert torch.equal((3.0 / da).cpu(), 3.0 / a)
    assert torch.equal(torch.add(da, db, alpha=0.25).cpu(), torch.add(a, b, alpha=0.25))
    assert torch.equal((da + torch.tensor(1.5)).cpu(), a + torch.tensor(1.5))  # 0-dim CPU tensor
    d0 = dev(torch.tensor(0.75))
    assert torch.equal((da * d0).cpu(), a * 0.75)  # 0-dim device tensor
    e = da.clone()
    e.add_(db).mul_(2.0).div_(dc)
    assert torch.equal(e.cpu(), ((a + b) * 2.0) / c)
    out = torch.empty(64, 128, device="supa")
    torch.mul(da, db, out=out)
    assert torch.equal(out.cpu(), a * b)
    # rsub, rounding modes
    assert torch.equal(torch.rsub(da, db).cpu(), torch.rsub(a, b))
    assert torch.equal(torch.div(da, dc, rounding_mode="floor").cpu(), torch.div(a, c, rounding_mode="floor"))
    assert torch.equal(torch.div(da, dc, rounding_mode="trunc").cpu(), torch.div(a, c, rounding_mode="trunc"))


@pytest.mark.parametrize("rows,cols", [(1, 8), (3, 1028), (7, 2048), (65, 1032), (513, 4100)])
def test_row_and_column_broadcasts(rows, cols, no_fallback):
    """Two-dim broadcasts (row vector, column vector, one element, and the
    bf16 + f32 promotion) over odd row counts and rows that do not fill a
    workgroup; integer-exact against the host kernels."""
    x = seeded((rows, cols), 40)
    xb = seeded((rows, cols), 41).to(torch.bfloat16)
    rowv = seeded((cols,), 42)
    colv = seeded((rows, 1), 43)
    one = seeded((1, 1), 44)
    dx, dxb, drow, dcol, done = dev(x), dev(xb), dev(rowv), dev(colv), dev(one)
    assert torch.equal((dx + drow).cpu(), x + rowv)
    assert torch.equal((dx * dcol).cpu(), x * colv)
    assert torch.equal((dx - done).cpu(), x - one)
    assert torch.equal((dxb + drow).cpu(), xb + rowv)  # bf16 + f32 -> f32
    assert torch.equal((drow + dxb * 2).cpu(), rowv + xb * 2)
    assert torch.equal(torch.div(dcol, drow).cpu(), torch.div(colv, rowv))  # outer-product shape


@pytest.mark.parametrize("shape", [(4, 7, 3, 40), (2, 33, 1, 8), (5, 3, 16, 1024)])
def test_per_channel_broadcasts(shape, no_fallback):
    """NCHW-like tensors with per-channel operands (strides (0, 1, 0) over the
    coalesced (HW, C, N) iteration), a per-sample scalar and a transposed
    view whose output inherits the permutation."""
    N, C, H, W = shape
    x = seeded(shape, 45)
    ch = seeded((C, 1, 1), 46)
    per_n = seeded((N, 1, 1, 1), 47)
    dx, dch, dn = dev(x), dev(ch), dev(per_n)
    assert torch.equal((dx + dch).cpu(), x + ch)
    assert torch.equal((dx * dch + dn).cpu(), x * ch + per_n)
    xb = seeded(shape, 48).to(torch.bfloat16)
    assert torch.equal((dev(xb) * dch).cpu(), xb * ch)  # bf16 * f32 -> f32
    xt = x.transpose(2, 3)
    got = dev(x).transpose(2, 3) + dev(seeded((W, 1), 49))
    assert got.stride() == (xt + seeded((W, 1), 49)).stride()
    assert torch.equal(got.cpu(), xt + seeded((W, 1), 49))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int64, torch.bool])
@pytest.mark.parametrize("shape", [(300, 517), (7, 64, 1000), (3, 1030, 20)])
def test_transpose_copies(shape, dtype, no_fallback):
    """The LDS-tiled transpose path: .contiguous() of transposed / permuted
    views (edge tiles included), a cast while transposing, and a unary op from
    a transposed input into a contiguous out=."""
    x = seeded(shape, 50, 3.0)
    x = x.to(dtype) if dtype != torch.bool else x > 0
    dx = dev(x)
    perms = [(1, 0)] if len(shape) == 2 else [(0, 2, 1), (2, 1, 0), (1, 2, 0)]
    for perm in perms:
        got = dx.permute(*perm).contiguous()
        assert got.is_contiguous()
        assert torch.equal(got.cpu(), x.permute(*perm).contiguous()), perm
    if dtype in (torch.float32, torch.bfloat16):
        xt = x.transpose(-1, -2)
        assert torch.equal(dev(x).transpose(-1, -2).to(torch.float32).contiguous().cpu(), xt.float().contiguous())
        out = torch.empty(xt.shape, dtype=dtype, device="supa")
        torch.neg(dev(x).transpose(-1, -2), out=out)
        assert torch.equal(out.cpu(), torch.neg(xt))


INT_DTYPES = (torch.uint8, torch.int8, torch.int32, torch.int64)


def _cast_source(src, dst, shape, seed):
    """Values every src -> dst conversion maps alike on both sides: with an
    integer on either side they stay in [0, 200) ([0, 128) with int8)."""
    x = seeded(shape, seed, 3.0)
    if src in INT_DTYPES or dst in INT_DTYPES:
        x = (x.abs() * 20.0).clamp(max=127.0 if torch.int8 in (src, dst) else 199.0)
    return x > 0 if src == torch.bool else x.to(src)


@pytest.mark.parametrize("src, dst", [
    (torch.float32, torch.bfloat16), (torch.float32, torch.float16), (torch.float64, torch.float32),
    (torch.float64, torch.bfloat16), (torch.float64, torch.uint8), (torch.int64, torch.int32),
    (torch.bfloat16, torch.float32), (torch.uint8, torch.float32), (torch.int8, torch.float64),
    (torch.float32, torch.int32), (torch.bool, torch.float32), (torch.uint8, torch.uint8)])
def test_transposing_casts(src, dst, no_fallback):
    """copy_ of a permuted view into a contiguous tensor of another dtype.  The
    float32 / bfloat16 / float16 pairs take the LDS-tiled transposes, which
    convert on the way out (element-size ratios 2 and 1/2 set the LDS swizzle);
    the other pairs take the per-element run-time-dtype kernel.  Two shapes: one
    whose tiled dims both end in partial tiles (208 = 3 x 64 + 16 rows, 1040
    columns: the 16-byte tile kernel) and one with odd sizes (the per-element
    tile kernel)."""
    for shape in [(2, 208, 1040), (3, 99, 517)]:
        x = _cast_source(src, dst, shape, 60)
        view_cpu = x.permute(0, 2, 1)
        out = torch.empty(view_cpu.shape, dtype=dst, device="supa")
        out.copy_(dev(x).permute(0, 2, 1))
        assert torch.equal(out.cpu(), view_cpu.to(dst).contiguous()), (shape, src, dst)


def test_transposed_and_strided_views(no_fallback):
    base = seeded((1, 5120, 1024), 9)
    a = base.transpose(1, 2)  # [1, 1024, 5120] with strides (5242880, 1, 1024): the reference's worst case
    b = seeded((1, 1024, 5120), 10)
    da = dev(base).transpose(1, 2)
    db = dev(b)
    got = da + db
    ref = a + b
    assert got.stride() == ref.stride()
    assert torch.equal(got.cpu(), ref)
    s = dev(seeded((300, 400), 11))[::3, 5:305:2]
    assert torch.equal(torch.sigmoid(s).cpu(), torch.from_numpy(O.unary(O.SIGMOID, s.cpu().numpy())))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_div_trunc_16bit_bit_exact(dtype, no_fallback):
    """bf16 / f16 trunc division truncates the quotient rounded to the 16-bit
    type, as the reference's kernel does (the oracle's rule, pinned against
    upstream CPU's vectorised path): bit-exact, contiguous and broadcast."""
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    a, b = seeded((1023, 517), 70).to(dtype), seeded((1023, 517), 71).to(dtype)
    got = torch.div(dev(a), dev(b), rounding_mode="trunc").cpu().float().numpy()
    assert np.array_equal(got, O.div_trunc_16(a.float().numpy(), b.float().numpy(), name))
    row = seeded((517,), 72).to(dtype)
    got = torch.div(dev(a), dev(row), rounding_mode="trunc").cpu().float().numpy()
    ref = O.div_trunc_16(a.float().numpy(), np.broadcast_to(row.float().numpy(), a.shape), name)
    assert np.array_equal(got, ref)
    # a CPU-scalar divisor truncates the float quotient (202 / 1.5 -> 134)
    a100 = (a.float() * 100).to(dtype)
    a100[0, 0] = 202.0
    for div in (1.5, -0.3, 7.0):
        got = torch.div(dev(a100), div, rounding_mode="trunc").cpu().float().numpy()
        assert np.array_equal(got, O.div_trunc_16_scalar(a100.float().numpy(), div, name)), div
        got_cpu_t = torch.div(dev(a100), torch.tensor(div), rounding_mode="trunc").cpu().float().numpy()
        assert np.array_equal(got_cpu_t, O.div_trunc_16_scalar(a100.float().numpy(), div, name)), div
    assert torch.div(dev(a100), 1.5, rounding_mode="trunc").cpu()[0, 0].item() == 134.0


def test_integer_bool_and_mixed_dtypes(no_fallback):
    g = torch.Generator().manual_seed(12)
    ia = torch.randint(-1000, 1000, (999,), generator=g)
    ib = torch.randint(1, 50, (999,), generator=g)
    dia, dib = dev(ia), dev(ib)
    for fn in (torch.add, torch.sub, torch.mul):
        assert torch.equal(fn(dia, dib).cpu(), fn(ia, ib))
    assert torch.equal(torch.div(dia, dib, rounding_mode="floor").cpu(), torch.div(ia, ib, rounding_mode="floor"))
    assert torch.equal(torch.div(dia, dib).cpu(), torch.div(ia, ib))  # true division promotes to float
    i8 = torch.randint(-100, 100, (1000,), generator=g, dtype=torch.int8)
    assert torch.equal((dev(i8) * dev(i8)).cpu(), i8 * i8)  # wrapping
    ba = torch.rand(500, generator=g) < 0.5
    bb = torch.rand(500, generator=g) < 0.5
    assert torch.equal((dev(ba) * dev(bb)).cpu(), ba * bb)
    assert torch.equal((dev(ba) + dev(bb)).cpu(), ba + bb)
    x16 = seeded((333,), 13, dtype=torch.bfloat16)
    f32 = seeded((333,), 14)
    assert torch.equal((dev(x16) + dev(f32)).cpu(), x16 + f32)
    assert torch.equal((dev(ia) + dev(f32[:1].expand(999).contiguous())).cpu(), ia + f32[:1].expand(999))


def test_empty_and_zero_dim(no_fallback):
    e = torch.empty(0, 5, device="supa")
    assert (e + e).shape == (0, 5)
    z = dev(torch.tensor(2.0))
    assert (z * z).item() == 4.0


def test_copy_fill_and_casts(no_fallback):
    x = seeded((257, 33), 15, 10.0)
    dx = dev(x)
    for dt in (torch.bfloat16, torch.float16, torch.float64, torch.int64, torch.int32, torch.bool):
        assert torch.equal(dx.to(dt).cpu(), x.to(dt))
    t = dx.t().contiguous()
    assert torch.equal(t.cpu(), x.t().contiguous())
    f = torch.empty(100, device="supa").fill_(0.1)
    assert torch.equal(f.cpu(), torch.full((100,), 0.1))
    z = torch.zeros(10, 10, dtype=torch.bfloat16, device="supa")
    assert torch.equal(z.cpu(), torch.zeros(10, 10, dtype=torch.bfloat16))


# ------------------------------------------------------------ c2 config
@pytest.mark.parametrize("transposed", [False, True])
def test_c2_full_size(transposed, no_fallback):
    """bf16 [64,2048,4096] + f32 bias [4096] -> f32, then gelu(tanh); the
    transposed leg is x given as a [64,4096,2048] tensor transposed."""
    g = torch.Generator().manual_seed(0)
    if transposed:
        x = torch.randn(64, 4096, 2048, generator=g).to(torch.bfloat16).transpose(1, 2)
    else:
        x = torch.randn(64, 2048, 4096, generator=g).to(torch.bfloat16)
    bias = torch.randn(4096, generator=g) * 0.02
    dx = torch.empty_strided(x.shape, x.stride(), dtype=torch.bfloat16, device="supa")
    dx.copy_(x)
    y = dx + dev(bias)
    assert y.dtype == torch.float32
    assert y.stride() == ((8388608, 1, 2048) if transposed else (8388608, 4096, 1))
    xf = x.float().numpy()  # logical order
    ref_y = O.binary(O.ADD, xf, bias.numpy())
    assert np.array_equal(y.cpu().numpy(), ref_y)
    z = F.gelu(y, approximate="tanh")
    assert z.stride() == y.stride()
    zc = z.cpu().numpy()
    del y, z
    assert O.gelu_tanh_forward_equal(zc, ref_y)


# ------------------------------------------------------------ c3 config
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cross_entropy_small_rows(dtype, no_fallback):
    N, V = 96, 128256
    logits = seeded((N, V), 20, 2.0, dtype)
    g = torch.Generator().manual_seed(21)
    t = torch.randint(0, V, (N,), generator=g)
    t[torch.randperm(N, generator=g)[:5]] = -100
    dl = dev(logits).requires_grad_()
    lsm = F.log_softmax(dl, dim=1)
    lsm.retain_grad()
    loss = F.nll_loss(lsm, dev(t), ignore_index=-100)
    loss.backward()
    y = lsm.detach().cpu().float().numpy()
    ref_lp = O.log_softmax(logits.float().numpy())
    if dtype == torch.float32:
        np.testing.assert_allclose(y, ref_lp, rtol=1e-5, atol=1e-5)
    else:
        assert bf16_ulp_dist(bits(lsm.detach()), O.f32_to_bf16(ref_lp)).max() <= 1
    out, tw = O.nll_loss(y, t.numpy(), None, "mean", -100)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert abs(loss.float().item() - float(out)) <= tol * abs(float(out))
    twv = O.round_bf16(tw).item() if dtype == torch.bfloat16 else float(tw)
    gn = O.nll_loss_backward(np.ones(1, np.float32), t.numpy(), N, V, twv, None, "mean", -100,
                             bf16=dtype == torch.bfloat16)
    gcpu = lsm.grad.cpu().float().numpy()
    assert np.array_equal(gcpu, O.round_bf16(gn) if dtype == torch.bfloat16 else gn)
    gin = O.log_softmax_backward(gcpu, y)
    if dtype == torch.float32:
        np.testing.assert_allclose(dl.grad.cpu().numpy(), gin, rtol=1e-5, atol=1e-9)
    else:
        assert bf16_ulp_dist(bits(dl.grad), O.f32_to_bf16(gin)).max() <= 1


# ------------------------------------------------------------- softmax
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(7, 13), (33, 1000), (5, 70000), (4, 128256)])
def test_softmax_forward_backward(shape, dtype, no_fallback):
    """_softmax and _softmax_backward_data against the oracle: register-resident
    rows, the streaming kernels (rows too long for registers), odd widths."""
    x = seeded(shape, 90, 3.0, dtype)
    g = seeded(shape, 91, 1.0, dtype)
    dx = dev(x).requires_grad_()
    y = torch.softmax(dx, -1)
    y.backward(dev(g))
    yc = y.detach().cpu()
    ref_y = O.softmax(x.float().numpy())
    ref_gi = O.softmax_backward(g.float().numpy(), yc.float().numpy())
    gi = dx.grad.cpu()
    if dtype == torch.float32:
        np.testing.assert_allclose(yc.numpy(), ref_y, rtol=1e-5, atol=1e-12)
        np.testing.assert_allclose(gi.numpy(), ref_gi, rtol=1e-5, atol=1e-9)
    elif dtype == torch.bfloat16:
        assert bf16_ulp_dist(bits(yc), O.f32_to_bf16(ref_y)).max() <= 1
        scale = np.abs(ref_gi).max()
        np.testing.assert_allclose(gi.float().numpy(), ref_gi, rtol=1e-2, atol=1e-2 * scale)
    else:
        np.testing.assert_allclose(yc.float().numpy(), ref_y, rtol=2e-3, atol=1e-7)
        np.testing.assert_allclose(gi.float().numpy(), ref_gi, rtol=2e-3, atol=2e-3 * np.abs(ref_gi).max())


def test_softmax_dims_and_edges(no_fallback):
    x = seeded((6, 50, 9), 92, 2.0)
    dx = dev(x)
    for d in (0, 1, 2):
        ref = np.moveaxis(O.softmax(np.moveaxis(x.numpy(), d, -1)), -1, d)
        np.testing.assert_allclose(torch.softmax(dx, d).cpu().numpy(), ref, rtol=1e-5, atol=1e-12)
    # NaN / +inf rows turn NaN, all -inf rows are NaN, the rest untouched
    e = seeded((4, 100), 93)
    e[0, 3], e[1, 9] = float("nan"), float("inf")
    e[2] = float("-inf")
    got = torch.softmax(dev(e), -1).cpu()
    assert got[:3].isnan().all() and not got[3].isnan().any()
    assert torch.allclose(got[3], torch.softmax(e[3], -1), rtol=1e-5, atol=1e-9)
    # 0-dim and empty
    assert torch.softmax(dev(torch.tensor(3.0)), 0).item() == 1.0
    assert torch.softmax(torch.zeros(0, 5, device="supa"), -1).shape == (0, 5)
    # half_to_float
    xb = seeded((8, 4096), 94, 2.0, torch.bfloat16)
    h = torch._softmax(dev(xb), -1, True)
    assert h.dtype == torch.float32
    np.testing.assert_allclose(h.cpu().numpy(), O.softmax(xb.float().numpy()), rtol=1e-5, atol=1e-12)


# ----------------------------------------------------------- nll_loss2d
@pytest.mark.parametrize("shape", [(3, 21, 17, 24), (2, 5, 7, 9)])
@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
@pytest.mark.parametrize("weighted", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_nll_loss2d(dtype, weighted, reduction, shape, no_fallback):
    """nll_loss2d forward and backward against the oracle (the row form over
    the N*H*W positions); the backward is exact, as the 2-D one is."""
    N, C, H, W = shape
    g = torch.Generator().manual_seed(97)
    lp = (torch.randn(shape, generator=g) * 2 - 3).to(dtype)
    t = torch.randint(0, C, (N, H, W), generator=g)
    t.view(-1)[torch.randperm(t.numel(), generator=g)[:7]] = -100
    w = (torch.rand(C, generator=g) + 0.5).to(dtype) if weighted else None
    red = {"none": 0, "mean": 1, "sum": 2}[reduction]
    out, tw = torch.ops.aten.nll_loss2d_forward(dev(lp), dev(t), None if w is None else dev(w), red, -100)
    wn = None if w is None else w.float().numpy()
    ref, rtw = O.nll_loss2d(lp.float().numpy(), t.numpy(), wn, reduction, -100)
    if reduction == "none":
        assert torch.equal(out.cpu(), torch.from_numpy(ref).to(dtype))
    else:
        tol = 1e-5 if dtype == torch.float32 else 1e-2
        assert abs(out.float().item() - float(ref)) <= tol * abs(float(ref))
        assert tw.float().item() == pytest.approx(float(rtw), rel=tol)
    go = (torch.randn((N, H, W), generator=g) if reduction == "none" else torch.tensor(1.3)).to(dtype)
    gi = torch.ops.aten.nll_loss2d_backward(dev(go), dev(lp), dev(t), None if w is None else dev(w), red, -100, tw)
    twv = float(tw.float().item())
    ref_gi = O.nll_loss2d_backward(go.float().numpy(), t.numpy(), shape, twv, wn, reduction, -100,
                                   bf16=dtype == torch.bfloat16)
    want = O.round_bf16(ref_gi) if dtype == torch.bfloat16 else ref_gi
    assert np.array_equal(gi.float().cpu().numpy(), want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_spatial_cross_entropy(dtype, no_fallback):
    """F.cross_entropy on [N, C, H, W] logits (log_softmax over dim 1, then
    nll_loss2d) and on [N, C, L] (upstream reshapes to 4-D) against the CPU."""
    g = torch.Generator().manual_seed(98)
    for shape, tshape in (((4, 19, 32, 40), (4, 32, 40)), ((2, 11, 300), (2, 300))):
        x = (torch.randn(shape, generator=g) * 2).to(dtype)
        t = torch.randint(0, shape[1], tshape, generator=g)
        t.view(-1)[:5] = -100
        dx = dev(x).requires_grad_()
        loss = F.cross_entropy(dx, dev(t), ignore_index=-100, label_smoothing=0.0)
        loss.backward()
        xc = x.float().clone().requires_grad_()
        ref = F.cross_entropy(xc, t, ignore_index=-100)
        ref.backward()
        tol = 1e-5 if dtype == torch.float32 else 2e-2
        assert loss.float().item() == pytest.approx(ref.item(), rel=tol)
        torch.testing.assert_close(dx.grad.float().cpu(), xc.grad, rtol=tol, atol=tol * xc.grad.abs().max().item())


# ---------------------------------------------------- fused cross-entropy
CE_TOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 2e-3}


@pytest.mark.parametrize("shape", [(96, 128256), (33, 1000), (7, 13)])
@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_fused_cross_entropy(dtype, reduction, shape, no_fallback, fused_ce):
    """Fused forward + backward against the float64 oracle on the same
    dtype-rounded logits; (7, 13) takes the kernels' scalar path (rows not a
    whole number of 16-byte vectors)."""
    N, C = shape
    logits = seeded(shape, 80, 2.0, dtype)
    g = torch.Generator().manual_seed(81)
    t = torch.randint(0, C, (N,), generator=g)
    t[torch.randperm(N, generator=g)[: max(1, N // 20)]] = -100
    dl = dev(logits).requires_grad_()
    loss = F.cross_entropy(dl, dev(t), ignore_index=-100, reduction=reduction)
    assert loss.dtype == dtype and loss.shape == ((N,) if reduction == "none" else ())
    go = (torch.ones(()) if reduction != "none" else seeded((N,), 82)).to(dtype)
    loss.backward(dev(go))
    x64 = logits.double().numpy()
    ref, lse, cnt = O.cross_entropy(x64, t.numpy(), reduction, -100)
    tol = CE_TOL[dtype]
    np.testing.assert_allclose(loss.detach().cpu().double().numpy(), ref, rtol=tol, atol=1e-6)
    gref = O.cross_entropy_backward(go.double().numpy(), x64, t.numpy(), lse, cnt, reduction, -100)
    gd = dl.grad.cpu()
    assert gd.dtype == dtype
    if dtype == torch.float32:
        np.testing.assert_allclose(gd.numpy(), gref, rtol=1e-5, atol=1e-6 * np.abs(gref).max())
    elif dtype == torch.bfloat16:
        assert bf16_ulp_dist(bits(gd), O.f64_to_bf16(gref)).max() <= 1
    else:
        np.testing.assert_allclose(gd.double().numpy(), gref, rtol=2e-3, atol=1e-7)
    # ignored rows have a zero gradient
    assert not gd[t == -100].any()


def confident_logits(shape, seed, dtype):
    """N(0, 2) logits whose even rows hold one dominant logit (60 to 72, at
    least 50 above the rest), so those rows' max term is the whole row sum
    even in float64: a log-probability of exactly 0 and a zero gradient at
    the dominant class.  Every probability stays above 2^-126 (the hardware
    exp flushes smaller results to 0, where upstream's expf keeps denormals)."""
    x = seeded(shape, seed, 2.0)
    N, C = shape
    g = torch.Generator().manual_seed(seed + 1)
    cols = torch.randint(0, C, (N,), generator=g)
    for r in range(0, N, 2):
        x[r, cols[r]] = 60.0 + 12.0 * r / N
    return x.to(dtype), cols


@pytest.mark.parametrize("dtype,shape", [(torch.bfloat16, (96, 128256)), (torch.bfloat16, (64, 32000)),
                                         (torch.float16, (64, 32000)), (torch.float32, (32, 128256)),
                                         (torch.float32, (64, 32000))])
def test_log_softmax_confident_rows(dtype, shape, no_fallback):
    """The row kernels' exp terms are exp(x - max): the dominant logit's
    log-probability is exactly 0, as in the oracle (the float64 row sum is 1)."""
    x, cols = confident_logits(shape, 300, dtype)
    out = torch.log_softmax(dev(x), dim=1)
    ref = O.log_softmax(x.float().numpy())
    rows = np.arange(0, shape[0], 2)
    assert (ref[rows, cols.numpy()[rows]] == 0).all()
    assert (out.cpu().float().numpy()[rows, cols.numpy()[rows]] == 0).all()
    if dtype == torch.float32:
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    elif dtype == torch.bfloat16:
        assert bf16_ulp_dist(bits(out), O.f32_to_bf16(ref)).max() <= 1
    else:
        np.testing.assert_allclose(out.cpu().float().numpy(), ref, rtol=1e-3, atol=1e-3)
    sm = torch.softmax(dev(x), dim=1)
    sref = O.softmax(x.float().numpy())
    if dtype == torch.float32:
        np.testing.assert_allclose(sm.cpu().numpy(), sref, rtol=1e-5, atol=1e-12)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_fused_cross_entropy_confident_rows(dtype, no_fallback, fused_ce):
    """Fused cross-entropy on rows with a dominant logit (the target on half of
    them): loss 0 and a zero gradient where the oracle has them, the rest of
    the gradient to the usual bar."""
    N, C = 64, 128256
    x, cols = confident_logits((N, C), 310, dtype)
    g = torch.Generator().manual_seed(312)
    t = torch.randint(0, C, (N,), generator=g)
    t[0::4] = cols[0::4]
    dl = dev(x).requires_grad_()
    loss = F.cross_entropy(dl, dev(t), reduction="none")
    loss.backward(dev(torch.ones(N, dtype=dtype)))
    x64 = x.double().numpy()
    ref, lse, cnt = O.cross_entropy(x64, t.numpy(), "none", -100)
    assert (loss.detach().cpu().double().numpy()[0::4] == 0).all() and (ref[0::4] == 0).all()
    np.testing.assert_allclose(loss.detach().cpu().double().numpy(), ref, rtol=CE_TOL[dtype], atol=1e-6)
    gref = O.cross_entropy_backward(np.ones(N), x64, t.numpy(), lse, cnt, "none", -100)
    gd = dl.grad.cpu()
    r4 = np.arange(0, N, 4)
    assert (gd.float().numpy()[r4, t.numpy()[r4]] == 0).all()
    if dtype == torch.float32:
        np.testing.assert_allclose(gd.numpy(), gref, rtol=1e-5, atol=1e-6 * np.abs(gref).max())
    else:
        assert bf16_ulp_dist(bits(gd), O.f64_to_bf16(gref)).max() <= 1


def test_fused_cross_entropy_matches_decomposition_and_edges(no_fallback, supa):
    """The fused path against the default log_softmax + nll_loss path on the
    same bf16 input (within the bf16 tolerance), every row ignored (mean NaN,
    sum 0, zero gradient), and an out-of-range target (IndexError at sync)."""
    N, V = 64, 32000
    logits = seeded((N, V), 83, 2.0, torch.bfloat16)
    g = torch.Generator().manual_seed(84)
    t = torch.randint(0, V, (N,), generator=g)
    t[:3] = -100
    res = {}
    was = supa.supa.fused_cross_entropy_enabled()
    for fused in (False, True):
        supa.supa.set_fused_cross_entropy_enabled(fused)
        try:
            dl = dev(logits).requires_grad_()
            loss = F.cross_entropy(dl, dev(t), ignore_index=-100)
            loss.backward()
            res[fused] = (loss.float().item(), dl.grad.float().cpu())
        finally:
            supa.supa.set_fused_cross_entropy_enabled(was)
    assert abs(res[True][0] - res[False][0]) <= 1e-2 * abs(res[False][0])
    gdiff = (res[True][1] - res[False][1]).abs().max().item()
    assert gdiff <= 1e-2 * res[False][1].abs().max().item()
    supa.supa.set_fused_cross_entropy_enabled(True)
    try:
        dl = dev(logits).requires_grad_()
        ign = dev(torch.full((N,), -100))
        loss = F.cross_entropy(dl, ign, ignore_index=-100)
        loss.backward()
        assert math.isnan(loss.float().item()) and not dl.grad.cpu().float().any()
        assert F.cross_entropy(dev(logits), ign, ignore_index=-100, reduction="sum").float().item() == 0.0
        bad = t.clone()
        bad[5] = V + 1
        F.cross_entropy(dev(logits), dev(bad), ignore_index=-100)
        with pytest.raises(IndexError):
            torch.supa.synchronize()
    finally:
        supa.supa.set_fused_cross_entropy_enabled(was)


def test_fused_cross_entropy_c3_full_size(no_fallback, fused_ce):
    """c3's shape through the fused path: per-row losses of 64 rows against
    the float64 oracle, the mean against the mean of the per-row losses, and
    each kept gradient row summing to ~0 with the target column < 0."""
    N, V = 8192, 128256
    g = torch.Generator(device="cpu").manual_seed(0)
    logits = (torch.randn(N, V, generator=g) * 2).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), generator=g)
    t[torch.randperm(N, generator=g)[:410]] = -100
    dl, dt = dev(logits), dev(t)
    rows = F.cross_entropy(dl, dt, ignore_index=-100, reduction="none").float().cpu()
    pick = torch.randperm(N, generator=g)[:64]
    ref, _, _ = O.cross_entropy(logits[pick].double().numpy(), t[pick].numpy(), "none", -100)
    np.testing.assert_allclose(rows[pick].double().numpy(), ref, rtol=1e-2)
    dlg = dl.clone().requires_grad_()
    loss = F.cross_entropy(dlg, dt, ignore_index=-100)
    keep = t != -100
    assert abs(loss.float().item() - rows[keep].double().mean().item()) <= 1e-2 * loss.float().item()
    loss.backward()
    gs = dlg.grad.float().sum(1).cpu()
    count = float(keep.sum())
    assert gs.abs().max().item() <= 0.02 / count
    gcpu = dlg.grad.cpu()
    tg = gcpu[torch.arange(N)[keep], t[keep]].float()
    assert (tg < 0).all()
    assert not gcpu[~keep].any()


def _prob_targets(n, c, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    x = (torch.randn(n, c, generator=g) * 2).to(dtype)
    p = torch.softmax(torch.randn(n, c, generator=g) * 3, 1)
    p[:2] *= 0.5  # rows whose mass is not one
    return x, p.to(dtype)


@pytest.mark.parametrize("routing", [None, True, False])
@pytest.mark.parametrize("reduction", ["none", "sum", "mean"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(64, 32000), (33, 1001)])
def test_cross_entropy_probability_targets(shape, dtype, reduction, routing, no_fallback, supa):
    """F.cross_entropy(x, p) with a class-probability target, forward and
    backward, against the float64 oracle (the oracle pinned to upstream CPU
    in test_oracle_vs_torch.py): float32 within rtol 1e-5, bfloat16 within
    1e-2, under each routing -- the reference's (None: float32 fused,
    bfloat16 decomposed), every dtype fused (True) and none (False).  The
    gradient is checked against the oracle's to 1e-5 (1e-2 for bf16) of the
    largest gradient element."""
    n, c = shape
    x, p = _prob_targets(n, c, 90 + c % 7, dtype)
    go = torch.randn(n, generator=torch.Generator().manual_seed(91)).to(dtype) if reduction == "none" \
        else torch.tensor(1.5).to(dtype)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    was = supa.supa.fused_cross_entropy_enabled()
    supa.supa.set_fused_cross_entropy_enabled(routing)
    try:
        dx = dev(x).requires_grad_()
        loss = F.cross_entropy(dx, dev(p), reduction=reduction)
        loss.backward(dev(go))
        got, gx = loss.detach().float().cpu().double().numpy(), dx.grad.float().cpu().double().numpy()
    finally:
        supa.supa.set_fused_cross_entropy_enabled(was)
    ref, lse, tsum = O.cross_entropy_prob(x.double().numpy(), p.double().numpy(), reduction)
    np.testing.assert_allclose(got, ref, rtol=tol, atol=tol * 1e-3)
    gref = O.cross_entropy_prob_backward(go.double().numpy(), x.double().numpy(), p.double().numpy(), lse, tsum,
                                         reduction)
    assert np.abs(gx - gref).max() <= tol * np.abs(gref).max()


def test_cross_entropy_probability_target_edges(no_fallback, supa):
    """A target that needs its own gradient takes the decomposition (the fused
    backward writes the logits' gradient only) and matches the CPU; a
    non-negative ignore_index with a probability target is refused as
    upstream refuses it; create_graph through the fused float32 paths (class
    and probability targets) gives a differentiable gradient whose second
    derivative matches the CPU's in float64."""
    x, p = _prob_targets(16, 300, 93, torch.float32)
    xs, ps = dev(x).requires_grad_(), dev(p).requires_grad_()
    F.cross_entropy(xs, ps).backward()
    xc, pc = x.clone().requires_grad_(), p.clone().requires_grad_()
    F.cross_entropy(xc, pc).backward()
    np.testing.assert_allclose(xs.grad.cpu().numpy(), xc.grad.numpy(), rtol=1e-4, atol=1e-7)
    np.testing.assert_allclose(ps.grad.cpu().numpy(), pc.grad.numpy(), rtol=1e-4, atol=1e-7)
    with pytest.raises(RuntimeError, match="ignore_index"):
        F.cross_entropy(dev(x), dev(p), ignore_index=3)
    t = torch.randint(0, 300, (16,), generator=torch.Generator().manual_seed(94))
    t[3] = -100
    w = torch.randn(16, 300, generator=torch.Generator().manual_seed(95))
    for tgt, tgt_dev in [(t, dev(t)), (p, dev(p))]:
        assert supa.supa.fused_cross_entropy_enabled() is None  # the reference's routing: float32 fused
        xd = dev(x).requires_grad_()
        gx, = torch.autograd.grad(F.cross_entropy(xd, tgt_dev, ignore_index=-100), xd, create_graph=True)
        (gx * dev(w)).sum().backward()
        xr = x.double().requires_grad_()
        gr, = torch.autograd.grad(F.cross_entropy(xr, tgt.double() if tgt.is_floating_point() else tgt,
                                                  ignore_index=-100), xr, create_graph=True)
        (gr * w.double()).sum().backward()
        np.testing.assert_allclose(gx.detach().cpu().double().numpy(), gr.detach().numpy(), rtol=1e-4, atol=1e-8)
        np.testing.assert_allclose(xd.grad.cpu().double().numpy(), xr.grad.numpy(), rtol=1e-3, atol=1e-7)


def test_cross_entropy_c3_full_size_properties(no_fallback):
    """[8192,128256] bf16 N(0,2), 5% ignore_index, mean: rows of the
    log-softmax sum to 1 in probability, 64 random rows match the oracle,
    the loss equals the mean of the selected log-probabilities, each grad row
    sums to ~0, and the target column carries (softmax - 1)/count."""
    N, V = 8192, 128256
    g = torch.Generator(device="cpu").manual_seed(0)
    logits = (torch.randn(N, V, generator=g) * 2).to(torch.bfloat16)
    t = torch.randint(0, V, (N,), generator=g)
    t[torch.randperm(N, generator=g)[:410]] = -100
    dl = dev(logits).requires_grad_()
    loss = F.cross_entropy(dl, dev(t), ignore_index=-100, reduction="mean")
    loss.backward()
    lsm = F.log_softmax(dl.detach(), dim=1)
    rows = torch.randperm(N, generator=g)[:64]
    y = lsm.cpu()[rows].float().numpy()
    ref = O.log_softmax(logits[rows].float().numpy())
    assert bf16_ulp_dist(O.f32_to_bf16(y), O.f32_to_bf16(ref)).max() <= 1
    p_sum = torch.exp(lsm.float()).sum(1).cpu().numpy()
    np.testing.assert_allclose(p_sum, 1.0, rtol=2e-2)
    keep = (t != -100)
    sel = lsm.cpu().float()[torch.arange(N)[keep], t[keep]]
    ref_loss = -sel.double().mean().item()
    assert abs(loss.float().item() - ref_loss) <= 1e-2 * abs(ref_loss)
    gsum = dl.grad.float().sum(1).cpu().numpy()
    assert np.abs(gsum).max() <= 1e-5
    count = float(keep.sum())
    gt = dl.grad.cpu().float()[torch.arange(N)[keep], t[keep]].double()
    expect = (torch.exp(sel.double()) - 1) / count
    np.testing.assert_allclose(gt.numpy(), expect.numpy(), rtol=3e-2, atol=1e-8)


def test_nll_out_of_range_target_raises_at_sync():
    import torch_supa  # noqa: F401
    lp = dev(torch.log_softmax(seeded((8, 10), 22), 1))
    t = dev(torch.tensor([0, 1, 2, 3, 4, 5, 6, 12]))
    loss = F.nll_loss(lp, t)
    with pytest.raises(IndexError):
        loss.item()
    # the flag is cleared after it is reported
    assert F.nll_loss(lp, dev(torch.tensor([0] * 8))).item() == pytest.approx(-lp[:, 0].mean().item(), rel=1e-6)


# ------------------------------------------------------------ c4 config
@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
def test_c4_full_size_losses(reduction, no_fallback):
    g = torch.Generator().manual_seed(0)
    x = torch.randn(32, 1048576, generator=g)
    t = torch.randn(32, 1048576, generator=g)
    tb = (torch.rand(32, 1048576, generator=g) < 0.3).float()
    pw = torch.rand(1048576, generator=g) * 1.5 + 0.5
    dx, dt, dtb, dpw = dev(x), dev(t), dev(tb), dev(pw)
    cases = [(O.MSE, lambda a, b: F.mse_loss(a, b, reduction=reduction), dt, t, None),
             (O.SMOOTH_L1, lambda a, b: F.smooth_l1_loss(a, b, reduction=reduction, beta=1.0), dt, t, None),
             (O.BCE_LOGITS, lambda a, b: F.binary_cross_entropy_with_logits(a, b, pos_weight=dpw,
                                                                             reduction=reduction), dtb, tb, pw)]
    for op, fn, dtarget, target, pwn in cases:
        xg = dx.clone().requires_grad_()
        loss = fn(xg, dtarget)
        go = torch.ones_like(loss) if reduction != "none" else dev(seeded((32, 1048576), 30))
        loss.backward(go)
        ref = O.loss(op, x.numpy(), target.numpy(), None if pwn is None else pwn.numpy(), reduction=reduction,
                     beta=1.0)
        got = loss.detach().cpu().numpy()
        if reduction == "none":
            assert np.array_equal(got, ref), op
        else:
            np.testing.assert_allclose(got, ref, rtol=1e-5)
        gref = O.loss_backward(op, go.cpu().numpy(), x.numpy(), target.numpy(),
                               None if pwn is None else pwn.numpy(), reduction=reduction, beta=1.0)
        assert np.array_equal(xg.grad.cpu().numpy(), gref), op


@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
@pytest.mark.parametrize("with_pw,with_w", [(False, False), (True, False), (False, True), (True, True)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.float64])
@pytest.mark.parametrize("shape", [(33, 4100), (5, 8200), (40, 1000), (3, 2, 4100)])
def test_fused_bce_backward_matches_op_sequence(shape, reduction, with_pw, with_w, dtype, no_fallback, supa):
    """The one-kernel BCE-with-logits input gradient is bit-identical to the
    autograd formula's op-by-op evaluation on the same kernels (and, in
    float32, to the oracle), for every pos_weight / weight combination; rows
    of more than 16 KiB take the one-vector row kernel (f32 / f64 at 4100
    columns, every dtype at 8200; the 3-d shape's outer dims flattened into
    rows, its weight per row), shorter ones the paired-row kernel."""
    *R, C = shape
    g = torch.Generator().manual_seed(101)
    x = (torch.randn(*R, C, generator=g) * 2).to(dtype)
    tb = (torch.rand(*R, C, generator=g) < 0.3).to(dtype)
    pw = (torch.rand(C, generator=g) * 1.5 + 0.5).to(dtype) if with_pw else None
    w = (torch.rand(*R, 1, generator=g) + 0.5).to(dtype) if with_w else None
    go = (torch.randn(*R, C, generator=g) if reduction == "none" else torch.ones(())).to(dtype)
    grads = {}
    for fused in (True, False):
        supa.supa.set_fused_bce_backward_enabled(fused)
        try:
            xg = dev(x).requires_grad_()
            loss = F.binary_cross_entropy_with_logits(xg, dev(tb), weight=None if w is None else dev(w),
                                                      pos_weight=None if pw is None else dev(pw),
                                                      reduction=reduction)
            loss.backward(dev(go))
            grads[fused] = xg.grad.cpu()
        finally:
            supa.supa.set_fused_bce_backward_enabled(True)
    assert torch.equal(grads[True], grads[False])
    if dtype == torch.float32:
        gref = O.loss_backward(O.BCE_LOGITS, go.numpy(), x.numpy(), tb.numpy(), None if pw is None else pw.numpy(),
                               None if w is None else w.numpy(), reduction=reduction)
        assert np.array_equal(grads[True].numpy(), gref)


def test_bce_double_backward_and_target_grad(supa):
    """create_graph: the gradient is built from differentiable ops, so a
    second derivative exists and matches upstream's on the CPU; a target
    that requires grad gets upstream's target gradient."""
    g = torch.Generator().manual_seed(102)
    x = torch.randn(16, 300, generator=g)
    t = torch.rand(16, 300, generator=g)
    pw = torch.rand(300, generator=g) + 0.5
    res = []
    for d in ("cpu", "supa"):
        xg = x.to(d).detach().requires_grad_()
        tg = t.to(d).detach().requires_grad_()
        loss = F.binary_cross_entropy_with_logits(xg, tg, pos_weight=pw.to(d))
        gx, gt = torch.autograd.grad(loss, (xg, tg), create_graph=True)
        (gx * gx).sum().backward()
        res.append((gx.detach().cpu(), gt.detach().cpu(), xg.grad.cpu()))
    for a, b in zip(*res):
        np.testing.assert_allclose(b.numpy(), a.numpy(), rtol=1e-5, atol=1e-8)


def test_sum_mean_dims(no_fallback):
    x = seeded((64, 1000, 3), 31)
    dx = dev(x)
    np.testing.assert_allclose(dx.sum().item(), x.double().sum().item(), rtol=1e-5)
    np.testing.assert_allclose(dx.mean().item(), x.double().mean().item(), rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(dx.sum(dim=1).cpu().numpy(), x.double().sum(1).numpy(), rtol=1e-5, atol=1e-5)
    np.testing.assert_allclose(dx.mean(dim=(0, 2), keepdim=True).cpu().numpy(),
                               x.double().mean((0, 2), keepdim=True).numpy(), rtol=1e-5, atol=1e-6)
    xb = seeded((4096, 33), 32, dtype=torch.bfloat16)
    np.testing.assert_allclose(dev(xb).sum(dtype=torch.float32).item(), xb.double().sum().item(), rtol=1e-5)


# ------------------------------------------------------------ c5 config
def test_c5_one_layer_fused_adamw_bit_exact(no_fallback):
    """One decoder layer of the c5 shapes (9 tensors, 202M parameters),
    torch.optim.AdamW(fused=True) for 10 steps on supa against the oracle."""
    shapes = [(4096, 4096)] * 4 + [(11008, 4096)] * 2 + [(4096, 11008)] + [(4096,)] * 2
    g = torch.Generator().manual_seed(0)
    params = [torch.randn(s, generator=g) * 0.02 for s in shapes]
    grads = [torch.randn(s, generator=g) * 1e-3 for s in shapes]
    dp = [dev(p).requires_grad_() for p in params]
    dg = [dev(x) for x in grads]
    opt = torch.optim.AdamW(dp, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, fused=True)
    for _ in range(10):
        for p, gr in zip(dp, dg):
            p.grad = gr
        opt.step()
    for i, s in enumerate(shapes):
        hp = params[i].numpy().ravel().copy()
        hg = grads[i].numpy().ravel().copy()
        hm, hv = np.zeros_like(hp), np.zeros_like(hp)
        for step in range(1, 11):
            O.adamw_step(hp, hg, hm, hv, float(step), 1e-4, 0.9, 0.999, 0.01, 1e-8)
        assert np.array_equal(dp[i].detach().cpu().numpy().ravel(), hp), i
        st = opt.state[dp[i]]
        assert np.array_equal(st["exp_avg"].cpu().numpy().ravel(), hm)
        assert np.array_equal(st["exp_avg_sq"].cpu().numpy().ravel(), hv)
        assert st["step"].item() == 10.0


@pytest.mark.parametrize("amsgrad", [False, True])
def test_fused_adam_bit_exact(amsgrad, no_fallback):
    """torch.optim.Adam(fused=True) (the _fused_adam_ kernel: weight decay on
    the gradient) for 6 steps on supa against the oracle's Adam step."""
    shapes = [(1024, 513), (4097,), (3, 5)]
    g = torch.Generator().manual_seed(3)
    params = [torch.randn(s, generator=g) * 0.5 for s in shapes]
    grads = [torch.randn(s, generator=g) * 1e-2 for s in shapes]
    dp = [dev(p).requires_grad_() for p in params]
    opt = torch.optim.Adam(dp, lr=1e-3, eps=1e-8, weight_decay=0.05, amsgrad=amsgrad, fused=True)
    for _ in range(6):
        for p, gr in zip(dp, grads):
            p.grad = dev(gr)
        opt.step()
    for i, s in enumerate(shapes):
        hp = params[i].numpy().ravel().copy()
        hg = grads[i].numpy().ravel().copy()
        hm, hv, hx = np.zeros_like(hp), np.zeros_like(hp), np.zeros_like(hp)
        for step in range(1, 7):
            O.adamw_step(hp, hg, hm, hv, float(step), 1e-3, 0.9, 0.999, 0.05, 1e-8, amsgrad=amsgrad,
                         vmax=hx if amsgrad else None, l2=True)
        assert np.array_equal(dp[i].detach().cpu().numpy().ravel(), hp), i
        assert np.array_equal(opt.state[dp[i]]["exp_avg_sq"].cpu().numpy().ravel(), hv)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("weight_decay", [0.0, 0.01])
def test_fused_adamw_plain_modes(dtype, weight_decay, no_fallback):
    """AdamW(fused=True) without weight decay and with it, float32 and
    float16, on shapes with full chunks, a partial chunk, a partial vector and
    an unaligned view's scalar path: bit-exact against the oracle's step
    (16-bit state rounded after every step)."""
    shapes = [(1024, 513), (4097,), (3, 5)]
    g = torch.Generator().manual_seed(76)
    params = [(torch.randn(s, generator=g) * 0.02).to(dtype) for s in shapes]
    grads = [(torch.randn(s, generator=g) * 1e-3).to(dtype) for s in shapes]
    dp = [dev(p).requires_grad_() for p in params]
    # an unaligned parameter: a view one element into its storage
    base = dev(torch.zeros(4098, dtype=dtype))
    off = base[1:].view(4097)
    off.copy_(dp[1].detach())
    dp[1] = off.requires_grad_()
    opt = torch.optim.AdamW(dp, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=weight_decay, fused=True)
    for _ in range(4):
        for p, gr in zip(dp, grads):
            p.grad = dev(gr)
        opt.step()
    rnd = (lambda a: a) if dtype == torch.float32 else \
        (lambda a: a.astype(np.float16).astype(np.float32))
    for i in range(len(shapes)):
        hp = params[i].float().numpy().ravel().copy()
        hg = grads[i].float().numpy().ravel().copy()
        hm, hv = np.zeros_like(hp), np.zeros_like(hp)
        for step in range(1, 5):
            O.adamw_step(hp, hg, hm, hv, float(step), 1e-3, 0.9, 0.999, weight_decay, 1e-8)
            for a in (hp, hm, hv):
                a[:] = rnd(a)
        assert np.array_equal(dp[i].detach().float().cpu().numpy().ravel(), hp), i
        st = opt.state[dp[i]]
        assert np.array_equal(st["exp_avg"].float().cpu().numpy().ravel(), hm), i
        assert np.array_equal(st["exp_avg_sq"].float().cpu().numpy().ravel(), hv), i


def test_foreach_list_and_scalar(no_fallback):
    shapes = [(4096, 4096), (4096,), (333, 17)]
    xs = [seeded(s, 40 + i) for i, s in enumerate(shapes)]
    ys = [seeded(s, 50 + i) for i, s in enumerate(shapes)]
    dxs, dys = [dev(x) for x in xs], [dev(y) for y in ys]
    torch._foreach_add_(dxs, dys, alpha=0.5)
    torch._foreach_mul_(dxs, 0.5)
    for dx, x, y in zip(dxs, xs, ys):
        ref = O.binary(O.MUL, O.binary(O.ADD, x.numpy(), y.numpy(), 0.5), np.float32(0.5))
        assert np.array_equal(dx.cpu().numpy(), ref)
    outs = torch._foreach_mul(dxs, dys)
    for o, dx, dy in zip(outs, dxs, dys):
        assert torch.equal(o.cpu(), dx.cpu() * dy.cpu())


def test_allocator_stats_and_reuse():
    import torch_supa  # noqa: F401
    torch.supa.synchronize()
    before = torch.supa.memory_stats()
    x = torch.empty(1 << 20, device="supa")
    mid = torch.supa.memory_allocated()
    assert mid >= before["allocated_bytes"] + (1 << 22)
    mallocs = torch.supa.memory_stats()["num_device_mallocs"]
    del x
    y = torch.empty(1 << 20, device="supa")
    assert torch.supa.memory_stats()["num_device_mallocs"] == mallocs  # served from the cache
    assert torch.supa.memory_allocated() == mid
    del y
    torch.supa.empty_cache()
    assert torch.supa.memory_reserved() <= torch.supa.memory_stats()["reserved_bytes"]


# ---------------------------------------------------------------- AMP
def test_amp_unscale_and_update_scale(no_fallback):
    """_amp_foreach_non_finite_check_and_unscale_ over a mixed-dtype list
    (with a non-contiguous member) and _amp_update_scale_ over a sequence of
    overflow flags, against upstream's CPU kernels."""
    xs = [seeded((1000, 33), 70, 100.0), seeded((4097,), 71, 100.0).to(torch.bfloat16),
          seeded((64, 50), 72).t(), seeded((7,), 73).to(torch.float16)]
    for inv, poison in ((0.125, False), (1.0, False), (0.5, True)):
        cpu = [x.clone() for x in xs]
        if poison:
            cpu[1][5] = float("inf")
        gpu = [dev(x) for x in cpu]
        fi_c, fi_g = torch.zeros(1), dev(torch.zeros(1))
        torch._amp_foreach_non_finite_check_and_unscale_(cpu, fi_c, torch.tensor([inv]))
        torch._amp_foreach_non_finite_check_and_unscale_(gpu, fi_g, dev(torch.tensor([inv])))
        for a, b in zip(cpu, gpu):
            assert torch.equal(a, b.cpu())
        assert fi_g.item() == fi_c.item() == float(poison)
    scale_c, tr_c = torch.tensor([65536.0]), torch.zeros(1, dtype=torch.int32)
    scale_g, tr_g = dev(scale_c.clone()), dev(tr_c.clone())
    for i, inf in enumerate([0, 0, 1, 0, 0, 0, 1, 1, 0, 0]):
        f = torch.tensor([float(inf)])
        torch._amp_update_scale_(scale_c, tr_c, f, 2.0, 0.5, 2)
        torch._amp_update_scale_(scale_g, tr_g, dev(f), 2.0, 0.5, 2)
        assert scale_g.item() == scale_c.item() and tr_g.item() == tr_c.item(), i


def test_grad_scaler_with_fused_adamw(supa):
    """torch.amp.GradScaler + AdamW(fused=True) on supa: the scaled backward,
    the non-finite check, the fused step with grad_scale / found_inf and the
    scale update match the oracle step for step, and an overflowing step is
    skipped while the scale backs off."""
    supa.supa.reset_fallback_counts()
    g = torch.Generator().manual_seed(74)
    shapes = [(256, 300), (300,), (17, 5)]
    p0 = [torch.randn(s, generator=g) * 0.02 for s in shapes]
    cs = [torch.randn(s, generator=g) * 1e-3 for s in shapes]
    dp = [dev(p).requires_grad_() for p in p0]
    dc = [dev(c) for c in cs]
    opt = torch.optim.AdamW(dp, lr=1e-3, weight_decay=0.01, fused=True)
    scaler = torch.amp.GradScaler("supa", init_scale=2.0 ** 10, growth_interval=2)
    hp = [p.numpy().ravel().copy() for p in p0]
    hm = [np.zeros_like(x) for x in hp]
    hv = [np.zeros_like(x) for x in hp]
    scale, tracker, step = 2.0 ** 10, 0, 0
    for it in range(5):
        opt.zero_grad()
        loss = sum((p * c).sum() for p, c in zip(dp, dc))
        if it == 2:
            loss = loss * float("inf")  # every gradient overflows
        scaler.scale(loss).backward()
        scaler.step(opt)
        scaler.update()
        overflow = it == 2
        if not overflow:
            step += 1
            for i in range(len(shapes)):
                hg = (cs[i].numpy().ravel() * np.float32(scale)).astype(np.float32)
                O.adamw_step(hp[i], hg, hm[i], hv[i], float(step), 1e-3, 0.9, 0.999, 0.01, 1e-8, grad_scale=scale)
        scale, tracker = O.amp_update_scale(scale, tracker, float(overflow), 2.0, 0.5, 2)
        assert scaler.get_scale() == scale, it
    for i in range(len(shapes)):
        np.testing.assert_allclose(dp[i].detach().cpu().numpy().ravel(), hp[i], rtol=1e-6, atol=1e-9)
    used = supa.supa.fallback_counts()
    assert not any("amp" in k or "adamw" in k for k in used), used


@pytest.mark.parametrize("amsgrad", [False, True])
@pytest.mark.parametrize("scaled", [False, True])
def test_fused_adamw_amsgrad_and_grad_scale_bit_exact(amsgrad, scaled, no_fallback):
    """_fused_adamw_ with amsgrad and / or GradScaler's grad_scale + found_inf
    (the compile-time kernel's AMS / GS forms) for 4 steps on full chunks, a
    partial chunk and a partial vector: p, g (unscaled, stored back), m, v and
    max_exp_avg_sq bit-exact against the oracle's step; then a step with
    found_inf = 1 changes nothing."""
    shapes = [(1024, 513), (4097,), (3, 5)]
    g = torch.Generator().manual_seed(77)
    params = [torch.randn(s, generator=g) * 0.5 for s in shapes]
    grads = [torch.randn(s, generator=g) * 1e-2 for s in shapes]
    scale = 1024.0 * 3.0 if scaled else None  # not a power of two: a real division
    dp = [dev(p) for p in params]
    dm = [torch.zeros_like(x) for x in dp]
    dv = [torch.zeros_like(x) for x in dp]
    dx = [torch.zeros_like(x) for x in dp]
    steps = [dev(torch.zeros(())) for _ in dp]
    hp = [p.numpy().ravel().copy() for p in params]
    hm = [np.zeros_like(x) for x in hp]
    hv = [np.zeros_like(x) for x in hp]
    hx = [np.zeros_like(x) for x in hp]
    gs = dev(torch.tensor(scale if scaled else 1.0))
    fi = dev(torch.zeros(()))
    for step in range(1, 5):
        dg = [dev(gr * scale) if scaled else dev(gr) for gr in grads]
        for t in steps:
            t.add_(1.0)
        torch._fused_adamw_(dp, dg, dm, dv, dx, steps, lr=1e-3, beta1=0.9, beta2=0.999, weight_decay=0.01,
                            eps=1e-8, amsgrad=amsgrad, maximize=False, grad_scale=gs if scaled else None,
                            found_inf=fi if scaled else None)
        for i in range(len(shapes)):
            hg = (grads[i].numpy().ravel() * np.float32(scale)).astype(np.float32) if scaled else \
                grads[i].numpy().ravel().copy()
            O.adamw_step(hp[i], hg, hm[i], hv[i], float(step), 1e-3, 0.9, 0.999, 0.01, 1e-8,
                         grad_scale=scale, amsgrad=amsgrad, vmax=hx[i] if amsgrad else None)
            if scaled:
                assert np.array_equal(dg[i].cpu().numpy().ravel(), hg), (step, i)
    for i in range(len(shapes)):
        assert np.array_equal(dp[i].cpu().numpy().ravel(), hp[i]), i
        assert np.array_equal(dm[i].cpu().numpy().ravel(), hm[i]), i
        assert np.array_equal(dv[i].cpu().numpy().ravel(), hv[i]), i
        if amsgrad:
            assert np.array_equal(dx[i].cpu().numpy().ravel(), hx[i]), i
    if scaled:
        before = [x.clone() for x in dp]
        fi.fill_(1.0)
        torch._fused_adamw_(dp, [dev(gr) for gr in grads], dm, dv, dx, steps, lr=1e-3, beta1=0.9, beta2=0.999,
                            weight_decay=0.01, eps=1e-8, amsgrad=amsgrad, maximize=False, grad_scale=gs,
                            found_inf=fi)
        for a, b in zip(dp, before):
            assert torch.equal(a.cpu(), b.cpu())


@pytest.mark.parametrize("adam", [False, True])
@pytest.mark.parametrize("weight_decay", [0.0, 0.01])
@pytest.mark.parametrize("tensor_lr", [False, True])
def test_fused_adam_maximize_and_device_lr_bit_exact(adam, weight_decay, tensor_lr, no_fallback):
    """_fused_adamw_ / _fused_adam_ with maximize=True, the lr a float or a
    device tensor (the tensor_lr overload, read on the device), for 4 steps
    on full chunks, a partial chunk and a partial vector: p, m and v
    bit-exact against the oracle's step.  Adam with weight decay under
    maximize runs the general kernel, every other case the plain one."""
    shapes = [(1024, 513), (4097,), (3, 5)]
    g = torch.Generator().manual_seed(91)
    params = [torch.randn(s, generator=g) * 0.5 for s in shapes]
    grads = [torch.randn(s, generator=g) * 1e-2 for s in shapes]
    lr = float(np.float32(7e-4))  # a float32 value, as the device tensor holds it
    dp = [dev(p) for p in params]
    dm = [torch.zeros_like(x) for x in dp]
    dv = [torch.zeros_like(x) for x in dp]
    steps = [dev(torch.zeros(())) for _ in dp]
    hp = [p.numpy().ravel().copy() for p in params]
    hm = [np.zeros_like(x) for x in hp]
    hv = [np.zeros_like(x) for x in hp]
    fn = torch._fused_adam_ if adam else torch._fused_adamw_
    lr_arg = dev(torch.tensor(lr)) if tensor_lr else lr
    for step in range(1, 5):
        dg = [dev(gr) for gr in grads]
        for t in steps:
            t.add_(1.0)
        fn(dp, dg, dm, dv, [], steps, lr=lr_arg, beta1=0.9, beta2=0.999, weight_decay=weight_decay, eps=1e-8,
           amsgrad=False, maximize=True)
        for i in range(len(shapes)):
            O.adamw_step(hp[i], grads[i].numpy().ravel().copy(), hm[i], hv[i], float(step), lr, 0.9, 0.999,
                         weight_decay, 1e-8, maximize=True, l2=adam)
    for i in range(len(shapes)):
        assert np.array_equal(dp[i].cpu().numpy().ravel(), hp[i]), i
        assert np.array_equal(dm[i].cpu().numpy().ravel(), hm[i]), i
        assert np.array_equal(dv[i].cpu().numpy().ravel(), hv[i]), i


def test_fused_adamw_bf16_params(no_fallback):
    """bf16 parameters and state: every element is loaded to float, stepped
    with the float32 arithmetic and stored back as bf16 (upstream's opmath
    rule), so the oracle's float step on bf16-rounded values, rounded after
    every step, is bit-identical."""
    shapes = [(1024, 513), (77,)]
    g = torch.Generator().manual_seed(75)
    params = [(torch.randn(s, generator=g) * 0.02).to(torch.bfloat16) for s in shapes]
    grads = [(torch.randn(s, generator=g) * 1e-3).to(torch.bfloat16) for s in shapes]
    dp = [dev(p).requires_grad_() for p in params]
    opt = torch.optim.AdamW(dp, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, fused=True)
    for _ in range(4):
        for p, gr in zip(dp, grads):
            p.grad = dev(gr)
        opt.step()
    for i in range(len(shapes)):
        hp = params[i].float().numpy().ravel().copy()
        hg = grads[i].float().numpy().ravel().copy()
        hm, hv = np.zeros_like(hp), np.zeros_like(hp)
        for step in range(1, 5):
            O.adamw_step(hp, hg, hm, hv, float(step), 1e-3, 0.9, 0.999, 0.01, 1e-8)
            for a in (hp, hm, hv):
                a[:] = O.round_bf16(a)
        assert np.array_equal(dp[i].detach().float().cpu().numpy().ravel(), hp), i
        st = opt.state[dp[i]]
        assert np.array_equal(st["exp_avg"].float().cpu().numpy().ravel(), hm)
        assert np.array_equal(st["exp_avg_sq"].float().cpu().numpy().ravel(), hv)


# ------------------------------------------------ pointwise ternary / minmax
def _exact(got, ref):
    torch.testing.assert_close(got.cpu(), ref, rtol=0, atol=0, equal_nan=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(1000,), (513, 4100)])
def test_addcmul_addcdiv_lerp_bit_exact(shape, dtype, no_fallback):
    """addcmul / addcdiv / lerp (Scalar and Tensor weight) are the oracle's
    float32 arithmetic rounded once to the tensor dtype."""
    x, y = seeded(shape, 70, 2.0, dtype), seeded(shape, 71, 2.0, dtype)
    z = seeded(shape, 72, 2.0)
    z = (z.sign() * (z.abs() + 0.25)).to(dtype)
    w = (torch.rand(shape, generator=torch.Generator().manual_seed(73)) * 1.4 - 0.2).to(dtype)
    dx, dy, dz, dw = dev(x), dev(y), dev(z), dev(w)
    f = [t.float().numpy() for t in (x, y, z, w)]

    def want(arr):
        return torch.from_numpy(arr).to(dtype)

    _exact(torch.addcmul(dx, dy, dz, value=-0.37), want(O.ternary(O.ADDCMUL, f[0], f[1], f[2], -0.37)))
    _exact(torch.addcdiv(dx, dy, dz, value=0.5), want(O.ternary(O.ADDCDIV, f[0], f[1], f[2], 0.5)))
    _exact(torch.lerp(dx, dy, dw), want(O.ternary(O.LERP, f[0], f[1], f[3])))
    for ws in (0.1, 0.75):
        wf = np.full(f[0].shape, np.float32(ws), np.float32)
        _exact(torch.lerp(dx, dy, ws), want(O.ternary(O.LERP, f[0], f[1], wf)))
    # in-place and out= forms run the same kernels
    e = dx.clone()
    e.addcmul_(dy, dz, value=2.0).lerp_(dy, 0.25)
    ref = O.ternary(O.ADDCMUL, f[0], f[1], f[2], 2.0)
    ref = O.ternary(O.LERP, want(ref).float().numpy(), f[1], np.full(ref.shape, 0.25, np.float32))
    _exact(e, want(ref))
    out = torch.empty_like(dx)
    torch.addcdiv(dx, dy, dz, out=out)
    _exact(out, want(O.ternary(O.ADDCDIV, f[0], f[1], f[2], 1.0)))
    if dtype == torch.float32:  # same results as upstream's CPU kernels where both round once
        assert torch.equal(torch.lerp(dx, dy, dw).cpu(), torch.lerp(x, y, w))


def test_pointwise_broadcast_and_integer(no_fallback):
    x = seeded((64, 1, 300), 74)
    y = seeded((300,), 75)
    z = seeded((1, 5, 1), 76)
    dx, dy, dz = dev(x), dev(y), dev(z)
    ref = O.ternary(O.ADDCMUL, *np.broadcast_arrays(x.numpy(), y.numpy(), z.numpy()), 0.5)
    _exact(torch.addcmul(dx, dy, dz, value=0.5), torch.from_numpy(np.ascontiguousarray(ref)))
    # integers: exact integer arithmetic, value an int
    a = torch.randint(-1000, 1000, (777,), generator=torch.Generator().manual_seed(77))
    b = torch.randint(-30, 30, (777,), generator=torch.Generator().manual_seed(78))
    c = torch.randint(-30, 30, (777,), generator=torch.Generator().manual_seed(79))
    assert torch.equal(torch.addcmul(dev(a), dev(b), dev(c), value=3).cpu(), torch.addcmul(a, b, c, value=3))
    with pytest.raises(RuntimeError, match="Integer division"):
        torch.addcdiv(dev(a), dev(b), dev(c))
    with pytest.raises(RuntimeError):
        torch.lerp(dx, dev(y.double()), 0.5)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int64])
def test_maximum_minimum_clamp(dtype, no_fallback):
    """Selection ops are exact: same values as upstream's CPU kernels,
    including NaN propagation and clamp with min > max."""
    g = torch.Generator().manual_seed(80)
    if dtype.is_floating_point:
        a = (torch.randn(257, 1031, generator=g) * 3).to(dtype)
        b = (torch.randn(257, 1031, generator=g) * 3).to(dtype)
        a[::13, ::7] = float("nan")
        b[::11, ::5] = float("nan")
    else:
        a = torch.randint(-100, 100, (257, 1031), generator=g, dtype=dtype)
        b = torch.randint(-100, 100, (257, 1031), generator=g, dtype=dtype)
    da, db = dev(a), dev(b)
    _exact(torch.maximum(da, db), torch.maximum(a, b))
    _exact(torch.minimum(da, db), torch.minimum(a, b))
    _exact(torch.maximum(da, db[:1]), torch.maximum(a, b[:1]))  # broadcast row
    _exact(torch.clamp(da, -1, 2), torch.clamp(a, -1, 2))
    _exact(torch.clamp(da, 2, -1), torch.clamp(a, 2, -1))  # min > max gives max
    _exact(torch.clamp(da, min=0), torch.clamp(a, min=0))
    _exact(torch.clamp(da, max=0), torch.clamp(a, max=0))
    _exact(torch.clamp_min(da, db), torch.clamp_min(a, b))
    _exact(torch.clamp_max(da, db), torch.clamp_max(a, b))
    e = da.clone()
    e.clamp_(-2, 1).clamp_min_(-1).clamp_max_(db)
    _exact(e, a.clone().clamp_(-2, 1).clamp_min_(-1).clamp_max_(b))
    out = torch.empty_like(da)
    torch.maximum(da, db, out=out)
    _exact(out, torch.maximum(a, b))
    if dtype == torch.int64:
        # an integer tensor clamped by a float bound promotes, as upstream
        _exact(torch.clamp(da, -1.5, 2.5), torch.clamp(a, -1.5, 2.5))


# --------------------------------------------- comparisons and selects
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int64])
def test_comparisons_where_masked_fill(dtype, no_fallback):
    """Exact logical ops: the same booleans / selections as upstream's CPU
    kernels, NaN included, over broadcasts, scalars, mixed dtypes and the
    in-place / out= forms."""
    g = torch.Generator().manual_seed(99)
    if dtype.is_floating_point:
        a = torch.randn(257, 1031, generator=g).to(dtype)
        b = torch.randn(257, 1031, generator=g).to(dtype)
        a[::13, ::7] = float("nan")
        b[:, ::9] = a[:, ::9]
    else:
        a = torch.randint(-5, 5, (257, 1031), generator=g, dtype=dtype)
        b = torch.randint(-5, 5, (257, 1031), generator=g, dtype=dtype)
    da, db = dev(a), dev(b)
    for fn in (torch.eq, torch.ne, torch.lt, torch.le, torch.gt, torch.ge):
        assert torch.equal(fn(da, db).cpu(), fn(a, b)), fn
        assert torch.equal(fn(da, 0.25).cpu(), fn(a, 0.25)), fn
        assert torch.equal(fn(da, db[0]).cpu(), fn(a, b[0])), fn  # row broadcast
    assert torch.equal((da < db.double()).cpu(), a < b.double())  # promotion
    out = torch.empty(257, 1031, dtype=torch.bool, device="supa")
    torch.ge(da, db, out=out)
    assert torch.equal(out.cpu(), a >= b)
    c = da.clone()
    c.lt_(db)
    assert torch.equal(c.cpu(), a.clone().lt_(b))
    if dtype.is_floating_point:
        assert torch.equal(torch.isnan(da).cpu(), torch.isnan(a))
    cond = da > 0
    _exact(torch.where(cond, da, db), torch.where(a > 0, a, b))  # NaN-aware equality
    _exact(torch.where(cond, da, 0), torch.where(a > 0, a, 0))
    _exact(torch.where(cond[0], da, db), torch.where((a > 0)[0], a, b))
    m = da.clone()
    m.masked_fill_(cond, -7)
    _exact(m, a.clone().masked_fill_(a > 0, -7))
    m = da.clone()
    m.masked_fill_((db > 0)[:, :1], torch.tensor(3))  # column mask, 0-dim value
    _exact(m, a.clone().masked_fill_((b > 0)[:, :1], torch.tensor(3)))
    _exact(torch.masked_fill(da, cond, 1), torch.masked_fill(a, a > 0, 1))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_half_with_float32_device_scalar(dtype, no_fallback):
    """A half-precision tensor with a 0-dim float32 device tensor: the common
    dtype is the half type (0-dim tensors do not promote a dimensioned one).
    Upstream's device kernels load both operands as the common type
    (Loops.cuh opmath_gpu_kernel_with_scalars -> BinaryFunctor<scalar_t,
    scalar_t>), so the float32 value is rounded to it first; the static
    kernels match the upstream CPU kernels given that rounded value, bit for
    bit, contiguous or not.  (Upstream's CPU kernels would use the unrounded
    value of a CPU 0-dim tensor: that is a different operand kind, bound as
    an immediate here.)"""
    x = seeded((257, 1030), 70, 3.0, dtype)
    s = torch.tensor(0.3000001, dtype=torch.float32)  # not representable in the half type
    sr = s.to(dtype)
    dx, ds = dev(x), dev(s)
    for got, want in (
        (dx * ds, x * sr),
        (ds * dx, sr * x),
        (dx + ds, x + sr),
        (torch.add(dx, ds, alpha=2), torch.add(x, sr, alpha=2)),
        (ds / dx, sr / x),
        (dx / ds, x / sr),
        (dx.t() * ds, x.t() * sr),
        (dx[:, 1::3] - ds, x[:, 1::3] - sr),
    ):
        assert got.dtype == dtype
        assert torch.equal(got.cpu(), want)
    y = dx.clone()
    y.mul_(ds)
    assert torch.equal(y.cpu(), x * sr)


def test_integer_and_bool_sums(no_fallback):
    """Sums of bool and integer tensors are int64 (upstream's rule), full and
    over dims, and a floating dtype argument converts first."""
    g = torch.Generator().manual_seed(71)
    b = torch.rand(300, 517, generator=g) > 0.3
    i32 = torch.randint(-1000, 1000, (300, 517), generator=g, dtype=torch.int32)
    i64 = torch.randint(-(2**40), 2**40, (4099,), generator=g)
    u8 = torch.randint(0, 255, (77, 5), generator=g, dtype=torch.uint8)
    for t in (b, i32, i64, u8):
        d = dev(t)
        got = d.sum()
        assert got.dtype == torch.int64 and torch.equal(got.cpu(), t.sum())
    for t, dims in ((b, 1), (i32, 0), (i32, (0, 1)), (u8, -1)):
        assert torch.equal(dev(t).sum(dims).cpu(), t.sum(dims))
        assert torch.equal(dev(t).sum(dims, keepdim=True).cpu(), t.sum(dims, keepdim=True))
    assert torch.equal(dev(i32).sum(dtype=torch.float32).cpu(), i32.sum(dtype=torch.float32))
    assert dev(torch.zeros(0, dtype=torch.bool)).sum().item() == 0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cross_entropy_label_smoothing(dtype, no_fallback):
    """The composite label-smoothing path (log_softmax, the nll term, a
    smoothing sum and the kept-row count over a bool mask) on the device,
    forward and backward, against upstream CPU."""
    g = torch.Generator().manual_seed(72)
    x = (torch.randn(300, 1000, generator=g) * 2).to(dtype)
    t = torch.randint(0, 1000, (300,), generator=g)
    t[::7] = -100
    for red in ("mean", "sum", "none"):
        dx = dev(x).requires_grad_()
        xc = x.clone().requires_grad_()
        got = F.cross_entropy(dx, dev(t), label_smoothing=0.1, reduction=red)
        want = F.cross_entropy(xc.float(), t, label_smoothing=0.1, reduction=red)
        tol = dict(rtol=1e-5, atol=1e-5) if dtype == torch.float32 else dict(rtol=2e-2, atol=2e-2)
        torch.testing.assert_close(got.float().cpu(), want.detach(), **tol)
        got.sum().backward()
        want.sum().backward()
        torch.testing.assert_close(dx.grad.float().cpu(), xc.grad.float(), **tol)
