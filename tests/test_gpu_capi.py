"""Parity through the C ABI (include/supa_amd.h) with raw device pointers: the
HIP kernels against the oracle on seeded inputs, with no PyTorch types in any
call.  Device buffers come from torch's HIP allocator (``cuda`` tensors)."""
import ctypes

import numpy as np
import pytest
import torch

import capi as A
import oracle as O
from helpers import bf16_ulp_dist, f32_ulp_dist

pytestmark = pytest.mark.gpu

DEV = "cuda"


def seeded(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def run(rc):
    torch.cuda.synchronize()
    assert rc == 0, A.lib().supa_amd_status_string(rc) if hasattr(A.lib(), "supa_amd_status_string") else rc


@pytest.mark.parametrize("n", [1, 7, 16, 4096 * 4096 + 3])
def test_add_mul_div_contiguous(n):
    L = A.lib()
    a, b = seeded((n,), 1), seeded((n,), 2)
    da, db = a.to(DEV), b.to(DEV)
    out = torch.empty(n, device=DEV)
    for fn, op in [(lambda d: L.supa_amd_add(d, 1.0, 1, None), O.ADD), (lambda d: L.supa_amd_mul(d, None), O.MUL),
                   (lambda d: L.supa_amd_div(d, 0, None), O.DIV)]:
        d = A.flat_desc(out, da, db)
        run(fn(ctypes.byref(d)))
        assert np.array_equal(out.cpu().numpy(), O.binary(op, a.numpy(), b.numpy())), op


def test_add_alpha_scalar_and_broadcast_nd():
    L = A.lib()
    a = seeded((64, 4096), 3)
    bias = seeded((4096,), 4, 0.02)
    da, dbias = a.to(DEV), bias.to(DEV)
    out = torch.empty(64, 4096, device=DEV)
    d = A.nd_desc([4096, 64], [(out, [1, 4096]), (da, [1, 4096]), (dbias, [1, 0])], A.F32)
    run(L.supa_amd_add(ctypes.byref(d), -0.5, 0, None))
    assert np.array_equal(out.cpu().numpy(), O.binary(O.ADD, a.numpy(), bias.numpy(), -0.5))
    # immediate scalar operand
    d = A.flat_desc(out, da, 2.5)
    run(L.supa_amd_mul(ctypes.byref(d), None))
    assert np.array_equal(out.cpu().numpy(), O.binary(O.MUL, a.numpy(), np.float32(2.5)))


def test_c2_mixed_dtype_both_legs():
    """bf16 x + f32 bias -> f32, contiguous and transposed-view x."""
    L = A.lib()
    x = seeded((8, 256, 512), 5, dtype=torch.bfloat16)
    bias = seeded((512,), 6, 0.02)
    dx, dbias = x.to(DEV), bias.to(DEV)
    ref = O.binary(O.ADD, x.float().numpy(), bias.numpy())
    out = torch.empty(8, 256, 512, device=DEV)
    d = A.nd_desc([512, 256 * 8], [(out, [1, 512]), (dx, [1, 512]), (dbias, [1, 0])], A.F32)
    run(L.supa_amd_add(ctypes.byref(d), 1.0, 1, None))
    assert np.array_equal(out.cpu().numpy(), ref)
    # transposed leg: memory order [8, 512, 256]; iterate fastest-first
    xt = seeded((8, 512, 256), 7, dtype=torch.bfloat16)
    dxt = xt.to(DEV)
    outt = torch.empty(8, 512, 256, device=DEV)
    d = A.nd_desc([256, 512, 8], [(outt, [1, 256, 131072]), (dxt, [1, 256, 131072]), (dbias, [0, 1, 0])], A.F32)
    run(L.supa_amd_add(ctypes.byref(d), 1.0, 1, None))
    reft = O.binary(O.ADD, xt.float().numpy().transpose(0, 2, 1), bias.numpy()).transpose(0, 2, 1)
    assert np.array_equal(outt.cpu().numpy(), reft)
    # gelu-tanh on the f32 result
    g = torch.empty_like(out)
    d = A.flat_desc(g, out)
    run(L.supa_amd_unary(ctypes.byref(d), A.GELU_TANH, None))
    assert O.gelu_tanh_forward_equal(g.cpu().numpy(), ref)


@pytest.mark.parametrize("op", [A.GELU, A.GELU_TANH, A.SILU, A.SIGMOID, A.TANH, A.EXP, A.LOG, A.ERF])
def test_unary_f32_bit_exact(op):
    L = A.lib()
    x = seeded((1 << 20,), 10 + op, 3.0)
    if op == A.LOG:
        x = x.abs() + 1e-3
    dx = x.to(DEV)
    out = torch.empty_like(dx)
    d = A.flat_desc(out, dx)
    run(L.supa_amd_unary(ctypes.byref(d), op, None))
    if op == A.GELU_TANH:
        assert O.gelu_tanh_forward_equal(out.cpu().numpy(), x.numpy())
        return
    assert np.array_equal(out.cpu().numpy().view(np.int32), O.unary(op, x.numpy()).view(np.int32))


@pytest.mark.parametrize("op", [A.GELU, A.GELU_TANH, A.SILU, A.SIGMOID, A.TANH])
def test_unary_backward_f32_bit_exact(op):
    L = A.lib()
    x = seeded((1 << 18,), 20 + op, 3.0)
    dy = seeded((1 << 18,), 30 + op)
    if op in (A.SIGMOID, A.TANH):
        x = torch.sigmoid(x) if op == A.SIGMOID else torch.tanh(x)
    dx, ddy = x.to(DEV), dy.to(DEV)
    out = torch.empty_like(dx)
    d = A.flat_desc(out, ddy, dx)
    run(L.supa_amd_unary_backward(ctypes.byref(d), op, None))
    assert np.array_equal(out.cpu().numpy(), O.unary_backward(op, dy.numpy(), x.numpy()))


def test_bf16_unary_within_one_ulp_of_f32_oracle():
    L = A.lib()
    x = seeded((1 << 18,), 40, 2.0, torch.bfloat16)
    dx = x.to(DEV)
    out = torch.empty_like(dx)
    d = A.flat_desc(out, dx)
    run(L.supa_amd_unary(ctypes.byref(d), A.GELU, None))
    ref = O.f32_to_bf16(O.unary(O.GELU, x.float().numpy()))
    assert np.array_equal(bits(out), ref)


def test_copy_casts():
    L = A.lib()
    x = seeded((1000, 33), 41, 100.0)
    dx = x.to(DEV)
    for dt in (torch.bfloat16, torch.float16, torch.float64, torch.int32, torch.int64, torch.bool, torch.uint8):
        out = torch.empty(1000, 33, dtype=dt, device=DEV)
        d = A.flat_desc(out, dx, common=torch.float32)
        run(L.supa_amd_copy(ctypes.byref(d), None))
        assert torch.equal(out.cpu(), x.to(dt)), dt


@pytest.mark.parametrize("rows, cols", [(4, 10), (64, 1000), (16, 128256), (3, 7)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_log_softmax_forward_backward(rows, cols, dtype):
    L = A.lib()
    x = seeded((rows, cols), 50, 2.0, dtype)
    g = seeded((rows, cols), 51, 1.0, dtype)
    dx, dg = x.to(DEV), g.to(DEV)
    y = torch.empty_like(dx)
    run(L.supa_amd_log_softmax_forward(dx.data_ptr(), A.dtype_code(dtype), y.data_ptr(), A.dtype_code(dtype),
                                       rows, cols, None))
    ref = O.log_softmax(x.float().numpy())
    if dtype == torch.float32:
        np.testing.assert_allclose(y.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    else:
        assert bf16_ulp_dist(bits(y), O.f32_to_bf16(ref)).max() <= 1
    gi = torch.empty_like(dx)
    run(L.supa_amd_log_softmax_backward(dg.data_ptr(), y.data_ptr(), A.dtype_code(dtype), gi.data_ptr(),
                                        A.dtype_code(dtype), rows, cols, None))
    refb = O.log_softmax_backward(g.float().numpy(), y.cpu().float().numpy())
    if dtype == torch.float32:
        np.testing.assert_allclose(gi.cpu().numpy(), refb, rtol=1e-5, atol=1e-5)
    else:
        assert bf16_ulp_dist(bits(gi), O.f32_to_bf16(refb)).max() <= 1


@pytest.mark.parametrize("reduction", [A.RED_MEAN, A.RED_SUM, A.RED_NONE])
def test_nll_forward_backward(reduction):
    L = A.lib()
    N, C = 300, 5000
    lp = torch.from_numpy(O.log_softmax(seeded((N, C), 60, 2.0).numpy()))
    g = torch.Generator().manual_seed(61)
    t = torch.randint(0, C, (N,), generator=g)
    t[torch.randperm(N, generator=g)[:15]] = -100
    w = torch.rand(C, generator=g) + 0.5
    dlp, dt, dw = lp.to(DEV), t.to(DEV), w.to(DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    red = {A.RED_MEAN: "mean", A.RED_SUM: "sum", A.RED_NONE: "none"}[reduction]
    out = torch.empty(N if reduction == A.RED_NONE else 1, device=DEV)
    tw = torch.zeros(1, device=DEV)
    run(L.supa_amd_nll_loss_forward(dlp.data_ptr(), A.F32, dt.data_ptr(), dw.data_ptr(), N, C, reduction, -100,
                                    out.data_ptr(), tw.data_ptr(), flag.data_ptr(), None))
    ro, rtw = O.nll_loss(lp.numpy(), t.numpy(), w.numpy(), red, -100)
    np.testing.assert_allclose(out.cpu().numpy().reshape(np.shape(ro)), ro, rtol=1e-5)
    if reduction != A.RED_NONE:
        np.testing.assert_allclose(tw.cpu().numpy()[0], rtw, rtol=1e-6)
    go = seeded((N,), 62) if reduction == A.RED_NONE else torch.ones(1)
    dgo = go.to(DEV)
    gi = torch.full((N, C), 7.0, device=DEV)  # every element must be overwritten
    run(L.supa_amd_nll_loss_backward(dgo.data_ptr(), A.F32, dt.data_ptr(), dw.data_ptr(), tw.data_ptr(), N, C,
                                     reduction, -100, gi.data_ptr(), flag.data_ptr(), None))
    rg = O.nll_loss_backward(go.numpy(), t.numpy(), N, C, float(tw.cpu()[0]), w.numpy(), red, -100)
    assert np.array_equal(gi.cpu().numpy(), rg)
    assert flag.item() == 0
    # an out-of-range target raises the flag and contributes nothing
    t_bad = t.clone()
    t_bad[5] = C + 3
    run(L.supa_amd_nll_loss_forward(dlp.data_ptr(), A.F32, t_bad.to(DEV).data_ptr(), None, N, C, A.RED_SUM, -100,
                                    out.data_ptr(), tw.data_ptr(), flag.data_ptr(), None))
    assert flag.item() == 1


@pytest.mark.parametrize("loss", [A.LOSS_MSE, A.LOSS_SMOOTH_L1, A.LOSS_BCE])
@pytest.mark.parametrize("reduction", [A.RED_NONE, A.RED_MEAN, A.RED_SUM])
def test_losses_forward(loss, reduction):
    L = A.lib()
    rows, cols = 32, 65536
    g = torch.Generator().manual_seed(70)
    x = torch.randn(rows, cols, generator=g)
    t = (torch.rand(rows, cols, generator=g) < 0.3).float() if loss == A.LOSS_BCE else torch.randn(rows, cols,
                                                                                                     generator=g)
    pw = torch.rand(cols, generator=g) * 1.5 + 0.5
    dx, dt, dpw = x.to(DEV), t.to(DEV), pw.to(DEV)
    red = {A.RED_NONE: "none", A.RED_MEAN: "mean", A.RED_SUM: "sum"}[reduction]
    opo = {A.LOSS_MSE: O.MSE, A.LOSS_SMOOTH_L1: O.SMOOTH_L1, A.LOSS_BCE: O.BCE_LOGITS}[loss]
    has_pw = loss == A.LOSS_BCE
    ref = O.loss(opo, x.numpy(), t.numpy(), pw.numpy() if has_pw else None, reduction=red, beta=1.0)
    ws = torch.zeros(L.supa_amd_loss_workspace_bytes(rows * cols), dtype=torch.uint8, device=DEV)
    ops = [(None, [1, cols]), (dx, [1, cols]), (dt, [1, cols])] + ([(dpw, [1, 0])] if has_pw else [])
    out = torch.empty(rows, cols, device=DEV) if reduction == A.RED_NONE else torch.empty(1, device=DEV)
    ops[0] = (out, [1, cols] if reduction == A.RED_NONE else [0, 0])
    d = A.nd_desc([cols, rows], ops, A.F32)
    for _ in range(2):  # the workspace counter must be left at zero
        run(L.supa_amd_loss_forward(ctypes.byref(d), loss, reduction, 1.0, int(has_pw), 0, out.data_ptr(),
                                    ws.data_ptr(), ws.numel(), None))
        if reduction == A.RED_NONE:
            assert np.array_equal(out.cpu().numpy(), ref)
        else:
            np.testing.assert_allclose(out.cpu().numpy()[0], ref, rtol=1e-5)


def test_sum_deterministic_and_accurate():
    L = A.lib()
    x = seeded((33554432 + 5,), 80)
    dx = x.to(DEV)
    out = torch.empty(1, device=DEV)
    ws = torch.zeros(L.supa_amd_sum_workspace_bytes(x.numel()), dtype=torch.uint8, device=DEV)
    d = A.nd_desc([x.numel()], [(out, [0]), (dx, [1])], A.F32)
    vals = []
    for _ in range(3):
        run(L.supa_amd_sum(ctypes.byref(d), 1.0, ws.data_ptr(), ws.numel(), None))
        vals.append(out.cpu().numpy()[0])
    assert vals[0] == vals[1] == vals[2]
    ref = O.sum_f32(x.numpy())
    assert abs(vals[0] - ref) <= 1e-5 * np.abs(x.numpy()).sum() / np.sqrt(x.numel())


def test_foreach_and_fused_adamw_bit_exact():
    L = A.lib()
    shapes = [(4096, 1024), (1024,), (333, 17), (11008, 64)]
    g = torch.Generator().manual_seed(90)
    params = [torch.randn(s, generator=g) * 0.02 for s in shapes]
    grads = [torch.randn(s, generator=g) * 1e-3 for s in shapes]
    dp = [p.to(DEV) for p in params]
    dg = [x.to(DEV) for x in grads]
    dm = [torch.zeros_like(p) for p in dp]
    dv = [torch.zeros_like(p) for p in dp]
    steps = [torch.zeros(1, device=DEV) for _ in shapes]
    numel = A.i64_array([p.numel() for p in dp])
    hp = [p.numpy().copy().ravel() for p in params]
    hm = [np.zeros_like(x) for x in hp]
    hv = [np.zeros_like(x) for x in hp]
    for step in range(1, 11):
        run(L.supa_amd_foreach_binary(0, len(steps), A.ptr_array(steps), A.ptr_array(steps), None,
                                      A.i64_array([1] * len(steps)), A.F32, 1.0, 1.0, None))
        run(L.supa_amd_fused_adamw(len(dp), A.ptr_array(dp), A.ptr_array(dg), A.ptr_array(dm), A.ptr_array(dv),
                                   None, A.ptr_array(steps), numel, A.F32, 1e-4, None, 0.9, 0.999, 0.01, 1e-8, 0, 0,
                                   None, None, None))
        for i in range(len(shapes)):
            O.adamw_step(hp[i], grads[i].numpy().ravel().copy(), hm[i], hv[i], float(step), 1e-4, 0.9, 0.999, 0.01,
                         1e-8)
    assert all(s.item() == 10.0 for s in steps)
    for i in range(len(shapes)):
        assert np.array_equal(dp[i].cpu().numpy().ravel(), hp[i]), i
        assert np.array_equal(dm[i].cpu().numpy().ravel(), hm[i]), i
        assert np.array_equal(dv[i].cpu().numpy().ravel(), hv[i]), i
    # foreach list add with alpha, then scalar mul
    out = [torch.empty_like(p) for p in dp]
    run(L.supa_amd_foreach_binary(0, len(dp), A.ptr_array(out), A.ptr_array(dp), A.ptr_array(dg), numel, A.F32,
                                  0.0, -2.0, None))
    for i in range(len(shapes)):
        assert np.array_equal(out[i].cpu().numpy().ravel(), O.binary(O.ADD, hp[i], grads[i].numpy().ravel(), -2.0))
    run(L.supa_amd_foreach_binary(1, len(dp), A.ptr_array(out), A.ptr_array(out), None, numel, A.F32, 0.5, 1.0, None))
    for i in range(len(shapes)):
        ref = O.binary(O.MUL, O.binary(O.ADD, hp[i], grads[i].numpy().ravel(), -2.0), np.float32(0.5))
        assert np.array_equal(out[i].cpu().numpy().ravel(), ref)


@pytest.mark.parametrize("dtype,code", [(torch.float32, A.F32), (torch.bfloat16, A.BF16)])
def test_fused_cross_entropy_capi(dtype, code):
    L = A.lib()
    N, C = 200, 4104
    x = seeded((N, C), 90, 2.0, dtype)
    g = torch.Generator().manual_seed(91)
    t = torch.randint(0, C, (N,), generator=g)
    t[torch.randperm(N, generator=g)[:9]] = -100
    dx, dt = x.to(DEV), t.to(DEV)
    lse = torch.empty(N, device=DEV)
    cnt = torch.empty(1, device=DEV)
    ws = torch.empty(L.supa_amd_cross_entropy_workspace_bytes(N) // 4, device=DEV)
    flag = torch.zeros(1, dtype=torch.int32, device=DEV)
    out = torch.empty((), dtype=dtype, device=DEV)
    run(L.supa_amd_cross_entropy_forward(dx.data_ptr(), code, dt.data_ptr(), N, C, -100, A.RED_MEAN, out.data_ptr(),
                                         lse.data_ptr(), cnt.data_ptr(), ws.data_ptr(), ws.numel() * 4,
                                         flag.data_ptr(), None))
    ref, rlse, rcnt = O.cross_entropy(x.double().numpy(), t.numpy(), "mean", -100)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert abs(out.double().item() - float(ref)) <= tol * abs(float(ref))
    assert cnt.item() == rcnt == N - 9
    np.testing.assert_allclose(lse.cpu().double().numpy(), rlse, rtol=1e-6)
    go = torch.ones((), dtype=dtype, device=DEV)
    gx = torch.full((N, C), 7.0, dtype=dtype, device=DEV)  # every element must be overwritten
    run(L.supa_amd_cross_entropy_backward(go.data_ptr(), dx.data_ptr(), code, dt.data_ptr(), lse.data_ptr(),
                                          cnt.data_ptr(), N, C, -100, A.RED_MEAN, gx.data_ptr(), flag.data_ptr(),
                                          None))
    gref = O.cross_entropy_backward(np.ones(1), x.double().numpy(), t.numpy(), rlse, rcnt, "mean", -100)
    if dtype == torch.float32:
        np.testing.assert_allclose(gx.cpu().numpy(), gref, rtol=1e-5, atol=1e-6 * np.abs(gref).max())
    else:
        assert bf16_ulp_dist(bits(gx), O.f64_to_bf16(gref)).max() <= 1
    assert flag.item() == 0


@pytest.mark.parametrize("reduction", [A.RED_NONE, A.RED_MEAN])
def test_bce_logits_backward_capi(reduction):
    L = A.lib()
    R, C = 8, 70000
    g = torch.Generator().manual_seed(95)
    x = torch.randn(R, C, generator=g)
    t = (torch.rand(R, C, generator=g) < 0.3).float()
    pw = torch.rand(C, generator=g) * 1.5 + 0.5
    w = torch.rand(R, C, generator=g) + 0.5
    go = torch.randn(R, C, generator=g) if reduction == A.RED_NONE else torch.ones(())
    dx, dt, dpw, dw, dgo = x.to(DEV), t.to(DEV), pw.to(DEV), w.to(DEV), go.to(DEV)
    gi = torch.empty(R, C, device=DEV)
    gstr = [1, C] if reduction == A.RED_NONE else [0, 0]
    d = A.nd_desc([C, R], [(gi, [1, C]), (dgo, gstr), (dx, [1, C]), (dt, [1, C]), (dpw, [1, 0]), (dw, [1, C])], A.F32)
    L.supa_amd_bce_logits_backward.argtypes = [ctypes.POINTER(A.EwDesc), ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                               ctypes.c_double, ctypes.c_void_p]
    run(L.supa_amd_bce_logits_backward(ctypes.byref(d), 1, 1, 1 if reduction == A.RED_MEAN else 0, float(R * C), None))
    red = "none" if reduction == A.RED_NONE else "mean"
    gref = O.loss_backward(O.BCE_LOGITS, go.numpy(), x.numpy(), t.numpy(), pw.numpy(), w.numpy(), reduction=red)
    assert np.array_equal(gi.cpu().numpy(), gref)


def _bits(t):
    return t.cpu().view({1: torch.uint8, 2: torch.int16, 4: torch.int32, 8: torch.int64}[t.element_size()])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_amp_unscale_capi(dtype):
    """_amp_foreach_non_finite_check_and_unscale_ through the C ABI against
    upstream torch's own CPU kernel on the same tensors: every element times
    inv_scale (1/3 rounds, 2^-16 is exact, exactly 1 leaves the tensors
    untouched), and found_inf set by one inf or NaN anywhere in the list.
    NaN elements compare as NaN: upstream's CPU kernel rewrites a bfloat16 NaN
    as 0xFFFF even when inv_scale is 1 (its vectorised bfloat16 conversion),
    where the device kernel leaves the element as it was."""
    L = A.lib()
    shapes = [(4096, 1030), (7,), (333, 17)]
    for inv, poison in [(1.0 / 3.0, None), (2.0 ** -16, None), (0.5, float("inf")), (1.0, float("nan")),
                        (0.25, float("-inf"))]:
        host = [seeded(s, 100 + i, 50.0).to(dtype) for i, s in enumerate(shapes)]
        if poison is not None:
            host[2].view(-1)[100] = poison
        devs = [h.to(DEV) for h in host]
        found = torch.zeros(1, device=DEV)
        inv_t = torch.tensor([inv], dtype=torch.float32)
        dinv = inv_t.to(DEV)
        run(L.supa_amd_amp_unscale(len(devs), A.ptr_array(devs), A.i64_array([t.numel() for t in devs]),
                                   A.dtype_code(dtype), found.data_ptr(), dinv.data_ptr(), None))
        ref_found = torch.zeros(1)
        torch._amp_foreach_non_finite_check_and_unscale_(host, ref_found, inv_t)
        assert found.item() == ref_found.item() == (0.0 if poison is None else 1.0), (inv, poison)
        for d, h in zip(devs, host):
            nan = torch.isnan(h)
            assert torch.equal(torch.isnan(d.cpu()), nan), (inv, poison, d.shape)
            assert torch.equal(_bits(d)[~nan], _bits(h)[~nan]), (inv, poison, d.shape)


def test_amp_update_scale_capi():
    """_amp_update_scale_ through the C ABI against upstream torch's CPU kernel
    over a run of overflow / clean steps (growth every 3 clean steps, backoff
    on overflow), then a growth that would overflow float32 (scale kept)."""
    L = A.lib()
    for start in [65536.0, 3.0e38]:
        scale = torch.tensor([start], device=DEV)
        tracker = torch.zeros(1, dtype=torch.int32, device=DEV)
        rs, rt = torch.tensor([start]), torch.zeros(1, dtype=torch.int32)
        for f in [0, 0, 0, 1, 0, 0, 0, 0, 1, 1, 0, 0, 0, 0]:
            fi = torch.tensor([float(f)])
            dfi = fi.to(DEV)
            run(L.supa_amd_amp_update_scale(scale.data_ptr(), tracker.data_ptr(), dfi.data_ptr(), 2.0, 0.5, 3, None))
            torch._amp_update_scale_(rs, rt, fi, 2.0, 0.5, 3)
            assert scale.item() == rs.item() and tracker.item() == rt.item(), (start, f)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16, torch.int64, torch.uint8,
                                   torch.bool])
def test_fill_capi(dtype):
    """fill_ through the C ABI (the value as an immediate scalar operand)
    against torch.full on the CPU, at sizes with and without a vector tail."""
    L = A.lib()
    values = [0, 1, 7] if dtype in (torch.uint8, torch.bool) else [0, 1, 3.25, -7, 0.1]
    if dtype == torch.int64:
        values = [0, 1, -7, 2 ** 40 + 3]
    for n in [1, 1000, 4096 * 1024 + 5]:
        out = torch.empty(n, dtype=dtype, device=DEV)
        for v in values:
            d = A.flat_desc(out, v)
            run(L.supa_amd_fill(ctypes.byref(d), None))
            assert torch.equal(out.cpu(), torch.full((n,), v, dtype=dtype)), (n, v)
