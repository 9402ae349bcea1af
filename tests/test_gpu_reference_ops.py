"""More of the reference's kernel tests, case for case, with their shapes,
dtypes, tolerances and comparisons (CPU result against the supa result):

* test_activation_{elu,hardsigmoid,hardswish,hardtanh,leaky_relu,
  log_sigmoid,mish,softplus,threshold,hardshrink,softshrink}_kernel.py:
  forward and backward at default parameters (threshold exact at
  (0.5 | 1.0, 20), elu and threshold in place too; hardswish's inputs of
  exactly +-3 moved off the kink);
* test_activation_glu_kernel.py (its bfloat16 atol 1e-2; it compares the
  gradients for bfloat16 only and the outputs again otherwise; here float32's
  gradients are compared too.  Upstream CPU's float16 glu backward rounds
  its steps to float16, so where 1 - sigmoid cancels it is a few percent
  from the device's float32 arithmetic, which the oracle checks bit for bit
  in test_gpu_activations.py) and test_activation_prelu_kernel.py
  (forward only there: its backward case waits on a sum it lacks; the
  backward is checked in test_gpu_activations.py);
* test_binary_div_floor_kernel.py, test_binary_div_trunc_kernel.py: true
  division, rounding_mode 'floor' / 'trunc' (float16 quotients kept within
  512 for floor, as there) and their backward;
* test_binary_mul_kernel.py: Tensor, one-element broadcast, in place, Scalar
  and in-place Scalar products (its mixed-dtype cases are in
  test_gpu_reference_shapes.py);
* test_pow_kernel.py (tensor ** tensor and tensor ** a 0-dim CPU int
  tensor, out of place and in place), test_abs_kernel.py (N(0, 1) and
  all-zero inputs, out of place and in place);
* test_lerp.py, test_linalg_vector_norm.py (bf16 input, float32
  accumulation), test_fused_adam_kernel.py, test_fused_sgd_kernel.py (one
  step of SGD(fused=True) on a cross-entropy loss against the CPU's
  unfused SGD);
* test_amp.py: GradScaler.scale and load_state_dict, and its clipping
  scaling cases (a two-layer Linear model trained with and without
  GradScaler + clip_grad_norm_; the matrix products are outside this path
  and take the CPU fallback, everything else runs on the device).  Its
  autocast case is not mirrored: device autocast is not part of this build."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu

SUPA = "supa"
RTOL = {torch.float32: 1.3e-6, torch.bfloat16: 1.6e-2, torch.float16: 1e-3}
ATOL = {torch.float32: 1e-5, torch.bfloat16: 1e-5, torch.float16: 1e-5}
DTYPES = [torch.float32, torch.bfloat16, torch.float16]
BR200 = [(16,), (1024, 512), (1023, 511), (1025, 513), (1028, 2135)]
_seed = [9000]


def rand(shape, dtype, lo=None, hi=None):
    _seed[0] += 1
    g = torch.Generator().manual_seed(_seed[0])
    x = torch.randn(shape, generator=g) if lo is None else torch.rand(shape, generator=g) * (hi - lo) + lo
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
ACTS = {
    "elu": F.elu, "hardsigmoid": F.hardsigmoid, "hardswish": F.hardswish, "hardtanh": F.hardtanh,
    "leaky_relu": F.leaky_relu, "log_sigmoid": torch.nn.LogSigmoid(), "mish": F.mish, "softplus": F.softplus,
    "hardshrink": F.hardshrink, "softshrink": F.softshrink,
}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", BR200)
@pytest.mark.parametrize("name", list(ACTS))
def test_activation_forward_backward(name, shape, dtype, no_fallback):
    """test_activation_<name>_kernel.py (requires_grad True there)."""
    xc = rand(shape, dtype)
    if name == "hardswish":  # test_activation_hardswish_kernel.py:36-42
        xc = torch.where(xc.abs() == 3, xc + 0.5, xc)
    xs = xc.to(SUPA)
    xc.requires_grad_(True)
    xs.requires_grad_(True)
    fn = ACTS[name]
    yc, ys = fn(xc), fn(xs)
    ref_allclose(yc, ys, RTOL[dtype], ATOL[dtype])
    gc, gs = pair(yc.shape, dtype)
    yc.backward(gc)
    ys.backward(gs)
    ref_allclose(xc.grad, xs.grad, RTOL[dtype], ATOL[dtype])


GLU_SHAPES = [(16,), (1024, 512), (1023, 510), (1025, 514), (1028, 2136)]
GLU_ATOL = {torch.float32: 1e-5, torch.bfloat16: 1e-2, torch.float16: 1e-5}


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", GLU_SHAPES)
def test_glu(shape, dtype, no_fallback):
    """test_activation_glu_kernel.py: glu over the last dim, forward and
    backward with an N(0, 1) upstream gradient."""
    xc, xs = pair(shape, dtype, True)
    yc, ys = F.glu(xc), F.glu(xs)
    ref_allclose(yc, ys, RTOL[dtype], GLU_ATOL[dtype])
    gc, gs = pair(yc.shape, dtype)
    yc.backward(gc)
    ys.backward(gs)
    if dtype == torch.float16:
        ref_allclose(yc, ys, RTOL[dtype], GLU_ATOL[dtype])
    else:
        ref_allclose(xc.grad, xs.grad, RTOL[dtype], GLU_ATOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", BR200)
def test_prelu(shape, dtype, no_fallback):
    """test_activation_prelu_kernel.py: nn.PReLU with one weight per channel
    (dim 1; one weight for a 1-d input), an N(0, 1) weight."""
    xc, xs = pair(shape, dtype)
    n = shape[1] if len(shape) >= 2 else 1
    wc, ws = pair((n,), dtype)
    ref_allclose(F.prelu(xc, wc), F.prelu(xs, ws), RTOL[dtype], ATOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", BR200)
def test_elu_inplace(shape, dtype, no_fallback):
    """test_activation_elu_kernel.py:43-52."""
    xc, xs = pair(shape, dtype)
    ref_allclose(F.elu_(xc), F.elu_(xs), RTOL[dtype], ATOL[dtype])


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("threshold", [0.5, 1.0])
@pytest.mark.parametrize("shape", BR200)
def test_threshold(shape, threshold, dtype, no_fallback):
    """test_activation_threshold_kernel.py: exact, forward, backward, in place
    (value 20)."""
    xc, xs = pair(shape, dtype, requires_grad=True)
    yc, ys = F.threshold(xc, threshold, 20), F.threshold(xs, threshold, 20)
    ref_allclose(yc, ys, 0, 0)
    gc, gs = pair(yc.shape, dtype)
    yc.backward(gc)
    ys.backward(gs)
    ref_allclose(xc.grad, xs.grad, 0, 0)
    xc, xs = pair(shape, dtype)
    ref_allclose(F.threshold_(xc, threshold, 20), F.threshold_(xs, threshold, 20), 0, 0)


# ------------------------------------------------------------ division
@pytest.mark.parametrize("mode", ["floor", "trunc"])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", BR200)
def test_div_rounding_modes(shape, dtype, mode, no_fallback):
    """test_binary_div_floor_kernel.py / test_binary_div_trunc_kernel.py:
    a / b (bf16 against atol 1e-2 in the floor file), rounding_mode, and the
    backward of both inputs."""
    ac, as_ = pair(shape, dtype)
    bc, bs = pair(shape, dtype)
    if mode == "floor":
        ref_allclose(ac / bc, as_ / bs, 0 if dtype == torch.bfloat16 else RTOL[dtype],
                     1e-2 if dtype == torch.bfloat16 else ATOL[dtype], equal_nan=True)
        if dtype == torch.float16:  # test_binary_div_floor_kernel.py:47-52: quotients within 512
            bc = torch.where(bc == 0, torch.ones_like(bc), bc)  # a zero divisor would never get there
            for _ in range(64):
                big = (ac / bc).abs() > 512
                if not bool(big.any()):
                    break
                bc = torch.where(big, bc * 2, bc)
            bs = bc.to(SUPA)
    ref_allclose(torch.div(ac, bc, rounding_mode=mode), torch.div(as_, bs, rounding_mode=mode), RTOL[dtype],
                 ATOL[dtype], equal_nan=True)
    ac, as_ = pair(shape, dtype, requires_grad=True)
    bc, bs = pair(shape, dtype, requires_grad=True)
    oc, os_ = torch.div(ac, bc, rounding_mode=mode), torch.div(as_, bs, rounding_mode=mode)
    gc, gs = pair(oc.shape, dtype)
    oc.backward(gc)
    os_.backward(gs)
    ref_allclose(ac.grad, as_.grad, RTOL[dtype], ATOL[dtype], equal_nan=True)
    ref_allclose(bc.grad, bs.grad, RTOL[dtype], ATOL[dtype], equal_nan=True)


# ------------------------------------------------------------ mul
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", BR200)
def test_mul_forms(shape, dtype, no_fallback):
    """test_binary_mul_kernel.py:31-90."""
    ac, as_ = pair(shape, dtype)
    bc, bs = pair(shape, dtype)
    ref_allclose(ac * bc, as_ * bs, RTOL[dtype], ATOL[dtype])
    b1 = rand([1], dtype)
    ref_allclose(ac * b1, as_ * b1.to(SUPA), RTOL[dtype], ATOL[dtype])
    ref_allclose(torch.mul(ac, 3.0), torch.mul(as_, 3.0), RTOL[dtype], ATOL[dtype])
    for v in [0.5, 1.0, 1000]:
        c, s = ac.clone(), as_.clone()
        c.mul_(v)
        s.mul_(v)
        ref_allclose(c, s, RTOL[dtype], ATOL[dtype])
    ac.mul_(bc)
    as_.mul_(bs)
    ref_allclose(ac, as_, RTOL[dtype], ATOL[dtype])


# ------------------------------------------------------------ lerp, vector norm
@pytest.mark.parametrize("shape", BR200)
def test_lerp(shape, no_fallback):
    """test_lerp.py:24-43 (float32, weight 0.5, rtol 1e-5, atol 5e-5)."""
    sc, ss = pair(shape, torch.float32)
    ec, es = pair(shape, torch.float32)
    ref_allclose(torch.lerp(sc, ec, 0.5), torch.lerp(ss, es, 0.5), 1e-5, 5e-5, equal_nan=True)


@pytest.mark.parametrize("shape, ord, dim, keepdim", [((1, 384, 1, 8, 8), 2, 1, True), ((1, 384, 8, 8), 2, 1, True),
                                                     ((128, 5120), 2, 1, False), ((32, 128, 64), 2, -1, False)])
def test_linalg_vector_norm_bf16_f32_accumulation(shape, ord, dim, keepdim, no_fallback):
    """test_linalg_vector_norm.py:28-50: bf16 input, dtype=float32."""
    xc, xs = pair(shape, torch.bfloat16)
    yc = torch.linalg.vector_norm(xc, ord=ord, dim=dim, keepdim=keepdim, dtype=torch.float32)
    ys = torch.linalg.vector_norm(xs, ord=ord, dim=dim, keepdim=keepdim, dtype=torch.float32)
    ref_allclose(yc, ys, 1e-5, 1e-5)


# ------------------------------------------------------------ fused Adam
@pytest.mark.parametrize("shape", [(1, 100), (512, 1024), (1025, 513), (1023, 511), (1028, 2135)])
def test_fused_adam_on_cross_entropy(shape, no_fallback):
    """test_fused_adam_kernel.py: as test_fused_adam_w_kernel.py with Adam."""
    wc = rand(shape, torch.float32, lo=-1, hi=1)
    ws = wc.to(SUPA)
    g = torch.Generator().manual_seed(_seed[0] + 3)
    target = torch.randint(0, shape[1], (shape[0],), generator=g)
    wc.requires_grad_(True)
    ws.requires_grad_(True)
    crit = torch.nn.CrossEntropyLoss()
    oc = torch.optim.Adam(params=[wc], lr=1e-2, weight_decay=0.01, fused=False)
    os_ = torch.optim.Adam(params=[ws], lr=1e-2, weight_decay=0.01, fused=True)
    ts = target.to(SUPA)
    for _ in range(5):
        crit(wc, target).backward()
        oc.step()
        wc.grad.zero_()
        crit(ws, ts).backward()
        os_.step()
        ws.grad.zero_()
        ref_allclose(wc, ws, 1e-2, 1e-3, equal_nan=True)


# ------------------------------------------------------------ GradScaler
def test_grad_scaling_scale(no_fallback):
    """test_amp.py:12-31: nested outputs scaled by init_scale 2."""
    scaler = torch.amp.GradScaler(SUPA, init_scale=2.0)
    t0 = torch.full((1,), 4.0, dtype=torch.bfloat16, device=SUPA)
    t1 = torch.full((1,), 4.0, dtype=torch.bfloat16, device=SUPA)
    out = scaler.scale((t1.clone(), (t0.clone(), t1.clone()), [t0.clone(), (t1.clone(), t0.clone())]))
    flat = [out[0], out[1][0], out[1][1], out[2][0], out[2][1][0], out[2][1][1]]
    assert all(float(v) == 8.0 for v in flat)
    assert scaler._scale.device == t1.device


def test_grad_scaling_state_dict(no_fallback):
    """test_amp.py:33-52."""
    for lazy in (True, False):
        s0 = torch.amp.GradScaler(SUPA, init_scale=3.0, growth_factor=4.0, backoff_factor=0.5, growth_interval=2)
        s1 = torch.amp.GradScaler(SUPA, init_scale=6.0, growth_factor=7.0, backoff_factor=0.8, growth_interval=1)
        s1._init_growth_tracker = 7
        if lazy:
            s1.scale(torch.full((1,), 4.0, dtype=torch.float32, device=SUPA))
            assert s1._scale.device.type == SUPA
        s1.load_state_dict(s0.state_dict())
        assert s1.get_scale() == 3.0 and s1.get_growth_factor() == 4.0
        assert s1.get_backoff_factor() == 0.5 and s1.get_growth_interval() == 2 and s1._init_growth_tracker == 0


def _scaling_case(run, unskipped, skipped, atol):
    """test_amp.py:54-101 (_create_scaling_case, _run_scaling_case)."""
    for enabled in (True, False):
        torch.manual_seed(3)
        mods = [torch.nn.Sequential(torch.nn.Linear(8, 8, bias=False), torch.nn.Linear(8, 8, bias=False)).to(SUPA)
                for _ in range(2)]
        for c, s in zip(mods[0].parameters(), mods[1].parameters()):
            s.data.copy_(c.data)
        opts = [torch.optim.SGD(m.parameters(), lr=1.0) for m in mods]
        g = torch.Generator().manual_seed(4)
        data = [(torch.randn((8, 8), generator=g).to(SUPA), torch.randn((8, 8), generator=g).to(SUPA))
                for _ in range(4)]
        loss_fn = torch.nn.MSELoss()
        scaler = torch.amp.GradScaler(SUPA, init_scale=128.0, growth_factor=2.0, enabled=enabled, growth_interval=1)
        run(data, mods[0], opts[0], scaler, loss_fn, 2, False)
        run(data, mods[1], opts[1], scaler, loss_fn, 2, True)
        if enabled:
            assert scaler.get_scale() == 128.0 * scaler.get_growth_factor() ** unskipped * \
                scaler.get_backoff_factor() ** skipped
        else:
            assert scaler.get_scale() == 1.0
        for c, s in zip(mods[0].parameters(), mods[1].parameters()):
            _rtol_equal(c.detach().cpu().numpy(), s.detach().cpu().numpy(), atol)


def _rtol_equal(x, y, prec):
    """assertRtolEqual (torch_supa/testing/common_utils.py:232-243), per
    element: within prec absolutely or relatively."""
    d = np.abs(y - x)
    assert bool(np.all((d <= prec) | (d / (np.maximum(np.abs(x), np.abs(y)) + 1e-9) <= prec))), float(d.max())


def _run_clipping(separate_unscale):
    def run(data, model, optimizer, scaler, loss_fn, skip_iter, try_scaling_api):
        max_norm = 0.2
        for i, (x, target) in enumerate(data):
            optimizer.zero_grad()
            loss = loss_fn(model(x), target)
            if try_scaling_api:
                scaler.scale(loss).backward()
                if separate_unscale:
                    if i == skip_iter and scaler.is_enabled():
                        model[1].weight.grad.data.fill_(float("inf"))
                    scaler.unscale_(optimizer)
                    torch.nn.utils.clip_grad_norm_(model.parameters(), max_norm)
                else:
                    torch.nn.utils.clip_grad_norm_(model.parameters(), max_norm * scaler.get_scale())
                    if i == skip_iter and scaler.is_enabled():
                        model[1].weight.grad.data.fill_(float("inf"))
                scaler.step(optimizer)
                scaler.update()
            else:
                loss.backward()
                torch.nn.utils.clip_grad_norm_(model.parameters(), max_norm)
                if (not scaler.is_enabled()) or (i != skip_iter):
                    optimizer.step()
    return run


@pytest.mark.parametrize("separate_unscale", [False, True])
def test_grad_scaling_clipping(separate_unscale, supa):
    """test_amp.py test_grad_scaling_clipping (atol 1e-5) and
    test_grad_scaling_clipping_separate_unscale (atol 1e-7)."""
    torch.supa.set_cpu_fallback_enabled(True)
    torch.supa.reset_fallback_counts()
    _scaling_case(_run_clipping(separate_unscale), unskipped=3, skipped=1, atol=1e-7 if separate_unscale else 1e-5)
    # only the Linear layers' matrix products left the device
    assert all("mm" in k for k in dict(torch.supa.fallback_counts())), torch.supa.fallback_counts()


SGD_SHAPES = [(1, 1000), (512, 1024), (1023, 511), (1025, 513), (1028, 2135)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", SGD_SHAPES)
def test_fused_sgd_on_cross_entropy(shape, dtype, no_fallback):
    """test_fused_sgd_kernel.py: weights uniform in [-1, 1] used as the
    logits of CrossEntropyLoss over random class targets; one step of
    SGD(lr 0.1, fused=True) on the device against SGD(fused=False) on the
    CPU, rtol 1e-3 / atol 1e-4."""
    wc, ws = pair(shape, dtype, lo=-1, hi=1)
    t = torch.empty(shape[0], dtype=torch.long).random_(shape[1], generator=torch.Generator().manual_seed(99))
    ts = t.to(SUPA)
    wc.requires_grad_(True)
    ws.requires_grad_(True)
    crit = torch.nn.CrossEntropyLoss()
    oc = torch.optim.SGD([wc], lr=0.1, momentum=0, weight_decay=0, dampening=0, nesterov=False, fused=False)
    os_ = torch.optim.SGD([ws], lr=0.1, momentum=0, weight_decay=0, dampening=0, nesterov=False, fused=True)
    crit(wc, t).backward()
    oc.step()
    crit(ws, ts).backward()
    os_.step()
    ref_allclose(wc, ws, 1e-3, 1e-4)


POW_PARAMS = [((1, 16), True), ((1, 16), False), ((512, 1024), True), ((512, 1024), False), ((1023, 511), True),
              ((1025, 513), True), ((1028, 2135), True), ((1023, 511), False), ((1025, 513), False),
              ((1028, 2135), False)]


@pytest.mark.parametrize("shape, scalar", POW_PARAMS)
def test_pow_ptwise(shape, scalar, no_fallback):
    """test_pow_kernel.py: float32; the exponent an N(0, 1) tensor or
    torch.tensor(2) (a 0-dim CPU int64 tensor, taken as a scalar)."""
    dtype = torch.float32
    x, x_s = pair(shape, dtype)
    if scalar:
        y = y_s = torch.tensor(2)
    else:
        y, y_s = pair(shape, dtype)
    out, out_s = torch.pow(x, y), torch.pow(x_s, y_s)
    x.pow_(y)
    x_s.pow_(y_s)
    ref_allclose(x, x_s, RTOL[dtype], ATOL[dtype], equal_nan=True)
    ref_allclose(out, out_s, RTOL[dtype], ATOL[dtype], equal_nan=True)
    ref_allclose(x_s.cpu(), out_s, RTOL[dtype], ATOL[dtype], equal_nan=True)


ABS_SHAPES = [(32,), (1024, 512), (1023, 511), (1025, 513), (1028, 2135)]


@pytest.mark.parametrize("zeros", [False, True])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("shape", ABS_SHAPES)
def test_abs_forms(shape, dtype, zeros, no_fallback):
    """test_abs_kernel.py: test_abs and test_abs_out (abs_) over N(0, 1) and
    all-zero (uniform in [0, 0]) inputs."""
    x, x_s = (torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype, device=SUPA)) if zeros else \
        pair(shape, dtype)
    y, y_s = torch.abs(x), torch.abs(x_s)
    ref_allclose(y, y_s, RTOL[dtype], ATOL[dtype], equal_nan=True)
    x.abs_()
    x_s.abs_()
    ref_allclose(x, y, RTOL[dtype], ATOL[dtype], equal_nan=True)
    ref_allclose(x, x_s.cpu(), RTOL[dtype], ATOL[dtype], equal_nan=True)
    ref_allclose(x_s.cpu(), y_s.cpu(), RTOL[dtype], ATOL[dtype], equal_nan=True)
