"""The _foreach_* family on the supa device: every fast-path form (List,
Scalar, ScalarList, Tensor; pointwise ternary; unary; zero_; norm) is one
multi-tensor launch whose results equal the oracle's elementwise arithmetic
bit for bit (f32; bf16 is the f32 result rounded once), and the default
torch.optim.AdamW (the foreach implementation) and clip_grad_norm_ run on it
with the CPU fallback disabled."""
import math

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

# ragged sizes: a partial last vector, a tensor smaller than one vector, and
# one that spans many chunks
SHAPES = [(4096 * 257 + 3,), (1000, 33), (5,), (64, 1024)]


def lists(seed, dtype=torch.float32, positive=False, n=len(SHAPES)):
    g = torch.Generator().manual_seed(seed)
    out = []
    for s in SHAPES[:n]:
        t = torch.randn(s, generator=g) * 2
        if positive:
            t = t.abs() + 0.25
        out.append(t.to(dtype))
    return out


def dev(ts):
    return [t.to("supa") for t in ts]


def f32(t):
    return t.float().numpy()


def want(arr, dtype):
    return torch.from_numpy(np.ascontiguousarray(arr)).to(dtype)


def same(got, ref):
    torch.testing.assert_close(got.cpu(), ref, rtol=0, atol=0, equal_nan=True)


BINARY = [  # (foreach name, oracle op, in-place name)
    ("add", O.ADD), ("sub", O.ADD), ("mul", O.MUL), ("div", O.DIV),
    ("maximum", O.MAXIMUM), ("minimum", O.MINIMUM), ("clamp_min", O.MAXIMUM), ("clamp_max", O.MINIMUM),
]


def oracle_binary(name, op, a, b, alpha=1.0):
    """The per-element oracle of one binary foreach op; sub is add of -y."""
    if not isinstance(b, np.ndarray):
        b = np.float32(b)
    if name == "sub":
        if b.ndim:
            return O.binary(O.ADD, a, b, -alpha)
        return O.binary(O.ADD, a, -b)
    return O.binary(op, a, b, alpha)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name,op", BINARY)
def test_binary_forms(name, op, dtype, no_fallback):
    xs, ys = lists(1, dtype), lists(2, dtype, positive=(name == "div"))
    dxs, dys = dev(xs), dev(ys)
    fn = getattr(torch, f"_foreach_{name}")
    fn_ = getattr(torch, f"_foreach_{name}_")
    # List (add / sub with alpha)
    kw = {"alpha": 0.5} if name in ("add", "sub") else {}
    for o, x, y in zip(fn(dxs, dys, **kw), xs, ys):
        same(o, want(oracle_binary(name, op, f32(x), f32(y), kw.get("alpha", 1.0)), dtype))
    # Scalar and ScalarList
    for o, x in zip(fn(dxs, 0.75), xs):
        same(o, want(oracle_binary(name, op, f32(x), 0.75), dtype))
    sl = [0.5, -1.25, 3.0, 0.1]
    for o, x, s in zip(fn(dxs, sl), xs, sl):
        same(o, want(oracle_binary(name, op, f32(x), s), dtype))
    # in place, then a second op on the result
    work = [t.clone() for t in dxs]
    fn_(work, dys, **kw)
    fn_(work, sl)
    for w, x, y, s in zip(work, xs, ys, sl):
        r = want(oracle_binary(name, op, f32(x), f32(y), kw.get("alpha", 1.0)), dtype)
        same(w, want(oracle_binary(name, op, f32(r), s), dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name,op", [("add", O.ADD), ("mul", O.MUL), ("div", O.DIV)])
def test_binary_tensor_form(name, op, dtype, no_fallback):
    """A 0-dim device tensor as the second operand (clip_grad_norm_'s
    `_foreach_mul_(grads, clip_coef)`), cast to the list dtype first."""
    xs = lists(3, dtype)
    dxs = dev(xs)
    other = torch.tensor(0.3, dtype=torch.float32)
    s = float(other.to(dtype).float())
    fn = getattr(torch, f"_foreach_{name}")
    kw = {"alpha": 2.0} if name == "add" else {}
    for o, x in zip(fn(dxs, other.to("supa"), **kw), xs):
        if name == "add":
            ref = O.binary(O.ADD, f32(x), np.full(x.shape, s, np.float32), 2.0)
        else:
            ref = O.binary(op, f32(x), np.float32(s))
        same(o, want(ref, dtype))
    work = [t.clone() for t in dxs]
    getattr(torch, f"_foreach_{name}_")(work, other.to("supa"), **kw)
    for w, o in zip(work, fn(dxs, other.to("supa"), **kw)):
        same(w, o.cpu())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_pointwise_forms(dtype, no_fallback):
    xs, ys, zs = lists(4, dtype), lists(5, dtype), lists(6, dtype, positive=True)
    ws = [(torch.rand(s, generator=torch.Generator().manual_seed(7)) * 1.4 - 0.2).to(dtype) for s in SHAPES]
    dxs, dys, dzs, dws = dev(xs), dev(ys), dev(zs), dev(ws)
    sl = [0.5, -1.25, 3.0, 0.1]
    for name, op in (("addcmul", O.ADDCMUL), ("addcdiv", O.ADDCDIV)):
        fn = getattr(torch, f"_foreach_{name}")
        for o, x, y, z in zip(fn(dxs, dys, dzs, value=-0.37), xs, ys, zs):
            same(o, want(O.ternary(op, f32(x), f32(y), f32(z), -0.37), dtype))
        for o, x, y, z, s in zip(fn(dxs, dys, dzs, sl), xs, ys, zs, sl):
            same(o, want(O.ternary(op, f32(x), f32(y), f32(z), s), dtype))
        for o, x, y, z, s in zip(fn(dxs, dys, dzs, torch.tensor(sl)), xs, ys, zs, sl):  # Tensor of scalars
            same(o, want(O.ternary(op, f32(x), f32(y), f32(z), s), dtype))
        work = [t.clone() for t in dxs]
        getattr(torch, f"_foreach_{name}_")(work, dys, dzs, sl)
        for w, x, y, z, s in zip(work, xs, ys, zs, sl):
            same(w, want(O.ternary(op, f32(x), f32(y), f32(z), s), dtype))
    for o, x, y, w in zip(torch._foreach_lerp(dxs, dys, dws), xs, ys, ws):
        same(o, want(O.ternary(O.LERP, f32(x), f32(y), f32(w)), dtype))
    for o, x, y in zip(torch._foreach_lerp(dxs, dys, 0.1), xs, ys):
        same(o, want(O.ternary(O.LERP, f32(x), f32(y), np.full(x.shape, 0.1, np.float32)), dtype))
    work = [t.clone() for t in dxs]
    torch._foreach_lerp_(work, dys, sl)
    for w, x, y, s in zip(work, xs, ys, sl):
        same(w, want(O.ternary(O.LERP, f32(x), f32(y), np.full(x.shape, s, np.float32)), dtype))


UNARY = [("sigmoid", O.SIGMOID), ("tanh", O.TANH), ("exp", O.EXP), ("log", O.LOG), ("erf", O.ERF),
         ("neg", O.NEG), ("reciprocal", O.RECIPROCAL), ("abs", O.ABS), ("sqrt", O.SQRT)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_unary_and_zero(dtype, no_fallback):
    xs = lists(8, dtype)
    pos = [t.abs() + 0.01 for t in xs]
    for name, op in UNARY:
        src = pos if name in ("log", "sqrt") else xs
        d = dev(src)
        for o, x in zip(getattr(torch, f"_foreach_{name}")(d), src):
            same(o, want(O.unary(op, f32(x)), dtype))
        getattr(torch, f"_foreach_{name}_")(d)
        for o, x in zip(d, src):
            same(o, want(O.unary(op, f32(x)), dtype))
    d = dev(xs)
    torch._foreach_zero_(d)
    for t in d:
        assert not t.cpu().any()


ROUNDING = ["sign", "floor", "ceil", "round", "trunc", "rsqrt"]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_rounding_unary_and_copy(dtype, no_fallback):
    """sign / floor / ceil / round / trunc / rsqrt and copy_ in one launch each:
    equal to the per-tensor supa op bit for bit, and (all but rsqrt, whose
    per-tensor kernel has its own test) to upstream CPU."""
    xs = lists(11, dtype)
    xs[1][0, :6] = torch.tensor([0.5, -0.5, 2.5, -2.5, -0.0, float("nan")])  # ties to even, -0, NaN
    d = dev(xs)
    for name in ROUNDING:
        src = [t.abs() + 0.01 for t in d] if name == "rsqrt" else d
        got = getattr(torch, f"_foreach_{name}")(src)
        for o, x in zip(got, src):
            same(o, getattr(torch, name)(x).cpu())
        work = [t.clone() for t in src]
        getattr(torch, f"_foreach_{name}_")(work)
        for w, o in zip(work, got):
            same(w, o.cpu())
        if name != "rsqrt":
            for o, x in zip(got, xs):
                same(o, getattr(torch, name)(x))
    dst = [torch.empty_like(t) for t in d]
    torch._foreach_copy_(dst, d)
    for a, x in zip(dst, xs):
        same(a, x)
    # a cast or a strided member takes copy_ per tensor
    mixed = [torch.empty(t.shape, dtype=torch.float64, device="supa") for t in d]
    torch._foreach_copy_(mixed, d)
    for a, x in zip(mixed, xs):
        same(a, x.double())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_pow_forms(dtype, no_fallback):
    """_foreach_pow (List, Scalar, ScalarList, ScalarAndTensor) and its in-place
    forms equal the per-tensor pow bit for bit, over every special exponent the
    per-tensor op routes (0, 1, +-0.5, -1, 2, 3, -2), general ones, and an
    exponent that is not exact in the dtype (per-tensor path)."""
    xs = lists(12, dtype, positive=True)
    xs[0][:4] = torch.tensor([0.0, float("nan"), float("inf"), 1.0])
    ys = [(t.float() * 0.5 - 0.3).to(dtype) for t in lists(13, dtype)]
    d, dy = dev(xs), dev(ys)
    for e in [0.0, 1.0, 0.5, -0.5, -1.0, 2.0, 3.0, -2.0, 1.75, -0.375, 2.5, 1.7, 2]:
        got = torch._foreach_pow(d, e)
        for o, t in zip(got, d):
            same(o, torch.pow(t, e).cpu())
        work = [t.clone() for t in d]
        torch._foreach_pow_(work, e)
        for w, o in zip(work, got):
            same(w, o.cpu())
    if dtype == torch.float32:
        # x*x, (x*x)*x and 1/(x*x) as upstream CPU evaluates them; sqrt the
        # correctly rounded root (this CPU build's float32 sqrt is not IEEE)
        for e in (2.0, 3.0, -2.0):
            for o, x in zip(torch._foreach_pow(d, e), xs):
                same(o, torch.pow(x, e))
        for o, x in zip(torch._foreach_pow(d, 0.5), xs):
            same(o, torch.sqrt(x.double()).float())
    sl = [2.0, -0.5, 1.25, 3]
    for o, t, e in zip(torch._foreach_pow(d, sl), d, sl):
        same(o, torch.pow(t, e).cpu())
    work = [t.clone() for t in d]
    torch._foreach_pow_(work, sl)
    for w, t, e in zip(work, d, sl):
        same(w, torch.pow(t, e).cpu())
    for o, t, e in zip(torch._foreach_pow(d, dy), d, dy):
        same(o, torch.pow(t, e).cpu())
    work = [t.clone() for t in d]
    torch._foreach_pow_(work, dy)
    for w, t, e in zip(work, d, dy):
        same(w, torch.pow(t, e).cpu())
    for base in (2.0, 0.75, 1.0, -1.5):
        for o, e in zip(torch._foreach_pow(base, dy), dy):
            same(o, torch.pow(base, e).cpu())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_norm(dtype, no_fallback):
    xs = lists(9, dtype) + [torch.zeros(0, dtype=dtype), torch.full((3000,), 0.5, dtype=dtype)]
    d = dev(xs)
    rtol = 1e-5 if dtype == torch.float32 else 1e-2
    for p in (1, 2, math.inf):
        norms = torch._foreach_norm(d, p)
        assert len(norms) == len(xs)
        for nm, x in zip(norms, xs):
            assert nm.dim() == 0 and nm.dtype == dtype
            ref = O.vector_norm(x.double().numpy(), p)
            if p == math.inf:  # the largest |x| is exact
                assert nm.item() == ref
            else:
                assert nm.item() == pytest.approx(ref, rel=rtol, abs=0)
        assert norms[-2].item() == 0.0
    # an f32 result for bf16 inputs, as with dtype=
    if dtype == torch.bfloat16:
        for nm, x in zip(torch._foreach_norm(d, 2, dtype=torch.float32), xs):
            assert nm.dtype == torch.float32
            assert nm.item() == pytest.approx(O.vector_norm(x.double().numpy(), 2), rel=1e-5)
    # NaN propagates
    bad = [t.clone() for t in d[:2]]
    bad[1][3] = float("nan")
    out = torch._foreach_norm(bad, 2)
    assert not math.isnan(out[0].item()) and math.isnan(out[1].item())


def test_many_tensors_span_launches(no_fallback):
    """More tensors than one launch's table (40), with empty ones mixed in."""
    g = torch.Generator().manual_seed(10)
    xs = [torch.randn(int(n), generator=g) for n in torch.randint(0, 3000, (97,), generator=g)]
    xs[5] = torch.zeros(0)
    d = dev(xs)
    torch._foreach_mul_(d, 1.5)
    torch._foreach_add_(d, d, alpha=-0.25)
    for t, x in zip(d, xs):
        r = O.binary(O.MUL, x.numpy(), np.float32(1.5))
        same(t, torch.from_numpy(O.binary(O.ADD, r, r, -0.25)))
    norms = torch._foreach_norm(d)
    for nm, t in zip(norms, d):
        assert nm.item() == pytest.approx(O.vector_norm(t.cpu().double().numpy(), 2), rel=1e-5)


def test_slow_path_matches_per_tensor(no_fallback):
    """Non-contiguous members and mixed dtypes take the per-tensor path."""
    x = torch.randn(64, 96)
    y = torch.randn(96, 64)
    dx, dy = x.to("supa"), y.to("supa")
    out = torch._foreach_add([dx.t(), dx], [dy, dy.t()], alpha=2.0)
    same(out[0], torch.add(x.t(), y, alpha=2.0))
    same(out[1], torch.add(x, y.t(), alpha=2.0))
    mixed = torch._foreach_mul([dx, dy.to(torch.bfloat16)], 0.5)
    assert mixed[1].dtype == torch.bfloat16
    same(mixed[0], x * 0.5)


@pytest.mark.parametrize("amsgrad", [False, True])
def test_default_adamw_is_foreach_and_matches_single_tensor(amsgrad, no_fallback):
    """torch.optim.AdamW's default (foreach) implementation on supa: every
    list op is native, and the parameters equal the single-tensor
    implementation's (the same ops one tensor at a time) bit for bit."""
    g = torch.Generator().manual_seed(11)
    shapes = [(1024, 257), (257,), (33, 7)]
    init = [torch.randn(s, generator=g) * 0.02 for s in shapes]
    grads = [[torch.randn(s, generator=g) * 1e-3 for s in shapes] for _ in range(3)]
    results = []
    for foreach in (True, False):
        ps = [p.clone().to("supa").requires_grad_() for p in init]
        opt = torch.optim.AdamW(ps, lr=1e-3, weight_decay=0.01, amsgrad=amsgrad, foreach=foreach)
        for step in grads:
            for p, gr in zip(ps, step):
                p.grad = gr.to("supa")
            opt.step()
        results.append([p.detach().cpu() for p in ps])
    for a, b in zip(*results):
        assert torch.equal(a, b)
    # and close to the CPU implementation (whose addcmul rounds once more)
    ps = [p.clone().requires_grad_() for p in init]
    opt = torch.optim.AdamW(ps, lr=1e-3, weight_decay=0.01, amsgrad=amsgrad, foreach=False)
    for step in grads:
        for p, gr in zip(ps, step):
            p.grad = gr
        opt.step()
    for a, p in zip(results[0], ps):
        torch.testing.assert_close(a, p.detach(), rtol=1e-5, atol=1e-7)


# ------------------------------------------- clip_grad_norm_ and its pieces
def test_cat_and_stack(no_fallback):
    a, b, e = torch.randn(3, 5), torch.randn(4, 5), torch.randn(0)
    d = [t.to("supa") for t in (a, b, e)]
    assert torch.equal(torch.cat(d).cpu(), torch.cat([a, b, e]))  # legacy 1-D empty input skipped
    x, y = torch.randn(6, 2, 7), torch.randn(6, 3, 7).to(torch.bfloat16)
    got = torch.cat([x.to("supa"), y.to("supa")], dim=1)
    assert got.dtype == torch.float32 and torch.equal(got.cpu(), torch.cat([x, y], dim=1))  # type promotion
    s = [torch.randn(()) for _ in range(5)]
    assert torch.equal(torch.stack([t.to("supa") for t in s]).cpu(), torch.stack(s))
    m = [torch.randn(4, 9) for _ in range(3)]
    assert torch.equal(torch.stack([t.to("supa") for t in m], dim=1).cpu(), torch.stack(m, dim=1))
    with pytest.raises(RuntimeError, match="Sizes of tensors must match"):
        torch.cat([d[0], torch.randn(2, 4).to("supa")])


def test_linalg_vector_norm(no_fallback):
    x = torch.randn(1000, 37)
    dx = x.to("supa")
    for p in (1, 2, math.inf):
        got = torch.linalg.vector_norm(dx, p)
        assert got.dim() == 0 and got.dtype == torch.float32
        assert got.item() == pytest.approx(O.vector_norm(x.double().numpy(), p), rel=1e-5)
    assert torch.linalg.vector_norm(dx, 2, keepdim=True).shape == (1, 1)
    h = torch.linalg.vector_norm(dx.bfloat16(), 2, dtype=torch.float32)
    assert h.dtype == torch.float32
    assert h.item() == pytest.approx(O.vector_norm(x.bfloat16().double().numpy(), 2), rel=1e-5)
    assert torch.linalg.vector_norm(torch.zeros(0, device="supa")).item() == 0.0


NORM_ORDS = [0.0, 1.0, 2.0, math.inf, -math.inf, 3.0, 0.5, -1.5]


@pytest.mark.parametrize("p", NORM_ORDS)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64])
def test_linalg_vector_norm_over_dims(p, dtype, no_fallback):
    """Norms over one dim, several dims and every element, each order the
    row-norm kernel knows: each row against the float64 oracle (rtol 1e-5;
    1e-2 for a bf16 result) and the layout against upstream CPU."""
    g = torch.Generator().manual_seed(int(abs(p) * 10) % 97 if math.isfinite(p) else 5)
    x = torch.randn(6, 37, 129, generator=g).to(dtype)
    x[1, 3, 7] = 0.0
    dx = x.to("supa")
    rtol = 1e-2 if dtype == torch.bfloat16 else 1e-5
    for dim, keepdim in [(-1, False), (0, True), ((0, 2), False), (None, False), ((2, 1, 0), True)]:
        got = torch.linalg.vector_norm(dx, p, dim=dim, keepdim=keepdim)
        want = torch.linalg.vector_norm(x.double(), p, dim=dim, keepdim=keepdim)
        assert got.shape == want.shape and got.dtype == dtype
        dims = tuple(range(3)) if dim is None else ((dim,) if isinstance(dim, int) else dim)
        dims = tuple(d % 3 for d in dims)
        keep = [d for d in range(3) if d not in dims]
        rows = x.double().permute(keep + list(dims)).reshape(-1, int(np.prod([x.shape[d] for d in dims])))
        ref = np.array([O.vector_norm(r.numpy(), p) for r in rows]).reshape(
            [x.shape[d] for d in keep] or [])
        np.testing.assert_allclose(got.double().cpu().reshape(ref.shape).numpy(), ref, rtol=rtol)
        torch.testing.assert_close(got.double().cpu(), want, rtol=rtol, atol=0)


@pytest.mark.parametrize("p", [2.0, math.inf, -math.inf, 0.0, 1.5])
def test_linalg_vector_norm_long_rows_two_launches(p, no_fallback):
    """Rows over 65536 elements (few of them) reduce per 16384-element chunk,
    then over the chunk partials; a ragged last chunk and a NaN row too."""
    g = torch.Generator().manual_seed(77)
    x = torch.randn(3, 200003, generator=g)
    x[2, 150001] = float("nan")
    got = torch.linalg.vector_norm(x.to("supa"), p, dim=1).cpu()
    ref = np.array([O.vector_norm(r.numpy(), p) for r in x.double()])
    np.testing.assert_allclose(got.double().numpy(), ref, rtol=1e-5)
    whole = torch.linalg.vector_norm(x[:2].to("supa"), p).item()  # every element, one row of 400006
    assert whole == pytest.approx(O.vector_norm(x[:2].double().numpy(), p), rel=1e-5)


def test_linalg_vector_norm_dtypes_and_edges(supa, no_fallback):
    x = torch.randn(33, 70)
    dx = x.to("supa")
    # a narrow input into f32 reads it directly; into f64 converts it first
    got = torch.linalg.vector_norm(dx.bfloat16(), 3.0, dim=1, dtype=torch.float32)
    want = torch.linalg.vector_norm(x.bfloat16(), 3.0, dim=1, dtype=torch.float32)
    assert got.dtype == torch.float32
    torch.testing.assert_close(got.cpu(), want, rtol=1e-5, atol=0)
    got = torch.linalg.vector_norm(dx, 2.0, dim=0, dtype=torch.float64)
    assert got.dtype == torch.float64
    torch.testing.assert_close(got.cpu(), torch.linalg.vector_norm(x.double(), 2.0, dim=0), rtol=1e-12, atol=0)
    out = torch.empty(5, device="supa")
    torch.linalg.vector_norm(dx, 0.5, dim=0, out=out)
    torch.testing.assert_close(out.cpu(), torch.linalg.vector_norm(x, 0.5, dim=0), rtol=1e-5, atol=0)
    # empty reductions: zeros for orders with an identity, empty outputs for empty kept dims
    e = torch.empty(0, 4, device="supa")
    assert torch.equal(torch.linalg.vector_norm(e, 2.0, dim=0).cpu(), torch.zeros(4))
    assert torch.linalg.vector_norm(e, -1.0, dim=1).shape == (0,)
    s = torch.tensor(-2.5, device="supa")
    assert torch.linalg.vector_norm(s, 3.0).item() == 2.5


def test_linalg_vector_norm_errors_take_the_counted_fallback(supa):
    """Orders without an identity on an empty reduction raise upstream's
    error from the CPU fallback, which counts the call."""
    supa.supa.reset_fallback_counts()
    with pytest.raises(RuntimeError, match="does not have an identity"):
        torch.linalg.vector_norm(torch.empty(0, device="supa"), math.inf)
    assert supa.supa.fallback_counts().get("aten::linalg_vector_norm", 0) == 1


@pytest.mark.parametrize("norm_type", [2.0, math.inf])
def test_clip_grad_norm(norm_type, no_fallback):
    """torch.nn.utils.clip_grad_norm_ (foreach): _foreach_norm, stack,
    linalg_vector_norm, clamp and _foreach_mul_.Tensor, all native."""
    g = torch.Generator().manual_seed(12)
    shapes = [(1024, 257), (257,), (33, 7)]
    grads = [torch.randn(s, generator=g) for s in shapes]
    ps = [torch.zeros(s, device="supa", requires_grad=True) for s in shapes]
    ps_cpu = [torch.zeros(s, requires_grad=True) for s in shapes]
    for p, pc, gr in zip(ps, ps_cpu, grads):
        p.grad = gr.to("supa")
        pc.grad = gr.clone()
    total = torch.nn.utils.clip_grad_norm_(ps, max_norm=1.0, norm_type=norm_type)
    total_cpu = torch.nn.utils.clip_grad_norm_(ps_cpu, max_norm=1.0, norm_type=norm_type)
    whole = np.concatenate([gr.double().numpy().ravel() for gr in grads])
    assert total.item() == pytest.approx(O.vector_norm(whole, norm_type), rel=1e-5)
    assert total.item() == pytest.approx(total_cpu.item(), rel=1e-5)
    for p, pc in zip(ps, ps_cpu):
        torch.testing.assert_close(p.grad.cpu(), pc.grad, rtol=1e-5, atol=1e-9)


def _store16(a, dtype):
    """float32 results stored in dtype, as float32."""
    return a if dtype == torch.float32 else torch.from_numpy(a).to(dtype).float().numpy()


SGD_CFGS = [dict(momentum=0.0), dict(momentum=0.9), dict(momentum=0.9, nesterov=True, weight_decay=0.01),
            dict(momentum=0.9, dampening=0.2, weight_decay=0.01, maximize=True),
            dict(momentum=0.0, weight_decay=0.05, grad_scale=8.0),
            dict(momentum=0.5, grad_scale=2.0, lr_tensor="supa"), dict(momentum=0.9, lr_tensor="cpu")]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("ci", range(len(SGD_CFGS)))
def test_fused_sgd_bit_exact(ci, dtype, no_fallback):
    """_fused_sgd_ over ragged tensors (one misaligned by an element, so it
    takes the scalar path) for three steps, fresh gradients each step:
    params, momentum buffers and (with grad_scale) the unscaled gradients
    equal the oracle's step bit for bit, the 16-bit ones being its float32
    results rounded once per step."""
    cfg = dict(SGD_CFGS[ci])
    gsc = cfg.pop("grad_scale", None)
    lr_kind = cfg.pop("lr_tensor", None)
    mom = cfg["momentum"] != 0
    lr = 0.01
    ps = [t.to("supa") for t in lists(80, dtype)]
    base = torch.zeros(1001, dtype=dtype, device="supa")
    odd = base[1:]
    odd.copy_(torch.randn(1000, generator=torch.Generator().manual_seed(81)).to(dtype))
    ps.append(odd)  # data pointer 2 or 4 bytes past 16-byte alignment
    ref_p = [f32(t.cpu()) for t in ps]
    ref_b = [np.zeros_like(a) for a in ref_p] if mom else None
    bufs = [torch.empty_like(t) for t in ps] if mom else []
    lr_arg = lr if lr_kind is None else torch.tensor(lr, device=lr_kind)
    scale = None if gsc is None else torch.tensor(gsc, device="supa")
    for step in range(3):
        grads = [t.to("supa") for t in lists(82 + step, dtype)] + [
            torch.randn(1000, generator=torch.Generator().manual_seed(90 + step)).to(dtype).to("supa")]
        ref_g = [f32(t.cpu()) for t in grads]
        torch._fused_sgd_(ps, grads, bufs, weight_decay=cfg.get("weight_decay", 0.0), momentum=cfg["momentum"],
                          lr=lr_arg, dampening=cfg.get("dampening", 0.0), nesterov=cfg.get("nesterov", False),
                          maximize=cfg.get("maximize", False), is_first_step=step == 0, grad_scale=scale)
        for i in range(len(ps)):
            p, g = ref_p[i].copy(), ref_g[i].copy()
            b = ref_b[i].copy() if mom else None
            # a tensor lr is a float32 value (read on the device, or item() on the host)
            O.sgd_step(p, g, b, np.float32(lr) if lr_kind else lr, first=step == 0, grad_scale=gsc, **cfg)
            ref_p[i] = _store16(p, dtype)
            assert np.array_equal(f32(ps[i].cpu()), ref_p[i]), (i, step)
            if mom:
                ref_b[i] = _store16(b, dtype)
                assert np.array_equal(f32(bufs[i].cpu()), ref_b[i]), (i, step)
            if gsc is not None:
                assert np.array_equal(f32(grads[i].cpu()), _store16(g, dtype)), (i, step)


def test_fused_sgd_found_inf_and_checks(no_fallback):
    """found_inf = 1 leaves every tensor unchanged, 0 steps; a momentum list
    needs momentum > 0 and its absence momentum == 0."""
    p = torch.randn(4099, generator=torch.Generator().manual_seed(85)).to("supa")
    g = torch.randn(4099, generator=torch.Generator().manual_seed(86)).to("supa")
    b = torch.randn(4099, generator=torch.Generator().manual_seed(87)).to("supa")
    p0, b0 = p.clone(), b.clone()
    one = torch.ones((), device="supa")
    torch._fused_sgd_([p], [g], [b], weight_decay=0.0, momentum=0.9, lr=0.1, dampening=0.0, nesterov=False,
                      maximize=False, is_first_step=False, found_inf=one)
    assert torch.equal(p.cpu(), p0.cpu()) and torch.equal(b.cpu(), b0.cpu())
    torch._fused_sgd_([p], [g], [b], weight_decay=0.0, momentum=0.9, lr=0.1, dampening=0.0, nesterov=False,
                      maximize=False, is_first_step=False, found_inf=one * 0)
    assert not torch.equal(p.cpu(), p0.cpu())
    with pytest.raises(RuntimeError, match="momentum"):
        torch._fused_sgd_([p], [g], [], weight_decay=0.0, momentum=0.9, lr=0.1, dampening=0.0, nesterov=False,
                          maximize=False, is_first_step=False)
    with pytest.raises(RuntimeError, match="momentum"):
        torch._fused_sgd_([p], [g], [b], weight_decay=0.0, momentum=0.0, lr=0.1, dampening=0.0, nesterov=False,
                          maximize=False, is_first_step=False)
