"""Pins the oracle against the upstream aten CPU kernels of torch 2.10.0 --
the kernels the reference's operator library is built from and the producer
of the reference outputs for this path -- plus closed forms and invariants.

Tolerances are the path's: bit-exact for IEEE add/mul/div, transcendental
activations within 2 float32 ulp where the formula is well conditioned (the
CPU's own approximation error is stated where it is not), losses and
reductions rtol 1e-5 float32 / 1e-2 bfloat16."""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import bf16_ulp_dist, f32_ulp_dist

SHAPES = [(16,), (1024, 512), (1023, 511), (1025, 513), (1028, 2135)]


def randn(shape, seed=0, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


# ------------------------------------------------------------- binary ops
@pytest.mark.parametrize("shape", SHAPES)
def test_binary_bit_exact_f32(shape):
    a, b = randn(shape, 0), randn(shape, 1)
    an, bn = a.numpy(), b.numpy()
    for op, ref in [(O.ADD, a + b), (O.MUL, a * b), (O.DIV, a / b),
                    (O.DIV_TRUNC, torch.div(a, b, rounding_mode="trunc")),
                    (O.DIV_FLOOR, torch.div(a, b, rounding_mode="floor"))]:
        got = O.binary(op, an, bn)
        assert np.array_equal(got.view(np.int32), ref.numpy().view(np.int32)), op


def test_c1_config_bit_exact():
    """[4096,4096] N(0,1) from seed 0, add/mul."""
    g = torch.Generator().manual_seed(0)
    a = torch.randn(4096, 4096, generator=g)
    b = torch.randn(4096, 4096, generator=g)
    assert np.array_equal(O.binary(O.ADD, a.numpy(), b.numpy()), torch.add(a, b, alpha=1).numpy())
    assert np.array_equal(O.binary(O.MUL, a.numpy(), b.numpy()), torch.mul(a, b).numpy())


def test_add_alpha_and_broadcast():
    a, b = randn((64, 256), 2), randn((256,), 3)
    for alpha in (1.0, 2.5, -0.75):
        got = O.binary(O.ADD, a.numpy(), b.numpy(), alpha)
        ref = torch.add(a, b, alpha=alpha).numpy()
        assert np.array_equal(got, ref), alpha


def test_bf16_binary_matches_cpu():
    a, b = randn((1024, 512), 4, dtype=torch.bfloat16), randn((1024, 512), 5, dtype=torch.bfloat16)
    af, bf = a.float().numpy(), b.float().numpy()
    for op, ref in [(O.ADD, a + b), (O.MUL, a * b), (O.DIV, a / b)]:
        got = O.f32_to_bf16(O.binary(op, af, bf))
        assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16)), op


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_div_trunc_16bit_rounds_the_quotient(dtype):
    """trunc division of 16-bit operands truncates the quotient rounded to the
    16-bit type (the reference's std::trunc(a / b) on scalar_t).  Upstream
    CPU's vectorised path computes the same thing (Vectorized<T> division,
    then trunc); 4096 elements are whole vectors, so no element takes its
    scalar tail, which truncates the float quotient instead.  The rule is not
    vacuous: on N(0, 1) pairs it differs from truncating the float quotient."""
    a, b = randn((4096,), 8, dtype=dtype), randn((4096,), 9, dtype=dtype)
    af, bf = a.float().numpy(), b.float().numpy()
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    got = O.div_trunc_16(af, bf, name)
    cpu = torch.div(a, b, rounding_mode="trunc").float().numpy()
    assert np.array_equal(got, cpu)
    assert (got != np.trunc(af / bf)).sum() > 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("divisor", [1.5, -0.3, 7.0, 0.0])
def test_div_trunc_16bit_by_a_cpu_scalar(dtype, divisor):
    """trunc division of 16-bit values by a CPU scalar truncates the float
    quotient (no rounding to the 16-bit type first).  Pinned against upstream
    CPU on whole vectors and a scalar tail (4099 elements); 202 / 1.5 is 134
    (the float quotient 134.67 truncated), where rounding the quotient to bf16
    first (135) would give 135."""
    a = randn((4099,), 10, dtype=dtype) * 100
    a[0] = 202.0
    af = a.float().numpy()
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    got = O.div_trunc_16_scalar(af, divisor, name)
    cpu = torch.div(a, divisor, rounding_mode="trunc").float().numpy()
    assert np.array_equal(got, cpu, equal_nan=True)
    if divisor == 1.5:
        assert got[0] == 134.0


_LOSS16 = {"mse": lambda a, b, red, beta: F.mse_loss(a, b, reduction=red),
           "smooth_l1": lambda a, b, red, beta: F.smooth_l1_loss(a, b, reduction=red, beta=beta),
           "huber": lambda a, b, red, beta: F.huber_loss(a, b, reduction=red, delta=beta)}


def _loss16_inputs(dtype, n=1 << 16):
    g = torch.Generator().manual_seed(41)
    x = (torch.rand(n, generator=g) * 2 - 1).to(dtype)
    t = (torch.rand(n, generator=g) * 2 - 1).to(dtype)
    gr = torch.rand(n, generator=g).to(dtype)
    return x, t, gr


def _cpu_loss16_grad(name, x, t, gr, red, beta):
    xx = x.clone().requires_grad_()
    y = _LOSS16[name](xx, t, red, beta)
    y.backward(gr if red == "none" else None)
    return xx.grad.float().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_loss_16bit_rounding_rule(dtype):
    """The 16-bit mse / smooth_l1 / huber rule (loss_16, loss_backward_16:
    the difference rounded to the type, every operation between two 16-bit
    values rounded) against the upstream CPU kernels that compute in
    scalar_t, bit for bit:
    * mse forward and backward (every reduction), in both types;
    * huber backward (every reduction, delta 1 and 0.3), in both types;
    * smooth_l1 forward at beta 1 in float16, huber forward at delta 1 in
      bfloat16 (upstream CPU's other 16-bit forward kernels widen to float32
      first and skip the rounding of the difference);
    and smooth_l1's backward at beta 1 equals huber's at delta 1 (the same
    operations).  The rule is not vacuous: without the rounding of the
    difference the mse forward differs from CPU on most elements."""
    name = "bf16" if dtype == torch.bfloat16 else "f16"
    x, t, gr = _loss16_inputs(dtype)
    xf, tf, gf = x.float().numpy(), t.float().numpy(), gr.float().numpy()
    cpu = F.mse_loss(x, t, reduction="none").float().numpy()
    assert np.array_equal(O.loss_16("mse", xf, tf, name, "none"), cpu)
    assert np.mean(O.round16((xf - tf) * (xf - tf), name) != cpu) > 0.1
    one = "smooth_l1" if dtype == torch.float16 else "huber"
    assert np.array_equal(O.loss_16(one, xf, tf, name, "none", 1.0),
                          _LOSS16[one](x, t, "none", 1.0).float().numpy())
    for red in ("none", "mean", "sum"):
        g = gf if red == "none" else 1.0
        assert np.array_equal(O.loss_backward_16("mse", g, xf, tf, name, red),
                              _cpu_loss16_grad("mse", x, t, gr, red, 1.0))
        for delta in (1.0, 0.3):
            assert np.array_equal(O.loss_backward_16("huber", g, xf, tf, name, red, delta),
                                  _cpu_loss16_grad("huber", x, t, gr, red, delta))
        assert np.array_equal(O.loss_backward_16("smooth_l1", g, xf, tf, name, red, 1.0),
                              O.loss_backward_16("huber", g, xf, tf, name, red, 1.0))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("name", ["mse", "smooth_l1", "huber"])
def test_loss_16bit_reductions(name, dtype):
    """loss_16's sum / mean add the rounded terms and round once: within one
    16-bit ulp of upstream CPU, which sums its 16-bit loss tensor in float32."""
    tname = "bf16" if dtype == torch.bfloat16 else "f16"
    x, t, _ = _loss16_inputs(dtype, 1 << 12)
    rtol = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    for red in ("mean", "sum"):
        got = float(O.loss_16(name, x.float().numpy(), t.float().numpy(), tname, red, 1.0))
        want = float(_LOSS16[name](x, t, red, 1.0))
        assert abs(got - want) <= rtol * abs(want)


def test_mixed_bf16_f32_promotion():
    """c2's add: bf16 x + f32 bias -> f32 (the bf16 value widens exactly)."""
    x = randn((8, 64, 128), 6, dtype=torch.bfloat16)
    bias = randn((128,), 7) * 0.02
    ref = x + bias
    assert ref.dtype == torch.float32
    got = O.binary(O.ADD, O.bf16_to_f32(x.view(torch.int16).numpy().view(np.uint16)), bias.numpy())
    assert np.array_equal(got, ref.numpy())


def test_integer_ops_match_cpu():
    g = torch.Generator().manual_seed(8)
    a = torch.randint(-1000, 1000, (4096,), generator=g)
    b = torch.randint(1, 50, (4096,), generator=g) * torch.where(torch.rand(4096, generator=g) < 0.5, -1, 1)
    for op, ref in [(O.ADD, a + b), (O.MUL, a * b), (O.DIV_TRUNC, torch.div(a, b, rounding_mode="trunc")),
                    (O.DIV_FLOOR, torch.div(a, b, rounding_mode="floor"))]:
        np.testing.assert_array_equal(O.binary_int(op, a.numpy(), b.numpy()), ref.numpy())


# ----------------------------------------------------------- activations
def test_well_conditioned_activations_within_2ulp():
    x = randn((1 << 20,), 10)
    for op, ref in [(O.SILU, F.silu(x)), (O.SIGMOID, torch.sigmoid(x)), (O.TANH, torch.tanh(x))]:
        assert f32_ulp_dist(O.unary(op, x.numpy()), ref.numpy()).max() <= 2, op


@pytest.mark.parametrize("name", ["gelu", "gelu_tanh", "silu", "sigmoid", "tanh"])
def test_activation_backward_vs_cpu(name):
    x = randn((1 << 18,), 12).requires_grad_()
    dy = randn((1 << 18,), 13)
    fn = {"gelu": F.gelu, "gelu_tanh": lambda t: F.gelu(t, approximate="tanh"), "silu": F.silu,
          "sigmoid": torch.sigmoid, "tanh": torch.tanh}[name]
    op = {"gelu": O.GELU, "gelu_tanh": O.GELU_TANH, "silu": O.SILU, "sigmoid": O.SIGMOID, "tanh": O.TANH}[name]
    y = fn(x)
    y.backward(dy)
    inp = y.detach().numpy() if name in ("sigmoid", "tanh") else x.detach().numpy()
    got = O.unary_backward(op, dy.numpy(), inp)
    np.testing.assert_array_less(np.abs(got - x.grad.numpy()), 1e-6 * np.abs(dy.numpy()) + 1e-30)


# ---------------------------------------------------- log_softmax / nll / CE
@pytest.mark.parametrize("shape", [(4, 10), (64, 1000), (3, 128256)])
def test_log_softmax_f32(shape):
    x = randn(shape, 20, 2.0)
    np.testing.assert_allclose(O.log_softmax(x.numpy()), F.log_softmax(x, -1).numpy(), rtol=1e-5, atol=1e-5)


def test_log_softmax_bf16_within_one_ulp():
    x = randn((16, 128256), 21, 2.0, torch.bfloat16)
    ref = F.log_softmax(x, -1).view(torch.int16).numpy().view(np.uint16)
    got = O.f32_to_bf16(O.log_softmax(x.float().numpy()))
    assert bf16_ulp_dist(got, ref).max() <= 1


def test_log_softmax_invariants():
    x = randn((32, 5000), 22, 3.0).numpy()
    y = O.log_softmax(x)
    lse = np.log(np.exp(y.astype(np.float64)).sum(-1))
    np.testing.assert_allclose(lse, 0.0, atol=2e-6)
    # uniform logits: every entry is -log(V)
    V = 128256
    u = O.log_softmax(np.zeros((2, V), np.float32))
    np.testing.assert_allclose(u, -math.log(V), rtol=1e-7)
    # backward rows sum to sum(g) - sum(softmax)*sum(g) = 0
    g = randn((32, 5000), 23).numpy()
    gi = O.log_softmax_backward(g, y)
    np.testing.assert_allclose(gi.astype(np.float64).sum(-1), 0.0, atol=5e-5)


def test_softmax_vs_cpu_and_invariants():
    x = randn((64, 3000), 24, 3.0)
    y = O.softmax(x.numpy())
    np.testing.assert_allclose(y, F.softmax(x, -1).numpy(), rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(y.astype(np.float64).sum(-1), 1.0, atol=1e-5)
    # softmax = exp(log_softmax)
    np.testing.assert_allclose(y, np.exp(O.log_softmax(x.numpy()).astype(np.float64)), rtol=1e-5, atol=1e-9)
    assert np.all(O.softmax(np.zeros((2, 1000), np.float32)) == np.float32(1e-3))
    # a NaN or +inf anywhere makes the row NaN; the other rows are untouched
    bad = x[:3].clone().numpy()
    bad[0, 5], bad[1, 7] = np.nan, np.inf
    yb = O.softmax(bad)
    assert np.isnan(yb[0]).all() and np.isnan(yb[1]).all() and not np.isnan(yb[2]).any()
    # backward against autograd on the CPU, and rows summing to zero
    g = randn((64, 3000), 25)
    xr = x.clone().requires_grad_()
    F.softmax(xr, -1).backward(g)
    gi = O.softmax_backward(g.numpy(), y)
    np.testing.assert_allclose(gi, xr.grad.numpy(), rtol=1e-5, atol=1e-8)  # g - sum cancels
    np.testing.assert_allclose(gi.astype(np.float64).sum(-1), 0.0, atol=1e-7)


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("weighted", [False, True])
def test_nll_and_cross_entropy_vs_cpu(reduction, weighted):
    N, C = 256, 1000
    logits = randn((N, C), 30, 2.0)
    g = torch.Generator().manual_seed(31)
    t = torch.randint(0, C, (N,), generator=g)
    t[torch.randperm(N, generator=g)[:13]] = -100
    w = (torch.rand(C, generator=g) + 0.5) if weighted else None
    lg = logits.clone().requires_grad_()
    loss = F.cross_entropy(lg, t, weight=w, ignore_index=-100, reduction=reduction)
    go = torch.ones_like(loss) if reduction != "none" else randn((N,), 32)
    loss.backward(go)
    lp = O.log_softmax(logits.numpy())
    out, tw = O.nll_loss(lp, t.numpy(), None if w is None else w.numpy(), reduction, -100)
    np.testing.assert_allclose(out, loss.detach().numpy(), rtol=1e-5, atol=1e-6)
    gnll = O.nll_loss_backward(go.numpy(), t.numpy(), N, C, tw, None if w is None else w.numpy(), reduction, -100)
    gin = O.log_softmax_backward(gnll, lp)
    np.testing.assert_allclose(gin, lg.grad.numpy(), rtol=1e-5, atol=1e-7)


def test_nll_closed_forms():
    V = 128256
    lp = O.log_softmax(np.zeros((4, V), np.float32))
    out, tw = O.nll_loss(lp, np.array([0, 5, 7, 9]), None, "mean", -100)
    assert abs(float(out) - math.log(V)) < 1e-5 and float(tw) == 4.0
    # every row ignored: mean is NaN (0/0), sum is 0
    out, tw = O.nll_loss(lp, np.full(4, -100), None, "mean", -100)
    assert np.isnan(out) and float(tw) == 0.0
    out, _ = O.nll_loss(lp, np.full(4, -100), None, "sum", -100)
    assert float(out) == 0.0
    # backward: one nonzero per non-ignored row, equal to -1/count
    gi = O.nll_loss_backward(np.ones(1, np.float32), np.array([1, -100, 3]), 3, 10, 2.0, None, "mean", -100)
    assert (gi != 0).sum() == 2 and gi[0, 1] == -0.5 and gi[2, 3] == -0.5 and not gi[1].any()
    with pytest.raises(IndexError):
        O.nll_loss(lp, np.array([0, V, 1, 2]), None, "mean", -100)


@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
def test_fused_cross_entropy_oracle_vs_cpu_f64(reduction):
    """The fused cross-entropy oracle (float64) against upstream's float64
    cross_entropy and its autograd gradient on the CPU, with ignore_index."""
    N, C = 200, 3001
    x = randn((N, C), 35, 3.0).double()
    g = torch.Generator().manual_seed(36)
    t = torch.randint(0, C, (N,), generator=g)
    t[torch.randperm(N, generator=g)[:11]] = -100
    xg = x.clone().requires_grad_()
    loss = F.cross_entropy(xg, t, ignore_index=-100, reduction=reduction)
    go = torch.ones_like(loss) if reduction != "none" else randn((N,), 37).double()
    loss.backward(go)
    out, lse, cnt = O.cross_entropy(x.numpy(), t.numpy(), reduction, -100)
    assert cnt == N - 11
    np.testing.assert_allclose(out, loss.detach().numpy(), rtol=1e-12, atol=1e-12)
    gx = O.cross_entropy_backward(go.numpy(), x.numpy(), t.numpy(), lse, cnt, reduction, -100)
    np.testing.assert_allclose(gx, xg.grad.numpy(), rtol=1e-10, atol=1e-15)


def test_fused_cross_entropy_closed_forms():
    V = 128256
    out, lse, cnt = O.cross_entropy(np.zeros((3, V)), np.array([0, 7, -100]), "mean", -100)
    assert abs(float(out) - math.log(V)) < 1e-12 and cnt == 2.0 and lse[2] == 0.0
    out, _, cnt = O.cross_entropy(np.zeros((2, 5)), np.array([-100, -100]), "mean", -100)
    assert np.isnan(out) and cnt == 0.0
    # gradient rows sum to zero; the target column carries (p - 1) * g
    x = np.random.default_rng(3).standard_normal((4, 50)) * 2
    t = np.array([3, 0, 49, -100])
    _, lse, cnt = O.cross_entropy(x, t, "sum", -100)
    gx = O.cross_entropy_backward(np.ones(1), x, t, lse, cnt, "sum", -100)
    np.testing.assert_allclose(gx.sum(1), 0.0, atol=1e-14)
    assert not gx[3].any()
    p = np.exp(x[0] - lse[0])
    assert abs(gx[0, 3] - (p[3] - 1.0)) < 1e-15
    with pytest.raises(IndexError):
        O.cross_entropy(x, np.array([0, 1, 50, 2]), "mean", -100)


@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
def test_cross_entropy_prob_oracle_vs_cpu_f64(reduction):
    """The probability-target cross-entropy oracle (float64) against
    upstream's float64 cross_entropy with class-probability targets and its
    autograd gradient on the CPU; targets that do not sum to one included
    (rows scaled by 0.5 and 2)."""
    N, C = 150, 2003
    x = randn((N, C), 45, 3.0).double()
    g = torch.Generator().manual_seed(46)
    p = torch.softmax(torch.randn(N, C, generator=g, dtype=torch.float64) * 2, 1)
    p[:5] *= 0.5
    p[5:9] *= 2.0
    xg = x.clone().requires_grad_()
    loss = F.cross_entropy(xg, p, reduction=reduction)
    go = torch.ones_like(loss) if reduction != "none" else randn((N,), 47).double()
    loss.backward(go)
    out, lse, tsum = O.cross_entropy_prob(x.numpy(), p.numpy(), reduction)
    np.testing.assert_allclose(out, loss.detach().numpy(), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(tsum, p.sum(1).numpy(), rtol=1e-14)
    gx = O.cross_entropy_prob_backward(go.numpy(), x.numpy(), p.numpy(), lse, tsum, reduction)
    np.testing.assert_allclose(gx, xg.grad.numpy(), rtol=1e-10, atol=1e-15)


def test_cross_entropy_prob_closed_forms():
    """Uniform logits with any probability target give log C per unit of
    target mass; a one-hot target equals the class-index form; the target
    softmax(x) gives the entropy; gradient rows of a unit-mass target sum
    to zero."""
    C = 1000
    t = np.random.default_rng(5).dirichlet(np.ones(C), size=3)
    out, _, tsum = O.cross_entropy_prob(np.zeros((3, C)), t, "none")
    np.testing.assert_allclose(out, math.log(C) * tsum, rtol=1e-13)
    x = np.random.default_rng(6).standard_normal((4, 50)) * 2
    idx = np.array([3, 0, 49, 7])
    oh = np.eye(50)[idx]
    a, lse_a, _ = O.cross_entropy_prob(x, oh, "none")
    b, lse_b, _ = O.cross_entropy(x, idx, "none", -100)
    np.testing.assert_allclose(a, b, rtol=1e-13)
    sm = np.exp(x - lse_a[:, None])
    ent, _, _ = O.cross_entropy_prob(x, sm, "none")
    np.testing.assert_allclose(ent, -(sm * np.log(sm)).sum(1), rtol=1e-12)
    gx = O.cross_entropy_prob_backward(np.ones(1), x, sm, lse_a, sm.sum(1), "sum")
    np.testing.assert_allclose(gx, 0.0, atol=1e-14)  # the target is the softmax: zero gradient
    gx = O.cross_entropy_prob_backward(np.ones(1), x, oh, lse_a, oh.sum(1), "mean")
    np.testing.assert_allclose(gx.sum(1), 0.0, atol=1e-15)
    out, _, _ = O.cross_entropy_prob(np.zeros((0, 5)), np.zeros((0, 5)), "mean")
    assert np.isnan(out)


def test_cross_entropy_bf16_decomposition_vs_cpu():
    """c3's semantics at a small row count: bf16 logits, 5% ignore_index,
    mean.  Each decomposed op is compared on the reference's own inputs (the
    backward consumes the forward's rounded output, so a 1-ulp difference in a
    forward element would otherwise be amplified by exp): _log_softmax within
    1 bf16 ulp, nll_loss within rtol 1e-2, nll_loss_backward bit-exact (the
    bf16 total_weight enters rounded), _log_softmax_backward within 1 ulp."""
    N, V = 64, 4096
    logits = randn((N, V), 33, 2.0, torch.bfloat16)
    g = torch.Generator().manual_seed(34)
    t = torch.randint(0, V, (N,), generator=g)
    t[torch.randperm(N, generator=g)[:3]] = -100
    lg = logits.clone().requires_grad_()
    lsm = F.log_softmax(lg, -1)
    lsm.retain_grad()
    loss = F.nll_loss(lsm, t, ignore_index=-100)
    loss.backward()
    bits = lambda x: x.detach().view(torch.int16).numpy().view(np.uint16)
    lp = O.log_softmax(logits.float().numpy())
    assert bf16_ulp_dist(O.f32_to_bf16(lp), bits(lsm)).max() <= 1
    y = lsm.detach().float().numpy()
    out, tw = O.nll_loss(y, t.numpy(), None, "mean", -100)
    assert abs(float(out) - loss.float().item()) <= 1e-2 * abs(loss.float().item())
    _, tw_ref = torch.ops.aten.nll_loss_forward(lsm.detach(), t, None, 1, -100)
    assert O.round_bf16(tw).item() == tw_ref.float().item()
    gnll = O.nll_loss_backward(np.ones(1, np.float32), t.numpy(), N, V, tw_ref.float().item(), None, "mean", -100,
                               bf16=True)
    assert np.array_equal(O.f32_to_bf16(gnll), bits(lsm.grad))
    gin = O.f32_to_bf16(O.log_softmax_backward(lsm.grad.float().numpy(), y))
    assert bf16_ulp_dist(gin, bits(lg.grad)).max() <= 1


# ------------------------------------------------------------------ losses
@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
def test_regression_losses_vs_cpu(reduction):
    x, t = randn((32, 4096), 40), randn((32, 4096), 41)
    for op, fn in [(O.MSE, lambda a, b: F.mse_loss(a, b, reduction=reduction)),
                   (O.SMOOTH_L1, lambda a, b: F.smooth_l1_loss(a, b, reduction=reduction, beta=1.0))]:
        xg = x.clone().requires_grad_()
        ref = fn(xg, t)
        go = torch.ones_like(ref) if reduction != "none" else randn(ref.shape, 42)
        ref.backward(go)
        got = O.loss(op, x.numpy(), t.numpy(), reduction=reduction, beta=1.0)
        np.testing.assert_allclose(got, ref.detach().numpy(), rtol=1e-5, atol=1e-7)
        gg = O.loss_backward(op, go.numpy(), x.numpy(), t.numpy(), reduction=reduction, beta=1.0)
        np.testing.assert_allclose(gg, xg.grad.numpy(), rtol=1e-5, atol=1e-12)


@pytest.mark.parametrize("reduction", ["none", "mean", "sum"])
@pytest.mark.parametrize("with_pw", [False, True])
def test_bce_with_logits_vs_cpu(reduction, with_pw):
    g = torch.Generator().manual_seed(43)
    x = torch.randn(32, 4096, generator=g)
    tb = (torch.rand(32, 4096, generator=g) < 0.3).float()
    pw = torch.rand(4096, generator=g) * 1.5 + 0.5 if with_pw else None
    xg = x.clone().requires_grad_()
    ref = F.binary_cross_entropy_with_logits(xg, tb, pos_weight=pw, reduction=reduction)
    go = torch.ones_like(ref) if reduction != "none" else torch.randn(ref.shape, generator=g)
    ref.backward(go)
    got = O.loss(O.BCE_LOGITS, x.numpy(), tb.numpy(), None if pw is None else pw.numpy(), reduction=reduction)
    np.testing.assert_allclose(got, ref.detach().numpy(), rtol=1e-5, atol=1e-6)
    gg = O.loss_backward(O.BCE_LOGITS, go.numpy(), x.numpy(), tb.numpy(), None if pw is None else pw.numpy(),
                         reduction=reduction)
    np.testing.assert_allclose(gg, xg.grad.numpy(), rtol=1e-5, atol=1e-9)


def test_loss_closed_forms():
    x = np.random.default_rng(44).standard_normal(1000).astype(np.float32)
    assert float(O.loss(O.MSE, x, x, reduction="sum")) == 0.0
    z = np.zeros(8, np.float32)
    t = np.array([0, 1] * 4, np.float32)
    pw = np.full(8, 3.0, np.float32)
    bce = O.loss(O.BCE_LOGITS, z, t, reduction="none")
    np.testing.assert_allclose(bce, math.log(2), rtol=1e-7)
    bce = O.loss(O.BCE_LOGITS, z, t, pw, reduction="none")
    np.testing.assert_allclose(bce, np.where(t == 1, 3 * math.log(2), math.log(2)), rtol=1e-7)
    # smooth_l1 is continuous at |d| = beta
    b = np.float32(1.0)
    eps = np.float32(1e-6)
    lo = O.loss(O.SMOOTH_L1, np.array([b - eps]), np.zeros(1, np.float32), reduction="none")
    hi = O.loss(O.SMOOTH_L1, np.array([b + eps]), np.zeros(1, np.float32), reduction="none")
    assert abs(float(lo[0]) - float(hi[0])) < 1e-5


# ----------------------------------------------------------------- AdamW
def test_adamw_first_step_closed_form():
    rng = np.random.default_rng(50)
    p = (rng.standard_normal(4096) * 0.02).astype(np.float32)
    g = (rng.standard_normal(4096) * 1e-3).astype(np.float32)
    m = np.zeros_like(p)
    v = np.zeros_like(p)
    p0 = p.astype(np.float64).copy()
    lr, b1, b2, wd, eps = 1e-4, 0.9, 0.999, 0.01, 1e-8
    O.adamw_step(p, g, m, v, 1.0, lr, b1, b2, wd, eps)
    gd = g.astype(np.float64)
    np.testing.assert_allclose(m, (1 - b1) * gd, rtol=1e-6)
    np.testing.assert_allclose(v, (1 - b2) * gd * gd, rtol=1e-6)
    expect = p0 * (1 - lr * wd) - lr * gd / (np.abs(gd) + eps)
    np.testing.assert_allclose(p, expect, rtol=1e-6, atol=1e-9)


def test_adamw_ten_steps_vs_cpu_and_restart():
    shapes = [(256, 256), (512, 256), (256,)]
    g = torch.Generator().manual_seed(51)
    params = [torch.randn(s, generator=g) * 0.02 for s in shapes]
    grads = [torch.randn(s, generator=g) * 1e-3 for s in shapes]
    tp = [p.clone().requires_grad_() for p in params]
    opt = torch.optim.AdamW(tp, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, fused=True)
    for _ in range(10):
        for t, gr in zip(tp, grads):
            t.grad = gr.clone()
        opt.step()
    for i in range(len(shapes)):
        p = params[i].numpy().copy().ravel()
        gr = grads[i].numpy().copy().ravel()
        m, v = np.zeros_like(p), np.zeros_like(p)
        for step in range(1, 11):
            O.adamw_step(p, gr, m, v, float(step), 1e-4, 0.9, 0.999, 0.01, 1e-8)
        np.testing.assert_allclose(p, tp[i].detach().numpy().ravel(), rtol=1e-5, atol=1e-9)
        # 10 steps == 5 steps, then a state round trip, then 5 more
        p2 = params[i].numpy().copy().ravel()
        m2, v2 = np.zeros_like(p2), np.zeros_like(p2)
        for step in range(1, 6):
            O.adamw_step(p2, gr, m2, v2, float(step), 1e-4, 0.9, 0.999, 0.01, 1e-8)
        p2, m2, v2 = (np.frombuffer(a.tobytes(), np.float32).copy() for a in (p2, m2, v2))
        for step in range(6, 11):
            O.adamw_step(p2, gr, m2, v2, float(step), 1e-4, 0.9, 0.999, 0.01, 1e-8)
        assert np.array_equal(p2, p) and np.array_equal(m2, m) and np.array_equal(v2, v)


def test_adam_l2_ten_steps_vs_cpu():
    """_fused_adam_ (weight decay added to the gradient) against upstream's
    CPU fused Adam; a plant of the AdamW form instead must fail."""
    shapes = [(256, 256), (300,)]
    g = torch.Generator().manual_seed(52)
    params = [torch.randn(s, generator=g) * 0.5 for s in shapes]
    grads = [torch.randn(s, generator=g) * 1e-3 for s in shapes]
    tp = [p.clone().requires_grad_() for p in params]
    opt = torch.optim.Adam(tp, lr=1e-3, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.1, fused=True)
    for _ in range(10):
        for t, gr in zip(tp, grads):
            t.grad = gr.clone()
        opt.step()
    for i in range(len(shapes)):
        p = params[i].numpy().copy().ravel()
        gr = grads[i].numpy().copy().ravel()
        m, v = np.zeros_like(p), np.zeros_like(p)
        pw, mw, vw = p.copy(), m.copy(), v.copy()
        for step in range(1, 11):
            O.adamw_step(p, gr, m, v, float(step), 1e-3, 0.9, 0.999, 0.1, 1e-8, l2=True)
            O.adamw_step(pw, gr, mw, vw, float(step), 1e-3, 0.9, 0.999, 0.1, 1e-8)
        want = tp[i].detach().numpy().ravel()
        np.testing.assert_allclose(p, want, rtol=1e-5, atol=1e-8)
        np.testing.assert_allclose(m, opt.state[tp[i]]["exp_avg"].numpy().ravel(), rtol=1e-4, atol=1e-9)
        assert not np.allclose(pw, want, rtol=1e-5, atol=1e-8)  # the decoupled form is a different update


# ------------------------------------------------------------------ AMP
def test_amp_unscale_vs_cpu():
    x = randn((5000,), 60, 1000.0)
    x[17] = float("inf")
    x[300] = float("nan")
    for inv, xs in ((0.125, x), (1.0, x), (3.0e-5, x[:100]), (0.5, x[400:])):
        ref = [xs.clone()]
        fi = torch.zeros(1)
        torch._amp_foreach_non_finite_check_and_unscale_(ref, fi, torch.tensor([inv]))
        got, bad = O.amp_unscale(xs.numpy(), inv)
        np.testing.assert_array_equal(got, ref[0].numpy())
        assert bad == bool(fi.item())


def test_amp_update_scale_vs_cpu():
    rng = np.random.default_rng(61)
    for growth, backoff, interval in ((2.0, 0.5, 3), (1.7, 0.3, 1), (65536.0, 0.5, 2)):
        scale = torch.tensor([65536.0])
        tracker = torch.zeros(1, dtype=torch.int32)
        s, t = 65536.0, 0
        for _ in range(40):
            inf = float(rng.random() < 0.2)
            torch._amp_update_scale_(scale, tracker, torch.tensor([inf]), growth, backoff, interval)
            s, t = O.amp_update_scale(s, t, inf, growth, backoff, interval)
            assert s == scale.item() and t == tracker.item()


# ------------------------------------------------- pointwise (ternary) ops
def test_maximum_minimum_vs_cpu():
    a, b = randn((3000,), 62), randn((3000,), 63)
    a[::7] = float("nan")
    b[::11] = float("nan")
    a[5], b[5] = 0.0, -0.0
    for op, fn in ((O.MAXIMUM, torch.maximum), (O.MINIMUM, torch.minimum)):
        got = O.binary(op, a.numpy(), b.numpy())
        ref = fn(a, b).numpy()
        np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
        m = ~np.isnan(ref)
        np.testing.assert_array_equal(got[m], ref[m])


@pytest.mark.parametrize("op", ["addcmul", "addcdiv"])
def test_addcmul_addcdiv_vs_exact_and_cpu(op):
    """self + v * (t1 op t2) as one fma: within half an ulp of the product
    rounding of the exact value, and within the CPU kernel's own rounding of
    upstream's CPU result (which multiplies (v * t1) * t2 first)."""
    x, y, z = randn((20000,), 64, 4.0), randn((20000,), 65, 4.0), randn((20000,), 66, 4.0)
    if op == "addcdiv":
        z = z.sign() * (z.abs() + 0.5)
    v = -0.37
    got = O.ternary(O.ADDCMUL if op == "addcmul" else O.ADDCDIV, x.numpy(), y.numpy(), z.numpy(), v)
    xd, yd, zd = x.double(), y.double(), z.double()
    t = yd * zd if op == "addcmul" else yd / zd
    exact = (xd + np.float32(v) * t).numpy()
    scale = (xd.abs() + (np.float32(v) * t).abs()).numpy()
    eps = 2.0 ** -24
    assert np.all(np.abs(got - exact) <= 2 * eps * scale)
    ref = (torch.addcmul if op == "addcmul" else torch.addcdiv)(x, y, z, value=v).numpy()
    assert np.all(np.abs(got - ref) <= 4 * eps * scale)


def test_lerp_vs_exact_and_cpu():
    x, e = randn((20000,), 67, 3.0), randn((20000,), 68, 3.0)
    w = torch.rand(20000, generator=torch.Generator().manual_seed(69)) * 1.4 - 0.2
    got = O.ternary(O.LERP, x.numpy(), e.numpy(), w.numpy())
    exact = (x.double() + w.double() * (e.double() - x.double())).numpy()
    scale = (x.double().abs() + e.double().abs()).numpy()
    eps = 2.0 ** -24
    assert np.all(np.abs(got - exact) <= 4 * eps * scale)
    np.testing.assert_allclose(got, torch.lerp(x, e, w).numpy(), rtol=0, atol=8 * eps * scale.max())
    # the weight-1 and weight-0 endpoints are exact
    assert np.array_equal(O.ternary(O.LERP, x.numpy(), e.numpy(), np.ones(20000, np.float32)), e.numpy())
    assert np.array_equal(O.ternary(O.LERP, x.numpy(), e.numpy(), np.zeros(20000, np.float32)), x.numpy())


def test_vector_norm_vs_cpu_and_closed_forms():
    x = randn((10007,), 81, 3.0).double()
    for p in (1, 2, float("inf")):
        assert O.vector_norm(x.numpy(), p) == pytest.approx(torch.linalg.vector_norm(x, p).item(), rel=1e-13)
    n = 4096
    assert O.vector_norm(np.ones(n), 2) == 64.0
    assert O.vector_norm(np.full(n, -0.5), 1) == n / 2
    assert O.vector_norm(np.array([3.0, -4.0]), 2) == 5.0
    assert O.vector_norm(np.array([1.0, -7.5, 2.0]), float("inf")) == 7.5
    assert O.vector_norm(np.zeros(0), 2) == 0.0
    assert math.isnan(O.vector_norm(np.array([1.0, float("nan")]), float("inf")))
    assert math.isnan(O.vector_norm(np.array([1.0, float("nan")]), 2))


@pytest.mark.parametrize("p", [0.0, 0.5, 3.0, -1.0, -2.5, float("-inf")])
def test_vector_norm_other_orders(p):
    """Orders beyond 1 / 2 / inf: against upstream CPU, and closed forms that
    a wrong exponent, a missing root or a sum-for-min swap would break."""
    x = randn((4099,), 83, 2.0).double()
    assert O.vector_norm(x.numpy(), p) == pytest.approx(torch.linalg.vector_norm(x, p).item(), rel=1e-12)
    n = 64
    if p == 0:
        assert O.vector_norm(np.array([0.0, -0.0, 2.0, float("nan"), -1e-300]), 0) == 3.0
    elif math.isinf(p):
        assert O.vector_norm(np.array([3.0, -0.25, 7.0]), p) == 0.25
    else:
        assert O.vector_norm(np.ones(n), p) == pytest.approx(n ** (1.0 / p), rel=1e-14)  # n^(1/p)
        assert O.vector_norm(np.array([2.0]), p) == pytest.approx(2.0, rel=1e-15)  # |x| for one element
    if p < 0:
        assert O.vector_norm(np.array([1.0, 0.0]), p) == 0.0  # a zero makes the sum inf, the root 0


def test_moments_vs_cpu_and_closed_forms():
    x = randn((5003,), 85, 3.0).double() + 7.0
    for c in (0.0, 1.0, 2.5):
        v, m = O.moments(x.numpy(), c)
        assert v == pytest.approx(torch.var(x, correction=c).item(), rel=1e-13)
        assert m == pytest.approx(x.mean().item(), rel=1e-14)
    n = 1000
    r = np.arange(n, dtype=np.float64)  # var of 0..n-1: n(n+1)/12 with Bessel's correction, (n^2-1)/12 without
    assert O.moments(r, 1)[0] == pytest.approx(n * (n + 1) / 12, rel=1e-14)
    assert O.moments(r, 0)[0] == pytest.approx((n * n - 1) / 12, rel=1e-14)
    assert O.moments(r, 0)[1] == (n - 1) / 2
    assert O.moments(np.full(17, 3.25), 1) == (0.0, 3.25)  # a constant: no spread, however large the mean
    assert O.moments(np.array([1.0, 3.0]), 2) == (float("inf"), 2.0)  # n <= correction: divides by zero
    assert math.isnan(O.moments(np.array([4.0]), 1)[0])  # 0 / 0
    assert all(math.isnan(v) for v in O.moments(np.zeros(0)))


@pytest.mark.parametrize("reduction", ["mean", "sum", "none"])
@pytest.mark.parametrize("weighted", [False, True])
def test_nll_loss2d_vs_cpu(reduction, weighted):
    g = torch.Generator().manual_seed(96)
    N, C, H, W = 3, 7, 5, 6
    lp = F.log_softmax(torch.randn(N, C, H, W, generator=g) * 2, 1)
    t = torch.randint(0, C, (N, H, W), generator=g)
    t[0, 1, 2] = t[2, 4, 0] = -100
    w = (torch.rand(C, generator=g) + 0.5) if weighted else None
    lpr = lp.clone().requires_grad_()
    ref = F.nll_loss(lpr, t, weight=w, ignore_index=-100, reduction=reduction)
    out, tw = O.nll_loss2d(lp.numpy(), t.numpy(), None if w is None else w.numpy(), reduction, -100)
    np.testing.assert_allclose(out, ref.detach().numpy(), rtol=1e-6, atol=1e-7)
    go = torch.randn(ref.shape, generator=g) if reduction == "none" else torch.tensor(1.0)
    ref.backward(go)
    gi = O.nll_loss2d_backward(go.numpy(), t.numpy(), (N, C, H, W), float(tw),
                               None if w is None else w.numpy(), reduction, -100)
    np.testing.assert_allclose(gi, lpr.grad.numpy(), rtol=1e-6, atol=1e-8)
    # total weight (mean/sum): the weight sum over the positions that count
    wt = np.ones(C, np.float32) if w is None else w.numpy()
    tf = t.numpy().ravel()
    if reduction != "none":
        assert float(tw) == pytest.approx(float(wt[tf[tf != -100]].sum()), rel=1e-6)


# --------------------------------------------- parameterised activations
ACTS = [  # (name, oracle act, params, torch forward on a tensor)
    ("leaky_relu", O.ACT_LEAKY_RELU, (0.01, 0.0, 0.0), lambda t: F.leaky_relu(t, 0.01)),
    ("elu", O.ACT_ELU, (1.0, 1.0, 1.0), F.elu),
    ("selu", O.ACT_ELU, (1.6732632423543772, 1.0507009873554805, 1.0), torch.selu),
    ("celu", O.ACT_ELU, (0.7, 1.0, 1.0 / 0.7), lambda t: F.celu(t, 0.7)),
    ("softplus", O.ACT_SOFTPLUS, (1.0, 20.0, 0.0), F.softplus),
    ("softplus_b2", O.ACT_SOFTPLUS, (2.0, 5.0, 0.0), lambda t: F.softplus(t, 2.0, 5.0)),
    ("hardswish", O.ACT_HARDSWISH, (0.0, 0.0, 0.0), F.hardswish),
    ("hardsigmoid", O.ACT_HARDSIGMOID, (0.0, 0.0, 0.0), F.hardsigmoid),
    ("mish", O.ACT_MISH, (0.0, 0.0, 0.0), F.mish),
    ("logsigmoid", O.ACT_LOG_SIGMOID, (0.0, 0.0, 0.0), F.logsigmoid),
    ("threshold", O.ACT_THRESHOLD, (0.5, -2.0, 0.0), lambda t: F.threshold(t, 0.5, -2.0)),
]


@pytest.mark.parametrize("name,act,ps,fn", ACTS, ids=[a[0] for a in ACTS])
def test_activation_forward_vs_cpu(name, act, ps, fn):
    """Within 2 ulp of double precision wherever upstream's CPU float32 is,
    and never more than 1 ulp worse than it (mish composes three
    primitives: 3.5 ulp against the CPU's 2.8)."""
    from helpers import sample_f32, ulp_vs_exact
    x = np.concatenate([sample_f32(1 << 20, seed=40, lo=-30.0, hi=30.0),
                        np.float32([0.0, -0.0, -3.0, 3.0, 20.0, 20.000002, -1e-30, 0.5, 0.49999997])])
    got = O.activation(act, x, *ps)
    exact = fn(torch.from_numpy(x.astype(np.float64))).numpy()
    cpu = fn(torch.from_numpy(x)).numpy()
    e_or, e_cpu = ulp_vs_exact(got, exact), ulp_vs_exact(cpu, exact)
    assert e_or.max() <= max(2.0, e_cpu.max() + 1.0), (name, float(e_or.max()), float(e_cpu.max()))


BWD = [  # (name, oracle act, params, flag, torch forward whose autograd backward is the reference)
    ("leaky_relu", O.ACT_LEAKY_RELU, (0.01, 0.0, 0.0), 0, lambda t: F.leaky_relu(t, 0.01)),
    ("hardtanh", O.ACT_HARDTANH, (-1.5, 2.0, 0.0), 0, lambda t: F.hardtanh(t, -1.5, 2.0)),
    ("elu", O.ACT_ELU, (1.0, 1.0, 1.0), 0, F.elu),
    ("selu", O.ACT_ELU, (1.6732632423543772, 1.0507009873554805, 1.0), 0, torch.selu),
    ("softplus", O.ACT_SOFTPLUS, (1.0, 20.0, 0.0), 0, F.softplus),
    ("hardswish", O.ACT_HARDSWISH, (0.0, 0.0, 0.0), 0, F.hardswish),
    ("hardsigmoid", O.ACT_HARDSIGMOID, (0.0, 0.0, 0.0), 0, F.hardsigmoid),
    ("mish", O.ACT_MISH, (0.0, 0.0, 0.0), 0, F.mish),
    ("logsigmoid", O.ACT_LOG_SIGMOID, (0.0, 0.0, 0.0), 0, F.logsigmoid),
    ("relu", O.ACT_THRESHOLD, (0.0, 0.0, 0.0), 0, F.relu),
]


@pytest.mark.parametrize("name,act,ps,flag,fn", BWD, ids=[b[0] for b in BWD])
def test_activation_backward_vs_cpu(name, act, ps, flag, fn):
    """Against autograd in double: within a few ulp of the gradient's scale
    |g| (1 + |x|) -- mish's and hardswish's gradients cross zero, so a
    relative bound would be meaningless there, as it is for the CPU's own."""
    from helpers import sample_f32
    x = sample_f32(1 << 19, seed=41, lo=-12.0, hi=12.0)
    g = sample_f32(1 << 19, seed=42, lo=-2.0, hi=2.0)
    xd = torch.from_numpy(x.astype(np.float64)).requires_grad_()
    fn(xd).backward(torch.from_numpy(g.astype(np.float64)))
    exact = xd.grad.numpy()
    # relu's backward reads the forward output (threshold_backward(grad, result, 0))
    inp = np.maximum(x, 0).astype(np.float32) if name == "relu" else x
    got = O.activation_backward(act, g, inp, *ps, flag).astype(np.float64)
    scale = np.abs(g).astype(np.float64) * (1.0 + np.abs(x))
    # 6 units: selu's float-rounded alpha * scale alone costs 4.4 (as on the CPU)
    assert np.all(np.abs(got - exact) <= 6 * 2.0 ** -24 * scale + 1e-30), name


def test_elu_backward_from_result():
    """elu_backward with is_result (the in-place form): x is the output."""
    x = randn((5000,), 43, 3.0)
    g = randn((5000,), 44)
    for alpha in (1.0, 0.5):
        y = F.elu(x.double(), alpha)
        xr = x.double().clone().requires_grad_()
        F.elu(xr, alpha).backward(g.double())
        got = O.activation_backward(O.ACT_ELU, g.numpy(), y.float().numpy(), alpha, 1.0, 1.0, 1)
        np.testing.assert_allclose(got, xr.grad.numpy(), rtol=2e-6, atol=1e-7)


def _dname(dtype):
    return {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_shrink_and_prelu_bit_exact(dtype):
    """hardshrink / softshrink (lambda 0.5, and 0.3, which no 16-bit type
    holds exactly) with their shared backward, and prelu with its backward:
    the oracle equals upstream CPU bit for bit, on inputs that include
    +-lambda, 0 and NaN.  At a NaN input the backward passes the gradient
    (upstream's scalar form, -lambda <= x <= lambda ? 0 : g, which the
    device kernel uses); upstream CPU's vectorised form gives 0 there, so the
    NaN gradient is pinned on a tensor short enough for CPU's scalar loop.
    Lambda is a value of the storage type (upstream's device kernels take
    value.to<scalar_t>()); upstream CPU's 16-bit softshrink keeps a float32
    lambda, so it is handed the rounded lambda for the comparison."""
    name = _dname(dtype)
    x = randn((4096,), 51, 1.0, dtype)
    g = randn((4096,), 52, 1.0, dtype)
    for lam in (0.5, 0.3):
        lam_t = torch.tensor(lam).to(dtype).item()
        x[:6] = torch.tensor([lam_t, -lam_t, 0.0, float("nan"), 2 * lam_t, -2 * lam_t]).to(dtype)
        xf, gf = x.float().numpy(), g.float().numpy()
        for kind, fn in (("hardshrink", F.hardshrink), ("softshrink", F.softshrink)):
            want = fn(x, lam_t).float().numpy()
            assert np.array_equal(O.shrink(kind, xf, lam, name), want, equal_nan=True), (kind, lam)
            xx = x.clone().requires_grad_()
            fn(xx, lam).backward(g)
            keep = ~np.isnan(xf)
            assert np.array_equal(O.shrink_backward(gf, xf, lam, name)[keep],
                                  xx.grad.float().numpy()[keep]), (kind, lam)
            xs = x[:6].clone().requires_grad_()
            fn(xs, lam).backward(g[:6])
            assert np.array_equal(O.shrink_backward(gf[:6], xf[:6], lam, name), xs.grad.float().numpy())
    xc = randn((8, 6, 5, 7), 53, 1.0, dtype)
    w = randn((6,), 54, 0.5, dtype)
    gc = randn((8, 6, 5, 7), 55, 1.0, dtype)
    xf, wf, gf = xc.float().numpy(), w.float().numpy().reshape(1, 6, 1, 1), gc.float().numpy()
    assert np.array_equal(O.prelu(xf, wf, name), F.prelu(xc, w).float().numpy())
    gi, gw = torch.ops.aten._prelu_kernel_backward(gc, xc, w.reshape(1, 6, 1, 1))
    ogi, ogw = O.prelu_backward(xf, wf, gf, name)
    assert np.array_equal(ogi, gi.float().numpy()) and np.array_equal(ogw, gw.float().numpy())


def test_glu_against_cpu_and_closed_forms():
    """glu and its backward: within 4 float32 ulps of upstream CPU (whose
    vectorised exp differs from the oracle's in the last bit; the sigmoid's
    division and the products add a rounding each), and exactly
    the closed forms at b = 0 (sigmoid 1/2: a / 2; gradients g / 2 and
    g a / 4) and at b = +-100 (sigmoid 1, and 0 once exp(100) overflows)."""
    x = randn((64, 258), 56)
    g = randn((64, 129), 57)
    a, b = x[:, :129].numpy(), x[:, 129:].numpy()
    assert f32_ulp_dist(O.glu(a, b), F.glu(x, -1).numpy()).max() <= 4
    xx = x.clone().requires_grad_()
    F.glu(xx, -1).backward(g)
    ga, gb = O.glu_backward(a, b, g.numpy())
    assert f32_ulp_dist(ga, xx.grad[:, :129].numpy()).max() <= 4
    # (1 - s) s cancels as s -> 1: an error of an ulp of s moves the second
    # half's gradient by up to |g a| 2^-24 whatever its own size
    gn = g.numpy()
    cpu_gb = xx.grad[:, 129:].numpy()
    assert np.all(np.abs(gb - cpu_gb) <= 4 * 2.0 ** -24 * np.abs(gn * a) + 4 * np.spacing(np.abs(cpu_gb)))
    zero = np.zeros_like(b)
    assert np.array_equal(O.glu(a, zero), a * np.float32(0.5))
    ga, gb = O.glu_backward(a, zero, gn)
    assert np.array_equal(ga, gn * np.float32(0.5)) and np.array_equal(gb, (gn * a) * np.float32(0.25))
    assert np.array_equal(O.glu(a, zero + 100), a)
    # exp(100) overflows float32: sigmoid 1 / (1 + inf) = 0, the product a signed zero
    assert np.array_equal(O.glu(a, zero - 100), a * np.float32(0))


def test_sgd_step_against_cpu_and_closed_forms():
    """The _fused_sgd_ step (double hyper-parameters, one rounding per
    expression) against upstream CPU's _fused_sgd_, which computes in float32
    (lr and momentum rounded to float32 too): within a float32 rounding of the
    operands' size, 2^-23 (|new| + |old value| + 1), over momentum / nesterov /
    dampening / weight decay / maximize / grad_scale (an ulp count would
    blow up where p - lr g cancels); and exactly the closed forms at lr =
    momentum = 0.5
    (products by 1/2 and the sums of two float32 values below are exact in
    double, so each stored value is that sum rounded once)."""
    rng = np.random.default_rng(70)
    p0 = rng.standard_normal(4096).astype(np.float32)
    g0 = rng.standard_normal(4096).astype(np.float32)
    cfgs = [dict(momentum=0.0), dict(momentum=0.9), dict(momentum=0.9, nesterov=True),
            dict(momentum=0.9, dampening=0.1, weight_decay=0.01), dict(momentum=0.0, weight_decay=0.05, maximize=True),
            dict(momentum=0.9, nesterov=True, weight_decay=0.01, maximize=True, grad_scale=4.0)]
    for cfg in cfgs:
        cfg = dict(cfg)
        gsc = cfg.pop("grad_scale", None)
        mom = cfg["momentum"] != 0
        p, g = p0.copy(), g0.copy()
        b = np.zeros_like(p) if mom else None
        tp, tg = torch.from_numpy(p0.copy()), torch.from_numpy(g0.copy())
        tb = [torch.zeros(4096)] if mom else []
        for step in range(3):
            first = step == 0
            p_prev, b_prev = p.copy(), (b.copy() if mom else None)
            O.sgd_step(p, g, b, 0.01, first=first, grad_scale=gsc, **cfg)
            torch._fused_sgd_([tp], [tg], tb, weight_decay=cfg.get("weight_decay", 0.0), momentum=cfg["momentum"],
                              lr=0.01, dampening=cfg.get("dampening", 0.0), nesterov=cfg.get("nesterov", False),
                              maximize=cfg.get("maximize", False), is_first_step=first,
                              grad_scale=None if gsc is None else torch.tensor(gsc))
            assert np.all(np.abs(p - tp.numpy()) <= 2.0 ** -23 * (np.abs(tp.numpy()) + np.abs(p_prev) + 1)), (cfg, step)
            assert np.array_equal(g, tg.numpy())
            if mom:
                assert np.all(np.abs(b - tb[0].numpy()) <= 2.0 ** -23 * (np.abs(tb[0].numpy()) + np.abs(b_prev) + 1)), \
                    (cfg, step)
            p, b = tp.numpy().copy(), (tb[0].numpy().copy() if mom else None)  # realign on CPU's state
    p, g = p0.copy(), g0.copy()
    O.sgd_step(p, g, None, 0.5)
    assert np.array_equal(p, (p0.astype(np.float64) - 0.5 * g0.astype(np.float64)).astype(np.float32))
    p, g, b = p0.copy(), g0.copy(), np.zeros_like(p0)
    O.sgd_step(p, g, b, 0.5, momentum=0.5, first=True)
    assert np.array_equal(b, g0)
    p1 = p.copy()
    O.sgd_step(p, g, b, 0.5, momentum=0.5)
    b2 = 0.5 * g0.astype(np.float64) + g0.astype(np.float64)
    assert np.array_equal(b, b2.astype(np.float32))
    # g takes the buffer rounded to float32 (g is float32), then p -= lr g
    assert np.array_equal(p, (p1.astype(np.float64) - 0.5 * b2.astype(np.float32).astype(np.float64)).astype(np.float32))
    p, g, b = p0.copy(), g0.copy(), g0.copy()
    O.sgd_step(p, g, b, 0.5, momentum=0.5, nesterov=True)
    bn = 0.5 * g0.astype(np.float64) + g0.astype(np.float64)
    gn = (g0.astype(np.float64) + 0.5 * bn).astype(np.float32)
    assert np.array_equal(p, (p0.astype(np.float64) - 0.5 * gn.astype(np.float64)).astype(np.float32))


def test_xlog1py_against_cpu():
    """xlog1py: 0 where x == 0 (even for y = -1, where log1p is -inf), NaN
    where y is NaN (even for x == 0), x log1p(y) otherwise within 4 float32
    ulps of upstream CPU (both log1p's within 2 ulps of exact)."""
    x = randn((4096,), 71)
    y = randn((4096,), 72).abs() * 3 - 0.9
    x[:4] = torch.tensor([0.0, 0.0, 2.0, 1.5])
    y[:4] = torch.tensor([-1.0, float("nan"), float("nan"), -1.0])
    got = O.xlog1py(x.numpy(), y.numpy())
    want = torch.special.xlog1py(x, y).numpy()
    assert got[0] == 0.0 and np.isnan(got[1]) and np.isnan(got[2]) and got[3] == -np.inf
    m = np.isfinite(want)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert f32_ulp_dist(got[m], want[m]).max() <= 4
