"""Native random ops on the supa device: uniform_, bernoulli_(p) and dropout
(native_dropout and its backward) against the oracle's Philox stream, bit
for bit, for the (seed, offset) the device generator hands the call; the
generator's seeding, state round trip and offset advance; the moments at
full size; and no CPU fallback on the path."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O
from helpers import f32_ulp_dist

pytestmark = pytest.mark.gpu


def state(dev=0):
    st = torch.supa.get_rng_state(dev).numpy().astype(np.uint64)
    seed = int(sum(int(st[i]) << (8 * i) for i in range(8)))
    off = int(sum(int(st[8 + i]) << (8 * i) for i in range(8)))
    return seed, off


def as_dtype(arr, dtype):
    return torch.from_numpy(arr).to(dtype)


DT = {torch.float32: "f32", torch.bfloat16: "bf16", torch.float16: "f16"}


def test_torch_manual_seed_reaches_the_device(supa):
    torch.manual_seed(1234)
    assert torch.supa.initial_seed() == 1234
    assert state() == (1234, 0)
    torch.supa.manual_seed(99)
    assert state() == (99, 0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("n", [1, 3, 4, 1000, 4093, 262147])
def test_uniform_bitexact(n, dtype, no_fallback):
    torch.supa.manual_seed(20 + n)
    t = torch.empty(n, dtype=dtype, device="supa")
    seed, off = state()
    t.uniform_(-1.5, 2.5)
    assert state() == (seed, off + 1)
    want = O.uniform(seed, off, n, -1.5, 2.5, DT[dtype])
    assert torch.equal(t.cpu(), as_dtype(want, dtype))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lo, hi", [(0.0, 1.0), (1.0, 2.0), (-3.0, 100.0)])
def test_uniform_stays_below_to(dtype, lo, hi, no_fallback):
    """[from, to) for every dtype: a value that rounds to `to` in a 16-bit
    type comes back as `from` (upstream's bound reversal), bit-exact with the
    oracle on 4M draws."""
    torch.supa.manual_seed(7)
    t = torch.empty(1 << 22, dtype=dtype, device="supa")
    seed, off = state()
    t.uniform_(lo, hi)
    c = t.cpu().float()
    assert float(c.min()) >= lo and float(c.max()) < hi
    assert torch.equal(t.cpu(), as_dtype(O.uniform(seed, off, t.numel(), lo, hi, DT[dtype]), dtype))


def test_uniform_noncontiguous_and_misaligned(no_fallback):
    torch.supa.manual_seed(5)
    base = torch.zeros(64, 130, device="supa")
    view = base[:, 1::2]
    seed, off = state()
    view.uniform_()
    want = O.uniform(seed, off, view.numel()).reshape(64, 65)
    assert torch.equal(view.cpu(), torch.from_numpy(want))
    assert torch.equal(base[:, 0::2].cpu(), torch.zeros(64, 65))
    flat = torch.zeros(1027, device="supa")
    seed, off = state()
    flat[1:].uniform_()  # storage offset 1: the unaligned tail path
    assert torch.equal(flat[1:].cpu(), torch.from_numpy(O.uniform(seed, off, 1026)))
    assert flat[0].item() == 0.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("p", [0.0, 0.3, 0.5, 1.0])
def test_bernoulli_bitexact(p, dtype, no_fallback):
    torch.supa.manual_seed(31)
    t = torch.empty(50001, dtype=dtype, device="supa")
    seed, off = state()
    t.bernoulli_(p)
    u = O.uniform(seed, off, t.numel())
    want = (u < np.float32(p)).astype(np.float32)
    assert torch.equal(t.cpu(), as_dtype(want, dtype))


def test_explicit_generator(no_fallback):
    g = torch.Generator(device="supa")
    g.manual_seed(77)
    t = torch.empty(999, device="supa").uniform_(generator=g)
    assert torch.equal(t.cpu(), torch.from_numpy(O.uniform(77, 0, 999)))
    t2 = torch.empty(999, device="supa").uniform_(generator=g)
    assert torch.equal(t2.cpu(), torch.from_numpy(O.uniform(77, 1, 999)))


def test_state_roundtrip_replays(no_fallback):
    torch.supa.manual_seed(8)
    torch.empty(10, device="supa").uniform_()
    st = torch.supa.get_rng_state()
    a = torch.empty(4097, device="supa").uniform_()
    b = torch.empty(4097, device="supa").uniform_()
    assert not torch.equal(a.cpu(), b.cpu())
    torch.supa.set_rng_state(st)
    assert torch.equal(torch.empty(4097, device="supa").uniform_().cpu(), a.cpu())


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("p", [0.1, 0.5, 0.0])
@pytest.mark.parametrize("shape", [(513, 1031), (7,), (4, 3, 5)])
def test_dropout_forward_backward_bitexact(shape, p, dtype, no_fallback):
    torch.supa.manual_seed(40)
    gen = torch.Generator().manual_seed(41)
    x = torch.randn(shape, generator=gen).to(dtype)
    g = torch.randn(shape, generator=gen).to(dtype)
    dx = x.to("supa").requires_grad_()
    seed, off = state()
    y = F.dropout(dx, p, training=True)
    y.backward(g.to("supa"))
    keep = 1.0 - p
    out, mask = O.dropout(seed, off, x.float().numpy(), keep)
    assert torch.equal(y.detach().cpu(), as_dtype(out.reshape(shape), dtype))
    scale = np.float32(1.0 / keep)  # autograd passes 1 / (1 - p) in double
    gw = (g.float().numpy().reshape(-1) * mask.astype(np.float32)) * scale
    assert torch.equal(dx.grad.cpu(), as_dtype(gw.reshape(shape), dtype))


def test_native_dropout_mask_and_edges(no_fallback):
    torch.supa.manual_seed(3)
    x = torch.randn(3001).to("supa")
    seed, off = state()
    out, mask = torch.ops.aten.native_dropout(x, 0.25, True)
    assert mask.dtype == torch.bool
    _, want_mask = O.dropout(seed, off, x.cpu().numpy(), 0.75)
    assert torch.equal(mask.cpu(), torch.from_numpy(want_mask))
    g = torch.randn(3001).to("supa")
    gi = torch.ops.aten.native_dropout_backward(g, mask, 1.0 / 0.75)
    want = (g.cpu().numpy() * want_mask.astype(np.float32)) * np.float32(1.0 / 0.75)
    assert torch.equal(gi.cpu(), torch.from_numpy(want))
    o1, m1 = torch.ops.aten.native_dropout(x, 1.0, True)
    assert torch.equal(o1.cpu(), torch.zeros(3001)) and not m1.cpu().any()
    o0, m0 = torch.ops.aten.native_dropout(x, 0.4, False)
    assert torch.equal(o0.cpu(), x.cpu()) and m0.cpu().all()
    e, em = torch.ops.aten.native_dropout(torch.empty(0, device="supa"), 0.5, True)
    assert e.numel() == 0 and em.numel() == 0
    assert torch.equal(F.dropout(x, 0.5, training=False).cpu(), x.cpu())


def test_moments_at_full_size(no_fallback):
    torch.supa.manual_seed(12)
    n = 1 << 26
    u = torch.empty(n, device="supa").uniform_()
    assert abs(u.mean().item() - 0.5) < 2e-4
    c = u - 0.5
    assert abs((c * c).mean().item() - 1.0 / 12) < 2e-4
    uc = u.cpu()
    assert 0.0 <= uc.min().item() and uc.max().item() < 1.0
    b = torch.empty(n, device="supa").bernoulli_(0.2)
    assert abs(b.mean().item() - 0.2) < 5 * (0.2 * 0.8 / n) ** 0.5
    # the last elements come from the same stream as the first
    tail = u[-5:].cpu().numpy()
    seed, off = 12, 0
    r = O.rng_u32(seed, off, n)[-5:]
    assert np.array_equal(tail, (r >> 8).astype(np.float32) * np.float32(2.0 ** -24))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_normal_against_oracle(dtype, no_fallback):
    torch.supa.manual_seed(51)
    t = torch.empty(100003, dtype=dtype, device="supa")
    seed, off = state()
    t.normal_(1.5, 0.25)
    assert state() == (seed, off + 1)
    want = O.normal(seed, off, t.numel(), 1.5, 0.25)
    got = t.cpu().float().numpy()
    if dtype == torch.float32:
        # double sin / cos / log on the device and on the host: equal after rounding to float
        # but for the rare value within a double rounding of a float midpoint
        assert (f32_ulp_dist(got, want) > 1).sum() == 0
        assert (got != want).mean() < 1e-3
    else:
        assert torch.equal(t.cpu(), torch.from_numpy(want).to(dtype)) or \
            (t.cpu() != torch.from_numpy(want).to(dtype)).float().mean().item() < 1e-3


def test_randn_like_and_moments(no_fallback):
    torch.supa.manual_seed(52)
    x = torch.randn(1 << 24, device="supa")
    assert abs(x.mean().item()) < 2e-3
    c = x - x.mean()
    assert abs((c * c).mean().item() - 1.0) < 2e-3
    y = torch.randn_like(x)
    assert not torch.equal(x.cpu()[:100], y.cpu()[:100])
    torch.supa.manual_seed(52)
    assert torch.equal(torch.randn(1 << 24, device="supa").cpu()[:1000], x.cpu()[:1000])
