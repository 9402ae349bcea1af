"""c5 at full size: torch.optim.AdamW(fused=True) over the 72 tensors of the
8-layer, 7B-decoder-like parameter list (1 619 066 880 float32 elements, two
multi-tensor launches per step: 40 + 32 tensors), 10 steps, against the
oracle's AdamW step tensor by tensor -- p, exp_avg, exp_avg_sq and step
bit-exact for every tensor -- then _foreach_add_.List(params, grads) and
_foreach_mul_.Scalar(params, 0.5) over the same list, bit-exact.

Inputs are drawn on the device by torch's seeded HIP generator (params
N(0, 0.02), grads N(0, 1e-3), drawn once and reused every step) and copied
into supa tensors; the host copies the oracle needs are made one tensor at a
time, in a pool of 12 threads, so host memory stays near 12 tensors'
worth."""
import concurrent.futures as cf

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu

C5_SHAPES = ([(4096, 4096)] * 4 + [(11008, 4096)] * 2 + [(4096, 11008)] + [(4096,)] * 2) * 8
LR, B1, B2, EPS, WD = 1e-4, 0.9, 0.999, 1e-8, 0.01


def _to_supa(src):
    import torch_supa
    dst = torch.empty(src.shape, dtype=src.dtype, device="supa")
    torch.cuda.synchronize()
    torch_supa._C.memcpy_d2d(dst.data_ptr(), src.data_ptr(), src.numel() * src.element_size())
    torch.supa.synchronize()
    return dst


@pytest.mark.timeout(600)
def test_c5_full_config_bit_exact(no_fallback):
    assert sum(int(np.prod(s)) for s in C5_SHAPES) == 1_619_066_880
    g = torch.Generator(device="cuda").manual_seed(0)
    p0 = [torch.randn(s, generator=g, device="cuda") * 0.02 for s in C5_SHAPES]
    g0 = [torch.randn(s, generator=g, device="cuda") * 1e-3 for s in C5_SHAPES]
    params = [_to_supa(p).requires_grad_() for p in p0]
    grads = [_to_supa(x) for x in g0]
    opt = torch.optim.AdamW(params, lr=LR, betas=(B1, B2), eps=EPS, weight_decay=WD, fused=True)
    for p, gr in zip(params, grads):
        p.grad = gr
    for _ in range(10):
        opt.step()
    torch.supa.synchronize()

    def check(i):
        hp = p0[i].cpu().numpy().ravel().copy()
        hg = g0[i].cpu().numpy().ravel().copy()
        hm, hv = np.zeros_like(hp), np.zeros_like(hp)
        for step in range(1, 11):
            O.adamw_step(hp, hg, hm, hv, float(step), LR, B1, B2, WD, EPS)
        st = opt.state[params[i]]
        bad = []
        if not np.array_equal(params[i].detach().cpu().numpy().ravel(), hp):
            bad.append("param")
        if not np.array_equal(st["exp_avg"].cpu().numpy().ravel(), hm):
            bad.append("exp_avg")
        if not np.array_equal(st["exp_avg_sq"].cpu().numpy().ravel(), hv):
            bad.append("exp_avg_sq")
        if st["step"].item() != 10.0:
            bad.append("step")
        return i, bad

    with cf.ThreadPoolExecutor(max_workers=12) as ex:
        for i, bad in ex.map(check, range(len(C5_SHAPES))):
            assert not bad, f"tensor {i} {C5_SHAPES[i]}: {bad} differ from the oracle"
    del opt

    # the list ops of c5 over the same 72 tensors (both multi-tensor tables):
    # p = (p + g) * 0.5, exact in float32
    with torch.no_grad():
        pd = [p.detach() for p in params]
        before = [p.clone() for p in pd]
        torch._foreach_add_(pd, grads)
        torch._foreach_mul_(pd, 0.5)
    torch.supa.synchronize()

    def check_list(i):
        ref = (before[i].cpu().numpy() + g0[i].cpu().numpy()) * np.float32(0.5)
        return i, np.array_equal(pd[i].cpu().numpy(), ref)

    with cf.ThreadPoolExecutor(max_workers=12) as ex:
        for i, ok in ex.map(check_list, range(len(C5_SHAPES))):
            assert ok, f"_foreach_add_.List / _foreach_mul_.Scalar differ on tensor {i}"
