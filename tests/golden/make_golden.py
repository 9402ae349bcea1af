"""Writes tests/golden/golden_cpu_aten.npz: small seeded inputs and the outputs
of the upstream aten CPU kernels of torch 2.10.0 (the reference's own tests
compare against exactly these kernels, differentially, with no stored
vectors; this file freezes one such comparison so the oracle is checked
against fixed data even where torch changes).

Run: python tests/golden/make_golden.py   (CPU only, a few seconds)."""
import os

import numpy as np
import torch
import torch.nn.functional as F

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden_cpu_aten.npz")


def main():
    g = torch.Generator().manual_seed(0)
    d = {}
    a = torch.randn(255, 33, generator=g)
    b = torch.randn(255, 33, generator=g)
    d["a"], d["b"] = a.numpy(), b.numpy()
    d["add"] = (a + b).numpy()
    d["add_alpha"] = torch.add(a, b, alpha=2.5).numpy()
    d["mul"] = (a * b).numpy()
    d["div"] = (a / b).numpy()
    d["div_floor"] = torch.div(a, b, rounding_mode="floor").numpy()
    d["silu"] = F.silu(a).numpy()
    d["sigmoid"] = torch.sigmoid(a).numpy()
    d["tanh"] = torch.tanh(a).numpy()
    d["gelu"] = F.gelu(a).numpy()
    d["gelu_tanh"] = F.gelu(a, approximate="tanh").numpy()
    x = torch.randn(6, 4096, generator=g) * 2
    d["lsm_x"] = x.numpy()
    d["lsm"] = F.log_softmax(x, -1).numpy()
    t = torch.randint(0, 4096, (6,), generator=g)
    t[3] = -100
    d["ce_t"] = t.numpy()
    xg = x.clone().requires_grad_()
    ce = F.cross_entropy(xg, t, ignore_index=-100)
    ce.backward()
    d["ce"] = ce.detach().numpy()
    d["ce_grad"] = xg.grad.numpy()
    xt = torch.randn(4, 1024, generator=g)
    tt = torch.randn(4, 1024, generator=g)
    tb = (torch.rand(4, 1024, generator=g) < 0.3).float()
    pw = torch.rand(1024, generator=g) * 1.5 + 0.5
    d["loss_x"], d["loss_t"], d["loss_tb"], d["loss_pw"] = xt.numpy(), tt.numpy(), tb.numpy(), pw.numpy()
    for red in ("none", "mean", "sum"):
        d[f"mse_{red}"] = F.mse_loss(xt, tt, reduction=red).numpy()
        d[f"sl1_{red}"] = F.smooth_l1_loss(xt, tt, reduction=red, beta=1.0).numpy()
        d[f"bce_{red}"] = F.binary_cross_entropy_with_logits(xt, tb, pos_weight=pw, reduction=red).numpy()
    p = torch.randn(1024, generator=g) * 0.02
    gr = torch.randn(1024, generator=g) * 1e-3
    d["adam_p0"], d["adam_g"] = p.numpy(), gr.numpy()
    pp = p.clone().requires_grad_()
    opt = torch.optim.AdamW([pp], lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, fused=True)
    for _ in range(10):
        pp.grad = gr.clone()
        opt.step()
    d["adam_p10"] = pp.detach().numpy()
    np.savez_compressed(OUT, **d)
    print("wrote", OUT, sum(v.nbytes for v in d.values()), "bytes (uncompressed)")


if __name__ == "__main__":
    main()
