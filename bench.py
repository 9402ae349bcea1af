"""Benchmark of the elementwise + loss operator path on one MI355X.

Prints ONE JSON line.  The headline workload (``value``) is BASELINE config 2,
contiguous leg: y = x + bias (x [64,2048,4096] bf16, bias [4096] f32, result
f32) followed by gelu(y, approximate='tanh'); one step is that pair of aten
ops over the whole tensor; ``value`` is algorithmic HBM bytes per step /
time per step, in GB/s.  ``per_config`` carries every other config
(c1 ops, c2 transposed leg, c3 cross-entropy fwd+bwd rows/s, c4 losses,
c5 fused AdamW), each as GB/s of algorithmic bytes and % of the 8 TB/s HBM
roofline.

Algorithmic bytes: every input read once, every output written once,
broadcast operands at their storage size (the per-op counts of the path's
measurement plan).  Inputs are resident in HBM before timing starts; they
are synthetic, drawn on the device with torch's seeded HIP generator and
copied into supa buffers.  Timing: HIP events on the stream the supa kernels
run on, between two device synchronisations; the headline is the median of
five batches of exactly --steps steps after --warmup untimed ones.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--configs c1,c2,c3,c4,c5]
"""
from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "torch-supa_amd"))
sys.path.insert(0, HERE)

PEAK_GBS = 8000.0  # MI355X HBM3E
METRIC = "achieved HBM GB/s and % of MI355X roofline per op; cross-entropy fwd+bwd rows/s"


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--configs", default="c1,c2,c3,c4,c5")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--probe", nargs="?", const="c2", default=None, metavar="CONFIG",
                    help="only launch the dominant kernels of CONFIG (c1..c5; default c2), after a copy-like "
                         "calibration kernel, three times each (for rocprofv3 --pmc)")
    ap.add_argument("--derive-counters", nargs="+", metavar="CSV",
                    help="CPU only: turn the counter_collection.csv files of rocprofv3 --pmc runs of "
                         "--probe CONFIG into profiles/<CONFIG>_counters.{json,md} (with --config)")
    ap.add_argument("--config", default="c2", help="the config of --derive-counters")
    ap.add_argument("--stats", default=None, help="with --derive-counters: the kernel_stats.csv of a "
                                                  "rocprofv3 --kernel-trace --stats run of the same probe")
    ap.add_argument("--render-kernel-stats", nargs=2, metavar=("STATS_CSV", "BENCH_LOG"),
                    help="CPU only: write profiles/kernel_stats_all_configs.md from the kernel_stats.csv of a "
                         "rocprofv3 --kernel-trace --stats run of bench.py --no-cpu and that run's output")
    ap.add_argument("--derive-traffic", nargs=2, metavar=("FETCH_CSV", "WRITE_CSV"),
                    help="CPU only: turn the counter_collection.csv files of two `rocprofv3 --pmc FETCH_SIZE` / "
                         "`--pmc WRITE_SIZE` runs of --probe into profiles/gelu_tanh_c2_traffic.json")
    return ap.parse_args()


BATCH_MS = 50.0  # a timed batch lasts at least this long
BATCHES = 5
HEADLINE_BATCHES = 5  # batches of exactly --steps steps for the headline
TIMING = (f"headline (value, ms_per_step, per_config.c2_contiguous.step): --warmup untimed steps, then the median of "
          f"{HEADLINE_BATCHES} batches of exactly --steps steps, each batch between device synchronisations and two "
          f"HIP events on the supa stream; other per_config entries: warm-up, then the median of {BATCHES} batches "
          f"of back-to-back calls, each batch at least {BATCH_MS:.0f} ms (or the config's call count if longer), "
          f"between two HIP events on the supa stream")


class Timer:
    """HIP events on the supa stream: warm-up calls, then BATCHES batches of
    back-to-back calls, each batch at least BATCH_MS long (and at least
    `iters` calls); returns the median batch's time per call in ms."""

    def __init__(self, torch):
        self.torch = torch

    def _batch(self, fn, k):
        t = self.torch
        t.supa.synchronize()
        e0, e1 = t.supa.Event(), t.supa.Event()
        e0.record()
        for _ in range(k):
            fn()
        e1.record()
        e1.synchronize()
        return e0.elapsed_time(e1) / k

    def time(self, fn, iters, warmup=2):
        for _ in range(warmup):
            fn()
        per_call = self._batch(fn, max(1, min(iters, 3)))  # sizes the batches
        k = max(iters, int(BATCH_MS / max(per_call, 1e-4)) + 1)
        times = sorted(self._batch(fn, k) for _ in range(BATCHES))
        return times[len(times) // 2]  # ms


def gen(torch, shape, seed, dtype, kind="normal", a=0.0, b=1.0):
    """Synthetic input: generated on the HIP device by torch, copied to supa."""
    import torch_supa
    g = torch.Generator(device="cuda").manual_seed(seed)
    if kind == "normal":
        src = torch.randn(shape, generator=g, device="cuda") * b + a
    elif kind == "uniform":
        src = torch.rand(shape, generator=g, device="cuda") * (b - a) + a
    else:  # bernoulli(p=a)
        src = (torch.rand(shape, generator=g, device="cuda") < a).float()
    src = src.to(dtype)
    dst = torch.empty(shape, dtype=dtype, device="supa")
    torch.cuda.synchronize()
    torch_supa._C.memcpy_d2d(dst.data_ptr(), src.data_ptr(), src.numel() * src.element_size())
    torch.supa.synchronize()
    del src
    return dst


def gbs(nbytes, ms):
    return nbytes / (ms * 1e-3) / 1e9


def entry(nbytes, ms):
    g = gbs(nbytes, ms)
    return {"ms": round(ms, 5), "bytes": int(nbytes), "GB/s": round(g, 1), "pct_roofline": round(100 * g / PEAK_GBS, 1)}


# ------------------------------------------------------------------ configs
def bench_c1(torch, timer):
    import torch.nn.functional as F
    n = 4096 * 4096
    # six (a, b, out) sets = 1.2 GB rotate so the 256 MB last-level cache cannot hold the working set
    sets = [(gen(torch, (4096, 4096), 10 + i, torch.float32), gen(torch, (4096, 4096), 20 + i, torch.float32),
             torch.empty(4096, 4096, device="supa")) for i in range(6)]
    res = {}
    for name, fn, nbytes in [
        ("add", lambda s: torch.add(s[0], s[1], alpha=1, out=s[2]), 12 * n),
        ("mul", lambda s: torch.mul(s[0], s[1], out=s[2]), 12 * n),
        ("gelu", lambda s: torch.ops.aten.gelu.out(s[0], approximate="none", out=s[2]), 8 * n),
        ("silu", lambda s: torch.ops.aten.silu.out(s[0], out=s[2]), 8 * n),
    ]:
        k = [0]

        def step():
            fn(sets[k[0] % 6])
            k[0] += 1
        ms = timer.time(step, 300, warmup=6)
        res[name] = entry(nbytes, ms)
    del sets
    return res


def c2_inputs(torch, transposed):
    if transposed:
        x = gen(torch, (64, 4096, 2048), 2, torch.bfloat16).transpose(1, 2)
    else:
        x = gen(torch, (64, 2048, 4096), 1, torch.bfloat16)
    bias = gen(torch, (4096,), 3, torch.float32, b=0.02)
    return x, bias


C1_N = 4096 * 4096
C2_N = 64 * 2048 * 4096
C2_ADD_BYTES = 2 * C2_N + 4 * C2_N + 4 * 4096
C2_GELU_BYTES = 8 * C2_N


def bench_c2(torch, timer, x, bias, iters=20, t_step=None):
    """c2's two aten ops alone (out= buffers) and the step; t_step, when
    given, is the headline's own measurement of the same step."""
    import torch.nn.functional as F
    y = torch.empty_strided(x.shape, x.stride(), dtype=torch.float32, device="supa")
    z = torch.empty_strided(x.shape, x.stride(), dtype=torch.float32, device="supa")
    t_add = timer.time(lambda: torch.add(x, bias, out=y), iters)
    t_gelu = timer.time(lambda: torch.ops.aten.gelu.out(y, approximate="tanh", out=z), iters)
    if t_step is None:
        t_step = timer.time(lambda: F.gelu(x + bias, approximate="tanh"), iters)
    return {"add": entry(C2_ADD_BYTES, t_add), "gelu_tanh": entry(C2_GELU_BYTES, t_gelu),
            "step": entry(C2_ADD_BYTES + C2_GELU_BYTES, t_step)}


C3_N, C3_V = 8192, 128256
C3_NV = C3_N * C3_V
C3_BYTES = {"_log_softmax": 4 * C3_NV, "nll_loss_forward": 81926, "nll_loss_backward": 2 * C3_NV + 65538,
            "_log_softmax_backward_data": 6 * C3_NV}


def bench_c3(torch, timer, iters=10):
    import torch.nn.functional as F
    logits = gen(torch, (C3_N, C3_V), 4, torch.bfloat16, b=2.0)
    g = torch.Generator(device="cuda").manual_seed(5)
    t = torch.randint(0, C3_V, (C3_N,), generator=g, device="cuda")
    t[torch.randperm(C3_N, generator=g, device="cuda")[:410]] = -100
    tgt = torch.empty(C3_N, dtype=torch.int64, device="supa")
    torch.cuda.synchronize()
    import torch_supa
    torch_supa._C.memcpy_d2d(tgt.data_ptr(), t.data_ptr(), C3_N * 8)
    logits.requires_grad_()

    def step():
        logits.grad = None
        loss = F.cross_entropy(logits, tgt, ignore_index=-100, reduction="mean")
        loss.backward()
    ms = timer.time(step, iters, warmup=2)
    res = {"fwd_bwd": dict(entry(sum(C3_BYTES.values()), ms), rows_per_s=round(C3_N / (ms * 1e-3), 1))}
    # the opt-in fused path (not the config's decomposition): forward reads the
    # logits once, backward reads them once and writes the gradient once --
    # 6 N V bytes plus per-row targets, lse and losses
    was = torch.supa.fused_cross_entropy_enabled()
    torch.supa.set_fused_cross_entropy_enabled(True)
    try:
        ms_f = timer.time(step, iters, warmup=2)
    finally:
        torch.supa.set_fused_cross_entropy_enabled(was)
    fused_bytes = 6 * C3_NV + C3_N * (8 + 4 + 4) * 2
    res["fused_fwd_bwd"] = dict(entry(fused_bytes, ms_f), rows_per_s=round(C3_N / (ms_f * 1e-3), 1),
                                speedup_vs_decomposition=round(ms / ms_f, 3))
    lx = logits.detach()
    lsm = torch.ops.aten._log_softmax(lx, 1, False)
    out, tw = torch.ops.aten.nll_loss_forward(lsm, tgt, None, 1, -100)
    go = torch.ones((), dtype=torch.bfloat16, device="supa")
    gn = torch.ops.aten.nll_loss_backward(go, lsm, tgt, None, 1, -100, tw)
    res["_log_softmax"] = entry(C3_BYTES["_log_softmax"], timer.time(
        lambda: torch.ops.aten._log_softmax.out(lx, 1, False, out=lsm), iters))
    res["nll_loss_forward"] = entry(C3_BYTES["nll_loss_forward"], timer.time(
        lambda: torch.ops.aten.nll_loss_forward(lsm, tgt, None, 1, -100), iters))
    res["nll_loss_backward"] = entry(C3_BYTES["nll_loss_backward"], timer.time(
        lambda: torch.ops.aten.nll_loss_backward.grad_input(go, lsm, tgt, None, 1, -100, tw, grad_input=gn), iters))
    gi = torch.empty_like(lx)
    res["_log_softmax_backward_data"] = entry(C3_BYTES["_log_softmax_backward_data"], timer.time(
        lambda: torch.ops.aten._log_softmax_backward_data.out(gn, lsm, 1, torch.bfloat16, out=gi), iters))
    del lsm, gn, gi, lx
    logits.grad = None
    del logits
    res["fp32_routing"] = bench_c3_fp32(torch, timer, tgt)
    return res


def bench_c3_fp32(torch, timer, tgt, iters=5):
    """c3's shape with float32 logits (not the config: the reference's routing
    of float32 cross-entropy).  fused: the default route, as the reference
    routes 2-d float32 logits to its fast path; decomposition: the
    log_softmax + nll_loss route that bfloat16 takes.  Also 512 rows with a
    probability target [512, 128256] float32, fused and decomposed."""
    import torch.nn.functional as F
    x = gen(torch, (C3_N, C3_V), 4, torch.float32, b=2.0).requires_grad_()
    was = torch.supa.fused_cross_entropy_enabled()
    out = {}
    try:
        for name, mode in (("fused", True), ("decomposition", False)):
            torch.supa.set_fused_cross_entropy_enabled(mode)

            def step():
                x.grad = None
                F.cross_entropy(x, tgt, ignore_index=-100).backward()
            ms = timer.time(step, iters, warmup=2)
            # fused: 4 NV forward + 8 NV backward; decomposition: _log_softmax 8 NV, nll_loss_backward 4 NV,
            # _log_softmax_backward_data 12 NV (float32 bytes)
            nbytes = (12 if mode else 24) * C3_NV
            out[name] = dict(entry(nbytes, ms), rows_per_s=round(C3_N / (ms * 1e-3), 1))
        out["fused_speedup"] = round(out["decomposition"]["ms"] / out["fused"]["ms"], 3)
        xp = x.detach()[:512].clone().requires_grad_()
        p = gen(torch, (512, C3_V), 11, torch.float32, kind="uniform", a=0.0, b=2.0 / C3_V)
        for name, mode in (("prob_fused", True), ("prob_decomposition", False)):
            torch.supa.set_fused_cross_entropy_enabled(mode)

            def stepp():
                xp.grad = None
                F.cross_entropy(xp, p).backward()
            ms = timer.time(stepp, iters, warmup=2)
            out[name] = {"ms": round(ms, 5), "rows": 512}
    finally:
        torch.supa.set_fused_cross_entropy_enabled(was)
    return out


def bench_c4(torch, timer, iters=21, sets=3):
    """c4 with `sets` independent input sets used round-robin, so no op reads
    its inputs back from the 256 MB MALL (one set of x, t is 256 MB)."""
    import torch.nn.functional as F
    R, C = 32, 1048576
    n = R * C
    xs = [gen(torch, (R, C), 6 + 10 * k, torch.float32) for k in range(sets)]
    ts = [gen(torch, (R, C), 7 + 10 * k, torch.float32) for k in range(sets)]
    tbs = [gen(torch, (R, C), 8 + 10 * k, torch.float32, kind="bernoulli", a=0.3) for k in range(sets)]
    pw = gen(torch, (C,), 9, torch.float32, kind="uniform", a=0.5, b=2.0)
    res = {}
    pwb = 4 * C

    def rot(fn):
        it = [0]

        def call():
            k = it[0] % sets
            it[0] += 1
            return fn(k)
        return call

    for red in ("none", "sum", "mean"):
        gos = ([gen(torch, (R, C), 11 + 10 * k, torch.float32) for k in range(sets)] if red == "none"
               else [torch.ones((), device="supa")] * sets)
        rc = {"none": 0, "mean": 1, "sum": 2}[red]
        fwd_b = 12 * n if red == "none" else 8 * n + 4
        bwd_b = 16 * n if red == "none" else 12 * n + 4
        res[f"mse_{red}_fwd"] = entry(fwd_b, timer.time(rot(lambda k: F.mse_loss(xs[k], ts[k], reduction=red)), iters))
        res[f"mse_{red}_bwd"] = entry(bwd_b, timer.time(
            rot(lambda k: torch.ops.aten.mse_loss_backward(gos[k], xs[k], ts[k], rc)), iters))
        res[f"smooth_l1_{red}_fwd"] = entry(fwd_b, timer.time(
            rot(lambda k: F.smooth_l1_loss(xs[k], ts[k], reduction=red, beta=1.0)), iters))
        res[f"smooth_l1_{red}_bwd"] = entry(bwd_b, timer.time(
            rot(lambda k: torch.ops.aten.smooth_l1_loss_backward(gos[k], xs[k], ts[k], rc, 1.0)), iters))
        bce_fwd_b = (12 * n if red == "none" else 8 * n + 4) + pwb
        res[f"bce_{red}_fwd"] = entry(bce_fwd_b, timer.time(
            rot(lambda k: F.binary_cross_entropy_with_logits(xs[k], tbs[k], pos_weight=pw, reduction=red)), iters))
        xgs = [x.detach().requires_grad_() for x in xs]
        losses = [F.binary_cross_entropy_with_logits(xg, tb, pos_weight=pw, reduction=red) for xg, tb in zip(xgs, tbs)]
        gsz = 4 if red != "none" else 4 * n
        # one fused kernel (the default): reads grad, x, target, pos_weight; writes grad_x
        bce_bwd_b = gsz + 12 * n + pwb
        res[f"bce_{red}_bwd"] = entry(bce_bwd_b, timer.time(
            rot(lambda k: torch.autograd.grad(losses[k], xgs[k], gos[k], retain_graph=True)), iters))
        del xgs, losses, gos
    return res


C5_SHAPES = ([(4096, 4096)] * 4 + [(11008, 4096)] * 2 + [(4096, 11008)] + [(4096,)] * 2) * 8


def bench_c5(torch, timer, steps=10):
    P = 0
    params, grads = [], []
    for i, s in enumerate(C5_SHAPES):
        params.append(gen(torch, s, 100 + i, torch.float32, b=0.02).requires_grad_())
        grads.append(gen(torch, s, 1000 + i, torch.float32, b=1e-3))
        n = 1
        for d in s:
            n *= d
        P += n
    opt = torch.optim.AdamW(params, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, fused=True)
    for p, g in zip(params, grads):
        p.grad = g
    ms = timer.time(opt.step, steps, warmup=1)
    res = {"fused_adamw_step": dict(entry(28 * P, ms), params=P)}
    # The default implementation (foreach=None picks foreach on supa): eight
    # list ops per step, 80P algorithmic bytes -- mul 8P, lerp 12P, mul 8P,
    # addcmul 12P (grads read once), sqrt 8P, div 8P, add 8P, addcdiv 16P.
    opt_fe = torch.optim.AdamW(params, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01)
    res["foreach_adamw_step"] = dict(entry(80 * P, timer.time(opt_fe.step, steps, warmup=1)), params=P)
    del opt_fe
    # clip_grad_norm_ over the 72 gradients: _foreach_norm (4P) + _foreach_mul_ (8P)
    res["clip_grad_norm_"] = entry(12 * P, timer.time(lambda: torch.nn.utils.clip_grad_norm_(params, 1e9), 3,
                                                      warmup=1))
    with torch.no_grad():
        pd = [p.detach() for p in params]
        res["_foreach_add_List"] = entry(12 * P, timer.time(lambda: torch._foreach_add_(pd, grads), 3, warmup=1))
        res["_foreach_mul_Scalar"] = entry(8 * P, timer.time(lambda: torch._foreach_mul_(pd, 1.0), 3, warmup=1))
        # GradScaler's unscale of the 72 gradients (inv_scale 1: check only, values kept)
        found_inf = torch.zeros(1, device="supa")
        inv = torch.ones(1, device="supa")
        res["_amp_foreach_non_finite_check_and_unscale_"] = entry(8 * P, timer.time(
            lambda: torch._amp_foreach_non_finite_check_and_unscale_(grads, found_inf, inv), 3, warmup=1))
    return res


# ------------------------------------------------------------ CPU baselines
def cpu_port_baseline():
    """The oracle (single-threaded C restatement) on a bounded sample of the
    headline workload: 1/16 of c2 (x [4,2048,4096]), repeated to ~10 s."""
    import numpy as np
    import oracle as O
    rng = np.random.default_rng(0)
    n = 4 * 2048 * 4096
    x = O.f32_to_bf16(rng.standard_normal(n, dtype=np.float32)).reshape(4, 2048, 4096)
    bias = (rng.standard_normal(4096, dtype=np.float32) * 0.02)
    t0 = time.perf_counter()
    reps = 0
    while True:
        y = O.binary(O.ADD, O.bf16_to_f32(x), bias)
        z = O.unary(O.GELU_TANH, y)
        reps += 1
        el = time.perf_counter() - t0
        if el >= 10.0:
            break
    per = el / reps
    nbytes = (2 * n + 4 * n + 4 * 4096) + 8 * n
    return {"value": round(nbytes / per / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"oracle/ C restatement, c2 workload on x[4,2048,4096] (1/16 of the config), "
                      f"{reps} reps, {per * 1e3:.1f} ms per rep incl. the bf16 widening"}


def _cpu_host_info(torch):
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return {"threads": torch.get_num_threads(), "cpu_count": os.cpu_count(), "cpu": cpu_model,
            "torch": torch.__version__}


def _cpu_time(fn, reps=3):
    """1 warm-up, then the median of `reps` wall-clock runs (seconds)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def _cpu_entry(nbytes, sec, sample):
    g = nbytes / sec / 1e9
    return {"ms": round(sec * 1e3, 3), "GB/s": round(g, 2), "sample": sample}


def cpu_aten_baselines(torch, configs):
    """Upstream aten CPU kernels of the installed torch, on the same seeded
    inputs (drawn on the CPU) and the same algorithmic bytes as the GPU
    figures, on this host's torch threads (OMP_NUM_THREADS; 16 on the GPU
    boxes): 1 warm-up, median of 3.  Bounded samples keep the whole baseline
    near a minute; each entry names its sample.  Reported beside the GPU
    figures, never a pass/fail bar."""
    import torch.nn.functional as F
    res = {"host": _cpu_host_info(torch)}
    g = torch.Generator().manual_seed(0)
    if "c1" in configs:
        a = torch.randn(4096, 4096, generator=g)
        b = torch.randn(4096, 4096, generator=g)
        o = torch.empty_like(a)
        n = a.numel()
        full = "full size [4096,4096] f32"
        res["c1"] = {
            "add": _cpu_entry(12 * n, _cpu_time(lambda: torch.add(a, b, alpha=1, out=o)), full),
            "mul": _cpu_entry(12 * n, _cpu_time(lambda: torch.mul(a, b, out=o)), full),
            "gelu": _cpu_entry(8 * n, _cpu_time(lambda: torch.ops.aten.gelu.out(a, approximate="none", out=o)), full),
            "silu": _cpu_entry(8 * n, _cpu_time(lambda: torch.ops.aten.silu.out(a, out=o)), full),
        }
        del a, b, o
    # c2 (the headline workload) on 1/16 of the config: x [4,2048,4096]
    x = torch.randn(4, 2048, 4096, generator=g).to(torch.bfloat16)
    bias = torch.randn(4096, generator=g) * 0.02
    n = x.numel()
    sample = "x[4,2048,4096] bf16 + bias f32 (1/16 of c2), contiguous"
    t_add = _cpu_time(lambda: x + bias)
    y = x + bias
    t_gelu = _cpu_time(lambda: F.gelu(y, approximate="tanh"))
    t_step = _cpu_time(lambda: F.gelu(x + bias, approximate="tanh"))
    res["c2_contiguous"] = {"add": _cpu_entry(2 * n + 4 * n + 16384, t_add, sample),
                            "gelu_tanh": _cpu_entry(8 * n, t_gelu, sample),
                            "step": _cpu_entry(14 * n + 16384, t_step, sample)}
    del x, y
    if "c3" in configs:
        rows = 512
        logits = (torch.randn(rows, C3_V, generator=g) * 2).to(torch.bfloat16).requires_grad_()
        t = torch.randint(0, C3_V, (rows,), generator=g)
        t[torch.randperm(rows, generator=g)[:round(0.05 * rows)]] = -100

        def step():
            logits.grad = None
            F.cross_entropy(logits, t, ignore_index=-100).backward()
        sec = _cpu_time(step)
        nbytes = sum(C3_BYTES.values()) * rows / C3_N
        res["c3"] = {"fwd_bwd": dict(_cpu_entry(nbytes, sec, f"{rows} of the 8192 rows (1/16), bf16 [{rows},128256]"),
                                     rows_per_s=round(rows / sec, 1))}
        del logits
    if "c4" in configs:
        R, C = 4, 1048576
        n = R * C
        xc = torch.randn(R, C, generator=g)
        tc = torch.randn(R, C, generator=g)
        tb = (torch.rand(R, C, generator=g) < 0.3).float()
        pw = torch.rand(C, generator=g) * 1.5 + 0.5
        sample = "4 of the 32 rows (1/8): [4,1048576] f32"
        c4 = {}
        for red in ("none", "sum", "mean"):
            fwd_b = 12 * n if red == "none" else 8 * n + 4
            c4[f"mse_{red}_fwd"] = _cpu_entry(fwd_b, _cpu_time(lambda: F.mse_loss(xc, tc, reduction=red)), sample)
            c4[f"smooth_l1_{red}_fwd"] = _cpu_entry(
                fwd_b, _cpu_time(lambda: F.smooth_l1_loss(xc, tc, reduction=red, beta=1.0)), sample)
            bwd_b = 16 * n if red == "none" else 12 * n + 4
            rc = {"none": 0, "mean": 1, "sum": 2}[red]
            gl = torch.randn(R, C, generator=g) if red == "none" else torch.ones(())
            c4[f"mse_{red}_bwd"] = _cpu_entry(bwd_b, _cpu_time(
                lambda: torch.ops.aten.mse_loss_backward(gl, xc, tc, rc)), sample)
            c4[f"smooth_l1_{red}_bwd"] = _cpu_entry(bwd_b, _cpu_time(
                lambda: torch.ops.aten.smooth_l1_loss_backward(gl, xc, tc, rc, 1.0)), sample)
            c4[f"bce_{red}_fwd"] = _cpu_entry(fwd_b + 4 * C, _cpu_time(
                lambda: F.binary_cross_entropy_with_logits(xc, tb, pos_weight=pw, reduction=red)), sample)
            xg = xc.detach().requires_grad_()
            loss = F.binary_cross_entropy_with_logits(xg, tb, pos_weight=pw, reduction=red)
            go = torch.ones_like(loss)
            gsz = 4 if red != "none" else 4 * n
            c4[f"bce_{red}_bwd"] = _cpu_entry(gsz + 12 * n + 4 * C, _cpu_time(
                lambda: torch.autograd.grad(loss, xg, go, retain_graph=True)), sample)
        res["c4"] = c4
        del xc, tc, tb
    if "c5" in configs:
        shapes = C5_SHAPES[:9]  # one decoder layer of the 8
        ps = [(torch.randn(s, generator=g) * 0.02).requires_grad_() for s in shapes]
        for p in ps:
            p.grad = torch.randn(p.shape, generator=g) * 1e-3
        P = sum(p.numel() for p in ps)
        opt = torch.optim.AdamW(ps, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, fused=True)
        sample = f"one layer of the 8 (9 tensors, {P} parameters), fused=True"
        res["c5"] = {"fused_adamw_step": dict(_cpu_entry(28 * P, _cpu_time(opt.step), sample), params=P)}
        del ps, opt
    return res


def _run_args(path, suffix):
    """(-d directory, -o prefix) of the rocprofv3 run that wrote `path`
    (`<dir>/<prefix><suffix>`), for the commands a summary records."""
    d, b = os.path.split(path)
    return (d or "."), (b[: -len(suffix)] if b.endswith(suffix) else b)


def _counters_in(path):
    import csv

    with open(path) as f:
        return sorted({r["Counter_Name"] for r in csv.DictReader(f)})


def traffic_from_profiles():
    p = os.path.join(HERE, "profiles", "gelu_tanh_c2_traffic.json")
    if os.path.exists(p):
        try:
            return json.load(open(p)).get("bytes_per_launch")
        except (OSError, ValueError):
            return None
    return None


PROBE_CAL_KERNEL = "UnaryOp<11, float>"  # abs.out: the calibration kernel
PROBE_GELU_KERNEL = "UnaryOp<1, float>"  # gelu(approximate='tanh')


def derive_traffic(fetch_csv, write_csv):
    """HBM bytes per launch of the c2 gelu kernel from two PMC runs of --probe.

    FETCH_SIZE and WRITE_SIZE are reported in KiB per dispatch; each is scaled
    by known / measured for the calibration kernel (abs.out over 2^28 f32:
    exactly 1 GiB read and 1 GiB written), then averaged over the gelu
    dispatches."""
    import csv

    names = set()

    def per_kernel(path):
        cal, gel = [], []
        with open(path) as f:
            for r in csv.DictReader(f):
                name, val = r["Kernel_Name"], float(r["Counter_Value"])
                if "k_contig" not in name:
                    continue
                if PROBE_CAL_KERNEL in name:
                    cal.append(val)
                elif PROBE_GELU_KERNEL in name:
                    gel.append(val)
                    names.add(name.split("(")[0].replace("void ", ""))
        if not cal or not gel:
            raise SystemExit(f"{path}: calibration or gelu dispatches missing")
        return sum(cal) / len(cal), sum(gel) / len(gel), len(gel)

    known_kib = float(1 << 20)
    f_cal, f_gel, nf = per_kernel(fetch_csv)
    w_cal, w_gel, nw = per_kernel(write_csv)
    f_scale, w_scale = known_kib / f_cal, known_kib / w_cal
    read_b = f_gel * f_scale * 1024
    write_b = w_gel * w_scale * 1024
    out = {
        "kernel": " / ".join(sorted(names)) + " -- gelu(tanh) f32 [64,2048,4096]",
        "bytes_per_launch": int(round(read_b + write_b)),
        "read_bytes": int(round(read_b)), "write_bytes": int(round(write_b)),
        "algorithmic_bytes": C2_GELU_BYTES,
        "fetch_kib_raw": round(f_gel, 1), "write_kib_raw": round(w_gel, 1),
        "fetch_scale": round(f_scale, 5), "write_scale": round(w_scale, 5),
        "calibration": "abs.out over 2^28 f32 (1 GiB read, 1 GiB written): FETCH_SIZE "
                       f"{f_cal:.1f} KiB, WRITE_SIZE {w_cal:.1f} KiB per dispatch",
        "dispatches": {"fetch": nf, "write": nw},
    }
    path = os.path.join(HERE, "profiles", "gelu_tanh_c2_traffic.json")
    with open(path, "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    md = ["# HBM traffic of the c2 gelu(tanh) kernel (rocprofv3 PMC)", "",
          f"Two counter runs of the bench's probe mode ({PROBE_REPS}x `abs.out` over 2^28 f32 as the calibration -- "
          f"exactly 1 GiB read and 1 GiB written per dispatch -- then {PROBE_REPS}x `gelu.out(approximate='tanh')` "
          "over the c2 f32 tensor [64,2048,4096]):", "", "```",
          "cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT",
          "timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE --output-format csv -d {} -o {} -- python3 bench.py --probe"
          .format(*_run_args(fetch_csv, "_counter_collection.csv")),
          "timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE --output-format csv -d {} -o {} -- python3 bench.py --probe"
          .format(*_run_args(write_csv, "_counter_collection.csv")),
          f"python3 bench.py --derive-traffic {fetch_csv} {write_csv}", "```", "",
          "The last command (CPU only) writes `gelu_tanh_c2_traffic.json` and this file; `bench.py` reports the "
          "json's `bytes_per_launch` as `roofline.traffic`.", f"Kernel: `{out['kernel']}`.", "",
          "| dispatch | FETCH_SIZE KiB | WRITE_SIZE KiB |", "|---|---:|---:|",
          f"| abs.out calibration (1 GiB each way) | {f_cal:.1f} | {w_cal:.1f} |",
          f"| gelu(tanh) c2 (2 GiB each way) | {f_gel:.1f} | {w_gel:.1f} |", "",
          f"FETCH_SIZE counts half of the bytes a streaming kernel reads on gfx950 (scale {f_scale:.5f} from the "
          f"calibration); WRITE_SIZE is exact (scale {w_scale:.5f}).  Scaled traffic of one gelu launch: "
          f"{int(round(read_b))} B read + {int(round(write_b))} B written = {out['bytes_per_launch']} B against "
          f"{C2_GELU_BYTES} B algorithmic ({out['bytes_per_launch'] / C2_GELU_BYTES:.4f}): no re-reads and no write "
          "amplification, so the gap to the roofline is achieved bandwidth, not extra traffic."]
    with open(os.path.join(HERE, "profiles", "gelu_tanh_c2_traffic.md"), "w") as f:
        f.write("\n".join(md) + "\n")
    print(json.dumps(out))


# (label, exact kernel name, launch grid in threads or None for any, algorithmic
# bytes per launch) of the bench's dominant kernels, for the roofline rows of
# --render-kernel-stats.  The grid singles out c1's launches of templates that
# other configs launch too (c4's and c5's muls run the same k_contig).
STATS_ROOFLINE_ROWS = [
    ("c2 gelu('tanh') f32 [64,2048,4096] -- the headline kernel",
     "sa::k_contig<64, 4, sa::UnaryOp<1, float>, float, float, float, float>", None, 8 * C2_N),
    ("c2 add bf16 x + f32 bias -> f32 (both legs)",
     "sa::k_row2d<64, 4, sa::AddOp<float>, float, float, float, sa::bf16, float>", None, C2_ADD_BYTES),
    ("c2 transposed leg: bf16 x `.contiguous()` (LDS-tiled transpose)",
     "sa::k_transpose_vec<sa::IdentityOp<float>, float, sa::bf16, sa::bf16, sa::bf16>", None, 4 * C2_N),
    ("c1 add f32 [4096,4096]", "sa::k_contig<64, 4, sa::AddOp<float>, float, float, float, float, float>",
     C1_N // 4, 12 * C1_N),
    ("c1 mul", "sa::k_contig<64, 4, sa::MulOp<float>, float, float, float, float, float>", C1_N // 4, 12 * C1_N),
    ("c1 gelu('none')", "sa::k_contig<64, 4, sa::UnaryOp<0, float>, float, float, float, float>", C1_N // 4,
     8 * C1_N),
    ("c1 silu", "sa::k_contig<64, 4, sa::UnaryOp<2, float>, float, float, float, float>", C1_N // 4, 8 * C1_N),
    ("c3 _log_softmax", "sa::k_lsm_fwd_split<sa::bf16, sa::bf16, true>", None, 4 * C3_NV),
    ("c3 nll_loss_backward", "sa::k_nll_bwd<sa::bf16, 8>", None, 2 * C3_NV + 65538),
    ("c3 _log_softmax_backward_data", "sa::k_lsm_bwd_split<sa::bf16, sa::bf16>", None, 6 * C3_NV),
    ("c3 fused cross-entropy forward (bf16 opt-in; float32 takes it by default)", "sa::k_ce_fwd<sa::bf16, true>", None, 2 * C3_NV),
    ("c3 fused cross-entropy backward (bf16 opt-in; float32 takes it by default)", "sa::k_ce_bwd<sa::bf16, true>", None, 4 * C3_NV),
    ("c5 _fused_adamw_ (two launches per step, 40 + 32 tensors; half of 28 B x 1.62 G each on average)",
     "sa::k_adamw_plain<float, 256l, 0, 1, false, false>", None, 14 * 1619066880),
]


def render_kernel_stats(stats_csv, bench_log):
    """profiles/kernel_stats_all_configs.md from the kernel_stats.csv of a
    `rocprofv3 --kernel-trace --stats` run of `bench.py --no-cpu`, the
    kernel_trace.csv beside it (each roofline row's launches, by grid) and
    that run's JSON line (the bench's live HIP-event timing of the same
    launches)."""
    import csv

    with open(stats_csv) as f:
        rows = [r for r in csv.DictReader(f) if "sa::" in r["Name"]]
    line = [l for l in open(bench_log) if l.startswith("{")][-1]
    bench = json.loads(line)

    def short(n):
        n = n.replace("void ", "")
        return n[: n.index(">(") + 1] if ">(" in n else n.split("(")[0]

    # per (kernel, grid) launch durations from the trace
    wanted = {name for _, name, _, _ in STATS_ROOFLINE_ROWS}
    durations = {}
    with open(stats_csv.replace("_kernel_stats.csv", "_kernel_trace.csv")) as f:
        for r in csv.DictReader(f):
            name = short(r["Kernel_Name"])
            if name in wanted:
                ns = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
                durations.setdefault((name, int(r["Grid_Size_X"])), []).append(ns)

    def launches(name, grid):
        got = [d for (n, g), v in durations.items() if n == name and (grid is None or g == grid) for d in v]
        return (len(got), sum(got) / len(got) / 1e3) if got else (0, None)

    by_name = {short(r["Name"]): r for r in rows}
    out = ["# Kernel statistics, every bench config (MI355X, gfx950)", "",
           "Commands (repo root on the GPU box; the second runs on any machine):", "", "```",
           "cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT",
           "rocprofv3 --kernel-trace --stats --output-format csv -d {} -o {} -- \\".format(
               *_run_args(stats_csv, "_kernel_stats.csv")),
           f"    python3 bench.py --no-cpu --steps 10 > {bench_log}",
           f"python3 bench.py --render-kernel-stats {stats_csv} {bench_log}", "```", "",
           "Every config runs: c1 with 6 rotating buffer sets, c2 both legs, c3 (decomposition and fused), c4 with "
           "3 rotating input sets, c5 = 72-tensor fused AdamW, the default foreach AdamW, clip_grad_norm_ and the "
           "foreach / AMP lines.  `k_contig<BS, VEC, ...>`, `k_row2d<BS, VEC, ...>`: BS threads per workgroup "
           "(64 = one wavefront).  Only this library's kernels are listed; the rest of the trace is torch's own "
           "input generation on its HIP device before the copies into supa tensors.  The roofline rows average "
           "the kernel trace's launches of that kernel at that grid (c1's rows: c1's grid of 4 194 304 threads, "
           "since c4 and c5 launch the same templates at other sizes); the table of all kernels averages every "
           "launch of a name.", "",
           "## Roofline rows (algorithmic bytes per launch / average duration)", "",
           "| kernel | name | grid (threads) | calls | avg us | algorithmic B | GB/s | % of 8 TB/s |",
           "|---|---|---:|---:|---:|---:|---:|---:|"]
    for label, name, grid, nbytes in STATS_ROOFLINE_ROWS:
        calls, us = launches(name, grid)
        if not calls:
            continue
        g = nbytes / (us * 1e-6) / 1e9
        out.append(f"| {label} | `{name}` | {'any' if grid is None else f'{grid:,}'} | {calls} | {us:.1f} | "
                   f"{nbytes:,} | {g:.0f} | {g / 80:.1f} |")
    rf = bench.get("roofline", {})
    calls, us = launches(STATS_ROOFLINE_ROWS[0][1], STATS_ROOFLINE_ROWS[0][2])
    if calls and rf.get("avg_launch_ms"):
        bus = rf["avg_launch_ms"] * 1e3
        out += ["", f"Cross-check of the headline's dominant kernel: {us:.1f} us average here, {bus:.1f} us in the "
                f"same run's live HIP-event timing (`bench.py` `roofline.avg_launch_ms`): within "
                f"{abs(us - bus) / bus * 100:.1f} %.  The bench reports roofline.achieved = {rf.get('achieved')} GB/s "
                f"(frac {rf.get('frac')}); HBM traffic per launch from the PMC runs "
                f"(`gelu_tanh_c2_traffic.md`): {rf.get('traffic')} B."]
    out += ["", "## All kernels", "", "| kernel | calls | avg us | min us | max us | % of GPU time |",
            "|---|---:|---:|---:|---:|---:|"]
    for r in rows:
        out.append(f"| `{short(r['Name'])}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.1f} | "
                   f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | {float(r['Percentage']):.4g} |")
    path = os.path.join(HERE, "profiles", "kernel_stats_all_configs.md")
    with open(path, "w") as f:
        f.write("\n".join(out) + "\n")
    print(path)


PROBE_REPS = 3


def _probe_ops(torch, cfg):
    """(name, fn) of the config's dominant aten calls, inputs already on the
    device."""
    import torch.nn.functional as F
    if cfg == "c1":
        a = gen(torch, (4096, 4096), 10, torch.float32)
        b = gen(torch, (4096, 4096), 20, torch.float32)
        o = torch.empty_like(a)
        return [("add", lambda: torch.add(a, b, out=o)), ("mul", lambda: torch.mul(a, b, out=o)),
                ("gelu", lambda: torch.ops.aten.gelu.out(a, approximate="none", out=o)),
                ("silu", lambda: torch.ops.aten.silu.out(a, out=o))]
    if cfg == "c2":
        x, bias = c2_inputs(torch, transposed=False)
        y = x + bias
        z = torch.empty_like(y)
        xt, _ = c2_inputs(torch, transposed=True)
        xc = torch.empty(xt.shape, dtype=xt.dtype, device="supa")
        return [("add", lambda: torch.add(x, bias, out=y)),
                ("gelu_tanh", lambda: torch.ops.aten.gelu.out(y, approximate="tanh", out=z)),
                ("transposed_contiguous", lambda: xc.copy_(xt))]
    if cfg == "c3":
        lx = gen(torch, (C3_N, C3_V), 4, torch.bfloat16, b=2.0)
        tgt = torch.randint(0, C3_V, (C3_N,)).to("supa")
        lsm = torch.ops.aten._log_softmax(lx, 1, False)
        out, tw = torch.ops.aten.nll_loss_forward(lsm, tgt, None, 1, -100)
        go = torch.ones((), dtype=torch.bfloat16, device="supa")
        gn = torch.ops.aten.nll_loss_backward(go, lsm, tgt, None, 1, -100, tw)
        gi = torch.empty_like(lx)
        return [("_log_softmax", lambda: torch.ops.aten._log_softmax.out(lx, 1, False, out=lsm)),
                ("nll_loss_forward", lambda: torch.ops.aten.nll_loss_forward(lsm, tgt, None, 1, -100)),
                ("nll_loss_backward", lambda: torch.ops.aten.nll_loss_backward.grad_input(
                    go, lsm, tgt, None, 1, -100, tw, grad_input=gn)),
                ("_log_softmax_backward_data", lambda: torch.ops.aten._log_softmax_backward_data.out(
                    gn, lsm, 1, torch.bfloat16, out=gi))]
    if cfg == "c4":
        R, C = 32, 1048576
        xc = gen(torch, (R, C), 6, torch.float32)
        tc = gen(torch, (R, C), 7, torch.float32)
        tb = gen(torch, (R, C), 8, torch.float32, kind="bernoulli", a=0.3)
        pw = gen(torch, (C,), 9, torch.float32, kind="uniform", a=0.5, b=2.0)
        xg = xc.detach().requires_grad_()
        loss = F.binary_cross_entropy_with_logits(xg, tb, pos_weight=pw, reduction="none")
        go = gen(torch, (R, C), 11, torch.float32)
        return [("mse_none_fwd", lambda: F.mse_loss(xc, tc, reduction="none")),
                ("mse_sum_fwd", lambda: F.mse_loss(xc, tc, reduction="sum")),
                ("bce_none_fwd", lambda: F.binary_cross_entropy_with_logits(xc, tb, pos_weight=pw,
                                                                             reduction="none")),
                ("bce_none_bwd", lambda: torch.autograd.grad(loss, xg, go, retain_graph=True))]
    if cfg == "c5":
        params, grads = [], []
        for i, sh in enumerate(C5_SHAPES):
            params.append(gen(torch, sh, 100 + i, torch.float32, b=0.02).requires_grad_())
            grads.append(gen(torch, sh, 1000 + i, torch.float32, b=1e-3))
        opt = torch.optim.AdamW(params, lr=1e-4, betas=(0.9, 0.999), eps=1e-8, weight_decay=0.01, fused=True)
        for p_, g_ in zip(params, grads):
            p_.grad = g_
        pd = [p_.detach() for p_ in params]
        return [("fused_adamw_step", opt.step),
                ("_foreach_add_List", lambda: torch._foreach_add_(pd, grads)),
                ("_foreach_mul_Scalar", lambda: torch._foreach_mul_(pd, 1.0))]
    raise SystemExit(f"--probe: unknown config {cfg}")


def probe(torch, cfg):
    """Kernel launches for counter collection: 3x abs.out over a 1 GiB f32
    buffer (reads 1 GiB, writes 1 GiB: the calibration of FETCH_SIZE and
    WRITE_SIZE), then each dominant aten call of the config 3 times, with a
    device synchronisation between calls."""
    cal = gen(torch, (1 << 28,), 42, torch.float32)
    cal_out = torch.empty_like(cal)
    for _ in range(PROBE_REPS):
        torch.ops.aten.abs.out(cal, out=cal_out)
    torch.supa.synchronize()
    del cal, cal_out
    ops = _probe_ops(torch, cfg)
    for name, fn in ops:
        for _ in range(PROBE_REPS):
            fn()
        torch.supa.synchronize()
        log(f"probe {cfg}: {name} x{PROBE_REPS}")
    print(json.dumps({"probe": cfg, "ops": [n for n, _ in ops], "reps": PROBE_REPS}))


# Algorithmic bytes per dispatch of each config's dominant kernels, keyed by
# substrings of the kernel name (the functor or kernel template).
PROBE_ALG_BYTES = {
    "c1": [("AddOp", 12 * C1_N), ("MulOp", 12 * C1_N), ("UnaryOpILi0EfE", 8 * C1_N), ("UnaryOpILi2EfE", 8 * C1_N),
           ("UnaryOp<0,", 8 * C1_N), ("UnaryOp<2,", 8 * C1_N)],
    "c2": [("AddOp", C2_ADD_BYTES), ("UnaryOp<1,", C2_GELU_BYTES), ("UnaryOpILi1EfE", C2_GELU_BYTES),
           ("k_transpose_vec", 4 * C2_N)],
    "c3": [("k_lsm_fwd_split", C3_BYTES["_log_softmax"]), ("k_nll_bwd", C3_BYTES["nll_loss_backward"]),
           ("k_lsm_bwd_split", C3_BYTES["_log_softmax_backward_data"])],
    "c4": [("MseOp", 12 * 32 * 1048576), ("BceBwdOp", 16 * 32 * 1048576 + 4 * 1048576)],
    # two k_adamw launches (40 + 32 tensors) per step: the average dispatch moves half of 28 P
    "c5": [("k_adamw", 14 * 1619066880)],
}


PROBE_NOTES = {
    "c1": "c1: [4096,4096] f32 add, mul, gelu('none'), silu (64 MiB operands; the probe runs one buffer set, "
          "so a repeat can hit the 256 MB MALL -- the bench rotates six sets)",
    "c2": "c2 contiguous: bf16 [64,2048,4096] + f32 bias -> f32, then gelu('tanh') over the f32 tensor; "
          "c2 transposed leg: `.contiguous()` of the bf16 [64,4096,2048] tensor's (1, 2) transpose",
    "c3": "c3: bf16 logits [8192,128256]: _log_softmax, nll_loss_forward, nll_loss_backward, "
          "_log_softmax_backward_data",
    "c4": "c4: [32,1048576] f32: mse 'none' and 'sum' forward, BCE-with-logits (pos_weight) 'none' forward "
          "and backward",
    "c5": "c5: AdamW(fused=True) step over the 72 tensors (1.62 G params), _foreach_add_.List, "
          "_foreach_mul_.Scalar",
}
CU_NUM = 256
ENGINE_GHZ = 2.4  # MI355X peak engine clock


def _fmt(v, nd=1):
    return "" if v is None else (f"{v:,.{nd}f}" if isinstance(v, float) else f"{v:,}")


def derive_counters(csvs, cfg, stats_csv=None):
    """Per-kernel averages of every counter in the given counter_collection.csv
    files (one file per rocprofv3 --pmc pass of --probe CFG).  FETCH_SIZE and
    WRITE_SIZE (KiB per dispatch) are scaled by known / measured for the
    calibration kernel (abs.out: 1 GiB read, 1 GiB written)."""
    import csv
    from collections import defaultdict

    vals = defaultdict(lambda: defaultdict(list))  # kernel -> counter -> values
    for path in csvs:
        with open(path) as f:
            for r in csv.DictReader(f):
                name = r["Kernel_Name"]
                vals[name][r["Counter_Name"]].append(float(r["Counter_Value"]))
    cal = [k for k in vals if "k_contig" in k and PROBE_CAL_KERNEL in k]
    if not cal:
        raise SystemExit("calibration dispatches (abs.out) missing")
    cal = cal[0]
    known_kib = float(1 << 20)
    scale = {}
    for c in ("FETCH_SIZE", "WRITE_SIZE"):
        if vals[cal].get(c):
            scale[c] = known_kib / (sum(vals[cal][c]) / len(vals[cal][c]))
    rows = []
    for name, cs in vals.items():
        if name == cal:
            continue
        row = {"kernel": name.split("(")[0].replace("void ", ""),
               "dispatches": max(len(v) for v in cs.values())}
        for c, v in sorted(cs.items()):
            row[c] = sum(v) / len(v)
        if "FETCH_SIZE" in scale and "FETCH_SIZE" in row:
            row["read_bytes"] = row["FETCH_SIZE"] * scale["FETCH_SIZE"] * 1024
        if "WRITE_SIZE" in scale and "WRITE_SIZE" in row:
            row["write_bytes"] = row["WRITE_SIZE"] * scale["WRITE_SIZE"] * 1024
        for sub, b in PROBE_ALG_BYTES.get(cfg, []):
            if sub in name:
                row["algorithmic_bytes"] = b
                break
        if "read_bytes" in row and "write_bytes" in row and row.get("algorithmic_bytes"):
            row["traffic_over_algorithmic"] = (row["read_bytes"] + row["write_bytes"]) / row["algorithmic_bytes"]
        rows.append(row)
    durations = {}
    if stats_csv:
        with open(stats_csv) as f:
            for r in csv.DictReader(f):
                durations[r["Name"].split("(")[0].replace("void ", "")] = (int(r["Calls"]), float(r["AverageNs"]))
    for row in rows:
        if row["kernel"] in durations:
            row["calls_traced"], row["avg_ns"] = durations[row["kernel"]]
            if row.get("algorithmic_bytes"):
                row["achieved_pct_of_8TBs"] = 100.0 * row["algorithmic_bytes"] / (row["avg_ns"] * 1e-9) / 8e12
        if row.get("SQ_WAVES"):
            row["valu_insts_per_wave"] = row.get("SQ_INSTS_VALU", 0.0) / row["SQ_WAVES"]
        if row.get("avg_ns"):
            # cycles of the traced kernel duration at the peak engine clock (a lower bound on busy
            # fractions when the clock runs below it)
            cyc = row["avg_ns"] * ENGINE_GHZ
            if "SQ_INSTS_VALU" in row:
                # wave64 VALU instructions issue in 4 cycles on a 16-lane SIMD (4 per CU); the f32
                # transcendentals are quarter rate
                issue = row["SQ_INSTS_VALU"] + 3.0 * row.get("SQ_INSTS_VALU_TRANS_F32", 0.0)
                row["valu_busy_pct"] = 100.0 * issue / CU_NUM / cyc
            if "SQ_WAVE_CYCLES" in row:
                row["waves_per_cu"] = 4.0 * row["SQ_WAVE_CYCLES"] / cyc / CU_NUM
            if "SQ_LDS_BANK_CONFLICT" in row:
                row["lds_bank_conflict_pct"] = 100.0 * row["SQ_LDS_BANK_CONFLICT"] / cyc / CU_NUM
    # this library's kernels (the probe's input generation runs torch's own HIP kernels)
    rows = [r for r in rows if r["kernel"].startswith("sa::")]
    rows.sort(key=lambda r: -(r.get("read_bytes", 0) + r.get("write_bytes", 0)))
    out = {"config": cfg, "calibration": "abs.out over 2^28 f32 (1 GiB read, 1 GiB written)",
           "scale": scale, "kernels": rows}
    base = os.path.join(HERE, "profiles", f"{cfg}_counters")
    with open(base + ".json", "w") as f:
        json.dump(out, f, indent=1)
        f.write("\n")
    # the commands that produced the inputs, from their paths
    cmds = []
    if stats_csv:
        cmds.append("rocprofv3 --kernel-trace --stats --output-format csv -d {} -o {} -- python3 bench.py --probe {}"
                    .format(*_run_args(stats_csv, "_kernel_stats.csv"), cfg))
    for path in csvs:
        cmds.append("rocprofv3 --pmc {} --output-format csv -d {} -o {} -- python3 bench.py --probe {}"
                    .format(" ".join(_counters_in(path)), *_run_args(path, "_counter_collection.csv"), cfg))
    cmds.append(f"python3 bench.py --derive-counters {' '.join(csvs)} --config {cfg}"
                + (f" --stats {stats_csv}" if stats_csv else ""))
    # the summary table
    lines = [f"# {cfg}: per-kernel counters (rocprofv3 on MI355X)", "", PROBE_NOTES.get(cfg, cfg) + ".", "",
             "Each dominant aten call runs 3 times after 3 calibration dispatches (`abs.out` over 2^28 f32: "
             "1 GiB read, 1 GiB written).  Commands (from the repository root, on the GPU box):", "", "```",
             "cd /tmp && export TMPDIR=/tmp && cd $GRAFT_REPO_ROOT",
             *cmds,
             "```", "",
             f"FETCH_SIZE scale {scale.get('FETCH_SIZE', 0):.5f}, WRITE_SIZE scale {scale.get('WRITE_SIZE', 0):.5f} "
             "(known bytes / counter for the calibration kernel).  Traffic = scaled FETCH + WRITE per dispatch.  "
             "Cycles = the traced average duration x 2.4 GHz (the peak engine clock, so the busy fractions are "
             "lower bounds).  VALU busy = 100 (SQ_INSTS_VALU + 3 SQ_INSTS_VALU_TRANS_F32) / CU_NUM / cycles "
             "(a wave64 VALU instruction issues in 4 cycles on one of a CU's 4 SIMDs; f32 transcendentals "
             "are quarter rate).  Waves per CU = 4 SQ_WAVE_CYCLES / cycles / CU_NUM (SQ_WAVE_CYCLES counts "
             "quad cycles; 32 waves fit a CU).  LDS bank conflicts = 100 SQ_LDS_BANK_CONFLICT / cycles / "
             "CU_NUM.  Only this library's kernels are listed (the probe's input generation runs torch's own "
             "HIP kernels).", "",
             "| kernel | avg us | algorithmic B | % of 8 TB/s | traffic B | traffic / alg | waves | VALU insts / wave "
             "| VALU busy % | waves / CU | LDS conflict % | transcendental f32 insts |",
             "|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for r in rows:
        tr = (r.get("read_bytes") or 0) + (r.get("write_bytes") or 0)
        lines.append("| `{}` | {} | {} | {} | {} | {} | {} | {} | {} | {} | {} | {} |".format(
            r["kernel"][:110], _fmt(r.get("avg_ns", 0) / 1e3 if r.get("avg_ns") else None),
            _fmt(r.get("algorithmic_bytes")), _fmt(r.get("achieved_pct_of_8TBs")), _fmt(int(tr)) if tr else "",
            _fmt(r.get("traffic_over_algorithmic"), 4), _fmt(int(r["SQ_WAVES"]) if r.get("SQ_WAVES") else None),
            _fmt(r.get("valu_insts_per_wave")), _fmt(r.get("valu_busy_pct")), _fmt(r.get("waves_per_cu")),
            _fmt(r.get("lds_bank_conflict_pct"), 3),
            _fmt(int(r["SQ_INSTS_VALU_TRANS_F32"]) if r.get("SQ_INSTS_VALU_TRANS_F32") is not None else None)))
    with open(base + ".md", "w") as f:
        f.write("\n".join(lines) + "\n")
    print(json.dumps(out))


def main():
    a = parse()
    if a.derive_traffic:
        derive_traffic(*a.derive_traffic)
        return
    if a.derive_counters:
        derive_counters(a.derive_counters, a.config, a.stats)
        return
    if a.render_kernel_stats:
        render_kernel_stats(*a.render_kernel_stats)
        return
    if a.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {a.gpus} is not supported "
              "(the path's multi-GPU sharding is a design, not a measured run)", file=sys.stderr)
        sys.exit(2)
    import torch
    import torch_supa  # noqa: F401
    import torch.nn.functional as F

    assert torch.supa.is_available(), "no supa device"
    timer = Timer(torch)
    if a.probe:
        probe(torch, a.probe)
        return
    configs = [c.strip() for c in a.configs.split(",") if c.strip()]
    per = {}

    # headline workload: c2 contiguous leg.  W untimed warm-up steps, then
    # HEADLINE_BATCHES batches of exactly K steps, each between two device
    # synchronisations and two HIP events on the supa stream; ms_per_step is
    # the median batch's time per step (the same figure as
    # per_config.c2_contiguous.step)
    log("c2: generating inputs")
    x, bias = c2_inputs(torch, transposed=False)
    for _ in range(a.warmup):
        F.gelu(x + bias, approximate="tanh")
    batch_ms = []
    for _ in range(HEADLINE_BATCHES):
        torch.supa.synchronize()
        e0, e1 = torch.supa.Event(), torch.supa.Event()
        e0.record()
        for _ in range(a.steps):
            F.gelu(x + bias, approximate="tanh")
        e1.record()
        e1.synchronize()
        torch.supa.synchronize()
        batch_ms.append(e0.elapsed_time(e1) / a.steps)
    ms_step = sorted(batch_ms)[len(batch_ms) // 2]
    step_bytes = C2_ADD_BYTES + C2_GELU_BYTES
    value = gbs(step_bytes, ms_step)
    # dominant kernel: gelu(tanh) over the f32 intermediate
    y = x + bias
    z = torch.empty_like(y)
    t_gelu = timer.time(lambda: torch.ops.aten.gelu.out(y, approximate="tanh", out=z), max(a.steps, 10))
    achieved = gbs(C2_GELU_BYTES, t_gelu)
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_GBS, 4), "traffic": traffic_from_profiles(),
                "kernel": "gelu(tanh) f32 [64,2048,4096] (k_contig)", "algorithmic_bytes": C2_GELU_BYTES,
                "avg_launch_ms": round(t_gelu, 5)}
    del y, z
    if "c2" in configs:
        per["c2_contiguous"] = bench_c2(torch, timer, x, bias, t_step=ms_step)
        del x, bias
        log("c2 transposed leg")
        xt, bt = c2_inputs(torch, transposed=True)
        per["c2_transposed"] = bench_c2(torch, timer, xt, bt)
        # .contiguous() of the transposed view (LDS-tiled transpose): 1 GiB read + 1 GiB written
        xc = torch.empty(xt.shape, dtype=xt.dtype, device="supa")
        per["c2_transposed"]["contiguous_copy"] = entry(2 * 2 * C2_N, timer.time(lambda: xc.copy_(xt), 10))
        del xc
        del xt, bt
    else:
        del x, bias
    torch.supa.empty_cache()
    if "c1" in configs:
        log("c1")
        per["c1"] = bench_c1(torch, timer)
        torch.supa.empty_cache()
    if "c3" in configs:
        log("c3")
        per["c3"] = bench_c3(torch, timer)
        torch.supa.empty_cache()
    if "c4" in configs:
        log("c4")
        per["c4"] = bench_c4(torch, timer)
        torch.supa.empty_cache()
    if "c5" in configs:
        log("c5")
        per["c5"] = bench_c5(torch, timer)
        torch.supa.empty_cache()
    fb = torch.supa.fallback_counts()

    cpu = None
    cpu_port = None
    if not a.no_cpu:
        log("cpu baselines")
        aten = cpu_aten_baselines(torch, configs)
        host = aten.pop("host")
        for k, v in aten.items():
            per.setdefault(k, {})["cpu_aten"] = v
        head = aten["c2_contiguous"]["step"]
        cpu = {"value": head["GB/s"], "unit": "GB/s", "cores": host["threads"], "kind": "reference",
               "sample": "upstream aten CPU kernels (torch " + host["torch"] + "), the reference outputs' "
                         "producer: c2 add + gelu(tanh) on " + head["sample"] + ", median of 3",
               "host": host}
        cpu_port = cpu_port_baseline()

    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16+f32 -> f32 (elementwise in f32)",
        "data": "synthetic: BASELINE config distributions drawn on the device by torch's seeded HIP generator",
        "config": {"workload": "c2 contiguous: add(x bf16 [64,2048,4096], bias f32 [4096]) -> f32, then "
                               "gelu(approximate='tanh'); one step = both aten ops",
                   "pct_roofline": round(100 * value / PEAK_GBS, 1), "parallelism": "none (1 GPU)"},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "cpu_port": cpu_port,
        "per_config": per,
        "cpu_fallback_ops": fb,
        "timing": TIMING,
        "host": platform.node(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
