"""Block mappings of the streaming kernels: the contiguous kernel (one
wavefront per workgroup, one vector per thread, an element tail in the last
workgroup) on a whole tensor against the same op over slices of it, and the
row-broadcast kernel's row pairing (a thread's two rows K apart) over row
counts that leave a tile part-filled.  Each result is compared bit for bit
with the same op computed over other launch shapes or by the upstream CPU
kernels, and a slice with the oracle."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

import oracle as O

pytestmark = pytest.mark.gpu

def chunked(fn, xs, pieces=8):
    """fn over `pieces` slices (other grids, other tails), rejoined."""
    n = xs[0].numel()
    step = ((n // pieces) // 64) * 64  # 64-element steps keep every slice 16-byte aligned
    outs, s = [], 0
    while s < n:
        e = min(n, s + step) if len(outs) < pieces - 1 else n
        outs.append(fn(*[x[s:e] for x in xs]))
        s = e
    return torch.cat(outs)


@pytest.mark.parametrize("dtype,vec", [(torch.float32, 4), (torch.bfloat16, 8)])
@pytest.mark.parametrize("approx", ["none", "tanh"])
def test_contiguous_gelu_whole_and_sliced(approx, dtype, vec, no_fallback):
    n = (1 << 22) * vec + 1000 * vec + 3  # a partial last workgroup and an element tail
    g = torch.Generator().manual_seed(60)
    x = (torch.randn(n, generator=g) * 3).to(dtype).to("supa")
    gy = torch.randn(n, generator=g).to(dtype).to("supa")
    y = F.gelu(x, approximate=approx)
    assert torch.equal(y.cpu(), chunked(lambda t: F.gelu(t, approximate=approx), [x]).cpu())
    gx = torch.ops.aten.gelu_backward(gy, x, approximate=approx)
    want_gx = chunked(lambda a, b: torch.ops.aten.gelu_backward(a, b, approximate=approx), [gy, x])
    assert torch.equal(gx.cpu(), want_gx.cpu())
    # head and tail against the oracle
    k = O.GELU if approx == "none" else O.GELU_TANH
    for sl in (slice(0, 4096), slice(n - 4099, n)):
        xs = x[sl].float().cpu().numpy()
        want = torch.from_numpy(O.unary(k, xs)).to(dtype)
        if approx == "tanh":  # the forward's tanh may be the other neighbour near a rounding boundary
            alt = torch.from_numpy(O.unary(O.GELU_TANH_FAST_ALT, xs)).to(dtype)
            assert bool(((y[sl].cpu() == want) | (y[sl].cpu() == alt)).all())
            continue
        assert torch.equal(y[sl].cpu(), want)


@pytest.mark.parametrize("rows,cols", [(5, 64), (9, 1024), (13, 2048), (33, 256), (67, 520), (130, 4096)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_row_pairing_part_tiles(rows, cols, dtype, no_fallback):
    """Row counts that are not multiples of the pairing tile (2K rows) for
    row, column and middle-dim broadcasts; bf16 outputs halve the row bytes
    and double K."""
    g = torch.Generator().manual_seed(61)
    x = torch.randn(rows, cols, generator=g).to(dtype)
    rowv = torch.randn(cols, generator=g).to(dtype)
    colv = torch.randn(rows, 1, generator=g).to(dtype)
    dx = x.to("supa")
    assert torch.equal((dx + rowv.to("supa")).cpu(), x + rowv)
    assert torch.equal((dx * colv.to("supa")).cpu(), x * colv)
    x3 = torch.randn(3, rows, cols, generator=g).to(dtype)
    assert torch.equal((x3.to("supa") - colv.to("supa")).cpu(), x3 - colv)  # per-(row) channel: MID
    xb = torch.randn(rows, cols, generator=g).to(torch.bfloat16)
    rowf = torch.randn(cols, generator=g)
    assert torch.equal((xb.to("supa") + rowf.to("supa")).cpu(), xb + rowf)  # bf16 + f32 -> f32
