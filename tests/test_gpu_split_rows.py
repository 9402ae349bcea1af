"""Rows split over several workgroups: log_softmax backward and log_softmax
/ softmax forward rows of 2 to 32 parts (at most 2048 16-byte vectors a
backward part, 2560 a forward part; a row spread evenly over its parts,
rounded up to whole wavefronts, but for backward rows of 6 or more parts,
which take full parts and a short last one).  The parts of a row exchange
their row partials through a per-stream buffer; a part that finds a peer's
slot still empty after its spin limit computes that peer's partial itself.

Covered here: parity with the oracle on rows that split and rows that do not
(one part: the one-row kernel; past the 32-part limit: the streaming
kernel), even and ragged parts,
the fallback (SUPA_AMD_ROW_SPLIT_SPIN=0: a part never waits) bit-identical to
the normal path, the path switched off (SUPA_AMD_ROW_SPLIT=0), launches
chunked over many rows, an in-place backward (never split), rows holding
+-inf and NaN, a graph capture (never split), two streams at once (a slot
buffer each) and more streams than a device has slot buffers (the rest run
the one-row kernel)."""
import numpy as np
import pytest
import torch

import oracle as O
from helpers import bf16_ulp_dist

pytestmark = pytest.mark.gpu

LSM_BWD = torch.ops.aten._log_softmax_backward_data


def seeded(shape, seed, scale=1.0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(dtype)


def bits16(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16)


def round16(a, dtype):
    """float32 array rounded to dtype (round to nearest even), as 16-bit patterns."""
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(dtype)
    return t.view(torch.int16).numpy().view(np.uint16)


def assert_close16(got, ref, dtype):
    """<= 1 ulp of dtype, NaN where the reference is NaN."""
    r = np.asarray(ref, np.float32)
    gf = got.cpu().float().numpy()
    assert np.array_equal(np.isnan(gf), np.isnan(r))
    fin = ~np.isnan(r)
    assert bf16_ulp_dist(bits16(got)[fin], round16(r, dtype)[fin]).max(initial=0) <= 1


def bwd_inputs(rows, cols, dtype, seed):
    x = seeded((rows, cols), seed, 2.0)
    y = O.log_softmax(x.numpy())
    g = seeded((rows, cols), seed + 1, 1.0)
    yd = torch.from_numpy(y).to(dtype)
    gd = g.to(dtype)
    return gd, yd


# cols -> backward parts of at most 2048 16-byte vectors (bf16 / f16: 8 elements a vector, float32 4):
# 16392 bf16 (2049 vectors, the fewest that split) splits in 2 parts of 1088, 40000 bf16 (5000 vectors) in 3
# of 1728, 65600 bf16 in 5 of 1664, 128264 bf16 in 7 full parts and one of 1697, 524288 bf16 in 32;
# 524296 bf16 and 524288 float32 stream
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("cols", [16392, 40000, 65600, 128256, 128264, 262144, 524288, 524296])
def test_log_softmax_backward_split_matches_oracle(dtype, cols, no_fallback):
    rows = 3 if cols > 200000 else 6
    g, y = bwd_inputs(rows, cols, dtype, 31)
    out = LSM_BWD(g.to("supa"), y.to("supa"), 1, dtype)
    ref = O.log_softmax_backward(g.float().numpy(), y.float().numpy())
    if dtype == torch.float32:
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-6)
    else:
        assert_close16(out, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
# cols -> forward parts of at most 2560 vectors: 20480 bf16 (2560 vectors) is one part (the one-row
# kernel), 20488 bf16 (the fewest that split) splits in 2 parts of 1344, 28664 bf16 in 2 of 1792, 65544
# bf16 in 4 of 2112 (the last 1857), 655360 bf16 in 32 full parts; 655368 bf16 and every float32 row past
# 327680 stream
@pytest.mark.parametrize("cols", [20480, 20488, 28664, 32000, 50304, 65536, 65544, 131080, 200000, 262144, 524288,
                                  655360, 655368])
def test_log_softmax_forward_split_matches_oracle(dtype, cols, no_fallback):
    x = seeded((3, cols), 41, 2.0, dtype)
    out = torch.log_softmax(x.to("supa"), dim=1)
    ref = O.log_softmax(x.float().numpy())
    if dtype == torch.float32:
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-5)
    else:
        assert_close16(out, ref, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_softmax_forward_split_matches_oracle(dtype, no_fallback):
    cols = 140000 if dtype == torch.bfloat16 else 128256
    x = seeded((4, cols), 43, 2.0, dtype)
    out = torch.softmax(x.to("supa"), dim=1)
    ref = O.softmax(x.float().numpy())
    if dtype == torch.float32:
        np.testing.assert_allclose(out.cpu().numpy(), ref, rtol=1e-5, atol=1e-9)
    else:
        assert_close16(out, ref, dtype)


@pytest.mark.parametrize("dtype,cols", [(torch.bfloat16, 128256), (torch.bfloat16, 50304), (torch.float32, 28672)])
def test_split_fallback_is_bit_identical(dtype, cols, no_fallback, monkeypatch):
    """With a spin limit of 0 a part never waits: every partial it finds
    unpublished it computes from the peer's data, in the peer's order (128256
    bf16: 8 full backward parts, 7 even forward parts of 2304 vectors; 50304
    bf16: 4 even backward parts of 1600, 3 forward parts of 2112; 28672
    float32: 4 backward parts of 1792, 3 forward parts of 2432)."""
    g, y = bwd_inputs(64, cols, dtype, 51)
    gd, yd = g.to("supa"), y.to("supa")
    xf = seeded((64, cols), 52, 2.0, dtype).to("supa")
    ref_b = LSM_BWD(gd, yd, 1, dtype)
    ref_f = torch.log_softmax(xf, dim=1)
    torch.supa.synchronize()
    monkeypatch.setenv("SUPA_AMD_ROW_SPLIT_SPIN", "0")
    for _ in range(3):
        assert torch.equal(LSM_BWD(gd, yd, 1, dtype).cpu(), ref_b.cpu())
        assert torch.equal(torch.log_softmax(xf, dim=1).cpu(), ref_f.cpu())


def test_split_switched_off_agrees(no_fallback, monkeypatch):
    """SUPA_AMD_ROW_SPLIT=0: the one-row backward; the two reduce the row sum
    in different orders, so they agree to 1 bf16 ulp."""
    g, y = bwd_inputs(16, 128256, torch.bfloat16, 61)
    gd, yd = g.to("supa"), y.to("supa")
    on = LSM_BWD(gd, yd, 1, torch.bfloat16)
    monkeypatch.setenv("SUPA_AMD_ROW_SPLIT", "0")
    off = LSM_BWD(gd, yd, 1, torch.bfloat16)
    assert bf16_ulp_dist(bits16(on), bits16(off)).max() <= 1


def test_split_many_rows_chunked(no_fallback):
    """32 parts a row: 2048 rows a launch, so 4100 rows take three launches
    that reuse the buffer; each row matches the same row computed alone."""
    rows, cols = 4100, 524288
    gen = torch.Generator().manual_seed(71)
    # per-row scaled copies of one random grad row keep the host side small;
    # every row's output is the same log-softmax row
    base_g = torch.randn(1, cols, generator=gen)
    base_y = torch.from_numpy(O.log_softmax((torch.randn(1, cols, generator=gen) * 2.0).numpy()))
    k = torch.arange(rows, dtype=torch.float32)[:, None]
    gd = (base_g.to("supa") * (1.0 + k.to("supa") / rows)).to(torch.bfloat16)
    yd = base_y.to(torch.bfloat16).to("supa").expand(rows, cols).contiguous()
    full = LSM_BWD(gd, yd, 1, torch.bfloat16)
    for lo, hi in ((0, 3), (2046, 2050), (4094, 4100)):
        part = LSM_BWD(gd[lo:hi].contiguous(), yd[lo:hi].contiguous(), 1, torch.bfloat16)
        assert torch.equal(full[lo:hi].cpu(), part.cpu()), (lo, hi)
    ref = O.log_softmax_backward(gd[4097:4100].float().cpu().numpy(), yd[4097:4100].float().cpu().numpy())
    assert_close16(full[4097:4100], ref, torch.bfloat16)
    del full, gd, yd


def test_split_backward_in_place(no_fallback):
    """grad_input written over grad: the host sees the overlap and keeps the
    one-row kernel (a split part may read a peer's grad)."""
    g, y = bwd_inputs(8, 128256, torch.bfloat16, 81)
    gd, yd = g.to("supa"), y.to("supa")
    ref = LSM_BWD(gd, yd, 1, torch.bfloat16)
    LSM_BWD.out(gd, yd, 1, torch.bfloat16, out=gd)
    assert bf16_ulp_dist(bits16(gd), bits16(ref)).max() <= 1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_split_forward_special_values(dtype, no_fallback):
    """+inf (in a bf16 word's high element next to a nonzero low one, and in a
    low element), -inf, an all -inf row, NaN and a dominant element (a tiny
    log-sum) against the oracle, NaN for NaN."""
    cols = 200000 if dtype != torch.float32 else 140000
    x = seeded((8, cols), 91, 2.0)
    x[0, 1001] = float("inf")
    x[0, 1000] = 1.5
    x[1, 70000] = float("inf")
    x[2, ::7] = float("-inf")
    x[3, :] = float("-inf")
    x[4, 12345] = float("nan")
    x[5, 99] = 60.0
    x[6, -1] = float("inf")
    x = x.to(dtype)
    out = torch.log_softmax(x.to("supa"), dim=1)
    ref = O.log_softmax(x.float().numpy())
    if dtype == torch.float32:
        o = out.cpu().numpy()
        assert np.array_equal(np.isnan(o), np.isnan(ref))
        fin = ~np.isnan(ref)
        np.testing.assert_allclose(o[fin], ref[fin], rtol=1e-5, atol=1e-5)
    else:
        assert_close16(out, ref, dtype)
    cpu = torch.log_softmax(x.float(), dim=1).numpy()
    assert np.array_equal(np.isnan(cpu), np.isnan(out.cpu().float().numpy()))


def test_backward_under_graph_capture():
    """A stream that is capturing a graph never takes the split kernels (their
    slot buffer is made with hipMalloc on a stream's first use, and the
    per-launch state must not be replayed blindly): the captured launch is the
    one-row kernel's, and every replay equals the eager result to 1 bf16 ulp.
    Called through the C ABI on torch's own HIP stream."""
    import ctypes

    import capi as A

    L = A.lib()
    rows, cols = 8, 128256
    g, y = bwd_inputs(rows, cols, torch.bfloat16, 101)
    dg, dy = g.to("cuda"), y.to("cuda")
    eager = torch.empty_like(dg)
    code = A.dtype_code(torch.bfloat16)
    assert L.supa_amd_log_softmax_backward(dg.data_ptr(), dy.data_ptr(), code, eager.data_ptr(), code, rows, cols,
                                           None) == 0
    torch.cuda.synchronize()
    out = torch.empty_like(dg)
    s = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        graph.capture_begin()
        rc = L.supa_amd_log_softmax_backward(dg.data_ptr(), dy.data_ptr(), code, out.data_ptr(), code, rows, cols,
                                             ctypes.c_void_p(s.cuda_stream))
        graph.capture_end()
    assert rc == 0
    for _ in range(3):
        out.fill_(0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert bf16_ulp_dist(bits16(out), bits16(eager)).max() <= 1
        assert not torch.equal(out, torch.zeros_like(out))


def test_split_on_two_streams(no_fallback):
    """Split launches on two streams at once keep their own slot buffers: each
    stream's results equal the same call's on the default stream bit for bit
    (a shared buffer would mix the two launches' row partials)."""
    data = [bwd_inputs(64, 128256, torch.bfloat16, seed) for seed in (111, 113)]
    data = [(g.to("supa"), y.to("supa")) for g, y in data]
    ref = [LSM_BWD(g, y, 1, torch.bfloat16).cpu() for g, y in data]
    s1, s2 = torch.supa.Stream(), torch.supa.Stream()
    while s2.stream_id == s1.stream_id:
        s2 = torch.supa.Stream()
    cur = torch.supa.current_stream()
    s1.wait_stream(cur)
    s2.wait_stream(cur)
    outs = []
    for _ in range(4):
        with torch.supa.stream(s1):
            o1 = LSM_BWD(data[0][0], data[0][1], 1, torch.bfloat16)
        with torch.supa.stream(s2):
            o2 = LSM_BWD(data[1][0], data[1][1], 1, torch.bfloat16)
        outs.append((o1, o2))
    cur.wait_stream(s1)
    cur.wait_stream(s2)
    for o1, o2 in outs:
        assert torch.equal(o1.cpu(), ref[0])
        assert torch.equal(o2.cpu(), ref[1])


def test_split_buffers_run_out(no_fallback, monkeypatch):
    """A device gives out 8 slot buffers; a stream after that takes the
    unsplit kernel.  Each of 16 streams gives exactly the split result or
    exactly the unsplit one (float32 outputs, where the two kernels' row sums,
    added in different orders, show)."""
    g, y = bwd_inputs(16, 128256, torch.float32, 121)
    gd, yd = g.to("supa"), y.to("supa")
    split = LSM_BWD(gd, yd, 1, torch.float32).cpu()
    monkeypatch.setenv("SUPA_AMD_ROW_SPLIT", "0")
    one_row = LSM_BWD(gd, yd, 1, torch.float32).cpu()
    monkeypatch.delenv("SUPA_AMD_ROW_SPLIT")
    assert not torch.equal(split, one_row)
    cur = torch.supa.current_stream()
    streams = {}
    while len(streams) < 16:
        s = torch.supa.Stream()
        streams[s.stream_id] = s
    kinds = []
    for s in streams.values():
        s.wait_stream(cur)
        with torch.supa.stream(s):
            o = LSM_BWD(gd, yd, 1, torch.float32)
        cur.wait_stream(s)
        o = o.cpu()
        kinds.append("split" if torch.equal(o, split) else ("one_row" if torch.equal(o, one_row) else "other"))
    assert "other" not in kinds
    assert "one_row" in kinds  # at most 7 of these streams (the default stream has one) got a buffer


def test_split_mixed_dtypes(no_fallback):
    """bf16 rows with float32 results (half_to_float forward; a float32
    grad_input from bf16 grad and output) through the split kernels."""
    x = seeded((4, 128256), 131, 2.0, torch.bfloat16)
    out = torch.ops.aten._log_softmax(x.to("supa"), 1, True)
    assert out.dtype == torch.float32
    np.testing.assert_allclose(out.cpu().numpy(), O.log_softmax(x.float().numpy()), rtol=1e-5, atol=1e-5)
    sm = torch.ops.aten._softmax(x.to("supa"), 1, True)
    np.testing.assert_allclose(sm.cpu().numpy(), O.softmax(x.float().numpy()), rtol=1e-5, atol=1e-9)
    g, y = bwd_inputs(4, 128256, torch.bfloat16, 133)
    gi = LSM_BWD(g.to("supa"), y.to("supa"), 1, torch.float32)
    assert gi.dtype == torch.float32
    ref = O.log_softmax_backward(g.float().numpy(), y.float().numpy())
    np.testing.assert_allclose(gi.cpu().numpy(), ref, rtol=1e-5, atol=1e-6)
