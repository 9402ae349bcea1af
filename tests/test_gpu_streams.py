"""Streams, events and the stream-aware caching allocator on the supa device
(the reference's SUPAStream.cpp:26-27,147 pool and thread-local current
stream; RecordStream.cpp:10-16 record_stream):

* the default stream is a non-blocking stream, not the legacy NULL stream;
  Stream() hands out the pool round-robin; ``with torch.supa.stream(s)`` and
  ``with s`` switch the thread's current stream and restore it;
* kernels run on the current stream: work split over two streams with an
  event between producer and consumer gives the serial result;
* a freed block is reused by the next allocation on its own stream, never by
  one on another stream; after record_stream its reuse waits until the other
  stream has finished the work queued before the free;
* allocator OOM: one injected hipMalloc failure is retried after releasing
  the cache; two raise torch.OutOfMemoryError, and the allocator keeps working.
"""
import threading

import numpy as np
import pytest
import torch

import oracle as O

pytestmark = pytest.mark.gpu


def test_default_stream_is_non_blocking_and_pool_round_robin(supa):
    d = torch.supa.default_stream()
    assert d.stream_id == 0 and d.hip_stream != 0  # not the legacy NULL stream
    assert torch.supa.current_stream() == d
    ids = {torch.supa.Stream().stream_id for _ in range(64)}
    assert ids == set(range(1, 33))
    s = torch.supa.Stream()
    assert s.device.type == "supa" and s.device_index == 0
    with torch.supa.stream(s):
        assert torch.supa.current_stream() == s
        s2 = torch.supa.Stream()
        with s2:
            assert torch.supa.current_stream() == s2
        assert torch.supa.current_stream() == s
    assert torch.supa.current_stream() == d


def test_current_stream_is_thread_local(supa):
    s = torch.supa.Stream()
    seen = {}

    def worker():
        seen["other"] = torch.supa.current_stream().stream_id

    with torch.supa.stream(s):
        t = threading.Thread(target=worker)
        t.start()
        t.join()
        assert torch.supa.current_stream() == s
    assert seen["other"] == 0


def test_two_streams_with_events_match_serial(no_fallback):
    g = torch.Generator().manual_seed(3)
    a = torch.randn(4096, 4096, generator=g)
    b = torch.randn(4096, 4096, generator=g)
    da, db = a.to("supa"), b.to("supa")
    s1, s2 = torch.supa.Stream(), torch.supa.Stream()
    while s2.stream_id == s1.stream_id:
        s2 = torch.supa.Stream()
    s1.wait_stream(torch.supa.current_stream())
    s2.wait_stream(torch.supa.current_stream())
    with torch.supa.stream(s1):
        x = torch.nn.functional.gelu(da, approximate="tanh")
        for _ in range(8):
            x = x * 1.0001
    with torch.supa.stream(s2):
        y = da + db
    ev = s1.record_event()
    s2.wait_event(ev)
    with torch.supa.stream(s2):
        z = x * y
    torch.supa.current_stream().wait_stream(s2)
    x0 = torch.nn.functional.gelu(da, approximate="tanh").cpu().numpy()  # default stream, same kernel
    assert O.gelu_tanh_forward_equal(x0, a.numpy())
    ref_x = x0
    for _ in range(8):
        ref_x = O.binary(O.MUL, ref_x, np.float32(1.0001))
    ref = O.binary(O.MUL, ref_x, O.binary(O.ADD, a.numpy(), b.numpy()))
    assert np.array_equal(z.cpu().numpy(), ref)


def _busy(s, x, n=200):
    """Queue about a few milliseconds of work on stream s."""
    with torch.supa.stream(s):
        y = x
        for _ in range(n):
            y = torch.nn.functional.gelu(y, approximate="tanh")
    return y


def test_allocator_reuse_is_per_stream(supa):
    torch.supa.synchronize()
    torch.supa.empty_cache()  # no other cached block of this size class
    n = (1 << 20) + 7919
    x = torch.empty(n, device="supa")
    p = x.data_ptr()
    del x
    s = torch.supa.Stream()
    with torch.supa.stream(s):
        y = torch.empty(n, device="supa")
    assert y.data_ptr() != p  # another stream never takes the block
    z = torch.empty(n, device="supa")
    assert z.data_ptr() == p  # its own stream does, at once
    del y, z
    torch.supa.synchronize()


def test_record_stream_defers_reuse(supa):
    torch.supa.synchronize()
    torch.supa.empty_cache()  # no other cached block of this size class
    m = (1 << 22) + 7919
    s = torch.supa.Stream()
    big = torch.randn(1 << 24).to("supa")
    x = torch.ones(m, device="supa")
    p = x.data_ptr()
    s.wait_stream(torch.supa.current_stream())  # s reads x and big after they are written
    keep = _busy(s, big)  # s is busy for a while
    with torch.supa.stream(s):
        y = x * 2  # s reads x after the busy work
    x.record_stream(s)
    del x
    assert torch.supa.memory_stats()["pending_blocks"] >= 1
    busy_before = not s.query()
    w = torch.empty(m, device="supa")
    busy_after = not s.query()
    assert busy_before  # milliseconds of queued work: s cannot have drained yet
    reused = w.data_ptr() == p
    if busy_after:  # s busy throughout the allocation: its event had not completed
        assert not reused
    s.synchronize()
    if reused:  # s drained before the allocation looked: w holds the block; give it back
        w = None
    w2 = torch.empty(m, device="supa")
    assert w2.data_ptr() == p  # s's event completed: the block is back
    assert torch.equal(y.cpu(), torch.full((m,), 2.0))
    del keep, w, w2, y
    torch.supa.synchronize()


def test_injected_oom_is_retried_then_raised(supa):
    from torch_supa import _C
    torch.supa.synchronize()
    torch.supa.empty_cache()  # every allocation below reaches hipMalloc
    before = torch.supa.memory_stats()["num_ooms_retried"]
    try:
        _C.inject_oom(1)
        t = torch.zeros(3 << 20, device="supa")
        assert torch.supa.memory_stats()["num_ooms_retried"] == before + 1
        assert float(t.sum()) == 0.0
        _C.inject_oom(2)
        with pytest.raises(torch.OutOfMemoryError):
            torch.empty(5 << 20, device="supa")
        assert torch.supa.memory_stats()["num_ooms_retried"] == before + 2
    finally:
        _C.inject_oom(0)
    u = torch.ones(5 << 20, device="supa")  # the allocator still works
    assert float(u.sum()) == float(5 << 20)


def test_index_errors_are_reported_per_stream(supa):
    """A bad nll target on a side stream sets that stream's error flag: a
    read on the default stream (which did not wait for it) does not report
    it; a read on the side stream after it synchronises does, once."""
    import torch.nn.functional as F
    torch.supa.synchronize()
    g = torch.Generator().manual_seed(5)
    lp = torch.log_softmax(torch.randn(8, 10, generator=g), 1).to("supa")
    bad = torch.tensor([0, 1, 2, 3, 4, 5, 6, 12]).to("supa")
    good = torch.zeros(8, dtype=torch.int64).to("supa")
    s = torch.supa.Stream()
    s.wait_stream(torch.supa.current_stream())
    with torch.supa.stream(s):
        loss_bad = F.nll_loss(lp, bad)
    s.synchronize()
    # the default stream's own work reads clean
    assert F.nll_loss(lp, good).item() == pytest.approx(-lp[:, 0].mean().item(), rel=1e-6)
    with torch.supa.stream(s):
        with pytest.raises(IndexError):
            loss_bad.item()
        assert F.nll_loss(lp, good).item() == pytest.approx(-lp[:, 0].mean().item(), rel=1e-6)  # cleared
    # torch.supa.synchronize() reads every stream's flag
    with torch.supa.stream(s):
        F.nll_loss(lp, bad)
    with pytest.raises(IndexError):
        torch.supa.synchronize()
    torch.supa.synchronize()  # cleared
