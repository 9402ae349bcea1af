"""The reference's runtime tests for the allocator, device queries, copies,
seeding, streams and events (test/test_supa.py), case for case where this
build has the piece, through torch.supa (the reference runs them as
torch.cuda under its transfer_to_supa mode):

* test_memory_allocation (caching_allocator_alloc / _delete against
  memory_allocated), test_out_of_memory (its message and the 1 EB refusal;
  a later kernel still runs), test_out_of_memory_retry (a failed request
  succeeds once a live block is freed into the cache),
  test_set_per_process_memory_fraction and test_get_per_process_memory_fraction;
* test_supa_get_device_name / _capability / _properties_uuid;
* test_copy_non_blocking (pinned host memory both ways, and a pinned view
  whose data pointer is not its storage's), test_to_cpu_blocking_by_default;
* test_torch_manual_seed_seeds_cuda_devices, test_manual_seed;
* test_streams, test_events, test_generic_stream_event (torch.Stream /
  torch.Event on the supa device through the device guard).

Not mirrored: the reference's timing sleeps (torch.cuda._sleep is a kernel
of torch's own HIP runtime, outside the supa stream), the assertion that the
default stream is the legacy NULL stream (this build's default stream is a
created non-blocking stream, so it never serialises with other HIP code in
the process), the repr spellings, pinned-memory registration, memory
snapshots, pools, expandable segments and the cuBLAS / cuDNN flags, which
are not part of this path."""
import gc

import pytest
import torch

pytestmark = pytest.mark.gpu

SUPA = "supa"


def S():
    return torch.supa


def test_memory_allocation(no_fallback):
    gc.collect()
    S().empty_cache()
    prev = S().memory_allocated()
    mem = S().caching_allocator_alloc(1)
    try:
        assert S().memory_allocated() > prev
    finally:
        S().caching_allocator_delete(mem)
    assert S().memory_allocated() == prev


def test_get_device_name_capability_properties(no_fallback):
    cur = S().current_device()
    assert S().get_device_name(cur) == S().get_device_name(None) == S().get_device_name()
    assert S().get_device_capability(cur) == S().get_device_capability(None) == S().get_device_capability()
    props = S().get_device_properties(cur)
    assert props.total_memory > 0 and props.multi_processor_count > 0
    assert props.gcnArchName.startswith("gfx950")
    uuid = props.uuid
    assert len(uuid.bytes) == 16 and all(0 <= b <= 255 for b in uuid.bytes)
    u = str(uuid)
    assert len(u) == 36 and u[8] == u[13] == u[18] == u[23] == "-"


def test_out_of_memory(no_fallback):
    tensor = torch.zeros(1024, device=SUPA)
    with pytest.raises(RuntimeError, match="SUPA out of memory. Tried to allocate 800000000.00 GiB. GPU "):
        torch.empty(1024 * 1024 * 1024 * 800000000, dtype=torch.int8, device=SUPA)
    with pytest.raises(RuntimeError, match="Tried to allocate more than 1EB memory"):
        torch.empty(1024 * 1024 * 1024 * 8000000000, dtype=torch.int8, device=SUPA)
    tensor.fill_(1)
    assert bool((tensor == 1).all())


def test_out_of_memory_retry(no_fallback):
    S().empty_cache()
    total = S().get_device_properties(0).total_memory
    size = int(total * 0.5)
    a = torch.empty(size, dtype=torch.int8, device=SUPA)
    with pytest.raises(RuntimeError, match="Tried to allocate"):
        torch.empty(size, dtype=torch.int8, device=SUPA)
    del a
    b = torch.empty(size, dtype=torch.int8, device=SUPA)
    del b
    S().empty_cache()
    S().reset_peak_memory_stats()


def test_set_per_process_memory_fraction(no_fallback):
    try:
        with pytest.raises(TypeError, match="Invalid type"):
            S().set_per_process_memory_fraction(1)
        with pytest.raises(ValueError, match="Invalid fraction value"):
            S().set_per_process_memory_fraction(-0.1)
        with pytest.raises(ValueError, match="Invalid fraction value"):
            S().set_per_process_memory_fraction(2.0)
        tensor = torch.zeros(1024, device=SUPA)
        S().empty_cache()
        total = S().get_device_properties(0).total_memory
        S().set_per_process_memory_fraction(0.5, 0)
        application = int(total * 0.499) - S().max_memory_reserved()
        tmp = torch.empty(application, dtype=torch.int8, device=SUPA)
        del tmp
        S().empty_cache()
        with pytest.raises(RuntimeError, match="out of memory"):
            torch.empty(int(total * 0.5), dtype=torch.int8, device=SUPA)
        tensor.fill_(1)
        assert bool((tensor == 1).all())
    finally:
        S().set_per_process_memory_fraction(1.0, 0)


def test_get_per_process_memory_fraction(no_fallback):
    init = S().get_per_process_memory_fraction()
    S().set_per_process_memory_fraction(1.0)
    assert S().get_per_process_memory_fraction() == 1.0
    S().set_per_process_memory_fraction(0.0)
    assert S().get_per_process_memory_fraction() == 0.0
    for val in torch.rand(3, generator=torch.Generator().manual_seed(3)):
        S().set_per_process_memory_fraction(float(val))
        assert S().get_per_process_memory_fraction() == float(val)
    S().set_per_process_memory_fraction(init)


def _copy_non_blocking(a, b):
    ev = S().Event()
    a.copy_(b, non_blocking=True)
    ev.record()
    ev.synchronize()
    assert torch.equal(a.cpu(), b.cpu())


def test_copy_non_blocking(no_fallback):
    _copy_non_blocking(torch.ones(1000, dtype=torch.uint8).to(SUPA), torch.zeros(1000, dtype=torch.uint8).pin_memory())
    _copy_non_blocking(torch.zeros(1000, dtype=torch.uint8).pin_memory(), torch.ones(1000, dtype=torch.uint8).to(SUPA))
    x_base = torch.zeros(1000, dtype=torch.uint8).pin_memory()
    x = x_base[1:]
    assert x.is_pinned() and x_base.is_pinned()
    assert x_base.data_ptr() != x.data_ptr()
    _copy_non_blocking(x, torch.ones(999, dtype=torch.uint8).to(SUPA))


def test_to_cpu_blocking_by_default(no_fallback):
    src = torch.randn(1000, generator=torch.Generator().manual_seed(4)).to(SUPA)
    dst = src.to(device="cpu")
    assert S().current_stream().query()
    assert torch.equal(src.cpu(), dst)
    assert not dst.is_pinned()


def test_manual_seed_forms(no_fallback):
    x = torch.zeros(4, 4).float().to(SUPA)
    torch.manual_seed(2)
    assert S().initial_seed() == 2
    x.uniform_()
    torch.manual_seed(2)
    y = x.clone().uniform_()
    assert torch.equal(x.cpu(), y.cpu())
    S().manual_seed(2)
    assert S().initial_seed() == 2
    x.uniform_()
    a = torch.bernoulli(torch.full_like(x, 0.5))
    S().manual_seed(2)
    y = x.clone().uniform_()
    b = torch.bernoulli(torch.full_like(x, 0.5))
    assert torch.equal(x.cpu(), y.cpu()) and torch.equal(a.cpu(), b.cpu())


def test_streams(no_fallback):
    default_stream = S().current_stream()
    user_stream = S().Stream()
    assert S().current_stream() == default_stream
    assert default_stream != user_stream
    assert user_stream.hip_stream != 0
    with S().stream(user_stream):
        assert S().current_stream() == user_stream
    assert user_stream.query()
    tensor1 = torch.ByteTensor(5).pin_memory()
    tensor2 = tensor1.to(SUPA, non_blocking=True) + 1
    default_stream.synchronize()
    assert default_stream.query()
    assert torch.equal(tensor2.cpu(), tensor1 + 1)


def test_events(no_fallback):
    stream = S().current_stream()
    event = S().Event(enable_timing=True)
    assert event.query()
    start = S().Event(enable_timing=True)
    stream.record_event(start)
    x = torch.randn(1 << 24, device=SUPA)
    for _ in range(4):
        x = x * 1.0001 + 0.5
    stream.record_event(event)
    event.synchronize()
    assert event.query()
    assert start.elapsed_time(event) > 0


def test_all_any_and_bernoulli_tensor(no_fallback):
    """The two ops those cases call that sit beside the path: all() / any()
    (NaN is true, an empty tensor is all-true and not any, uint8 stays uint8)
    and bernoulli_ with a tensor of probabilities (p = 0 and 1 exact, p = 0.3
    within five standard deviations over 2^20 draws)."""
    x = torch.tensor([1.0, float("nan"), -2.0], device=SUPA)
    assert bool(x.all()) and bool(x.any())
    assert not bool(torch.tensor([1.0, 0.0], device=SUPA).all())
    assert not bool(torch.zeros(5, device=SUPA).any())
    e = torch.empty(0, device=SUPA)
    assert bool(e.all()) and not bool(e.any())
    u8 = torch.tensor([3, 0], dtype=torch.uint8, device=SUPA)
    assert u8.all().dtype == torch.uint8 and int(u8.any()) == 1
    p = torch.tensor([0.0, 1.0] * 4096, device=SUPA)
    assert torch.equal(torch.bernoulli(p).cpu(), p.cpu())
    n = 1 << 20
    m = float(torch.bernoulli(torch.full((n,), 0.3, device=SUPA)).mean())
    assert abs(m - 0.3) < 5 * (0.3 * 0.7 / n) ** 0.5


def test_generic_stream_event(no_fallback):
    """test_supa.py's test_generic_stream_event: torch.Stream / torch.Event on
    the supa device, through the device guard's stream and event methods."""
    stream = torch.Stream(SUPA)
    assert stream.device_index == S().current_device()
    s = S().Stream(stream_id=stream.stream_id, device_index=stream.device_index, device_type=stream.device_type)
    assert isinstance(s, torch.Stream) and torch.Stream in type(s).mro()
    assert stream.stream_id == s.stream_id
    assert stream.stream_id != S().current_stream().stream_id
    event1 = torch.Event(SUPA, enable_timing=True)
    event2 = torch.Event(SUPA, enable_timing=True)
    a = torch.randn(1000, generator=torch.Generator().manual_seed(5))
    b = torch.randn(1000, generator=torch.Generator().manual_seed(6))
    with S().stream(s):
        a_s = a.to(SUPA, non_blocking=True)
        b_s = b.to(SUPA, non_blocking=True)
        assert stream.stream_id == S().current_stream().stream_id
    event1.record(stream)
    event1.synchronize()
    assert event1.query()
    c = a_s + b_s
    event2.record()
    event2.synchronize()
    assert event2.query()
    assert torch.equal(c.cpu(), a + b)
    assert event1.elapsed_time(event2) >= 0
