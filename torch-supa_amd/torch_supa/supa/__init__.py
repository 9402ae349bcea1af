"""``torch.supa``: device module of the supa (MI355X) backend.

The subset of the reference's ``torch.supa`` (``torch_supa/supa/*.py``,
``csrc/supa/Module.cpp:1133-1162``) that the elementwise + loss path and its
harnesses use: device queries, synchronisation, streams (a pool of 32 per
device, a thread-local current stream) and events, allocator statistics, the
device generator's seeding API, and the switches of the opt-in kernels and of
the CPU fallback.
"""
from __future__ import annotations

import torch

from .. import _C


def is_available() -> bool:
    return _C.device_count() > 0


def device_count() -> int:
    return _C.device_count()


def current_device() -> int:
    return _C.current_device()


def set_device(device) -> None:
    idx = _index(device)
    if idx is not None:
        _C.set_device(idx)


def _index(device):
    if device is None:
        return None
    if isinstance(device, int):
        return device
    device = torch.device(device)
    return device.index if device.index is not None else _C.current_device()


def synchronize(device=None) -> None:
    _C.synchronize(_index(device) if device is not None else _C.current_device())


def is_initialized() -> bool:
    return True


def _is_in_bad_fork() -> bool:
    return False


def _lazy_init() -> None:
    return None


def get_amp_supported_dtype():
    return [torch.float16, torch.bfloat16]


def memory_stats(device=None) -> dict:
    return _C.memory_stats(_index(device) if device is not None else _C.current_device())


def memory_allocated(device=None) -> int:
    return memory_stats(device)["allocated_bytes"]


def max_memory_allocated(device=None) -> int:
    return memory_stats(device)["peak_allocated_bytes"]


def memory_reserved(device=None) -> int:
    return memory_stats(device)["reserved_bytes"]


def reset_peak_memory_stats(device=None) -> None:
    _C.reset_peak_memory_stats(_index(device) if device is not None else _C.current_device())


def empty_cache() -> None:
    _C.empty_cache()


def max_memory_reserved(device=None) -> int:
    return memory_stats(device)["peak_reserved_bytes"]


def mem_get_info(device=None):
    """(free, total) device memory in bytes."""
    return _C.mem_get_info(_index(device) if device is not None else _C.current_device())


# The reference's allocator API (torch_supa/supa/memory.py:79-180): raw blocks
# of the caching allocator for other frameworks, and a per-process cap on the
# memory it reserves.
def caching_allocator_alloc(size, device=None, stream=None) -> int:
    """A block of `size` bytes from the caching allocator for `stream` (a
    torch.supa.Stream or a hipStream_t as an int; the device's current stream
    by default); returns its address.  Release it with
    caching_allocator_delete."""
    idx = _index(device) if device is not None else _C.current_device()
    if stream is None:
        stream = current_stream(idx)
    if isinstance(stream, Stream):
        stream = stream.hip_stream
    if not isinstance(stream, int):
        raise TypeError("Invalid type for stream argument, must be `torch.supa.Stream` or `int` representing a "
                        "pointer to a existing stream")
    return _C.raw_alloc(int(size), idx, stream)


def caching_allocator_delete(mem_ptr: int) -> None:
    _C.raw_delete(int(mem_ptr))


def set_per_process_memory_fraction(fraction, device=None) -> None:
    """Cap the memory the caching allocator reserves on `device` at
    fraction x its total memory; a request beyond the cap (after releasing
    the cache) raises an out-of-memory error."""
    idx = _index(device) if device is not None else _C.current_device()
    if not isinstance(fraction, float):
        raise TypeError("Invalid type for fraction argument, must be `float`")
    if fraction < 0 or fraction > 1:
        raise ValueError(f"Invalid fraction value: {fraction}. Allowed range: 0~1")
    _C.set_memory_fraction(fraction, idx)


def get_per_process_memory_fraction(device=None) -> float:
    return _C.get_memory_fraction(_index(device) if device is not None else _C.current_device())


class _UUID:
    """A device UUID: 16 bytes, printed as 8-4-4-4-12 hex digits."""

    def __init__(self, raw: bytes):
        self.bytes = bytes(raw)

    def __str__(self):
        h = self.bytes.hex()
        return f"{h[:8]}-{h[8:12]}-{h[12:16]}-{h[16:20]}-{h[20:]}"

    __repr__ = __str__


class _DeviceProperties:
    """hipGetDeviceProperties' fields: name, total_memory, major, minor,
    multi_processor_count, gcnArchName, L2_cache_size, uuid."""

    def __init__(self, d: dict):
        self.name = d["name"]
        self.total_memory = d["total_memory"]
        self.major = d["major"]
        self.minor = d["minor"]
        self.multi_processor_count = d["multi_processor_count"]
        self.gcnArchName = d["gcn_arch_name"]
        self.L2_cache_size = d["l2_cache_size"]
        self.uuid = _UUID(d["uuid"])

    def __repr__(self):
        return (f"_SupaDeviceProperties(name='{self.name}', major={self.major}, minor={self.minor}, "
                f"gcnArchName='{self.gcnArchName}', total_memory={self.total_memory // (1 << 20)}MB, "
                f"multi_processor_count={self.multi_processor_count}, uuid={self.uuid})")


def get_device_properties(device=None) -> _DeviceProperties:
    return _DeviceProperties(_C.device_properties(_index(device) if device is not None else _C.current_device()))


def get_device_name(device=None) -> str:
    return get_device_properties(device).name


def get_device_capability(device=None):
    p = get_device_properties(device)
    return p.major, p.minor


# Each supa device has a default Philox generator (seed + call offset) that
# the native random ops (uniform_, bernoulli_, dropout) draw from.
# torch.manual_seed reaches manual_seed_all through the PrivateUse1 module
# hooks (it checks _is_in_bad_fork, then calls manual_seed_all).  Same API as
# the reference's torch_supa/supa/random.py:26-172.
def manual_seed(seed: int) -> None:
    _C.rng_manual_seed(_C.current_device(), int(seed) & 0xFFFFFFFFFFFFFFFF)


def manual_seed_all(seed: int) -> None:
    for d in range(device_count()):
        _C.rng_manual_seed(d, int(seed) & 0xFFFFFFFFFFFFFFFF)


def seed() -> None:
    _C.rng_seed(_C.current_device())


def seed_all() -> None:
    s = _C.rng_seed(0) if device_count() else 0
    for d in range(1, device_count()):
        _C.rng_manual_seed(d, s)


def initial_seed() -> int:
    return _C.rng_initial_seed(_C.current_device())


def get_rng_state(device=None) -> torch.Tensor:
    """16 bytes (uint8, CPU): the seed, then the call offset, little endian."""
    return _C.rng_get_state(_index(device) if device is not None else _C.current_device())


def set_rng_state(state: torch.Tensor, device=None) -> None:
    _C.rng_set_state(_index(device) if device is not None else _C.current_device(), state)


def get_rng_state_all() -> list:
    return [_C.rng_get_state(d) for d in range(device_count())]


def set_rng_state_all(states) -> None:
    for d, st in enumerate(states):
        _C.rng_set_state(d, st)


def set_cpu_fallback_enabled(on: bool) -> None:
    """Enable/disable the boxed CPU fallback for ops without a supa kernel."""
    _C.set_cpu_fallback_enabled(bool(on))


def set_fused_cross_entropy_enabled(on) -> None:
    """Routing of 2-d cross_entropy (f32/bf16/f16 logits; int64 class targets
    or a probability target of the logits' shape and dtype; no class weight,
    no label smoothing) to the fused kernels: one read of the logits (and
    target) forward, one read + one write backward.
    None (the default): the reference's routing -- float32 logits fused,
    bfloat16 / float16 through the log_softmax + nll_loss decomposition.
    True: every floating dtype fused.  False: none fused."""
    _C.set_fused_cross_entropy_mode(-1 if on is None else (1 if on else 0))


def fused_cross_entropy_enabled():
    """None (the reference's routing: float32 fused), True or False."""
    m = int(_C.fused_cross_entropy_mode())
    return None if m < 0 else bool(m)


def set_fused_bce_backward_enabled(on: bool) -> None:
    """Compute binary_cross_entropy_with_logits' input gradient in one kernel
    (on by default; bit-identical to the autograd formula's op-by-op
    evaluation, which is used when off, under create_graph, or for mixed
    dtypes)."""
    _C.set_fused_bce_backward_enabled(bool(on))


def fused_bce_backward_enabled() -> bool:
    return bool(_C.fused_bce_backward_enabled())


def set_accurate_gelu_enabled(on: bool) -> None:
    """Evaluate gelu without the cancellation of 1 + erf(x/sqrt2) and
    1 + tanh(u) for x << 0: 'none' as x - (x/2) erfc(|x|/sqrt2) or
    (x/2) erfc(|x|/sqrt2), 'tanh' as x / (1 + exp(-2u)).  Off by default: the
    default is the reference's formula, (x/2)(1 + erf) / (x/2)(1 + tanh),
    whose results these forms do not reproduce for x << 0."""
    _C.set_accurate_gelu_enabled(bool(on))


def accurate_gelu_enabled() -> bool:
    return bool(_C.accurate_gelu_enabled())


def fallback_counts() -> dict:
    """Ops that went through the CPU fallback since the last reset, with counts."""
    return dict(_C.fallback_counts())


def reset_fallback_counts() -> None:
    _C.reset_fallback_counts()


# c10::DeviceType::PrivateUse1, the device type of supa streams
_SUPA_DEVICE_TYPE = 20


class Stream(torch.Stream):
    """A supa stream: an in-order queue on one device (the reference's
    torch_supa/supa/streams.py).  ``Stream()`` takes a stream of the device's
    pool of 32 (round-robin, as the reference's getStreamFromPool; every stream
    is non-blocking and has the default priority); ``stream_id=0`` is the
    device's default stream.  ``with s:`` makes it the current stream of its
    device on this thread."""

    def __new__(cls, device=None, priority=0, stream_id=None, device_index=None, device_type=None):
        if stream_id is None:
            device_index = _index(device) if device is not None else _C.current_device()
            stream_id = _C.pool_stream_id(device_index)
        elif device_index is None:
            device_index = _index(device) if device is not None else _C.current_device()
        return super().__new__(cls, stream_id=int(stream_id), device_index=int(device_index),
                               device_type=_SUPA_DEVICE_TYPE)

    @property
    def hip_stream(self) -> int:
        """The hipStream_t of this stream, as an integer."""
        return _C.stream_ptr(self.device_index, self.stream_id)

    def synchronize(self) -> None:
        _C.stream_synchronize(self.device_index, self.stream_id)

    def query(self) -> bool:
        return _C.stream_query(self.device_index, self.stream_id)

    def record_event(self, event: "Event" = None) -> "Event":
        event = Event() if event is None else event
        event.record(self)
        return event

    def wait_event(self, event: "Event") -> None:
        event.wait(self)

    def wait_stream(self, stream: "Stream") -> None:
        self.wait_event(stream.record_event())

    def __enter__(self):
        self._prev = _C.set_current_stream_id(self.device_index, self.stream_id)
        return self

    def __exit__(self, *exc):
        _C.set_current_stream_id(self.device_index, self._prev)
        return False

    def __eq__(self, other):
        return isinstance(other, torch.Stream) and (self.stream_id, self.device_index, self.device_type) == (
            other.stream_id, other.device_index, other.device_type)

    def __hash__(self):
        return hash((self.stream_id, self.device_index, self.device_type))

    def __repr__(self):
        return f"torch.supa.Stream(device=supa:{self.device_index}, stream_id={self.stream_id})"


def current_stream(device=None) -> Stream:
    """The current stream of `device` on this thread (the default stream
    until set_stream or ``with stream(...)`` changes it)."""
    idx = _index(device) if device is not None else _C.current_device()
    return Stream(stream_id=_C.current_stream_id(idx), device_index=idx)


def default_stream(device=None) -> Stream:
    idx = _index(device) if device is not None else _C.current_device()
    return Stream(stream_id=0, device_index=idx)


def set_stream(s: Stream) -> None:
    if s is not None:
        _C.set_current_stream_id(s.device_index, s.stream_id)


class stream:  # noqa: N801 (the torch.cuda.stream spelling)
    """Context manager: `s` is the current stream of its device inside."""

    def __init__(self, s):
        self.s = s

    def __enter__(self):
        if self.s is not None:
            self._prev = _C.set_current_stream_id(self.s.device_index, self.s.stream_id)
        return self.s

    def __exit__(self, *exc):
        if self.s is not None:
            _C.set_current_stream_id(self.s.device_index, self._prev)
        return False


class Event:
    """A device event (hipEvent_t): recorded on a stream (the current one by
    default), waited on by streams, timed against another event."""

    def __init__(self, enable_timing: bool = True):
        self._h = _C.event_create()

    def record(self, stream: Stream = None) -> None:
        if stream is None:
            _C.event_record(self._h)
        else:
            _C.event_record(self._h, stream.device_index, stream.stream_id)

    def wait(self, stream: Stream = None) -> None:
        if stream is None:
            _C.event_wait(self._h)
        else:
            _C.event_wait(self._h, stream.device_index, stream.stream_id)

    def query(self) -> bool:
        return _C.event_query(self._h)

    def synchronize(self) -> None:
        _C.event_synchronize(self._h)

    def elapsed_time(self, end: "Event") -> float:
        return _C.event_elapsed_ms(self._h, end._h)

    def __del__(self):
        try:
            _C.event_destroy(self._h)
        except Exception:
            pass
