"""``torch.supa``: device module of the supa (MI355X) backend.

The subset of the reference's ``torch.supa`` (``torch_supa/supa/*.py``,
``csrc/supa/Module.cpp:1133-1162``) that the elementwise + loss path and its
harnesses use: device queries, synchronisation, allocator statistics, a timing
event, RNG seeding hooks (random numbers are drawn on the CPU and copied), and
the CPU-fallback switch.
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


# Random numbers for this backend are drawn by the CPU generator (the CPU
# fallback runs the sampling ops); seeding therefore goes to the CPU generator.
def manual_seed(seed: int) -> None:
    torch.random.default_generator.manual_seed(int(seed))


def manual_seed_all(seed: int) -> None:
    manual_seed(seed)


def seed() -> None:
    torch.random.seed()


def seed_all() -> None:
    torch.random.seed()


def initial_seed() -> int:
    return torch.random.initial_seed()


def get_rng_state(device=None):
    return torch.random.get_rng_state()


def set_rng_state(state, device=None) -> None:
    torch.random.set_rng_state(state)


def set_cpu_fallback_enabled(on: bool) -> None:
    """Enable/disable the boxed CPU fallback for ops without a supa kernel."""
    _C.set_cpu_fallback_enabled(bool(on))


def set_fused_cross_entropy_enabled(on: bool) -> None:
    """Route 2-d cross_entropy (f32/bf16/f16 logits, int64 targets, no class
    weight, no label smoothing) through the fused kernels: one read of the
    logits forward, one read + one write backward.  Off by default: the
    default is the reference's log_softmax + nll_loss decomposition."""
    _C.set_fused_cross_entropy_enabled(bool(on))


def fused_cross_entropy_enabled() -> bool:
    return bool(_C.fused_cross_entropy_enabled())


def set_fused_bce_backward_enabled(on: bool) -> None:
    """Compute binary_cross_entropy_with_logits' input gradient in one kernel
    (on by default; bit-identical to the autograd formula's op-by-op
    evaluation, which is used when off, under create_graph, or for mixed
    dtypes)."""
    _C.set_fused_bce_backward_enabled(bool(on))


def fused_bce_backward_enabled() -> bool:
    return bool(_C.fused_bce_backward_enabled())


def fallback_counts() -> dict:
    """Ops that went through the CPU fallback since the last reset, with counts."""
    return dict(_C.fallback_counts())


def reset_fallback_counts() -> None:
    _C.reset_fallback_counts()


class Event:
    """A device event on the stream the supa kernels run on."""

    def __init__(self, enable_timing: bool = True):
        self._h = _C.event_create()

    def record(self) -> None:
        _C.event_record(self._h)

    def synchronize(self) -> None:
        _C.event_synchronize(self._h)

    def elapsed_time(self, end: "Event") -> float:
        return _C.event_elapsed_ms(self._h, end._h)

    def __del__(self):
        try:
            _C.event_destroy(self._h)
        except Exception:
            pass
