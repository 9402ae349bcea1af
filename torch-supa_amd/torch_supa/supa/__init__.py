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
