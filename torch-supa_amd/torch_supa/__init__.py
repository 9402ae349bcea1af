"""MI355X PrivateUse1 backend for PyTorch: the elementwise + loss operator path.

Importing this package loads ``_C`` (whose static registrars install the
allocator, device guard, hooks and every ``TORCH_LIBRARY_IMPL(aten,
PrivateUse1, ...)`` kernel), renames the PrivateUse1 backend to ``"supa"`` --
the device name of BIRENSUPA/torch-supa (``torch_supa/__init__.py:78-85``), so
models written for it run unchanged -- and registers ``torch.supa``.

The device path has no CPU substitute: if the compiled extension is missing
the import fails, naming the build command.
"""
from __future__ import annotations

import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
KERNELS_LIB = os.path.join(_HERE, "libsupa_amd_kernels.so")

try:
    from . import _C  # noqa: F401  (static registration happens on load)
except ImportError as e:  # pragma: no cover - exercised only without a build
    raise ImportError(
        "torch_supa: the compiled extension is missing or failed to load "
        f"({e}); build it with `python torch-supa_amd/build.py`"
    ) from e

from . import supa as _supa_module  # noqa: E402

BACKEND_NAME = "supa"


def _register() -> None:
    if torch._C._get_privateuse1_backend_name() != BACKEND_NAME:
        torch.utils.rename_privateuse1_backend(BACKEND_NAME)
    if not hasattr(torch, BACKEND_NAME):
        torch._register_device_module(BACKEND_NAME, _supa_module)
    if not hasattr(torch.Tensor, "is_" + BACKEND_NAME):
        torch.utils.generate_methods_for_privateuse1_backend(
            for_tensor=True, for_module=True, for_storage=True, unsupported_dtype=None
        )


_register()

supa = _supa_module

__all__ = ["supa", "KERNELS_LIB", "BACKEND_NAME"]
