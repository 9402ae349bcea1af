"""The C-ABI library loads (without touching a GPU) and exports every entry
point include/supa_amd.h declares; argument errors come back as status codes
without any device work."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "supa_amd.h")
LIB = os.path.join(ROOT, "torch-supa_amd", "torch_supa", "libsupa_amd_kernels.so")


def declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(supa_amd_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    import torch  # noqa: F401  (load torch's HIP runtime first: one runtime per process)
    assert os.path.exists(LIB), "build the library first: python torch-supa_amd/build.py"
    return ctypes.CDLL(LIB)


def test_every_declared_symbol_is_exported(lib):
    names = declared()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_status_strings_and_version(lib):
    lib.supa_amd_status_string.restype = ctypes.c_char_p
    with open(HEADER) as f:
        ver = int(re.search(r"#define SUPA_AMD_ABI_VERSION (\d+)", f.read()).group(1))
    assert lib.supa_amd_abi_version() == ver
    assert lib.supa_amd_status_string(0) == b"success"
    assert b"invalid" in lib.supa_amd_status_string(-1)


def test_argument_errors_need_no_device(lib):
    # NULL descriptor / bad mode: rejected before any launch
    assert lib.supa_amd_add(None, ctypes.c_double(1.0), ctypes.c_int64(1), None) == -1
    assert lib.supa_amd_div(None, 7, None) == -1
    assert lib.supa_amd_log_softmax_forward(None, 6, None, 6, 1, 1, None) == -1
    lib.supa_amd_sum_workspace_bytes.restype = ctypes.c_int64
    assert lib.supa_amd_sum_workspace_bytes(ctypes.c_int64(1 << 30)) > 0
    i64 = ctypes.c_int64
    lib.supa_amd_cross_entropy_workspace_bytes.restype = i64
    assert lib.supa_amd_cross_entropy_workspace_bytes(i64(1000)) == 4000
    # fused cross-entropy: bad reduction, missing output, missing workspace
    fake = ctypes.c_void_p(256)  # never dereferenced: the checks come first
    assert lib.supa_amd_cross_entropy_forward(fake, 6, fake, i64(4), i64(10), i64(-100), 9, fake, fake, fake,
                                              fake, i64(16), None, None) == -1
    assert lib.supa_amd_cross_entropy_forward(fake, 6, fake, i64(4), i64(10), i64(-100), 1, None, fake, fake,
                                              fake, i64(16), None, None) == -1
    assert lib.supa_amd_cross_entropy_forward(fake, 6, fake, i64(4), i64(10), i64(-100), 1, fake, fake, fake,
                                              None, i64(0), None, None) == -4
    assert lib.supa_amd_cross_entropy_backward(None, fake, 6, fake, fake, fake, i64(4), i64(10), i64(-100), 1,
                                               fake, None, None) == -1
    # probability targets: the same checks, and the float32 target sums
    assert lib.supa_amd_cross_entropy_prob_forward(fake, fake, 6, i64(4), i64(10), 9, fake, fake, fake, fake,
                                                   i64(16), None) == -1
    assert lib.supa_amd_cross_entropy_prob_forward(fake, fake, 6, i64(4), i64(10), 1, fake, fake, None, fake,
                                                   i64(16), None) == -1
    assert lib.supa_amd_cross_entropy_prob_forward(fake, fake, 6, i64(4), i64(10), 1, fake, fake, fake, None,
                                                   i64(0), None) == -4
    assert lib.supa_amd_cross_entropy_prob_forward(fake, fake, 4, i64(4), i64(10), 1, fake, fake, fake, fake,
                                                   i64(16), None) == -2  # int64 logits
    assert lib.supa_amd_cross_entropy_prob_backward(fake, fake, None, 6, fake, fake, i64(4), i64(10), 1, fake,
                                                    None) == -1
    assert lib.supa_amd_cross_entropy_prob_backward(fake, fake, fake, 6, fake, fake, i64(4), i64(0), 1, fake,
                                                    None) == -1


def test_foreach_argument_errors(lib):
    i64 = ctypes.c_int64
    lib.supa_amd_foreach_norm_workspace_bytes.restype = i64
    numel = (i64 * 3)(1000, 0, 5000)  # f32: 2048-element chunks -> 1 + 0 + 3 partials of 4 bytes
    assert lib.supa_amd_foreach_norm_workspace_bytes(3, numel, 6) == 16
    assert lib.supa_amd_foreach_norm_workspace_bytes(3, numel, 4) == -2  # int64: no kernel
    fake = (ctypes.c_void_p * 3)(256, 256, 256)
    # ord 3 is not a fast-path norm; a missing workspace is reported before any launch
    assert lib.supa_amd_foreach_norm(3, fake, numel, 6, ctypes.c_double(3.0), fake, 6, None, i64(0), None) == -1
    assert lib.supa_amd_foreach_norm(3, fake, numel, 6, ctypes.c_double(2.0), fake, 6, None, i64(0), None) == -4
    # bad form; a ScalarList form without scalars; lerp from a device scalar
    d0 = ctypes.c_double(0.0)
    assert lib.supa_amd_foreach(0, 7, 3, fake, fake, fake, None, numel, 6, None, d0, None, None) == -1
    assert lib.supa_amd_foreach(2, 1, 3, fake, fake, None, None, numel, 6, None, d0, None, None) == -1
    assert lib.supa_amd_foreach(7, 2, 3, fake, fake, fake, None, numel, 6, None, d0, fake, None) == -1
    assert lib.supa_amd_foreach(99, 1, 3, fake, fake, None, None, numel, 6, None, d0, None, None) == -1
