"""supa_amd_sum_noalloc (the allocation-free entry point, workspace in the
library's own device array) against supa_amd_sum with a caller-provided
workspace, through the C ABI: bit-identical results on two calls in a row,
the second on a smaller input, for sum and mean over float32 and bfloat16
inputs; oversize requests are refused.  Device memory for the operands
comes from torch's HIP allocator; the entry point itself allocates nothing."""
import ctypes

import numpy as np
import pytest
import torch

import capi as A
import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def run(rc):
    assert rc == 0, rc


def _sum_both(L, x, scale, dtype_code):
    """The same reduction through both entry points; the one-element outputs
    (in x's dtype) as raw bytes."""
    out_ref = torch.empty(1, dtype=x.dtype, device=DEV)
    out_na = torch.empty(1, dtype=x.dtype, device=DEV)
    ws = torch.empty(L.supa_amd_sum_workspace_bytes(x.numel()), dtype=torch.uint8, device=DEV)
    d_ref = A.nd_desc([x.numel()], [(out_ref, [0]), (x, [1])], dtype_code)
    d_na = A.nd_desc([x.numel()], [(out_na, [0]), (x, [1])], dtype_code)
    run(L.supa_amd_sum(ctypes.byref(d_ref), scale, ws.data_ptr(), ws.numel(), None))
    run(L.supa_amd_sum_noalloc(ctypes.byref(d_na), scale, None))
    torch.cuda.synchronize()
    return out_ref.cpu(), out_na.cpu()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_sum_matches_workspace_sum_twice(dtype):
    L = A.lib()
    L.supa_amd_sum_noalloc.argtypes = [ctypes.POINTER(A.EwDesc), ctypes.c_double, ctypes.c_void_p]
    L.supa_amd_sum_noalloc_max_workspace_bytes.restype = ctypes.c_int64
    assert L.supa_amd_sum_noalloc_max_workspace_bytes() >= L.supa_amd_sum_workspace_bytes(1 << 40)
    code = A.F32 if dtype == torch.float32 else A.BF16
    g = torch.Generator().manual_seed(11)
    big = torch.randn(33554432 + 3, generator=g).to(dtype)
    small = torch.randn(1000, generator=g).to(dtype)
    for x, scale in [(big, 1.0), (small, 1.0), (big, 1.0 / big.numel()), (small, 1.0 / small.numel())]:
        dx = x.to(DEV)
        ref, na = _sum_both(L, dx, scale, code)
        assert ref.view(torch.uint8).tolist() == na.view(torch.uint8).tolist(), (x.numel(), scale, ref, na)
        # and both are the sum: within the float32 accumulation's error, then
        # one rounding to the output dtype
        want = float(O.sum_f32(x.float().numpy())) * scale
        tol = 1e-5 * np.abs(x.float().numpy()).sum() * scale / np.sqrt(x.numel())
        if dtype == torch.bfloat16:
            tol += abs(want) * 2.0 ** -8
        assert abs(float(na.float()) - want) <= tol + 1e-30


def test_noalloc_rejects_bad_arguments():
    L = A.lib()
    L.supa_amd_sum_noalloc.argtypes = [ctypes.POINTER(A.EwDesc), ctypes.c_double, ctypes.c_void_p]
    assert L.supa_amd_sum_noalloc(None, 1.0, None) == -1
