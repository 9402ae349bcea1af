"""ctypes binding of include/supa_amd.h for the tests: the boundary a
non-PyTorch caller would use (plain pointers, sizes and POD descriptors).
Device memory for these tests comes from torch's HIP allocator (``cuda``
tensors); only raw pointers cross the boundary."""
import ctypes
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.path.join(ROOT, "torch-supa_amd", "torch_supa", "libsupa_amd_kernels.so")

MAX_DIMS = 8
MAX_OPERANDS = 6

U8, I8, I16, I32, I64, F16, F32, F64, BOOL, BF16 = 0, 1, 2, 3, 4, 5, 6, 7, 11, 15
GELU, GELU_TANH, SILU, SIGMOID, TANH, EXP, LOG, ERF, RELU, NEG = range(10)
LOSS_MSE, LOSS_SMOOTH_L1, LOSS_BCE = 0, 1, 2
RED_NONE, RED_MEAN, RED_SUM = 0, 1, 2


class Operand(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("strides", ctypes.c_int64 * MAX_DIMS), ("dtype", ctypes.c_int32),
                ("is_scalar", ctypes.c_int32), ("scalar", ctypes.c_double), ("iscalar", ctypes.c_int64)]


class EwDesc(ctypes.Structure):
    _fields_ = [("sizes", ctypes.c_int64 * MAX_DIMS), ("ndim", ctypes.c_int32), ("noperands", ctypes.c_int32),
                ("common_dtype", ctypes.c_int32), ("reserved", ctypes.c_int32),
                ("op", Operand * MAX_OPERANDS)]


_lib = None


def lib():
    global _lib
    if _lib is None:
        import torch  # noqa: F401  (torch's HIP runtime is the process's runtime)
        L = ctypes.CDLL(LIB_PATH)
        vp, i32, i64, dbl = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_double
        P = ctypes.POINTER(EwDesc)
        sig = {
            "supa_amd_add": [P, dbl, i64, vp], "supa_amd_mul": [P, vp], "supa_amd_div": [P, ctypes.c_int, vp],
            "supa_amd_unary": [P, ctypes.c_int, vp], "supa_amd_unary_backward": [P, ctypes.c_int, vp],
            "supa_amd_copy": [P, vp], "supa_amd_fill": [P, vp],
            "supa_amd_loss_forward": [P, ctypes.c_int, ctypes.c_int, dbl, ctypes.c_int, ctypes.c_int, vp, vp, i64, vp],
            "supa_amd_loss_backward": [P, ctypes.c_int, dbl, dbl, vp],
            "supa_amd_sum": [P, dbl, vp, i64, vp],
            "supa_amd_sum_rows": [vp, i32, vp, i32, i64, i64, dbl, vp],
            "supa_amd_log_softmax_forward": [vp, i32, vp, i32, i64, i64, vp],
            "supa_amd_log_softmax_backward": [vp, vp, i32, vp, i32, i64, i64, vp],
            "supa_amd_nll_loss_forward": [vp, i32, vp, vp, i64, i64, ctypes.c_int, i64, vp, vp, vp, vp],
            "supa_amd_nll_loss_backward": [vp, i32, vp, vp, vp, i64, i64, ctypes.c_int, i64, vp, vp, vp],
            "supa_amd_foreach_binary": [ctypes.c_int, i32, vp, vp, vp, vp, i32, dbl, dbl, vp],
            "supa_amd_fused_adamw": [i32, vp, vp, vp, vp, vp, vp, vp, i32, dbl, vp, dbl, dbl, dbl, dbl,
                                     ctypes.c_int, ctypes.c_int, vp, vp, vp],
            "supa_amd_cross_entropy_forward": [vp, i32, vp, i64, i64, i64, ctypes.c_int, vp, vp, vp, vp, i64, vp, vp],
            "supa_amd_cross_entropy_backward": [vp, vp, i32, vp, vp, vp, i64, i64, i64, ctypes.c_int, vp, vp, vp],
            "supa_amd_amp_unscale": [i32, vp, vp, i32, vp, vp, vp],
            "supa_amd_amp_update_scale": [vp, vp, vp, dbl, dbl, i64, vp],
        }
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        L.supa_amd_status_string.restype = ctypes.c_char_p
        L.supa_amd_sum_workspace_bytes.restype = i64
        L.supa_amd_sum_workspace_bytes.argtypes = [i64]
        L.supa_amd_loss_workspace_bytes.restype = i64
        L.supa_amd_loss_workspace_bytes.argtypes = [i64]
        L.supa_amd_cross_entropy_workspace_bytes.restype = i64
        L.supa_amd_cross_entropy_workspace_bytes.argtypes = [i64]
        _lib = L
    return _lib


def dtype_code(t):
    import torch
    return {torch.uint8: U8, torch.int8: I8, torch.int16: I16, torch.int32: I32, torch.int64: I64,
            torch.float16: F16, torch.float32: F32, torch.float64: F64, torch.bool: BOOL,
            torch.bfloat16: BF16}[t]


def flat_desc(out, *ins, common=None):
    """Descriptor for operands that all have out's element count, iterated in
    one dimension over each operand's own (contiguous or stride-0) layout."""
    d = EwDesc()
    n = out.numel()
    d.ndim = 1
    d.sizes[0] = n
    d.noperands = 1 + len(ins)
    d.common_dtype = dtype_code(common if common is not None else out.dtype)
    for k, t in enumerate((out,) + ins):
        o = d.op[k]
        if isinstance(t, (int, float)):
            o.is_scalar = 1
            o.scalar = float(t)
            o.iscalar = int(t)
            o.dtype = d.common_dtype
            continue
        o.data = t.data_ptr()
        o.dtype = dtype_code(t.dtype)
        o.strides[0] = 0 if t.numel() == 1 and n > 1 else 1
    return d


def nd_desc(sizes, operands, common):
    """Descriptor from explicit fastest-first sizes and per-operand
    (tensor, strides) pairs."""
    d = EwDesc()
    d.ndim = len(sizes)
    for i, s in enumerate(sizes):
        d.sizes[i] = s
    d.noperands = len(operands)
    d.common_dtype = common
    for k, (t, st) in enumerate(operands):
        o = d.op[k]
        o.data = t.data_ptr()
        o.dtype = dtype_code(t.dtype)
        for i, s in enumerate(st):
            o.strides[i] = s
    return d


def ptr_array(ts):
    arr = (ctypes.c_void_p * len(ts))(*[t.data_ptr() for t in ts])
    return arr


def i64_array(vals):
    return (ctypes.c_int64 * len(vals))(*vals)
