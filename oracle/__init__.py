"""TEST INFRASTRUCTURE ONLY -- numpy front end of the CPU oracle.

The oracle restates, in plain C (``oracle/oracle.c``, ``oracle/oracle_math.h``),
the arithmetic the reference runs for the elementwise + loss operator path.  Only
``tests/``, ``bench.py``'s ``cpu_baseline`` leg and ``__graft_entry__.smoke()``
may import this package, and only as the checker.  The shipped library never
imports it; its device path fails loudly when the HIP extension is missing.

This module does the plumbing the C side leaves out: broadcasting, dtype
conversion (bfloat16 travels as ``uint16`` bit patterns), and integer arithmetic
(done with numpy's wrapping integer ops, which are the C semantics the
reference's integer kernels use).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

# op codes shared with oracle.c
ADD, MUL, DIV, DIV_TRUNC, DIV_FLOOR, MAXIMUM, MINIMUM = 0, 1, 2, 3, 4, 5, 6
ADDCMUL, ADDCDIV, LERP = 0, 1, 2
GELU, GELU_TANH, SILU, SIGMOID, TANH, EXP, LOG, ERF, RELU, NEG, RECIPROCAL, ABS, SQRT, EXPM1, LOG1P = range(15)
# the opt-in cancellation-free gelu forms (C-ABI codes SUPA_AMD_GELU_LOGERFC / _TANH_LOGISTIC)
GELU_LOGERFC, GELU_TANH_LOGISTIC = 22, 23
# oracle only: gelu('tanh') with the other binary32 neighbour of tanh where the
# device's forward quotient may round the other way (see gelu_tanh_forward_equal)
GELU_TANH_FAST_ALT = 100
(ACT_LEAKY_RELU, ACT_HARDTANH, ACT_ELU, ACT_SOFTPLUS, ACT_HARDSWISH, ACT_HARDSIGMOID, ACT_MISH, ACT_LOG_SIGMOID,
 ACT_THRESHOLD) = range(9)
MSE, SMOOTH_L1, BCE_LOGITS = 0, 1, 2
REDUCTION = {"none": 0, "mean": 1, "sum": 2}

_f32p = ctypes.POINTER(ctypes.c_float)
_u32p = ctypes.POINTER(ctypes.c_uint32)
_f64p = ctypes.POINTER(ctypes.c_double)
_u16p = ctypes.POINTER(ctypes.c_uint16)
_i64p = ctypes.POINTER(ctypes.c_int64)


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the library path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _SO


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            build()
        L = ctypes.CDLL(_SO)
        i64, c_int, c_float, c_double = ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_double
        sig = {
            "or_f32_to_bf16": (None, [_f32p, _u16p, i64]),
            "or_bf16_to_f32": (None, [_u16p, _f32p, i64]),
            "or_f64_to_bf16": (None, [_f64p, _u16p, i64]),
            "or_binary_f32": (None, [c_int, _f32p, _f32p, _f32p, i64, c_float]),
            "or_binary_f64": (None, [c_int, _f64p, _f64p, _f64p, i64, c_double]),
            "or_unary_f32": (None, [c_int, _f32p, _f32p, i64]),
            "or_ternary_f32": (None, [c_int, _f32p, _f32p, _f32p, _f32p, i64, c_float]),
            "or_unary_backward_f32": (None, [c_int, _f32p, _f32p, _f32p, i64]),
            "or_activation_f32": (None, [c_int, _f32p, _f32p, i64, c_float, c_float, c_float]),
            "or_activation_backward_f32": (None, [c_int, _f32p, _f32p, _f32p, i64, c_float, c_float, c_float,
                                                  c_int]),
            "or_log_softmax_fwd": (None, [_f32p, _f32p, i64, i64]),
            "or_log_softmax_bwd": (None, [_f32p, _f32p, _f32p, i64, i64]),
            "or_softmax_fwd": (None, [_f32p, _f32p, i64, i64]),
            "or_philox4x32_10": (None, [_u32p, _u32p, _u32p]),
            "or_rng_u32": (None, [ctypes.c_uint64, ctypes.c_uint64, i64, _u32p]),
            "or_uniform_f32": (None, [ctypes.c_uint64, ctypes.c_uint64, i64, c_float, c_float, _u32p, _f32p]),
            "or_normal_f32": (None, [ctypes.c_uint64, ctypes.c_uint64, i64, c_double, c_double, _f32p]),
            "or_dropout_f32": (None, [ctypes.c_uint64, ctypes.c_uint64, i64, _f32p, c_float, _u32p, _f32p,
                                      ctypes.POINTER(ctypes.c_uint8)]),
            "or_softmax_bwd": (None, [_f32p, _f32p, _f32p, i64, i64]),
            "or_nll_loss_fwd": (c_int, [_f32p, _i64p, _f32p, i64, i64, c_int, i64, _f32p, _f32p]),
            "or_ce_prob_fwd": (None, [_f64p, _f64p, i64, i64, c_int, _f64p, _f64p, _f64p]),
            "or_ce_prob_bwd": (None, [_f64p, _f64p, _f64p, _f64p, _f64p, i64, i64, c_int, _f64p]),
            "or_nll_loss_bwd": (c_int, [_f32p, _i64p, _f32p, i64, i64, c_int, i64, c_float, c_int, _f32p]),
            "or_loss_fwd": (None, [c_int, _f32p, _f32p, _f32p, _f32p, i64, c_int, c_float, _f32p]),
            "or_loss_bwd": (None, [c_int, _f32p, _f32p, _f32p, _f32p, _f32p, i64, c_int, c_float, _f32p]),
            "or_sum_f32": (c_double, [_f32p, i64]),
            "or_amp_unscale_f32": (c_int, [_f32p, i64, c_float]),
            "or_amp_update_scale": (None, [_f32p, ctypes.POINTER(ctypes.c_int32), c_float, c_double, c_double, i64]),
            "or_ce_fwd": (c_int, [_f64p, _i64p, i64, i64, i64, c_int, _f64p, _f64p, _f64p]),
            "or_ce_bwd": (None, [_f64p, _f64p, _i64p, _f64p, c_double, i64, i64, i64, c_int, _f64p]),
            "or_adamw_step": (None, [_f32p, _f32p, _f32p, _f32p, i64, c_float, c_double, c_double,
                                     c_double, c_double, c_double, c_int, _f32p, c_int, _f32p, c_int]),
            "or_sgd_step": (None, [_f32p, _f32p, _f32p, i64, c_double, c_double, c_double, c_double, c_int, c_int,
                                   c_int, _f32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a, ptype):
    if a is None:
        return None
    return a.ctypes.data_as(ptype)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ------------------------------------------------------------------ casts --
def f32_to_bf16(x) -> np.ndarray:
    """float32 -> bfloat16 bit patterns (uint16), round to nearest even."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().or_f32_to_bf16(_p(x, _f32p), _p(out, _u16p), x.size)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().or_bf16_to_f32(_p(h, _u16p), _p(out, _f32p), h.size)
    return out


def f64_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float64)
    out = np.empty(x.shape, np.uint16)
    lib().or_f64_to_bf16(_p(x, _f64p), _p(out, _u16p), x.size)
    return out


def round_bf16(x) -> np.ndarray:
    """float32 values rounded through bfloat16 and back (float32 result)."""
    return bf16_to_f32(f32_to_bf16(x))


# ------------------------------------------------------------ elementwise --
def binary(op: int, a, b, alpha: float = 1.0, dtype=np.float32) -> np.ndarray:
    """Binary op on float32/float64 operands after numpy broadcasting.

    For integer dtypes use :func:`binary_int`."""
    a, b = np.broadcast_arrays(np.asarray(a), np.asarray(b))
    if dtype == np.float64:
        a, b = _c(a, np.float64), _c(b, np.float64)
        out = np.empty(a.shape, np.float64)
        lib().or_binary_f64(op, _p(a, _f64p), _p(b, _f64p), _p(out, _f64p), a.size, float(alpha))
        return out
    a, b = _c(a, np.float32), _c(b, np.float32)
    out = np.empty(a.shape, np.float32)
    lib().or_binary_f32(op, _p(a, _f32p), _p(b, _f32p), _p(out, _f32p), a.size, float(alpha))
    return out


def div_trunc_16(a, b, dtype: str) -> np.ndarray:
    """Trunc division of bfloat16 / float16 operands (given as float32
    values): std::trunc(a / b) on the storage type (BinaryDivTruncKernel.cu:
    46-52), the float32 quotient rounded to the 16-bit type, then truncated.
    dtype: "bf16" or "f16"; float32 result."""
    q = binary(DIV, a, b)
    q = round_bf16(q) if dtype == "bf16" else np.asarray(q, np.float32).astype(np.float16).astype(np.float32)
    return np.trunc(q)


def div_trunc_16_scalar(a, b: float, dtype: str) -> np.ndarray:
    """Trunc division of bfloat16 / float16 values (given as float32) by a
    CPU scalar b: the float32 quotient a / float(b) truncated, then rounded to
    the 16-bit type.  The reference's is_cpu_scalar branch
    (BinaryDivTruncKernel.cu:30-41) truncates the float product a * (1 / b)
    without the 16-bit rounding; upstream CPU truncates the float quotient
    a / b.  dtype: "bf16" or "f16"; float32 result."""
    q = np.trunc(binary(DIV, a, np.full(np.shape(a), np.float32(b), np.float32)))
    return round_bf16(q) if dtype == "bf16" else np.asarray(q, np.float32).astype(np.float16).astype(np.float32)


def binary_int(op: int, a, b, alpha: int = 1, dtype=np.int64) -> np.ndarray:
    """Wrapping integer arithmetic (UfuncCUDA_add.cu:13-16 add, BinaryInternal.h
    mul, BinaryDivTruncKernel.cu / BinaryDivFloorKernel.cu integer paths)."""
    a = np.asarray(a, dtype=dtype)
    b = np.asarray(b, dtype=dtype)
    with np.errstate(over="ignore"):
        if op == ADD:
            return (a + (b * dtype(alpha)).astype(dtype)).astype(dtype)
        if op == MUL:
            return (a * b).astype(dtype)
        if op == DIV_TRUNC:
            q = np.abs(a) // np.abs(b)
            return np.where((a < 0) != (b < 0), -q, q).astype(dtype)
        if op == DIV_FLOOR:
            return np.floor_divide(a, b).astype(dtype)
    raise ValueError(op)


def unary(op: int, x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.float32)
    lib().or_unary_f32(op, _p(x, _f32p), _p(out, _f32p), x.size)
    return out


def gelu_tanh_forward_equal(got, x) -> bool:
    """Whether a device gelu('tanh') forward result equals the oracle's.

    The forward kernel takes tanh's binary64 quotient m / (m + 2) without the
    final residual correction that makes it the exact binary64 quotient (the
    correction costs two binary64 fma per element on the headline kernel):
    its quotient is within 2^-48.5 (relative) of m / (m + 2), so its tanh
    equals the oracle's except where m / (m + 2) lies that close to a binary32
    rounding boundary, where it may be the other neighbour.  Each element of
    ``got`` must equal the oracle's gelu('tanh') of ``x`` or, where the
    quotient is within 2^-44 of a boundary, the value with that other
    neighbour (``GELU_TANH_FAST_ALT``).  NaN matches NaN."""
    got = np.asarray(got, np.float32)
    ref = unary(GELU_TANH, x)
    if got.shape != ref.shape:
        return False
    ok = (got == ref) | (np.isnan(got) & np.isnan(ref))
    if ok.all():
        return True
    alt = unary(GELU_TANH_FAST_ALT, x)
    return bool(np.all(ok | (got == alt)))


def unary_backward(op: int, dy, x) -> np.ndarray:
    dy, x = np.broadcast_arrays(np.asarray(dy), np.asarray(x))
    dy, x = _c(dy, np.float32), _c(x, np.float32)
    out = np.empty(x.shape, np.float32)
    lib().or_unary_backward_f32(op, _p(dy, _f32p), _p(x, _f32p), _p(out, _f32p), x.size)
    return out


def activation(act: int, x, p0=0.0, p1=0.0, p2=0.0) -> np.ndarray:
    """Parameterised activation forward (float32)."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.float32)
    lib().or_activation_f32(act, _p(x, _f32p), _p(out, _f32p), x.size, p0, p1, p2)
    return out


def activation_backward(act: int, g, x, p0=0.0, p1=0.0, p2=0.0, flag=0) -> np.ndarray:
    g, x = np.broadcast_arrays(np.asarray(g), np.asarray(x))
    g, x = _c(g, np.float32), _c(x, np.float32)
    out = np.empty(x.shape, np.float32)
    lib().or_activation_backward_f32(act, _p(g, _f32p), _p(x, _f32p), _p(out, _f32p), x.size, p0, p1, p2, flag)
    return out


# ------------------------------------------------------------- row ops --
def ternary(op: int, a, b, c, value=1.0) -> np.ndarray:
    """addcmul / addcdiv (value) / lerp (c = weight) in float32, broadcast."""
    a, b, c = np.broadcast_arrays(np.asarray(a, np.float32), np.asarray(b, np.float32), np.asarray(c, np.float32))
    a, b, c = _c(a, np.float32), _c(b, np.float32), _c(c, np.float32)
    out = np.empty(a.shape, np.float32)
    lib().or_ternary_f32(op, _p(a, _f32p), _p(b, _f32p), _p(c, _f32p), _p(out, _f32p), a.size,
                         float(np.float32(value)))
    return out


def log_softmax(x) -> np.ndarray:
    """log_softmax over the last dim (float32 in, float32 out)."""
    x = _c(x, np.float32)
    cols = x.shape[-1]
    rows = x.size // max(cols, 1)
    out = np.empty(x.shape, np.float32)
    lib().or_log_softmax_fwd(_p(x, _f32p), _p(out, _f32p), rows, cols)
    return out


def log_softmax_backward(g, y) -> np.ndarray:
    g, y = _c(g, np.float32), _c(y, np.float32)
    cols = g.shape[-1]
    rows = g.size // max(cols, 1)
    out = np.empty(g.shape, np.float32)
    lib().or_log_softmax_bwd(_p(g, _f32p), _p(y, _f32p), _p(out, _f32p), rows, cols)
    return out


def softmax(x) -> np.ndarray:
    """softmax over the last dim (float32 in, float32 out)."""
    x = _c(x, np.float32)
    cols = x.shape[-1]
    rows = x.size // max(cols, 1)
    out = np.empty(x.shape, np.float32)
    lib().or_softmax_fwd(_p(x, _f32p), _p(out, _f32p), rows, cols)
    return out


def softmax_backward(g, y) -> np.ndarray:
    g, y = _c(g, np.float32), _c(y, np.float32)
    cols = g.shape[-1]
    rows = g.size // max(cols, 1)
    out = np.empty(g.shape, np.float32)
    lib().or_softmax_bwd(_p(g, _f32p), _p(y, _f32p), _p(out, _f32p), rows, cols)
    return out


def nll_loss(logp, target, weight=None, reduction="mean", ignore_index=-100):
    """Returns (output, total_weight) as float32 arrays."""
    logp = _c(logp, np.float32)
    target = _c(target, np.int64)
    n, c = logp.shape
    w = None if weight is None else _c(weight, np.float32)
    red = REDUCTION[reduction]
    out = np.empty(n if red == 0 else 1, np.float32)
    tw = np.zeros(1, np.float32)
    rc = lib().or_nll_loss_fwd(_p(logp, _f32p), _p(target, _i64p), _p(w, _f32p), n, c, red,
                               ignore_index, _p(out, _f32p), _p(tw, _f32p))
    if rc != 0:
        raise IndexError("nll_loss: target out of bounds")
    return (out if red == 0 else out.reshape(())), tw.reshape(())


def nll_loss_backward(grad_out, target, n, c, total_weight, weight=None, reduction="mean",
                      ignore_index=-100, bf16=False) -> np.ndarray:
    g = _c(grad_out, np.float32).reshape(-1)
    target = _c(target, np.int64)
    w = None if weight is None else _c(weight, np.float32)
    out = np.empty((n, c), np.float32)
    rc = lib().or_nll_loss_bwd(_p(g, _f32p), _p(target, _i64p), _p(w, _f32p), n, c,
                               REDUCTION[reduction], ignore_index, float(total_weight),
                               1 if bf16 else 0, _p(out, _f32p))
    if rc != 0:
        raise IndexError("nll_loss_backward: target out of bounds")
    return out


def nll_loss2d(logp, target, weight=None, reduction="mean", ignore_index=-100):
    """nll_loss2d (NF:11967; upstream LossNLL2d): the [N, C, H, W] problem is
    nll_loss over the N*H*W positions, each a row of C log-probabilities.
    Returns (output [N, H, W] or scalar, total_weight)."""
    logp = np.asarray(logp, np.float32)
    n, c, h, w = logp.shape
    rows = np.ascontiguousarray(np.moveaxis(logp, 1, -1).reshape(-1, c))
    out, tw = nll_loss(rows, np.asarray(target, np.int64).reshape(-1), weight, reduction, ignore_index)
    return (out.reshape(n, h, w) if reduction == "none" else out), tw


def nll_loss2d_backward(grad_out, target, shape, total_weight, weight=None, reduction="mean",
                        ignore_index=-100, bf16=False) -> np.ndarray:
    """grad_input [N, C, H, W] of nll_loss2d (NF:11981), through the row form."""
    n, c, h, w = shape
    g = nll_loss_backward(np.asarray(grad_out, np.float32).reshape(-1), np.asarray(target, np.int64).reshape(-1),
                          n * h * w, c, total_weight, weight, reduction, ignore_index, bf16)
    return np.ascontiguousarray(np.moveaxis(g.reshape(n, h, w, c), -1, 1))


def amp_unscale(x, inv_scale):
    """Returns (x * inv_scale as float32, found_inf)."""
    x = np.array(x, np.float32, copy=True).reshape(-1)
    bad = lib().or_amp_unscale_f32(_p(x, _f32p), x.size, float(np.float32(inv_scale)))
    return x, bool(bad)


def amp_update_scale(scale, tracker, found_inf, growth, backoff, interval):
    """Returns the new (scale, tracker)."""
    s = np.array([scale], np.float32)
    t = np.array([tracker], np.int32)
    lib().or_amp_update_scale(_p(s, _f32p), t.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), float(found_inf),
                              float(growth), float(backoff), int(interval))
    return float(s[0]), int(t[0])


def cross_entropy(x, target, reduction="mean", ignore_index=-100):
    """Fused cross-entropy in float64 (x: [n, c], any float dtype, converted
    to float64).  Returns (loss, lse, count): loss [n] for 'none', a 0-d array
    otherwise."""
    x = _c(x, np.float64)
    n, c = x.shape
    target = _c(target, np.int64)
    red = REDUCTION[reduction]
    loss = np.empty(n if red == 0 else 1, np.float64)
    lse = np.empty(n, np.float64)
    cnt = np.zeros(1, np.float64)
    rc = lib().or_ce_fwd(_p(x, _f64p), _p(target, _i64p), n, c, ignore_index, red, _p(loss, _f64p),
                         _p(lse, _f64p), _p(cnt, _f64p))
    if rc != 0:
        raise IndexError("cross_entropy: target out of bounds")
    return (loss if red == 0 else loss.reshape(())), lse, float(cnt[0])


def cross_entropy_backward(g, x, target, lse, count, reduction="mean", ignore_index=-100) -> np.ndarray:
    """Gradient of cross_entropy w.r.t. x in float64 (lse, count from cross_entropy)."""
    x = _c(x, np.float64)
    n, c = x.shape
    g = _c(g, np.float64).reshape(-1)
    target = _c(target, np.int64)
    lse = _c(lse, np.float64)
    out = np.empty((n, c), np.float64)
    lib().or_ce_bwd(_p(g, _f64p), _p(x, _f64p), _p(target, _i64p), _p(lse, _f64p), float(count), n, c,
                    ignore_index, REDUCTION[reduction], _p(out, _f64p))
    return out


def cross_entropy_prob(x, t, reduction="mean"):
    """Cross-entropy with probability targets in float64 (x, t: [n, c], any
    float dtype, converted to float64).  Returns (loss, lse, tsum): loss [n]
    for 'none', a 0-d array otherwise; tsum[i] = sum_j t[i, j]."""
    x = _c(x, np.float64)
    n, c = x.shape
    t = _c(np.broadcast_to(t, x.shape), np.float64)
    red = REDUCTION[reduction]
    out = np.empty(n if red == 0 else 1, np.float64)
    lse = np.empty(n, np.float64)
    tsum = np.empty(n, np.float64)
    lib().or_ce_prob_fwd(_p(x, _f64p), _p(t, _f64p), n, c, red, _p(out, _f64p), _p(lse, _f64p), _p(tsum, _f64p))
    return (out if red == 0 else out.reshape(())), lse, tsum


def cross_entropy_prob_backward(g, x, t, lse, tsum, reduction="mean") -> np.ndarray:
    """Gradient of cross_entropy_prob w.r.t. x in float64."""
    x = _c(x, np.float64)
    n, c = x.shape
    g = _c(g, np.float64).reshape(-1)
    t = _c(np.broadcast_to(t, x.shape), np.float64)
    lse, tsum = _c(lse, np.float64), _c(tsum, np.float64)
    out = np.empty((n, c), np.float64)
    lib().or_ce_prob_bwd(_p(g, _f64p), _p(x, _f64p), _p(t, _f64p), _p(lse, _f64p), _p(tsum, _f64p), n, c,
                         REDUCTION[reduction], _p(out, _f64p))
    return out


def loss(op: int, x, t, pos_weight=None, weight=None, reduction="mean", beta=1.0):
    x = _c(x, np.float32)
    t = _c(np.broadcast_to(t, x.shape), np.float32)
    pw = None if pos_weight is None else _c(np.broadcast_to(pos_weight, x.shape), np.float32)
    w = None if weight is None else _c(np.broadcast_to(weight, x.shape), np.float32)
    red = REDUCTION[reduction]
    out = np.empty(x.shape if red == 0 else (1,), np.float32)
    lib().or_loss_fwd(op, _p(x, _f32p), _p(t, _f32p), _p(pw, _f32p), _p(w, _f32p), x.size, red,
                      float(beta), _p(out, _f32p))
    return out if red == 0 else out.reshape(())


def loss_backward(op: int, grad, x, t, pos_weight=None, weight=None, reduction="mean", beta=1.0):
    x = _c(x, np.float32)
    t = _c(np.broadcast_to(t, x.shape), np.float32)
    pw = None if pos_weight is None else _c(np.broadcast_to(pos_weight, x.shape), np.float32)
    w = None if weight is None else _c(np.broadcast_to(weight, x.shape), np.float32)
    red = REDUCTION[reduction]
    g = _c(grad, np.float32).reshape(-1)
    out = np.empty(x.shape, np.float32)
    lib().or_loss_bwd(op, _p(g, _f32p), _p(x, _f32p), _p(t, _f32p), _p(pw, _f32p), _p(w, _f32p),
                      x.size, red, float(beta), _p(out, _f32p))
    return out


def round16(v, dtype: str) -> np.ndarray:
    """float32 values rounded to bfloat16 ("bf16") or float16 ("f16") and back."""
    v = np.asarray(v, np.float32)
    return round_bf16(v) if dtype == "bf16" else v.astype(np.float16).astype(np.float32)


def loss_16(name: str, x, t, dtype: str, reduction="mean", beta=1.0):
    """mse / smooth_l1 / huber forward on bfloat16 or float16 operands
    (given as float32 values), as upstream's device kernels compute them in
    scalar_t (mse_kernel_cuda, smooth_l1_kernel_cuda, huber_kernel_cuda): an
    operation between two c10::BFloat16 / c10::Half values is done in float32
    and rounded back to the type, one between such a value and a float stays
    in float32.  So d = x - t is rounded; mse squares d and rounds; smooth_l1
    and huber take z = |d| in float32 with beta / delta and 0.5 * beta in the
    16-bit type, and round the result.  A reduction adds the rounded terms
    (in float64 here, float32 on the device) and rounds the sum or mean.
    name: "mse", "smooth_l1" or "huber"; float32 result."""
    x = np.asarray(x, np.float32)
    t = np.broadcast_to(np.asarray(t, np.float32), x.shape)
    d = round16(x - t, dtype)
    if name == "mse":
        term = round16(d * d, dtype)
    else:
        b = round16(np.float32(beta), dtype)
        half_b = round16(np.float32(0.5) * b, dtype)
        z = np.abs(d)
        with np.errstate(divide="ignore", invalid="ignore"):
            quad = (np.float32(0.5) * z) * z
            if name == "smooth_l1":
                term = np.where(z < b, quad / b, z - half_b)
            else:
                term = np.where(z < b, quad, b * (z - half_b))
        term = round16(term.astype(np.float32), dtype)
    if reduction == "none":
        return term
    s = term.astype(np.float64).sum()
    if reduction == "mean":
        s = s / term.size
    return round16(np.float32(s), dtype).reshape(())


def loss_backward_16(name: str, grad, x, t, dtype: str, reduction="mean", beta=1.0) -> np.ndarray:
    """The gradients of :func:`loss_16` w.r.t. x (mse_backward_cuda_kernel,
    smooth_l1_backward_cuda_kernel, huber_backward_cuda_kernel): every
    operand is a 16-bit value (norm = 2/n or 2 for mse, 1/n or 1 otherwise,
    rounded to the type) and every operation is rounded:
      mse:       (norm d) g
      smooth_l1: -norm g below -beta, norm g above beta, ((norm d) g) / beta
      huber:     (-norm g) delta, (norm g) delta, (norm d) g
    grad is n values for 'none', one otherwise; float32 result."""
    x = np.asarray(x, np.float32)
    t = np.broadcast_to(np.asarray(t, np.float32), x.shape)
    g = np.asarray(grad, np.float32)
    g = np.broadcast_to(g.reshape(x.shape) if reduction == "none" else g.reshape(()), x.shape)
    norm = (2.0 if name == "mse" else 1.0) / (x.size if reduction == "mean" else 1)
    n = round16(np.float32(norm), dtype)
    d = round16(x - t, dtype)
    r = lambda v: round16(v, dtype)  # noqa: E731
    if name == "mse":
        return r(r(d * n) * g)
    b = r(np.float32(beta))
    if name == "smooth_l1":
        with np.errstate(divide="ignore", invalid="ignore"):
            mid = r(r(r(n * d) * g) / b)
        return np.where(d < -b, r(-n * g), np.where(d > b, r(n * g), mid)).astype(np.float32)
    return np.where(d < -b, r(r(-n * g) * b), np.where(d > b, r(r(n * g) * b), r(r(n * d) * g))).astype(np.float32)


def sgd_step(p, g, buf, lr, momentum=0.0, dampening=0.0, weight_decay=0.0, nesterov=False, maximize=False,
             first=False, grad_scale=None):
    """In-place _fused_sgd_ step on float32 numpy arrays (p, buf and, with
    grad_scale, g are updated); buf is None without momentum."""
    for a in (p, g) + (() if buf is None else (buf,)):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    gs = None if grad_scale is None else np.asarray([grad_scale], np.float32)
    lib().or_sgd_step(_p(p, _f32p), _p(g, _f32p), _p(buf, _f32p), p.size, float(weight_decay), float(momentum),
                      float(lr), float(dampening), 1 if nesterov else 0, 1 if maximize else 0, 1 if first else 0,
                      _p(gs, _f32p))


def xlog1py(x, y, dtype="f32") -> np.ndarray:
    """xlog1py_kernel_cuda: NaN for a NaN y, 0 for x == 0, else x log1p(y)
    with the oracle's log1p, in float32."""
    x, y = np.broadcast_arrays(np.asarray(x, np.float32), np.asarray(y, np.float32))
    with np.errstate(invalid="ignore"):
        r = np.where(np.isnan(y), y, np.where(x == 0, np.float32(0), x * unary(LOG1P, y)))
    return _store(r.astype(np.float32), dtype)


def _store(v, dtype: str) -> np.ndarray:
    """A float32 result stored in dtype ("f32", "bf16", "f16"), as float32."""
    v = np.asarray(v, np.float32)
    return v if dtype == "f32" else round16(v, dtype)


def shrink(kind: str, x, lambd=0.5, dtype="f32") -> np.ndarray:
    """hardshrink / softshrink (upstream ActivationHardshrinkKernel.cu,
    ActivationSoftshrinkKernel.cu) on dtype values given as float32, lambda
    in the storage type:
      hardshrink: -lambda <= x <= lambda ? 0 : x
      softshrink: NaN stays NaN; x > lambda ? x - lambda : x < -lambda ? x + lambda : 0."""
    x = np.asarray(x, np.float32)
    lam = _store(np.float32(lambd), dtype)
    with np.errstate(invalid="ignore"):
        inside = (x >= -lam) & (x <= lam)
        if kind == "hardshrink":
            return np.where(inside, np.float32(0), x).astype(np.float32)
        r = np.where(x > lam, x - lam, np.where(x < -lam, x + lam, np.float32(0)))
    return _store(np.where(np.isnan(x), x, r), dtype)


def shrink_backward(g, x, lambd=0.5, dtype="f32") -> np.ndarray:
    """shrink_backward_kernel: -lambda <= x <= lambda ? 0 : g."""
    x, g = np.broadcast_arrays(np.asarray(x, np.float32), np.asarray(g, np.float32))
    lam = _store(np.float32(lambd), dtype)
    return np.where((x >= -lam) & (x <= lam), np.float32(0), g).astype(np.float32)


def _sigmoid_f32(b) -> np.ndarray:
    """1 / (1 + exp(-b)) in float32 with the oracle's exp."""
    b = np.asarray(b, np.float32)
    return (np.float32(1) / (np.float32(1) + unary(EXP, -b))).astype(np.float32)


def glu(a, b, dtype="f32") -> np.ndarray:
    """glu's halves (upstream glu_kernel): a sigmoid(b) in float32."""
    return _store(np.asarray(a, np.float32) * _sigmoid_f32(b), dtype)


def glu_backward(a, b, g, dtype="f32"):
    """glu_backward_kernel: (sigmoid(b) g, ((1 - s) s) g a) for the two halves."""
    a, b, g = (np.asarray(v, np.float32) for v in (a, b, g))
    s = _sigmoid_f32(b)
    return _store(s * g, dtype), _store((((np.float32(1) - s) * s) * g) * a, dtype)


def prelu(x, w, dtype="f32") -> np.ndarray:
    """prelu_kernel: x > 0 ? x : w x (w broadcast to x)."""
    x, w = np.broadcast_arrays(np.asarray(x, np.float32), np.asarray(w, np.float32))
    return _store(np.where(x > 0, x, w * x), dtype)


def prelu_backward(x, w, g, dtype="f32"):
    """prelu_backward_kernel: (x > 0 ? g : w g, x > 0 ? 0 : x g), both at the
    broadcast shape."""
    x, w, g = np.broadcast_arrays(*(np.asarray(v, np.float32) for v in (x, w, g)))
    pos = x > 0
    return _store(np.where(pos, g, w * g), dtype), _store(np.where(pos, np.float32(0), x * g), dtype)


def sum_f32(x) -> float:
    x = _c(x, np.float32)
    return float(lib().or_sum_f32(_p(x, _f32p), x.size))


def adamw_step(p, g, m, v, step, lr, beta1, beta2, weight_decay, eps, maximize=False,
               grad_scale=None, amsgrad=False, vmax=None, l2=False):
    """In-place AdamW step on float32 numpy arrays (p, m, v and, with
    grad_scale, g are updated); l2=True is the Adam step (_fused_adam_)."""
    for a in (p, g, m, v):
        assert a.dtype == np.float32 and a.flags.c_contiguous
    gs = None if grad_scale is None else np.asarray([grad_scale], np.float32)
    if amsgrad:
        assert vmax is not None and vmax.dtype == np.float32
    lib().or_adamw_step(_p(p, _f32p), _p(g, _f32p), _p(m, _f32p), _p(v, _f32p), p.size,
                        float(step), lr, beta1, beta2, weight_decay, eps, 1 if maximize else 0,
                        _p(gs, _f32p), 1 if amsgrad else 0, _p(vmax, _f32p), 1 if l2 else 0)


def vector_norm(x, ord=2.0) -> float:
    """||x||_ord accumulated in float64: the quantity upstream's _foreach_norm
    (ForeachReduceOp.cu) and linalg_vector_norm (ReduceNormKernel.cu's
    NormZeroOps / NormOneOps / NormTwoOps / AbsMaxOps / AbsMinOps / NormOps)
    estimate in float.  ord 0 counts the non-zeros (a NaN counts), +-inf is
    the largest / smallest |x|, any other p is (sum |x|^p)^(1/p).  A NaN
    gives NaN (except ord 0) and an empty x gives 0 (_foreach_norm's value;
    linalg_vector_norm raises instead for a negative or infinite order)."""
    x = np.asarray(x, dtype=np.float64).ravel()
    if x.size == 0:
        return 0.0
    a = np.abs(x)
    if ord == 0:
        return float(np.count_nonzero(x))
    if np.isnan(a).any():
        return float("nan")
    if ord == 1:
        return float(a.sum())
    if ord == 2:
        return float(np.sqrt((a * a).sum()))
    if ord == float("inf"):
        return float(a.max())
    if ord == float("-inf"):
        return float(a.min())
    with np.errstate(divide="ignore", over="ignore"):
        return float(np.power(np.power(a, ord).sum(), 1.0 / ord))


def moments(x, correction=1.0):
    """(variance, mean) of x in float64, the quantities upstream's var / std
    / var_mean / std_mean (ReduceMomentKernel.cu over WelfordOps in
    SharedReduceOps.h) estimate in float: the two-pass sum of squared
    deviations over max(0, n - correction).  n <= correction divides by
    zero (inf, or NaN for a zero sum); an empty x gives NaN, NaN."""
    x = np.asarray(x, dtype=np.float64).ravel()
    n = x.size
    if n == 0:
        return float("nan"), float("nan")
    mean = x.sum() / n
    m2 = ((x - mean) ** 2).sum()
    div = n - correction if n > correction else 0.0
    with np.errstate(divide="ignore", invalid="ignore"):
        return float(np.float64(m2) / np.float64(div)), float(mean)


# ------------------------------------------------------------ random numbers
def philox4x32_10(ctr, key) -> np.ndarray:
    c = np.ascontiguousarray(ctr, np.uint32)
    k = np.ascontiguousarray(key, np.uint32)
    out = np.empty(4, np.uint32)
    lib().or_philox4x32_10(_p(c, _u32p), _p(k, _u32p), _p(out, _u32p))
    return out


def rng_u32(seed: int, offset: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint32)
    lib().or_rng_u32(seed, offset, n, _p(out, _u32p))
    return out


def uniform(seed: int, offset: int, n: int, lo=0.0, hi=1.0, dtype="f32") -> np.ndarray:
    """uniform_(lo, hi) for storage dtype "f32", "bf16" or "f16", as float32
    values: fma(u, hi - lo, lo) in float, rounded to the storage type, and a
    value equal to hi rounded to that type replaced by lo (upstream
    uniform_kernel, DistributionTemplates.h: the result stays in [lo, hi))."""
    scratch = np.empty(n, np.uint32)
    out = np.empty(n, np.float32)
    lib().or_uniform_f32(seed, offset, n, lo, hi, _p(scratch, _u32p), _p(out, _f32p))
    rnd = {"f32": lambda a: np.asarray(a, np.float32),
           "bf16": lambda a: bf16_to_f32(f32_to_bf16(np.asarray(a, np.float32))),
           "f16": lambda a: np.asarray(a, np.float32).astype(np.float16).astype(np.float32)}[dtype]
    out = rnd(out)
    return np.where(out == rnd(np.float32([hi]))[0], rnd(np.float32([lo]))[0], out).astype(np.float32)


def normal(seed: int, offset: int, n: int, mean=0.0, std=1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().or_normal_f32(seed, offset, n, mean, std, _p(out, _f32p))
    return out


def dropout(seed: int, offset: int, x, keep: float):
    """Returns (out, mask) of dropout with keep probability `keep`."""
    x = _c(x, np.float32).reshape(-1)
    scratch = np.empty(x.size, np.uint32)
    out = np.empty(x.size, np.float32)
    mask = np.empty(x.size, np.uint8)
    lib().or_dropout_f32(seed, offset, x.size, _p(x, _f32p), keep, _p(scratch, _u32p), _p(out, _f32p),
                         mask.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)))
    return out, mask.astype(bool)
