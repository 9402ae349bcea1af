"""The reference's copy and cast tests, case for case, exact (rtol = atol = 0
there too unless noted):

* test/test_copy.py: host <-> device round trips of (6, 2, 3, 4) ... (6,)
  in every storage dtype, a narrowed host-to-device copy_, copy_ into an
  empty_strided destination, the general as_strided copy with storage
  offsets, and the shallow .data swap.  Its test_depromotion expects moving a
  float64 tensor to the device to fail (the reference's hardware has no
  float64); MI355X has it and this build supports float64, so that case is
  not mirrored;
* test/test_copy_.py: type-casting copies into a non-contiguous destination,
  a broadcasting copy, a sliced broadcasting copy, and the permute(0, 2, 1)
  [1, 12288, 2048] bfloat16 copy;
* test/test_cast.py: .to(dtype) for every ordered pair of bool, int8, int32,
  int64, uint8, bfloat16, float16 and float32 on (1,), (8, 507),
  (133, 16, 16), (1, 3, 64, 64) and on a 0-dim tensor, with its value ranges
  ([0, 255] with uint8 on either side, [-128, 127] with int8, [-1000, 1000]
  otherwise), and its two vector cases."""
import itertools

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SUPA = "supa"
_seed = [5000]


def _gen():
    _seed[0] += 1
    return torch.Generator().manual_seed(_seed[0])


def uniform(shape, dtype, lo, hi):
    """create_random_tensor(mode=uniform): integers in [lo, hi] for the wide
    integer types, a float draw truncated into the 8-bit types, a float
    uniform(lo, hi) for the floating types, random bools."""
    g = _gen()
    if dtype == torch.bool:
        return torch.randint(0, 2, shape, generator=g).bool()
    if dtype in (torch.int32, torch.int64, torch.int16):
        return torch.randint(lo, hi + 1, shape, generator=g).to(dtype)
    x = torch.rand(shape, generator=g, dtype=torch.float64) * (hi - lo) + lo
    # clamped after the cast, so that a 16-bit type's rounding cannot leave
    # the range (127 or 255 rounding up would make an 8-bit cast undefined)
    return x.to(dtype).clamp(lo, hi) if dtype.is_floating_point else x.to(dtype)


def normal(shape, dtype=torch.float32):
    return torch.randn(shape, generator=_gen()).to(dtype)


def exact(cpu, dev):
    dev = dev.cpu()
    assert cpu.dtype == dev.dtype and cpu.shape == dev.shape
    if cpu.is_floating_point():
        assert torch.equal(torch.isnan(cpu), torch.isnan(dev))
        m = ~torch.isnan(cpu)
        assert torch.equal(cpu[m], dev[m])
    else:
        assert torch.equal(cpu, dev)


# ------------------------------------------------------------ test_copy.py
COPY_DTYPES = [torch.float32, torch.bfloat16, torch.float16, torch.uint8, torch.int8, torch.int16, torch.int32,
               torch.int64, torch.bool]


@pytest.mark.parametrize("dtype", COPY_DTYPES)
@pytest.mark.parametrize("shape", [(6, 2, 3, 4), (6, 2, 3), (6, 2), (6,)])
def test_copy_round_trip(shape, dtype, no_fallback):
    """test_copy.py:59-73: x * 17 cast to the dtype (bool: above the median),
    to the device and back."""
    x = normal(shape)
    x = x > torch.median(x) if dtype == torch.bool else (x * 17).to(dtype)
    exact(x, x.clone().to(SUPA))


def test_copy_h2d_narrow(no_fallback):
    """test_copy.py:75-81."""
    x = torch.zeros([8], dtype=torch.float32)
    x.narrow(0, 0, 4).copy_(torch.ones([4], dtype=torch.float32))
    xs = torch.zeros([8], dtype=torch.float32).to(SUPA)
    xs.narrow(0, 0, 4).copy_(torch.ones([4], dtype=torch.float32))
    exact(x, xs)


STRIDED_DTYPES = [torch.float32, torch.bfloat16, torch.int32, torch.int64]


@pytest.mark.parametrize("dtype", STRIDED_DTYPES)
def test_empty_strided_copy(dtype, no_fallback):
    """test_copy.py:83-95: copy_ of a float32 tensor into an empty_strided
    (2, 4, 2, 2) / (32, 4, 2, 1) destination of the dtype."""
    y = torch.empty_strided((2, 4, 2, 2), (32, 4, 2, 1), dtype=dtype)
    ys = torch.empty_strided((2, 4, 2, 2), (32, 4, 2, 1), dtype=dtype, device=SUPA)
    x = torch.randn((2, 4, 2, 2), generator=_gen())
    y.copy_(x)
    ys.copy_(x.to(SUPA))
    exact(y, ys)


@pytest.mark.parametrize("dtype", STRIDED_DTYPES)
def test_general_strided_copy(dtype, no_fallback):
    """test_copy.py:97-111: as_strided source [192, 32] / [778, 1] at offset
    1643552 of a (16, 192, 778) tensor into [192, 32] / [32, 1] at offset 67584
    of a (16, 192, 32) tensor."""
    src = normal((16, 192, 778), dtype) if dtype.is_floating_point else uniform((16, 192, 778), dtype, -5, 5)
    dst = normal((16, 192, 32), dtype) if dtype.is_floating_point else uniform((16, 192, 32), dtype, -5, 5)
    src_s, dst_s = src.to(SUPA), dst.to(SUPA)
    a = torch.as_strided(src, [192, 32], [778, 1], storage_offset=1643552)
    a_s = torch.as_strided(src_s, [192, 32], [778, 1], storage_offset=1643552)
    b = torch.as_strided(dst, [192, 32], [32, 1], storage_offset=67584)
    b_s = torch.as_strided(dst_s, [192, 32], [32, 1], storage_offset=67584)
    b.copy_(a)
    b_s.copy_(a_s)
    exact(b, b_s)
    exact(dst, dst_s)  # nothing outside the view was touched


def test_tensor_shallow_copy(no_fallback):
    """test_copy.py:113-116."""
    a = normal((3, 2, 1))
    s = normal((3, 2, 1)).to(SUPA)
    s.data = a
    exact(a, s)


# ------------------------------------------------------------ test_copy_.py
def _uncontiguous(shape, dtype):
    """generate_uncontiguous_tensor (common_utils.py:312-327): a tensor of the
    first two dims swapped, transposed back."""
    t = list(shape)
    t[0], t[1] = t[1], t[0]
    x = normal(tuple(t), dtype)
    return x.transpose(0, 1), x.to(SUPA).transpose(0, 1)


@pytest.mark.parametrize("shape1, dtype1, shape2, dtype2", [
    ((2, 16, 2048), torch.bfloat16, (32, 2048), torch.float32),
    ((1, 2, 3), torch.bfloat16, (2, 3), torch.float32)])
def test_typecast_copy(shape1, dtype1, shape2, dtype2, no_fallback):
    """test_copy_.py:31-42: a bfloat16 tensor reshaped and copied into a
    non-contiguous float32 destination."""
    x = normal(shape1, dtype1)
    xs = x.to(SUPA)
    y, ys = _uncontiguous(shape2, dtype2)
    y.copy_(x.reshape(shape2))
    ys.copy_(xs.reshape(shape2))
    exact(y, ys)


def test_broadcast_copy(no_fallback):
    """test_copy_.py:44-52: (2, 1) bfloat16 broadcast into (2, 3) float32."""
    x = normal((2, 1), torch.bfloat16)
    y = normal((2, 3))
    ys = y.to(SUPA)
    y.copy_(x)
    ys.copy_(x.to(SUPA))
    exact(y, ys)


def test_broadcast_sliced_copy(no_fallback):
    """test_copy_.py:54-63: x[3::6] of a (6, 23, 45, 34) bfloat16 tensor
    broadcast into (3, 23, 45, 34)."""
    x = normal((6, 23, 45, 34), torch.bfloat16)
    xs = x.to(SUPA)
    y = normal((3, 23, 45, 34), torch.bfloat16)
    ys = y.to(SUPA)
    y.copy_(x[3::6, :, :, :])
    ys.copy_(xs[3::6, :, :, :])
    exact(y, ys)


def test_permute_021_bfloat16_large(no_fallback):
    """test_copy_.py:65-79: [1, 12288, 2048] bfloat16, the source viewed with
    strides (25165824, 1, 12288)."""
    dst = normal((1, 12288, 2048), torch.bfloat16)
    src = normal((1, 12288, 2048), torch.bfloat16)
    dst_s, src_s = dst.to(SUPA), src.to(SUPA)
    d = torch.as_strided(dst, [1, 12288, 2048], [25165824, 2048, 1])
    d_s = torch.as_strided(dst_s, [1, 12288, 2048], [25165824, 2048, 1])
    s = torch.as_strided(src, [1, 12288, 2048], [25165824, 1, 12288])
    s_s = torch.as_strided(src_s, [1, 12288, 2048], [25165824, 1, 12288])
    torch.ops.aten.copy_(d, s)
    torch.ops.aten.copy_(d_s, s_s)
    exact(d, d_s)


# ------------------------------------------------------------ test_cast.py
CAST_NAMES = ["bool", "int8", "int", "long", "uint8", "bfloat16", "half", "float32"]
CAST_PAIRS = list(itertools.permutations(CAST_NAMES, 2))


def _range(src, dst):
    """test_cast.py:45-55."""
    if torch.uint8 in (src, dst):
        return 0, 255
    if torch.int8 in (src, dst):
        return -128, 127
    return -1000, 1000


@pytest.mark.parametrize("src_name, dst_name", CAST_PAIRS)
@pytest.mark.parametrize("shape", [(1,), (8, 507), (133, 16, 16), (1, 3, 64, 64)])
def test_cast(shape, src_name, dst_name, no_fallback):
    """test_cast.py:57-70."""
    src, dst = getattr(torch, src_name), getattr(torch, dst_name)
    x = uniform(shape, src, *_range(src, dst))
    exact(x.to(dst), x.to(SUPA).to(dst))


@pytest.mark.parametrize("src_name, dst_name", CAST_PAIRS)
def test_cast_scalar(src_name, dst_name, no_fallback):
    """test_cast.py:72-80: a 0-dim 3.0."""
    src, dst = getattr(torch, src_name), getattr(torch, dst_name)
    x = torch.tensor(3.0).to(src)
    exact(x.to(dst), x.to(SUPA).to(dst))


@pytest.mark.parametrize("shape, src, dst", [((128,), torch.float32, torch.bfloat16),
                                             ((9126,), torch.int32, torch.bfloat16)])
def test_cast_vector_cases(shape, src, dst, no_fallback):
    """test_cast.py:20 (its vector cases)."""
    x = uniform(shape, src, -1000, 1000)
    exact(x.to(dst), x.to(SUPA).to(dst))
