"""The reference's small tensor tests, case for case: test_tensor_factories.py
(eye n and n x m exact, empty, empty_strided's strides), test_native_ci.py's
test_deterministic_empty_float32 (every factory form filled with NaN under
deterministic algorithms; here also the integer maximum and resize_'s new
bytes, as upstream), test_equal.py
(torch.equal on random pairs in three dtypes, plus equal and NaN pairs
here), test_resize.py (resize_ to the same element count keeps the data) and
test_cuda_scalar.py (_local_scalar_dense reads the first element of any
tensor, as upstream's does), test_one_hot_fused.py (one_hot, whose
scatter_ runs on the device) and test_normalize_fused.py (F.normalize: the
vector norm, clamp_min and the division, all device kernels; the reference
calls its own torch.normalize, which upstream torch does not have)."""
import contextlib
import copy

import numpy as np

import pytest
import torch

pytestmark = pytest.mark.gpu

SUPA = "supa"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def test_eye(no_fallback):
    assert torch.equal(torch.eye(8, device=SUPA).cpu(), torch.eye(8))
    assert torch.equal(torch.eye(8, 4, device=SUPA).cpu(), torch.eye(8, 4))
    assert torch.equal(torch.eye(3, 7, dtype=torch.bfloat16, device=SUPA).cpu(), torch.eye(3, 7, dtype=torch.bfloat16))
    out = torch.empty(0, device=SUPA)
    torch.eye(5, 6, out=out)
    assert torch.equal(out.cpu(), torch.eye(5, 6))
    assert torch.eye(0, device=SUPA).shape == (0, 0)


def test_empty_and_empty_strided(no_fallback):
    assert torch.empty((2, 3), device=SUPA).shape == (2, 3)
    c = torch.empty_strided((2, 3), (1, 2))
    s = torch.empty_strided((2, 3), (1, 2), device=SUPA)
    assert c.stride() == s.stride() and c.size() == s.size()


@contextlib.contextmanager
def _deterministic_fill_enabled():
    was_enabled = torch.are_deterministic_algorithms_enabled()
    was_warn_only = torch.is_deterministic_algorithms_warn_only_enabled()
    was_fill = torch.utils.deterministic.fill_uninitialized_memory
    torch.use_deterministic_algorithms(True)
    torch.utils.deterministic.fill_uninitialized_memory = True
    try:
        yield
    finally:
        torch.use_deterministic_algorithms(was_enabled, warn_only=was_warn_only)
        torch.utils.deterministic.fill_uninitialized_memory = was_fill


def _factories(dtype):
    """test_native_ci.py:51-78: the factory forms of the reference's test."""
    return [
        lambda: torch.empty(10, 9, device=SUPA, dtype=dtype),
        lambda: torch.empty(10, 9, out=torch.zeros(1, device=SUPA, dtype=dtype)),
        lambda: torch.empty_like(torch.zeros(10, 9, device=SUPA, dtype=dtype)),
        lambda: torch.empty_like(torch.zeros(10, 9, device=SUPA, dtype=dtype), memory_format=torch.contiguous_format),
        lambda: torch.empty_strided((10, 9), (1, 5), device=SUPA, dtype=dtype),
        lambda: torch.empty_permuted((2, 3, 5), (1, 0, 2), device=SUPA, dtype=dtype),
    ]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_deterministic_empty_is_nan(dtype, no_fallback):
    for i, gen_fn in enumerate(_factories(dtype)):
        torch.supa.empty_cache()
        with _deterministic_fill_enabled():
            result = gen_fn()
        assert result.device.type == "supa"
        assert bool(result.isnan().all()), i


def test_deterministic_empty_integers_and_resize(no_fallback):
    """Integers take the type's maximum (upstream fill_empty_deterministic_);
    resize_ fills the bytes a grown storage adds and keeps the old ones."""
    with _deterministic_fill_enabled():
        t = torch.empty(7, 5, device=SUPA, dtype=torch.int32)
        assert bool((t.cpu() == torch.iinfo(torch.int32).max).all())
        t = torch.empty_strided((4, 3), (1, 4), device=SUPA, dtype=torch.int64)
        assert bool((t.cpu() == torch.iinfo(torch.int64).max).all())
        x = torch.arange(6, dtype=torch.float32).to(SUPA)
        x.resize_(4, 3)
        got = x.cpu().flatten()
        assert torch.equal(got[:6], torch.arange(6, dtype=torch.float32))
        assert bool(got[6:].isnan().all())
    # with the switch off, nothing is filled (no extra kernel): the values are
    # whatever the block held, so only the shape is checked
    assert torch.empty(10, 9, device=SUPA).shape == (10, 9)


@pytest.mark.parametrize("dtype", DTYPES)
def test_equal(dtype, no_fallback):
    g = torch.Generator().manual_seed(7)
    a, b = torch.randn(1, 16, generator=g).to(dtype), torch.randn(1, 16, generator=g).to(dtype)
    assert torch.equal(a.to(SUPA), b.to(SUPA)) == torch.equal(a, b)
    assert torch.equal(a.to(SUPA), a.clone().to(SUPA))
    n = a.clone()
    n[0, 3] = float("nan")
    assert torch.equal(n.to(SUPA), n.clone().to(SUPA)) == torch.equal(n, n.clone()) is False
    assert not torch.equal(a.to(SUPA), a[:, :8].to(SUPA))


@pytest.mark.parametrize("dtype", DTYPES)
def test_resize(dtype, no_fallback):
    x = torch.randn(2, 2, 4, 3, generator=torch.Generator().manual_seed(8)).to(dtype)
    y = x.to(SUPA)
    x.resize_(1, 2, 3, 4)
    y.resize_(1, 2, 3, 4)
    assert torch.equal(y.cpu(), x)


@pytest.mark.parametrize("shape", [(2, 3, 3, 3), (16, 16, 16, 1024), (16, 16, 15, 2135), (16, 16, 15, 511),
                                   (16, 15, 15, 1257)])
def test_local_scalar_dense(shape, no_fallback):
    x = torch.randn(shape, generator=torch.Generator().manual_seed(9))
    xs = copy.deepcopy(x).to(SUPA)
    assert torch.ops.aten._local_scalar_dense.default(x) == torch.ops.aten._local_scalar_dense.default(xs)


@pytest.mark.parametrize("shape, num_classes", [((8,), 4), ((64,), 32), ((1000,), 10), ((4, 16), 7), ((1024,), 128),
                                                ((262144,), 32)])
def test_one_hot(shape, num_classes, no_fallback):
    """test_one_hot_fused.py: int64 result of shape + [num_classes], exact."""
    idx = torch.randint(0, num_classes, shape, dtype=torch.int64, generator=torch.Generator().manual_seed(20260605))
    out = torch.nn.functional.one_hot(idx.to(SUPA).contiguous(), num_classes=num_classes)
    assert out.dtype == torch.int64 and list(out.shape) == list(shape) + [num_classes]
    assert torch.equal(out.cpu(), torch.nn.functional.one_hot(idx, num_classes=num_classes))


@pytest.mark.parametrize("shape", [(7, 48), (8, 64), (9, 96), (31, 128), (5, 192), (8, 256), (11, 384), (8, 512)])
def test_normalize(shape, no_fallback):
    """test_normalize_fused.py: p = 2 over the last dim, eps 1e-12, rtol 1e-5
    / atol 1e-6."""
    x = torch.randn(shape, generator=torch.Generator().manual_seed(20260604))
    want = torch.nn.functional.normalize(x, p=2.0, dim=-1, eps=1.0e-12)
    got = torch.nn.functional.normalize(x.to(SUPA).contiguous(), p=2.0, dim=-1, eps=1.0e-12)
    np.testing.assert_allclose(want.numpy(), got.cpu().numpy(), rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int64, torch.bool])
@pytest.mark.parametrize("dim", [0, 1, -1])
def test_scatter_value(dim, dtype, no_fallback):
    """scatter_ / scatter with a scalar against the CPU, exact: an index
    smaller than self along the other dims, a transposed destination, the
    out-of-place and out= forms; an index past the destination's size is
    reported (as an IndexError) at the next synchronisation."""
    g = torch.Generator().manual_seed(31)
    base = (torch.randn(6, 9, 11, generator=g) * 4).to(dtype)
    d = dim % 3
    isz = [5, 7, 8]
    isz[d] = 13
    index = torch.randint(0, base.shape[d], isz, generator=g)
    value = True if dtype == torch.bool else (7 if dtype == torch.int64 else -2.5)
    want = base.clone().scatter_(dim, index, value)
    got = base.to(SUPA).scatter_(dim, index.to(SUPA), value)
    assert torch.equal(got.cpu(), want)
    assert torch.equal(torch.scatter(base.to(SUPA), dim, index.to(SUPA), value).cpu(), want)
    t = base.transpose(0, 2).contiguous().transpose(0, 2)
    ts = base.transpose(0, 2).contiguous().to(SUPA).transpose(0, 2)
    assert torch.equal(ts.scatter_(dim, index.to(SUPA), value).cpu(), t.scatter_(dim, index, value))
    out = torch.empty(0, dtype=dtype, device=SUPA)
    torch.scatter(base.to(SUPA), dim, index.to(SUPA), value, out=out)
    assert torch.equal(out.cpu(), want)
    bad = index.clone()
    bad.view(-1)[5] = base.shape[d]
    with pytest.raises(IndexError, match="scatter_ index"):
        base.to(SUPA).scatter_(dim, bad.to(SUPA), value).cpu()


def test_scatter_value_conversions(no_fallback):
    """The scalar in the destination's type, as upstream's value.to<T>(): a
    float scalar into bool is value != 0 (0.5 -> True), into an integer type
    it truncates, and an integer destination refuses a value it cannot hold;
    a destination that overlaps itself is refused."""
    g = torch.Generator().manual_seed(32)
    index = torch.randint(0, 9, (4, 9), generator=g)
    for dtype, value in [(torch.bool, 0.5), (torch.bool, 0.0), (torch.int32, 3.75), (torch.int64, -2.5),
                         (torch.uint8, 200.0)]:
        base = torch.zeros(4, 9, dtype=dtype)
        want = base.clone().scatter_(1, index, value)
        got = base.to(SUPA).scatter_(1, index.to(SUPA), value)
        assert torch.equal(got.cpu(), want), (dtype, value)
    with pytest.raises(RuntimeError):
        torch.zeros(4, 9, dtype=torch.int8, device=SUPA).scatter_(1, index.to(SUPA), 1e10)
    with pytest.raises(RuntimeError, match="unsupported operation|overlap"):
        torch.zeros(1, device=SUPA).expand(4, 9).scatter_(1, index.to(SUPA), 1.0)
