"""The reference's small tensor tests, case for case: test_tensor_factories.py
(eye n and n x m exact, empty, empty_strided's strides), test_equal.py
(torch.equal on random pairs in three dtypes, plus equal and NaN pairs
here), test_resize.py (resize_ to the same element count keeps the data) and
test_cuda_scalar.py (_local_scalar_dense reads the first element of any
tensor, as upstream's does)."""
import copy

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
