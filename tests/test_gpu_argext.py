"""max / min reductions with their index on the supa device (amax / amin,
max.dim / min.dim, argmax / argmin, max() / min()), against upstream's CPU
kernels, exact: NaN propagates and its first position wins, ties go to the
first index, rows longer than one launch's chunk reduce in two launches."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def data(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    if dtype == torch.bool:
        return torch.rand(shape, generator=g) > 0.7
    if not dtype.is_floating_point:
        return torch.randint(-50, 50, shape, generator=g).to(dtype)  # plenty of ties
    x = torch.randn(shape, generator=g)
    x = torch.round(x * 8) / 8  # ties in float too
    return x.to(dtype)


def eq(got, want):
    got = got.cpu()
    assert got.dtype == want.dtype and got.shape == want.shape
    if got.is_floating_point():
        assert torch.equal(torch.isnan(got), torch.isnan(want))
        assert torch.equal(torch.nan_to_num(got), torch.nan_to_num(want))
    else:
        assert torch.equal(got, want)


DTYPES = [torch.float32, torch.bfloat16, torch.float16, torch.float64, torch.int32, torch.int64, torch.uint8,
          torch.bool]


@pytest.mark.parametrize("dtype", DTYPES)
def test_amax_amin(dtype, no_fallback):
    x = data((7, 33, 129), 110, dtype)
    dx = x.to("supa")
    for fn in (torch.amax, torch.amin):
        for dim in ((-1,), (0,), (0, 2), (1, 2), ()):
            for keep in (False, True):
                eq(fn(dx, dim=dim, keepdim=keep), fn(x, dim=dim, keepdim=keep))


@pytest.mark.parametrize("dtype", DTYPES)
def test_max_min_dim_argmax(dtype, no_fallback):
    x = data((65, 300), 111, dtype)
    if dtype.is_floating_point:
        x[3, 17] = float("nan")
        x[3, 40] = float("nan")
        x[5, :] = float("nan")
    dx = x.to("supa")
    for dim in (0, 1, -1):
        for keep in (False, True):
            for fn in (torch.max, torch.min):
                gv, gi = fn(dx, dim=dim, keepdim=keep)
                wv, wi = fn(x, dim=dim, keepdim=keep)
                eq(gv, wv)
                eq(gi, wi)
            if dtype != torch.bool:
                eq(torch.argmax(dx, dim=dim, keepdim=keep), torch.argmax(x, dim=dim, keepdim=keep))
                eq(torch.argmin(dx, dim=dim, keepdim=keep), torch.argmin(x, dim=dim, keepdim=keep))
    if dtype != torch.bool:
        eq(torch.argmax(dx), torch.argmax(x))
        eq(torch.argmin(dx, keepdim=True), torch.argmin(x, keepdim=True))
    eq(torch.max(dx), torch.max(x))
    eq(torch.min(dx), torch.min(x))


def test_long_rows_two_launches(no_fallback):
    g = torch.Generator().manual_seed(112)
    x = torch.randn(3, 300007, generator=g)
    x[1, 250001] = 9.0
    x[1, 5] = 9.0  # tie: the first wins
    x[2, 123456] = float("nan")
    dx = x.to("supa")
    for fn in (torch.max, torch.min):
        gv, gi = fn(dx, dim=1)
        wv, wi = fn(x, dim=1)
        eq(gv, wv)
        eq(gi, wi)
    big = torch.randn(10_000_019, generator=g)
    big[7_777_777] = 50.0
    eq(torch.argmax(big.to("supa")), torch.argmax(big))
    eq(torch.max(big.to("supa")), torch.max(big))
    eq(torch.amin(big.to("supa")), torch.amin(big))


def test_logsumexp_and_errors(no_fallback):
    x = torch.randn(64, 1000, generator=torch.Generator().manual_seed(113))
    torch.testing.assert_close(torch.logsumexp(x.to("supa"), -1).cpu(), torch.logsumexp(x, -1), rtol=1e-6, atol=1e-6)
    with pytest.raises(RuntimeError):
        torch.amax(torch.empty(3, 0, device="supa"), dim=1)
    with pytest.raises(RuntimeError):
        torch.max(torch.empty(0, device="supa"))
