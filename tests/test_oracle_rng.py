"""The oracle's Philox4x32-10 stream and its uniform / bernoulli / dropout
restatements.  Philox itself is pinned by the Random123 known-answer
vectors (kat_vectors of Random123 1.09, philox4x32 with 10 rounds); the
word -> float mapping and the dropout arithmetic by their closed forms; the
distributions by moments at sizes where a wrong mapping (a dropped shift, a
2^-32 scale, keep and drop swapped) falls far outside the tolerance."""
import numpy as np
import pytest

import oracle as O

KAT = [  # (counter, key, expected), Random123 philox4x32_10
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    assert O.philox4x32_10(ctr, key).tolist() == want


def test_stream_layout():
    # element i is word i % 4 of philox((i/4 lo, i/4 hi, offset lo, offset hi), (seed lo, seed hi))
    seed, off = 0x0123456789ABCDEF, 0x1122334455667788
    r = O.rng_u32(seed, off, 11)
    for q in range(3):
        w = O.philox4x32_10([q, 0, off & 0xFFFFFFFF, off >> 32], [seed & 0xFFFFFFFF, seed >> 32])
        assert r[4 * q:4 * q + 4].tolist() == w[: len(r[4 * q:4 * q + 4])].tolist()
    # the counter's high word carries from the low one
    big = O.philox4x32_10([0, 1, 0, 0], [1, 0])
    assert not np.array_equal(big, O.philox4x32_10([0, 0, 0, 0], [1, 0]))
    # offsets and seeds give unrelated streams
    a, b, c = O.rng_u32(1, 0, 4096), O.rng_u32(1, 1, 4096), O.rng_u32(2, 0, 4096)
    assert (a == b).mean() < 0.01 and (a == c).mean() < 0.01


def test_uniform_closed_form_and_moments():
    seed, off = 7, 3
    u = O.uniform(seed, off, 1 << 20)
    r = O.rng_u32(seed, off, 1 << 20)
    np.testing.assert_array_equal(u, (r >> 8).astype(np.float32) * np.float32(2.0 ** -24))
    assert u.min() >= 0.0 and u.max() < 1.0
    assert abs(u.mean() - 0.5) < 3e-3 and abs(u.var() - 1.0 / 12) < 2e-3
    v = O.uniform(seed, off, 4096, -2.0, 6.0)
    np.testing.assert_array_equal(v, (u[:4096] * np.float32(8.0) + np.float32(-2.0)).astype(np.float32))
    assert v.min() >= -2.0 and v.max() < 6.0


@pytest.mark.parametrize("keep", [0.9, 0.5, 0.125, 1.0])
def test_dropout(keep):
    n = 1 << 18
    x = np.random.default_rng(4).standard_normal(n).astype(np.float32)
    out, mask = O.dropout(11, 5, x, keep)
    u = O.uniform(11, 5, n)
    np.testing.assert_array_equal(mask, u < np.float32(keep))
    scale = np.float32(1.0 / np.float64(np.float32(keep)))
    np.testing.assert_array_equal(out, np.where(mask, x * scale, np.float32(0.0) * x))
    assert abs(mask.mean() - keep) < 5 * np.sqrt(keep * (1 - keep) / n) + 1e-9
    if keep == 1.0:
        assert mask.all() and np.array_equal(out, x)


def test_normal_moments_and_pairs():
    """Box-Muller pairs: z0^2 + z1^2 = -2 log u1 and atan2(z1, z0) = 2 pi u2
    for the words the stream layout assigns; moments of N(0, 1)."""
    n = 1 << 20
    z = O.normal(21, 4, n).astype(np.float64)
    r = O.rng_u32(21, 4, n)
    u1 = ((r[0::2] >> 8).astype(np.float64) + 1) * 2.0 ** -24
    u2 = (r[1::2] >> 8).astype(np.float64) * 2.0 ** -24
    np.testing.assert_allclose(z[0::2] ** 2 + z[1::2] ** 2, -2 * np.log(u1), rtol=1e-6, atol=1e-6)
    ang = np.mod(np.arctan2(z[1::2], z[0::2]), 2 * np.pi)
    d = np.abs(ang - 2 * np.pi * u2)
    assert np.minimum(d, 2 * np.pi - d).max() < 1e-5
    assert abs(z.mean()) < 5e-3 and abs(z.var() - 1) < 5e-3
    assert abs(((z - z.mean()) ** 3).mean()) < 1e-2 and abs((z ** 4).mean() - 3) < 3e-2
    w = O.normal(21, 4, 1000, mean=2.0, std=0.5)
    np.testing.assert_allclose(w, (2.0 + 0.5 * z[:1000]).astype(np.float32), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("dtype", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("lo, hi", [(0.0, 1.0), (1.0, 2.0), (-3.0, 100.0)])
def test_uniform_range_is_half_open(dtype, lo, hi):
    """uniform_ stays in [from, to) after rounding to the storage type: about
    0.2 % of bf16 draws on (0, 1) round up to 1.0 and are mapped back to
    `from` (upstream uniform_kernel's bound reversal); float32 never rounds
    up (u <= 1 - 2^-24)."""
    u = O.uniform(3, 9, 1 << 22, lo, hi, dtype)
    assert u.min() >= lo and u.max() < hi
    raw = O.uniform(3, 9, 1 << 22, lo, hi, "f32")
    if dtype == "f32":
        assert np.array_equal(u, raw)
    else:
        # the only change besides rounding: values that rounded to `to`
        rnd = O.bf16_to_f32(O.f32_to_bf16(raw)) if dtype == "bf16" else raw.astype(np.float16).astype(np.float32)
        moved = rnd != u
        assert np.all(rnd[moved] == np.float32(hi)) and np.all(u[moved] == np.float32(lo))
