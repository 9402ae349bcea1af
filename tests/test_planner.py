"""The iteration planner (csrc/host/planner.cpp) against upstream PyTorch's
own layout decisions, by brute force over random shapes, permutations,
broadcasts and slices: the output strides it picks for a new result must be
the strides the upstream CPU TensorIterator gives the same op, and its
coalesced iteration space must address exactly the elements of each operand."""
import itertools
import random

import numpy as np
import pytest
import torch

torch_supa = pytest.importorskip("torch_supa")
_C = torch_supa._C


def plan(out, *ins):
    ops = [dict(is_output=True, allocate=out is None)] if out is None else [
        dict(is_output=True, sizes=list(out.shape), strides=list(out.stride()))]
    for t in ins:
        if t is None:
            ops.append(dict(scalar=True))
        else:
            ops.append(dict(sizes=list(t.shape), strides=list(t.stride())))
    return _C.plan(ops)


def random_operand(rng, shape, allow_bcast=True):
    """A view with the given logical shape: maybe permuted storage, maybe
    sliced, maybe broadcast along some dims."""
    nd = len(shape)
    perm = list(range(nd))
    if rng.random() < 0.5:
        rng.shuffle(perm)
    bshape = [1 if (allow_bcast and rng.random() < 0.2) else s for s in shape]
    base_shape = [bshape[p] for p in perm]
    step = 2 if rng.random() < 0.2 else 1
    base = torch.empty([s * step if i == nd - 1 else s for i, s in enumerate(base_shape)] or [1])
    if nd:
        base = base[..., ::step] if step > 1 else base
        t = base.permute([perm.index(i) for i in range(nd)])
    else:
        t = base.reshape(())
    return t.expand(shape) if list(t.shape) != list(shape) else t


@pytest.mark.parametrize("seed", range(40))
def test_output_strides_match_torch(seed):
    rng = random.Random(seed)
    nd = rng.randint(0, 5)
    shape = [rng.choice([1, 2, 3, 5, 8]) for _ in range(nd)]
    a = random_operand(rng, shape)
    b = random_operand(rng, shape[rng.randint(0, nd):] if nd else [])
    ref = torch.add(a, b)
    p = plan(None, a, b)
    assert p["shape"] == list(ref.shape)
    assert p["out_strides"][0] == list(ref.stride()), (a.stride(), b.stride(), ref.stride())


def test_transposed_c2_leg():
    """c2's transposed leg: x [64,2048,4096] with strides (8388608,1,2048);
    the result inherits the permutation and the iteration space becomes
    3 coalesced dims with the bias broadcast along the innermost."""
    x = torch.empty(64, 4096, 2048).transpose(1, 2)
    bias = torch.empty(4096)
    p = plan(None, x, bias)
    assert p["out_strides"][0] == [8388608, 1, 2048]
    assert p["it_sizes"] == [2048, 4096, 64]
    assert p["it_strides"][2] == [0, 1, 0]
    y = torch.empty(64, 2048, 4096)
    p = plan(None, y, bias)
    assert p["out_strides"][0] == [8388608, 4096, 1]
    assert p["it_sizes"] == [4096, 131072]
    assert p["it_strides"] == [[1, 4096], [1, 4096], [1, 0]]


def brute_offsets(sizes, strides):
    offs = []
    for idx in itertools.product(*[range(s) for s in reversed(sizes)]):
        offs.append(sum(i * s for i, s in zip(reversed(idx), strides)))
    return offs


@pytest.mark.parametrize("seed", range(40))
def test_iteration_space_addresses_every_element(seed):
    rng = random.Random(1000 + seed)
    nd = rng.randint(1, 4)
    shape = [rng.choice([1, 2, 3, 4]) for _ in range(nd)]
    a = random_operand(rng, shape)
    b = random_operand(rng, shape)
    p = plan(None, a, b)
    ref = torch.empty_strided(p["shape"], p["out_strides"][0])
    # enumerate the plan's iteration space; the k-th element of every operand
    # must be the same logical index
    it = p["it_sizes"]
    n = int(np.prod(it)) if it else 1
    assert n == int(np.prod(shape)) if shape else 1
    offs = [brute_offsets(it, st) for st in p["it_strides"]]
    # map storage offsets back to logical indices
    def logical(t, off_list):
        lut = {}
        for idx in itertools.product(*[range(s) for s in t.shape]):
            o = sum(i * s for i, s in zip(idx, t.stride()))
            lut.setdefault(o, []).append(idx)
        return [lut[o] for o in off_list]
    lo = logical(ref, offs[0])
    la = logical(a, offs[1])
    lb = logical(b, offs[2])
    for k in range(n):
        assert len(lo[k]) == 1
        assert lo[k][0] in la[k] and lo[k][0] in lb[k]


def test_broadcast_errors_and_scalars():
    with pytest.raises(ValueError):
        plan(None, torch.empty(3, 4), torch.empty(5))
    p = plan(None, torch.empty(3, 4), None)
    assert p["shape"] == [3, 4] and p["it_strides"][2] == [0]
    p = plan(None, torch.empty(0, 4), torch.empty(4))
    assert p["numel"] == 0
