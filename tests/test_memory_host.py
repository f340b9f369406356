"""CPU checks of the bounded memory's representative choice (onereel_amd.memory.BoundaryMemory.select is torch ops,
device-agnostic): against the oracle's selection (oracle/memory.py, memory.py:58-93) on separated groups, through the
warm update path, and the layout of the (rep, valid) result."""
import torch

from onereel_amd.memory import BoundaryMemory
from oracle import memory as OM


def _groups(g, k, per, H, D, noise=0.01):
    base = torch.randn(k, H, D, generator=g)
    return torch.cat([base[i].expand(per, -1, -1) for i in range(k)]) + noise * torch.randn(k * per, H, D, generator=g)


def test_select_matches_oracle_on_separated_groups():
    """members spread enough (noise 0.1) that the nearest member of each group is not a tie at the fp32 rounding of
    the product's |x|^2 - 2 x.c + |c|^2 distances (the oracle takes explicit differences)"""
    g = torch.Generator().manual_seed(7)
    xs = _groups(g, 5, 9, 3, 16, noise=0.1)
    got, gv = BoundaryMemory(5).select('a', xs)
    ref, rv = OM.select(xs, 5)
    for h in range(3):
        assert sorted(got[h][gv[h]].tolist()) == sorted(ref[h][rv[h]].tolist())


def test_warm_update_keeps_a_converged_choice():
    """the second call on a key starts from the stored centroids and runs the short update without the convergence
    read: on the same candidates it returns the same representatives and valid flags"""
    g = torch.Generator().manual_seed(8)
    xs = _groups(g, 6, 7, 2, 32)
    mem = BoundaryMemory(8)
    r1, v1 = mem.select('k', xs)
    r2, v2 = mem.select('k', xs)
    assert torch.equal(r1, r2) and torch.equal(v1, v2)


def test_rep_valid_layout():
    """valid representatives come first, are distinct candidates, one per non-empty cluster; padding is 0 / False"""
    g = torch.Generator().manual_seed(9)
    x = torch.randn(200, 4, 16, generator=g)
    M = 32
    rep, valid = BoundaryMemory(M).select('l', x)
    assert rep.shape == (4, M) and valid.shape == (4, M)
    for h in range(4):
        n = int(valid[h].sum())
        assert n > 0 and bool(valid[h, :n].all()) and not bool(valid[h, n:].any())
        chosen = rep[h, :n].tolist()
        assert len(set(chosen)) == n and all(0 <= r < 200 for r in chosen)
        assert int(rep[h, n:].abs().sum()) == 0
