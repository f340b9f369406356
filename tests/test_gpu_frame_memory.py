"""GPU parity of frame memory's pooling and representative selection (or_frame_pool, or_frame_select) with the
oracle's restatement of FrameMemory.collect / select (src/onereel/frame_memory.py:76-132)."""
import numpy as np
import pytest
import torch

from onereel_amd.frame_memory import FrameMemory
from onereel_amd.layout import SceneLayout
from oracle import frame_memory as OF

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]
DEV = 'cuda'


def _groups(sizes, dim, noise, seed):
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(len(sizes), dim, generator=g)
    x = torch.cat([base[i].expand(n, -1) for i, n in enumerate(sizes)]) + noise * torch.randn(sum(sizes), dim,
                                                                                              generator=g)
    return torch.nn.functional.normalize(x, dim=-1)


@pytest.mark.parametrize('N,C,row0,T', [(100, 3072, 5, 7), (1590 * 3, 3072, 0, 1590), (37, 128, 20, 10)])
def test_frame_pool_matches_index_add_and_is_deterministic(N, C, row0, T):
    print(f'frame pool N={N} C={C} row0={row0} T={T}', flush=True)
    g = torch.Generator().manual_seed(N)
    hs = torch.randn(N, C, generator=g).to(torch.bfloat16)
    n_frames = (row0 + N + T - 1) // T + 1
    frame = (torch.arange(N) + row0) // T
    lay = SceneLayout([n_frames], halo=0)
    outs = []
    for _ in range(2):
        fm = FrameMemory(budget=2)
        fm.reset(lay, 2)
        gframe = frame.to(DEV)
        fm.collect(gframe, hs.to(DEV), layer=0)
        assert fm.frame_layout(gframe) == (row0, T)
        outs.append((fm.sums[0].cpu(), fm.counts[0].cpu()))
    s_ref, c_ref = OF.pool(frame, hs, n_frames)
    assert torch.equal(outs[0][0], outs[1][0])
    assert torch.equal(outs[0][1], c_ref.float())
    assert (outs[0][0].double() - s_ref).abs().max() <= 1e-5 * max(1.0, float(s_ref.abs().max()))


def test_frame_pool_general_frame_map_uses_index_add():
    g = torch.Generator().manual_seed(9)
    hs = torch.randn(40, 64, generator=g).to(torch.bfloat16)
    frame = torch.randperm(40, generator=g) % 7
    frame[3] = -1
    fm = FrameMemory(budget=2)
    fm.reset(SceneLayout([7], halo=0), 2)
    gframe = frame.to(DEV)
    fm.collect(gframe, hs.to(DEV), layer=0)
    assert fm.frame_layout(gframe) is None
    s_ref, c_ref = OF.pool(frame, hs, 7)
    assert (fm.sums[0].cpu().double() - s_ref).abs().max() < 1e-4 and torch.equal(fm.counts[0].cpu(), c_ref.float())


@pytest.mark.parametrize('sizes,dim,k,mode,sink', [
    ([5, 4], 16, 2, 'all', ()),                        # the reference test's two groups
    ([60, 60, 60, 60], 3072, 4, 'all', ()),            # 240 frames of 3072 features, four groups
    ([13, 40, 7, 28, 2, 50], 512, 6, 'all', ()),
    ([30, 30, 30], 256, 3, 'all', (0,)),               # the sink is not a candidate; it takes a budget slot
])
def test_frame_select_matches_oracle(sizes, dim, k, mode, sink):
    print(f'frame select sizes={sizes} dim={dim} k={k}', flush=True)
    feats = _groups(sizes, dim, 0.05, len(sizes))
    n = sum(sizes)
    lay = SceneLayout([n], halo=0)
    fm = FrameMemory(budget=k + len(sink), candidates=mode, sink=sink)
    fm.reset(lay, 2)
    got = fm.select(feats.to(DEV))
    ref = OF.select(feats, OF.candidates(lay.ranges, n, mode, sink), k)
    assert got == ref
    if not sink:
        assert len(got) == len(sizes)


def test_frame_select_boundary_candidates():
    feats = torch.nn.functional.normalize(torch.randn(12, 8, generator=torch.Generator().manual_seed(1)), dim=-1)
    lay = SceneLayout([4, 4, 4], halo=0)
    fm = FrameMemory(budget=3, candidates='boundary')
    fm.reset(lay, 4)
    got = fm.select(feats.to(DEV))
    assert got == fm.select(feats.to(DEV))                         # deterministic
    assert set(got) <= {0, 3, 4, 7, 8, 11}
    assert got == OF.select(feats, [0, 3, 4, 7, 8, 11], 3)


def test_frame_memory_step_cycle():
    """reset -> step 0 (fallback halo) -> collect + finish -> step 1 reads the chosen representatives
    (tests/test_onereel_frame_memory.py:19-38 of the reference, on the device)"""
    lay = SceneLayout([3, 3, 3], halo=0)
    fm = FrameMemory(budget=2, fallback=(1, 'adj'))
    fm.reset(lay, n_layers=8)
    assert fm.layer == 4 and lay.extra == {0: [3], 1: [2, 6], 2: [5]}
    fm.begin_step(0)
    feats = _groups([5, 4], 16, 0.01, 0)
    frame = torch.arange(9).repeat_interleave(4)
    fm.collect(frame.to(DEV), feats.repeat_interleave(4, 0).to(torch.bfloat16).to(DEV))
    fm.finish()
    assert lay.extra == {0: [3], 1: [2, 6], 2: [5]}
    fm.begin_step(1)
    reps = fm.history[-1]
    assert len(reps) == 2 and min(reps) < 5 <= max(reps)
    for j, (lo, hi) in enumerate(lay.ranges):
        assert lay.extra[j] == [f for f in reps if not lo <= f < hi]


def test_frame_map_cache_follows_new_and_changed_maps():
    """collect with one frame map, drop it, then collect a map of the same length but another T (the caching
    allocator may give it the old map's memory), then change that map in place: the pooled sums follow the map of
    each call"""
    N, C = 60, 64
    g = torch.Generator().manual_seed(5)
    hs = torch.randn(N, C, generator=g).to(torch.bfloat16)
    ghs = hs.to(DEV)
    fm = FrameMemory(budget=2)
    fm.reset(SceneLayout([20], halo=0), 2)
    f1 = (torch.arange(N) // 6).to(DEV)
    fm.collect(f1, ghs, layer=0)
    del f1
    for T, inplace in ((4, False), (3, True)):
        fm.sums, fm.counts = {}, {}
        if inplace:
            f2.copy_((torch.arange(N) // T).to(DEV))
        else:
            f2 = (torch.arange(N) // T).to(DEV)
        fm.collect(f2, ghs, layer=0)
        assert fm.frame_layout(f2) == (0, T)
        s_ref, c_ref = OF.pool(f2.cpu(), hs, 20)
        assert torch.equal(fm.counts[0].cpu(), c_ref.float())
        assert (fm.sums[0].cpu().double() - s_ref).abs().max() < 1e-4
