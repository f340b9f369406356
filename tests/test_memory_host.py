"""CPU checks of the bounded memory's host side (onereel_amd.memory): the boundary candidates against the oracle, the
plan a frame-major model builds (pieces, their query rows and local keys), and that the representative choice has no
CPU path."""
import pytest
import torch

from onereel_amd import _lib as L
from onereel_amd.layout import SceneLayout
from onereel_amd.memory import BoundaryMemory, _Static, candidate_frames, candidates, frame_plan, make_plan
from oracle import memory as OM


@pytest.mark.parametrize('lengths', [[3, 5, 2, 4], [1, 2, 1], [6]])
def test_boundary_candidates_match_oracle(lengths):
    lay = SceneLayout(lengths, halo=0)
    T = 7
    rows, scene = candidates(lay, T, 'cpu')
    ref_rows, ref_scene = OM.boundary_rows(lay.ranges, T)
    assert torch.equal(rows, ref_rows) and torch.equal(scene, ref_scene)
    frames, owner = candidate_frames(lay)
    assert len(frames) == len(set(frames)) and owner == sorted(owner)


def test_frame_plan_pieces():
    """video pieces read their scene's frames and sentence and the memory; sentence pieces their scene's frames and
    sentence; consecutive query rows are recognised (the in-place query path)"""
    lay = SceneLayout([2, 3], halo=0)
    T, S = 4, 20
    tr = [(0, 3), (3, 5)]
    p = frame_plan(lay, T, torch.arange(S), S, [(j, lo * T, hi * T) for j, (lo, hi) in enumerate(lay.ranges)], tr,
                   {0, 1}, S, 'cpu')
    assert p.host_qlen == [8, 12, 3, 2] and p.host_lens == [11, 14, 11, 14]
    assert p.q_first == [0, 8, 20, 23]
    assert p.mem.tolist() == [True, True, False, False] and p.scene.tolist() == [0, 1, 0, 1]
    assert p.pad[1, :14].tolist() == list(range(8, 20)) + [23, 24]
    assert p.cand.tolist() == [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 16, 17, 18, 19]
    assert p.owner.tolist() == [0] * 8 + [1] * 8
    q = make_plan([(0, [5, 3, 4], [1, 2], True), (1, [], [0], True)], [0], [0], 'cpu')
    assert q.q_first == [None] and q.host_qlen == [3]          # empty pieces dropped, permuted rows not in place


def test_select_has_no_cpu_path():
    with pytest.raises(TypeError, match='GPU'):
        BoundaryMemory(4).select('k', torch.randn(10, 2, 64))
    assert issubclass(L.HipTypeError, RuntimeError)


def test_sentence_pieces_read_their_video_pieces_local_rows_in_place():
    """the head-major tables on the host: a sentence piece (no memory) with its scene's local rows takes its video
    piece's key offset and packs nothing of its own; every segment's local rows (row * H + head) start at its k_off,
    and a video piece keeps room for M foreign representatives after them"""
    lay = SceneLayout([2, 3], halo=0)
    T, S, H, M = 4, 20, 2, 3
    tr = [(0, 3), (3, 5)]
    p = frame_plan(lay, T, torch.arange(S), S, [(j, lo * T, hi * T) for j, (lo, hi) in enumerate(lay.ranges)], tr,
                   {0, 1}, S, 'cpu')
    st = _Static(p, H, S + 5, 'cpu')
    assert st.share == [None, None, 0, 1]
    k_off, kidx = st.slots(M)
    assert kidx.numel() == H * sum(st.lens[i] + M for i in (0, 1))
    starts = [sum(st.lens[:i]) for i in range(st.n + 1)]
    for h in range(H):
        for i in range(st.n):
            o = int(k_off[h * st.n + i])
            assert torch.equal(kidx[o:o + st.lens[i]].long(), st.local[starts[i]:starts[i + 1]] * H + h), (h, i)
        assert int(k_off[h * st.n + 1]) - int(k_off[h * st.n]) == st.lens[0] + M


def test_plan_rows_are_checked_before_any_launch():
    """the kernels dereference key and query rows unchecked: a plan naming a negative key row, or query rows outside
    the query buffer, is rejected once per plan on the host, and the public row helpers check every call's rows"""
    from onereel_amd.scene import _check_row_range
    bad_key = make_plan([(0, [0, 1], [3, -1], True)], [0], [0], 'cpu')
    with pytest.raises(L.HipValueError, match='>= 0'):
        _Static(bad_key, 2, 4, 'cpu')
    bad_query = make_plan([(0, [5, 3, 9], [1, 2], True)], [0], [0], 'cpu')
    with pytest.raises(L.HipValueError, match='query buffer'):
        _Static(bad_query, 2, 8, 'cpu')
    _check_row_range(torch.tensor([0, 7, 3], dtype=torch.int32), 8, 'rows')
    for rows in ([0, 8], [-1, 2]):
        with pytest.raises(L.HipValueError, match='outside'):
            _check_row_range(torch.tensor(rows, dtype=torch.int32), 8, 'rows')
