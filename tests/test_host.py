"""CPU tests of the product's host side: the drop-in Python API against the reference's known answers, and the C ABI
(every declared symbol exported, the host planner's sizes against the oracle, argument errors) without a GPU."""
import ctypes
import json
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from onereel_amd import _lib as L
from onereel_amd import comm, hunyuan15 as HY
from onereel_amd.frame_memory import FrameMemory
from onereel_amd.layout import SceneLayout
from onereel_amd.scene import _desc
from oracle import layout as OL

ROOT = Path(__file__).resolve().parents[1]
GOLD = json.loads((ROOT / 'tests' / 'golden' / 'known_answers.json').read_text())
RT, HD = GOLD['reference_tests'], GOLD['hand_derived']


def _extra(d):
    return {int(j): list(v) for j, v in d.items()}


def test_layout_api_known_answers():
    g = RT['halo_order']
    lay = SceneLayout(g['lengths'], halo=2)
    assert lay.halo_frames(0) == g['halo_frames']['0'] and lay.halo_frames(1) == g['halo_frames']['1']
    assert lay.key_frames(1) == g['key_frames_1'] and list(lay.key_range(1)) == g['key_range_1']
    assert SceneLayout(g['lengths'], halo=2, sides='next').halo_frames(1) == g['next_halo_frames_1']
    assert SceneLayout.even(21, 3).lengths == RT['even_21_3']['lengths']
    assert SceneLayout.even(20, 3).scene_of_frame().tolist() == [f * 3 // 20 for f in range(20)]
    g = RT['extra_shared']
    lay = SceneLayout(g['lengths'], halo=0, extra=_extra(g['extra']))
    assert lay.shared_frames(0) == g['shared_frames_0'] and lay.key_frames(1) == g['key_frames_1']
    assert [list(x) for x in comm.runs(RT['runs']['frames'])] == RT['runs']['out']
    assert [list(x) for x in comm.frame_tokens([3, 4, 1, 2], 10)] == RT['frame_tokens']['out']
    assert comm.merge([(5, 7), (0, 2), (2, 3), (6, 9)]) == [(0, 3), (5, 9)]
    assert comm.clip([(0, 3), (5, 9)], 2, 6) == [(2, 3), (5, 6)]
    with pytest.raises(AssertionError):
        SceneLayout([2, 0])
    with pytest.raises(AssertionError):
        SceneLayout([2, 2], sides='both')


def test_frame_memory_api():
    g = RT['fallback_extra']
    lay = SceneLayout(g['lengths'], halo=0)
    fm = FrameMemory(budget=2, fallback=(1, 'adj'))
    fm.reset(lay, n_layers=8)
    assert fm.layer == 4 and lay.extra == _extra(g['extra'])
    fm.begin_step(0)
    fm.set_representatives([7, 1])
    assert lay.extra == _extra(g['extra'])
    fm.begin_step(1)
    assert lay.extra == {0: [7], 1: [1, 7], 2: [1]}
    g = RT['sink_extra']
    lay = SceneLayout(g['lengths'], halo=0)
    fm = FrameMemory(budget=3, fallback=(0, 'adj'), sink=(0,))
    fm.reset(lay, n_layers=4)
    assert lay.extra == _extra(g['extra']) and 0 not in fm.candidate_frames()
    c = FrameMemory(budget=3, candidates='boundary')
    c.reset(SceneLayout([4, 4, 4], halo=0), 4)
    assert c.candidate_frames() == [0, 3, 4, 7, 8, 11]


def test_position_helpers_known_answers():
    g = HD['shared_pos_layout']
    lay = SceneLayout(g['lengths'], halo=0, extra=_extra(g['extra']))
    ctx = HY.Context(lay, T=24, scene_rope=True)
    for j in range(4):
        assert HY.adjacent_positions(lay, j) == g['adjacent_positions'][str(j)]
        assert HY.shared_positions(ctx, j) == g['scene_rope_shared_positions'][str(j)]
    for f, p in g['scene_rope_frame_position'].items():
        assert HY.frame_position(ctx, int(f)) == p
    ctx = HY.Context(lay, shared_pos='switch', shared_switch=5, cfg=True)
    ctx.fwd = 10
    assert ctx.step() == 4 and not ctx.adjacent()
    ctx.fwd = 11
    assert ctx.step() == 5 and ctx.adjacent() and ctx.cond()


def _header_symbols(name='onereel_hip.h'):
    text = (ROOT / 'include' / name).read_text()
    return sorted(set(re.findall(r'^\s*(?:int|int64_t|const char\*)\s+(or_\w+)\s*\(', text, re.M)))


def test_library_exports_every_declared_symbol():
    syms = _header_symbols()
    h = ctypes.CDLL(str(L.LIB_PATH))
    for s in syms:
        assert hasattr(h, s), s
    assert set(syms) == set(L.SIGNATURES)
    assert L.lib().or_version().startswith(b'onereel_hip')
    # the DiT harness's kernels live in their own library, which finds the path's library beside it
    dit = _header_symbols('onereel_dit.h')
    assert dit and set(dit) == set(L.DIT_SIGNATURES) and not set(dit) & set(syms)
    for s in dit:
        assert not hasattr(h, s), s
        assert hasattr(L.dit_lib(), s), s
    # so do bench.py's measurement kernels
    bench = _header_symbols('onereel_bench.h')
    assert bench and set(bench) == set(L.BENCH_SIGNATURES) and not set(bench) & (set(syms) | set(dit))
    for s in bench:
        assert not hasattr(h, s), s
        assert hasattr(L.bench_lib(), s), s


def _random_layout(rng):
    n = int(rng.integers(1, 7))
    lengths = rng.integers(1, 6, n).tolist()
    F = sum(lengths)
    extra = {j: rng.integers(0, F, int(rng.integers(0, 4))).tolist() for j in range(n) if rng.random() < 0.7}
    return SceneLayout(lengths, halo=int(rng.integers(0, 3)), sides=['adj', 'prev', 'next'][int(rng.integers(3))],
                       extra=extra)


def test_host_planner_sizes_match_oracle():
    rng = np.random.default_rng(0)
    for _ in range(200):
        lay = _random_layout(rng)
        T = int(rng.integers(1, 9))
        counts = rng.integers(0, 5, lay.n_scenes).tolist()
        Le = sum(counts) + int(rng.integers(0, 3))
        scene_rope, adjacent, with_text = (bool(rng.integers(2)) for _ in range(3))
        d = _desc(lay, T, counts, Le, scene_rope, None, adjacent, with_text)
        sz = L.LayoutSizes()
        L.check(L.lib().or_layout_plan(ctypes.byref(d), ctypes.byref(sz)), 'plan')
        olay = OL.SceneLayout(lay.lengths, lay.halo, lay.sides, lay.extra)
        sc = OL.hunyuan_scopes(olay, T, counts if with_text else [0] * lay.n_scenes, Le, scene_rope=scene_rope,
                               adjacent=adjacent, with_text=with_text)
        assert (sz.n_seg, sz.sum_q, sz.sum_k) == (len(sc.lq), int(sc.cu_q[-1]), int(sc.cu_k[-1]))
        assert (sz.max_q, sz.max_k) == (max(sc.lq), max(sc.lk))
        rows = np.concatenate([sc.q_rope, sc.k_rope, sc.k_move_a, sc.k_move_b])
        assert sz.max_rope_row >= rows.max()
        if with_text:   # text keys read in place from the video segments: only V_j's keys are packed
            d = _desc(lay, T, counts, Le, scene_rope, None, adjacent, with_text, text_keys_in_place=True)
            s2 = L.LayoutSizes()
            L.check(L.lib().or_layout_plan(ctypes.byref(d), ctypes.byref(s2)), 'plan')
            assert (s2.n_seg, s2.sum_q, s2.max_q, s2.max_k) == (sz.n_seg, sz.sum_q, sz.max_q, sz.max_k)
            assert s2.sum_k == sum(lk for lk, kind in zip(sc.lk, sc.kind) if kind == 'v')


def test_host_planner_sizes_of_rank_shares_match_oracle():
    """q_lo / q_hi (one rank's share): segment sizes against the oracle's token_range scopes, the segments the rank
    does not run empty; ranges cut scenes mid-frame"""
    rng = np.random.default_rng(5)
    for _ in range(200):
        lay = _random_layout(rng)
        T = int(rng.integers(1, 9))
        counts = rng.integers(0, 5, lay.n_scenes).tolist()
        S = lay.n_frames * T
        a = int(rng.integers(0, S))
        b = int(rng.integers(a + 1, S + 1))
        scene_rope, adjacent, with_text, in_place = (bool(rng.integers(2)) for _ in range(4))
        in_place = in_place and with_text
        d = _desc(lay, T, counts, sum(counts), scene_rope, None, adjacent, with_text, in_place, q_range=(a, b))
        sz = L.LayoutSizes()
        L.check(L.lib().or_layout_plan(ctypes.byref(d), ctypes.byref(sz)), 'plan')
        olay = OL.SceneLayout(lay.lengths, lay.halo, lay.sides, lay.extra)
        sc = OL.hunyuan_scopes(olay, T, counts if with_text else [0] * lay.n_scenes, sum(counts),
                               scene_rope=scene_rope, adjacent=adjacent, with_text=with_text, token_range=(a, b))
        assert sz.n_seg == lay.n_scenes * (2 if with_text else 1)
        assert (sz.sum_q, sz.max_q, sz.max_k) == (int(sc.cu_q[-1]), max(sc.lq), max(sc.lk))
        packed = [lk for lk, kind in zip(sc.lk, sc.kind) if kind == 'v' or not in_place]
        assert sz.sum_k == sum(packed)


def test_query_range_errors():
    lay = SceneLayout([2, 3], halo=0)
    for q_range, msg in (((3, 3), 'query range'), ((-1, 4), 'query range'), ((0, 21), 'query range'),
                         ((2, 0), 'q_lo / q_hi'), ((0, -1), 'q_lo / q_hi')):
        d = _desc(lay, 4, [1, 1], 2, False, None, False, True, q_range=q_range)
        with pytest.raises(L.HipPathError, match=msg):
            L.check(L.lib().or_layout_plan(ctypes.byref(d), ctypes.byref(L.LayoutSizes())), 'or_layout_plan')


def test_text_keys_in_place_needs_text_scopes():
    d = _desc(SceneLayout([2, 3], halo=0), 4, [1, 1], 2, False, None, False, False)
    d.text_keys_in_place = 1
    with pytest.raises(L.HipPathError, match='text_keys_in_place'):
        L.check(L.lib().or_layout_plan(ctypes.byref(d), ctypes.byref(L.LayoutSizes())), 'or_layout_plan')


@pytest.mark.parametrize('bad, msg', [
    (dict(extra={0: [9]}), 'extra frame 9'),
    (dict(T=0), 'T must be positive'),
    (dict(counts=[5, 5], Le=4), 'text counts'),
    (dict(n=65), 'scenes'),
])
def test_layout_argument_errors(bad, msg):
    n = bad.get('n', 2)
    if n > 64:
        with pytest.raises(ValueError, match=msg):
            _desc(SceneLayout([1] * n, halo=0), 4, [0] * n, 0, False, None, False, True)
        return
    lay = SceneLayout([2, 3], halo=0, extra=bad.get('extra', {}))
    d = _desc(lay, bad.get('T', 4), bad.get('counts', [1, 1]), bad.get('Le', 2), False, None, False, True)
    with pytest.raises(L.HipPathError, match=msg):
        L.check(L.lib().or_layout_plan(ctypes.byref(d), ctypes.byref(L.LayoutSizes())), 'or_layout_plan')


def test_varlen_argument_errors_without_gpu():
    a = L.VarlenArgs()
    a.D, a.H, a.n_seg = 96, 1, 1
    with pytest.raises(L.HipPathError, match='head_dim 96'):
        L.check(L.lib().or_varlen_fwd(ctypes.byref(a), None), 'or_varlen_fwd')
    a.D = 128
    with pytest.raises(L.HipPathError, match='required'):
        L.check(L.lib().or_varlen_fwd(ctypes.byref(a), None), 'or_varlen_fwd')
    with pytest.raises(L.HipPathError, match='H\\*D'):
        L.check(L.lib().or_pack_gather(1, 1, None, None, 4096, 4096, 0, 1, None, None, None, None, 0, 1, 64, 128, 1,
                                       None, None), 'or_pack_gather')
    assert L.lib().or_varlen_workspace_size(8, 51392, 16, 128) > 0


def test_product_has_no_cpu_fallback():
    """the product package never imports the oracle, and its compute entry points refuse CPU tensors"""
    for p in (ROOT / 'onereel_amd').rglob('*.py'):
        assert not re.search(r'^\s*(from|import)\s+oracle', p.read_text(), re.M), p
    from onereel_amd import scene
    x = torch.zeros(4, 2, 64, dtype=torch.bfloat16)
    with pytest.raises(TypeError, match='GPU'):
        scene.varlen(x, x, x, torch.zeros(2, dtype=torch.int32), torch.zeros(2, dtype=torch.int32), 4, 4)


def test_argument_errors_are_runtime_errors():
    """as FlashAttention's argument and dtype errors are RuntimeErrors, so are the host layer's (they are also
    ValueError / TypeError)"""
    from onereel_amd import attention as A
    from onereel_amd import scene
    x = torch.zeros(4, 2, 64, dtype=torch.float32)
    for call in (lambda: scene.varlen(x, x, x, torch.zeros(2, dtype=torch.int32), torch.zeros(2, dtype=torch.int32),
                                      4, 4),
                 lambda: A.merge_lse(torch.zeros(3, 2, 8, dtype=torch.bfloat16), torch.zeros(2, 3), x, x),
                 lambda: A.overlapping_ranges(x, x, x, [(1, 4)], [(0, 4)])):
        with pytest.raises(RuntimeError) as e:
            call()
        assert isinstance(e.value, (ValueError, TypeError)), type(e.value)



def test_rotate_and_memory_argument_errors_without_gpu():
    """or_rotate_rows, or_memory_select and or_memory_index refuse bad shapes, missing arrays, short strides and
    misaligned buffers before they launch anything (device pointers are never dereferenced on the host)"""
    rot = L.lib().or_rotate_rows
    x, idx, rope, cos, sin, out = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 0x60000

    def rotate(x=x, xs=2048, rope=rope, cos=cos, n_rope=100, H=16, D=128, out=out, os_=2048):
        return L.check(rot(x, xs, 10, idx, rope, cos, sin, n_rope, 12, H, D, out, os_, None), 'or_rotate_rows')
    for kw, msg in ((dict(D=12), 'multiple of 8'), (dict(H=64, D=128), 'exceed'), (dict(rope=None), 'required'),
                    (dict(cos=None), 'required'), (dict(n_rope=0), 'required'), (dict(xs=1024), 'cover H \\* D'),
                    (dict(os_=2040), 'cover H \\* D'), (dict(x=x + 8), '16-byte aligned'),
                    (dict(out=out + 2), '16-byte aligned')):
        with pytest.raises(L.HipPathError, match=msg):
            rotate(**kw)
    assert rot(x, 2048, 10, idx, rope, cos, sin, 100, 0, 16, 128, out, 2048, None) == 0   # nothing to do
    sel = L.lib().or_memory_select
    keys, rows, cent, rep, valid, ws = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000, 0x100000

    def select(B=100, H=2, D=128, M=8, iters=2, keys=keys, stride=256, ws=ws, wsb=1 << 30):
        return L.check(sel(keys, 1, rows, stride, B, H, D, M, cent, None, iters, rep, valid, ws, wsb, None),
                       'or_memory_select')
    for kw, msg in ((dict(D=96), 'D 64 or 128'), (dict(M=101), 'outside'), (dict(M=0), 'outside'),
                    (dict(iters=-1), 'iters'), (dict(keys=None), 'required'), (dict(stride=128), 'required'),
                    (dict(ws=ws + 64), 'aligned workspace'), (dict(wsb=16), 'aligned workspace'),
                    (dict(keys=keys + 4), '16-byte aligned')):
        with pytest.raises(L.HipPathError, match=msg):
            select(**kw)
    idxf = L.lib().or_memory_index
    a = 0x10000
    with pytest.raises(L.HipPathError, match='pieces, heads'):
        L.check(idxf(a, a, a, a, a, a, a, a, 0, 2, 8, a, a, None), 'or_memory_index')
    with pytest.raises(L.HipPathError, match='every array'):
        L.check(idxf(a, a, None, a, a, a, a, a, 3, 2, 8, a, a, None), 'or_memory_index')


def test_fused_residual_layernorm_argument_errors_without_gpu():
    """or_residual_layernorm_modulate (libonereel_dit.so) refuses bad widths, a missing or misaligned addend and an
    output that is x or a before it launches anything (device pointers are never dereferenced on the host); its
    messages come through the path library's or_last_error"""
    f = L.dit_lib().or_residual_layernorm_modulate
    x, a, out = 0x10000, 0x20000, 0x30000

    def call(x=x, a=a, out=out, C=512, a_stride=512):
        return L.dit_check(f(x, a, None, out, 4, C, C, a_stride, C, 1e-6, None, None, None, None, None),
                       'or_residual_layernorm_modulate')
    for kw, msg in ((dict(C=100), 'multiple of 8'), (dict(C=9000), 'multiple of 8'), (dict(a=None), 'a must be'),
                    (dict(a=a + 8), 'a must be'), (dict(a_stride=256), 'a must be'), (dict(out=x), 'must not be'),
                    (dict(out=a), 'must not be'), (dict(x=x + 4), '16-byte aligned')):
        with pytest.raises(L.HipPathError, match=msg):
            call(**kw)


def test_mfma_ceiling_argument_errors_without_gpu():
    """or_mfma_ceiling (libonereel_bench.so) refuses missing or misaligned buffers, a bad operand count, grid,
    iteration count or mode before it launches anything"""
    f = L.bench_lib().or_mfma_ceiling
    ops, out = 0x10000, 0x20000

    def call(ops=ops, n=64, out=out, blocks=256, iters=800, mode=0):
        return L.bench_check(f(ops, n, out, blocks, iters, mode, None), 'or_mfma_ceiling')
    for kw, msg in ((dict(ops=None), 'required'), (dict(out=None), 'required'), (dict(n=0), 'n_vec'),
                    (dict(ops=ops + 8), 'aligned'), (dict(out=out + 2), 'aligned'), (dict(blocks=0), 'blocks'),
                    (dict(blocks=70000), 'blocks'), (dict(iters=12), 'multiple of 8'), (dict(iters=0), 'multiple of 8'),
                    (dict(mode=3), 'mode')):
        with pytest.raises(L.HipPathError, match=msg):
            call(**kw)


def test_generated_key_loop_is_current(tmp_path):
    """the tracked asm key loop of the 64-query attention kernel is exactly what its generator writes (the build
    regenerates it; a stale tracked copy would differ from the code that runs)"""
    import subprocess
    import sys
    csrc = ROOT / 'onereel_amd' / 'csrc'
    out = tmp_path / 'attn_ring64.inc'
    subprocess.run([sys.executable, str(csrc / 'gen_attn_ring64.py'), '--out', str(out)], check=True)
    assert out.read_bytes() == (csrc / 'attn_ring64.inc').read_bytes()


def test_plan_workspace_is_per_head_count_and_head_dim():
    """ScopePlan.workspace keys its buffer on (heads, head_dim): the size or_varlen_fwd needs depends on both, so a
    plan reused at another head_dim gets a buffer of that size (no GPU: the buffer is allocated on the CPU here)"""
    from onereel_amd.scene import ScopePlan
    plan = ScopePlan.__new__(ScopePlan)
    plan.n_seg, plan.sum_q, plan.device, plan._ws = 8, 700, torch.device('cpu'), {}
    sizes = {(H, D): int(L.lib().or_varlen_workspace_size(8, 700, H, D)) for H, D in ((16, 64), (16, 128), (4, 128))}
    assert sizes[(16, 64)] != sizes[(16, 128)]
    for (H, D), n in sizes.items():
        assert plan.workspace(H, D).numel() == n
    assert plan.workspace(16, 64) is plan.workspace(16, 64)


def test_host_api_agrees_with_oracle_on_random_layouts():
    """the product's host API (SceneLayout frame lists, comm runs, RoPE position helpers, FrameMemory extras) against
    the oracle on random layouts: repeated and out-of-range-of-scene extra frames, every halo side, scene RoPE over
    other scene lengths"""
    rng = np.random.default_rng(11)
    for _ in range(400):
        n = int(rng.integers(1, 7))
        lengths = rng.integers(1, 6, n).tolist()
        F = sum(lengths)
        extra = {j: rng.integers(0, F, int(rng.integers(0, 6))).tolist() for j in range(n) if rng.random() < 0.8}
        halo, sides = int(rng.integers(0, 4)), ['adj', 'prev', 'next'][int(rng.integers(3))]
        rl = None
        if rng.random() < 0.3:
            rl, left = [], F
            while left > 0:
                rl.append(int(rng.integers(1, left + 1)))
                left -= rl[-1]
        lay, olay = SceneLayout(lengths, halo, sides, extra), OL.SceneLayout(lengths, halo, sides, extra)
        assert lay.ranges == olay.ranges and lay.frames == olay.frames
        for j in range(n):
            assert lay.halo_frames(j) == olay.halo_frames(j) and lay.shared_frames(j) == olay.shared_frames(j)
            assert lay.key_frames(j) == olay.key_frames(j)
            kf = olay.key_frames(j)
            assert lay.key_range(j) == (min(kf), max(kf) + 1)
            assert [tuple(r) for r in comm.runs(kf)] == [tuple(r) for r in OL.runs(kf)]
        for scene_rope in (False, True):
            ctx = HY.Context(lay, scene_rope=scene_rope, rope_lengths=rl)
            for j in range(n):
                assert HY.adjacent_positions(lay, j) == OL.adjacent_positions(olay, j)
                assert HY.shared_positions(ctx, j) == OL.shared_positions(olay, j, scene_rope, rl)
            assert [HY.frame_position(ctx, f) for f in range(F)] == [OL.frame_position(olay, f, scene_rope, rl)
                                                                     for f in range(F)]
        reps = sorted(set(rng.integers(0, F, 3).tolist()))
        sink = tuple(sorted(set(rng.integers(0, F, int(rng.integers(0, 2))).tolist())))
        fm = FrameMemory(budget=4, fallback=(int(rng.integers(0, 3)), sides), sink=sink)
        fm.reset(SceneLayout(lengths, halo=0), 4)
        om = OL.FrameMemoryExtra(budget=4, fallback=fm.fallback, sink=sink)
        olay0 = OL.SceneLayout(lengths, 0)
        om.reset(olay0)
        assert fm.layout.extra == olay0.extra
        fm.set_representatives(reps)
        fm.begin_step(1)
        om.propose(reps)
        om.begin_step(1)
        assert fm.layout.extra == olay0.extra
    for F in range(1, 30):
        for k in range(1, F + 1):
            sc = [f * k // F for f in range(F)]
            assert SceneLayout.even(F, k).lengths == [sc.count(j) for j in range(k)]


def test_partition_known_answers():
    """rank token ranges against the reference's own known answers: equal scenes split at the scene boundary, a
    boundary that falls inside a frame, Algorithm 1's invariants for 2, 3, 4 and 8 ranks (contiguous ranges, at most
    n - 1 cut scenes, every rank within one query's cost of the mean work), the clamp that keeps a query per rank,
    and the equal Ulysses split"""
    g = RT['partition_equal_scenes']
    lay = SceneLayout(g['lengths'], halo=g['halo'])
    assert [list(x) for x in comm.partition(lay, g['n'], g['T'], 'scene')] == g['own']
    g = RT['partition_mid_frame']
    lay = SceneLayout(g['lengths'], halo=g['halo'])
    b = comm.partition(lay, g['n'], g['T'], 'scene')[0][1]
    assert g['boundary_above'] < b < g['boundary_below'] and b % g['T'] != 0
    assert [list(x) for x in comm.partition(lay, g['n'], g['T'], 'ulysses')] == g['ulysses']
    g = RT['partition_invariants']
    lay, T = SceneLayout(g['lengths'], halo=g['halo']), g['T']
    cost = comm.query_cost(lay, T)
    per_token = np.concatenate([[c] * (m * T) for c, m in zip(cost, lay.lengths)])
    for n in g['ranks']:
        own = comm.partition(lay, n, T, 'scene')
        assert own[0][0] == 0 and own[-1][1] == lay.n_frames * T
        assert all(x[1] == y[0] and x[0] < x[1] for x, y in zip(own, own[1:]))
        assert sum(any(lo * T < x[0] < hi * T for x in own) for lo, hi in lay.ranges) <= n - 1
        work = [per_token[a:b].sum() for a, b in own]
        assert max(abs(w - sum(work) / n) for w in work) <= per_token.max() + 1e-9
    g = RT['balanced_clamp']
    assert [list(x) for x in comm.balanced(g['sizes'], g['cost'], g['n'])] == g['own']


def test_partition_against_brute_force():
    """Algorithm 1 on random scene sizes and costs against a direct search over every query: boundary p is the query
    nearest to where the running work reaches p / n of the total (work measured in whole queries of the scene the
    goal falls in), clamped to keep a query per rank; the 'scenes' granularity cuts only at scene starts, and 'tokens'
    splits evenly"""
    rng = np.random.default_rng(3)
    for _ in range(300):
        k = int(rng.integers(1, 7))
        sizes = rng.integers(1, 30, k).tolist()
        cost = (rng.random(k) * 3 + 0.1).tolist()
        n = int(rng.integers(1, min(sum(sizes), 6) + 1))
        own = comm.balanced(sizes, cost, n)
        L_ = sum(sizes)
        per = np.repeat(cost, sizes)
        cw = np.concatenate([[0.0], np.cumsum(per)])    # work before query t
        b = [0]
        for p in range(1, n):
            goal = p * cw[-1] / n
            # queries whose start lies in the scene holding the goal, nearest by work
            j = min(int(np.searchsorted(np.cumsum(np.asarray(sizes) * cost), goal - 1e-9)), k - 1)
            lo = sum(sizes[:j])
            cand = np.arange(lo, lo + sizes[j] + 1)
            at = int(cand[np.argmin(np.abs(cw[cand] - goal))])
            b.append(min(max(at, b[-1] + 1), L_ - (n - p)))
        b.append(L_)
        exp = list(zip(b[:-1], b[1:]))
        # a goal half-way between two queries may round either way: allow one query of difference there
        assert all(abs(x[0] - y[0]) <= 1 for x, y in zip(own, exp)), (sizes, cost, n, own, exp)
        assert own[0][0] == 0 and own[-1][1] == L_ and all(x[0] < x[1] for x in own)
    lay = SceneLayout([3, 5, 7, 9], halo=1)
    sc = comm.partition(lay, 3, 10, 'scene', granularity='scenes')
    assert all(a in (0, 30, 80, 150) for a, _ in sc) and len({a for a, _ in sc}) == 3
    assert comm.partition(lay, 3, 10, 'scene', granularity='tokens') == [(0, 80), (80, 160), (160, 240)]
    with pytest.raises(ValueError):
        comm.partition(lay, 7, 10, 'ulysses')


def test_bench_refuses_several_gpus_and_bad_shares():
    """bench.py measures one GPU: --gpus above 1 exits with status 2 and says so, before touching a GPU; a rank share
    outside [0, P) is an argument error"""
    import subprocess
    import sys
    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / 'bench.py'), '--gpus', '2'], capture_output=True, text=True,
                       timeout=300, cwd=root)
    assert r.returncode == 2 and 'single-GPU' in r.stdout + r.stderr
    r = subprocess.run([sys.executable, str(root / 'bench.py'), '--share', '3/3', '--no-cpu'], capture_output=True,
                       text=True, timeout=300, cwd=root)
    assert r.returncode != 0 and 'rank R in [0, P)' in r.stdout + r.stderr


def test_abi_structs_match_the_header(tmp_path):
    """the ctypes argument structs have the C header's field offsets and sizes (gcc on the header itself)"""
    import shutil
    import subprocess
    if shutil.which('gcc') is None:
        pytest.skip('needs gcc')
    pairs = [('or_layout_desc', L.LayoutDesc), ('or_layout_sizes', L.LayoutSizes), ('or_layout_out', L.LayoutOut),
             ('or_varlen_args', L.VarlenArgs), ('or_pack_args', L.PackArgs)]
    lines = ['#include <stddef.h>', '#include <stdio.h>', f'#include "{ROOT / "include" / "onereel_hip.h"}"',
             'int main(void) {']
    for cname, cls in pairs:
        lines.append(f'  printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for f in cls._fields_:
            lines.append(f'  printf("{cname} {f[0]} %zu\\n", offsetof({cname}, {f[0]}));')
    lines += ['  return 0;', '}']
    src, exe = tmp_path / 'abi.c', tmp_path / 'abi'
    src.write_text('\n'.join(lines) + '\n')
    subprocess.run(['gcc', '-std=c11', '-o', str(exe), str(src)], check=True)
    got = dict(l.rsplit(' ', 1) for l in subprocess.run([str(exe)], check=True, capture_output=True,
                                                        text=True).stdout.splitlines())
    for cname, cls in pairs:
        assert int(got[f'{cname} sizeof']) == ctypes.sizeof(cls), cname
        for f in cls._fields_:
            assert int(got[f'{cname} {f[0]}']) == getattr(cls, f[0]).offset, (cname, f[0])


def test_drop_in_varlen_rejects_bad_offsets_and_ranges_without_gpu():
    """attention.varlen / varlen_lse / overlapping_ranges check caller offsets and key ranges on the host before any
    launch: the kernels index q / k / v rows by them without bounds checks"""
    import torch
    from onereel_amd import attention as A
    q = torch.zeros(10, 2, 64, dtype=torch.bfloat16)
    k = torch.zeros(12, 2, 64, dtype=torch.bfloat16)
    cu = lambda *x: torch.tensor(x, dtype=torch.int32)
    A.check_cu_seqlens(cu(0, 4, 10), 10, 6, 'cu_q')          # good offsets pass
    for c, n, mx, msg in ((cu(1, 4, 10), 10, 9, 'start at 0'), (cu(0, 5, 3), 10, 9, 'not decrease'),
                          (cu(0, 4, 11), 10, 9, 'at most at 10'), (cu(0, 4, 10), 10, 5, 'exceeds'),
                          (cu(0), 10, 9, 'at least 2')):
        with pytest.raises(L.HipValueError, match=msg):
            A.check_cu_seqlens(c, n, mx, 'cu_q')
    with pytest.raises(L.HipValueError, match='cu_k'):
        A.varlen(q, k, k, cu(0, 4, 10), cu(0, 6, 13), 6, 7)
    with pytest.raises(L.HipValueError, match='one offset per segment'):
        A.varlen_lse(q, k, k, cu(0, 4, 10), cu(0, 12), 6, 12)
    with pytest.raises(L.HipValueError, match='inside the 12 rows'):
        A.overlapping_ranges(q, k, k, [(0, 4), (4, 10)], [(0, 6), (6, 13)])
    with pytest.raises(L.HipValueError, match='inside the 12 rows'):
        A.overlapping_ranges(q, k, k, [(0, 4), (4, 10)], [(5, 3), (0, 2)])
    with pytest.raises(L.HipValueError, match='pair up'):
        A.overlapping_ranges(q, k, k, [(0, 4), (4, 10)], [(0, 6)])
