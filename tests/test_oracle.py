"""Pins the CPU oracle (oracle/) before it is trusted as the checker of the HIP path.

Sources of truth, none of them the oracle's own formulas: the reference's test known answers and hand-derived values
(tests/golden/known_answers.json), textbook identities (complex multiplication for RoPE, an explicit float64 softmax
for attention), the reference's RoPE-composition invariant (tests/test_shared_pos.py of the reference), and a brute-
force masked attention over the scope definition (src/onereel/README.md:11-15).
"""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import layout as OL

GOLD = json.loads((Path(__file__).parent / 'golden' / 'known_answers.json').read_text())
RT, HD = GOLD['reference_tests'], GOLD['hand_derived']


def _extra(d):
    return {int(j): list(v) for j, v in d.items()}


# ---------------------------------------------------------------------------------------------- layout known answers
def test_even_and_scene_of_frame():
    g = RT['even_21_3']
    assert OL.SceneLayout.even(g['n_frames'], g['n_scenes']).lengths == g['lengths']
    assert OL.SceneLayout.even(20, 3).scene_of_frame() == [f * 3 // 20 for f in range(20)]


def test_halo_order_and_sides():
    g = RT['halo_order']
    lay = OL.SceneLayout(g['lengths'], halo=g['halo'])
    for j, exp in g['halo_frames'].items():
        assert lay.halo_frames(int(j)) == exp
    assert lay.key_frames(1) == g['key_frames_1']
    assert list(lay.key_range(1)) == g['key_range_1']
    assert OL.SceneLayout(g['lengths'], halo=2, sides='next').halo_frames(1) == g['next_halo_frames_1']
    assert OL.SceneLayout(g['lengths'], halo=2, sides='prev').halo_frames(1) == g['prev_halo_frames_1']
    assert OL.SceneLayout(RT['halo_zero']['lengths'], halo=0).halo_frames(0) == []


def test_runs_and_frame_tokens():
    assert [list(r) for r in OL.runs(RT['runs']['frames'])] == RT['runs']['out']
    g = RT['frame_tokens']
    assert [list(r) for r in OL.frame_tokens(g['frames'], g['T'])] == g['out']


def test_shared_frames_with_extra():
    g = RT['extra_shared']
    lay = OL.SceneLayout(g['lengths'], halo=0, extra=_extra(g['extra']))
    assert lay.shared_frames(0) == g['shared_frames_0']
    assert lay.key_frames(1) == g['key_frames_1']
    assert lay.shared_frames(2) == g['shared_frames_2']


@pytest.mark.parametrize('name', ['fallback_extra', 'sink_extra'])
def test_frame_memory_fallback(name):
    g = RT[name]
    lay = OL.SceneLayout(g['lengths'], halo=0)
    fm = OL.FrameMemoryExtra(budget=g['budget'], fallback=tuple(g['fallback']), sink=tuple(g['sink']))
    fm.reset(lay)
    assert lay.extra == _extra(g['extra'])


def test_frame_memory_next_step_applies_reps():
    """tests/test_onereel_frame_memory.py:19-36: same step unchanged, next step extra[j] = reps outside scene j"""
    lay = OL.SceneLayout([3, 3, 3], halo=0)
    fm = OL.FrameMemoryExtra(budget=2, fallback=(1, 'adj'))
    fm.reset(lay)
    fm.begin_step(0)
    fm.propose([7, 1])
    assert lay.extra == {0: [3], 1: [2, 6], 2: [5]}
    fm.begin_step(1)
    assert fm.history[-1] == [1, 7]
    for j, (lo, hi) in enumerate(lay.ranges):
        assert lay.extra[j] == [f for f in [1, 7] if not lo <= f < hi]


def test_hunyuan480p_extra_from_reps():
    g = HD['hunyuan480p_4x8x1590']
    lay = OL.SceneLayout(g['lengths'], halo=0)
    fm = OL.FrameMemoryExtra(budget=4, fallback=(0, 'adj'))
    fm.reset(lay)
    fm.propose(g['reps'])
    fm.begin_step(1)
    assert lay.extra == _extra(g['extra'])
    assert [list(x) for x in OL.frame_tokens(lay.key_frames(0), g['T'])] == g['key_frame_tokens_0']


def test_shared_repeat_kept_as_reference():
    """layout.py:69 filters extra[j] against the halo list only: a repeated extra frame stays repeated"""
    lay = OL.SceneLayout([2, 2, 2], halo=1, extra={0: [5, 5, 2, 0]})
    assert lay.shared_frames(0) == [2, 5, 5]


# ---------------------------------------------------------------------------------------------- positions
def test_positions_hand_derived():
    g = HD['shared_pos_layout']
    lay = OL.SceneLayout(g['lengths'], halo=0, extra=_extra(g['extra']))
    for j in range(lay.n_scenes):
        assert lay.shared_frames(j) == g['shared_frames'][str(j)]
        assert OL.adjacent_positions(lay, j) == g['adjacent_positions'][str(j)]
        assert OL.shared_positions(lay, j, False) == g['adjacent_positions'][str(j)]
        assert OL.shared_positions(lay, j, True) == g['scene_rope_shared_positions'][str(j)]
    for f, p in g['scene_rope_frame_position'].items():
        assert OL.frame_position(lay, int(f), True) == p
    assert OL.frame_position(lay, 17, False) == 17


def test_scene_rope_rows_hand_and_brute():
    g = HD['scene_rope_rows_3_3_T2']
    assert OL.scene_rope_rows(OL.SceneLayout(g['lengths'], halo=0), g['T']).tolist() == g['rows']
    lay = OL.SceneLayout([5, 2, 4], halo=0)
    rows = OL.scene_rope_rows(lay, 3)
    brute = [OL.frame_position(lay, t // 3, True) * 3 + t % 3 for t in range(lay.n_frames * 3)]
    assert rows.tolist() == brute


def test_adjacent_positions_with_repeats():
    """a repeated shared frame takes the position of its last occurrence (dict semantics, hunyuan15.py:98-100)"""
    lay = OL.SceneLayout([3, 3, 3], halo=0, extra={1: [0, 0, 7]})
    assert lay.shared_frames(1) == [0, 0, 7]
    assert OL.adjacent_positions(lay, 1) == [2, 2, 6]
    assert OL.shared_positions(lay, 1, True) == [5, 5, 6]


# ---------------------------------------------------------------------------------------------- scopes
@pytest.mark.parametrize('variant', ['scene_rope_adjacent', 'scene_rope_source', 'global_adjacent'])
def test_tiny_scopes_hand_derived(variant):
    g = HD['tiny_scopes']
    lay = OL.SceneLayout(g['lengths'], halo=g['halo'], extra=_extra(g['extra']))
    sc = OL.hunyuan_scopes(lay, g['T'], g['counts'], g['text_rows'], scene_rope=variant.startswith('scene'),
                           adjacent=variant.endswith('adjacent'))
    assert sc.lq == g['lq'] and sc.lk == g['lk']
    assert sc.cu_q.tolist() == g['cu_q'] and sc.cu_k.tolist() == g['cu_k']
    assert sc.q_src.tolist() == g['q_src'] and sc.k_src.tolist() == g['k_src']
    exp = g[variant]
    assert sc.q_rope.tolist() == exp['q_rope']
    assert sc.k_rope.tolist() == exp['k_rope']
    if 'k_move_a' in exp:
        assert sc.k_move_a.tolist() == exp['k_move_a'] and sc.k_move_b.tolist() == exp['k_move_b']


def test_config_scope_sizes():
    g = HD['cpu_plumbing_2x3x64']
    sc = OL.hunyuan_scopes(OL.SceneLayout(g['lengths'], halo=0, extra=_extra(g['extra'])), g['T'], g['counts'])
    assert sc.lq == g['lq'] and sc.lk == g['lk']
    assert OA.useful_flops(sc.lq, sc.lk, 2, 64) == pytest.approx(g['useful_flop_H2_D64'], rel=1e-3)
    g = HD['hunyuan480p_4x8x1590']
    sc = OL.hunyuan_scopes(OL.SceneLayout(g['lengths'], halo=0, extra=_extra(g['extra'])), g['T'], g['counts'],
                           scene_rope=True, adjacent=True)
    assert sc.cu_q.tolist() == g['cu_q'] and sc.cu_k.tolist() == g['cu_k']
    assert (sc.max_q, sc.max_k) == (g['max_q'], g['max_k'])
    assert OA.useful_flops(sc.lq, sc.lk, 16, 128) == pytest.approx(g['useful_flop_H16_D128'], rel=1e-4)
    g = HD['wan704_3x11x880']
    lay = OL.SceneLayout(g['lengths'], halo=g['halo'], sides=g['sides'])
    sc = OL.hunyuan_scopes(lay, g['T'], g['counts'])
    assert sc.lq == g['lq'] and sc.lk == g['lk']
    _, kr = OL.wan_ranges(lay, g['T'])
    assert [[a // g['T'], b // g['T']] for a, b in kr] == g['wan_k_ranges_frames']
    g = HD['uneven_K12']
    rng = np.random.default_rng(12)
    lengths = rng.integers(2, 17, 12).tolist()
    text = rng.integers(64, 257, 12).tolist()
    assert lengths == g['lengths']
    F = sum(lengths)
    reps = sorted({int(x) for x in np.linspace(0, F - 1, 4).round()})
    lay = OL.SceneLayout(lengths, halo=0)
    fm = OL.FrameMemoryExtra(budget=4, fallback=(0, 'adj'))
    fm.reset(lay)
    fm.propose(reps)
    fm.begin_step(1)
    sc = OL.hunyuan_scopes(lay, 1590, text)
    assert (int(sc.cu_q[-1]), int(sc.cu_k[-1])) == (g['sum_lq'], g['sum_lk'])
    assert OA.useful_flops(sc.lq, sc.lk, 16, 128) == pytest.approx(g['useful_flop_H16_D128'], rel=1e-3)


def test_scopes_brute_force_membership():
    """every packed key row of V_j is a token of key_frames(j) or of sentence j, in the order own frames, shared
    frames, text; every video token is a query of exactly one scope"""
    lay = OL.SceneLayout([3, 4, 2], halo=1, sides='adj', extra={0: [8], 2: [0, 1]})
    T, counts = 3, [2, 0, 3]
    sc = OL.hunyuan_scopes(lay, T, counts, 7)
    S = lay.n_frames * T
    assert sorted(sc.q_src[sc.q_src < S].tolist()) == list(range(S))
    tr = OL.text_ranges(counts)
    for s, (kind, j) in enumerate(zip(sc.kind, sc.scene)):
        keys = sc.k_src[sc.cu_k[s]:sc.cu_k[s + 1]].tolist()
        frames = lay.key_frames(j) if kind == 'v' else lay.frames[j]
        exp = [f * T + x for f in frames for x in range(T)] + [S + t for t in range(*tr[j])]
        assert keys == exp


def test_rank_shares_partition_the_one_gpu_scopes():
    """token_range: for any split of the video tokens into rank ranges, the ranks' video segments of a scene, in rank
    order, hold exactly that scene's one-GPU queries and each the scene's one-GPU keys (rows and RoPE / move rows);
    every sentence segment appears on exactly one rank (the one holding its scene's first token), equal to the
    one-GPU one; the range covering every token gives the one-GPU scopes"""
    rng = np.random.default_rng(11)
    for it in range(40):
        n = int(rng.integers(1, 6))
        lengths = rng.integers(1, 5, n).tolist()
        F = sum(lengths)
        extra = {j: rng.integers(0, F, int(rng.integers(0, 3))).tolist() for j in range(n) if rng.random() < 0.6}
        lay = OL.SceneLayout(lengths, int(rng.integers(0, 3)), ['adj', 'prev', 'next'][int(rng.integers(3))], extra)
        T = int(rng.integers(1, 7))
        counts = rng.integers(0, 4, n).tolist()
        kw = dict(scene_rope=bool(rng.integers(2)), adjacent=bool(rng.integers(2)))
        S = F * T
        full = OL.hunyuan_scopes(lay, T, counts, **kw)
        whole = OL.hunyuan_scopes(lay, T, counts, token_range=(0, S), **kw)
        for a in ('cu_q', 'cu_k', 'q_src', 'k_src', 'q_rope', 'k_rope', 'k_move_a', 'k_move_b'):
            assert np.array_equal(getattr(full, a), getattr(whole, a)), a
        P = int(rng.integers(1, min(S, 5) + 1))
        cuts = sorted(rng.choice(np.arange(1, S), P - 1, replace=False).tolist()) if P > 1 else []
        bounds = [0] + cuts + [S]
        seg = lambda sc, i, a, cu: np.asarray(getattr(sc, a))[sc.__dict__[cu][i]:sc.__dict__[cu][i + 1]]
        ref = {(k, j): i for i, (k, j) in enumerate(zip(full.kind, full.scene))}
        rope_of = dict(zip(full.q_src.tolist(), full.q_rope.tolist()))     # every query row appears once
        got_q = {key: [] for key in ref}
        for r in range(P):
            sh = OL.hunyuan_scopes(lay, T, counts, token_range=(bounds[r], bounds[r + 1]), **kw)
            for i, key in enumerate(zip(sh.kind, sh.scene)):
                rows = seg(sh, i, 'q_src', 'cu_q')
                got_q[key].append(rows)
                assert seg(sh, i, 'q_rope', 'cu_q').tolist() == [rope_of[x] for x in rows.tolist()], key
                for a in ('k_src', 'k_rope', 'k_move_a', 'k_move_b'):
                    assert np.array_equal(seg(sh, i, a, 'cu_k'), seg(full, ref[key], a, 'cu_k')), (key, a)
        for key, i in ref.items():
            parts = got_q[key]
            assert len(parts) >= 1 and (key[0] == 'v' or len(parts) == 1), key
            assert np.array_equal(np.concatenate(parts), seg(full, i, 'q_src', 'cu_q')), key


# ---------------------------------------------------------------------------------------------- RoPE
def test_rope_matches_complex_multiplication():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(40, 3, 16, generator=g)
    ang = torch.rand(40, 8, generator=g) * 6.0
    cos, sin = ang.cos().repeat_interleave(2, 1), ang.sin().repeat_interleave(2, 1)
    out = OA.apply_rotary_emb(x, cos, sin)
    z = torch.view_as_complex(x.double().reshape(40, 3, 8, 2).contiguous())
    w = torch.polar(torch.ones(40, 8, dtype=torch.float64), ang.double())[:, None]
    ref = torch.view_as_real(z * w).reshape(40, 3, 16)
    assert (out.double() - ref).abs().max() < 1e-5
    assert OA.apply_rotary_emb(x.bfloat16(), cos, sin).dtype == torch.bfloat16


@pytest.mark.parametrize('scene_rope', [False, True])
def test_move_shared_composition_invariant(scene_rope):
    """tests/test_shared_pos.py of the reference: a shared key rotated at its own frame and moved by _move_shared
    equals the key rotated at its adjacent position (max err < 1e-4, fp32), on its synthetic 3D table"""
    cos, sin = OA.rope_table_3d(30, 4, 6, 128)
    T = 24
    g = HD['shared_pos_layout']
    lay = OL.SceneLayout(g['lengths'], halo=0, extra=_extra(g['extra']))
    sc = OL.hunyuan_scopes(lay, T, [0] * 4, 0, scene_rope=scene_rope, adjacent=True, with_text=False)
    src_rows = torch.as_tensor(OL.scene_rope_rows(lay, T) if scene_rope else np.arange(lay.n_frames * T))
    gen = torch.Generator().manual_seed(0)
    k0 = torch.randn(int(sc.cu_k[-1]), 2, 128, generator=gen)
    ksrc = torch.as_tensor(sc.k_src)
    rotated = OA.apply_rotary_emb(k0, cos[src_rows[ksrc]], sin[src_rows[ksrc]])
    moved = OA.move_shared(rotated, sc.k_move_a, sc.k_move_b, cos, sin)
    direct = OA.rotate_rows(k0, sc.k_rope, cos, sin)
    assert (moved - direct).abs().max().item() < 1e-4
    assert (torch.as_tensor(sc.k_move_a) >= 0).sum() == sum(len(lay.shared_frames(j)) for j in range(4)) * T


# ---------------------------------------------------------------------------------------------- attention
def test_packed_attention_matches_explicit_softmax():
    g = torch.Generator().manual_seed(1)
    lq, lk = [5, 1, 17], [9, 3, 30]
    H, D = 2, 16
    q = torch.randn(sum(lq), H, D, generator=g)
    k = torch.randn(sum(lk), H, D, generator=g)
    v = torch.randn(sum(lk), H, D, generator=g)
    cq, ck = np.cumsum([0] + lq), np.cumsum([0] + lk)
    out = OA.packed_attention(q, k, v, cq, ck)
    for s in range(3):
        qs, ks, vs = (x.double() for x in (q[cq[s]:cq[s + 1]], k[ck[s]:ck[s + 1]], v[ck[s]:ck[s + 1]]))
        for h in range(H):
            p = torch.exp((qs[:, h] @ ks[:, h].T) / D ** 0.5)
            ref = (p / p.sum(1, keepdim=True)) @ vs[:, h]
            assert (out[cq[s]:cq[s + 1], h].double() - ref).abs().max() < 1e-5


@pytest.mark.parametrize('case', [
    dict(lengths=[3, 3], halo=0, extra={0: [5], 1: [0]}, T=8, counts=[4, 4], Le=8),     # the 2-scene CPU-plumbing shape, smaller T
    dict(lengths=[2, 3, 2], halo=1, extra={}, T=4, counts=[3, 0, 2], Le=7),             # halo, empty sentence, padding
    dict(lengths=[4, 2], halo=2, sides='next', extra={}, T=5, counts=[2, 2], Le=4),
])
def test_packed_layer_equals_masked_brute_force(case):
    """packed scopes + per-scope SDPA + write-back == dense masked softmax over the scope definition"""
    lay = OL.SceneLayout(case['lengths'], halo=case['halo'], sides=case.get('sides', 'adj'), extra=case['extra'])
    T, Le = case['T'], case['Le']
    g = torch.Generator().manual_seed(2)
    S, H, D = lay.n_frames * T, 2, 16
    q, k, v = (torch.randn(S, H, D, generator=g) for _ in range(3))
    eq, ek, ev = (torch.randn(Le, H, D, generator=g) for _ in range(3))
    sc = OL.hunyuan_scopes(lay, T, case['counts'], Le)
    ov, ot = OA.scene_layer(sc, q, k, v, eq, ek, ev, mode='none')
    rv, rt = OA.masked_reference(lay, T, case['counts'], q, k, v, eq, ek, ev)
    assert (ov - rv).abs().max() < 1e-5
    assert (ot - rt).abs().max() < 1e-5
    assert ot[sum(case['counts']):].abs().max() == 0 if Le > sum(case['counts']) else True


# ------------------------------------------------------------------------------------------------ log-sum-exp merge
@pytest.mark.parametrize('split', [0, 1, 37, 60, 61])
def test_merge_lse_of_disjoint_key_sets_is_attention_over_their_union(split):
    """attention over keys [0, split) and [split, 61), merged, equals attention over all 61 keys (float64); an empty
    side (split 0 or 61) leaves the other side unchanged"""
    g = torch.Generator().manual_seed(split)
    q, k, v = (torch.randn(n, 3, 16, generator=g, dtype=torch.float64) for n in (9, 61, 61))
    o1, l1 = OA.attention_lse(q, k[:split], v[:split])
    o2, l2 = OA.attention_lse(q, k[split:], v[split:])
    o, lse = OA.merge_lse(o1, l1, o2, l2)
    ref_o, ref_l = OA.attention_lse(q, k, v)
    assert (o - ref_o).abs().max() < 1e-12
    assert (lse - ref_l).abs().max() < 1e-12


def test_attention_lse_matches_packed_attention_and_logsumexp():
    """the float64 dense helper agrees with the oracle's packed attention and with an explicit log(sum(exp))"""
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(n, 2, 32, generator=g) for n in (7, 19, 19))
    o, lse = OA.attention_lse(q, k, v)
    ref = OA.packed_attention(q, k, v, np.array([0, 7]), np.array([0, 19]))
    assert (o.float() - ref).abs().max() < 1e-5
    s = torch.einsum('nhd,mhd->hnm', q.double(), k.double()) / 32 ** 0.5
    assert (lse - s.exp().sum(-1).log()).abs().max() < 1e-10


def test_merge_lse_first_step_of_a_ring():
    """a ring starts from o = 0, lse = -inf: the first merge returns the partial result exactly"""
    g = torch.Generator().manual_seed(5)
    o_s = torch.randn(4, 2, 8, generator=g).to(torch.bfloat16)
    l_s = torch.randn(2, 4, generator=g)
    o, lse = OA.merge_lse(torch.zeros(4, 2, 8), torch.full((2, 4), -float('inf')), o_s, l_s)
    assert torch.equal(o, o_s.float()) and torch.allclose(lse, l_s, atol=0, rtol=0)


# ------------------------------------------------------------------------------------------- Wan RMSNorm + RoPE
def test_wan_qk_norm_rope_textbook_forms():
    """unit RMS before the weight, and each head's pair rotation is the complex product (x1 + i x2)(c + i s); the
    weight scales elementwise before the rotation"""
    from oracle import wan as OW
    g = torch.Generator().manual_seed(7)
    S, H, D = 5, 4, 16
    x = torch.randn(S, H * D, generator=g, dtype=torch.float64)
    ang = torch.randn(S, D // 2, generator=g, dtype=torch.float64)
    cos = ang.cos().repeat_interleave(2, 1)
    sin = ang.sin().repeat_interleave(2, 1)
    ones = torch.ones(H * D, dtype=torch.float64)
    no_rot = OW.qk_norm_rope(x, ones, 0.0, torch.ones(S, D, dtype=torch.float64), torch.zeros(S, D, dtype=torch.float64), H)
    assert torch.allclose(no_rot.reshape(S, -1).pow(2).mean(-1), torch.ones(S, dtype=torch.float64))
    w = torch.rand(H * D, generator=g, dtype=torch.float64) + 0.5
    out = OW.qk_norm_rope(x, w, 1e-6, cos, sin, H)
    y = (x / (x.pow(2).mean(-1, keepdim=True) + 1e-6).sqrt() * w).view(S, H, D // 2, 2)
    z = torch.complex(y[..., 0], y[..., 1]) * torch.polar(torch.ones_like(ang), ang)[:, None, :]
    assert (out.view(S, H, D // 2, 2) - torch.stack([z.real, z.imag], -1)).abs().max() < 1e-12


# ------------------------------------------------------------------------------------------------- frame memory
def _groups(sizes, dim, noise, seed):
    """frames in len(sizes) groups of near-identical unit features (the reference test's construction)"""
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(len(sizes), dim, generator=g, dtype=torch.float64)
    x = torch.cat([base[i].expand(n, -1) for i, n in enumerate(sizes)])
    x = x + noise * torch.randn(x.shape, generator=g, dtype=torch.float64)
    return torch.nn.functional.normalize(x, dim=-1)


def test_frame_memory_select_one_medoid_per_group():
    """tests/test_onereel_frame_memory.py:19-38: two groups of frames (5 and 4) give one representative each"""
    from oracle import frame_memory as OF
    feats = _groups([5, 4], 16, 0.01, 0)
    reps = OF.select(feats, list(range(9)), 2)
    assert len(reps) == 2 and min(reps) < 5 <= max(reps)


@pytest.mark.parametrize('sizes,seed', [([5, 4], 1), ([7, 3, 9, 5], 2), ([1, 12, 6], 3)])
def test_frame_memory_select_medoids_by_construction(sizes, seed):
    """well-separated groups: each representative is the member of its group closest to the group's normalised mean"""
    from oracle import frame_memory as OF
    feats = _groups(sizes, 32, 0.05, seed)
    reps = OF.select(feats, list(range(sum(sizes))), len(sizes))
    exp, lo = [], 0
    for n in sizes:
        m = torch.nn.functional.normalize(feats[lo:lo + n].mean(0), dim=0)
        exp.append(lo + int((feats[lo:lo + n] @ m).argmax()))
        lo += n
    assert reps == sorted(exp)


def test_frame_memory_candidates_sink_and_pool():
    """tests/test_onereel_frame_memory.py:41-60: boundary candidates, the sink excluded; pooling = per-frame sums"""
    from oracle import frame_memory as OF
    ranges = [(0, 4), (4, 8), (8, 12)]
    assert OF.candidates(ranges, 12, 'boundary') == [0, 3, 4, 7, 8, 11]
    assert 0 not in OF.candidates([(0, 3), (3, 6), (6, 9)], 9, 'all', sink=(0,))
    g = torch.Generator().manual_seed(4)
    feats = torch.nn.functional.normalize(torch.randn(12, 8, generator=g, dtype=torch.float64), dim=-1)
    assert OF.select(feats, [0, 3, 4, 7, 8, 11], 3) == OF.select(feats, [0, 3, 4, 7, 8, 11], 3)
    assert set(OF.select(feats, [0, 3, 4, 7, 8, 11], 3)) <= {0, 3, 4, 7, 8, 11}
    hs = torch.randn(10, 3, generator=g)
    frame = torch.tensor([0, 0, 1, 1, 1, -1, 2, 2, 2, 2])
    s, c = OF.pool(frame, hs, 4)
    assert torch.allclose(s[1], hs[2:5].double().sum(0)) and c.tolist() == [2, 3, 4, 0]


# ------------------------------------------------------------------------------------------ bounded memory (per head)
def test_memory_select_keeps_every_candidate_when_the_budget_covers_them():
    """tests/test_onereel_memory.py:63-73 of the reference"""
    from oracle import memory as OM
    rows, _ = OM.boundary_rows([(0, 3), (3, 7), (7, 9)], 8)
    k = torch.randn(9 * 8, 2, 32, generator=torch.Generator().manual_seed(1))
    rep, valid = OM.select(k[rows], len(rows))
    for h in range(2):
        assert sorted(rep[h][valid[h]].tolist()) == list(range(len(rows)))


def test_memory_select_representative_is_the_nearest_member():
    """tests/test_onereel_memory.py:76-94 of the reference: every representative is at least as near its centroid as
    any other member of its cluster (distances recomputed here)"""
    from oracle import memory as OM
    x = torch.randn(120, 3, 16, generator=torch.Generator().manual_seed(2))
    rep, valid, c = OM.select(x, 12, centroids=True)
    xn = torch.nn.functional.normalize(x.float().transpose(0, 1), dim=-1)
    for h in range(3):
        z = torch.cdist(xn[h], c[h]).argmin(-1)
        reps = rep[h][valid[h]].tolist()
        assert len(reps) == len(set(z.tolist()))          # one representative per non-empty cluster
        for r in reps:
            members = (z == z[r]).nonzero().flatten()
            d = (xn[h, members] - c[h, z[r]]).pow(2).sum(-1)
            assert d.min() >= (xn[h, r] - c[h, z[r]]).pow(2).sum() - 1e-6


def test_memory_select_one_representative_per_separated_group():
    from oracle import memory as OM
    g = torch.Generator().manual_seed(3)
    base = torch.randn(4, 2, 16, generator=g)
    x = torch.cat([base[i].expand(10, -1, -1) for i in range(4)]) + 0.01 * torch.randn(40, 2, 16, generator=g)
    rep, valid = OM.select(x, 4)
    for h in range(2):
        assert sorted(r // 10 for r in rep[h][valid[h]].tolist()) == [0, 1, 2, 3]


def test_memory_masked_reference_equals_dense_masked_softmax():
    """MemoryAttention's per-head scopes (memory.py:140-174; the reference test's per-head reference,
    tests/test_onereel_memory.py:21-37) as one dense float64 softmax over all keys under a boolean mask built from
    the scope definition: a video query of scene j sees scene j's frames, sentence j and, for its head, the valid
    representatives of the other scenes; a sentence query of scene j sees scene j's frames and sentence j. The
    oracle's gathered form agrees; restricted to some rows it gives those rows and zeros elsewhere"""
    from oracle import memory as OM
    g = torch.Generator().manual_seed(9)
    ranges, T, H, D = [(0, 2), (2, 5), (5, 6)], 4, 2, 16
    tr = [(0, 2), (2, 3), (3, 6)]
    S, Le = 6 * T, 7                                        # one padding text row
    q, k, v = (torch.randn(S, H, D, generator=g) for _ in range(3))
    eq, ek, ev = (torch.randn(Le, H, D, generator=g) for _ in range(3))
    rows, owner = OM.boundary_rows(ranges, T)
    M = 5
    rep = torch.stack([torch.randperm(len(rows), generator=g)[:M] for _ in range(H)])
    valid = torch.ones(H, M, dtype=torch.bool)
    valid[1, 3:] = False
    rv, rt = OM.masked_reference(q, k, v, eq, ek, ev, ranges, T, rows[rep], owner[rep], valid, tr)
    scene_of = [j for j, (lo, hi) in enumerate(ranges) for _ in range((hi - lo) * T)]
    kk, vv = torch.cat([k, ek]).double(), torch.cat([v, ev]).double()
    for h in range(H):
        mask = torch.zeros(S + Le, S + Le, dtype=torch.bool)   # [query row of q ; eq] x [key row of k ; ek]
        for j, (lo, hi) in enumerate(ranges):
            t0, t1 = tr[j]
            own = list(range(lo * T, hi * T)) + [S + t for t in range(t0, t1)]
            far = [int(rows[r]) for r, ok in zip(rep[h], valid[h]) if ok and scene_of[int(rows[r])] != j]
            for qr in range(lo * T, hi * T):
                mask[qr, own + far] = True
            for t in range(t0, t1):
                mask[S + t, own] = True
        qq = torch.cat([q, eq])[:, h].double()
        s = (qq @ kk[:, h].T) * D ** -0.5
        s = s.masked_fill(~mask, float('-inf'))
        p = torch.softmax(s, -1).nan_to_num(0.0)               # the padding text row sees no key: zero output
        o = p @ vv[:, h]
        assert torch.allclose(rv[:, h].double(), o[:S], atol=1e-5)
        assert torch.allclose(rt[:, h].double(), o[S:], atol=1e-5)
    vr, trs = [1, 9, 13, 23], [0, 4]
    sv, st = OM.masked_reference(q, k, v, eq, ek, ev, ranges, T, rows[rep], owner[rep], valid, tr, video_rows=vr,
                                 text_rows=trs)
    assert torch.allclose(sv[vr], rv[vr], atol=1e-6) and torch.allclose(st[trs], rt[trs], atol=1e-6)
    assert sv[[r for r in range(S) if r not in vr]].abs().max() == 0


def test_memory_select_warm_start():
    """a warm call (two passes from stored centroids) that starts from the centroids a converged cold call ended on,
    over the same keys, is a fixed point: the same centroids and representatives; from the cold start's own
    centroids it gives what the cold call's first two passes give"""
    from oracle import memory as OM
    g = torch.Generator().manual_seed(4)
    base = torch.randn(5, 2, 16, generator=g)
    x = torch.cat([base[i].expand(8, -1, -1) for i in range(5)]) + 0.1 * torch.randn(40, 2, 16, generator=g)
    rep, valid, c = OM.select(x, 5, centroids=True)
    rep2, valid2, c2 = OM.select(x, 5, iters=2, centroids=True, start=c)
    assert torch.equal(rep, rep2) and torch.equal(valid, valid2) and torch.equal(c, c2)
    xn = torch.nn.functional.normalize(x.float().transpose(0, 1), dim=-1)
    c0 = xn[:, torch.linspace(0, 39, 5).round().long()]
    a = OM.select(x, 5, iters=2, centroids=True, start=c0)
    b = OM.select(x, 5, iters=2, centroids=True)
    assert all(torch.equal(u, w) for u, w in zip(a, b))


@pytest.mark.parametrize('mode', ['raw', 'rotated', 'none'])
@pytest.mark.parametrize('adjacent', [False, True])
def test_sampled_row_references_match_the_full_pack(mode, adjacent):
    """the GPU tests' sampled-row references (per-segment gathers) give exactly the rows of the oracle's full pack
    and of its packed attention, on the CPU-plumbing layout"""
    import helpers as Hp
    case = Hp.layout_case('cpu_plumbing')
    H, D, T = case['H'], case['D'], case['T']
    S = sum(case['lengths']) * T
    q, k, v = (Hp.rand_bf16((S, H, D), s) for s in (1, 2, 3))
    eq, ek, ev = (Hp.rand_bf16((case['Le'], H, D), s) for s in (4, 5, 6))
    cos, sin = OA.rope_table_3d(*case['table'], D)
    sc = OL.hunyuan_scopes(OL.SceneLayout(case['lengths'], 0, 'adj', case['extra']), T, case['counts'], case['Le'],
                           scene_rope=True, adjacent=adjacent)
    qp, kp, vp = OA.pack(sc, q, k, v, eq, ek, ev, cos, sin, mode=mode)
    sel = Hp.sample_packed(sc.cu_k, 50)
    ks, vs = Hp.packed_rows_reference(sc, k, ek, v, ev, sel, cos, sin, mode=mode)
    assert torch.equal(ks.view(torch.int16), kp[sel].view(torch.int16))
    assert torch.equal(vs.view(torch.int16), vp[sel].view(torch.int16))
    qmode = 'raw' if mode == 'raw' else 'none'
    selq = Hp.sample_packed(sc.cu_q, 30)
    qs = Hp.packed_rows_reference(sc, k, ek, v, ev, selq, cos, sin, mode=qmode, which='q', q=q, eq=eq)
    assert torch.equal(qs.view(torch.int16), OA.pack(sc, q, k, v, eq, ek, ev, cos, sin, mode=qmode)[0][selq]
                       .view(torch.int16))
    rows = Hp.sample_rows(sc.cu_q, 20)
    full = OA.packed_attention(qp, kp, vp, sc.cu_q, sc.cu_k)[rows]
    assert (Hp.scope_rows_reference(sc, q, k, v, eq, ek, ev, rows, cos, sin, mode=mode) - full).abs().max() < 1e-5
