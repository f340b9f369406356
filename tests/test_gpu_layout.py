"""GPU parity, bit-exact: the layout kernel, the K/V/Q pack-gather (with RoPE and _move_shared) and the scatter
against the oracle, through the C ABI, at the benchmark layouts' full sizes and on edge-case layouts."""
import numpy as np
import pytest
import torch

from helpers import bits, layout_case, packed_rows_reference, rand_bf16, sample_packed
from onereel_amd import scene
from onereel_amd.layout import SceneLayout
from onereel_amd.scene import ScopePlan, pack_rows, rotate_queries, scatter
from oracle import attention as OA
from oracle import layout as OL

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]

DEV = 'cuda'


def _plans(case, adjacent, with_text=True):
    lay = SceneLayout(case['lengths'], halo=case['halo'], sides=case['sides'], extra=case['extra'])
    counts = case['counts'] if with_text else None
    Le = case['Le'] if with_text else 0
    plan = ScopePlan(lay, case['T'], counts, Le, case['scene_rope'], case['rope_lengths'], adjacent, with_text, DEV,
                     moves=True)
    olay = OL.SceneLayout(case['lengths'], case['halo'], case['sides'], case['extra'])
    sc = OL.hunyuan_scopes(olay, case['T'], case['counts'] if with_text else [0] * len(case['lengths']), Le,
                           scene_rope=case['scene_rope'], rope_lengths=case['rope_lengths'], adjacent=adjacent,
                           with_text=with_text)
    return plan, sc


def _check_plan(plan, sc, adjacent):
    torch.cuda.synchronize()
    eq = lambda t, a: np.array_equal(t.cpu().numpy().astype(np.int64), np.asarray(a, np.int64))
    assert eq(plan.cu_q, sc.cu_q) and eq(plan.cu_k, sc.cu_k)
    first = [int(sc.q_src[a]) if b > a else -1 for a, b in zip(sc.cu_q[:-1], sc.cu_q[1:])]
    got_first = plan.seg_q_src.cpu().numpy()
    assert all(f == -1 or f == g for f, g in zip(first, got_first))
    assert eq(plan.q_src, sc.q_src) and eq(plan.k_src, sc.k_src)
    assert eq(plan.q_rope, sc.q_rope) and eq(plan.k_rope, sc.k_rope)
    if adjacent:
        assert eq(plan.k_move_a, sc.k_move_a) and eq(plan.k_move_b, sc.k_move_b)
    assert (plan.n_seg, plan.sum_q, plan.sum_k) == (len(sc.lq), int(sc.cu_q[-1]), int(sc.cu_k[-1]))
    _check_values_in_place(plan, sc)


def _check_values_in_place(plan, sc):
    """v_lead / v_row / v_src: the first v_lead keys of every segment (whole 32-key blocks of its scene's own frames)
    are consecutive token rows from v_row, so their values can be read in place: the oracle's key rows of those keys
    are exactly v_row, v_row + 1, ...; v_lead is the largest such multiple of 32 within the own frames. v_runs: each
    video segment's first shared frames (the oracle's frames, in its order), each T consecutive token rows of the
    plan's (oracle-checked) key rows. The pack's value rows (v_src) are the key rows except those in the leading
    run's and the runs' whole key blocks, which are -1"""
    k_src = np.asarray(sc.k_src)
    v_lead, v_row, k_len = (getattr(plan, a).cpu().numpy() for a in ('v_lead', 'v_row', 'k_len'))
    lay = plan.layout
    starts = np.cumsum([0] + list(lay.lengths))
    cu = np.asarray(sc.cu_k)
    for s in range(plan.n_seg):
        j = sc.scene[s]
        own = int(lay.lengths[j]) * plan.T
        assert v_row[s] == starts[j] * plan.T
        assert v_lead[s] == (own // 32 * 32 if k_len[s] > 0 else 0), (s, v_lead[s], own)
        assert v_lead[s] % 32 == 0 and v_lead[s] <= k_len[s]
        assert np.array_equal(k_src[cu[s]:cu[s] + v_lead[s]], v_row[s] + np.arange(v_lead[s])), s
    got = plan.v_src.cpu().numpy().astype(np.int64)
    pcu = plan.cu_k.cpu().numpy()
    pk = plan.k_src.cpu().numpy().astype(np.int64)
    want = pk.copy()
    for s in range(plan.n_seg):   # the segments that own packed rows (T_j owns none with its keys in place)
        want[pcu[s]:pcu[s] + min(v_lead[s], pcu[s + 1] - pcu[s])] = -1
    if plan.v_runs is not None:
        runs = plan.v_runs.cpu().numpy().reshape(plan.n_seg, scene.L.VALUE_RUNS, 3)
        T = plan.T
        for s in range(plan.n_seg):
            j = sc.scene[s]
            video = not plan.with_text or s % 2 == 0
            own, txt = int(lay.lengths[j]) * T, (plan.counts[j] if plan.with_text else 0)
            nsh = (int(k_len[s]) - own - txt) // T if video and k_len[s] > 0 else 0
            n = min(nsh, scene.L.VALUE_RUNS)
            assert (runs[s, n:] == 0).all(), s
            for r in range(n):
                x0, cnt, t = (int(x) for x in runs[s, r])
                assert cnt == T and t % T == 0, (s, r, runs[s, r])
                # the run's keys are the token rows t.. in the plan's key rows (checked against the oracle's)
                assert np.array_equal(pk[pcu[s] + x0:pcu[s] + x0 + T], t + np.arange(T)), (s, r)
                a, b = -(-x0 // 32) * 32, (x0 + T) // 32 * 32
                if b > a:
                    want[pcu[s] + a:pcu[s] + b] = -1
    assert np.array_equal(got, want)


@pytest.mark.parametrize('name', ['cpu_plumbing', 'hunyuan480p', 'wan704', 'uneven_K2', 'uneven_K4', 'uneven_K8',
                                  'uneven_K12'])
@pytest.mark.parametrize('adjacent', [False, True])
def test_layout_kernel_bit_exact_configs(name, adjacent):
    case = layout_case(name)
    print(f'layout {name} adjacent={adjacent}', flush=True)
    plan, sc = _plans(case, adjacent)
    _check_plan(plan, sc, adjacent)
    if name == 'hunyuan480p':
        assert plan.cu_q.tolist() == [0, 12720, 12848, 25568, 25696, 38416, 38544, 51264, 51392]
        assert plan.cu_k.tolist() == [0, 17618, 30466, 48084, 60932, 78550, 91398, 109016, 121864]


def test_layout_kernel_bit_exact_random_layouts():
    rng = np.random.default_rng(7)
    for it in range(60):
        n = int(rng.integers(1, 9))
        lengths = rng.integers(1, 7, n).tolist()
        F = sum(lengths)
        extra = {j: rng.integers(0, F, int(rng.integers(0, 5))).tolist() for j in range(n) if rng.random() < 0.7}
        rope_lengths = None
        if rng.random() < 0.3:   # scene RoPE over different scene lengths than the attention layout
            rl = []
            left = F
            while left > 0:
                x = int(rng.integers(1, left + 1))
                rl.append(x)
                left -= x
            rope_lengths = rl
        case = dict(lengths=lengths, halo=int(rng.integers(0, 3)), sides=['adj', 'prev', 'next'][int(rng.integers(3))],
                    extra=extra, T=int(rng.integers(1, 12)), counts=rng.integers(0, 6, n).tolist(),
                    scene_rope=bool(rng.integers(2)), rope_lengths=rope_lengths)
        case['Le'] = sum(case['counts']) + int(rng.integers(0, 3))
        adjacent = bool(rng.integers(2))
        with_text = bool(rng.integers(2))
        plan, sc = _plans(case, adjacent, with_text)
        _check_plan(plan, sc, adjacent)


def test_layout_kernel_max_scenes():
    lengths = [1 + (j % 3) for j in range(64)]
    F = sum(lengths)
    case = dict(lengths=lengths, halo=1, sides='adj', extra={j: [(7 * j) % F, (11 * j + 3) % F] for j in range(64)},
                T=5, counts=[j % 4 for j in range(64)], Le=200, scene_rope=True, rope_lengths=None)
    for adjacent in (False, True):
        plan, sc = _plans(case, adjacent)
        _check_plan(plan, sc, adjacent)


def test_layout_kernel_more_runs_than_blocks():
    """64 scenes of 40 frames with T = 3: over 8000 (segment, frame) runs, more than the kernel's 2048 blocks, so
    blocks take several runs each"""
    lengths = [40] * 64
    F = sum(lengths)
    case = dict(lengths=lengths, halo=2, sides='adj', extra={j: [(97 * j) % F] for j in range(0, 64, 3)}, T=3,
                counts=[(5 * j) % 7 for j in range(64)], Le=250, scene_rope=True, rope_lengths=None)
    for adjacent in (False, True):
        print(f'layout 64 x 40 frames adjacent={adjacent}', flush=True)
        plan, sc = _plans(case, adjacent)
        _check_plan(plan, sc, adjacent)


def _check_in_place(case, adjacent):
    """text keys in place: V_j's packed rows are _segments' V_j rows with the sentence moved ahead of the shared frames
    (own frames, sentence, shared frames), T_j packs none, and T_j's key range (k_off, k_len) covers exactly the rows
    of _segments' T_j (own frames, then sentence), in order; every per-key array (source row, RoPE row, the two
    _move_shared rows) follows the same order"""
    lay = SceneLayout(case['lengths'], halo=case['halo'], sides=case['sides'], extra=case['extra'])
    plan = ScopePlan(lay, case['T'], case['counts'], case['Le'], case['scene_rope'], case['rope_lengths'], adjacent,
                     True, DEV, moves=True, text_keys_in_place=True)
    _, sc = _plans(case, adjacent)
    torch.cuda.synchronize()
    n = len(case['lengths'])
    names = ('k_src', 'k_rope') + (('k_move_a', 'k_move_b') if adjacent else ())
    got = {a: getattr(plan, a).cpu().numpy() for a in names}
    ref = {a: np.asarray(getattr(sc, a)) for a in got}
    cu_q, cu_k, k_off, k_len = (getattr(plan, a).cpu().tolist() for a in ('cu_q', 'cu_k', 'k_off', 'k_len'))
    assert cu_q == list(sc.cu_q)
    assert (plan.sum_k, plan.max_k) == (sum(sc.lk[0::2]), max(sc.lk))
    assert k_len == list(sc.lk)
    for j in range(n):
        v, t = 2 * j, 2 * j + 1
        own, txt, lk = sc.lq[v], sc.lq[t], sc.lk[v]
        assert cu_k[t + 1] - cu_k[t] == 0 and k_off[v] == cu_k[v] and k_off[t] == cu_k[v]
        b, rb = cu_k[v], sc.cu_k[v]
        order = np.r_[rb:rb + own, rb + lk - txt:rb + lk, rb + own:rb + lk - txt]
        for a in got:
            assert np.array_equal(got[a][b:b + lk], ref[a][order]), (j, a)
            tb = sc.cu_k[t]
            assert np.array_equal(got[a][k_off[t]:k_off[t] + k_len[t]], ref[a][tb:tb + sc.lk[t]]), (j, a)
    _check_values_in_place(plan, sc)


@pytest.mark.parametrize('name', ['cpu_plumbing', 'hunyuan480p', 'uneven_K4', 'uneven_K12'])
@pytest.mark.parametrize('adjacent', [False, True])
def test_layout_text_keys_in_place(name, adjacent):
    print(f'layout text keys in place {name} adjacent={adjacent}', flush=True)
    _check_in_place(layout_case(name), adjacent)


def test_layout_text_keys_in_place_random_layouts():
    """random layouts with empty sentences, halos and extra frames"""
    rng = np.random.default_rng(17)
    for it in range(30):
        n = int(rng.integers(1, 8))
        lengths = rng.integers(1, 6, n).tolist()
        F = sum(lengths)
        extra = {j: rng.integers(0, F, int(rng.integers(0, 4))).tolist() for j in range(n) if rng.random() < 0.7}
        case = dict(lengths=lengths, halo=int(rng.integers(0, 3)), sides=['adj', 'prev', 'next'][int(rng.integers(3))],
                    extra=extra, T=int(rng.integers(1, 10)), counts=rng.integers(0, 5, n).tolist(),
                    scene_rope=bool(rng.integers(2)), rope_lengths=None)
        case['Le'] = sum(case['counts']) + int(rng.integers(0, 3))
        _check_in_place(case, bool(rng.integers(2)))


def _check_rank_share(case, adjacent, q_range, in_place, with_text=True):
    """one rank's share (q_range): each segment the rank runs holds the oracle's token_range segment (query rows and
    RoPE rows; key rows, RoPE and _move_shared rows, in the in-place order when the text keys are read in place), and
    every other segment is empty"""
    lay = SceneLayout(case['lengths'], halo=case['halo'], sides=case['sides'], extra=case['extra'])
    in_place = in_place and with_text
    counts = case['counts'] if with_text else [0] * len(case['lengths'])
    Le = case['Le'] if with_text else 0
    plan = ScopePlan(lay, case['T'], counts if with_text else None, Le, case['scene_rope'], case['rope_lengths'],
                     adjacent, with_text, DEV, moves=True, text_keys_in_place=in_place, q_range=q_range)
    olay = OL.SceneLayout(case['lengths'], case['halo'], case['sides'], case['extra'])
    sc = OL.hunyuan_scopes(olay, case['T'], counts, Le, scene_rope=case['scene_rope'],
                           rope_lengths=case['rope_lengths'], adjacent=adjacent, with_text=with_text,
                           token_range=q_range)
    torch.cuda.synchronize()
    T, n = case['T'], len(case['lengths'])
    names = ('q_src', 'q_rope', 'k_src', 'k_rope') + (('k_move_a', 'k_move_b') if adjacent else ())
    got = {a: getattr(plan, a).cpu().numpy() for a in names}
    ref = {a: np.asarray(getattr(sc, a)) for a in names}
    cu_q, cu_k, k_off, k_len, first = (getattr(plan, a).cpu().tolist()
                                       for a in ('cu_q', 'cu_k', 'k_off', 'k_len', 'seg_q_src'))
    per = 2 if with_text else 1
    ran = {(per * j + (kind == 't')): i for i, (kind, j) in enumerate(zip(sc.kind, sc.scene))}
    assert plan.n_seg == per * n and plan.sum_q == int(sc.cu_q[-1])
    for s in range(per * n):
        lq = cu_q[s + 1] - cu_q[s]
        if s not in ran:
            assert lq == 0 and k_len[s] == 0 and cu_k[s + 1] == cu_k[s], s
            continue
        i, j = ran[s], s // per
        qa, qb, ka, kb = sc.cu_q[i], sc.cu_q[i + 1], sc.cu_k[i], sc.cu_k[i + 1]
        assert lq == qb - qa and k_len[s] == kb - ka, s
        assert qb == qa or first[s] == ref['q_src'][qa], s
        for a in ('q_src', 'q_rope'):
            assert np.array_equal(got[a][cu_q[s]:cu_q[s + 1]], ref[a][qa:qb]), (s, a)
        order = np.arange(ka, kb)
        if in_place and s % 2 == 0:   # own frames, sentence, shared frames
            own, txt = len(lay.frames[j]) * T, counts[j]
            order = np.r_[ka:ka + own, kb - txt:kb, ka + own:kb - txt]
        if in_place and s % 2 == 1:
            assert cu_k[s + 1] == cu_k[s] and k_off[s] == cu_k[s - 1], s
        else:
            assert k_off[s] == cu_k[s] and cu_k[s + 1] - cu_k[s] == kb - ka, s
        for a in names[2:]:
            assert np.array_equal(got[a][k_off[s]:k_off[s] + k_len[s]], ref[a][order]), (s, a)


def _equal_token_ranges(case, P):
    S = sum(case['lengths']) * case['T']
    return [(r * S // P, (r + 1) * S // P) for r in range(P)]


@pytest.mark.parametrize('name, P', [('cpu_plumbing', 3), ('hunyuan480p', 3), ('hunyuan480p', 8), ('uneven_K4', 5),
                                     ('uneven_K12', 8)])
def test_layout_rank_shares(name, P):
    """the layer's video tokens split over P ranks by equal token counts (cutting scenes and frames): every rank's
    share, with and without the text keys in place, in both shared-position modes"""
    case = layout_case(name)
    for r, q_range in enumerate(_equal_token_ranges(case, P)):
        for adjacent in (False, True):
            for in_place in (False, True):
                print(f'layout rank share {name} rank {r}/{P} {q_range} adjacent={adjacent} in_place={in_place}',
                      flush=True)
                _check_rank_share(case, adjacent, q_range, in_place)


def test_layout_rank_shares_random_layouts():
    rng = np.random.default_rng(23)
    for it in range(40):
        n = int(rng.integers(1, 8))
        lengths = rng.integers(1, 6, n).tolist()
        F = sum(lengths)
        extra = {j: rng.integers(0, F, int(rng.integers(0, 4))).tolist() for j in range(n) if rng.random() < 0.7}
        case = dict(lengths=lengths, halo=int(rng.integers(0, 3)), sides=['adj', 'prev', 'next'][int(rng.integers(3))],
                    extra=extra, T=int(rng.integers(1, 10)), counts=rng.integers(0, 5, n).tolist(),
                    scene_rope=bool(rng.integers(2)), rope_lengths=None)
        case['Le'] = sum(case['counts']) + int(rng.integers(0, 3))
        S = F * case['T']
        a = int(rng.integers(0, S))
        _check_rank_share(case, bool(rng.integers(2)), (a, int(rng.integers(a + 1, S + 1))), bool(rng.integers(2)),
                          with_text=bool(rng.integers(2)))


def _tables(case):
    F, Hh, Ww = case['table']
    assert Hh * Ww == case['T']
    return OA.rope_table_3d(F, Hh, Ww, case['D'])


@pytest.mark.parametrize('name', ['cpu_plumbing', 'hunyuan480p', 'wan704'])
@pytest.mark.parametrize('adjacent', [False, True])
def test_pack_gather_bit_exact(name, adjacent):
    case = layout_case(name)
    print(f'pack {name} adjacent={adjacent}', flush=True)
    H, D, T = case['H'], case['D'], case['T']
    S = sum(case['lengths']) * T
    plan, sc = _plans(case, adjacent)
    cos, sin = _tables(case)
    q, k, v = (rand_bf16((S, H, D), s) for s in (1, 2, 3))
    eq, ek, ev = (rand_bf16((case['Le'], H, D), s) for s in (4, 5, 6))
    gq, gk, gv, geq, gek, gev = (x.to(DEV) for x in (q, k, v, eq, ek, ev))
    gcos, gsin = cos.to(DEV), sin.to(DEV)
    for mode in ('raw', 'rotated', 'none'):
        kp, vp = pack_rows(plan, gk, gek, 'k', b_video=gv, b_text=gev, cos=gcos, sin=gsin, mode=mode)
        qp = pack_rows(plan, gq, geq, 'q', cos=gcos, sin=gsin, mode='raw' if mode == 'raw' else 'none')
        rq, rk, rv = OA.pack(sc, q, k, v, eq, ek, ev, cos, sin, mode=mode)
        torch.cuda.synchronize()
        assert torch.equal(bits(vp.cpu()), bits(rv)), mode
        assert torch.equal(bits(kp.cpu()), bits(rk)), mode
        assert torch.equal(bits(qp.cpu()), bits(rq)), mode
        del kp, vp, qp


@pytest.mark.parametrize('name', ['uneven_K2', 'uneven_K4', 'uneven_K8', 'uneven_K12'])
@pytest.mark.parametrize('adjacent', [False, True])
def test_pack_gather_bit_exact_uneven_sweep(name, adjacent):
    """the uneven scene-count sweep (2-12 scenes of 2-16 frames x 1590 tokens, 64-256 text rows, frame memory 4):
    every packed K / V / Q row the GPU writes, for 4000 sampled rows plus every segment's first and last row, equals
    the oracle's row bit for bit in all three RoPE modes"""
    case = layout_case(name)
    print(f'pack {name} adjacent={adjacent}', flush=True)
    H, D, T = case['H'], case['D'], case['T']
    S = sum(case['lengths']) * T
    plan, sc = _plans(case, adjacent)
    cos, sin = _tables(case)
    q, k, v = (rand_bf16((S, H, D), s) for s in (1, 2, 3))
    eq, ek, ev = (rand_bf16((case['Le'], H, D), s) for s in (4, 5, 6))
    gq, gk, gv, geq, gek, gev = (x.to(DEV) for x in (q, k, v, eq, ek, ev))
    gcos, gsin = cos.to(DEV), sin.to(DEV)
    sel_k, sel_q = sample_packed(sc.cu_k, 4000, 1), sample_packed(sc.cu_q, 4000, 2)
    for mode in ('raw', 'rotated', 'none'):
        kp, vp = pack_rows(plan, gk, gek, 'k', b_video=gv, b_text=gev, cos=gcos, sin=gsin, mode=mode)
        qmode = 'raw' if mode == 'raw' else 'none'
        qp = pack_rows(plan, gq, geq, 'q', cos=gcos, sin=gsin, mode=qmode)
        rk, rv = packed_rows_reference(sc, k, ek, v, ev, sel_k, cos, sin, mode=mode)
        rq = packed_rows_reference(sc, k, ek, v, ev, sel_q, cos, sin, mode=qmode, which='q', q=q, eq=eq)
        tk, tq = torch.as_tensor(sel_k).to(DEV), torch.as_tensor(sel_q).to(DEV)
        assert torch.equal(bits(kp[tk].cpu()), bits(rk)), mode
        assert torch.equal(bits(vp[tk].cpu()), bits(rv)), mode
        assert torch.equal(bits(qp[tq].cpu()), bits(rq)), mode
        del kp, vp, qp


@pytest.mark.parametrize('name', ['cpu_plumbing', 'hunyuan480p', 'uneven_K4'])
@pytest.mark.parametrize('adjacent', [False, True])
def test_rotate_queries_bit_exact(name, adjacent):
    """or_rotate_rows through rotate_queries: every video query row, rotated at its scene-RoPE row and written to its
    own token row, equals the oracle's packed (rotated) query row bit for bit; text rows are not touched"""
    case = layout_case(name)
    print(f'rotate queries {name} adjacent={adjacent}', flush=True)
    H, D, T = case['H'], case['D'], case['T']
    S = sum(case['lengths']) * T
    plan, sc = _plans(case, adjacent)
    cos, sin = _tables(case)
    q = rand_bf16((S, H, D), 7)
    eq = rand_bf16((case['Le'], H, D), 8)
    qr = rotate_queries(plan, q.to(DEV), cos.to(DEV), sin.to(DEV)).cpu()
    vid = np.nonzero(np.asarray(sc.q_src) < S)[0]
    assert len(np.unique(np.asarray(sc.q_src)[vid])) == S          # every video row is some segment's query
    sel = vid if S * H * D <= (1 << 22) else np.unique(np.concatenate([vid[::37], vid[[0, -1]]]))
    ref = packed_rows_reference(sc, q, eq, q, eq, sel, cos, sin, mode='raw', which='q', q=q, eq=eq)
    assert torch.equal(bits(qr[torch.as_tensor(np.asarray(sc.q_src)[sel])]), bits(ref))


@pytest.mark.parametrize('name', ['cpu_plumbing', 'hunyuan480p'])
def test_scatter_bit_exact(name):
    case = layout_case(name)
    H, D, T = case['H'], case['D'], case['T']
    S = sum(case['lengths']) * T
    plan, sc = _plans(case, False)
    o = rand_bf16((plan.sum_q, H, D), 9)
    le_pad = case['Le'] + 3        # text rows past the valid tokens must come back zero
    ov = torch.full((S, H, D), 7.0, dtype=torch.bfloat16, device=DEV)
    ot = torch.full((le_pad, H, D), 7.0, dtype=torch.bfloat16, device=DEV)
    plan2 = ScopePlan(SceneLayout(case['lengths'], halo=case['halo'], sides=case['sides'], extra=case['extra']), T,
                      case['counts'], le_pad, case['scene_rope'], None, False, True, DEV)
    scatter(plan2, o.to(DEV), ov, ot)
    rv, rt = OA.write_back(sc, o, le_pad, torch.bfloat16)
    torch.cuda.synchronize()
    assert torch.equal(bits(ov.cpu()), bits(rv))
    assert torch.equal(bits(ot.cpu()), bits(rt))
