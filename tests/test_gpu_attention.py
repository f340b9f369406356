"""GPU parity of the attention kernel and of the whole scene-attention layer against the fp32 oracle, through the
C ABI. Tolerance (bf16 kernel vs fp32 reference on the same packing): max-abs <= 2e-2 and mean-abs <= 2e-3."""
import numpy as np
import pytest
import torch

from helpers import Attn as _Attn
from helpers import assert_close, attn_rows_reference, layout_case, rand_bf16, sample_rows, scope_rows_reference
from onereel_amd import _lib as L
from onereel_amd import attention as A
from onereel_amd import comm
from onereel_amd import hunyuan15 as HY
from onereel_amd import scene
from onereel_amd import wan as W
from onereel_amd.layout import SceneLayout
from oracle import attention as OA
from oracle import layout as OL

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]
DEV = 'cuda'


def _segments_case(lq, lk, H, D, seed):
    q = rand_bf16((sum(lq), H, D), seed)
    k = rand_bf16((sum(lk), H, D), seed + 1)
    v = rand_bf16((sum(lk), H, D), seed + 2)
    return q, k, v, np.cumsum([0] + lq), np.cumsum([0] + lk)


@pytest.mark.parametrize('D', [64, 128])
@pytest.mark.parametrize('lq,lk,H', [
    ([1], [1], 1),
    ([5, 1, 17], [9, 3, 30], 2),
    ([63, 64, 65], [64, 63, 129], 3),
    ([256, 257, 300, 7], [1000, 64, 65, 2049], 2),
    ([0, 40, 0, 12], [5, 77, 9, 200], 4),          # empty query segments
    ([7, 300, 20], [0, 50, 0], 2),                 # segments without keys (O = 0) beside one with keys
    ([300, 45, 129], [700, 130, 33], 11),          # more heads than item queues, not a multiple of them
])
def test_varlen_matches_fp32_reference(lq, lk, H, D):
    print(f'varlen lq={lq} lk={lk} H={H} D={D}', flush=True)
    q, k, v, cq, ck = _segments_case(lq, lk, H, D, 11)
    o = A.varlen(q.to(DEV), k.to(DEV), v.to(DEV), torch.tensor(cq, dtype=torch.int32, device=DEV),
                 torch.tensor(ck, dtype=torch.int32, device=DEV), max(lq), max(lk))
    ref = OA.packed_attention(q, k, v, cq, ck)
    assert_close(o.cpu(), ref, what='varlen')


@pytest.mark.parametrize('D', [64, 128])
@pytest.mark.parametrize('growth', [0.05, -0.0009])
def test_varlen_running_max_moves(growth, D):
    """keys scaled by (1 + growth * key index): with growth > 0 the scores keep rising along the keys, so the online
    max moves up many times inside an item (rescale of O and l, the shifted scores and the -m seed); with growth < 0
    the first block holds the maximum and later blocks underflow towards 0. Both kernels: O-only and with lse."""
    lq, lk, H = [300, 64, 5], [1000, 77, 33], 2
    print(f'varlen running max growth={growth} D={D}', flush=True)
    q, k, v, cq, ck = _segments_case(lq, lk, H, D, 31)
    for s in range(len(lk)):
        f = 1.0 + growth * torch.arange(lk[s], dtype=torch.float32)
        k[ck[s]:ck[s + 1]] = (k[ck[s]:ck[s + 1]].float() * f[:, None, None]).bfloat16()
    ref = OA.packed_attention(q, k, v, cq, ck)
    args = (q.to(DEV), k.to(DEV), v.to(DEV), torch.tensor(cq, dtype=torch.int32, device=DEV),
            torch.tensor(ck, dtype=torch.int32, device=DEV), max(lq), max(lk))
    assert_close(A.varlen(*args).cpu(), ref, what='varlen, moving max')
    o, lse = A.varlen_lse(*args)
    assert_close(o.cpu(), ref, what='varlen_lse, moving max')
    for s in range(3):
        qs, ks = q[cq[s]:cq[s + 1]].float(), k[ck[s]:ck[s + 1]].float()
        lref = torch.logsumexp(torch.einsum('qhd,khd->hqk', qs, ks) * D ** -0.5, -1)
        assert (lse[:, cq[s]:cq[s + 1]].cpu() - lref).abs().max() < 2e-3


@pytest.mark.parametrize('lq,lk,H', [([1000], [20000], 4), ([300, 7], [5000, 3000], 3),
                                     ([40, 0, 600], [9000, 50, 2500], 2)])
def test_varlen_key_split_of_few_items(lq, lk, H):
    """few work items over long key ranges: the planner cuts each item into up to 8 parts by key blocks (one part per
    block) and merge_kernel combines the parts by their lse. O (O-only and lse calls) and lse against the fp32
    oracle; the workspace's split count shows that the items were split."""
    D = 128
    print(f'key split lq={lq} lk={lk} H={H}', flush=True)
    q, k, v, cq, ck = _segments_case(lq, lk, H, D, 51)
    dq, dk, dv = q.to(DEV), k.to(DEV), v.to(DEV)
    tq, tk = torch.tensor(cq, dtype=torch.int32, device=DEV), torch.tensor(ck, dtype=torch.int32, device=DEV)
    ref = OA.packed_attention(q, k, v, cq, ck)
    ws = torch.zeros(int(L.lib().or_varlen_workspace_size(len(lq), sum(lq), H, D)), dtype=torch.uint8, device=DEV)
    o = scene.varlen(dq, dk, dv, tq, tk, max(lq), max(lk), workspace=ws)
    assert_close(o.cpu(), ref, what='key-split varlen')
    assert int(ws.view(torch.int32)[3]) > 0
    o, lse = A.varlen_lse(dq, dk, dv, tq, tk, max(lq), max(lk))
    assert_close(o.cpu(), ref, what='key-split varlen_lse')
    for s in range(len(lq)):
        if lq[s] == 0:
            continue
        qs, ks = q[cq[s]:cq[s + 1]].float(), k[ck[s]:ck[s + 1]].float()
        lref = torch.logsumexp(torch.einsum('qhd,khd->hqk', qs, ks) * D ** -0.5, -1)
        assert (lse[:, cq[s]:cq[s + 1]].cpu() - lref).abs().max() < 2e-3


def test_varlen_random_shapes():
    """random segment counts, query / key lengths (empty segments included), head counts and head dims, O-only and
    with lse, against the fp32 oracle: covers whole items and key-split items with every part count the planner
    picks (the shortest segment bounds it)"""
    rng = np.random.default_rng(2024)
    for case in range(12):
        n = int(rng.integers(1, 6))
        lq = rng.integers(0, 300, n).tolist()
        if sum(lq) == 0:
            lq[0] = 1
        lk = rng.integers(1, 2000, n).tolist()
        H, D = int(rng.integers(1, 7)), int(rng.choice([64, 128]))
        with_lse = bool(rng.integers(2))
        print(f'random varlen case {case}: lq={lq} lk={lk} H={H} D={D} lse={with_lse}', flush=True)
        q, k, v, cq, ck = _segments_case(lq, lk, H, D, 100 + case)
        args = (q.to(DEV), k.to(DEV), v.to(DEV), torch.tensor(cq, dtype=torch.int32, device=DEV),
                torch.tensor(ck, dtype=torch.int32, device=DEV), max(lq), max(lk))
        ref = OA.packed_attention(q, k, v, cq, ck)
        if not with_lse:
            assert_close(A.varlen(*args).cpu(), ref, what=f'random varlen case {case}')
            continue
        o, lse = A.varlen_lse(*args)
        assert_close(o.cpu(), ref, what=f'random varlen_lse case {case}')
        for s in range(n):
            if lq[s] == 0:
                continue
            qs, ks = q[cq[s]:cq[s + 1]].float(), k[ck[s]:ck[s + 1]].float()
            lref = torch.logsumexp(torch.einsum('qhd,khd->hqk', qs, ks) * D ** -0.5, -1)
            assert (lse[:, cq[s]:cq[s + 1]].cpu() - lref).abs().max() < 2e-3


@pytest.mark.parametrize('seed,H,D', [(77, 8, 128), (78, 5, 128), (79, 8, 64)])
def test_varlen_many_items_per_block(seed, H, D):
    """several work items per work-group (1.8-5.6 per CU at 256 CUs), so that each item's key loop loads the next
    item's queries at its exit: segments without keys (items with no key loop) and without queries between them,
    O and lse against the fp32 oracle over every row"""
    rng = np.random.default_rng(seed)
    n = 30
    lq = rng.integers(1, 1500, n).tolist()
    lk = rng.integers(1, 700, n).tolist()
    for s in rng.choice(n, 4, replace=False):
        lk[s] = 0
    for s in rng.choice(n, 2, replace=False):
        lq[s] = 0
    print(f'varlen many items: lq={lq} lk={lk} H={H} D={D}', flush=True)
    q, k, v, cq, ck = _segments_case(lq, lk, H, D, 300 + seed)
    args = (q.to(DEV), k.to(DEV), v.to(DEV), torch.tensor(cq, dtype=torch.int32, device=DEV),
            torch.tensor(ck, dtype=torch.int32, device=DEV), max(lq), max(lk))
    ref = OA.packed_attention(q, k, v, cq, ck)
    o = A.varlen(*args)
    assert_close(o.cpu(), ref, what='varlen, many items per block')
    # each item's result does not depend on which work-group ran it or when: repeated calls are bit-identical (a
    # race between the wavefronts of a work-group, or between items, would show as a difference)
    for _ in range(3):
        assert torch.equal(A.varlen(*args), o)
    o, lse = A.varlen_lse(*args)
    assert_close(o.cpu(), ref, what='varlen_lse, many items per block')
    for s in range(n):
        if lq[s] == 0:
            continue
        if lk[s] == 0:
            assert torch.isneginf(lse[:, cq[s]:cq[s + 1]].cpu()).all()
            continue
        qs, ks = q[cq[s]:cq[s + 1]].float(), k[ck[s]:ck[s + 1]].float()
        lref = torch.logsumexp(torch.einsum('qhd,khd->hqk', qs, ks) * D ** -0.5, -1)
        assert (lse[:, cq[s]:cq[s + 1]].cpu() - lref).abs().max() < 2e-3


def test_key_split_of_overlapping_ranges():
    """Wan-style in-place key ranges with few work items (3 scenes x 400 tokens per frame, 2 heads): the split parts
    take their key blocks from inside each scene's range"""
    H, D, T = 2, 128, 400
    lay = OL.SceneLayout([3, 4, 2], halo=2, sides='next')
    S = lay.n_frames * T
    qq, kk, vv = (rand_bf16((S, H, D), s) for s in (61, 62, 63))
    qr, kr = OL.wan_ranges(lay, T)
    o = A.overlapping_ranges(qq.to(DEV), kk.to(DEV), vv.to(DEV), qr, kr).cpu()
    cq = [0] + [b for _, b in qr]
    ref = OA.packed_attention(qq, kk, vv, cq, None, k_off=[a for a, _ in kr], k_len=[b - a for a, b in kr])
    assert_close(o, ref, what='key-split overlapping_ranges')


def test_varlen_lse_and_packed_api():
    lq, lk, H, D = [70, 3, 129], [90, 300, 5], 2, 128
    q, k, v, cq, ck = _segments_case(lq, lk, H, D, 21)
    o, lse = A.varlen_lse(q.to(DEV), k.to(DEV), v.to(DEV), torch.tensor(cq, dtype=torch.int32, device=DEV),
                          torch.tensor(ck, dtype=torch.int32, device=DEV), max(lq), max(lk))
    ref = OA.packed_attention(q, k, v, cq, ck)
    assert_close(o.cpu(), ref, what='varlen_lse out')
    for s in range(3):
        qs, ks = q[cq[s]:cq[s + 1]].float(), k[ck[s]:ck[s + 1]].float()
        lref = torch.logsumexp(torch.einsum('qhd,khd->hqk', qs, ks) * D ** -0.5, -1)
        assert (lse[:, cq[s]:cq[s + 1]].cpu() - lref).abs().max() < 2e-3
    segs = [(q[cq[s]:cq[s + 1]].to(DEV), k[ck[s]:ck[s + 1]].to(DEV), v[ck[s]:ck[s + 1]].to(DEV)) for s in range(3)]
    outs = A.packed(segs)
    assert [x.shape[0] for x in outs] == lq
    assert_close(torch.cat(outs).cpu(), ref, what='packed')
    outs = A.packed_lse(segs)
    assert torch.allclose(torch.cat([l for _, l in outs], 1), lse)


def test_dense_and_overlapping_ranges():
    H, D = 2, 128
    q = rand_bf16((2, 150, H, D), 31)
    k = rand_bf16((2, 170, H, D), 32)
    v = rand_bf16((2, 170, H, D), 33)
    o = A.dense(q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    for b in range(2):
        ref = OA.packed_attention(q[b], k[b], v[b], [0, 150], [0, 170])
        assert_close(o[b], ref, what='dense')
    # Wan-style overlapping key ranges read in place: scene j reads frames [lo, hi + 2)
    T = 40
    lay = OL.SceneLayout([3, 4, 2], halo=2, sides='next')
    S = lay.n_frames * T
    qq, kk, vv = (rand_bf16((S, H, D), s) for s in (41, 42, 43))
    qr, kr = OL.wan_ranges(lay, T)
    o = A.overlapping_ranges(qq.to(DEV), kk.to(DEV), vv.to(DEV), qr, kr).cpu()
    cq = [0] + [b for _, b in qr]
    ref = OA.packed_attention(qq, kk, vv, cq, None, k_off=[a for a, _ in kr], k_len=[b - a for a, b in kr])
    assert_close(o, ref, what='overlapping_ranges')


def _layer_inputs(case, seed=0):
    H, D, T = case['H'], case['D'], case['T']
    S = sum(case['lengths']) * T
    q, k, v = (rand_bf16((S, H, D), seed + i) for i in range(3))
    eq, ek, ev = (rand_bf16((case['Le'], H, D), seed + 3 + i) for i in range(3))
    F, Hh, Ww = case['table']
    cos, sin = OA.rope_table_3d(F, Hh, Ww, D)
    return q, k, v, eq, ek, ev, cos, sin


@pytest.mark.parametrize('name,per_seg,rotate_q,in_place', [
    ('cpu_plumbing', None, 'pre', False), ('cpu_plumbing', None, 'load', False), ('cpu_plumbing', None, 'pre', True),
    ('hunyuan480p', 48, 'pre', False), ('hunyuan480p', 48, 'load', False), ('hunyuan480p', 48, 'pre', True),
    ('wan704', 48, 'pre', False), ('wan704', 48, 'pre', True), ('uneven_K2', 32, 'pre', False),
    ('uneven_K4', 24, 'pre', False), ('uneven_K4', 24, 'pre', True), ('uneven_K8', 24, 'pre', False),
    ('uneven_K12', 24, 'pre', False), ('uneven_K12', 24, 'pre', True)])
@pytest.mark.parametrize('adjacent', [False, True])
def test_scene_layer_matches_oracle(name, per_seg, rotate_q, in_place, adjacent):
    """the fused layer (K/V pack with RoPE, the video queries rotated once ahead of the attention call or on its Q
    load, in-place output; with in_place, each text segment's keys read from its video segment's packed rows) against
    the oracle's packing plus per-scope fp32 attention; full outputs for the CPU-plumbing layout, sampled query rows
    (every segment's first / last rows included) at the full-size configs, each segment's reference built from that
    segment's keys alone"""
    case = layout_case(name)
    print(f'layer {name} adjacent={adjacent} rotate_q={rotate_q} text keys in place={in_place}', flush=True)
    q, k, v, eq, ek, ev, cos, sin = _layer_inputs(case)
    lay = SceneLayout(case['lengths'], halo=case['halo'], sides=case['sides'], extra=case['extra'])
    plan = scene.ScopePlan(lay, case['T'], case['counts'], case['Le'], case['scene_rope'], None, adjacent, True, DEV,
                           text_keys_in_place=in_place)
    if in_place:
        assert plan.sum_k < int(plan.k_len.sum())
    g = [x.to(DEV) for x in (q, k, v, eq, ek, ev, cos, sin)]
    ov, ot = scene.scene_attention(plan, *g[:6], g[6], g[7], mode='raw', fused=True, rotate_q=rotate_q)
    olay = OL.SceneLayout(case['lengths'], case['halo'], case['sides'], case['extra'])
    sc = OL.hunyuan_scopes(olay, case['T'], case['counts'], case['Le'], scene_rope=case['scene_rope'],
                           adjacent=adjacent)
    rows = np.arange(int(sc.cu_q[-1])) if per_seg is None else sample_rows(sc.cu_q, per_seg)
    ref = scope_rows_reference(sc, q, k, v, eq, ek, ev, rows, cos, sin, mode='raw')
    got = torch.cat([ov, ot]).cpu()[torch.as_tensor(sc.q_src[rows])]
    assert_close(got, ref, what=f'{name} layer')
    valid = sum(case['counts'])
    if case['Le'] > valid:
        assert ot[valid:].abs().max().item() == 0


def _random_layer_case(rng):
    """a random layout: 2-7 scenes of 1-6 frames, 160-1590 tokens per frame (a Hh x Ww grid), 1-200 text tokens
    per scene, a halo of 0-1 frames or frame memory of up to 4 representatives, 4-12 heads of 128"""
    K = int(rng.integers(2, 8))
    lengths = rng.integers(1, 7, K).tolist()
    F = sum(lengths)
    Hh, Ww = int(rng.integers(8, 31)), int(rng.integers(20, 54))
    counts = rng.integers(1, 201, K).tolist()
    halo = int(rng.integers(0, 2))
    sides = str(rng.choice(['adj', 'next', 'prev']))
    extra = {}
    if halo == 0 and F > 1:
        lay = OL.SceneLayout(lengths, halo=0)
        reps = sorted({int(x) for x in rng.choice(F, min(F, int(rng.integers(1, 5))), replace=False)})
        fm = OL.FrameMemoryExtra(budget=4, fallback=(0, 'adj'))
        fm.reset(lay)
        fm.propose(reps)
        fm.begin_step(1)
        extra = lay.extra
    return dict(lengths=lengths, halo=halo, sides=sides, extra=extra, T=Hh * Ww, counts=counts, Le=sum(counts) + 3,
                H=int(rng.choice([4, 8, 12])), D=128, scene_rope=bool(rng.integers(2)), rope_lengths=None,
                table=(F + 8, Hh, Ww))


@pytest.mark.parametrize('seed', range(6))
def test_scene_layer_random_layouts(seed):
    """random layouts through the fused layer (query rotation ahead of the call or on the load, text keys in place
    or packed, both shared-frame positions), 24 sampled rows per segment against the oracle, and a second call
    bit-identical to the first"""
    rng = np.random.default_rng(500 + seed)
    case = _random_layer_case(rng)
    adjacent, in_place = bool(rng.integers(2)), bool(rng.integers(2))
    rotate_q = str(rng.choice(['pre', 'load']))
    print(f'random layer {seed}: {case} adjacent={adjacent} in_place={in_place} rotate_q={rotate_q}', flush=True)
    q, k, v, eq, ek, ev, cos, sin = _layer_inputs(case, seed=40 + seed)
    lay = SceneLayout(case['lengths'], halo=case['halo'], sides=case['sides'], extra=case['extra'])
    plan = scene.ScopePlan(lay, case['T'], case['counts'], case['Le'], case['scene_rope'], None, adjacent, True, DEV,
                           text_keys_in_place=in_place)
    g = [x.to(DEV) for x in (q, k, v, eq, ek, ev, cos, sin)]
    ov, ot = scene.scene_attention(plan, *g[:6], g[6], g[7], mode='raw', fused=True, rotate_q=rotate_q)
    ov2, ot2 = scene.scene_attention(plan, *g[:6], g[6], g[7], mode='raw', fused=True, rotate_q=rotate_q)
    assert torch.equal(ov2, ov) and torch.equal(ot2, ot)
    olay = OL.SceneLayout(case['lengths'], case['halo'], case['sides'], case['extra'])
    sc = OL.hunyuan_scopes(olay, case['T'], case['counts'], case['Le'], scene_rope=case['scene_rope'],
                           adjacent=adjacent)
    rows = sample_rows(sc.cu_q, 24)
    ref = scope_rows_reference(sc, q, k, v, eq, ek, ev, rows, cos, sin, mode='raw')
    got = torch.cat([ov, ot]).cpu()[torch.as_tensor(sc.q_src[rows])]
    assert_close(got, ref, what=f'random layer {seed}')


@pytest.mark.parametrize('rotate_q', ['pre', 'load'])
def test_scene_layer_repeatable_at_480p(rotate_q):
    """the full 480p layer (3264 work items, ~13 per work-group, partly filled query tiles with idle wavefronts)
    run four times with every output bit-identical. This checks that the results are deterministic across launches
    (item order and work-group assignment vary between them); it does not show the absence of races: a race whose
    outcome is the same in every run, or that these runs happen not to hit, passes. The item-boundary transitions are
    checked row by row against the oracle in tests/test_gpu_item_boundary.py"""
    case = layout_case('hunyuan480p')
    print(f'layer hunyuan480p repeatability rotate_q={rotate_q}', flush=True)
    g = [x.to(DEV) for x in _layer_inputs(case)]
    lay = SceneLayout(case['lengths'], halo=case['halo'], sides=case['sides'], extra=case['extra'])
    plan = scene.ScopePlan(lay, case['T'], case['counts'], case['Le'], case['scene_rope'], None, True, True, DEV,
                           text_keys_in_place=True)
    ov, ot = scene.scene_attention(plan, *g[:6], g[6], g[7], mode='raw', fused=True, rotate_q=rotate_q)
    assert torch.isfinite(ov).all() and torch.isfinite(ot).all()
    for _ in range(3):
        ov2, ot2 = scene.scene_attention(plan, *g[:6], g[6], g[7], mode='raw', fused=True, rotate_q=rotate_q)
        assert torch.equal(ov2, ov) and torch.equal(ot2, ot)


@pytest.mark.parametrize('rotate_q', ['pre', 'load'])
def test_scene_layer_head_chunks_at_480p(rotate_q):
    """heads are independent (the reference checks its path bit-exact across head chunkings 1/2/3/4/16,
    tests/dist_onereel_kv_chunks.py:29-37): the 480p layer run on chunks of the heads, through views of the same
    q / k / v / text rows (row stride 16 heads), gives the full layer's rows for those heads. Bit for bit while the
    chunk's call has at least 4 rounds of work items on the GPU (16 and 8 heads: 12.75 and 6.4 rounds), where items are
    cut exactly as in the full call; the chunks of 4, 3, 2 and 1 heads have fewer rounds, so the planner splits their
    last items by keys and merges the parts in fp32, which rounds differently: within a bf16 step of the full layer.
    The views' rows are wider than their heads: with rotate_q='pre' the rotated video queries land in a new buffer of
    narrower rows, and the layer lays the text queries out likewise"""
    case = layout_case('hunyuan480p')
    g = [x.to(DEV) for x in _layer_inputs(case, 5)]
    lay = SceneLayout(case['lengths'], halo=case['halo'], sides=case['sides'], extra=case['extra'])
    plan = scene.ScopePlan(lay, case['T'], case['counts'], case['Le'], case['scene_rope'], None, True, True, DEV,
                           text_keys_in_place=True)
    print(f'layer hunyuan480p, all 16 heads, rotate_q={rotate_q}', flush=True)
    ov, ot = scene.scene_attention(plan, *g[:6], g[6], g[7], mode='raw', fused=True, rotate_q=rotate_q)
    H = case['H']
    for size in (8, 4, 3, 2, 1):
        lo = 0
        while lo < H:
            hi = min(lo + size, H)
            print(f'layer hunyuan480p, heads [{lo}, {hi})', flush=True)
            cv, ct = scene.scene_attention(plan, *(x[:, lo:hi] for x in g[:6]), g[6], g[7], mode='raw', fused=True,
                                           rotate_q=rotate_q)
            if size == 8:
                assert torch.equal(cv, ov[:, lo:hi]) and torch.equal(ct, ot[:, lo:hi]), (lo, hi)
            else:
                for got, want in ((cv, ov[:, lo:hi]), (ct, ot[:, lo:hi])):
                    d = (got.float() - want.float()).abs()
                    assert d.max().item() <= 2 ** -7 * max(1.0, want.float().abs().max().item()), (lo, hi)
                    assert d.mean().item() <= 1e-4, (lo, hi)
            lo = hi


@pytest.mark.parametrize('name,P,per_seg', [('cpu_plumbing', 3, None), ('hunyuan480p', 3, 32),
                                            ('uneven_K4', 5, 24)])
def test_scene_layer_rank_shares(name, P, per_seg):
    """the layer's video tokens split over P ranks by the work-balanced partition (Algorithm 1; it cuts scenes,
    mid-frame at the full-size shapes): each rank's share, fused with in-place text keys, on its query rows against
    the oracle's token_range scopes; the sentence rows of scenes another rank runs stay zero (the reference's
    ot = eq.new_zeros before its all-reduce), and the ranks' outputs together give the one-GPU layer's"""
    case = layout_case(name)
    q, k, v, eq, ek, ev, cos, sin = _layer_inputs(case, 9)
    g = [x.to(DEV) for x in (q, k, v, eq, ek, ev, cos, sin)]
    lay = SceneLayout(case['lengths'], halo=case['halo'], sides=case['sides'], extra=case['extra'])
    olay = OL.SceneLayout(case['lengths'], case['halo'], case['sides'], case['extra'])
    T = case['T']
    adjacent = True
    full = scene.ScopePlan(lay, T, case['counts'], case['Le'], case['scene_rope'], None, adjacent, True, DEV,
                           text_keys_in_place=True)
    fv, ft = scene.scene_attention(full, *g, mode='raw', fused=True)
    text_sum = torch.zeros_like(ft)
    own = comm.partition(lay, P, T, 'scene', case['counts'])
    assert any(lo * T < a < hi * T for a, _ in own[1:] for lo, hi in lay.ranges)    # a scene is cut
    for r, (a, b) in enumerate(own):
        print(f'layer rank share {name} rank {r}/{P} tokens [{a}, {b})', flush=True)
        plan = scene.ScopePlan(lay, T, case['counts'], case['Le'], case['scene_rope'], None, adjacent, True, DEV,
                               text_keys_in_place=True, q_range=(a, b))
        ov, ot = scene.scene_attention(plan, *g, mode='raw', fused=True)
        sc = OL.hunyuan_scopes(olay, T, case['counts'], case['Le'], scene_rope=case['scene_rope'],
                               adjacent=adjacent, token_range=(a, b))
        rows = np.arange(int(sc.cu_q[-1])) if per_seg is None else sample_rows(sc.cu_q, per_seg)
        ref = scope_rows_reference(sc, q, k, v, eq, ek, ev, rows, cos, sin, mode='raw')
        got = torch.cat([ov, ot]).cpu()[torch.as_tensor(sc.q_src[rows])]
        assert_close(got, ref, what=f'{name} rank {r} of {P}')
        # the same rows of the one-GPU layer (equal up to the order of a key split's partial sums)
        assert_close(ov[a:b].cpu(), fv[a:b].cpu(), what=f'rank {r} against the one-GPU layer')
        # the reference's data flow (Q, K, V packed, varlen on packed rows, scatter) and the queries rotated on the
        # attention kernel's load give the same rows
        for kw in (dict(fused=False), dict(fused=True, rotate_q='load')):
            ov2, ot2 = scene.scene_attention(plan, *g, mode='raw', **kw)
            assert_close(ov2[a:b].cpu(), ov[a:b].cpu(), what=f'rank {r} {kw}')
            assert_close(ot2.cpu(), ot.cpu(), what=f'rank {r} {kw} text')
            del ov2, ot2
        tr = OL.text_ranges(case['counts'])
        for j, (lo, _) in enumerate(lay.ranges):
            t0, t1 = tr[j]
            if not a <= lo * T < b and t1 > t0:
                assert ot[t0:t1].abs().max().item() == 0, (r, j)
        text_sum += ot                                    # each sentence row is written by one rank alone
    assert_close(text_sum.cpu(), ft.cpu(), what='sentence rows over the ranks')


@pytest.mark.parametrize('adjacent', [False, True])
def test_scene_layer_reference_flow_and_rotated_inputs(adjacent):
    """fused=False (Q/K/V packed, varlen on packed tensors, scatter) and mode 'rotated' (already rotated q / k, shared
    keys re-rotated by _move_shared's two rotations) give the oracle's result; text padding rows stay zero"""
    case = dict(layout_case('cpu_plumbing'), Le=40)
    q, k, v, eq, ek, ev, cos, sin = _layer_inputs(case, 5)
    lay = SceneLayout(case['lengths'], halo=0, extra=case['extra'])
    olay = OL.SceneLayout(case['lengths'], 0, 'adj', case['extra'])
    sc = OL.hunyuan_scopes(olay, case['T'], case['counts'], case['Le'], scene_rope=True, adjacent=adjacent)
    g = [x.to(DEV) for x in (q, k, v, eq, ek, ev, cos, sin)]
    rv, rt = OA.scene_layer(sc, q, k, v, eq, ek, ev, cos, sin, mode='raw')
    # already-rotated inputs, as the reference's Processor.scene receives them
    rows = torch.as_tensor(OL.scene_rope_rows(olay, case['T']))
    qr = OA.apply_rotary_emb(q, cos[rows], sin[rows])
    kr = OA.apply_rotary_emb(k, cos[rows], sin[rows])
    rv2, rt2 = OA.scene_layer(sc, qr, kr, v, eq, ek, ev, cos, sin, mode='rotated')
    for in_place in (False, True):
        plan = scene.ScopePlan(lay, case['T'], case['counts'], case['Le'], True, None, adjacent, True, DEV,
                               moves=True, text_keys_in_place=in_place)
        ov, ot = scene.scene_attention(plan, *g, mode='raw', fused=False)
        assert_close(ov.cpu(), rv, what=f'unfused video, text keys in place={in_place}')
        assert_close(ot.cpu(), rt, what=f'unfused text, text keys in place={in_place}')
        assert ot[32:].abs().max().item() == 0
        for fused in (True, False):
            ov2, ot2 = scene.scene_attention(plan, qr.to(DEV), kr.to(DEV), *g[2:], mode='rotated', fused=fused)
            assert_close(ov2.cpu(), rv2, what=f'rotated video fused={fused} in place={in_place}')
            assert_close(ot2.cpu(), rt2, what=f'rotated text fused={fused} in place={in_place}')


@pytest.mark.parametrize('adjacent', [False, True])
def test_reference_flow_and_processor_scene_at_480p(adjacent):
    """at the HunyuanVideo-1.5 480p shape (4 x 8 frames x 1590 + 128 text, frame memory 4, 16 x 128), before
    (step 0, 'source') and after (step 5, 'adjacent') the shared-position switch: the reference's packed flow
    (Q / K / V packed, varlen on packed tensors, scatter) on raw inputs, and the reference's own entry
    Processor.scene on already-rotated q / k (shared keys re-rotated by _move_shared's two rotations through the full
    rotary table), fused and packed, on sampled query rows against the oracle"""
    case = layout_case('hunyuan480p')
    T = case['T']
    print(f'480p reference flow adjacent={adjacent}', flush=True)
    q, k, v, eq, ek, ev, cos, sin = _layer_inputs(case, 7)
    lay = SceneLayout(case['lengths'], halo=0, extra=case['extra'])
    olay = OL.SceneLayout(case['lengths'], 0, 'adj', case['extra'])
    sc = OL.hunyuan_scopes(olay, T, case['counts'], case['Le'], scene_rope=True, adjacent=adjacent)
    rows = sample_rows(sc.cu_q, 24, seed=3)
    src = torch.as_tensor(sc.q_src[rows])
    g = [x.to(DEV) for x in (q, k, v, eq, ek, ev, cos, sin)]
    plan = scene.ScopePlan(lay, T, case['counts'], case['Le'], True, None, adjacent, True, DEV, moves=True)
    ov, ot = scene.scene_attention(plan, *g, mode='raw', fused=False)
    ref = scope_rows_reference(sc, q, k, v, eq, ek, ev, rows, cos, sin, mode='raw')
    assert_close(torch.cat([ov, ot]).cpu()[src], ref, what='480p packed flow, raw inputs')
    del ov, ot
    rr = torch.as_tensor(OL.scene_rope_rows(olay, T))
    qr = OA.apply_rotary_emb(q, cos[rr], sin[rr])
    kr = OA.apply_rotary_emb(k, cos[rr], sin[rr])
    ref = scope_rows_reference(sc, qr, kr, v, eq, ek, ev, rows, cos, sin, mode='rotated')
    ctx = HY.Context(lay, T=T, scene_rope=True, shared_pos='switch', shared_switch=5, cfg=True)
    ctx.counts = {True: case['counts']}
    ctx.fwd = 11 if adjacent else 1                       # step 5 or step 0, conditional branch
    ctx._rot_full = (g[6], g[7])
    assert ctx.adjacent() == adjacent
    gqr, gkr = qr.to(DEV), kr.to(DEV)
    for fused in (True, False):
        ctx.fused = fused
        ov, ot = HY.Processor(ctx, 0).scene(gqr, gkr, g[2], g[3], g[4], g[5])
        assert_close(torch.cat([ov, ot]).cpu()[src], ref, what=f'480p Processor.scene fused={fused}')
        del ov, ot


@torch.no_grad()
def test_processor_call_matches_oracle_layer():
    """Processor.__call__ (diffusers signature) = projections -> oracle layer (RoPE + scopes + attention) -> outputs,
    at step >= shared_switch (moved shared frames) with scene RoPE"""
    gen = torch.Generator().manual_seed(3)
    H, D, T = 2, 64, 16
    C = H * D
    lay = SceneLayout([3, 2, 3], halo=0, extra={0: [4, 7], 1: [0, 7], 2: [0, 4]})
    counts = [5, 3, 4]
    Le = 14
    attn = _Attn(C, H, gen)
    hs = (torch.randn(1, lay.n_frames * T, C, generator=gen) * 0.5).bfloat16()
    ehs = (torch.randn(1, Le, C, generator=gen) * 0.5).bfloat16()
    cos, sin = OA.rope_table_3d(lay.n_frames, 4, 4, D)
    ctx = HY.Context(lay, T=T, scene_rope=True, shared_pos='switch', shared_switch=1, cfg=False)
    ctx.counts = {True: counts}
    ctx.fwd = 2                                                            # step 1 >= switch: adjacent
    proc = HY.Processor(ctx, 0)
    attn_g = _Attn(C, H, torch.Generator().manual_seed(3)).to(DEV)
    attn_g.load_state_dict(attn.state_dict())
    out, eout = proc(attn_g, hs.to(DEV), ehs.to(DEV), None, (cos.to(DEV), sin.to(DEV)))
    # reference: the same projections on the CPU, the oracle's layer, the same output projections
    q, k, v = (f(hs).unflatten(2, (H, -1)) for f in (attn.to_q, attn.to_k, attn.to_v))
    q, k = attn.norm_q(q), attn.norm_k(k)
    eq, ek, ev = (f(ehs).unflatten(2, (H, -1)) for f in (attn.add_q_proj, attn.add_k_proj, attn.add_v_proj))
    eq = attn.norm_added_q(eq)
    sc = OL.hunyuan_scopes(OL.SceneLayout([3, 2, 3], 0, 'adj', lay.extra), T, counts, Le, scene_rope=True,
                           adjacent=True)
    rv, rt = OA.scene_layer(sc, q[0].bfloat16(), k[0].bfloat16(), v[0].bfloat16(), eq[0].bfloat16(),
                            ek[0].bfloat16(), ev[0].bfloat16(), cos, sin, mode='raw')
    assert_close(proc.scene_raw(*(x[0].bfloat16().to(DEV) for x in (q, k, v, eq, ek, ev)), cos.to(DEV),
                                sin.to(DEV))[0].cpu(), rv, what='scene_raw')
    ref_out = attn.to_out[1](attn.to_out[0](rv.bfloat16().flatten(1, 2)[None]))
    ref_eout = attn.to_add_out(rt.bfloat16().flatten(1, 2)[None])
    assert_close(out.cpu(), ref_out, max_abs=5e-2, mean_abs=5e-3, what='processor hs')
    assert_close(eout.cpu(), ref_eout, max_abs=5e-2, mean_abs=5e-3, what='processor ehs')
    assert HY.scene_rope_rows(ctx, DEV).cpu().tolist() == OL.scene_rope_rows(OL.SceneLayout([3, 2, 3], 0), T).tolist()


@torch.no_grad()
def test_wan_self_and_cross_ranges():
    H, D, T = 3, 128, 24
    ctx = W.Context(SceneLayout([3, 4, 2], halo=2, sides='next'), T=T, text_len=20)
    S = 9 * T
    q, k, v = (rand_bf16((S, H, D), s) for s in (51, 52, 53))
    o = W.self_ranges(ctx, q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    qr, kr = OL.wan_ranges(OL.SceneLayout([3, 4, 2], 2, 'next'), T)
    ref = OA.packed_attention(q, k, v, [0] + [b for _, b in qr], None, k_off=[a for a, _ in kr],
                              k_len=[b - a for a, b in kr])
    assert_close(o, ref, what='wan self zero-copy')
    # with frame-memory extras: packed video-only scopes
    ctx.layout = SceneLayout([3, 4, 2], halo=0, extra={0: [5, 8], 1: [0], 2: [1, 4]})
    o = W.self_ranges(ctx, q.to(DEV), k.to(DEV), v.to(DEV)).cpu()
    sc = OL.hunyuan_scopes(OL.SceneLayout([3, 4, 2], 0, 'adj', ctx.layout.extra), T, [0, 0, 0], 0, with_text=False)
    qp, kp, vp = OA.pack(sc, q, k, v, q[:0], k[:0], v[:0], mode='none')
    ref = OA.write_back(sc, OA.packed_attention(qp, kp, vp, sc.cu_q, sc.cu_k), 0)[0]
    assert_close(o, ref, what='wan self packed')
    # cross-attention: scene j reads sentence j
    e = rand_bf16((60, H, D), 54)
    ev = rand_bf16((60, H, D), 55)
    o = W.cross_ranges(ctx, q.to(DEV), e.to(DEV), ev.to(DEV)).cpu()
    cq = [0, 3 * T, 7 * T, 9 * T]
    ref = OA.packed_attention(q, e, ev, cq, None, k_off=[0, 20, 40], k_len=[20, 20, 20])
    assert_close(o, ref, what='wan cross')


def test_native_library_is_the_in_tree_build():
    """the HIP path runs from the in-tree libonereel_hip.so (no fallback exists)"""
    L.lib()
    maps = open('/proc/self/maps').read()
    assert str(L.LIB_PATH) in maps


@pytest.mark.parametrize('split', [0, 1, 300, 777])
def test_lse_merge_of_two_key_sets(split):
    """varlen_lse over keys [0, split) and [split, 777) of each segment, merged by or_lse_merge: equals the oracle's
    ring._merge of the same partial results (fp32, 1e-5) and attention over all keys (bf16 tolerance)"""
    print(f'lse merge split={split}', flush=True)
    H, D, nk = 3, 128, 777
    lq = [65, 130]
    q = rand_bf16((sum(lq), H, D), 41)
    k = rand_bf16((2 * nk, H, D), 42)
    v = rand_bf16((2 * nk, H, D), 43)
    cq = torch.tensor([0, lq[0], sum(lq)], dtype=torch.int32, device=DEV)

    def part(a, b):
        # an empty key set is passed as zero-length segments over a one-row buffer (the kernel's Lk = 0 path)
        kk = torch.cat([k[s * nk + a:s * nk + b] for s in range(2)] + [k[:1]]).to(DEV)
        vv = torch.cat([v[s * nk + a:s * nk + b] for s in range(2)] + [v[:1]]).to(DEV)
        ck = torch.tensor([0, b - a, 2 * (b - a)], dtype=torch.int32, device=DEV)
        return A.varlen_lse(q.to(DEV), kk, vv, cq, ck, max(lq), max(b - a, 1))

    o1, l1 = part(0, split)
    o2, l2 = part(split, nk)
    ref_o, ref_l = OA.merge_lse(o1.float().cpu(), l1.cpu(), o2.cpu(), l2.cpu())
    o, lse = o1.float(), l1.clone()
    A.merge_lse(o, lse, o2, l2)
    torch.cuda.synchronize()
    assert (o.cpu() - ref_o).abs().max() < 1e-5 and (lse.cpu() - ref_l).abs().max() < 1e-5
    full = OA.packed_attention(q, k, v, np.array([0, lq[0], sum(lq)]), np.array([0, nk, 2 * nk]))
    assert_close(o.cpu(), full, what='merged attention')
    if split in (0, nk):   # one side empty: the other side's result, unchanged
        keep, other = (o2, l2) if split == 0 else (o1, l1)
        assert torch.equal(o.cpu(), keep.float().cpu()) and torch.equal(lse.cpu(), other.cpu())


@pytest.mark.parametrize('S,heads,D', [(257, 24, 128), (64, 4, 128), (33, 16, 64)])
def test_wan_qk_fused_norm_rope(S, heads, D):
    """or_rmsnorm_rope (through wan._qk) against the oracle's fp32 restatement of _qk (wan.py:64-74): both fp32 with
    one rounding, so they differ by at most one bf16 step and almost never; q and k read from strided views"""
    print(f'wan _qk S={S} heads={heads} D={D}', flush=True)
    from oracle import wan as OW
    C = heads * D
    g = torch.Generator().manual_seed(S)
    qkv = (torch.randn(S, 3 * C, generator=g) * 3).to(torch.bfloat16)       # a fused projection: q / k are views
    wq, wk = (torch.rand(C, generator=g) + 0.5).to(torch.bfloat16), (torch.rand(C, generator=g) + 0.5).to(torch.bfloat16)
    ang = torch.randn(S, D // 2, generator=g)
    cos, sin = ang.cos().repeat_interleave(2, 1), ang.sin().repeat_interleave(2, 1)
    dev = qkv.to(DEV)
    qo, ko = W._qk(dev[None, :, :C], dev[None, :, C:2 * C], wq.to(DEV), wk.to(DEV), 1e-6, cos[None, :, None].to(DEV),
                   sin[None, :, None].to(DEV), heads)
    assert qo.shape == (1, S, heads, D)
    for got, x, w in ((qo, qkv[:, :C], wq), (ko, qkv[:, C:2 * C], wk)):
        ref = OW.qk_norm_rope(x, w, 1e-6, cos, sin, heads)
        got = got[0].cpu()
        diff = (got.float() - ref.float()).abs()
        assert (diff <= ref.float().abs() * 2 ** -7 + 1e-6).all(), diff.max()
        assert (got.view(torch.int16) == ref.view(torch.int16)).float().mean() > 0.99
