"""GPU parity of the head-major bounded memory (onereel_amd.memory, csrc/memory.hip) with the oracle:

- the representative choice (or_memory_select) against the oracle's restatement of BoundaryMemory.select on
  separated groups of keys, cold and warm (a second call from the stored centroids on perturbed keys), at head_dim 64
  and 128, with more clusters than one LDS chunk, from bf16 and fp32 keys; the reference's own memory tests (every
  candidate kept when the budget covers them; each representative the nearest member of its cluster);
- the packed single-head attention (or_memory_index, pack, varlen with in-place queries, or gather / scatter) against
  fp32 attention over each piece's local keys plus its head's foreign representatives: the reference test's layouts
  (tests/test_onereel_memory.py) on two calls in a row, a plan with permuted query rows, and the HunyuanVideo-1.5 480p
  layer's shape on sampled rows."""
import numpy as np
import pytest
import torch

from helpers import assert_close
from onereel_amd.layout import SceneLayout
from onereel_amd.memory import BoundaryMemory, MemoryAttention, candidates, frame_plan, make_plan
from oracle import memory as OM

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]
DEV = 'cuda'


def _groups(g, k, per, H, D, noise):
    base = torch.randn(k, H, D, generator=g)
    return torch.cat([base[i].expand(per, -1, -1) for i in range(k)]) + noise * torch.randn(k * per, H, D, generator=g)


def _same_sets(got, gv, ref, rv):
    for h in range(got.shape[0]):
        assert sorted(got[h][gv[h]].cpu().tolist()) == sorted(ref[h][rv[h]].tolist()), h


@pytest.mark.parametrize('k,per,H,D,M,dtype', [
    (5, 9, 3, 64, 5, torch.float32),
    (6, 7, 2, 128, 6, torch.bfloat16),
    (40, 5, 2, 128, 40, torch.float32),
    (150, 3, 2, 64, 150, torch.float32),      # M > 128: two centroid chunks of the distance pass
])
def test_select_matches_oracle_cold_and_warm(k, per, H, D, M, dtype):
    """one cluster per group (M = the group count; more clusters than groups split a group by the noise, and a
    two-member cluster's members are equidistant from its mean: ties that fp32 rounding decides), members spread
    (noise 0.1) so that the nearest member of each group is not a tie at the fp32 rounding of the |x|^2 - 2 x.c +
    |c|^2 distances (the oracle takes explicit differences); the warm call on perturbed keys runs two passes from the
    stored centroids, as the oracle does from its own"""
    print(f'select k={k} per={per} H={H} D={D} M={M} {dtype}', flush=True)
    g = torch.Generator().manual_seed(7 + D + M)
    xs = _groups(g, k, per, H, D, 0.1).to(dtype)
    mem = BoundaryMemory(M)
    got, gv = mem.select('a', xs.to(DEV))
    ref, rv, c_ref = OM.select(xs, M, centroids=True)
    _same_sets(got, gv, ref, rv)
    assert mem.centroids['a'].shape == (H, min(M, k * per), D)
    xs2 = (xs.float() + 0.02 * torch.randn(xs.shape, generator=g)).to(dtype)
    got2, gv2 = mem.select('a', xs2.to(DEV))
    ref2, rv2 = OM.select(xs2, M, iters=2, start=c_ref)
    _same_sets(got2, gv2, ref2, rv2)


@pytest.mark.parametrize('k,per,H,D', [(100, 30, 2, 64), (40, 60, 1, 128)])
def test_select_matches_oracle_beyond_one_sort_chunk(k, per, H, D):
    """3000 and 2400 candidates, past the 1024 that one pass of the grouping kernel's wavefronts covers (each then
    sorts several 64-candidate chunks and carries a running per-cluster count between them), in k separated groups
    with M = k: the oracle's representatives, cold and warm, and every stored centroid the mean of the normalised keys
    of its cluster (members recomputed here in float64 from the final centroids: a wrong grouping would give wrong
    means)"""
    print(f'select beyond one sort chunk k={k} per={per} H={H} D={D}', flush=True)
    g = torch.Generator().manual_seed(k + per)
    B = k * per
    # groups interleaved over the candidates, except that the cold start's evenly spaced candidates are one member
    # of each group (so that no group starts with two centroids and splits: a split's members sit near two centroids
    # at once, a tie that the fp32 rounding of the distances decides)
    init = torch.linspace(0, B - 1, k).round().long()
    rest = torch.ones(B, dtype=torch.bool)
    rest[init] = False
    group = torch.empty(B, dtype=torch.long)
    group[init] = torch.arange(k)
    group[rest] = torch.arange(k).repeat_interleave(per - 1)[torch.randperm(B - k, generator=g)]
    centers = torch.randn(k, H, D, generator=g)
    xs = centers[group] + 0.1 * torch.randn(B, H, D, generator=g)
    mem = BoundaryMemory(k)
    got, gv = mem.select('b', xs.to(DEV))
    c = mem.centroids['b'].cpu().double()
    xn = torch.nn.functional.normalize(xs.double().transpose(0, 1), dim=-1)
    for h in range(H):
        z = torch.cdist(xn[h], c[h]).argmin(-1)
        assert torch.equal(torch.unique(z), torch.arange(k))       # one cluster per group, none empty
        for i in range(k):
            assert torch.allclose(c[h, i], xn[h, z == i].mean(0), atol=1e-5), (h, i)
    ref, rv, c_ref = OM.select(xs, k, centroids=True)
    _same_sets(got, gv, ref, rv)
    xs2 = xs + 0.02 * torch.randn(xs.shape, generator=g)
    got2, gv2 = mem.select('b', xs2.to(DEV))
    ref2, rv2 = OM.select(xs2, k, iters=2, start=c_ref)
    _same_sets(got2, gv2, ref2, rv2)


def test_select_keeps_every_candidate_when_the_budget_covers_them():
    lay = SceneLayout([3, 4, 2], halo=0)
    T, H, D = 8, 2, 64
    rows, _ = candidates(lay, T, DEV)
    k = torch.randn(lay.n_frames * T, H, D, generator=torch.Generator().manual_seed(1)).to(DEV)
    rep, valid = BoundaryMemory(len(rows)).select('x', k[rows])
    for h in range(H):
        assert sorted(rep[h][valid[h]].tolist()) == list(range(len(rows)))


@pytest.mark.parametrize('B,H,D,M', [(300, 3, 64, 12), (2000, 2, 128, 128), (777, 1, 128, 200)])
def test_select_nearest_member_and_layout(B, H, D, M):
    """each representative is the member of its cluster nearest the returned centroids (clusters and distances
    recomputed here in float64), the representatives are distinct, valid ones come first, padding is (0, False)"""
    g = torch.Generator().manual_seed(B)
    x = torch.randn(B, H, D, generator=g)
    mem = BoundaryMemory(M)
    rep, valid = mem.select('y', x.to(DEV))
    c = mem.centroids['y'].cpu().double()
    xn = torch.nn.functional.normalize(x.double().transpose(0, 1), dim=-1)
    for h in range(H):
        n = int(valid[h].sum())
        assert n > 0 and bool(valid[h, :n].all()) and not bool(valid[h, n:].any())
        chosen = rep[h, :n].cpu().tolist()
        assert len(set(chosen)) == n and int(rep[h, n:].abs().sum()) == 0
        d = torch.cdist(xn[h], c[h]) ** 2
        z = d.argmin(-1)
        for r in chosen:
            members = (z == z[r]).nonzero().flatten()
            assert d[members, z[r]].min() >= d[r, z[r]] - 1e-5


def _inputs(lengths, counts, T, H, D, seed):
    g = torch.Generator().manual_seed(seed)
    S, Le = sum(lengths) * T, sum(counts)
    q, k, v = (torch.randn(S + Le, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
    tr, c = [], 0
    for n in counts:
        tr.append((c, c + n))
        c += n
    return q, k, v, tr


def _piece_reference(q, k, v, pieces, cand, owner, rep, valid, sample=None, seed=0):
    """fp32 softmax attention per (piece, head) over the piece's local keys plus, when it reads the memory, its head's
    valid representatives of other scenes: {piece index: (query rows, out [rows, H, D])}"""
    H, D = q.shape[1], q.shape[2]
    rng = np.random.default_rng(seed)
    out = {}
    for i, (scene, qrows, krows, reads) in enumerate(pieces):
        qrows = np.asarray(qrows)
        if sample is not None and len(qrows) > sample:
            qrows = np.unique(np.concatenate([qrows[[0, -1]], rng.choice(qrows, sample, replace=False)]))
        o = torch.empty(len(qrows), H, D)
        for h in range(H):
            far = [int(cand[r]) for r, ok in zip(rep[h].tolist(), valid[h].tolist())
                   if ok and reads and int(owner[r]) != scene]
            keys = torch.as_tensor(list(krows) + far)
            p = torch.softmax(q[qrows, h].float() @ k[keys, h].float().T * D ** -0.5, -1)
            o[:, h] = p @ v[keys, h].float()
        out[i] = (qrows, o)
    return out


def _frame_pieces(lay, T, S, tr):
    own = {j: [f * T + t for f in lay.frames[j] for t in range(T)] + [S + t for t in range(*tr[j])]
           for j in range(lay.n_scenes)}
    return ([(j, list(range(lo * T, hi * T)), own[j], True) for j, (lo, hi) in enumerate(lay.ranges)] +
            [(j, [S + t for t in range(*tr[j])], own[j], False) for j in range(lay.n_scenes)])


@pytest.mark.parametrize('lengths,M,D', [([3, 5, 2, 4], 8, 64), ([2, 2, 2], 1000, 64), ([6, 1, 3], 5, 128)])
def test_memory_attention_two_calls_match_reference(lengths, M, D):
    """the reference test's layouts (16 tokens per frame, 4 heads): a cold call, then a warm call on new keys and
    values (the stored centroids move two passes); each against fp32 attention with the representatives an identical
    memory picks (the choice is deterministic)"""
    print(f'memory attention lengths={lengths} M={M} D={D}', flush=True)
    T, H = 16, 4
    lay = SceneLayout(lengths, halo=0)
    S = lay.n_frames * T
    counts = [5, 7, 3, 6][:lay.n_scenes]
    plan_q = None
    mem, twin = MemoryAttention(BoundaryMemory(M)), BoundaryMemory(M)
    for call in range(2):
        q, k, v, tr = _inputs(lengths, counts, T, H, D, call)
        if plan_q is None:
            plan_q = frame_plan(lay, T, torch.arange(S), S, [(j, lo * T, hi * T) for j, (lo, hi) in
                                                            enumerate(lay.ranges)], tr, set(range(lay.n_scenes)), S,
                                DEV)
        out = mem(('l0', True), q.to(DEV), k.to(DEV), v.to(DEV), plan_q).cpu()
        rows, owner = candidates(lay, T, 'cpu')
        rep, valid = twin.select(('l0', True), k.to(DEV)[rows.to(DEV)])
        ref = _piece_reference(q, k, v, _frame_pieces(lay, T, S, tr), rows, owner, rep.cpu(), valid.cpu())
        for i, (qr, o) in ref.items():
            assert_close(out[qr], o, what=f'call {call} piece {i}')


def test_memory_attention_permuted_query_rows():
    """a plan whose pieces list their query rows out of order (the gather / scatter path); rows no piece names stay
    zero"""
    T, H, D, M = 8, 2, 128, 6
    lay = SceneLayout([3, 2], halo=0)
    S = lay.n_frames * T
    q, k, v, tr = _inputs([3, 2], [0, 0], T, H, D, 5)
    rows, owner = candidates(lay, T, 'cpu')
    g = np.random.default_rng(3)
    pieces = [(0, g.permutation(24)[:20].tolist(), list(range(24)), True), (1, list(range(39, 23, -1)),
                                                                           list(range(24, 40)), True)]
    plan = make_plan(pieces, rows, owner, DEV)
    out = MemoryAttention(BoundaryMemory(M))('p', q.to(DEV), k.to(DEV), v.to(DEV), plan).cpu()
    rep, valid = BoundaryMemory(M).select('p', k.to(DEV)[rows.to(DEV)])
    ref = _piece_reference(q, k, v, pieces, rows, owner, rep.cpu(), valid.cpu())
    named = set()
    for i, (qr, o) in ref.items():
        assert_close(out[qr], o, what=f'permuted piece {i}')
        named |= set(qr.tolist())
    rest = [r for r in range(S) if r not in named]
    assert out[rest].abs().max().item() == 0


def test_memory_attention_at_480p_shape():
    """the HunyuanVideo-1.5 480p layer's shape (4 scenes x 8 frames x 1590 tokens + 128 text each, 16 heads x 128,
    M = 128): two calls in a row, sampled query rows of every piece against fp32 attention over the same keys"""
    T, H, D, M = 1590, 16, 128, 128
    lengths, counts = [8] * 4, [128] * 4
    lay = SceneLayout(lengths, halo=0)
    S = lay.n_frames * T
    dev_gen = torch.Generator(device=DEV)
    mem, twin = MemoryAttention(BoundaryMemory(M)), BoundaryMemory(M)
    tr = [(128 * j, 128 * j + 128) for j in range(4)]
    plan = frame_plan(lay, T, torch.arange(S), S, [(j, lo * T, hi * T) for j, (lo, hi) in enumerate(lay.ranges)], tr,
                      set(range(4)), S, DEV)
    rows, owner = candidates(lay, T, 'cpu')
    pieces = _frame_pieces(lay, T, S, tr)
    for call in range(2):
        print(f'memory attention 480p call {call}', flush=True)
        dev_gen.manual_seed(40 + call)
        q, k, v = (torch.randn(S + 512, H, D, generator=dev_gen, device=DEV).to(torch.bfloat16) for _ in range(3))
        out = mem(('layer', True), q, k, v, plan).cpu()
        rep, valid = twin.select(('layer', True), k[rows.to(DEV)])
        assert int(valid.sum(1).min()) > 100        # 128 clusters over 12720 keys: almost all non-empty
        ref = _piece_reference(q.cpu(), k.cpu(), v.cpu(), pieces, rows, owner, rep.cpu(), valid.cpu(), sample=12,
                               seed=call)
        for i, (qr, o) in ref.items():
            assert_close(out[qr], o, what=f'480p call {call} piece {i}')


@torch.no_grad()
def test_processor_call_routes_the_bounded_memory_at_480p():
    """Processor.__call__ (diffusers signature) with Context.memory = 128 at the HunyuanVideo-1.5 480p shape (4 scenes
    x 8 frames x 1590 tokens + 128 text tokens each and 6 padding rows, 16 heads x 128, scene RoPE), as the reference
    routes it (hunyuan15.py:200-201,305-334): the projections, q / k rotated once in token order, the head-major
    bounded memory, the output projections. Sampled rows of both outputs against oracle.memory.masked_reference over
    the same module's projections, rotated by the oracle's apply_rotary_emb, with the representatives that an
    identical memory picks from those keys (the choice is deterministic), then projected by the same output layers"""
    from helpers import Attn
    from onereel_amd import hunyuan15 as HY
    from oracle import attention as OA
    from oracle import layout as OL
    gen = torch.Generator().manual_seed(8)
    T, H, D, M = 1590, 16, 128, 128
    C = H * D
    lengths, counts = [8] * 4, [128] * 4
    lay = SceneLayout(lengths, halo=0)
    S, Le = lay.n_frames * T, sum(counts) + 6
    attn = Attn(C, H, gen).to(DEV)
    hs = (torch.randn(1, S, C, generator=gen) * 0.5).bfloat16().to(DEV)
    ehs = (torch.randn(1, Le, C, generator=gen) * 0.5).bfloat16().to(DEV)
    cos, sin = OA.rope_table_3d(lay.n_frames, 30, 53, D)
    ctx = HY.Context(lay, T=T, scene_rope=True, cfg=False, memory=M)
    ctx.counts, ctx.fwd = {True: counts}, 1
    print('processor with bounded memory, 480p', flush=True)
    out, eout = HY.Processor(ctx, 0)(attn, hs, ehs, None, (cos.to(DEV), sin.to(DEV)))
    assert ctx._mem is not None and len(ctx._mem.plans) == 1 and (0, True) in ctx._mem.memory.centroids
    q, k, v = (f(hs).unflatten(2, (H, -1)) for f in (attn.to_q, attn.to_k, attn.to_v))
    q, k = attn.norm_q(q), attn.norm_k(k)
    eq, ek, ev = (f(ehs).unflatten(2, (H, -1)) for f in (attn.add_q_proj, attn.add_k_proj, attn.add_v_proj))
    eq = attn.norm_added_q(eq)
    rr = torch.as_tensor(OL.scene_rope_rows(OL.SceneLayout(lengths, 0), T))
    qr, kr = (OA.apply_rotary_emb(x[0].bfloat16().cpu(), cos[rr], sin[rr]) for x in (q, k))
    cand, owner = candidates(lay, T, 'cpu')
    rep, valid = BoundaryMemory(M).select((0, True), kr.to(DEV)[cand.to(DEV)])
    rep, valid = rep.cpu(), valid.cpu()
    tr = [(128 * j, 128 * j + 128) for j in range(4)]
    rng = np.random.default_rng(0)
    vr = sorted({r for lo, hi in lay.ranges for r in [lo * T, hi * T - 1, *rng.integers(lo * T, hi * T, 10).tolist()]})
    trs = sorted({t for a, b in tr for t in [a, b - 1, *rng.integers(a, b, 4).tolist()]})
    rv, rt = OM.masked_reference(qr, kr, v[0].cpu(), eq[0].cpu(), ek[0].cpu(), ev[0].cpu(), lay.ranges, T, cand[rep],
                                 owner[rep], valid, tr, video_rows=vr, text_rows=trs)
    ref_out = attn.to_out[0](rv[vr].bfloat16().flatten(1).to(DEV)).cpu()
    ref_eout = attn.to_add_out(rt[trs].bfloat16().flatten(1).to(DEV)).cpu()
    assert_close(out[0, vr].cpu(), ref_out, max_abs=5e-2, mean_abs=5e-3, what='480p processor hs with memory')
    assert_close(eout[0, trs].cpu(), ref_eout, max_abs=5e-2, mean_abs=5e-3, what='480p processor ehs with memory')
    # the padding text rows attend to nothing: their output is the projection of zeros
    pad = attn.to_add_out(torch.zeros(1, C, dtype=torch.bfloat16, device=DEV)).cpu()
    assert torch.equal(eout[0, sum(counts):].cpu(), pad.expand(6, -1))


@torch.no_grad()
def test_wan_self_attention_routes_the_bounded_memory():
    """the Wan processor's self-attention with Context.memory = M (wan.py:100-101,154-173): every scene's queries over
    its frames plus its head's representatives of the other scenes, against oracle.memory.masked_reference (no
    text scopes), on two calls in a row (cold, then warm from the stored centroids, as an identical memory picks)"""
    from onereel_amd import wan as W
    T, H, D, M = 24, 3, 128, 6
    lay = SceneLayout([3, 4, 2], halo=0)
    S = lay.n_frames * T
    ctx = W.Context(lay, T=T, memory=M)
    twin = BoundaryMemory(M)
    cand, owner = candidates(lay, T, 'cpu')
    empty = torch.zeros(0, H, D, dtype=torch.bfloat16)
    for call in range(2):
        q, k, v = (torch.randn(S, H, D, generator=torch.Generator().manual_seed(20 + 3 * call + i)).bfloat16()
                   for i in range(3))
        o = W.memory_self(ctx, q.to(DEV), k.to(DEV), v.to(DEV), 4).cpu()
        rep, valid = twin.select((4, True), k.to(DEV)[cand.to(DEV)])
        rep, valid = rep.cpu(), valid.cpu()
        rv, _ = OM.masked_reference(q, k, v, empty, empty, empty, lay.ranges, T, cand[rep], owner[rep], valid,
                                    [(0, 0)] * 3)
        assert_close(o, rv, what=f'wan memory call {call}')


def test_select_matches_oracle_at_480p_shape():
    """the HunyuanVideo-1.5 480p layer's candidate count (12 720 boundary keys per head: 4 scenes x 2 frames x 1590
    tokens), 16 heads x 128, M = 128: keys in 128 separated groups laid out in candidate order (so that the cold
    start's evenly spaced candidates seed one centroid per group), cold and then warm on perturbed keys. On heads
    whose representatives are not decided by rounding (every cluster's nearest member nearer its centroid than the
    next member by more than 1e-5, float64; checked here, not assumed), the GPU's representatives are the oracle's"""
    B, H, D, M = 8 * 1590, 16, 128, 128
    g = torch.Generator().manual_seed(480)
    group = torch.arange(B) * M // B
    centers = torch.randn(M, H, D, generator=g)
    noise = 0.05 * torch.randn(B, H, D, generator=g)
    noise[torch.unique(group, return_inverse=False, return_counts=True)[1].cumsum(0) - 7] = 0.0
    xs = centers[group] + noise        # one member of each group at its centre: its medoid by a wide margin
    xs2 = xs + 0.01 * torch.randn(B, H, D, generator=g)
    mem = BoundaryMemory(M)
    print('select at the 480p shape, cold and warm', flush=True)
    got, gv = mem.select('480p', xs.to(DEV).to(torch.bfloat16))
    c1 = mem.centroids['480p'].clone()
    got2, gv2 = mem.select('480p', xs2.to(DEV).to(torch.bfloat16))
    checked = 0
    for h in (0, 7, 15):
        x = xs[:, h:h + 1].to(torch.bfloat16)
        ref, rv, c_ref = OM.select(x, M, centroids=True)
        x2 = xs2[:, h:h + 1].to(torch.bfloat16)
        ref2, rv2 = OM.select(x2, M, iters=2, start=c_ref)
        # the margin: per cluster, the gap between its nearest and next-nearest member (float64, oracle centroids)
        xn = torch.nn.functional.normalize(x.double()[:, 0], dim=-1)
        d = torch.cdist(xn, c_ref[0].double()) ** 2
        z = d.argmin(-1)
        gaps = [(lambda s: float(s[1] - s[0]) if len(s) > 1 else 1.0)(d[z == i, i].sort().values)
                for i in range(M) if bool((z == i).any())]
        if min(gaps) <= 1e-5:
            continue
        checked += 1
        assert sorted(got[h][gv[h]].tolist()) == sorted(ref[0][rv[0]].tolist()), h
        assert torch.allclose(c1[h].cpu().double(), c_ref[0].double(), atol=1e-5), h
        assert sorted(got2[h][gv2[h]].tolist()) == sorted(ref2[0][rv2[0]].tolist()), h
    assert checked >= 2


@pytest.mark.parametrize('lengths,T,H,D,M', [([3, 5, 2, 4], 16, 4, 64, 8), ([6, 1, 3], 16, 4, 128, 5),
                                             ([8] * 4, 1590, 16, 128, 128)])
def test_multi_head_and_single_head_forms_agree(lengths, T, H, D, M):
    """the multi-head form (local keys packed as whole rows, their leading token run's values read in place, each
    head's representatives in its own head slot, per-head key counts) and the single-head form (segment per head and
    piece over rows of D elements) give the same output bits: the same keys in the same order for every (piece, head),
    read from other addresses; two calls in a row (cold, then warm)"""
    print(f'memory forms agree lengths={lengths} T={T} H={H} D={D} M={M}', flush=True)
    lay = SceneLayout(lengths, halo=0)
    S = lay.n_frames * T
    counts = [128] * len(lengths) if T > 100 else [5, 7, 3, 6][:len(lengths)]
    tr, c = [], 0
    for x in counts:
        tr.append((c, c + x))
        c += x
    plan = frame_plan(lay, T, torch.arange(S), S, [(j, lo * T, hi * T) for j, (lo, hi) in enumerate(lay.ranges)], tr,
                      set(range(lay.n_scenes)), S, DEV)
    mh, sh = MemoryAttention(BoundaryMemory(M)), MemoryAttention(BoundaryMemory(M), head_major=True)
    g = torch.Generator(device=DEV)
    for call in range(2):
        g.manual_seed(70 + call)
        q, k, v = (torch.randn(S + c, H, D, generator=g, device=DEV).to(torch.bfloat16) for _ in range(3))
        a = mh(('l', True), q, k, v, plan)
        b = sh(('l', True), q, k, v, plan)
        assert torch.equal(a, b), (call, (a.float() - b.float()).abs().max().item())
