"""GPU parity of the keys and values read in place: the attention kernels' value stream switching from token-order
rows (or_varlen_args.v_tok, the first v_lead keys of a segment) to packed rows, the key stream likewise (k_tok,
k_lead), the one-launch pack of a layer (or_pack_layer: keys, the values not read in place, the rotated queries), and
the layer with and without in-place values."""
import numpy as np
import pytest
import torch

from helpers import assert_close, layout_case, rand_bf16
from onereel_amd import scene
from onereel_amd.layout import SceneLayout
from oracle import attention as OA
from oracle import layout as OL

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]
DEV = 'cuda'
POISON = 3.0e4   # packed value rows the kernel must not read hold this (a read would move O far out of tolerance)


def _lse_ref(q, k, cq, ck, D):
    out = []
    for s in range(len(cq) - 1):
        qs, ks = q[cq[s]:cq[s + 1]].float(), k[ck[s]:ck[s + 1]].float()
        out.append(torch.logsumexp(torch.einsum('qhd,khd->hqk', qs, ks) * D ** -0.5, -1))
    return torch.cat(out, 1)


def _in_place_case(lq, lk, lead_blocks, H, D, seed):
    """segments with lq queries and lk keys; segment s takes the values of its first 32 * lead_blocks[s] keys from a
    token-order tensor (at a random row), the others from the packed values, whose rows under the in-place keys hold
    POISON. Returns the device arguments and the values as one packed tensor (the reference)."""
    rng = np.random.default_rng(seed)
    q = rand_bf16((sum(lq), H, D), seed)
    k = rand_bf16((sum(lk), H, D), seed + 1)
    v = rand_bf16((sum(lk), H, D), seed + 2)
    cq, ck = np.cumsum([0] + lq), np.cumsum([0] + lk)
    lead = [32 * b for b in lead_blocks]
    n_tok = sum(lead) + 500
    vtok = rand_bf16((n_tok, H, D), seed + 3)
    rows = [int(rng.integers(0, n_tok - x + 1)) for x in lead]
    vpacked = v.clone()
    for s in range(len(lk)):
        assert lead[s] <= lk[s]
        v[ck[s]:ck[s] + lead[s]] = vtok[rows[s]:rows[s] + lead[s]]      # the values the kernel must use
        vpacked[ck[s]:ck[s] + lead[s]] = POISON
    t = lambda x: torch.tensor(x, dtype=torch.int32, device=DEV)
    dev = dict(q=q.to(DEV), k=k.to(DEV), v=vpacked.to(DEV), cu_q=t(cq), cu_k=t(ck), max_q=max(lq), max_k=max(lk),
               v_tok=vtok.to(DEV), v_lead=t(lead), v_row=t(rows))
    return q, k, v, cq, ck, dev


def _run(dev, lse=False, vfull=None):
    a = dict(dev)
    q, k, v, cu_q, cu_k, mq, mk = (a.pop(x) for x in ('q', 'k', 'v', 'cu_q', 'cu_k', 'max_q', 'max_k'))
    if vfull is not None:      # every value packed: no in-place rows
        v, a = vfull, {}
    if not lse:
        return scene.varlen(q, k, v, cu_q, cu_k, mq, mk, **a)
    out = torch.empty_like(q)
    l = torch.empty(q.shape[1], q.shape[0], dtype=torch.float32, device=DEV)
    scene.varlen(q, k, v, cu_q, cu_k, mq, mk, out=out, lse=l, **a)
    return out, l


# lead blocks: none, one, the ring fill's range (2..6 for 8 slots), the key loop's (7 on), every whole block
@pytest.mark.parametrize('D', [128, 64])
@pytest.mark.parametrize('lq,lk,lead_blocks,H', [
    ([300, 40, 257, 5], [40, 700, 1000, 300], [0, 1, 6, 9], 3),
    ([129, 64, 500], [230, 250, 2049], [7, 2, 64], 2),
    ([33, 1, 700, 90], [64, 32, 257, 5000], [2, 1, 8, 156], 4),
    ([640, 0, 77], [3000, 100, 32], [93, 3, 1], 8),
])
def test_varlen_values_in_place(lq, lk, lead_blocks, H, D):
    """O and lse against the fp32 oracle on the values the in-place rows name, and bit-identical to the same call
    with every value packed (the kernels read the same value bits either way)"""
    print(f'values in place lq={lq} lk={lk} lead blocks={lead_blocks} H={H} D={D}', flush=True)
    q, k, v, cq, ck, dev = _in_place_case(lq, lk, lead_blocks, H, D, 71)
    ref = OA.packed_attention(q, k, v, cq, ck)
    o = _run(dev)
    assert_close(o.cpu(), ref, what='values in place')
    assert torch.equal(o, _run(dev, vfull=v.to(DEV)))
    o2, lse = _run(dev, lse=True)
    assert_close(o2.cpu(), ref, what='values in place, lse call')
    assert (lse.cpu() - _lse_ref(q, k, cq, ck, D)).abs().max() < 2e-3


@pytest.mark.parametrize('lq,lk,lead_blocks,H', [([1000], [20000], [600], 4), ([300, 7], [5000, 3000], [150, 40], 3),
                                                 ([256, 256], [4000, 4000], [3, 125], 2)])
def test_varlen_values_in_place_key_split(lq, lk, lead_blocks, H):
    """few work items over long key ranges, split into key parts: each part's in-place blocks are those of its key
    range (none, some, or all of its blocks)"""
    D = 128
    print(f'values in place, key split lq={lq} lk={lk} lead blocks={lead_blocks} H={H}', flush=True)
    q, k, v, cq, ck, dev = _in_place_case(lq, lk, lead_blocks, H, D, 91)
    ref = OA.packed_attention(q, k, v, cq, ck)
    ws = torch.zeros(int(scene.L.lib().or_varlen_workspace_size(len(lq), sum(lq), H, D)), dtype=torch.uint8,
                     device=DEV)
    a = dict(dev)
    qq, kk, vv, cu_q, cu_k, mq, mk = (a.pop(x) for x in ('q', 'k', 'v', 'cu_q', 'cu_k', 'max_q', 'max_k'))
    o = scene.varlen(qq, kk, vv, cu_q, cu_k, mq, mk, workspace=ws, **a)
    assert int(ws.view(torch.int32)[3]) > 0          # items were split
    assert_close(o.cpu(), ref, what='values in place, key split')
    o2, lse = _run(dev, lse=True)
    assert_close(o2.cpu(), ref, what='values in place, key split, lse call')
    assert (lse.cpu() - _lse_ref(q, k, cq, ck, D)).abs().max() < 2e-3


def test_varlen_values_in_place_rows_past_the_token_rows():
    """in-place blocks that would reach past the token-order rows are taken from the packed rows instead (here the
    packed rows hold the right values there), so no read leaves v_tok"""
    H, D = 2, 128
    lq, lk = [100], [640]
    q, k, v = rand_bf16((100, H, D), 5), rand_bf16((640, H, D), 6), rand_bf16((640, H, D), 7)
    vtok = v[:300].clone()                      # 300 token rows: 9 whole blocks fit from row 0
    t = lambda x: torch.tensor(x, dtype=torch.int32, device=DEV)
    o = scene.varlen(q.to(DEV), k.to(DEV), v.to(DEV), t([0, 100]), t([0, 640]), 100, 640, v_tok=vtok.to(DEV),
                     v_lead=t([640]), v_row=t([0]))
    assert_close(o.cpu(), OA.packed_attention(q, k, v, [0, 100], [0, 640]), what='in-place blocks cut at v_tok')


def _layer(name, adjacent, in_place_text=True, q_range=None):
    case = layout_case(name)
    H, D, T = case['H'], case['D'], case['T']
    S = sum(case['lengths']) * T
    g = [rand_bf16((S, H, D), i).to(DEV) for i in range(3)] + \
        [rand_bf16((case['Le'], H, D), 3 + i).to(DEV) for i in range(3)]
    cos, sin = (x.to(DEV) for x in OA.rope_table_3d(*case['table'], D))
    lay = SceneLayout(case['lengths'], halo=case['halo'], sides=case['sides'], extra=case['extra'])
    plan = scene.ScopePlan(lay, T, case['counts'], case['Le'], case['scene_rope'], None, adjacent, True, DEV,
                           text_keys_in_place=in_place_text, q_range=q_range)
    return case, plan, g, cos, sin


@pytest.mark.parametrize('name', ['cpu_plumbing', 'hunyuan480p', 'uneven_K12', 'wan704'])
@pytest.mark.parametrize('adjacent', [False, True])
def test_pack_layer_bit_exact(name, adjacent):
    """one or_pack_layer launch writes the keys or_pack_gather writes, the value rows whose v_src is not -1 as
    or_pack_gather writes them (and no other value row), and the queries or_rotate_rows writes, bit for bit"""
    print(f'pack layer {name} adjacent={adjacent}', flush=True)
    case, plan, (q, k, v, eq, ek, ev), cos, sin = _layer(name, adjacent)
    H, D = q.shape[1], q.shape[2]
    kref, vref = scene.pack_rows(plan, k, ek, 'k', b_video=v, b_text=ev, cos=cos, sin=sin, mode='raw')
    qref = scene.rotate_queries(plan, q, cos, sin)
    kbuf = torch.empty(plan.sum_k, H, D, dtype=torch.bfloat16, device=DEV)
    vbuf = torch.full_like(kbuf, 7.0)
    qbuf = torch.empty_like(q)
    scene.pack_layer(plan, k, ek, v, ev, cos, sin, 'raw', kbuf, vbuf, q=q, qbuf=qbuf)
    bits = lambda x: x.view(torch.int16)
    assert torch.equal(bits(kbuf), bits(kref))
    assert torch.equal(bits(qbuf), bits(qref))
    copied = plan.v_src >= 0
    assert torch.equal(bits(vbuf[copied]), bits(vref[copied]))
    assert bool((vbuf[~copied] == 7.0).all())
    n_in_place = int((~copied).sum())
    # the video segments own the packed rows: their leading runs and their value runs' whole key blocks
    runs = plan.v_runs.view(plan.n_seg, scene.L.VALUE_RUNS, 3).tolist()
    whole = sum(max((x0 + n) // 32 - -(-x0 // 32), 0) * 32 for seg in runs for x0, n, _ in seg if n > 0)
    assert whole > 0 and n_in_place == sum(int(x) for x in plan.v_lead.tolist()[0::2]) + whole
    # keys only (mode 'rotated' with moves, no query rotation): the same keys as or_pack_gather
    plan2 = scene.ScopePlan(plan.layout, case['T'], case['counts'], case['Le'], case['scene_rope'], None, adjacent,
                            True, DEV, moves=True, text_keys_in_place=True)
    kr2, vr2 = scene.pack_rows(plan2, k, ek, 'k', b_video=v, b_text=ev, cos=cos, sin=sin, mode='rotated')
    kb2, vb2, _ = scene.pack_layer(plan2, k, ek, v, ev, cos, sin, 'rotated', values_in_place=False)
    assert torch.equal(bits(kb2), bits(kr2)) and torch.equal(bits(vb2), bits(vr2))


@pytest.mark.parametrize('name,q_range', [('hunyuan480p', None), ('uneven_K12', None), ('cpu_plumbing', None),
                                          ('hunyuan480p', (8000, 30000))])
@pytest.mark.parametrize('adjacent', [False, True])
def test_layer_values_in_place_bit_identical(name, q_range, adjacent):
    """the fused layer with the own-frame values and the shared frames' values (value runs) read in place gives the
    same output bits as with every value packed (text keys in place and packed; one rank's share)"""
    for in_place_text in (True, False):
        print(f'layer values in place {name} adjacent={adjacent} text keys in place={in_place_text} '
              f'q_range={q_range}', flush=True)
        _, plan, g, cos, sin = _layer(name, adjacent, in_place_text, q_range)
        ov, ot = scene.scene_attention(plan, *g, cos, sin, mode='raw', fused=True, values_in_place=True)
        ov2, ot2 = scene.scene_attention(plan, *g, cos, sin, mode='raw', fused=True, values_in_place=False)
        assert torch.equal(ov, ov2) and torch.equal(ot, ot2)
        del ov, ot, ov2, ot2


def _kv_in_place_case(lq, lk, v_blocks, k_blocks, H, D, seed):
    """as _in_place_case, with the keys too: segment s reads the K rows of its first 32 * k_blocks[s] keys and the V
    rows of its first 32 * v_blocks[s] from token-order tensors that hold them at one common row (the packed rows
    under them hold POISON)"""
    rng = np.random.default_rng(seed)
    q = rand_bf16((sum(lq), H, D), seed)
    k = rand_bf16((sum(lk), H, D), seed + 1)
    v = rand_bf16((sum(lk), H, D), seed + 2)
    cq, ck = np.cumsum([0] + lq), np.cumsum([0] + lk)
    lead = [32 * max(a, b) for a, b in zip(v_blocks, k_blocks)]
    n_tok = sum(lead) + 300
    ktok, vtok = rand_bf16((n_tok, H, D), seed + 3), rand_bf16((n_tok, H, D), seed + 4)
    rows = [int(rng.integers(0, n_tok - x + 1)) for x in lead]
    kp, vp = k.clone(), v.clone()
    for s in range(len(lk)):
        kl, vl = 32 * k_blocks[s], 32 * v_blocks[s]
        assert max(kl, vl) <= lk[s]
        k[ck[s]:ck[s] + kl] = ktok[rows[s]:rows[s] + kl]
        v[ck[s]:ck[s] + vl] = vtok[rows[s]:rows[s] + vl]
        kp[ck[s]:ck[s] + kl] = POISON
        vp[ck[s]:ck[s] + vl] = POISON
    t = lambda x: torch.tensor(x, dtype=torch.int32, device=DEV)
    dev = dict(q=q.to(DEV), k=kp.to(DEV), v=vp.to(DEV), cu_q=t(cq), cu_k=t(ck), max_q=max(lq), max_k=max(lk),
               v_tok=vtok.to(DEV), v_lead=t([32 * b for b in v_blocks]), v_row=t(rows), k_tok=ktok.to(DEV),
               k_lead=t([32 * b for b in k_blocks]))
    return q, k, v, cq, ck, dev


# K lead blocks: none, the ring head (1, 2), the ring fill (3 .. 8), the key loop (9 on), every whole block; the V
# lead blocks independent of them
@pytest.mark.parametrize('D', [128, 64])
@pytest.mark.parametrize('lq,lk,v_blocks,k_blocks,H', [
    ([300, 40, 257, 5], [40, 700, 1000, 300], [0, 1, 6, 9], [1, 2, 3, 9], 8),
    ([129, 64, 500], [230, 250, 2049], [7, 0, 64], [7, 5, 8], 3),
    ([33, 1, 700, 90], [64, 32, 257, 5000], [2, 1, 0, 156], [0, 1, 8, 100], 2),
    ([640, 0, 77], [3000, 100, 32], [93, 3, 1], [93, 2, 0], 5),
])
def test_varlen_keys_and_values_in_place(lq, lk, v_blocks, k_blocks, H, D):
    """keys and values read in place with separate leads (each stream's base switching at its own block, in the ring
    head, the ring fill or the loop): O and lse against the fp32 oracle, and O bit-identical to the call with every
    key and value packed"""
    print(f'keys and values in place lq={lq} lk={lk} v blocks={v_blocks} k blocks={k_blocks} H={H} D={D}', flush=True)
    q, k, v, cq, ck, dev = _kv_in_place_case(lq, lk, v_blocks, k_blocks, H, D, 171)
    ref = OA.packed_attention(q, k, v, cq, ck)
    o = _run(dev)
    assert_close(o.cpu(), ref, what='keys and values in place')
    full = dict(q=dev['q'], k=k.to(DEV), v=v.to(DEV), cu_q=dev['cu_q'], cu_k=dev['cu_k'], max_q=dev['max_q'],
                max_k=dev['max_k'])
    assert torch.equal(o, _run(full))
    o2, lse = _run(dev, lse=True)
    assert_close(o2.cpu(), ref, what='keys and values in place, lse call')
    assert (lse.cpu() - _lse_ref(q, k, cq, ck, D)).abs().max() < 2e-3


@pytest.mark.parametrize('D', [128, 64])
def test_varlen_keys_in_place_without_values(D):
    """k_tok without v_tok: every value packed, the keys' base switching at each segment's own point (ring head, ring
    fill, loop, every whole block)"""
    lq, lk, k_blocks = [300, 64, 257, 33, 500], [40, 700, 1000, 300, 96], [1, 2, 8, 9, 3]
    print(f'keys in place only lq={lq} lk={lk} k blocks={k_blocks} D={D}', flush=True)
    q, k, v, cq, ck, dev = _kv_in_place_case(lq, lk, [0] * len(lk), k_blocks, 4, D, 181)
    for x in ('v_tok', 'v_lead'):
        dev.pop(x)
    dev['v'] = v.to(DEV)
    ref = OA.packed_attention(q, k, v, cq, ck)
    o = _run(dev)
    assert_close(o.cpu(), ref, what='keys in place, values packed')
    full = dict(q=dev['q'], k=k.to(DEV), v=dev['v'], cu_q=dev['cu_q'], cu_k=dev['cu_k'], max_q=dev['max_q'],
                max_k=dev['max_k'])
    assert torch.equal(o, _run(full))


@pytest.mark.parametrize('lq,lk,v_blocks,k_blocks,H', [([1000], [20000], [600], [602], 4),
                                                       ([300, 7], [5000, 3000], [150, 0], [140, 40], 3)])
def test_varlen_keys_in_place_key_split(lq, lk, v_blocks, k_blocks, H):
    """key parts of split items with keys and values in place: each part's in-place blocks of each stream"""
    D = 128
    print(f'keys in place, key split lq={lq} lk={lk} v={v_blocks} k={k_blocks} H={H}', flush=True)
    q, k, v, cq, ck, dev = _kv_in_place_case(lq, lk, v_blocks, k_blocks, H, D, 191)
    ref = OA.packed_attention(q, k, v, cq, ck)
    ws = torch.zeros(int(scene.L.lib().or_varlen_workspace_size(len(lq), sum(lq), H, D)), dtype=torch.uint8,
                     device=DEV)
    a = dict(dev)
    qq, kk, vv, cu_q, cu_k, mq, mk = (a.pop(x) for x in ('q', 'k', 'v', 'cu_q', 'cu_k', 'max_q', 'max_k'))
    o = scene.varlen(qq, kk, vv, cu_q, cu_k, mq, mk, workspace=ws, **a)
    assert int(ws.view(torch.int32)[3]) > 0
    assert_close(o.cpu(), ref, what='keys in place, key split')


def _blocks_in_place(x0, n, t, n_tok, lk, prev):
    """the whole key blocks [bs, be) of a value run (keys x0 .. x0 + n - 1 from token rows t ..) that the attention
    kernel reads in place: inside the segment's whole blocks and the token rows, past `prev` (the leading run's or
    the previous run's end), as or_varlen_args.v_runs states"""
    bs = max(-(-x0 // 32), prev)
    be = min((x0 + n) // 32, lk // 32, (n_tok - t + x0) // 32)
    return (bs, be) if be > bs else (prev, prev)


def _runs_case(lq, lk, lead_blocks, runs, H, seed, n_tok=None):
    """segments with lq queries and lk keys, of which the first 32 * lead_blocks[s] take their values from token rows
    v_row[s].. and the keys of each run (x0, n) of runs[s] from token rows t.. (t random, the run possibly reaching
    past the token rows); the packed rows under every block read in place hold POISON. Returns the oracle inputs
    (the values each key really has) and the device arguments."""
    D = 128
    rng = np.random.default_rng(seed)
    q = rand_bf16((sum(lq), H, D), seed)
    k = rand_bf16((sum(lk), H, D), seed + 1)
    v = rand_bf16((sum(lk), H, D), seed + 2)
    cq, ck = np.cumsum([0] + lq), np.cumsum([0] + lk)
    need = sum(32 * b for b in lead_blocks) + sum(n for rs in runs for _, n in rs)
    n_tok = n_tok or need + 200
    vtok = rand_bf16((n_tok, H, D), seed + 3)
    vp = v.clone()
    rows = []
    tab = np.zeros((len(lk), scene.L.VALUE_RUNS, 3), dtype=np.int32)
    for s in range(len(lk)):
        lead = 32 * lead_blocks[s]
        row = int(rng.integers(0, n_tok - lead + 1))
        rows.append(row)
        la = min(min(lead, lk[s]) // 32, (n_tok - row) // 32)
        v[ck[s]:ck[s] + 32 * la] = vtok[row:row + 32 * la]
        vp[ck[s]:ck[s] + 32 * la] = POISON
        prev = la
        for r, (x0, n) in enumerate(runs[s]):
            t = int(rng.integers(0, n_tok - n + 1)) if rng.random() < 0.8 else n_tok - n // 2   # some reach past
            tab[s, r] = (x0, n, t)
            bs, be = _blocks_in_place(x0, n, t, n_tok, lk[s], prev)
            if be > bs:
                a, b = 32 * bs, 32 * be
                v[ck[s] + a:ck[s] + b] = vtok[t + a - x0:t + b - x0]
                vp[ck[s] + a:ck[s] + b] = POISON
                prev = be
    t32 = lambda x: torch.tensor(np.asarray(x), dtype=torch.int32, device=DEV)
    dev = dict(q=q.to(DEV), k=k.to(DEV), v=vp.to(DEV), cu_q=t32(cq), cu_k=t32(ck), max_q=max(lq), max_k=max(lk),
               v_tok=vtok.to(DEV), v_lead=t32([32 * b for b in lead_blocks]), v_row=t32(rows),
               v_runs=t32(tab.reshape(-1)))
    return q, k, v, cq, ck, dev


# value runs past the leading one: runs whose first whole block falls in the ring fill or the loop, a run starting
# on the block where the previous one (or the lead) ends, runs with no whole block, runs reaching past the token
# rows or the segment, segments without a lead (their first event is a run's start), up to four runs per segment
RUN_CASES = [
    ([300, 40, 257], [3000, 1500, 700],
     [10, 2, 0], [[(330, 1590), (1920, 600)], [(64, 100), (170, 900), (1070, 33), (1110, 380)], [(5, 400)]]),
    ([129, 640], [5000, 4000], [20, 0], [[(700, 1590), (2290, 1590), (3880, 1000)], [(0, 1000), (1000, 1600)]]),
    ([77, 5, 300, 1], [200, 96, 4096, 64], [1, 0, 3, 0],
     [[(40, 150)], [(1, 31)], [(96, 992), (1088, 992), (2080, 992), (3072, 992)], [(0, 64)]]),
]


@pytest.mark.parametrize('lq,lk,lead_blocks,runs', RUN_CASES)
def test_varlen_value_runs(lq, lk, lead_blocks, runs):
    """values read in place from several runs per segment (the value stream moving at every run's start and end):
    O and lse against the fp32 oracle, O bit-identical to the call with every value packed"""
    H = 4
    print(f'value runs lq={lq} lk={lk} lead={lead_blocks} runs={runs}', flush=True)
    q, k, v, cq, ck, dev = _runs_case(lq, lk, lead_blocks, runs, H, 211)
    ref = OA.packed_attention(q, k, v, cq, ck)
    o = _run(dev)
    assert_close(o.cpu(), ref, what='value runs')
    assert torch.equal(o, _run(dev, vfull=v.to(DEV)))
    o2, lse = _run(dev, lse=True)
    assert_close(o2.cpu(), ref, what='value runs, lse call')
    assert (lse.cpu() - _lse_ref(q, k, cq, ck, 128)).abs().max() < 2e-3


@pytest.mark.parametrize('lq,lk,lead_blocks,runs,H', [
    ([1000], [20000], [100], [[(3300, 1590), (4890, 1590), (8000, 5000), (15000, 4999)]], 4),
    ([300, 7], [5000, 3000], [0, 20], [[(100, 2000), (2200, 2800)], [(700, 1590), (2290, 700)]], 3)])
def test_varlen_value_runs_key_split(lq, lk, lead_blocks, runs, H):
    """key parts of split items over value runs: parts that start inside a run, between runs and in the lead walk
    the segment's event list to their first block"""
    print(f'value runs, key split lq={lq} lk={lk} lead={lead_blocks} runs={runs} H={H}', flush=True)
    q, k, v, cq, ck, dev = _runs_case(lq, lk, lead_blocks, runs, H, 223)
    ref = OA.packed_attention(q, k, v, cq, ck)
    ws = torch.zeros(int(scene.L.lib().or_varlen_workspace_size(len(lq), sum(lq), H, 128)), dtype=torch.uint8,
                     device=DEV)
    a = dict(dev)
    qq, kk, vv, cu_q, cu_k, mq, mk = (a.pop(x) for x in ('q', 'k', 'v', 'cu_q', 'cu_k', 'max_q', 'max_k'))
    o = scene.varlen(qq, kk, vv, cu_q, cu_k, mq, mk, workspace=ws, **a)
    assert int(ws.view(torch.int32)[3]) > 0
    assert_close(o.cpu(), ref, what='value runs, key split')


def test_varlen_value_runs_need_head_dim_128():
    q = torch.zeros(64, 2, 64, dtype=torch.bfloat16, device=DEV)
    t32 = lambda x: torch.tensor(x, dtype=torch.int32, device=DEV)
    with pytest.raises(scene.L.HipPathError, match='head_dim 128'):
        scene.varlen(q, q, q, t32([0, 64]), t32([0, 64]), 64, 64, v_tok=q, v_lead=t32([0]), v_row=t32([0]),
                     v_runs=t32([0] * (3 * scene.L.VALUE_RUNS)))


def test_layer_value_runs_random_layouts():
    """random layouts (halo frames, extra frames, frames of T tokens not a multiple of 32, empty sentences, both
    shared-frame layouts, text keys in place or packed): the fused layer with its values read in place (each scope's
    leading run and its shared frames' value runs) gives the bits of the layer with every value packed"""
    rng = np.random.default_rng(29)
    H, D = 2, 128
    n_runs = 0
    for it in range(16):
        n = int(rng.integers(1, 6))
        lengths = rng.integers(1, 5, n).tolist()
        F = sum(lengths)
        extra = {j: sorted({int(x) for x in rng.integers(0, F, int(rng.integers(0, 6)))}) for j in range(n)
                 if rng.random() < 0.8}
        T = int(rng.integers(20, 140))
        counts = rng.integers(0, 40, n).tolist()
        Le = sum(counts) + int(rng.integers(0, 3))
        lay = SceneLayout(lengths, halo=int(rng.integers(0, 3)), sides=['adj', 'prev', 'next'][int(rng.integers(3))],
                          extra=extra)
        adjacent, tkip = bool(rng.integers(2)), bool(rng.integers(2))
        print(f'random layer {it}: lengths={lengths} T={T} halo={lay.halo} sides={lay.sides} extra={extra} '
              f'counts={counts} adjacent={adjacent} text keys in place={tkip}', flush=True)
        plan = scene.ScopePlan(lay, T, counts, Le, True, None, adjacent, True, DEV, text_keys_in_place=tkip)
        runs = plan.v_runs.view(plan.n_seg, scene.L.VALUE_RUNS, 3)
        n_runs += int((runs[:, :, 1] > 0).sum())
        g = [rand_bf16((F * T, H, D), 40 + 6 * it + i).to(DEV) for i in range(3)] + \
            [rand_bf16((Le, H, D), 43 + 6 * it + i).to(DEV) for i in range(3)]
        ang = torch.rand(plan.max_rope_row + 1, D // 2, generator=torch.Generator().manual_seed(it)) * 6.2832
        cos, sin = (f(ang).repeat_interleave(2, 1).contiguous().to(DEV) for f in (torch.cos, torch.sin))
        ov, ot = scene.scene_attention(plan, *g, cos, sin, mode='raw', fused=True, values_in_place=True)
        ov2, ot2 = scene.scene_attention(plan, *g, cos, sin, mode='raw', fused=True, values_in_place=False)
        assert torch.equal(ov, ov2) and torch.equal(ot, ot2), it
    assert n_runs > 20
