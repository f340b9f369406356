"""GPU parity of the attention kernels' work-item boundaries, on a persistent grid capped to a few work-groups
(ONEREEL_ATTN_MAX_BLOCKS, read by the library at every call) so that each work-group walks dozens to hundreds of
items in a row. Every output row and every lse against the fp32 oracle, at head_dim 128 (attn8_kernel) and 64
(attn4_kernel).

The transitions between two items of one work-group that these calls drive:
- claim ahead: while its XCD's queue holds more than 64 items, a work-group claims its next item before running the
  current one, and the current item's key loop loads the next item's queries into a128..a191 at its exit;
- the crossing of that threshold, after which it claims after each item (kLater), and the claims that then find
  their own queue empty and take items from the other XCDs' queues;
- items without keys (nb == 0: O = 0, lse = -inf), which run no key loop, so the next item loads its own queries;
- query tiles whose last wavefronts lie past the segment (dead wavefronts: a key loop of barriers and DMA only),
  followed by an item whose wavefronts are all live;
- items whose values (and keys) are partly read in place (each stream's base switching in the ring head, the ring
  fill or the loop), and items whose value streams move several times (value runs), next to items whose values and
  keys are all packed;
- key-split parts of the last items (capped grid, few items), several parts per work-group, merged afterwards.
"""
import numpy as np
import pytest
import torch

from helpers import assert_close, rand_bf16
from onereel_amd import _lib as L
from onereel_amd import scene
from oracle import attention as OA

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]
DEV = 'cuda'


def _lse_ref(q, k, cq, ck, D):
    out = torch.full((q.shape[1], q.shape[0]), -float('inf'))
    for s in range(len(cq) - 1):
        if cq[s + 1] == cq[s] or ck[s + 1] == ck[s]:
            continue
        qs, ks = q[cq[s]:cq[s + 1]].float(), k[ck[s]:ck[s + 1]].float()
        out[:, cq[s]:cq[s + 1]] = torch.logsumexp(torch.einsum('qhd,khd->hqk', qs, ks) * D ** -0.5, -1)
    return out


def _check(lq, lk, H, D, seed, lead_blocks=None, expect_split=False, keys_too=False):
    """one O + lse call against the oracle over every row; with lead_blocks, the first 32 * lead_blocks[s] values of
    segment s (and with keys_too its keys) are read from token-order tensors (the packed rows there hold a poison
    value)"""
    q = rand_bf16((sum(lq), H, D), seed)
    k = rand_bf16((sum(lk), H, D), seed + 1)
    v = rand_bf16((sum(lk), H, D), seed + 2)
    cq, ck = np.cumsum([0] + lq), np.cumsum([0] + lk)
    t = lambda x: torch.tensor(np.asarray(x), dtype=torch.int32, device=DEV)
    extra = {}
    vdev = v.to(DEV)
    if lead_blocks is not None:
        lead = [32 * b for b in lead_blocks]
        vtok = torch.cat([v[ck[s]:ck[s] + lead[s]] for s in range(len(lk))] + [rand_bf16((64, H, D), seed + 3)])
        rows = np.cumsum([0] + lead)[:-1]
        vp = v.clone()
        for s in range(len(lk)):
            vp[ck[s]:ck[s] + lead[s]] = 3.0e4
        vdev = vp.to(DEV)
        extra = dict(v_tok=vtok.to(DEV), v_lead=t(lead), v_row=t(rows))
        if keys_too:
            ktok = torch.cat([k[ck[s]:ck[s] + lead[s]] for s in range(len(lk))] + [rand_bf16((64, H, D), seed + 4)])
            kpk = k.clone()
            for s in range(len(lk)):
                kpk[ck[s]:ck[s] + lead[s]] = 3.0e4
            extra.update(k_tok=ktok.to(DEV), k_lead=t(lead))
    kdev = kpk.to(DEV) if lead_blocks is not None and keys_too else k.to(DEV)
    ws = torch.zeros(int(L.lib().or_varlen_workspace_size(len(lq), sum(lq), H, D)), dtype=torch.uint8, device=DEV)
    o = torch.empty(sum(lq), H, D, dtype=torch.bfloat16, device=DEV)
    lse = torch.empty(H, sum(lq), dtype=torch.float32, device=DEV)
    scene.varlen(q.to(DEV), kdev, vdev, t(cq), t(ck), max(lq), max(lk), out=o, lse=lse, workspace=ws, **extra)
    o2 = scene.varlen(q.to(DEV), kdev, vdev, t(cq), t(ck), max(lq), max(lk), **extra)   # O-only kernel path
    split = int(ws.view(torch.int32)[3])
    assert (split > 0) == expect_split, split
    ref = OA.packed_attention(q, k, v, cq, ck)
    assert_close(o.cpu(), ref, what='O (lse call)')
    assert_close(o2.cpu(), ref, what='O')
    lref = _lse_ref(q, k, cq, ck, D)
    fin = torch.isfinite(lref)
    assert torch.equal(torch.isfinite(lse.cpu()), fin)
    assert (lse.cpu()[fin] - lref[fin]).abs().max() < 2e-3


def _many_items(seed, n=40):
    rng = np.random.default_rng(seed)
    lq = rng.integers(1, 1500, n).tolist()       # partial last tiles: dead wavefronts
    lk = rng.integers(1, 400, n).tolist()
    for s in rng.choice(n, 6, replace=False):
        lk[s] = 0                                # items without keys
    for s in rng.choice(n, 3, replace=False):
        lq[s] = 0                                # segments without queries
    return lq, lk


@pytest.mark.parametrize('blocks', [1, 4])
@pytest.mark.parametrize('D', [128, 64])
def test_many_items_per_work_group(monkeypatch, blocks, D):
    """40 segments, 8 heads, about 130 query tiles per head: with 1 or 4 work-groups every queue's own items exceed
    the claim-ahead threshold at first and fall below it later, work-groups steal from the other queues, and items
    without keys or with dead wavefronts sit between live ones"""
    monkeypatch.setenv('ONEREEL_ATTN_MAX_BLOCKS', str(blocks))
    lq, lk = _many_items(11 + blocks)
    print(f'item boundaries: {blocks} work-groups, D={D}, lq={lq}, lk={lk}', flush=True)
    _check(lq, lk, 8, D, 200 + blocks, expect_split=False)


@pytest.mark.parametrize('keys_too', [False, True])
@pytest.mark.parametrize('D', [128, 64])
def test_many_items_with_values_in_place(monkeypatch, D, keys_too):
    """the same walk with every segment's first whole key blocks' values (and keys) read in place (0 to all of them),
    so that items whose streams switch in the ring head, the ring fill, the loop, or not at all follow each other on
    one work-group"""
    monkeypatch.setenv('ONEREEL_ATTN_MAX_BLOCKS', '4')
    lq, lk = _many_items(21)
    rng = np.random.default_rng(5)
    lead = [int(rng.integers(0, x // 32 + 1)) for x in lk]
    print(f'item boundaries, in place (keys too: {keys_too}): D={D}, lq={lq}, lk={lk}, lead blocks={lead}', flush=True)
    _check(lq, lk, 8, D, 300, lead_blocks=lead, keys_too=keys_too)


@pytest.mark.parametrize('lq,lk,H,lead', [([300, 40], [5000, 3000], 2, None), ([700], [9000], 3, None),
                                          ([300, 40], [5000, 3000], 2, [100, 30])])
def test_key_split_parts_on_few_work_groups(monkeypatch, lq, lk, H, lead):
    """few items on a grid of 4 work-groups: the last items are cut into key parts, several parts per work-group, each
    storing fp32 partials merged by lse afterwards (with values in place: parts before, across and after the switch)"""
    monkeypatch.setenv('ONEREEL_ATTN_MAX_BLOCKS', '4')
    print(f'item boundaries, key split on 4 work-groups: lq={lq} lk={lk} H={H} lead={lead}', flush=True)
    _check(lq, lk, H, 128, 400, lead_blocks=lead, expect_split=True)


def test_many_items_with_value_runs(monkeypatch):
    """the walk of test_many_items_per_work_group with every segment's values read in place from a leading run and
    up to two further runs (value events in the ring fill, in the loop, at a key-split part's start), on 4
    work-groups: items whose value streams move several times follow items whose streams do not move"""
    monkeypatch.setenv('ONEREEL_ATTN_MAX_BLOCKS', '4')
    lq, lk = _many_items(31)
    rng = np.random.default_rng(9)
    H, D = 8, 128
    q = rand_bf16((sum(lq), H, D), 500)
    k = rand_bf16((sum(lk), H, D), 501)
    v = rand_bf16((sum(lk), H, D), 502)
    cq, ck = np.cumsum([0] + lq), np.cumsum([0] + lk)
    n_tok = 4 * sum(lk) + 64
    vtok = rand_bf16((n_tok, H, D), 503)
    vp = v.clone()
    lead, rows, tab = [], [], np.zeros((len(lk), L.VALUE_RUNS, 3), dtype=np.int32)
    for s, n in enumerate(lk):
        la = int(rng.integers(0, n // 32 + 1))
        row = int(rng.integers(0, n_tok - 32 * la + 1))
        lead.append(32 * la)
        rows.append(row)
        v[ck[s]:ck[s] + 32 * la] = vtok[row:row + 32 * la]
        vp[ck[s]:ck[s] + 32 * la] = 3.0e4
        x, prev = 32 * la + int(rng.integers(0, 40)), la
        for r in range(int(rng.integers(0, 3))):
            cnt = int(rng.integers(1, 200))
            if x >= n:
                break
            t = int(rng.integers(0, n_tok - cnt + 1))
            tab[s, r] = (x, cnt, t)
            bs, be = max(-(-x // 32), prev), min((x + cnt) // 32, n // 32)
            if be > bs:
                v[ck[s] + 32 * bs:ck[s] + 32 * be] = vtok[t + 32 * bs - x:t + 32 * be - x]
                vp[ck[s] + 32 * bs:ck[s] + 32 * be] = 3.0e4
                prev = be
            x += cnt + int(rng.integers(0, 40))
    print(f'item boundaries, value runs: lq={lq}, lk={lk}, lead={lead}, runs={tab.tolist()}', flush=True)
    t32 = lambda x: torch.tensor(np.asarray(x), dtype=torch.int32, device=DEV)
    o = scene.varlen(q.to(DEV), k.to(DEV), vp.to(DEV), t32(cq), t32(ck), max(lq), max(lk), v_tok=vtok.to(DEV),
                     v_lead=t32(lead), v_row=t32(rows), v_runs=t32(tab.reshape(-1)))
    assert_close(o.cpu(), OA.packed_attention(q, k, v, cq, ck), what='O, value runs')
