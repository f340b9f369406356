"""GPU parity of the head-major bounded memory (onereel_amd.memory) with the oracle: packed single-head attention on
the pack / varlen / scatter kernels against a per-head masked float32 reference, and the per-head representative
choice (the reference's tests/test_onereel_memory.py)."""
import pytest
import torch

from onereel_amd.layout import SceneLayout
from onereel_amd.memory import BoundaryMemory, MemoryAttention, candidates, frame_plan
from oracle import memory as OM

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]
DEV = 'cuda'


@pytest.mark.parametrize('lengths,M,D', [([3, 5, 2, 4], 8, 64), ([2, 2, 2], 1000, 64), ([6, 1, 3], 5, 128)])
def test_memory_attention_matches_masked_reference(lengths, M, D):
    print(f'memory attention lengths={lengths} M={M} D={D}', flush=True)
    g = torch.Generator().manual_seed(0)
    T, H = 16, 4
    lay = SceneLayout(lengths, halo=0)
    S = lay.n_frames * T
    counts = [5, 7, 3, 6][:lay.n_scenes]
    tr, c = [], 0
    for n in counts:
        tr.append((c, c + n))
        c += n
    q, k, v = (torch.randn(S, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
    eq, ek, ev = (torch.randn(c, H, D, generator=g).to(torch.bfloat16) for _ in range(3))
    plan = frame_plan(lay, T, torch.arange(S), S, [(j, lo * T, hi * T) for j, (lo, hi) in enumerate(lay.ranges)], tr,
                      set(range(lay.n_scenes)), S, DEV)
    mem = MemoryAttention(BoundaryMemory(M))
    out = mem(('l0', True), torch.cat([q, eq]).to(DEV), torch.cat([k, ek]).to(DEV), torch.cat([v, ev]).to(DEV), plan)
    ov, ot = out[:S].cpu(), out[S:].cpu()
    # the representatives a fresh memory picks (deterministic) feed the reference
    rows, owner = candidates(lay, T, DEV)
    rep, valid = BoundaryMemory(M).select(('l0', True), k.to(DEV)[rows])
    rv, rt = OM.masked_reference(q, k, v, eq, ek, ev, lay.ranges, T, rows[rep].cpu(), owner[rep].cpu(), valid.cpu(),
                                 tr)
    rel = lambda a, b: ((a.float() - b).norm() / b.norm()).item()
    assert rel(ov, rv) < 2e-2 and rel(ot, rt) < 2e-2
    assert (ov.float() - rv).abs().max() < 2e-2 and (ot.float() - rt).abs().max() < 2e-2


def test_select_keeps_every_candidate_when_the_budget_covers_them():
    lay = SceneLayout([3, 4, 2], halo=0)
    T, H, D = 8, 2, 32
    rows, _ = candidates(lay, T, DEV)
    k = torch.randn(lay.n_frames * T, H, D, generator=torch.Generator().manual_seed(1)).to(DEV)
    rep, valid = BoundaryMemory(len(rows)).select('x', k[rows])
    for h in range(H):
        assert sorted(rep[h][valid[h]].tolist()) == list(range(len(rows)))


def test_select_nearest_member_and_oracle_on_separated_groups():
    g = torch.Generator().manual_seed(2)
    x = torch.randn(300, 3, 16, generator=g)
    mem = BoundaryMemory(12)
    rep, valid = mem.select('y', x.to(DEV))
    c = mem.centroids['y'].cpu()
    xn = torch.nn.functional.normalize(x.float().transpose(0, 1), dim=-1)
    for h in range(3):
        z = torch.cdist(xn[h], c[h]).argmin(-1)
        for r in rep[h][valid[h]].cpu().tolist():
            members = (z == z[r]).nonzero().flatten()
            d = (xn[h, members] - c[h, z[r]]).pow(2).sum(-1)
            assert d.min() >= (xn[h, r] - c[h, z[r]]).pow(2).sum() - 1e-5
    base = torch.randn(4, 2, 16, generator=g)
    xs = torch.cat([base[i].expand(10, -1, -1) for i in range(4)]) + 0.01 * torch.randn(40, 2, 16, generator=g)
    got, gv = BoundaryMemory(4).select('z', xs.to(DEV))
    ref, rv = OM.select(xs, 4)
    for h in range(2):
        assert sorted(got[h][gv[h]].cpu().tolist()) == sorted(ref[h][rv[h]].tolist())
