"""Shared test inputs: the benchmark workload layouts (CPU plumbing, HunyuanVideo-1.5 480p, Wan2.2 704x1280, uneven
sweep) and seeded bf16 tensors (identical bits on CPU and GPU)."""
from __future__ import annotations

import numpy as np
import torch

from oracle import layout as OL


def layout_case(name: str):
    """-> dict(lengths, halo, sides, extra, T, counts, Le, H, D, scene_rope, rope_lengths, table (F, Hh, Ww))"""
    if name == 'cpu_plumbing':  # CPU plumbing: 2 scenes x 3 frames x 64 tokens + 16 text, 1 rep per scene
        return dict(lengths=[3, 3], halo=0, sides='adj', extra={0: [5], 1: [0]}, T=64, counts=[16, 16], Le=32, H=2,
                    D=64, scene_rope=True, rope_lengths=None, table=(6, 8, 8))
    if name == 'hunyuan480p':  # HunyuanVideo-1.5 480p: 4 x 8 frames x 1590 (30 x 53) + 128 text, memory 4
        return dict(lengths=[8] * 4, halo=0, sides='adj', extra={0: [10, 21, 31], 1: [0, 21, 31], 2: [0, 10, 31],
                                                                  3: [0, 10, 21]},
                    T=1590, counts=[128] * 4, Le=512, H=16, D=128, scene_rope=True, rope_lengths=None,
                    table=(32, 30, 53))
    if name == 'wan704':  # Wan2.2 704x1280 joint scopes: 3 x 11 x 880 (22 x 40) + 128 text, sides=next
        return dict(lengths=[11] * 3, halo=2, sides='next', extra={}, T=880, counts=[128] * 3, Le=384, H=24, D=128,
                    scene_rope=False, rope_lengths=None, table=(33, 22, 40))
    if name.startswith('uneven_K'):  # uneven sweep, K scenes (seed K)
        K = int(name.split('K')[1])
        rng = np.random.default_rng(K)
        lengths = rng.integers(2, 17, K).tolist()
        text = rng.integers(64, 257, K).tolist()
        F = sum(lengths)
        reps = sorted({int(x) for x in np.linspace(0, F - 1, 4).round()})
        lay = OL.SceneLayout(lengths, halo=0)
        fm = OL.FrameMemoryExtra(budget=4, fallback=(0, 'adj'))
        fm.reset(lay)
        fm.propose(reps)
        fm.begin_step(1)
        return dict(lengths=lengths, halo=0, sides='adj', extra=lay.extra, T=1590, counts=text, Le=sum(text), H=16,
                    D=128, scene_rope=True, rope_lengths=None, table=(F, 30, 53))
    raise KeyError(name)


def rand_bf16(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(torch.bfloat16)


def bits(x: torch.Tensor) -> torch.Tensor:
    return x.contiguous().view(torch.int16) if x.dtype == torch.bfloat16 else x


def attn_rows_reference(qp, kp, vp, cu_q, cu_k, rows, k_off=None, k_len=None):
    """fp32 softmax(q k^T / sqrt(D)) v for the packed query rows `rows` (CPU tensors), grouped per segment"""
    rows = torch.as_tensor(rows)
    cu_q = torch.as_tensor(cu_q)
    seg = torch.searchsorted(cu_q, rows, right=True) - 1
    D = qp.shape[-1]
    out = torch.empty(len(rows), qp.shape[1], D)
    for s in seg.unique().tolist():
        m = seg == s
        if k_off is None:
            a, b = int(cu_k[s]), int(cu_k[s + 1])
        else:
            a = int(k_off[s])
            b = a + int(k_len[s])
        q = qp[rows[m]].float().transpose(0, 1)
        k = kp[a:b].float().transpose(0, 1)
        v = vp[a:b].float().transpose(0, 1)
        p = torch.softmax(q @ k.transpose(1, 2) * D ** -0.5, -1)
        out[m] = (p @ v).transpose(0, 1)
    return out


def sample_rows(cu_q, per_seg, seed=0):
    """up to per_seg query rows of every segment (its first and last rows included)"""
    g = np.random.default_rng(seed)
    out = []
    for s in range(len(cu_q) - 1):
        a, b = int(cu_q[s]), int(cu_q[s + 1])
        if b == a:
            continue
        n = b - a
        pick = {a, b - 1} | set((a + g.choice(n, min(n, per_seg), replace=False)).tolist())
        out += sorted(pick)
    return np.array(out)


def assert_close(got, ref, max_abs=2e-2, mean_abs=2e-3, what=''):
    d = (got.float() - ref.float()).abs()
    assert torch.isfinite(got.float()).all(), f'{what}: non-finite output'
    assert d.max().item() <= max_abs, f'{what}: max-abs {d.max().item():.3e} > {max_abs}'
    assert d.mean().item() <= mean_abs, f'{what}: mean-abs {d.mean().item():.3e} > {mean_abs}'


def gather_src(video, text, src):
    """rows `src` of the virtual concatenation [video ; text] (text row t encoded as len(video) + t), without
    materialising the concatenation"""
    src = torch.as_tensor(np.asarray(src, dtype=np.int64))
    nv = video.shape[0]
    out = torch.empty((len(src),) + tuple(video.shape[1:]), dtype=video.dtype)
    vid = src < nv
    out[vid] = video[src[vid]]
    if bool((~vid).any()):
        out[~vid] = text[src[~vid] - nv]
    return out


def scope_rows_reference(sc, q, k, v, eq, ek, ev, rows, cos=None, sin=None, mode='raw'):
    """fp32 softmax(q k^T / sqrt(D)) v of the packed query rows `rows` of the oracle's scopes `sc`, each segment's
    queries and keys gathered (and rotated per `mode`, as the oracle's pack does: 'raw' RoPE at the layout's rotary
    rows, 'rotated' the _move_shared re-rotation of shared keys, 'none') from the token-order tensors for that
    segment alone. Returns [len(rows), H, D] in the order of `rows`."""
    from oracle import attention as OA
    rows = np.asarray(rows)
    cu_q, cu_k = np.asarray(sc.cu_q), np.asarray(sc.cu_k)
    seg = np.searchsorted(cu_q, rows, side='right') - 1
    D = q.shape[-1]
    out = torch.empty(len(rows), q.shape[1], D)
    for s in np.unique(seg):
        m = seg == s
        r = rows[m]
        a, b = int(cu_k[s]), int(cu_k[s + 1])
        qs = gather_src(q, eq, np.asarray(sc.q_src)[r])
        ks = gather_src(k, ek, np.asarray(sc.k_src)[a:b])
        vs = gather_src(v, ev, np.asarray(sc.k_src)[a:b])
        if mode == 'raw':
            qs = OA.rotate_rows(qs, np.asarray(sc.q_rope)[r], cos, sin)
            ks = OA.rotate_rows(ks, np.asarray(sc.k_rope)[a:b], cos, sin)
        elif mode == 'rotated':
            ks = OA.move_shared(ks, np.asarray(sc.k_move_a)[a:b], np.asarray(sc.k_move_b)[a:b], cos, sin)
        else:
            assert mode == 'none', mode
        qh, kh, vh = (x.float().transpose(0, 1) for x in (qs, ks, vs))
        p = torch.softmax(qh @ kh.transpose(1, 2) * D ** -0.5, -1)
        out[torch.as_tensor(m)] = (p @ vh).transpose(0, 1)
    return out


def packed_rows_reference(sc, k, ek, v, ev, sel, cos=None, sin=None, mode='raw', which='k', q=None, eq=None):
    """the oracle's packed rows `sel` (bf16, bit for bit what its pack writes) without packing the others: keys and
    values (which='k', rotated per `mode`), or queries (which='q', rotated when mode == 'raw')"""
    from oracle import attention as OA
    sel = np.asarray(sel)
    if which == 'q':
        qs = gather_src(q, eq, np.asarray(sc.q_src)[sel])
        return OA.rotate_rows(qs, np.asarray(sc.q_rope)[sel], cos, sin) if mode == 'raw' else qs
    src = np.asarray(sc.k_src)[sel]
    ks, vs = gather_src(k, ek, src), gather_src(v, ev, src)
    if mode == 'raw':
        ks = OA.rotate_rows(ks, np.asarray(sc.k_rope)[sel], cos, sin)
    elif mode == 'rotated':
        ks = OA.move_shared(ks, np.asarray(sc.k_move_a)[sel], np.asarray(sc.k_move_b)[sel], cos, sin)
    return ks, vs


def sample_packed(cu, n, seed=0):
    """n random packed rows plus the first and last row of every non-empty segment, sorted"""
    cu = np.asarray(cu)
    g = np.random.default_rng(seed)
    edges = [x for a, b in zip(cu[:-1], cu[1:]) if b > a for x in (a, b - 1)]
    return np.unique(np.concatenate([g.integers(0, int(cu[-1]), n), np.asarray(edges, dtype=np.int64)]))


class Attn(torch.nn.Module):
    """the attention-module attributes a diffusers HunyuanVideo-1.5 block hands its processor"""

    def __init__(self, C, H, gen):
        super().__init__()
        self.heads = H
        mk = lambda: torch.nn.Linear(C, C, dtype=torch.bfloat16)
        self.to_q, self.to_k, self.to_v = mk(), mk(), mk()
        self.add_q_proj, self.add_k_proj, self.add_v_proj = mk(), mk(), mk()
        self.norm_q = torch.nn.RMSNorm(C // H, eps=1e-6, dtype=torch.bfloat16)
        self.norm_k = torch.nn.RMSNorm(C // H, eps=1e-6, dtype=torch.bfloat16)
        self.norm_added_q = torch.nn.RMSNorm(C // H, eps=1e-6, dtype=torch.bfloat16)
        self.norm_added_k = None
        self.to_out = torch.nn.ModuleList([mk(), torch.nn.Dropout(0.0)])
        self.to_add_out = mk()
        with torch.no_grad():
            for p in self.parameters():
                p.copy_(torch.randn(p.shape, generator=gen) * 0.05)
