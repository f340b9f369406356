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
