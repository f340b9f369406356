"""Oracle: bounded cross-scene memory with per-head representatives, on the CPU.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`). Restates src/onereel/memory.py:

- `boundary_rows`     candidate_frames / candidates (memory.py:30-45): the first and last frame of every scene (each
                      frame once), all their tokens, with their scene
- `select`            BoundaryMemory.select (memory.py:58-93): k-means over the L2-normalised candidate keys of each
                      head, from M evenly spaced candidates (round(linspace(0, B-1, M)), at most 50 passes) or, for a
                      warm call, from the stored centroids (at most 2 passes); squared Euclidean distance, an empty
                      cluster keeps its centroid, stop when the centroids are unchanged; per non-empty cluster the
                      member nearest its centroid, then the lowest index
- `masked_reference`  what MemoryAttention (memory.py:140-174) computes, per head and scene: softmax over the scene's
                      own video keys, its sentence and the other scenes' representatives of that head (video queries),
                      or over the scene's video keys and its sentence (sentence queries), in float32 — the per-head
                      reference of the reference's tests/test_onereel_memory.py:21-37

Pinned in tests/test_oracle.py by the reference's own memory tests (tests/test_onereel_memory.py:63-94: every
candidate kept when the budget covers them; each representative is the nearest member of its cluster) and by
construction (well-separated groups of keys give one representative per group).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def boundary_rows(ranges, T):
    """(rows, scene) of the boundary frames' tokens"""
    rows, scene = [], []
    for j, (lo, hi) in enumerate(ranges):
        for f in dict.fromkeys((lo, hi - 1)):
            rows += list(range(f * T, (f + 1) * T))
            scene += [j] * T
    return torch.tensor(rows), torch.tensor(scene)


def select(kc, M, iters=50, centroids=False, start=None):
    """kc [B, H, D] -> (rep [H, M] candidate positions, valid [H, M]) (and the final centroids [H, M, D]). start:
    the centroids a warm call begins from (memory.py:67-72, then ITERS_UPDATE passes); None: the cold start from M
    evenly spaced candidates"""
    x = F.normalize(kc.float().transpose(0, 1), dim=-1)
    H, B, D = x.shape
    M = min(M, B)
    c = x[:, torch.linspace(0, B - 1, M).round().long()].clone() if start is None else start.float().clone()
    for it in range(iters + 1):
        d = ((x[:, :, None, :] - c[:, None, :, :]) ** 2).sum(-1)          # [H, B, M], explicit differences
        z = d.argmin(-1)
        if it == iters:
            break
        new = c.clone()
        for h in range(H):
            for i in range(M):
                m = z[h] == i
                if m.any():
                    new[h, i] = x[h, m].mean(0)
        if torch.equal(new, c):
            break
        c = new
    rep = torch.zeros(H, M, dtype=torch.long)
    valid = torch.zeros(H, M, dtype=torch.bool)
    for h in range(H):
        dist = d[h, torch.arange(B), z[h]]
        r = 0
        for i in range(M):
            m = (z[h] == i).nonzero().flatten()
            if len(m):
                best = m[torch.argsort(dist[m], stable=True)[0]]   # nearest, then lowest index (m ascending)
                rep[h, r], valid[h, r] = best, True
                r += 1
    return (rep, valid, c) if centroids else (rep, valid)


def masked_reference(q, k, v, eq, ek, ev, ranges, T, rep_row, rep_scene, valid, text_ranges, video_rows=None,
                     text_rows=None):
    """per head and scene softmax in float32 over the scope's keys -> (video out [S, H, D], text out [Le, H, D]).
    video_rows / text_rows (optional): only these query rows (of q / of eq) are computed, the others stay zero."""
    S, H, D = q.shape
    ov, ot = torch.zeros(S, H, D), torch.zeros(ek.shape[0], H, D)
    kk, vv = torch.cat([k, ek]).float(), torch.cat([v, ev]).float()
    pick = lambda rows, a, b: torch.arange(a, b) if rows is None else torch.as_tensor(
        [r for r in rows if a <= r < b], dtype=torch.long)
    for h in range(H):
        for j, (lo, hi) in enumerate(ranges):
            t0, t1 = text_ranges[j]
            local = list(range(lo * T, hi * T)) + [S + t for t in range(t0, t1)]
            far = [int(r) for r, s, ok in zip(rep_row[h], rep_scene[h], valid[h]) if ok and int(s) != j]
            keys = torch.tensor(local + far)
            qr = pick(video_rows, lo * T, hi * T)
            p = torch.softmax(q[qr, h].float() @ kk[keys, h].T * D ** -0.5, -1)
            ov[qr, h] = p @ vv[keys, h]
            keys = torch.tensor(local)
            tr = pick(text_rows, t0, t1)
            p = torch.softmax(eq[tr, h].float() @ kk[keys, h].T * D ** -0.5, -1)
            ot[tr, h] = p @ vv[keys, h]
    return ov, ot
