"""Oracle: frame-memory pooling and representative selection, on the CPU.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`). Restates:

- `pool`        FrameMemory.collect (src/onereel/frame_memory.py:76-85): per-frame sums and counts of the rows with
                frame >= 0 (index_add_), in float64
- `features`    FrameMemory.finish (:87-101) on one GPU: L2-normalised per-frame means (counts clamped at 1)
- `candidates`  FrameMemory.candidate_frames (:107-112): every frame, or the first and last frame of every scene,
                minus the sink
- `select`      FrameMemory.select (:114-132): farthest-point initialisation from candidate 0 (largest 1 - dot to the
                nearest chosen centre, first on ties), k-means with the dot product (first centre on ties, a centre
                without members kept, stop when the centres are unchanged), then per non-empty cluster the member
                most similar to its centre (first on ties); ascending

Pinned in tests/test_oracle.py by the reference's own frame-memory tests (tests/test_onereel_frame_memory.py:19-60:
one medoid per group of near-identical frames, determinism, boundary candidates, the sink) and by construction: for
well-separated groups the clusters are the groups and each medoid is the member closest to its group's normalised
mean, computed there independently.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def pool(frame, hs, n_frames):
    """frame [N] (-1: not video), hs [N, C] -> (sums [n_frames, C], counts [n_frames]) float64"""
    frame = torch.as_tensor(frame)
    keep = frame >= 0
    sums = torch.zeros(n_frames, hs.shape[-1], dtype=torch.float64)
    counts = torch.zeros(n_frames, dtype=torch.float64)
    sums.index_add_(0, frame[keep], hs[keep].double())
    counts.index_add_(0, frame[keep], torch.ones(int(keep.sum()), dtype=torch.float64))
    return sums, counts


def features(sums, counts):
    return F.normalize(sums / counts.clamp_min(1)[..., None], dim=-1)


def candidates(ranges, n_frames, mode='all', sink=()):
    cand = range(n_frames) if mode == 'all' else sorted({f for lo, hi in ranges for f in (lo, hi - 1)})
    return [f for f in cand if f not in sink]


def select(feats, cand, k, iters=20):
    """feats [F, C] (rows normalised), cand: candidate frames, k clusters -> ascending representative frames"""
    cand_t = torch.tensor(cand)
    x = feats[cand_t]
    centre = [0]
    for _ in range(k - 1):
        d = (1 - x @ x[centre].T).min(1).values
        centre.append(int(d.argmax()))
    c = x[centre].clone()
    for _ in range(iters):
        z = (x @ c.T).argmax(1)
        new = torch.stack([F.normalize(x[z == i].mean(0), dim=0) if (z == i).any() else c[i] for i in range(k)])
        if torch.equal(new, c):
            break
        c = new
    z = (x @ c.T).argmax(1)
    reps = []
    for i in range(k):
        m = (z == i).nonzero().flatten()
        if len(m):
            reps.append(int(cand_t[m[(x[m] @ c[i]).argmax()]]))
    return sorted(reps)
