"""Token-interval helpers of the single-GPU path (src/onereel/parallel/comm.py:69-85,115-123).

The multi-GPU exchange of the reference (HaloExchange, partitions, Ulysses all-to-all) is not implemented: the path
runs on one GPU.
"""
from __future__ import annotations


def merge(iv) -> list:
    """union of half-open intervals, sorted and merged (comm.py:69-77)"""
    out = []
    for lo, hi in sorted(x for x in iv if x[0] < x[1]):
        if out and lo <= out[-1][1]:
            out[-1][1] = max(out[-1][1], hi)
        else:
            out.append([lo, hi])
    return [tuple(x) for x in out]


def clip(iv, a: int, b: int) -> list:
    """comm.py:80-81"""
    return [(max(lo, a), min(hi, b)) for lo, hi in iv if lo < b and hi > a]


def runs(frames) -> list:
    """frame list (in order) -> contiguous runs (comm.py:115-123)"""
    out = []
    for f in frames:
        if out and out[-1][1] == f:
            out[-1][1] = f + 1
        else:
            out.append([f, f + 1])
    return [tuple(r) for r in out]


def frame_tokens(frames, T: int) -> list:
    """frame list -> contiguous token intervals [lo*T, hi*T), order kept (comm.py:84-85)"""
    return [(lo * T, hi * T) for lo, hi in runs(frames)]
