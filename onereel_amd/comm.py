"""Frame-run and token-interval helpers of the one-GPU path (the single-GPU part of src/onereel/parallel/comm.py:
`merge` :69-77, `clip` :80-81, `frame_tokens` :84-85, `runs` :115-123).

On the device these runs are implicit: the layout kernel walks each scope's key frames and writes their token rows.
The host helpers serve callers of the reference module. The multi-GPU exchange (partitions, halo exchange, Ulysses
all-to-all) is not part of the one-GPU path.
"""
from __future__ import annotations

from itertools import groupby


def merge(iv) -> list:
    """the union of half-open intervals as sorted, disjoint intervals; intervals that touch are joined and empty
    ones dropped"""
    out = []
    for lo, hi in sorted((a, b) for a, b in iv if a < b):
        if out and lo <= out[-1][1]:
            out[-1] = (out[-1][0], max(out[-1][1], hi))
        else:
            out.append((lo, hi))
    return out


def clip(iv, a: int, b: int) -> list:
    """each interval intersected with [a, b); intervals outside it dropped"""
    return [(max(lo, a), min(hi, b)) for lo, hi in iv if hi > a and lo < b]


def runs(frames) -> list:
    """maximal stretches of frames that rise by one, in list order: [3, 4, 5, 1, 2] -> [(3, 6), (1, 3)]"""
    out = []
    for _, grp in groupby(enumerate(frames), key=lambda p: p[1] - p[0]):
        fs = [f for _, f in grp]
        out.append((fs[0], fs[-1] + 1))
    return out


def frame_tokens(frames, T: int) -> list:
    """the token rows of a frame list (frame-major, T tokens per frame) as intervals, one per run of frames"""
    return [(lo * T, hi * T) for lo, hi in runs(frames)]
