"""Scene layout over the latent frames of one video: the drop-in `SceneLayout` (src/onereel/layout.py:10-78).

Host-side API object. The per-token index arrays of a layout are never built here: `onereel_amd.scene` hands the
layout to the device layout kernel (`or_layout_build`), which derives the same frame lists on the GPU.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch


@dataclass
class SceneLayout:
    """lengths: latent frames per scene, in order. A scene also reads `halo` frames of the neighbouring scenes nearest
    to it: both neighbours ('adj'), only the previous ('prev') or only the next ('next'), and the frames in extra[j]
    (frame memory: representative frames of other scenes, replaced every denoising step). layout.py:10-22"""
    lengths: list
    halo: int = 2
    sides: str = 'adj'
    extra: dict = field(default_factory=dict)

    def __post_init__(self):
        assert self.sides in ('adj', 'prev', 'next'), self.sides
        assert all(n > 0 for n in self.lengths), self.lengths

    @classmethod
    def even(cls, n_frames: int, n_scenes: int, **kw) -> 'SceneLayout':
        """scene of frame f = f * n_scenes // n_frames (layout.py:25-28)"""
        sc = [f * n_scenes // n_frames for f in range(n_frames)]
        return cls([sc.count(j) for j in range(n_scenes)], **kw)

    @property
    def n_frames(self) -> int:
        return sum(self.lengths)

    @property
    def n_scenes(self) -> int:
        return len(self.lengths)

    @property
    def is_even(self) -> bool:
        return list(self.lengths) == SceneLayout.even(self.n_frames, self.n_scenes).lengths

    @property
    def ranges(self) -> list:
        out, s = [], 0
        for n in self.lengths:
            out.append((s, s + n))
            s += n
        return out

    @property
    def frames(self) -> list:
        return [list(range(lo, hi)) for lo, hi in self.ranges]

    def scene_of_frame(self) -> torch.Tensor:
        return torch.repeat_interleave(torch.arange(self.n_scenes), torch.tensor(self.lengths))

    def halo_frames(self, j: int) -> list:
        """frames of other scenes that scene j reads: the previous neighbour's last frames, then the next one's first"""
        fr, k, out = self.frames, self.halo, []
        if k == 0:
            return out
        if j > 0 and self.sides in ('adj', 'prev'):
            out += fr[j - 1][-k:]
        if j + 1 < self.n_scenes and self.sides in ('adj', 'next'):
            out += fr[j + 1][:k]
        return out

    def shared_frames(self, j: int) -> list:
        """frames of other scenes that scene j reads: its halo frames, then its extra frames in order"""
        lo, hi = self.ranges[j]
        out = self.halo_frames(j)
        return out + [f for f in sorted(self.extra.get(j, ())) if not lo <= f < hi and f not in out]

    def key_frames(self, j: int) -> list:
        """scene j's own frames, then its shared frames (the key order of the packed varlen layout)"""
        return self.frames[j] + self.shared_frames(j)

    def key_range(self, j: int) -> tuple:
        """scene j's keys as one contiguous frame range (scene plus halo are adjacent)"""
        kf = self.key_frames(j)
        return min(kf), max(kf) + 1
