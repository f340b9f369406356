"""`SceneLayout`, the drop-in for src/onereel/layout.py:10-78: the same constructor, fields, methods and results.

The object answers frame-list questions on the host (which frames a scene owns, which frames of other scenes it also
reads, in which order). The per-token index arrays of a layer are never built here: `onereel_amd.scene` copies the
fields into an `or_layout_desc`, and the device layout kernel derives every scene's shared frames by the same rules
(csrc/common.h, `scene_shared_frames`). Frame lists are computed arithmetically from the scene boundaries.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from itertools import accumulate

import torch

SIDES = ('adj', 'prev', 'next')


@dataclass
class SceneLayout:
    """Latent frames 0 .. n_frames-1 cut into consecutive scenes.

    lengths: frame count of every scene, in order, each positive.
    halo:    frames of each neighbouring scene that a scene also reads (context across the cut).
    sides:   which neighbours give them: 'adj' the previous and the next scene, 'prev' or 'next' only that one.
    extra:   scene index -> further frames it reads, e.g. the frame memory's representatives (reassigned per step).
    """
    lengths: list
    halo: int = 2
    sides: str = 'adj'
    extra: dict = field(default_factory=dict)

    def __post_init__(self):
        if self.sides not in SIDES:
            raise AssertionError(f'sides must be one of {SIDES}, got {self.sides!r}')
        if not all(n > 0 for n in self.lengths):
            raise AssertionError(f'every scene needs at least one frame: {self.lengths}')

    @classmethod
    def even(cls, n_frames: int, n_scenes: int, **kw) -> 'SceneLayout':
        """n_scenes scenes over n_frames frames where frame f falls in scene floor(f * n_scenes / n_frames): scene j
        then starts at frame ceil(j * n_frames / n_scenes)"""
        starts = [-(-j * n_frames // n_scenes) for j in range(n_scenes + 1)]
        return cls([b - a for a, b in zip(starts, starts[1:])], **kw)

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
        """per scene (first frame, one past its last frame)"""
        return [(int(end - n), int(end)) for n, end in zip(self.lengths, accumulate(self.lengths))]

    @property
    def frames(self) -> list:
        return [list(range(a, b)) for a, b in self.ranges]

    def scene_of_frame(self) -> torch.Tensor:
        """scene index of every frame (int64 [n_frames])"""
        return torch.arange(self.n_scenes).repeat_interleave(torch.tensor(self.lengths))

    def halo_frames(self, j: int) -> list:
        """neighbour frames scene j reads: the last `halo` frames before its first frame (sides 'adj' / 'prev'), then
        the first `halo` frames after its last one (sides 'adj' / 'next'), each clipped to that neighbour's frames"""
        if self.halo <= 0:
            return []
        bounds = self.ranges
        out = []
        if j > 0 and self.sides != 'next':
            a, b = bounds[j - 1]
            out.extend(range(max(a, b - self.halo), b))
        if j + 1 < len(bounds) and self.sides != 'prev':
            a, b = bounds[j + 1]
            out.extend(range(a, min(b, a + self.halo)))
        return out

    def shared_frames(self, j: int) -> list:
        """frames scene j reads beyond its own: the halo frames, then extra[j] in ascending order without scene j's
        own frames and without frames the halo already gave (a frame that extra[j] lists twice is read twice)"""
        first, end = self.ranges[j]
        halo = self.halo_frames(j)
        taken = set(halo).union(range(first, end))
        return halo + [f for f in sorted(self.extra.get(j, ())) if f not in taken]

    def key_frames(self, j: int) -> list:
        """scene j's own frames, then its shared frames: the key order of its packed scope"""
        first, end = self.ranges[j]
        return list(range(first, end)) + self.shared_frames(j)

    def key_range(self, j: int) -> tuple:
        """(lowest, one past the highest) key frame of scene j; one contiguous range when its shared frames are
        adjacent to it (halo only)"""
        first, end = self.ranges[j]
        shared = self.shared_frames(j)
        return min([first] + shared), max([end - 1] + shared) + 1
