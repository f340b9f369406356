"""Frame memory: the per-step `SceneLayout.extra` that the scene-attention layout reads (src/onereel/frame_memory.py).

On the hot path is the part that turns representative frames into every scene's extra key frames: `reset` (step 0
reads the fallback halo frames and the sink), `_extra`, `begin_step` (a new step applies the previous step's
representatives) and `use_layer` (frame_memory.py:34-74). The representatives themselves come from the conditional
pass's k-means over pooled frame features (`collect` / `finish` / `select`, frame_memory.py:76-132); that selection
is not built in this package yet, so representatives are supplied with `set_representatives`.
"""
from __future__ import annotations

from .layout import SceneLayout


class FrameMemory:
    def __init__(self, budget: int = 4, candidates: str = 'all', layer: int | None = None, fallback=(2, 'adj'),
                 sink=(), per_layer: bool = False, iters: int = 20):
        assert candidates in ('all', 'boundary'), candidates
        assert len(sink) < budget, 'the sink frames are part of the budget'
        self.budget, self.candidates, self.layer, self.fallback, self.iters = budget, candidates, layer, fallback, iters
        self.sink, self.per_layer = tuple(sink), per_layer
        self.layout, self.step, self.pending = None, -1, None
        self.history, self.extra = [], None          # history: per step the representatives in use

    def reset(self, layout: SceneLayout, n_layers: int):
        """a new request: fallback halo frames (and the sink) at step 0 (frame_memory.py:34-44)"""
        self.layout, self.step, self.pending, self.history = layout, -1, None, []
        self.n_layers = n_layers
        if self.layer is None:
            self.layer = n_layers // 2
        h, sides = self.fallback
        halo = SceneLayout(layout.lengths, halo=h, sides=sides)
        first = self._extra([], halo)
        layout.extra = first
        self.extra = {l: first for l in range(n_layers)} if self.per_layer else first

    def _extra(self, reps, halo=None) -> dict:
        """scene -> frames of other scenes it reads: the sink, the representatives (and the fallback halo frames)"""
        out = {}
        for j, (lo, hi) in enumerate(self.layout.ranges):
            fr = set(self.sink) | set(reps) | set(halo.halo_frames(j) if halo else ())
            out[j] = sorted(f for f in fr if not lo <= f < hi)
        return out

    def observes(self, layer: int) -> bool:
        return self.per_layer or layer == self.layer

    def set_representatives(self, reps):
        """the representatives chosen in this step (what `finish` leaves pending); applied at the next step. With
        per_layer, a dict layer -> representatives."""
        self.pending = reps

    def begin_step(self, step: int):
        """at every transformer forward: a new step applies the representatives chosen in the previous one"""
        if step == self.step:
            return
        self.step = step
        if self.pending is not None:
            reps, self.pending = self.pending, None
            self.history.append(reps)
            if self.per_layer:
                self.extra = {l: self._extra(r) for l, r in reps.items()}
            else:
                self.extra = self._extra(reps)
                self.layout.extra = self.extra

    def use_layer(self, layer: int):
        """per_layer: the extra frames of this layer (called before each block)"""
        if self.per_layer and self.extra is not None:
            self.layout.extra = self.extra[layer]

    def candidate_frames(self) -> list:
        if self.candidates == 'all':
            cand = range(self.layout.n_frames)
        else:
            cand = sorted({f for lo, hi in self.layout.ranges for f in (lo, hi - 1)})
        return [f for f in cand if f not in self.sink]

    def collect(self, frame, hs, layer=None):
        raise NotImplementedError('frame-memory feature pooling is not built in onereel_amd; '
                                  'pass the representatives with set_representatives')

    def finish(self):
        raise NotImplementedError('frame-memory k-means selection is not built in onereel_amd; '
                                  'pass the representatives with set_representatives')

    def select(self, feats):
        raise NotImplementedError('frame-memory k-means selection is not built in onereel_amd')
