"""Frame memory: per-step representative frames and the `SceneLayout.extra` they give (src/onereel/frame_memory.py).

- `reset`, `_extra`, `begin_step`, `use_layer` (frame_memory.py:34-74): step 0 reads the fallback halo frames and the
  sink; a new step applies the representatives chosen in the previous one; per-layer extras for the ablation.
- `collect` (:76-85): an observed layer's video rows pooled per latent frame by `or_frame_pool` (deterministic: each
  frame's rows are added in row order). Rows in the frame-major order the one-GPU processors use
  (frame = (row0 + r) // T) take the kernel; any other frame map (a ring permutation) falls back to torch's
  index_add_ on the GPU, as the reference does.
- `finish` (:87-101): features = L2-normalised frame means (torch, [F, C] on the GPU), then `select` per layer.
- `select` (:114-132): farthest-point initialisation, k-means with the dot product, medoid per cluster: one workgroup
  (`or_frame_select`) instead of a Python loop of small launches, with one device-to-host copy of the k chosen frames.
  There is one GPU, so the reference's all-reduce of the sums is the identity.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import _lib as L
from .layout import SceneLayout


class FrameMemory:
    def __init__(self, budget: int = 4, candidates: str = 'all', layer: int | None = None, fallback=(2, 'adj'),
                 sink=(), per_layer: bool = False, iters: int = 20):
        assert candidates in ('all', 'boundary'), candidates
        assert len(sink) < budget, 'the sink frames are part of the budget'
        self.budget, self.candidates, self.layer, self.fallback, self.iters = budget, candidates, layer, fallback, iters
        self.sink, self.per_layer = tuple(sink), per_layer
        self.layout, self.step, self.pending, self.sums, self.counts = None, -1, None, {}, {}
        self.history, self.extra = [], None          # history: per step the representatives in use
        self._rows = {}                              # frame tensor -> (row0, T) when its rows are frame-major

    def reset(self, layout: SceneLayout, n_layers: int):
        """a new request: fallback halo frames (and the sink) at step 0 (frame_memory.py:34-44)"""
        self.layout, self.step, self.pending, self.sums, self.counts, self.history = layout, -1, None, {}, {}, []
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

    @staticmethod
    def frame_major(frame: np.ndarray):
        """(row0, T) with frame[r] == (row0 + r) // T for every row, or None"""
        n = len(frame)
        if n == 0 or (frame < 0).any():
            return None
        d = np.diff(frame)
        if ((d != 0) & (d != 1)).any():
            return None
        cuts = np.flatnonzero(d) + 1
        runs = np.diff(np.concatenate([[0], cuts, [n]]))
        if len(runs) > 2:
            T = int(runs[1])
            if (runs[1:-1] != T).any() or runs[0] > T or runs[-1] > T:
                return None
        else:
            T = int(runs.max())
        return int(frame[0]) * T + (T - int(runs[0])), T

    def collect(self, frame, hs, layer=None):
        """frame [N] latent frame of each local row (-1: not video); hs [N, C] hidden states of an observed layer
        (frame_memory.py:76-85)"""
        layer = self.layer if layer is None else layer
        n_frames = self.layout.n_frames
        if layer not in self.sums:
            self.sums[layer] = torch.zeros(n_frames, hs.shape[-1], dtype=torch.float32, device=hs.device)
            self.counts[layer] = torch.zeros(n_frames, dtype=torch.float32, device=hs.device)
        key = (frame.data_ptr(), frame.numel(), str(frame.device))
        if key not in self._rows:
            self._rows[key] = self.frame_major(frame.detach().cpu().numpy())
        rows = self._rows[key]
        x = hs.reshape(-1, hs.shape[-1])
        if rows is not None and x.dtype == torch.bfloat16 and x.stride(1) == 1 and x.shape[-1] % 8 == 0 and \
                x.data_ptr() % 16 == 0 and x.stride(0) % 8 == 0:
            row0, T = rows
            L.check(L.lib().or_frame_pool(x.data_ptr(), x.shape[0], x.shape[1], x.stride(0), row0, T, n_frames,
                                          self.sums[layer].data_ptr(), self.counts[layer].data_ptr(),
                                          L.stream_handle(x.device)), 'or_frame_pool')
        else:
            keep = frame >= 0
            self.sums[layer].index_add_(0, frame[keep], x[keep].float())
            self.counts[layer].index_add_(0, frame[keep], torch.ones_like(frame[keep], dtype=torch.float32))

    @torch.no_grad()
    def finish(self):
        """after the conditional pass: choose the next step's representatives from the pooled features
        (frame_memory.py:87-101; one GPU, so no all-reduce)"""
        if not self.sums:
            return
        layers = sorted(self.sums)
        sums = torch.stack([self.sums[l] for l in layers])
        counts = torch.stack([self.counts[l] for l in layers])
        self.sums, self.counts = {}, {}
        feats = F.normalize(sums / counts.clamp_min(1)[..., None], dim=-1)
        if self.per_layer:
            self.pending = {l: self.select(f) for l, f in zip(layers, feats)}
        else:
            self.pending = self.select(feats[0])

    def select(self, feats: torch.Tensor) -> list:
        """k-means (cosine) over the candidate frames; the medoid (nearest member, lowest index on ties) of each
        cluster, ascending (frame_memory.py:114-132)"""
        cand = self.candidate_frames()
        k = min(self.budget - len(self.sink), len(cand))
        if k <= 0:
            return []
        n_frames, C = feats.shape
        if any(not 0 <= f < n_frames for f in cand):
            raise L.HipValueError(f'candidate frames outside [0, {n_frames})')
        x = feats.to(torch.float32).contiguous()
        dev = x.device
        ct = torch.tensor(cand, dtype=torch.int32, device=dev)
        reps = torch.empty(k, dtype=torch.int32, device=dev)
        work = torch.empty(8, C, dtype=torch.float32, device=dev)
        L.check(L.lib().or_frame_select(x.data_ptr(), n_frames, C, ct.data_ptr(), len(cand), k, self.iters,
                                        reps.data_ptr(), work.data_ptr(), L.stream_handle(dev)), 'or_frame_select')
        return [int(r) for r in reps.cpu().tolist() if r >= 0]
