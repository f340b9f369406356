"""Frame memory on the GPU: the drop-in `FrameMemory` of src/onereel/frame_memory.py (same constructor, attributes and
methods, same results).

Once per denoising step (per layer with per_layer=True), the observed layer's video hidden states are summed per
latent frame on the GPU (`collect` -> `or_frame_pool`), the per-frame means are L2-normalised and clustered by one
workgroup (`finish` -> `select` -> `or_frame_select`: farthest-point start, k-means by dot product, one medoid per
cluster), and the chosen frames become, from the next step on, the extra key frames of every other scene
(`begin_step` writes `SceneLayout.extra`). Step 0 has no features yet: scenes read the sink frames and the halo frames
of a fallback layout. One GPU holds every token, so the per-frame sums need no all-reduce.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import _lib as L
from .layout import SceneLayout


class FrameMemory:
    """budget: representative frames per step, the sink frames included; candidates: 'all' frames, or 'boundary' (the
    first and last frame of every scene); layer: the observed layer (None: n_layers // 2 at reset); fallback: (halo,
    sides) of the frames scenes read at step 0; sink: frames every scene reads at every step; per_layer: every layer
    observes and gets its own representatives (the ablation); iters: k-means passes at most."""

    def __init__(self, budget: int = 4, candidates: str = 'all', layer: int | None = None, fallback=(2, 'adj'),
                 sink=(), per_layer: bool = False, iters: int = 20):
        if candidates not in ('all', 'boundary'):
            raise AssertionError(f"candidates must be 'all' or 'boundary', got {candidates!r}")
        if len(sink) >= budget:
            raise AssertionError('the sink frames are part of the budget')
        self.budget, self.candidates, self.layer, self.fallback = budget, candidates, layer, fallback
        self.sink, self.per_layer, self.iters = tuple(sink), per_layer, iters
        self.extra = None
        self._start(None)

    def _start(self, layout):
        """per-request state: no step seen, nothing pending or pooled; history[i] = representatives of step i + 1"""
        self.layout, self.step, self.pending, self.history = layout, -1, None, []
        self.sums, self.counts = {}, {}
        self._frame_map = None          # (frame tensor, its version counter, frame_major of it): collect's cache

    def reset(self, layout: SceneLayout, n_layers: int):
        """a new request on `layout`: at step 0 every scene reads the sink and the fallback halo frames
        (layout.extra is set here)"""
        self._start(layout)
        self.n_layers = n_layers
        if self.layer is None:
            self.layer = n_layers // 2
        halo, sides = self.fallback
        step0 = self._extra([], SceneLayout(layout.lengths, halo=halo, sides=sides))
        layout.extra = step0
        self.extra = dict.fromkeys(range(n_layers), step0) if self.per_layer else step0

    def _extra(self, reps, halo=None) -> dict:
        """scene -> the frames of other scenes it reads: the sink and the representatives (and the halo frames of the
        fallback layout `halo`), ascending, without the scene's own frames"""
        common = set(self.sink).union(reps)
        out = {}
        for j, (first, end) in enumerate(self.layout.ranges):
            wanted = common.union(halo.halo_frames(j)) if halo is not None else common
            out[j] = sorted(wanted.difference(range(first, end)))
        return out

    def observes(self, layer: int) -> bool:
        """whether `collect` is called for this layer"""
        return self.per_layer or layer == self.layer

    def set_representatives(self, reps):
        """representatives chosen outside `finish` (per_layer: layer -> frames); they take effect at the next step"""
        self.pending = reps

    def begin_step(self, step: int):
        """called at every transformer forward; the first forward of a new step applies what the previous step chose"""
        if step == self.step:
            return
        self.step = step
        if self.pending is None:
            return
        reps, self.pending = self.pending, None
        self.history.append(reps)
        if self.per_layer:
            self.extra = {layer: self._extra(r) for layer, r in reps.items()}
            return
        self.extra = self._extra(reps)
        self.layout.extra = self.extra

    def use_layer(self, layer: int):
        """per_layer: point the layout at this layer's extra frames (called before each block)"""
        if self.per_layer and self.extra is not None:
            self.layout.extra = self.extra[layer]

    def candidate_frames(self) -> list:
        """frames a representative may be, ascending, the sink frames left out"""
        if self.candidates == 'all':
            pool = range(self.layout.n_frames)
        else:
            pool = sorted({f for a, b in self.layout.ranges for f in (a, b - 1)})
        sink = set(self.sink)
        return [f for f in pool if f not in sink]

    @staticmethod
    def frame_major(frame: np.ndarray):
        """(row0, T) when frame[r] == (row0 + r) // T for every row r (the one-GPU processors' token order), else None"""
        n = len(frame)
        if n == 0 or (frame < 0).any():
            return None
        step = np.diff(frame)
        if ((step != 0) & (step != 1)).any():
            return None
        cuts = np.flatnonzero(step) + 1
        run = np.diff(np.concatenate([[0], cuts, [n]]))
        if len(run) > 2:
            T = int(run[1])
            if (run[1:-1] != T).any() or run[0] > T or run[-1] > T:
                return None
        else:
            T = int(run.max())
        return int(frame[0]) * T + (T - int(run[0])), T

    def frame_layout(self, frame: torch.Tensor):
        """frame_major of a frame map, read back to the host once per map: the cache holds the tensor itself (so its
        memory cannot be reused by another map) and its version counter (so in-place changes are seen)"""
        hit = self._frame_map
        if hit is None or hit[0] is not frame or hit[1] != frame._version:
            hit = (frame, frame._version, self.frame_major(frame.detach().cpu().numpy()))
            self._frame_map = hit
        return hit[2]

    def collect(self, frame, hs, layer=None):
        """pool an observed layer's rows into per-frame sums: frame [N] latent frame of each row (-1: not video), hs
        [N, C] hidden states, both on the GPU. Frame-major maps run the deterministic pool kernel (rows added in row
        order); any other map (a ring permutation) uses torch's index_add_ on the GPU."""
        if not (frame.is_cuda and hs.is_cuda):
            raise L.HipTypeError('frame and hs must be GPU tensors')
        layer = self.layer if layer is None else layer
        if layer not in self.sums:
            n_frames = self.layout.n_frames
            self.sums[layer] = torch.zeros(n_frames, hs.shape[-1], dtype=torch.float32, device=hs.device)
            self.counts[layer] = torch.zeros(n_frames, dtype=torch.float32, device=hs.device)
        x = hs.reshape(-1, hs.shape[-1])
        rows = self.frame_layout(frame)
        if rows is not None and x.dtype == torch.bfloat16 and x.stride(1) == 1 and x.shape[-1] % 8 == 0 and \
                x.data_ptr() % 16 == 0 and x.stride(0) % 8 == 0:
            row0, T = rows
            L.check(L.lib().or_frame_pool(x.data_ptr(), x.shape[0], x.shape[1], x.stride(0), row0, T,
                                          self.layout.n_frames, self.sums[layer].data_ptr(),
                                          self.counts[layer].data_ptr(), L.stream_handle(x.device)), 'or_frame_pool')
            return
        video = frame >= 0
        self.sums[layer].index_add_(0, frame[video], x[video].float())
        self.counts[layer].index_add_(0, frame[video], torch.ones_like(frame[video], dtype=torch.float32))

    @torch.no_grad()
    def finish(self):
        """after the conditional pass: the next step's representatives from the pooled features (one GPU holds every
        frame's sums, so there is nothing to all-reduce)"""
        if not self.sums:
            return
        layers = sorted(self.sums)
        sums = torch.stack([self.sums[layer] for layer in layers])
        counts = torch.stack([self.counts[layer] for layer in layers])
        self.sums, self.counts = {}, {}
        feats = F.normalize(sums / counts.clamp_min(1)[..., None], dim=-1)
        if self.per_layer:
            self.pending = {layer: self.select(f) for layer, f in zip(layers, feats)}
        else:
            self.pending = self.select(feats[0])

    def select(self, feats: torch.Tensor) -> list:
        """feats [n_frames, C] L2-normalised frame features on the GPU -> the representatives, ascending: k-means with
        the dot product over the candidate frames (farthest-point start from the first candidate), then per non-empty
        cluster the member most similar to its centre, the lowest frame on ties. One workgroup (or_frame_select) and
        one read-back of the k chosen frames."""
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
