"""Oracle: scene layout, frame-memory extras, token runs, scene-RoPE positions and the packed scope index arrays.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`). Plain Python / numpy restatement of the reference:

- `SceneLayout`                      follows src/onereel/layout.py:10-78
- `FrameMemoryExtra`                 follows src/onereel/frame_memory.py:24-69 (`reset`, `_extra`, `begin_step`; the
                                     k-means `select` is not on the hot path: representatives are given)
- `runs`, `frame_tokens`             follow src/onereel/parallel/comm.py:84-85,115-123
- `frame_position`, `scene_rope_rows`, `adjacent_positions`, `shared_positions`, `text_ranges`
                                     follow src/onereel/models/hunyuan15.py:87-124,443-454
- `hunyuan_scopes`                   follows `_segments` (hunyuan15.py:153-170) as called by `Processor.scene` on one GPU
                                     (hunyuan15.py:212-251: every scene local, every sentence queried), with the packing
                                     of `attention.packed` (src/onereel/attention.py:65-71) and the rows of `own_rows`
                                     (hunyuan15.py:225) and `_move_shared` (hunyuan15.py:127-150)
- `wan_scopes`                       follows `wan.Processor.ranges` (src/onereel/models/wan.py:110-124)

Row space of every index array: the virtual concatenation [video tokens (F*T rows, frame-major) ; text rows (Le)].
A text row t is encoded as F*T + t.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class SceneLayout:
    """layout.py:10-78. lengths: latent frames per scene; halo frames of the neighbours per `sides`; extra[j]: frames
    of other scenes that scene j also reads."""
    lengths: list
    halo: int = 2
    sides: str = 'adj'
    extra: dict = field(default_factory=dict)

    def __post_init__(self):
        assert self.sides in ('adj', 'prev', 'next'), self.sides          # layout.py:21
        assert all(n > 0 for n in self.lengths), self.lengths           # layout.py:22

    @classmethod
    def even(cls, n_frames, n_scenes, **kw):
        """layout.py:25-28: scene of frame f = f * n_scenes // n_frames"""
        sc = [f * n_scenes // n_frames for f in range(n_frames)]
        return cls([sc.count(j) for j in range(n_scenes)], **kw)

    @property
    def n_frames(self):
        return sum(self.lengths)

    @property
    def n_scenes(self):
        return len(self.lengths)

    @property
    def ranges(self):
        """layout.py:43-45"""
        out, s = [], 0
        for n in self.lengths:
            out.append((s, s + n))
            s += n
        return out

    @property
    def frames(self):
        return [list(range(lo, hi)) for lo, hi in self.ranges]

    def scene_of_frame(self):
        return [j for j, n in enumerate(self.lengths) for _ in range(n)]

    def halo_frames(self, j):
        """layout.py:54-63: previous neighbour's last `halo` frames, then the next neighbour's first"""
        fr, k, out = self.frames, self.halo, []
        if k == 0:
            return out
        if j > 0 and self.sides in ('adj', 'prev'):
            out += fr[j - 1][-k:]
        if j + 1 < self.n_scenes and self.sides in ('adj', 'next'):
            out += fr[j + 1][:k]
        return out

    def shared_frames(self, j):
        """layout.py:65-69: halo frames, then sorted extra frames outside the scene and not in the halo list (the
        filter tests against the halo list only, so a frame repeated in extra[j] stays repeated)"""
        lo, hi = self.ranges[j]
        out = self.halo_frames(j)
        return out + [f for f in sorted(self.extra.get(j, ())) if not lo <= f < hi and f not in out]

    def key_frames(self, j):
        """layout.py:71-73"""
        return self.frames[j] + self.shared_frames(j)

    def key_range(self, j):
        """layout.py:75-78"""
        kf = self.key_frames(j)
        return min(kf), max(kf) + 1


class FrameMemoryExtra:
    """frame_memory.py:24-69, the part that feeds the layout: step 0 reads the fallback halo frames (and the sink),
    later steps the sink plus the representatives chosen in the previous step, minus each scene's own frames, sorted."""

    def __init__(self, budget=4, fallback=(2, 'adj'), sink=()):
        assert len(sink) < budget                                       # frame_memory.py:28
        self.budget, self.fallback, self.sink = budget, fallback, tuple(sink)
        self.layout, self.step, self.pending, self.history, self.extra = None, -1, None, [], None

    def reset(self, layout):
        """frame_memory.py:34-44"""
        self.layout, self.step, self.pending, self.history = layout, -1, None, []
        h, sides = self.fallback
        first = self._extra([], SceneLayout(layout.lengths, halo=h, sides=sides))
        layout.extra = first
        self.extra = first

    def _extra(self, reps, halo=None):
        """frame_memory.py:46-52"""
        out = {}
        for j, (lo, hi) in enumerate(self.layout.ranges):
            fr = set(self.sink) | set(reps) | set(halo.halo_frames(j) if halo else ())
            out[j] = sorted(f for f in fr if not lo <= f < hi)
        return out

    def propose(self, reps):
        """stands in for `finish` (frame_memory.py:88-101): the representatives the next step applies"""
        self.pending = sorted(reps)

    def begin_step(self, step):
        """frame_memory.py:57-69"""
        if step == self.step:
            return
        self.step = step
        if self.pending is not None:
            reps, self.pending = self.pending, None
            self.history.append(reps)
            self.extra = self._extra(reps)
            self.layout.extra = self.extra


def runs(frames):
    """comm.py:115-123: frame list (in order) -> contiguous runs"""
    out = []
    for f in frames:
        if out and out[-1][1] == f:
            out[-1][1] = f + 1
        else:
            out.append([f, f + 1])
    return [tuple(r) for r in out]


def frame_tokens(frames, T):
    """comm.py:84-85"""
    return [(lo * T, hi * T) for lo, hi in runs(frames)]


def text_ranges(counts):
    """hunyuan15.py:87-89: sentence j's rows [c_j, c_{j+1}) of the valid-first text sequence"""
    c = np.cumsum([0] + list(counts))
    return [(int(c[j]), int(c[j + 1])) for j in range(len(c) - 1)]


def frame_position(lay, f, scene_rope, rope_lengths=None):
    """hunyuan15.py:103-113: temporal RoPE index of latent frame f"""
    if not scene_rope:
        return f
    start = 0
    for n in list(rope_lengths or lay.lengths):
        if f < start + n:
            return f - start + (start > 0)
        start += n
    raise IndexError(f)


def scene_rope_rows(lay, T, rope_lengths=None):
    """hunyuan15.py:443-454: per video token, the rotary row at its frame index within its scene (+1 after scene 0)"""
    lengths = list(rope_lengths or lay.lengths)
    start = np.repeat(np.cumsum([0] + lengths[:-1]), lengths)
    local = np.arange(sum(lengths)) - start + (start > 0)
    return (local[:, None] * T + np.arange(T)[None]).reshape(-1).astype(np.int64)


def adjacent_positions(lay, j):
    """hunyuan15.py:92-100: global RoPE, shared_pos 'adjacent'. A dict keeps the last index of a repeated frame."""
    lo, hi = lay.ranges[j]
    shared = lay.shared_frames(j)
    before, after = sorted(f for f in shared if f < lo), sorted(f for f in shared if f >= hi)
    pos = {f: lo - len(before) + i for i, f in enumerate(before)}
    pos.update({f: hi + i for i, f in enumerate(after)})
    return [pos[f] for f in shared]


def shared_positions(lay, j, scene_rope, rope_lengths=None):
    """hunyuan15.py:116-124"""
    if not scene_rope:
        return adjacent_positions(lay, j)
    shared = lay.shared_frames(j)
    last = max(frame_position(lay, f, True, rope_lengths) for f in lay.frames[j])
    pos = {f: last + 1 + i for i, f in enumerate(sorted(shared))}
    return [pos[f] for f in shared]


def _rows(frames, T):
    """the token rows of a frame list in order: own_rows (hunyuan15.py:225) = cat of frame_tokens runs"""
    parts = [np.arange(lo, hi) for lo, hi in frame_tokens(frames, T)]
    return np.concatenate(parts) if parts else np.zeros(0, np.int64)


@dataclass
class Scopes:
    """packed scope index arrays (all int64 numpy); kind[s] is 'v' or 't'"""
    kind: list
    scene: list
    lq: list
    lk: list
    cu_q: np.ndarray
    cu_k: np.ndarray
    q_src: np.ndarray        # [sum lq] query row (= write-back row of its output)
    k_src: np.ndarray        # [sum lk] key / value row
    q_rope: np.ndarray       # [sum lq] rotary row of a raw query (-1: text, no RoPE)
    k_rope: np.ndarray       # [sum lk] rotary row of a raw key (shared frames at their adjacent row when moved)
    k_move_a: np.ndarray     # [sum lk] pre-rotated keys: _move_shared's first (inverse) rotation row, -1 if not moved
    k_move_b: np.ndarray     # [sum lk] pre-rotated keys: _move_shared's second rotation row, -1 if not moved
    n_video: int
    text_rows: int

    @property
    def max_q(self):
        return max(self.lq)

    @property
    def max_k(self):
        return max(self.lk)


def hunyuan_scopes(lay, T, counts, text_rows=None, scene_rope=False, rope_lengths=None, adjacent=False,
                   with_text=True, token_range=None):
    """Processor.scene on one GPU (hunyuan15.py:212-251) -> the packed layout of its single `A.packed` call.

    token_range=(a, b): one rank's share with several ranks (hunyuan15.py:219-224): the scenes overlapping video
    tokens [a, b), each with its queries clipped to the range (`mine`) and its full keys, and the sentence segment of
    the scenes whose first token lies in the range (`text_for`). The reference packs these segments in two calls
    (scenes whose keys are all local first, then the others, hunyuan15.py:236-246); they are listed here in scene
    order, each segment's rows as the reference builds them.

    Segment order (hunyuan15.py:158-169): V_0, T_0, V_1, T_1, ... V_j: queries = scene j's video rows; keys =
    key_frames(j) rows then sentence j's rows. T_j: queries = sentence j's rows; keys = frames(j) rows then sentence
    j's rows. `adjacent`: shared_pos 'adjacent', or 'switch' at a step >= shared_switch (hunyuan15.py:162).
    with_text=False gives video-only scopes (the Wan self-attention packing, wan.py:113-119)."""
    F = lay.n_frames
    S = F * T
    tr = text_ranges(counts) if with_text else [(0, 0)] * lay.n_scenes
    Le = (tr[-1][1] if tr else 0) if text_rows is None else text_rows
    rows = scene_rope_rows(lay, T, rope_lengths) if scene_rope else np.arange(S, dtype=np.int64)
    ra, rb = token_range if token_range is not None else (0, S)
    kind, scene, lq, lk = [], [], [], []
    qs, ks, qr, kr, ka, kb = [], [], [], [], [], []
    for j, (lo, hi) in enumerate(lay.ranges):
        if not (lo * T < rb and hi * T > ra):           # not one of this rank's scenes (mine)
            continue
        t0, t1 = tr[j]
        keys = lay.key_frames(j)
        text = S + np.arange(t0, t1)
        n_own = len(lay.frames[j]) * T
        # V_j: the scene's video queries inside the range
        q = np.arange(max(lo * T, ra), min(hi * T, rb))
        kv = _rows(keys, T)
        rope_k = rows[kv].copy()
        move_a = np.full(len(kv), -1, np.int64)
        move_b = np.full(len(kv), -1, np.int64)
        shared = lay.shared_frames(j)
        if adjacent and shared:
            # _move_shared (hunyuan15.py:127-150): shared keys re-rotated by d = dst - src frames, through table rows
            # a and a + d (a = max(0, -d)) of the same spatial position
            for i, (f, dst) in enumerate(zip(shared, shared_positions(lay, j, scene_rope, rope_lengths))):
                d = dst - frame_position(lay, f, scene_rope, rope_lengths)
                a = 0 if d >= 0 else -d
                sl = slice(n_own + i * T, n_own + (i + 1) * T)
                rope_k[sl] = dst * T + np.arange(T)
                move_a[sl] = a * T + np.arange(T)
                move_b[sl] = (a + d) * T + np.arange(T)
        kind.append('v'), scene.append(j), lq.append(len(q)), lk.append(len(kv) + len(text))
        qs.append(q), qr.append(rows[q])
        ks += [kv, text]
        kr += [rope_k, np.full(len(text), -1, np.int64)]
        ka += [move_a, np.full(len(text), -1, np.int64)]
        kb += [move_b, np.full(len(text), -1, np.int64)]
        if with_text and ra <= lo * T < rb:
            # T_j (text_for: the scene's first token lies in the range; every scene on one GPU, hunyuan15.py:223)
            kv = _rows(lay.frames[j], T)
            kind.append('t'), scene.append(j), lq.append(t1 - t0), lk.append(len(kv) + len(text))
            qs.append(text), qr.append(np.full(len(text), -1, np.int64))
            ks += [kv, text]
            kr += [rows[kv], np.full(len(text), -1, np.int64)]
            ka += [np.full(len(kv) + len(text), -1, np.int64)]
            kb += [np.full(len(kv) + len(text), -1, np.int64)]
    cat = lambda xs: np.concatenate(xs).astype(np.int64) if xs else np.zeros(0, np.int64)
    return Scopes(kind, scene, lq, lk, np.cumsum([0] + lq), np.cumsum([0] + lk), cat(qs), cat(ks), cat(qr), cat(kr),
                  cat(ka), cat(kb), S, Le)


def wan_ranges(lay, T):
    """wan.py:120-124: (q_ranges, k_ranges) of the zero-copy overlapping key ranges (no extra frames)"""
    q_ranges = [(lo * T, hi * T) for lo, hi in lay.ranges]
    k_ranges = []
    for j in range(lay.n_scenes):
        a, b = lay.key_range(j)
        assert b - a == len(lay.key_frames(j)), 'halo must be contiguous with its scene'      # wan.py:123
        k_ranges.append((a * T, b * T))
    return q_ranges, k_ranges
