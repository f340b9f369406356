"""HunyuanVideo-1.5 scene attention on one MI355X: the drop-in attention processor (src/onereel/models/hunyuan15.py).

`Processor.__call__` keeps the diffusers processor signature (hunyuan15.py:177-210): the QKV projections and the
RMSNorms run as the model's own torch modules; the scene-attention layer (RoPE, scope packing, varlen attention,
write-back) runs as HIP kernels through `onereel_amd.scene`, with the scene RoPE fused into the K pack and the Q
load. With `Context.memory` = M > 0 the processor runs the head-major bounded memory instead
(`Processor.memory`, hunyuan15.py:200-201,305-334): q / k rotated once in token order, then `onereel_amd.memory`'s
MemoryAttention over every scene's frames, sentence and M representatives per head of the other scenes. The
multi-GPU modes of the reference (K/V gathering, Ulysses, ring) and subject links are not implemented.
"""
from __future__ import annotations

from bisect import bisect_right
from dataclasses import dataclass, field
from itertools import accumulate

import torch

from . import _lib as L
from .frame_memory import FrameMemory
from .layout import SceneLayout
from .memory import BoundaryMemory, MemoryAttention, frame_plan
from .scene import ScopePlan, rotate_queries, scene_attention


@dataclass
class Context:
    """the fields of the reference Context (hunyuan15.py:34-79) that the single-GPU scene path reads"""
    layout: SceneLayout
    mode: str = 'scene'
    cfg: bool = True
    shared_pos: str = 'source'           # 'source' | 'adjacent' | 'switch' (adjacent from step shared_switch on)
    shared_switch: int = 10
    scene_rope: bool = False             # temporal RoPE index restarts at every scene (+1 after scene 0)
    rope_lengths: list = None            # scene lengths for scene_rope (default: the attention layout's)
    memory: int = 0                      # M > 0: bounded cross-scene memory of M representatives per head (halo 0)
    frame_memory: FrameMemory = None
    T: int = 0
    fwd: int = 0
    counts: dict = field(default_factory=dict)   # CFG branch (True = cond) -> MLLM tokens per sentence
    fused: bool = True                   # Q read and outputs written in place (False: the reference's packed flow)
    _cache: dict = field(default_factory=dict)
    _rot_full: tuple = None
    _mem: MemoryAttention = None         # the bounded memory's state (centroids per layer and branch, plans)

    def step(self) -> int:
        """denoising step of the current forward (forwards count from 1; with CFG a step takes two forwards)"""
        return (self.fwd - 1) // (2 if self.cfg else 1)

    def cond(self) -> bool:
        """the current forward is the conditional branch (the first of each CFG pair; always without CFG)"""
        return not self.cfg or (self.fwd - 1) % 2 == 0

    def text_ranges(self) -> list:
        c, out = 0, []
        for n in self.counts[self.cond()]:
            out.append((c, c + n))
            c += n
        return out

    def adjacent(self) -> bool:
        """shared frames at their adjacent positions in this step (hunyuan15.py:162)"""
        return self.shared_pos == 'adjacent' or (self.shared_pos == 'switch' and self.step() >= self.shared_switch)


def adjacent_positions(lay: SceneLayout, j: int) -> list:
    """shared_pos 'adjacent' under global RoPE (hunyuan15.py:92-100): per shared frame of scene j, in shared_frames
    order, its temporal position. Frames before the scene occupy the slots just before its first frame and frames
    after it the slots from its end on, each group in time order; a frame listed twice takes its later slot."""
    first, end = lay.ranges[j]
    shared = lay.shared_frames(j)
    early = [f for f in shared if f < first]
    late = [f for f in shared if f >= end]
    return [first - 1 - sum(e > f for e in early) if f < first else end - 1 + sum(x <= f for x in late)
            for f in shared]


def frame_position(ctx: Context, f: int) -> int:
    """temporal RoPE index of latent frame f (hunyuan15.py:103-113): f itself, or with scene_rope its offset inside
    its rope scene plus one in every scene after the first; IndexError past the rope scenes"""
    if not ctx.scene_rope:
        return f
    ends = list(accumulate(ctx.rope_lengths or ctx.layout.lengths))
    s = bisect_right(ends, f)
    if s == len(ends):
        raise IndexError(f)
    start = ends[s - 1] if s else 0
    return f - start + (start > 0)


def shared_positions(ctx: Context, j: int) -> list:
    """per shared frame of scene j, in shared_frames order, its temporal RoPE index under shared_pos 'adjacent'
    (hunyuan15.py:116-124): with scene_rope the shared frames follow the scene's last position in time order (a frame
    listed twice takes its later slot); with global RoPE `adjacent_positions`"""
    lay = ctx.layout
    if not ctx.scene_rope:
        return adjacent_positions(lay, j)
    first, end = lay.ranges[j]
    top = max(frame_position(ctx, f) for f in range(first, end))
    shared = lay.shared_frames(j)
    return [top + sum(x <= f for x in shared) for f in shared]


def _key(ctx: Context, Le: int, adjacent: bool, moves: bool, device):
    lay = ctx.layout
    return ('plan', tuple(lay.lengths), lay.halo, lay.sides, tuple((j, tuple(v)) for j, v in sorted(lay.extra.items())),
            ctx.T, tuple(ctx.counts[ctx.cond()]), Le, ctx.scene_rope, tuple(ctx.rope_lengths or ()), adjacent, moves,
            str(device))


def scope_plan(ctx: Context, Le: int, device, moves: bool = False) -> ScopePlan:
    """the device layout of this step's scopes, cached per (layout, extra, counts, step mode)"""
    adjacent = ctx.adjacent()
    key = _key(ctx, Le, adjacent, moves, device)
    if key not in ctx._cache:
        ctx._cache[key] = ScopePlan(ctx.layout, ctx.T, ctx.counts[ctx.cond()], Le, ctx.scene_rope, ctx.rope_lengths,
                                    adjacent, True, device, moves=moves, text_keys_in_place=True)
    return ctx._cache[key]


def scene_rope_rows(ctx: Context, device) -> torch.Tensor:
    """per video token row, its rotary row at the frame index within its scene (hunyuan15.py:443-454), built by the
    device layout kernel (the queries of the video-only scopes, in token order)"""
    lengths = list(ctx.rope_lengths or ctx.layout.lengths)
    key = ('scene_rope', tuple(lengths), ctx.T, str(device))
    if key not in ctx._cache:
        plan = ScopePlan(SceneLayout(lengths, halo=0), ctx.T, None, 0, True, None, False, False, device)
        ctx._cache[key] = plan.q_rope.long()
    return ctx._cache[key]


def memory_attention(ctx: Context) -> MemoryAttention:
    """the context's bounded memory of ctx.memory representatives per head, created on first use (the reference's
    setup creates it, hunyuan15.py:590-592): it replaces the halo frames, so the layout has none"""
    if ctx._mem is None:
        if ctx.layout.halo != 0:
            raise L.HipValueError('the bounded memory replaces the halo frames: use halo = 0')
        ctx._mem = MemoryAttention(BoundaryMemory(ctx.memory))
    return ctx._mem


def rotate_tokens(ctx: Context, x: torch.Tensor, cos, sin) -> torch.Tensor:
    """x [F*T, H, D] rotated at every video token's rotary row (its scene row with scene_rope), in token order: the
    q / k RoPE of Processor.__call__ (hunyuan15.py:183-191) as one or_rotate_rows launch"""
    lay = ctx.layout
    key = ('tokens', tuple(lay.lengths), ctx.T, ctx.scene_rope, tuple(ctx.rope_lengths or ()), str(x.device))
    if key not in ctx._cache:
        ctx._cache[key] = ScopePlan(SceneLayout(list(lay.lengths), halo=0), ctx.T, None, 0, ctx.scene_rope,
                                    ctx.rope_lengths, False, False, x.device)
    return rotate_queries(ctx._cache[key], x, cos, sin)


class Processor:
    """the HunyuanVideo-1.5 attention processor with scene attention (hunyuan15.py:173-251), one GPU"""

    def __init__(self, ctx: Context, layer: int):
        self.ctx, self.layer = ctx, layer

    def __call__(self, attn, hidden_states, encoder_hidden_states=None, attention_mask=None, image_rotary_emb=None):
        ctx = self.ctx
        cos, sin = image_rotary_emb
        ctx._rot_full = image_rotary_emb
        q, k, v = (f(hidden_states).unflatten(2, (attn.heads, -1)) for f in (attn.to_q, attn.to_k, attn.to_v))
        q, k = attn.norm_q(q), attn.norm_k(k)
        q, k, v = (x[0].to(torch.bfloat16) for x in (q, k, v))
        eq, ek, ev = (f(encoder_hidden_states).unflatten(2, (attn.heads, -1))
                      for f in (attn.add_q_proj, attn.add_k_proj, attn.add_v_proj))
        if attn.norm_added_q is not None:
            eq = attn.norm_added_q(eq)
        if attn.norm_added_k is not None:
            ek = attn.norm_added_k(ek)
        eq, ek, ev = (x[0].to(torch.bfloat16) for x in (eq, ek, ev))
        if ctx.memory:
            q, k = rotate_tokens(ctx, q, cos, sin), rotate_tokens(ctx, k, cos, sin)
            hs, ehs = self.memory(q, k, v, eq, ek, ev)
        else:
            hs, ehs = self.scene_raw(q, k, v, eq, ek, ev, cos, sin)
        hs = attn.to_out[1](attn.to_out[0](hs.flatten(1, 2)[None].to(hidden_states.dtype)))
        ehs = attn.to_add_out(ehs.flatten(1, 2)[None].to(hidden_states.dtype))
        return hs, ehs

    def scene_raw(self, q, k, v, eq, ek, ev, cos, sin):
        """scene attention of q / k BEFORE RoPE: rotation fused into the kernels (video rows rotated at their scene
        rotary rows, moved shared keys at their adjacent rows, text rows not rotated)"""
        ctx = self.ctx
        plan = scope_plan(ctx, eq.shape[0], q.device)
        return scene_attention(plan, q, k, v, eq, ek, ev, cos, sin, mode='raw', fused=ctx.fused)

    def scene(self, q, k, v, eq, ek, ev):
        """the reference's entry (hunyuan15.py:212-251): q / k already rotated; shared keys re-rotated by
        _move_shared's two rotations through ctx._rot_full when the shared frames sit at adjacent positions"""
        ctx = self.ctx
        adjacent = ctx.adjacent()
        plan = scope_plan(ctx, eq.shape[0], q.device, moves=adjacent)
        cos, sin = ctx._rot_full if adjacent else (None, None)
        return scene_attention(plan, q, k, v, eq, ek, ev, cos, sin, mode='rotated', fused=ctx.fused)

    def memory(self, q, k, v, eq, ek, ev):
        """the bounded cross-scene memory on one GPU (hunyuan15.py:305-334, world 1): q / k already rotated. Every
        scene's video queries read its frames, its sentence and M representatives per head of the other scenes'
        boundary keys; its sentence queries read its frames and its sentence. Returns (video out, text out); text
        rows past the valid tokens are zero."""
        ctx, T, lay = self.ctx, self.ctx.T, self.ctx.layout
        mem = memory_attention(ctx)
        Sq = q.shape[0]
        if Sq != lay.n_frames * T:
            raise L.HipValueError(f'{Sq} video rows, the layout has {lay.n_frames * T}')
        pk = (ctx.cond(), Sq, k.shape[0])
        if pk not in mem.plans:
            pieces = [(j, lo * T, hi * T) for j, (lo, hi) in enumerate(lay.ranges)]
            mem.plans[pk] = frame_plan(lay, T, torch.arange(Sq), k.shape[0], pieces, ctx.text_ranges(),
                                       set(range(lay.n_scenes)), Sq, q.device)
        out = mem((self.layer, ctx.cond()), torch.cat([q, eq]), torch.cat([k, ek]), torch.cat([v, ev]), mem.plans[pk])
        return out[:Sq], out[Sq:]
