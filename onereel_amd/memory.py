"""Bounded cross-scene memory with per-head representatives (src/onereel/memory.py), on the HIP kernels.

The candidates are the boundary frames of every scene (first and last frame, each once). Per layer, CFG branch and
head, the L2-normalised candidate keys are clustered into at most M groups (k-means; warm-started from the previous
centroids after the first call), and each non-empty cluster keeps the candidate nearest its centroid. A scene's
queries then read their local keys plus the other scenes' representatives of their head, in one softmax.

Representatives differ per head, so the attention is head-major: every (head, query piece) pair is one single-head
segment of one varlen launch over rows of D elements, row = token * H + head. The reference gathers and scatters those
rows with torch indexing around FlashAttention (memory.py:145-174); here the same per-head index arrays drive:

- the pack kernel (queries; keys and values in one pass);
- the varlen kernel with one head;
- the scatter kernel.

The clustering (`BoundaryMemory.select`) keeps the reference's torch formulation on the GPU: batched matmuls for the
distances (hipBLASLt) and stable sorts for the deterministic choice (memory.py:48-93).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F

from .layout import SceneLayout
from .scene import gather_rows, scatter_rows, varlen

ITERS_INIT, ITERS_UPDATE = 50, 2


def candidate_frames(layout: SceneLayout):
    """boundary frames (first and last frame of every scene, each frame once) and their scene (memory.py:30-37)"""
    frames, owner = [], []
    for j, (lo, hi) in enumerate(layout.ranges):
        for f in dict.fromkeys((lo, hi - 1)):
            frames.append(f)
            owner.append(j)
    return frames, owner


def candidates(layout: SceneLayout, T: int, device):
    """video rows (frame-major, all tokens) of the boundary frames and their scene (memory.py:40-45)"""
    frames, owner = candidate_frames(layout)
    rows = torch.cat([torch.arange(f * T, (f + 1) * T, device=device) for f in frames])
    scene = torch.tensor(owner, device=device).repeat_interleave(T)
    return rows, scene


class BoundaryMemory:
    """per (layer, branch) key: centroids [H, M, D] carried across steps (memory.py:48-56)"""

    def __init__(self, M: int = 128):
        self.M = M
        self.centroids = {}

    def reset(self):
        self.centroids = {}

    @torch.no_grad()
    def select(self, key, kc: torch.Tensor):
        """kc [B, H, D] candidate keys -> (rep [H, M] candidate positions, valid [H, M]); one representative per
        non-empty cluster (nearest member, then lowest index), padded with valid = False (memory.py:58-93)"""
        x = F.normalize(kc.float().transpose(0, 1), dim=-1)
        H, B, D = x.shape
        M = min(self.M, B)
        c = self.centroids.get(key)
        if c is None or c.shape != (H, M, D):
            c = x[:, torch.linspace(0, B - 1, M, device=x.device).round().long()].clone()
            iters = ITERS_INIT
        else:
            iters = ITERS_UPDATE
        xx = (x * x).sum(-1, keepdim=True)
        for it in range(iters + 1):
            d = xx - 2 * x @ c.transpose(1, 2) + (c * c).sum(-1)[:, None]
            z = d.argmin(-1)
            if it == iters:
                break
            oh = F.one_hot(z, M).float()
            s, n = oh.transpose(1, 2) @ x, oh.sum(1)
            prev = c
            c = torch.where((n > 0)[..., None], s / n.clamp_min(1)[..., None], c)
            # the first clustering stops once the centroids stand still; the warm updates run their few iterations
            # without that host read (an iteration after convergence changes nothing, so the result is the same)
            if iters == ITERS_INIT and torch.equal(c, prev):
                break
        self.centroids[key] = c
        dist = d.gather(-1, z[..., None])[..., 0]
        o1 = dist.argsort(dim=-1, stable=True)
        o2 = z.gather(-1, o1).argsort(dim=-1, stable=True)
        order = o1.gather(-1, o2)
        zs = z.gather(-1, order)
        first = torch.ones_like(zs, dtype=torch.bool)
        first[:, 1:] = zs[:, 1:] != zs[:, :-1]
        rank = first.cumsum(-1) - 1
        # each cluster's first member goes to column rank; the other members to a spare column M, dropped after
        # (scatters instead of boolean indexing, which would read the selection's size back to the host)
        col = torch.where(first, rank, M)
        rep = torch.zeros(H, M + 1, dtype=torch.long, device=x.device).scatter_(1, col, order)[:, :M]
        valid = torch.zeros(H, M + 1, dtype=torch.bool, device=x.device).scatter_(1, col, first)[:, :M]
        return rep, valid


@dataclass
class Plan:
    """query pieces of one layer (memory.py:96-106)"""
    qrows: torch.Tensor                  # [sum Q] query rows, piece after piece
    qlen: torch.Tensor                   # [n] queries per piece
    pad: torch.Tensor                    # [n, Lmax] local key rows per piece (padded)
    pmask: torch.Tensor                  # [n, Lmax]
    lens: torch.Tensor                   # [n] local keys per piece
    scene: torch.Tensor                  # [n] scene of each piece
    mem: torch.Tensor                    # [n] the piece reads the memory
    cand: torch.Tensor                   # [B] key-buffer rows of the boundary candidates
    owner: torch.Tensor                  # [B] their scene
    max_qlen: int = 0                    # host copies: the longest piece's queries, local keys, and all local keys
    max_len: int = 0
    sum_len: int = 0


def make_plan(pieces, cand, owner, device) -> Plan:
    """pieces: [(scene, query rows, local key rows, reads memory)]; cand / owner: candidate key rows and their scene
    (memory.py:109-121)"""
    t = lambda x: torch.as_tensor(x, dtype=torch.long, device=device)
    pieces = [(j, t(q), t(k), m) for j, q, k, m in pieces if len(q)]
    lens = [len(k) for _, _, k, _ in pieces]
    pad = torch.zeros(len(pieces), max(lens), dtype=torch.long, device=device)
    pmask = torch.zeros_like(pad, dtype=torch.bool)
    for i, (_, _, k, _) in enumerate(pieces):
        pad[i, :len(k)] = k
        pmask[i, :len(k)] = True
    return Plan(qrows=torch.cat([q for _, q, _, _ in pieces]), qlen=t([len(q) for _, q, _, _ in pieces]), pad=pad,
                pmask=pmask, lens=t(lens), scene=t([j for j, _, _, _ in pieces]),
                mem=torch.tensor([m for *_, m in pieces], dtype=torch.bool, device=device), cand=t(cand),
                owner=t(owner), max_qlen=max(len(q) for _, q, _, _ in pieces), max_len=max(lens), sum_len=sum(lens))


def frame_plan(layout: SceneLayout, T: int, token_row, Lv: int, q_pieces, text_ranges=None, text_for=(), Sq: int = 0,
               device='cuda') -> Plan:
    """frame-major models (memory.py:124-137). Key buffer: Lv video rows (video token t at token_row[t]), then the
    text tokens; query buffer: Sq video rows, then the text tokens. q_pieces: [(scene, video query row lo, hi)]. Video
    queries read their scene, their sentence and the memory; sentence queries (scenes in text_for) read their scene
    and sentence."""
    token_row = torch.as_tensor(token_row)
    ar = lambda a, b: torch.arange(a, b)
    frows = lambda fs: token_row[torch.cat([ar(f * T, (f + 1) * T) for f in fs])]
    text = lambda j: Lv + ar(*text_ranges[j]) if text_ranges else ar(0, 0)
    pieces = [(j, ar(lo, hi), torch.cat([frows(layout.frames[j]), text(j)]), True) for j, lo, hi in q_pieces]
    pieces += [(j, Sq + ar(*text_ranges[j]), torch.cat([frows(layout.frames[j]), text(j)]), False)
               for j in sorted(text_for)]
    cf, owner = candidate_frames(layout)
    return make_plan(pieces, frows(cf), torch.tensor(owner).repeat_interleave(T), device)


class MemoryAttention:
    """packed head-major attention with the bounded memory (memory.py:140-174); plans are cached by the caller"""

    def __init__(self, memory: BoundaryMemory):
        self.memory = memory
        self.plans = {}

    def __call__(self, key, q, k, v, p: Plan) -> torch.Tensor:
        """q [Sq, H, D], k / v [L, H, D] bf16 buffers -> [Sq, H, D] (rows outside the plan's queries are zero)"""
        Sq, H, D = q.shape
        L = k.shape[0]
        dev = q.device
        rep, valid = self.memory.select(key, k[p.cand])
        rep_row, rep_scene = p.cand[rep], p.owner[rep]
        n = len(p.qlen)
        hh = torch.arange(H, device=dev)[:, None, None]
        foreign = valid[:, None, :] & (rep_scene[:, None, :] != p.scene[None, :, None]) & p.mem[None, :, None]
        idx = torch.cat([p.pad[None].expand(H, -1, -1), rep_row[:, None, :].expand(-1, n, -1)], -1) * H + hh
        keep = torch.cat([p.pmask[None].expand(H, -1, -1), foreign], -1).flatten()
        # the kept key rows, compacted in (head, piece, position) order without reading their count back: kidx is
        # sized for every representative kept (host-known bound); rows past the last segment are row 0, packed but
        # never read (each segment reads its cu_k range)
        Mr = rep.shape[1]
        bound = H * (p.sum_len + n * Mr)
        at = torch.where(keep, keep.cumsum(0) - 1, bound)
        kidx = torch.zeros(bound + 1, dtype=torch.int32, device=dev).scatter_(0, at, idx.flatten().to(torch.int32))
        kidx = kidx[:bound]
        qidx = (p.qrows[None] * H + hh[:, 0]).flatten().to(torch.int32)
        lq = p.qlen.repeat(H)
        lk = (p.lens[None] + foreign.sum(-1)).flatten()
        cu_q = F.pad(lq.cumsum(0), (1, 0)).to(torch.int32)
        cu_k = F.pad(lk.cumsum(0), (1, 0)).to(torch.int32)
        # single-head rows: row * H + head of the [rows, H, D] buffers
        qp = gather_rows(q.reshape(Sq * H, 1, D), qidx)
        kp, vp = gather_rows(k.reshape(L * H, 1, D), kidx, v.reshape(L * H, 1, D))
        # max_q / max_k as host bounds (the kernel checks only that a segment's keys span under 2 GiB)
        o = varlen(qp, kp, vp, cu_q, cu_k, p.max_qlen, p.max_len + Mr)
        out = q.new_zeros(Sq * H, 1, D)
        scatter_rows(o, qidx, out)
        return out.view(Sq, H, D)
