"""Bounded cross-scene memory with per-head representatives: the drop-in for src/onereel/memory.py (the same names,
fields and results), on HIP kernels.

Every scene reads its own context (its frames and sentence) plus, per head, at most M representative keys of the
other scenes, chosen among the boundary frames' keys (the first and last frame of every scene) by k-means over the
L2-normalised keys: 50 passes the first time a (layer, branch) key is seen, 2 warm passes from the stored centroids
after that, one medoid per non-empty cluster. Representatives differ per head, so the attention runs head-major: each
(head, query piece) pair is one single-head segment over rows of D elements, row = token * H + head.

Per call, all on the caller's stream and without host reads, when every piece's query rows are consecutive (the
frame plans of the models):

    or_memory_select   k-means + medoids for every head (fp32 MFMA distances, fixed-order sums, device-side stop)
    or_memory_foreign  each (piece, head)'s foreign representatives: source and packed rows, per-head key counts
    or_pack_layer      the local K / V rows of every piece past its in-place run (whole rows, all heads)
    or_pack_layer      the foreign K / V rows, one head each, into their head slots after the local rows
    or_varlen_fwd      multi-head attention over the pieces: queries read and outputs written in place, the leading
                       run of each piece's local keys and values (its scene's frames, whole 32-key blocks) read in
                       place from k and v, head h of piece i over its first k_len_head[i, h] keys (local, then its
                       own representatives)

Otherwise (query rows in any order) the single-head form runs: segment (head, piece) over rows of D elements, row =
token * H + head, with or_memory_index, or_pack_gather of single-head rows, gathered queries and a scatter.

A plan's static parts (segment offsets, the local key rows, the query rows) are built once per (plan, H) and kept.
A piece that does not read the memory and has the local rows of another (a scene's sentence queries beside its
video queries) reads them in place from that piece's rows, so they are packed once.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib as L
from .layout import SceneLayout
from .scene import gather_rows, pack_job, scatter_rows, varlen

ITERS_INIT, ITERS_UPDATE = 50, 2


def candidate_frames(layout: SceneLayout):
    """(frames, owner): each scene's first and last frame, a one-frame scene's frame once, and the scene of each"""
    frames, owner = [], []
    for j, (first, end) in enumerate(layout.ranges):
        ends = [first] if end - first == 1 else [first, end - 1]
        frames += ends
        owner += [j] * len(ends)
    return frames, owner


def candidates(layout: SceneLayout, T: int, device):
    """(rows, scene): the token rows (frame-major, T per frame) of the boundary frames and the scene of each row"""
    frames, owner = candidate_frames(layout)
    f = torch.tensor(frames, dtype=torch.long)
    rows = (f[:, None] * T + torch.arange(T)).flatten()
    scene = torch.tensor(owner, dtype=torch.long).repeat_interleave(T)
    return rows.to(device), scene.to(device)


class BoundaryMemory:
    """M representatives per head; `centroids` maps a (layer, CFG branch) key to that key's fp32 [H, M, D]
    centroids, carried from one denoising step to the next"""

    def __init__(self, M: int = 128):
        self.M = M
        self.centroids = {}
        self._init_cols = {}
        self._ws = {}

    def reset(self):
        self.centroids = {}

    def _start_columns(self, B: int, M: int, device):
        """the cold start's candidates: M evenly spaced over [0, B - 1], rounded half to even (torch.linspace)"""
        key = (B, M, str(device))
        if key not in self._init_cols:
            cols = torch.linspace(0, B - 1, M).round().to(torch.int32)
            self._init_cols[key] = cols.to(device)
        return self._init_cols[key]

    def _workspace(self, B, H, D, M, iters, device):
        n = int(L.lib().or_memory_select_workspace_size(B, H, D, M, iters))
        if n < 0:
            raise L.HipValueError(f'no k-means workspace for B={B} H={H} D={D} M={M}')
        ws = self._ws.get(str(device))
        if ws is None or ws.numel() < n:
            ws = torch.empty(n + 256, dtype=torch.uint8, device=device)
            self._ws[str(device)] = ws
        off = (-ws.data_ptr()) % 256
        return ws[off:off + n]

    @torch.no_grad()
    def select(self, key, kc: torch.Tensor):
        """kc [B, H, D] candidate keys (bf16 or fp32, on the GPU) -> (rep [H, M] int64 candidate positions,
        valid [H, M] bool): per head one representative per non-empty cluster, in cluster order, then padding
        (0, False)"""
        if kc.dim() != 3:
            raise L.HipValueError(f'kc must be [B, H, D], got {tuple(kc.shape)}')
        B, H, D = kc.shape
        kc = kc if kc.stride(2) == 1 and kc.stride(1) == D else kc.contiguous()
        return self._select(key, kc, None, B, H, D)

    def _select(self, key, keys: torch.Tensor, rows, B: int, H: int, D: int):
        """k-means over rows `rows` (int32 device tensor, or None for rows 0..B-1) of keys [rows, H, D]"""
        if not keys.is_cuda or keys.dtype not in (torch.bfloat16, torch.float32):
            raise L.HipTypeError(f'keys must be a bf16 or fp32 GPU tensor, got {keys.dtype} on {keys.device}')
        dev = keys.device
        M = min(self.M, B)
        c = self.centroids.get(key)
        cold = c is None or tuple(c.shape) != (H, M, D)
        if cold:
            c = torch.empty(H, M, D, dtype=torch.float32, device=dev)
            init = self._start_columns(B, M, dev)
        iters = ITERS_INIT if cold else ITERS_UPDATE
        rep = torch.empty(H, M, dtype=torch.long, device=dev)
        valid = torch.empty(H, M, dtype=torch.bool, device=dev)
        ws = self._workspace(B, H, D, M, iters, dev)
        with torch.cuda.device(dev):
            L.check(L.lib().or_memory_select(keys.data_ptr(), int(keys.dtype == torch.float32), L.ptr(rows),
                                             keys.stride(0), B, H, D, M, c.data_ptr(),
                                             init.data_ptr() if cold else None, iters, rep.data_ptr(),
                                             valid.data_ptr(), ws.data_ptr(), ws.numel(), L.stream_handle(dev)),
                    'or_memory_select')
        self.centroids[key] = c
        return rep, valid


@dataclass
class Plan:
    """one layer's query pieces (the fields of memory.py:96-106), plus host copies of the sizes that the varlen call
    needs (filled by make_plan; a Plan built field by field gets them from one read of lens / qlen)"""
    # field names as memory.py:102-111 (make_plan's result); n pieces, B boundary candidates
    qrows: torch.Tensor                  # [sum of qlen] the pieces' query rows, concatenated in piece order
    qlen: torch.Tensor                   # [n] how many query rows each piece has
    pad: torch.Tensor                    # [n, Lmax] each piece's own key rows, right-padded to the longest
    pmask: torch.Tensor                  # [n, Lmax] True where pad holds a real row
    lens: torch.Tensor                   # [n] how many own key rows each piece has
    scene: torch.Tensor                  # [n] the scene a piece belongs to
    mem: torch.Tensor                    # [n] whether a piece also attends to the other scenes' representatives
    cand: torch.Tensor                   # [B] key rows that may be chosen as representatives
    owner: torch.Tensor                  # [B] the scene each candidate row comes from
    host_qlen: list | None = None        # qlen on the host
    host_lens: list | None = None        # lens on the host
    q_first: list | None = None          # per piece its first query row when its rows are consecutive, else None


def make_plan(pieces, cand, owner, device) -> Plan:
    """pieces: [(scene, query rows, local key rows, reads the memory)]; pieces without queries are dropped. cand /
    owner: the key-buffer rows of the boundary candidates and their scene."""
    as_long = lambda x: torch.as_tensor(x, dtype=torch.long)
    kept = [(j, as_long(q), as_long(k), bool(m)) for j, q, k, m in pieces if len(q)]
    if not kept:
        raise L.HipValueError('a plan needs at least one piece with queries')
    n = len(kept)
    lens = [int(k.numel()) for _, _, k, _ in kept]
    width = max(lens)
    pad = torch.zeros(n, width, dtype=torch.long)
    pmask = torch.zeros(n, width, dtype=torch.bool)
    for i, (_, _, k, _) in enumerate(kept):
        pad[i, :lens[i]] = k
        pmask[i, :lens[i]] = True

    def first_row(q):
        return int(q[0]) if bool((q == q[0] + torch.arange(q.numel())).all()) else None

    put = lambda x: x.to(device)
    return Plan(qrows=put(torch.cat([q for _, q, _, _ in kept])), qlen=put(as_long([q.numel() for _, q, _, _ in kept])),
                pad=put(pad), pmask=put(pmask), lens=put(as_long(lens)), scene=put(as_long([j for j, *_ in kept])),
                mem=put(torch.tensor([m for *_, m in kept], dtype=torch.bool)), cand=put(as_long(cand)),
                owner=put(as_long(owner)), host_qlen=[int(q.numel()) for _, q, _, _ in kept], host_lens=lens,
                q_first=[first_row(q) for _, q, _, _ in kept])


def frame_plan(layout: SceneLayout, T: int, token_row, Lv: int, q_pieces, text_ranges=None, text_for=(), Sq: int = 0,
               device='cuda') -> Plan:
    """the pieces of a frame-major model (memory.py:124-137). Key buffer: Lv video rows (video token t at row
    token_row[t]), then the text tokens; query buffer: Sq video rows, then the text tokens. q_pieces: [(scene, first
    video query row, end)]. Video queries read their scene's frames, their sentence and the memory; the sentence
    queries of the scenes in text_for read their scene's frames and their sentence."""
    token_row = torch.as_tensor(token_row)

    def video_rows(frames):
        tok = (torch.as_tensor(frames, dtype=torch.long)[:, None] * T + torch.arange(T)).flatten()
        return token_row[tok]

    def sentence(j):
        if not text_ranges:
            return torch.zeros(0, dtype=torch.long)
        a, b = text_ranges[j]
        return Lv + torch.arange(a, b)

    own = {j: torch.cat([video_rows(layout.frames[j]), sentence(j)]) for j in range(layout.n_scenes)}
    pieces = [(j, torch.arange(lo, hi), own[j], True) for j, lo, hi in q_pieces]
    for j in sorted(text_for):
        a, b = text_ranges[j]
        pieces.append((j, Sq + torch.arange(a, b), own[j], False))
    frames, owner = candidate_frames(layout)
    return make_plan(pieces, video_rows(frames), torch.tensor(owner).repeat_interleave(T), device)


class _Static:
    """the per-(plan, H) device tables of the head-major call: segment (head h, piece i) is number h * n + i"""

    def __init__(self, p: Plan, H: int, Sq: int, device):
        qlen = p.host_qlen if p.host_qlen is not None else [int(x) for x in p.qlen.tolist()]
        lens = p.host_lens if p.host_lens is not None else [int(x) for x in p.lens.tolist()]
        n, B = len(qlen), int(p.cand.numel())
        self.n, self.B, self.H, self.qlen, self.lens = n, B, H, qlen, lens
        self.max_q = max(qlen)
        first = p.q_first if p.q_first is not None else [None] * n
        # queries in place: every piece's rows consecutive, inside [0, Sq), and no two pieces sharing a row
        spans = sorted((f, f + c) for f, c in zip(first, qlen) if f is not None)
        self.in_place = (all(f is not None for f in first) and spans[0][0] >= 0 and spans[-1][1] <= Sq and
                         all(a[1] <= b[0] for a, b in zip(spans, spans[1:])))
        self.covers_all = self.in_place and sum(qlen) == Sq
        t32 = lambda x: torch.tensor(x, dtype=torch.int32, device=device)
        cu = [0]
        for _ in range(H):
            for c in qlen:
                cu.append(cu[-1] + c)
        self.cu_q, self.sum_q = t32(cu), cu[-1]
        if self.in_place:
            self.seg_q_src = t32([first[i] * H + h for h in range(H) for i in range(n)])
            self.first_q = t32(first)
            self.cu_piece = t32([0] + [sum(qlen[:i + 1]) for i in range(n)])
        else:
            rows = p.qrows.to(device=device, dtype=torch.int64)
            lo, hi = int(rows.min()), int(rows.max())        # once per plan
            if lo < 0 or hi >= Sq:
                raise L.HipValueError(f'plan query rows span [{lo}, {hi}], the query buffer has {Sq} rows')
            self.qidx = (rows[None] * H + torch.arange(H, device=device)[:, None]).flatten().to(torch.int32)
        local = p.pad.to(device)[p.pmask.to(device)]           # the local key rows, piece after piece
        # the key-buffer rows the plan names (once per plan): none negative, the largest checked against each call's
        # buffer (the kernels dereference them unchecked)
        lo = min(int(local.min()) if local.numel() else 0, int(p.cand.min()) if p.cand.numel() else 0)
        if lo < 0:
            raise L.HipValueError(f'plan key rows include {lo}: rows must be >= 0')
        self.max_key_row = max(int(local.max()) if local.numel() else -1, int(p.cand.max()))
        self.local = local.to(torch.int64)
        # a piece that does not read the memory and has the same local rows as another piece (a scene's sentence
        # queries beside its video queries) reads that piece's local rows in place: its keys are their slot's first
        # rows, and it packs none of its own (compared once per plan)
        mem = [bool(x) for x in p.mem.tolist()]
        scene = [int(x) for x in p.scene.tolist()]
        starts = [0]
        for c in lens:
            starts.append(starts[-1] + c)
        part = lambda i: self.local[starts[i]:starts[i + 1]]
        self.share = [None] * n
        for i in range(n):
            if mem[i]:
                continue
            # candidates: pieces of the same scene with as many local rows, those reading the memory first
            for o in sorted((o for o in range(n) if scene[o] == scene[i] and lens[o] == lens[i] and o != i),
                            key=lambda o: (not mem[o], o)):
                if self.share[o] is None and (mem[o] or o < i) and torch.equal(part(o), part(i)):
                    self.share[i] = o
                    break
        self.mem = mem
        self.cand64 = p.cand.to(device=device, dtype=torch.int64).contiguous()
        self.cand32 = self.cand64.to(torch.int32)
        self.owner64 = p.owner.to(device=device, dtype=torch.int64).contiguous()
        self.scene64 = p.scene.to(device=device, dtype=torch.int64).contiguous()
        self.piece_len = t32(lens)
        self.piece_mem = p.mem.to(device=device, dtype=torch.uint8).contiguous()
        self._slots = {}
        self.device = device

    def multi_head(self, M: int):
        """the multi-head form's per-M tables: per piece its packed row offset (k_off), largest key count (k_len),
        in-place run (lead: whole 32-key blocks of keys and values from token row v_row); the pack job of the local
        rows past the run (src, dst), and the packed row count. A piece that shares another's local rows gets that
        piece's offset and run."""
        key = ('mh', M)
        if key not in self._slots:
            n, lens = self.n, self.lens
            starts = [0]
            for c in lens:
                starts.append(starts[-1] + c)
            local = self.local.cpu()
            off, o = [0] * n, 0
            for i in range(n):
                if self.share[i] is None:
                    off[i] = o
                    o += lens[i] + (M if self.mem[i] else 0)
            for i in range(n):
                if self.share[i] is not None:
                    off[i] = off[self.share[i]]
            v_row, v_lead = [0] * n, [0] * n
            src, dst = [], []
            for i in range(n):
                rows = local[starts[i]:starts[i + 1]]
                run = 0
                if len(rows):
                    step = (rows - rows[0]) == torch.arange(len(rows))
                    run = len(rows) if bool(step.all()) else int((~step).nonzero()[0])
                    v_row[i] = int(rows[0])
                v_lead[i] = run // L.KEY_BLOCK * L.KEY_BLOCK
                if self.share[i] is None:
                    src += rows[v_lead[i]:].tolist()
                    dst += range(off[i] + v_lead[i], off[i] + lens[i])
            t32 = lambda x: torch.tensor(x, dtype=torch.int32, device=self.device)
            k_len = [lens[i] + (M if self.mem[i] else 0) for i in range(n)]
            self._slots[key] = dict(k_off=t32(off), k_len=t32(k_len), max_k=max(k_len), v_row=t32(v_row),
                                    lead=t32(v_lead), src=t32(src), dst=t32(dst), rows=o)
        return self._slots[key]

    def slots(self, M: int):
        """(k_off, kidx) for M representatives: segment (h, i) owns kidx[k_off .. k_off + lens[i] + M) (+ 0 when
        the piece does not read the memory), its local rows (row * H + h) first, written once here; the foreign rows
        after them are rewritten by each call. A piece that shares another's local rows gets that piece's k_off."""
        if M not in self._slots:
            H, n = self.H, self.n
            off, o = [0] * (H * n), 0
            for h in range(H):
                for i in range(n):
                    if self.share[i] is None:
                        off[h * n + i] = o
                        o += self.lens[i] + (M if self.mem[i] else 0)
                for i in range(n):
                    if self.share[i] is not None:
                        off[h * n + i] = off[h * n + self.share[i]]
            k_off = torch.tensor(off, dtype=torch.int32, device=self.device)
            kidx = torch.zeros(o, dtype=torch.int32, device=self.device)
            own = [i for i in range(n) if self.share[i] is None]
            pos = torch.cat([torch.arange(self.lens[i]) for i in own]).to(self.device)
            piece = torch.cat([torch.full((self.lens[i],), i) for i in own]).to(self.device)
            rows = torch.cat([self.local[sum(self.lens[:i]):sum(self.lens[:i + 1])] for i in own])
            for h in range(H):
                kidx[k_off[h * n + piece].long() + pos] = (rows * H + h).to(torch.int32)
            self._slots[M] = (k_off, kidx)
        return self._slots[M]


class MemoryAttention:
    """packed head-major attention with the bounded memory (memory.py:140-174); plans are cached by the caller"""

    def __init__(self, memory: BoundaryMemory, head_major: bool = False):
        self.memory = memory
        self.plans = {}
        self._static = {}
        self.head_major = head_major   # True: the single-head form even when the queries can be read in place

    def _tables(self, p: Plan, H: int, Sq: int, device) -> _Static:
        key = (id(p), H, Sq, str(device))
        hit = self._static.get(key)
        if hit is None or hit[0] is not p:
            hit = (p, _Static(p, H, Sq, device))
            self._static[key] = hit
        return hit[1]

    def __call__(self, key, q, k, v, p: Plan) -> torch.Tensor:
        """q [Sq, H, D], k / v [L, H, D] bf16 on the GPU -> [Sq, H, D] (rows outside the plan's queries are zero)"""
        Sq, H, D = q.shape
        Lk = k.shape[0]
        if k.shape[1:] != (H, D) or v.shape != k.shape:
            raise L.HipValueError(f'k / v must be [rows, {H}, {D}] alike')
        for x in (q, k, v):
            if x.stride(2) != 1 or x.stride(1) != D or x.stride(0) != H * D:
                raise L.HipValueError('q, k and v must be contiguous [rows, H, D]')
        dev = q.device
        st = self._tables(p, H, Sq, dev)
        if st.n * H > 4096:
            raise L.HipValueError(f'{st.n} pieces x {H} heads = {st.n * H} single-head segments; the varlen call '
                                  f'takes at most 4096')
        if st.max_key_row >= Lk:
            raise L.HipValueError(f'the plan reads key row {st.max_key_row}, the key buffer has {Lk} rows')
        rep, valid = self.memory._select(key, k, st.cand32, st.B, H, D)
        M = rep.shape[1]
        if st.in_place and not self.head_major:
            return self._multi_head(st, q, k, v, rep, valid, M)
        k_off, kidx = st.slots(M)
        k_len = torch.empty(st.n * H, dtype=torch.int32, device=dev)
        L.check(L.lib().or_memory_index(rep.data_ptr(), valid.data_ptr(), st.cand64.data_ptr(), st.owner64.data_ptr(),
                                        st.scene64.data_ptr(), st.piece_mem.data_ptr(), st.piece_len.data_ptr(),
                                        k_off.data_ptr(), st.n, H, M, kidx.data_ptr(), k_len.data_ptr(),
                                        L.stream_handle(dev)), 'or_memory_index')
        # single-head rows: row * H + head of the [rows, H, D] buffers
        kp, vp = gather_rows(k.view(Lk * H, 1, D), kidx, v.view(Lk * H, 1, D), check=False)  # rows checked per plan
        max_k = max(st.lens) + M
        if st.in_place:
            out = torch.empty_like(q) if st.covers_all else torch.zeros_like(q)
            qv, ov = q.view(Sq * H, 1, D), out.view(Sq * H, 1, D)
            varlen(qv, kp, vp, st.cu_q, None, st.max_q, max_k, k_off=k_off, k_len=k_len, out=ov,
                   seg_q_src=st.seg_q_src, n_q_video=Sq * H, sum_q=st.sum_q, q_row_step=H)
            return out
        qp = gather_rows(q.view(Sq * H, 1, D), st.qidx, check=False)
        o = varlen(qp, kp, vp, st.cu_q, None, st.max_q, max_k, k_off=k_off, k_len=k_len)
        out = torch.zeros_like(q)
        scatter_rows(o, st.qidx, out.view(Sq * H, 1, D), check=False)
        return out

    def _multi_head(self, st: _Static, q, k, v, rep, valid, M: int) -> torch.Tensor:
        """every piece one multi-head segment: its local keys (the leading run of token rows, whole key blocks of it,
        read in place from k / v, the rest packed as whole rows) then, per head, that head's representatives of the
        other scenes in its own head slot"""
        Sq, H, D = q.shape
        Lk = k.shape[0]
        dev = q.device
        n, mh = st.n, st.multi_head(M)
        fsrc = torch.empty(n * H * M, dtype=torch.int32, device=dev)
        fdst = torch.empty_like(fsrc)
        k_len_head = torch.empty(n * H, dtype=torch.int32, device=dev)
        L.check(L.lib().or_memory_foreign(rep.data_ptr(), valid.data_ptr(), st.cand64.data_ptr(),
                                          st.owner64.data_ptr(), st.scene64.data_ptr(), st.piece_mem.data_ptr(),
                                          st.piece_len.data_ptr(), mh['k_off'].data_ptr(), n, H, M, fsrc.data_ptr(),
                                          fdst.data_ptr(), k_len_head.data_ptr(), L.stream_handle(dev)),
                'or_memory_foreign')
        R = mh['rows']
        kp = torch.empty(R, H, D, dtype=k.dtype, device=dev)
        vp = torch.empty_like(kp)
        # local rows past the in-place run (checked once per plan), then the representatives (rows of the checked
        # candidates), one head each
        if mh['src'].numel():
            pack_job(k, v, mh['src'], mh['dst'], kp, vp)
        pack_job(k.view(Lk * H, 1, D), v.view(Lk * H, 1, D), fsrc, fdst, kp.view(R * H, 1, D), vp.view(R * H, 1, D))
        out = torch.empty_like(q) if st.covers_all else torch.zeros_like(q)
        varlen(q, kp, vp, st.cu_piece, None, st.max_q, mh['max_k'], k_off=mh['k_off'], k_len=mh['k_len'], out=out,
               seg_q_src=st.first_q, n_q_video=Sq, sum_q=sum(st.qlen), v_tok=v, v_lead=mh['lead'],
               v_row=mh['v_row'], k_tok=k, k_lead=mh['lead'], k_len_head=k_len_head)
        return out
