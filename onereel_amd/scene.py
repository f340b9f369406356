"""The scene-attention layer engine: device layout, K/V pack-gather, varlen attention and write-back.

One layer of `Processor.scene` on one GPU (src/onereel/models/hunyuan15.py:212-251) runs here as at most five
launches on the caller's current stream, with no host synchronisation:

    ScopePlan.build      or_layout_build   cu_seqlens, gather rows, RoPE rows (cached per layout and step mode)
    pack_layer           or_pack_layer     K rows of every scope (rotated on the way), the V rows the attention call
                                           does not read in place, and the video queries rotated once in token
                                           order, one pass
    attention            or_varlen_fwd     Q read in place, the own-frame values read in place, output written in place
    zero text padding    or_scatter        ot rows past the valid text (ot = eq.new_zeros in the reference)

`mode` says what q / k hold: 'raw' (before RoPE: the fused path, the table row of every query and key comes from
the layout), 'rotated' (already rotated, as the reference's `scene` receives them: shared keys are re-rotated by
_move_shared's two rotations when the shared frames are moved), or 'none' (no RoPE at all).
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib as L
from .layout import SceneLayout

MODES = ('raw', 'rotated', 'none')


def _desc(lay: SceneLayout, T: int, counts, text_rows: int, scene_rope: bool, rope_lengths, adjacent: bool,
          with_text: bool, text_keys_in_place: bool = False, q_range=None) -> L.LayoutDesc:
    d = L.LayoutDesc()
    n = lay.n_scenes
    if n > L.OR_MAX_SCENES:
        raise L.HipValueError(f'{n} scenes exceed the maximum {L.OR_MAX_SCENES}')
    d.n_scenes, d.T, d.halo = n, int(T), int(lay.halo)
    d.sides = ('adj', 'prev', 'next').index(lay.sides)
    d.with_text, d.scene_rope, d.adjacent = int(with_text), int(scene_rope), int(adjacent)
    d.text_rows = int(text_rows)
    d.text_keys_in_place = int(bool(text_keys_in_place) and bool(with_text))
    if q_range is not None:
        d.q_lo, d.q_hi = int(q_range[0]), int(q_range[1])
    for j, x in enumerate(lay.lengths):
        d.lengths[j] = int(x)
    counts = list(counts) if with_text else [0] * n
    if len(counts) != n:
        raise L.HipValueError(f'{len(counts)} sentence counts for {n} scenes')
    for j, c in enumerate(counts):
        d.counts[j] = int(c)
    rl = list(rope_lengths) if rope_lengths else []
    if len(rl) > L.OR_MAX_SCENES:
        raise L.HipValueError('too many rope_lengths')
    d.n_rope_lengths = len(rl)
    for s, x in enumerate(rl):
        d.rope_lengths[s] = int(x)
    e = 0
    d.extra_ptr[0] = 0
    for j in range(n):
        fr = list(lay.extra.get(j, ()))
        if e + len(fr) > L.OR_MAX_EXTRA:
            raise L.HipValueError(f'more than {L.OR_MAX_EXTRA} extra frames')
        for f in fr:
            d.extra[e] = int(f)
            e += 1
        d.extra_ptr[j + 1] = e
    return d


class ScopePlan:
    """The packed layout of one request's scopes, built on the device by `or_layout_build`.

    Attributes (int32 device tensors): cu_q, cu_k [n_seg+1], seg_q_src, k_off, k_len, v_lead, v_row [n_seg], q_src /
    q_rope [sum_q], k_src / k_rope / v_src [sum_k], and for mode 'rotated' with moved shared frames k_move_a /
    k_move_b [sum_k]. v_lead / v_row / v_src: every segment's first keys are its scene's own frames, consecutive token
    rows; the attention call reads the values of v_lead of them (whole key blocks) in place from token row v_row on,
    and the pack copies only the values of the other keys (v_src[r] = -1 for the rows read in place). With
    value_runs, v_runs [n_seg * VALUE_RUNS * 3] lists each video segment's first shared frames (key offset, count,
    token row), whose whole key blocks are read in place too (head_dim 128), and v_src is -1 for them as well.
    Host ints: n_seg, sum_q, sum_k, max_q, max_k, n_video, text_rows, max_rope_row.

    text_keys_in_place: each scene's video segment packs its keys as own frames, sentence, shared frames, and the
    text segment (whose keys are the same own-frame and sentence rows) reads the first of them in place (k_off,
    k_len) instead of packing its own copy; the default packs every segment in the reference's order.

    q_range=(a, b): one rank's share of the layer when the video tokens are split over several ranks
    (hunyuan15.py:219-224): the video queries in tokens [a, b) (each scene's clipped to the range, with the scene's
    full keys) and the sentences of the scenes whose first token lies in the range; the other segments are empty.
    Query and key rows stay global token rows."""

    def __init__(self, lay: SceneLayout, T: int, counts=None, text_rows: int | None = None, scene_rope=False,
                 rope_lengths=None, adjacent=False, with_text=True, device=None, moves=False,
                 text_keys_in_place=False, q_range=None, value_runs=True):
        counts = list(counts) if counts is not None else [0] * lay.n_scenes
        if text_rows is None:
            text_rows = sum(counts) if with_text else 0
        self.layout, self.T, self.counts, self.text_rows = lay, int(T), counts, int(text_rows)
        self.scene_rope, self.adjacent, self.with_text = bool(scene_rope), bool(adjacent), bool(with_text)
        self.text_keys_in_place = bool(text_keys_in_place) and self.with_text
        self.q_range = None if q_range is None else (int(q_range[0]), int(q_range[1]))
        self.desc = _desc(lay, T, counts, text_rows, scene_rope, rope_lengths, adjacent, with_text,
                          self.text_keys_in_place, self.q_range)
        sz = L.LayoutSizes()
        L.check(L.lib().or_layout_plan(ctypes.byref(self.desc), ctypes.byref(sz)), 'or_layout_plan')
        self.n_seg, self.sum_q, self.sum_k = sz.n_seg, sz.sum_q, sz.sum_k
        self.max_q, self.max_k, self.n_video, self.max_rope_row = sz.max_q, sz.max_k, sz.n_video, sz.max_rope_row
        dev = torch.device(device) if device is not None else torch.device('cuda', torch.cuda.current_device())
        new = lambda n: torch.empty(int(n), dtype=torch.int32, device=dev)
        self.cu_q, self.cu_k, self.seg_q_src = new(self.n_seg + 1), new(self.n_seg + 1), new(self.n_seg)
        self.k_off, self.k_len = new(self.n_seg), new(self.n_seg)
        self.v_lead, self.v_row, self.v_src = new(self.n_seg), new(self.n_seg), new(self.sum_k)
        self.v_runs = new(self.n_seg * L.VALUE_RUNS * 3) if value_runs else None
        self.q_src, self.q_rope = new(self.sum_q), new(self.sum_q)
        self.k_src, self.k_rope = new(self.sum_k), new(self.sum_k)
        self.k_move_a = new(self.sum_k) if moves and adjacent else None
        self.k_move_b = new(self.sum_k) if moves and adjacent else None
        self.device = dev
        self._ws = {}
        self.build()

    def build(self):
        """(re)run the layout kernel on the current stream"""
        out = L.LayoutOut(*(L.ptr(t) for t in (self.cu_q, self.cu_k, self.seg_q_src, self.q_src, self.q_rope,
                                                self.k_src, self.k_rope, self.k_move_a, self.k_move_b, self.k_off,
                                                self.k_len, self.v_lead, self.v_row, self.v_src, self.v_runs)))
        with torch.cuda.device(self.device):
            L.check(L.lib().or_layout_build(ctypes.byref(self.desc), ctypes.byref(out), L.stream_handle()),
                    'or_layout_build')
        return self

    def workspace(self, H: int, D: int) -> torch.Tensor:
        """the attention workspace of this plan's calls with H heads of D dims (its size depends on both), kept"""
        key = (int(H), int(D))
        if key not in self._ws:
            n = L.lib().or_varlen_workspace_size(int(self.n_seg), int(self.sum_q), int(H), int(D))
            self._ws[key] = torch.empty(int(n), dtype=torch.uint8, device=self.device)
        return self._ws[key]

    def index_bytes(self) -> int:
        """bytes the layout kernel writes"""
        n = 2 * (self.n_seg + 1) + 5 * self.n_seg + 2 * self.sum_q + 3 * self.sum_k
        if self.v_runs is not None:
            n += self.v_runs.numel()
        if self.k_move_a is not None:
            n += 2 * self.sum_k
        return 4 * n


def _rows2d(x: torch.Tensor, H: int, D: int):
    """(tensor, row stride) of a [rows, H, D] view whose (H, D) part is contiguous"""
    if x.dim() != 3 or x.shape[1] != H or x.shape[2] != D:
        raise L.HipValueError(f'expected [rows, {H}, {D}], got {tuple(x.shape)}')
    if x.stride(2) != 1 or x.stride(1) != D:
        raise L.HipValueError('heads and head dims must be contiguous')
    return x, x.stride(0)


def _with_row_stride(x: torch.Tensor, stride: int) -> torch.Tensor:
    """x [rows, H, D] itself when its rows are `stride` elements apart, else a copy of its rows laid out that way (the
    attention call reads video and text query rows with one row stride)"""
    if x.stride(0) == stride:
        return x
    rows, H, D = x.shape
    buf = torch.empty(rows, stride, dtype=x.dtype, device=x.device)[:, :H * D].view(rows, H, D)
    buf.copy_(x)
    return buf


def _check_bf16(*xs):
    for x in xs:
        if x is not None and (x.dtype != torch.bfloat16 or not x.is_cuda):
            raise L.HipTypeError(f'expected a bf16 GPU tensor, got {x.dtype} on {x.device}')


def _tables(cos, sin, D):
    if cos is None:
        return None, None, 0
    if cos.dim() != 2 or cos.shape[1] != D or sin.shape != cos.shape:
        raise L.HipValueError(f'rotary tables must be [rows, {D}]')
    cos = cos.to(torch.float32).contiguous()
    sin = sin.to(torch.float32).contiguous()
    return cos, sin, cos.shape[0]


def pack_rows(plan: ScopePlan, video: torch.Tensor, text: torch.Tensor | None, which: str, out=None,
              b_video=None, b_text=None, b_out=None, cos=None, sin=None, mode='none'):
    """Gather the packed rows of the plan's queries (which='q') or keys (which='k') from [video ; text]; with b_*,
    the value rows of the same keys in the same pass. Keys / queries are rotated per `mode`."""
    H, D = video.shape[1], video.shape[2]
    _check_bf16(video, text, b_video, b_text)
    _, vs = _rows2d(video, H, D)
    ts = _rows2d(text, H, D)[1] if text is not None and text.shape[0] else vs
    if b_video is not None:
        if _rows2d(b_video, H, D)[1] != vs or (b_text is not None and b_text.shape[0] and b_text.stride(0) != ts):
            raise L.HipValueError('value rows must have the strides of the key rows')
    n = plan.sum_q if which == 'q' else plan.sum_k
    src = plan.q_src if which == 'q' else plan.k_src
    rope = move = None
    if mode == 'raw':
        rope = plan.q_rope if which == 'q' else plan.k_rope
    elif mode == 'rotated' and which == 'k' and plan.adjacent:
        if plan.k_move_a is None:
            raise L.HipValueError('plan was built without move rows (moves=True)')
        rope, move = plan.k_move_b, plan.k_move_a
    elif mode not in MODES:
        raise L.HipValueError(mode)
    cos, sin, n_rows = _tables(cos, sin, D) if rope is not None else (None, None, 0)
    if rope is not None and cos is None:
        raise L.HipValueError('RoPE needs the (cos, sin) tables')
    if rope is not None and plan.max_rope_row >= n_rows:
        raise L.HipValueError(f'layout needs rotary row {plan.max_rope_row} but the table has {n_rows} rows')
    out = out if out is not None else torch.empty(n, H, D, dtype=video.dtype, device=video.device)
    if b_video is not None and b_out is None:
        b_out = torch.empty(n, H, D, dtype=video.dtype, device=video.device)
    L.check(L.lib().or_pack_gather(video.data_ptr(), L.ptr(text if text is not None and text.shape[0] else None),
                                   L.ptr(b_video), L.ptr(b_text if b_text is not None and b_text.shape[0] else None),
                                   vs, ts, plan.n_video, src.data_ptr(), L.ptr(rope), L.ptr(move),
                                   L.ptr(cos), L.ptr(sin), n_rows, n, H, D, out.data_ptr(), L.ptr(b_out),
                                   L.stream_handle(video.device)), 'or_pack_gather')
    return (out, b_out) if b_video is not None else out


def n_seg_of(cu_q: torch.Tensor) -> int:
    return cu_q.numel() - 1


def pack_job(k, v, src, dst, k_out, v_out, v_src=None):
    """one or_pack_layer launch without RoPE: packed row dst[r] of k_out / v_out = row src[r] of k / v (nothing for
    src[r] < 0; values from row v_src[r] when given, none where it is < 0). k, v, k_out, v_out: [rows, H, D] bf16 with
    contiguous rows; the index arrays are int32 GPU tensors whose rows the caller has checked."""
    H, D = k.shape[1], k.shape[2]
    _check_bf16(k, v, k_out, v_out)
    for t in (k, v, k_out, v_out):
        if not t.is_contiguous():
            raise L.HipValueError('pack_job takes contiguous [rows, H, D] tensors')
    for t in (src, dst, v_src):
        if t is not None and (t.dtype != torch.int32 or not t.is_cuda or not t.is_contiguous() or
                              t.numel() != src.numel()):
            raise L.HipTypeError('src / dst / v_src must be contiguous int32 GPU tensors of one length')
    a = L.PackArgs()
    a.k_video, a.v_video, a.video_row_stride, a.text_row_stride, a.n_video = k.data_ptr(), v.data_ptr(), H * D, \
        H * D, k.shape[0]
    a.k_src, a.v_src, a.k_dst, a.n_keys = src.data_ptr(), L.ptr(v_src), dst.data_ptr(), src.numel()
    a.k_out, a.v_out, a.H, a.D = k_out.data_ptr(), v_out.data_ptr(), H, D
    L.check(L.lib().or_pack_layer(ctypes.byref(a), L.stream_handle(k.device)), 'or_pack_layer')


def _check_row_range(idx: torch.Tensor, n: int, what: str):
    """every entry of the int32 device tensor idx in [0, n): the kernels dereference them unchecked, so a row out of
    range is an error here, before any launch (one device reduction and one host read)"""
    if idx.numel() == 0:
        return
    lo, hi = (int(x) for x in torch.aminmax(idx))
    if lo < 0 or hi >= n:
        raise L.HipValueError(f'{what}: rows span [{lo}, {hi}], outside [0, {n})')


def gather_rows(src: torch.Tensor, idx: torch.Tensor, b_src: torch.Tensor | None = None, check: bool = True):
    """rows idx of src [N, H, D] (and of b_src, same shape and stride) packed into new [len(idx), H, D] tensors in
    one pass of or_pack_gather; idx: int32 GPU tensor of rows in [0, N), checked on the host unless check=False (for
    callers whose indices are validated once per plan)"""
    N, H, D = src.shape
    _check_bf16(src, b_src)
    _, ss = _rows2d(src, H, D)
    if b_src is not None and (b_src.shape != src.shape or _rows2d(b_src, H, D)[1] != ss):
        raise L.HipValueError('b_src must have the shape and row stride of src')
    if idx.dtype != torch.int32 or not idx.is_cuda or not idx.is_contiguous():
        raise L.HipTypeError('idx must be a contiguous int32 GPU tensor')
    if check:
        _check_row_range(idx, N, 'gather_rows')
    n = idx.numel()
    out = torch.empty(n, H, D, dtype=src.dtype, device=src.device)
    b_out = torch.empty_like(out) if b_src is not None else None
    L.check(L.lib().or_pack_gather(src.data_ptr(), None, L.ptr(b_src), None, ss, ss, N, idx.data_ptr(), None, None,
                                   None, None, 0, n, H, D, out.data_ptr(), L.ptr(b_out),
                                   L.stream_handle(src.device)), 'or_pack_gather')
    return (out, b_out) if b_src is not None else out


def scatter_rows(packed: torch.Tensor, idx: torch.Tensor, out: torch.Tensor, check: bool = True):
    """out[idx[r]] = packed[r] for out [N, H, D] (rows not named keep their contents), one pass of or_scatter; idx
    in [0, N), checked on the host unless check=False"""
    n, H, D = packed.shape
    _check_bf16(packed, out)
    _, os_ = _rows2d(out, H, D)
    if idx.dtype != torch.int32 or not idx.is_cuda or not idx.is_contiguous() or idx.numel() != n:
        raise L.HipTypeError('idx must be a contiguous int32 GPU tensor with one entry per packed row')
    if check:
        _check_row_range(idx, out.shape[0], 'scatter_rows')
    L.check(L.lib().or_scatter(packed.data_ptr(), idx.data_ptr(), n, out.shape[0], out.data_ptr(), None, os_, os_, 0,
                               0, H, D, L.stream_handle(out.device)), 'or_scatter')
    return out


def varlen(q, k, v, cu_q, cu_k, max_q, max_k, *, k_off=None, k_len=None, out=None, lse=None, seg_q_src=None,
           q_text=None, o_text=None, n_q_video=None, q_rope=None, cos=None, sin=None, sum_q=None, workspace=None,
           scale=None, noalloc=False, q_row_step=1, v_tok=None, v_lead=None, v_row=None, k_len_head=None,
           k_tok=None, k_lead=None, v_runs=None):
    """or_varlen_fwd on torch tensors. Returns out (allocated [Nq, H, D] when not given). noalloc=True calls
    or_varlen_fwd_noalloc instead: no workspace, the library's fixed per-GPU array (calls must not overlap on a GPU).
    q_row_step > 1 (with seg_q_src): query i of segment s is row seg_q_src[s] + i * q_row_step of q and of out.
    v_tok (with v_lead, v_row): the values of segment s's first v_lead[s] keys are rows v_row[s].. of v_tok (row stride
    of k), the others rows k_off[s] + v_lead[s].. of v; k_tok with k_lead (and v_row) likewise for the keys.
    v_runs [n_seg * VALUE_RUNS * 3] (with v_tok, head_dim 128): further runs of each segment's values in v_tok, entry
    (key offset, key count, token row), whose whole key blocks are read in place.
    k_len_head [n_seg * H] (with k_len): head h of segment s attends to its first k_len_head[s * H + h] keys."""
    H, D = k.shape[1], k.shape[2]
    _check_bf16(q, k, v, q_text, out, o_text)
    _, qs = _rows2d(q, H, D)
    _, ks = _rows2d(k, H, D)
    if _rows2d(v, H, D)[1] != ks:
        raise L.HipValueError('k and v must have the same row stride')
    if q_text is not None and q_text.shape[0] and q_text.stride(0) != qs:
        raise L.HipValueError('q and q_text must have the same row stride')
    n_seg = (cu_q.numel() - 1)
    if k_len_head is not None and (k_len is None or k_len_head.numel() != n_seg_of(cu_q) * H):
        raise L.HipValueError('k_len_head needs k_len and one entry per segment and head')
    for t in (cu_q, cu_k, k_off, k_len, seg_q_src, q_rope, v_lead, v_row, k_len_head, k_lead, v_runs):
        if t is not None and (t.dtype != torch.int32 or not t.is_cuda or not t.is_contiguous()):
            raise L.HipTypeError('index arrays must be contiguous int32 GPU tensors')
    if v_tok is not None:
        _check_bf16(v_tok)
        if v_lead is None or v_row is None:
            raise L.HipValueError('v_tok needs v_lead and v_row')
        if _rows2d(v_tok, H, D)[1] != ks:
            raise L.HipValueError('v_tok must have the row stride of k and v')
    if v_runs is not None:
        if v_tok is None or D != 128 or k_len_head is not None:
            raise L.HipValueError('v_runs needs v_tok and head_dim 128 (and no k_len_head)')
        if v_runs.numel() != n_seg_of(cu_q) * L.VALUE_RUNS * 3:
            raise L.HipValueError(f'v_runs needs {L.VALUE_RUNS} (offset, count, row) entries per segment')
    if k_tok is not None:
        _check_bf16(k_tok)
        if k_lead is None or v_row is None:
            raise L.HipValueError('k_tok needs k_lead and v_row')
        if _rows2d(k_tok, H, D)[1] != ks:
            raise L.HipValueError('k_tok must have the row stride of k and v')
    if sum_q is None:
        sum_q = q.shape[0] if seg_q_src is None else None
        if sum_q is None:
            raise L.HipValueError('sum_q is required with seg_q_src')
    if out is None:
        out = torch.empty(q.shape[0], H, D, dtype=torch.bfloat16, device=q.device)
    _, os_ = _rows2d(out, H, D)
    if o_text is not None and o_text.shape[0] and o_text.stride(0) != os_:
        raise L.HipValueError('o and o_text must have the same row stride')
    cos, sin, n_rope_rows = _tables(cos, sin, D) if q_rope is not None else (None, None, 0)
    if workspace is None and not noalloc:
        nb = L.lib().or_varlen_workspace_size(int(n_seg), int(sum_q), int(H), int(D))
        workspace = torch.empty(int(nb), dtype=torch.uint8, device=q.device)
    a = L.VarlenArgs()
    a.q, a.q_text, a.k, a.v = q.data_ptr(), L.ptr(q_text if q_text is not None and q_text.shape[0] else None), \
        k.data_ptr(), v.data_ptr()
    a.o, a.o_text, a.lse = out.data_ptr(), L.ptr(o_text if o_text is not None and o_text.shape[0] else None), \
        L.ptr(lse)
    a.cu_q, a.cu_k, a.k_off, a.k_len = L.ptr(cu_q), L.ptr(cu_k), L.ptr(k_off), L.ptr(k_len)
    a.seg_q_src, a.q_rope, a.cos_table, a.sin_table = L.ptr(seg_q_src), L.ptr(q_rope), L.ptr(cos), L.ptr(sin)
    a.n_rope_rows = n_rope_rows
    a.n_q_video = q.shape[0] if n_q_video is None else int(n_q_video)
    a.q_row_stride, a.k_row_stride, a.o_row_stride = qs, ks, os_
    a.n_seg, a.sum_q, a.max_q, a.max_k, a.H, a.D = int(n_seg), int(sum_q), int(max_q), int(max_k), H, D
    a.scale = float(D ** -0.5 if scale is None else scale)
    a.q_row_step = int(q_row_step)
    if v_tok is not None:
        a.v_tok, a.v_lead, a.v_row, a.v_tok_rows = v_tok.data_ptr(), v_lead.data_ptr(), v_row.data_ptr(), v_tok.shape[0]
    a.v_runs = L.ptr(v_runs)
    a.k_len_head = L.ptr(k_len_head)
    if k_tok is not None:
        a.k_tok, a.k_lead, a.v_row, a.k_tok_rows = k_tok.data_ptr(), k_lead.data_ptr(), v_row.data_ptr(), k_tok.shape[0]
    if noalloc:
        a.workspace, a.workspace_bytes = None, 0
        with torch.cuda.device(q.device):
            L.check(L.lib().or_varlen_fwd_noalloc(ctypes.byref(a), L.stream_handle(q.device)), 'or_varlen_fwd_noalloc')
        return out
    a.workspace, a.workspace_bytes = workspace.data_ptr(), workspace.numel()
    L.check(L.lib().or_varlen_fwd(ctypes.byref(a), L.stream_handle(q.device)), 'or_varlen_fwd')
    return out


def scatter(plan: ScopePlan, packed: torch.Tensor, ov: torch.Tensor, ot: torch.Tensor | None):
    """write packed outputs back to token order (ov rows / ot rows), and zero ot's rows past the valid text"""
    H, D = packed.shape[1], packed.shape[2]
    _check_bf16(packed, ov, ot)
    _, vs = _rows2d(ov, H, D)
    ts = _rows2d(ot, H, D)[1] if ot is not None and ot.shape[0] else vs
    valid = sum(plan.counts) if plan.with_text else 0
    Le = ot.shape[0] if ot is not None else 0
    L.check(L.lib().or_scatter(packed.data_ptr(), plan.q_src.data_ptr(), plan.sum_q, plan.n_video, ov.data_ptr(),
                               L.ptr(ot if Le else None), vs, ts, valid, Le, H, D, L.stream_handle(packed.device)),
            'or_scatter')
    return ov, ot


def zero_text_padding(plan: ScopePlan, ot: torch.Tensor):
    """ot rows [sum(counts), Le) = 0 (the reference's ot = eq.new_zeros leaves them so)"""
    H, D = ot.shape[1], ot.shape[2]
    valid = sum(plan.counts) if plan.with_text else 0
    if ot.shape[0] <= valid:
        return ot
    _, ts = _rows2d(ot, H, D)
    L.check(L.lib().or_scatter(None, None, 0, plan.n_video, None, ot.data_ptr(), ts, ts, valid, ot.shape[0], H, D,
                               L.stream_handle(ot.device)), 'or_scatter')
    return ot


def rotate_queries(plan: ScopePlan, q, cos, sin, out=None):
    """every video query row rotated at its scene-RoPE table row, in token order (or_rotate_rows over the plan's
    packed queries; text rows are not rotated and stay in the text tensor): [F*T, H, D] bf16"""
    H, D = q.shape[1], q.shape[2]
    _check_bf16(q, out)
    _, qs = _rows2d(q, H, D)
    cos, sin, n_rows = _tables(cos, sin, D)
    if cos is None:
        raise L.HipValueError('RoPE needs the (cos, sin) tables')
    if plan.max_rope_row >= n_rows:
        raise L.HipValueError(f'layout needs rotary row {plan.max_rope_row} but the table has {n_rows} rows')
    out = torch.empty(plan.n_video, H, D, dtype=q.dtype, device=q.device) if out is None else out
    _, os_ = _rows2d(out, H, D)
    if out.shape[0] < plan.n_video:
        raise L.HipValueError(f'out holds {out.shape[0]} rows, the layout has {plan.n_video} video rows')
    L.check(L.lib().or_rotate_rows(q.data_ptr(), qs, plan.n_video, plan.q_src.data_ptr(), plan.q_rope.data_ptr(),
                                   cos.data_ptr(), sin.data_ptr(), n_rows, plan.sum_q, H, D, out.data_ptr(), os_,
                                   L.stream_handle(q.device)), 'or_rotate_rows')
    return out


def pack_layer(plan: ScopePlan, k, ek, v, ev, cos=None, sin=None, mode='raw', kbuf=None, vbuf=None, q=None,
               qbuf=None, values_in_place=True):
    """One launch of or_pack_layer: the plan's packed keys (rotated per `mode`, as pack_rows) into kbuf, the values
    into vbuf (only the rows the attention call does not read in place when values_in_place: plan.v_src), and, when q
    is given, the video queries rotated once in token order into qbuf (as rotate_queries). Returns (kbuf, vbuf,
    qbuf)."""
    H, D = k.shape[1], k.shape[2]
    _check_bf16(k, ek, v, ev, q, kbuf, vbuf, qbuf)
    _, vs = _rows2d(k, H, D)
    ts = _rows2d(ek, H, D)[1] if ek is not None and ek.shape[0] else vs
    if _rows2d(v, H, D)[1] != vs or (ev is not None and ev.shape[0] and ev.stride(0) != ts):
        raise L.HipValueError('value rows must have the strides of the key rows')
    if mode not in MODES:
        raise L.HipValueError(mode)
    rope = move = None
    if mode == 'raw':
        rope = plan.k_rope
    elif mode == 'rotated' and plan.adjacent:
        if plan.k_move_a is None:
            raise L.HipValueError('plan was built without move rows (moves=True)')
        rope, move = plan.k_move_b, plan.k_move_a
    need_tab = rope is not None or q is not None
    cos, sin, n_rows = _tables(cos, sin, D) if need_tab else (None, None, 0)
    if need_tab and cos is None:
        raise L.HipValueError('RoPE needs the (cos, sin) tables')
    if need_tab and plan.max_rope_row >= n_rows:
        raise L.HipValueError(f'layout needs rotary row {plan.max_rope_row} but the table has {n_rows} rows')
    new = lambda n: torch.empty(n, H, D, dtype=torch.bfloat16, device=k.device)
    kbuf = new(plan.sum_k) if kbuf is None else kbuf
    vbuf = new(plan.sum_k) if vbuf is None else vbuf
    for t in (kbuf, vbuf):
        if t.shape[0] < plan.sum_k or not t.is_contiguous():
            raise L.HipValueError(f'pack buffers must be contiguous with {plan.sum_k} rows')
    a = L.PackArgs()
    a.k_video, a.k_text = k.data_ptr(), L.ptr(ek if ek is not None and ek.shape[0] else None)
    a.v_video, a.v_text = v.data_ptr(), L.ptr(ev if ev is not None and ev.shape[0] else None)
    a.video_row_stride, a.text_row_stride, a.n_video = vs, ts, plan.n_video
    a.k_src, a.k_rope, a.k_move_from = plan.k_src.data_ptr(), L.ptr(rope), L.ptr(move)
    a.v_src = plan.v_src.data_ptr() if values_in_place else None
    a.n_keys, a.k_out, a.v_out = plan.sum_k, kbuf.data_ptr(), vbuf.data_ptr()
    if q is not None:
        _, qs = _rows2d(q, H, D)
        if q.shape[0] != plan.n_video:
            raise L.HipValueError(f'{q.shape[0]} video query rows, layout has {plan.n_video}')
        qbuf = torch.empty_like(q) if qbuf is None else qbuf
        _, qos = _rows2d(qbuf, H, D)
        if qbuf.shape[0] < plan.n_video:
            raise L.HipValueError(f'qbuf holds {qbuf.shape[0]} rows, the layout has {plan.n_video} video rows')
        a.q, a.q_row_stride, a.q_src, a.q_rope = q.data_ptr(), qs, plan.q_src.data_ptr(), plan.q_rope.data_ptr()
        a.n_queries, a.q_out, a.q_out_row_stride = plan.sum_q, qbuf.data_ptr(), qos
    a.cos_table, a.sin_table, a.n_rope_rows = L.ptr(cos), L.ptr(sin), n_rows
    a.H, a.D = H, D
    L.check(L.lib().or_pack_layer(ctypes.byref(a), L.stream_handle(k.device)), 'or_pack_layer')
    return kbuf, vbuf, qbuf


def scene_attention(plan: ScopePlan, q, k, v, eq, ek, ev, cos=None, sin=None, mode='raw', fused=True,
                    kbuf=None, vbuf=None, qbuf=None, rotate_q='pre', values_in_place=True):
    """(ov, ot) of one scene-attention layer. q / k / v [F*T, H, D] and eq / ek / ev [Le, H, D] bf16 on the GPU.

    fused=True: one pack launch (K rows, the V rows not read in place, and the video queries rotated once when
    mode is 'raw' and rotate_q='pre', into qbuf when given), then the attention call with Q read in place, the
    own-frame values and the shared frames' values (value runs, head_dim 128) read in place from v (values_in_place,
    when v's rows are H * D elements apart, as the packed rows are) and the outputs written in place. rotate_q='load' rotates the queries on the attention kernel's Q load instead.
    fused=False: the reference's data flow (Q, K, V packed, one varlen call on packed tensors, write-back by the
    scatter kernel).

    With a plan for one rank's share (q_range), ov rows outside the rank's video tokens are zero, as are ot rows of
    the sentences the rank does not run (ot = eq.new_zeros in the reference)."""
    if mode not in MODES:
        raise L.HipValueError(mode)
    H, D = q.shape[1], q.shape[2]
    if q.shape[0] != plan.n_video:
        raise L.HipValueError(f'{q.shape[0]} video rows, layout has {plan.n_video}')
    if plan.with_text and eq.shape[0] != plan.text_rows:
        raise L.HipValueError(f'{eq.shape[0]} text rows, layout has {plan.text_rows}')
    # one rank's share writes only its own rows: the others stay zero
    make = torch.zeros if plan.q_range is not None else torch.empty
    ov = make(q.shape, dtype=q.dtype, device=q.device)
    ot = make(eq.shape[0], H, D, dtype=q.dtype, device=q.device) if eq is not None else None
    qmode = 'raw' if mode == 'raw' else 'none'
    if fused:
        if rotate_q not in ('pre', 'load'):
            raise L.HipValueError(f"rotate_q must be 'pre' or 'load', got {rotate_q!r}")
        on_load = qmode == 'raw' and rotate_q == 'load'
        pre = qmode == 'raw' and not on_load
        # the value runs past the leading one are read in place by the head_dim 128 kernel only: with another
        # head_dim such a plan packs every value
        in_place = (bool(values_in_place) and v.dim() == 3 and v.stride(0) == H * D and v.is_contiguous()
                    and (plan.v_runs is None or D == 128))
        kp, vp, qr = pack_layer(plan, k, ek, v, ev, cos, sin, mode, kbuf, vbuf, q=q if pre else None, qbuf=qbuf,
                                values_in_place=in_place)
        vi = dict(v_tok=v, v_lead=plan.v_lead, v_row=plan.v_row, v_runs=plan.v_runs) if in_place else {}
        qq = qr if pre else q
        # the text queries in the video queries' row stride (a copy of the Le text rows when q and eq are views with
        # different strides, e.g. a head range of wider rows whose video queries were rotated into a new buffer)
        et = _with_row_stride(eq, qq.stride(0)) if eq is not None and eq.shape[0] else eq
        varlen(qq, kp, vp, plan.cu_q, plan.cu_k, plan.max_q, plan.max_k, k_off=plan.k_off,
               k_len=plan.k_len, out=ov, seg_q_src=plan.seg_q_src, q_text=et, o_text=ot, n_q_video=plan.n_video,
               q_rope=plan.q_rope if on_load else None, cos=cos, sin=sin, sum_q=plan.sum_q,
               workspace=plan.workspace(H, D), **vi)
        if ot is not None:
            zero_text_padding(plan, ot)
    else:
        kp, vp = pack_rows(plan, k, ek, 'k', out=kbuf, b_video=v, b_text=ev, b_out=vbuf, cos=cos, sin=sin, mode=mode)
        qp = pack_rows(plan, q, eq, 'q', cos=cos, sin=sin, mode=qmode)
        op = varlen(qp, kp, vp, plan.cu_q, plan.cu_k, plan.max_q, plan.max_k, k_off=plan.k_off, k_len=plan.k_len,
                    workspace=plan.workspace(H, D))
        scatter(plan, op, ov, ot)
    return ov, ot
