"""Oracle: RoPE, packing, per-scope attention and write-back of one scene-attention layer, on the CPU.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`). Restates:

- `apply_rotary_emb`   diffusers 0.41.0.dev0 @ e0415c41 `apply_rotary_emb(x, (cos, sin), use_real=True,
                       use_real_unbind_dim=-1, sequence_dim=1)` (a third-party dependency, absent here), as the
                       reference calls it (src/onereel/models/hunyuan15.py:148-149,189-190) and exercises it
                       (tests/test_shared_pos.py:15-25): interleaved pairs (2i, 2i+1), rot(x) = (-x_odd, x_even),
                       out = x*cos + rot(x)*sin in fp32 (two products and a sum, each rounded), cast to x's dtype
- `rotate_video`       Processor.__call__'s RoPE of the video q / k rows (hunyuan15.py:183-191)
- `move_shared`        _move_shared (hunyuan15.py:127-150): two rotations through table rows a and a + d
- `pack`, `packed_attention`
                       attention.packed (src/onereel/attention.py:65-71) with the FlashAttention varlen semantics it
                       calls (attention.py:39-43): per segment softmax(q k^T * D^-0.5) v, non-causal, in fp32 via
                       torch.nn.functional.scaled_dot_product_attention per scope (no mask)
- `scene_layer`        Processor.scene on one GPU (hunyuan15.py:212-251): ov[q rows] = video outputs, ot = zeros then
                       text outputs (rows past the valid text stay 0)
- `merge_lse`          ring._merge (src/onereel/parallel/ring.py:63-70): a partial (o_s, lse_s) folded into the
                       running fp32 (o, lse); the same weights as Processor._far_lse's merge (hunyuan15.py:270-275)
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F


def apply_rotary_emb(x, cos, sin):
    """x [S, H, D] (any float dtype), cos / sin [S, D] fp32 -> [S, H, D] in x's dtype"""
    xr, xi = x.reshape(*x.shape[:-1], -1, 2).unbind(-1)
    x_rot = torch.stack([-xi, xr], dim=-1).flatten(-2)
    c, s = cos[:, None, :], sin[:, None, :]
    return (x.float() * c + x_rot.float() * s).to(x.dtype)


def rotate_rows(x, rope_rows, cos, sin):
    """rows of x with rope_rows[i] >= 0 rotated at that table row; the others unchanged"""
    rope_rows = torch.as_tensor(rope_rows)
    out = x.clone()
    m = rope_rows >= 0
    if bool(m.any()):
        out[m] = apply_rotary_emb(x[m], cos[rope_rows[m]], sin[rope_rows[m]])
    return out


def move_shared(k_rows, move_a, move_b, cos, sin):
    """_move_shared's re-rotation of already rotated keys: x = R(-a) k (cast), then R(b) x (cast), on the rows where
    move_a >= 0 (hunyuan15.py:148-150)"""
    move_a, move_b = torch.as_tensor(move_a), torch.as_tensor(move_b)
    out = k_rows.clone()
    m = move_a >= 0
    if bool(m.any()):
        x = apply_rotary_emb(k_rows[m], cos[move_a[m]], -sin[move_a[m]])
        out[m] = apply_rotary_emb(x, cos[move_b[m]], sin[move_b[m]])
    return out


def gather_rows(video, text, src):
    """rows of the virtual concatenation [video ; text] (text row t encoded as n_video + t)"""
    src = torch.as_tensor(src)
    return torch.cat([video, text])[src]


def pack(sc, q, k, v, eq, ek, ev, cos=None, sin=None, mode='raw'):
    """the packed (q, k, v) of every scope. mode 'raw': q / k rows are rotated here at the scope's rotary rows (the
    reference's Processor.__call__ RoPE, then _move_shared on the shared keys, composed as one rotation at the
    destination row); 'rotated': q / k are already rotated, shared keys re-rotated by move_shared exactly as
    _move_shared does; 'none': no rotation at all"""
    qp = gather_rows(q, eq, sc.q_src)
    kp = gather_rows(k, ek, sc.k_src)
    vp = gather_rows(v, ev, sc.k_src)
    if mode == 'raw':
        qp = rotate_rows(qp, sc.q_rope, cos, sin)
        kp = rotate_rows(kp, sc.k_rope, cos, sin)
    elif mode == 'rotated':
        kp = move_shared(kp, sc.k_move_a, sc.k_move_b, cos, sin)
    else:
        assert mode == 'none', mode
    return qp, kp, vp


def packed_attention(qp, kp, vp, cu_q, cu_k, k_off=None, k_len=None):
    """fp32 softmax(q k^T / sqrt(D)) v per segment (torch SDPA on the CPU, no mask). k_off / k_len: the keys of
    segment s are kp[k_off[s] : k_off[s] + k_len[s]] (overlapping ranges, attention.py:74-84); else cu_k."""
    D = qp.shape[-1]
    out = torch.zeros(qp.shape, dtype=torch.float32)
    for s in range(len(cu_q) - 1):
        a, b = int(cu_q[s]), int(cu_q[s + 1])
        if b == a:
            continue
        if k_off is None:
            c, d = int(cu_k[s]), int(cu_k[s + 1])
        else:
            c = int(k_off[s])
            d = c + int(k_len[s])
        qs, ks, vs = (x.float().transpose(0, 1)[None] for x in (qp[a:b], kp[c:d], vp[c:d]))
        o = F.scaled_dot_product_attention(qs, ks, vs, scale=D ** -0.5)
        out[a:b] = o[0].transpose(0, 1)
    return out


def write_back(sc, o, text_rows, dtype=torch.float32):
    """hunyuan15.py:226,231-235: ov[q rows] = out; ot = zeros, then the text rows of every sentence"""
    H, D = o.shape[1:]
    ov = torch.zeros(sc.n_video, H, D, dtype=dtype)
    ot = torch.zeros(text_rows, H, D, dtype=dtype)
    src = torch.as_tensor(sc.q_src)
    vid = src < sc.n_video
    ov[src[vid]] = o[vid].to(dtype)
    ot[src[~vid] - sc.n_video] = o[~vid].to(dtype)
    return ov, ot


def scene_layer(sc, q, k, v, eq, ek, ev, cos=None, sin=None, mode='raw'):
    """one layer of scene attention on one GPU: (ov, ot) in fp32"""
    qp, kp, vp = pack(sc, q, k, v, eq, ek, ev, cos, sin, mode)
    o = packed_attention(qp, kp, vp, sc.cu_q, sc.cu_k)
    return write_back(sc, o, eq.shape[0])


def rope_table_3d(F_, Hh, Ww, D, theta=1e4):
    """a 3D RoPE table built as tests/test_shared_pos.py:16-20 builds it (temporal, height, width frequencies on
    separate pair groups, interleaved real pairs): D/2 pairs split as (D/8, 3D/16, 3D/16) -> cos, sin [F*Hh*Ww, D]"""
    f, y, x = torch.meshgrid(torch.arange(F_), torch.arange(Hh), torch.arange(Ww), indexing='ij')
    nt, ny = D // 8, 3 * D // 16
    groups = [(f, nt), (y, ny), (x, D // 2 - nt - ny)]
    ang = torch.cat([p.reshape(-1, 1).float() * (theta ** (-torch.arange(n).float() / n)) for p, n in groups], 1)
    return ang.cos().repeat_interleave(2, 1).contiguous(), ang.sin().repeat_interleave(2, 1).contiguous()


def useful_flops(lq, lk, H, D):
    """experiments/kernel_breakdown.py:101: sum over segments of 4 * Lq * Lk * H * D"""
    return float(sum(4.0 * a * b * H * D for a, b in zip(lq, lk)))


def masked_reference(lay, T, counts, q, k, v, eq, ek, ev):
    """brute-force scope semantics (src/onereel/README.md:11-15; the mask of experiments/kernel_breakdown.py:78-86):
    each query of the joint token set [video ; text] attends every key its scope allows, in original order, via a
    dense fp32 masked softmax. Independent of any packing order. q..ev already rotated."""
    S, Le = q.shape[0], eq.shape[0]
    F_ = lay.n_frames
    frame_scene = np.repeat(np.arange(lay.n_scenes), lay.lengths)
    c = np.cumsum([0] + list(counts))
    allow = np.zeros((S + Le, S + Le), bool)
    tok_frame = np.arange(S) // T
    for j in range(lay.n_scenes):
        vq = np.nonzero(frame_scene[tok_frame] == j)[0]
        keys = set(lay.key_frames(j))
        vk = np.nonzero(np.isin(tok_frame, list(keys)))[0]
        tt = S + np.arange(c[j], c[j + 1])
        own = np.nonzero(frame_scene[tok_frame] == j)[0]
        allow[np.ix_(vq, np.concatenate([vk, tt]))] = True
        allow[np.ix_(tt, np.concatenate([own, tt]))] = True
    assert F_ * T == S
    qq, kk, vv = (torch.cat([a, b]).float() for a, b in ((q, eq), (k, ek), (v, ev)))
    D = q.shape[-1]
    s = torch.einsum('qhd,khd->hqk', qq, kk) / D ** 0.5
    s = s.masked_fill(~torch.as_tensor(allow)[None], float('-inf'))
    p = torch.softmax(s, -1).nan_to_num(0.0)
    o = torch.einsum('hqk,khd->qhd', p, vv)
    return o[:S], o[S:]


def merge_lse(o, lse, o_s, lse_s):
    """ring._merge (ring.py:63-70), out of place: o [N, H, D] fp32, lse [H, N] fp32, o_s [N, H, D] (cast to o's dtype,
    as the reference's o_s.float()), lse_s [H, N] -> (o, lse) merged. m = max(lse, lse_s), 0 where infinite; w1 = exp(lse - m), w2 = exp(lse_s - m);
    o * (w1 / den) + o_s * (w2 / den) with den = w1 + w2; lse = m + log(den). Pinned in tests/test_oracle.py by the
    identity it exists for: merging attention over two disjoint key sets equals attention over their union."""
    m = torch.maximum(lse, lse_s)
    m = torch.where(torch.isinf(m), torch.zeros_like(m), m)
    w1, w2 = torch.exp(lse - m), torch.exp(lse_s - m)
    den = w1 + w2
    out = o * (w1 / den).transpose(0, 1)[..., None] + o_s.to(o.dtype) * (w2 / den).transpose(0, 1)[..., None]
    return out, m + torch.log(den)


def attention_lse(q, k, v):
    """dense attention of q [N, H, D] over k / v [M, H, D] in float64: (out [N, H, D], lse [H, N], natural log of the
    scaled scores' exp-sum; -inf and out 0 when M == 0)"""
    q, k, v = q.double(), k.double(), v.double()
    D = q.shape[-1]
    if k.shape[0] == 0:
        return torch.zeros_like(q), torch.full((q.shape[1], q.shape[0]), -float('inf'), dtype=torch.float64)
    s = torch.einsum('nhd,mhd->hnm', q, k) * D ** -0.5
    lse = torch.logsumexp(s, -1)
    out = torch.einsum('hnm,mhd->nhd', torch.softmax(s, -1), v)
    return out, lse
