"""Oracle: the Wan self-attention's query / key normalisation and RoPE (`_qk`), on the CPU.

TEST INFRASTRUCTURE ONLY (see `oracle/__init__.py`). Restates `_qk` (src/onereel/models/wan.py:64-74): torch's
F.rms_norm over the whole row of C = heads * D elements (diffusers' 'rms_norm_across_heads') with weight w and eps,
then per head the interleaved RoPE with c = cos[..., 0::2] and s = sin[..., 1::2]:
(x1 * c - x2 * s, x1 * s + x2 * c) for x1 = y[..., 0::2], x2 = y[..., 1::2], cast back to the input dtype
(type_as). The reference compiles `_qk` with torch.compile, whose fused graph keeps the chain in fp32 and rounds once;
this restatement does the same. Pinned in tests/test_oracle.py against the textbook forms: the RMS of the normalised
row is 1 before the weight, and the rotation of each pair is the complex product (x1 + i x2)(c + i s).
"""
from __future__ import annotations

import torch


def qk_norm_rope(x, w, eps, cos, sin, heads):
    """x [S, C] (bf16), w [C], cos / sin [S, D] -> [S, heads, D] in x's dtype"""
    S, C = x.shape
    D = C // heads
    ft = torch.promote_types(x.dtype, torch.float32)     # fp32 for bf16 / fp32 inputs, float64 for float64
    xf = x.to(ft)
    y = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.to(ft)
    y = y.view(S, heads, D)
    x1, x2 = y[..., 0::2], y[..., 1::2]
    c, s = cos.to(ft)[:, None, 0::2], sin.to(ft)[:, None, 1::2]
    return torch.stack([x1 * c - x2 * s, x1 * s + x2 * c], -1).flatten(-2).to(x.dtype)
