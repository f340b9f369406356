"""A random-init Wan2.2-TI2V-5B-shaped DiT forward: the end-to-end step time around the scene-attention path.

The reference runs diffusers' WanTransformer3DModel (third-party, not vendored; its blocks get the scene processors
at src/onereel/models/wan.py:77-108). Per block that model has:

- AdaLN-modulated self-attention: the processor's `_qk` (RMSNorm + RoPE, wan.py:64-74), scene scopes;
- cross-attention of every scene to its own sentence (wan.py:84-89);
- a GELU feed forward.

This module rebuilds that block structure with random N(0, 0.02) bf16 weights (no checkpoint is available offline).
It runs the attention through onereel_amd.wan's processors:

- self-attention: the fused RMSNorm + RoPE kernel, then the scene layout, pack and varlen kernels (frame-memory
  scopes);
- cross-attention: the varlen kernel's zero-copy key ranges.

GEMMs stay torch ops (hipBLASLt). The block's LayerNorm + modulation and gated residual adds are HIP passes instead of
chains of torch kernels over fp32 temporaries: every residual add runs in one pass with the LayerNorm that follows it
(`or_residual_layernorm_modulate`: the next norm of the block, or the next block's first norm, or the output norm),
and only the first norm runs alone (`or_layernorm_modulate`). Shapes of
Wan2.2-TI2V-5B: hidden 3072 = 24 heads x 128, FFN 14336, 30 blocks, eps 1e-6, patch (1, 2, 2) over 48 latent
channels, text width 4096 projected to 3072.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn.functional as F

from . import _lib as L
from . import wan
from .layout import SceneLayout


@dataclass
class DiTConfig:
    dim: int = 3072
    heads: int = 24
    ffn: int = 14336
    blocks: int = 30
    eps: float = 1e-6
    in_channels: int = 48
    patch: int = 4                   # (1, 2, 2) patch: 4 latent positions per token
    text_dim: int = 4096
    freq_dim: int = 256
    std: float = 0.02


def _rows(x: torch.Tensor):
    C = x.shape[-1]
    x2 = x.reshape(-1, C)
    if x.dtype != torch.bfloat16 or x2.stride(1) != 1:
        raise L.HipValueError('expected bf16 rows with contiguous elements')
    return x2, C


def _vec(t, C):
    """per-column parameter as a contiguous fp32 [C] vector at a 16-byte aligned address (the kernels read it in
    16-byte pieces)"""
    if t is None:
        return None
    v = t.reshape(C).to(torch.float32).contiguous()
    return v if v.data_ptr() % 16 == 0 else v.clone()


def layernorm_modulate(x, eps, weight=None, bias=None, scale=None, shift=None):
    """bf16 [..., C] -> bf16 LayerNorm(x) [* weight + bias] [* (1 + scale) + shift], fp32 inside, one HIP pass (the
    block's x.float() / layer_norm / modulation / .to(bf16) chain)"""
    x2, C = _rows(x)
    out = torch.empty(x2.shape, dtype=torch.bfloat16, device=x.device)
    w, b, sc, sh = (_vec(t, C) for t in (weight, bias, scale, shift))
    d = L.dit_lib()
    L.dit_check(d.or_layernorm_modulate(x2.data_ptr(), out.data_ptr(), x2.shape[0], C, x2.stride(0), C, float(eps),
                                        L.ptr(w), L.ptr(b), L.ptr(sc), L.ptr(sh), L.stream_handle(x.device)),
                'or_layernorm_modulate')
    return out.view(x.shape)


def gated_residual_(x, a, gate=None):
    """x = bf16(float(x) + float(a) * gate) in place (x = x + a without a gate), one HIP pass"""
    x2, C = _rows(x)
    a2, Ca = _rows(a)
    if Ca != C or a2.shape[0] != x2.shape[0]:
        raise L.HipValueError('x and a must have the same rows')
    g = _vec(gate, C)
    d = L.dit_lib()
    L.dit_check(d.or_gated_residual(x2.data_ptr(), a2.data_ptr(), L.ptr(g), x2.shape[0], C, x2.stride(0),
                                    a2.stride(0), L.stream_handle(x.device)), 'or_gated_residual')
    return x


def residual_layernorm_modulate_(x, a, eps, gate=None, weight=None, bias=None, scale=None, shift=None):
    """gated_residual_(x, a, gate), then layernorm_modulate of the updated x, in one HIP pass over the rows (the same
    bits as the two calls); x is updated in place and the normalised rows are returned"""
    x2, C = _rows(x)
    a2, Ca = _rows(a)
    if Ca != C or a2.shape[0] != x2.shape[0]:
        raise L.HipValueError('x and a must have the same rows')
    out = torch.empty(x2.shape, dtype=torch.bfloat16, device=x.device)
    g, w, b, sc, sh = (_vec(t, C) for t in (gate, weight, bias, scale, shift))
    d = L.dit_lib()
    L.dit_check(d.or_residual_layernorm_modulate(x2.data_ptr(), a2.data_ptr(), L.ptr(g), out.data_ptr(), x2.shape[0],
                                                 C, x2.stride(0), a2.stride(0), C, float(eps), L.ptr(w), L.ptr(b),
                                                 L.ptr(sc), L.ptr(sh), L.stream_handle(x.device)),
                'or_residual_layernorm_modulate')
    return out.view(x.shape)


class Linear:
    def __init__(self, n_in, n_out, std, gen, device):
        self.weight = (torch.randn(n_out, n_in, generator=gen, device=device) * std).to(torch.bfloat16)
        self.bias = (torch.randn(n_out, generator=gen, device=device) * std).to(torch.bfloat16)

    def __call__(self, x):
        return F.linear(x, self.weight, self.bias)

    def gelu_tanh(self, x):
        """GELU(x W^T + b, approximate='tanh') with the activation in the GEMM's epilogue (hipBLASLt through
        torch._addmm_activation): the activation is applied to the fp32 accumulator and the [.., n_out] output is
        written once, instead of a separate GELU pass over it"""
        x2 = x.reshape(-1, x.shape[-1])
        y = torch._addmm_activation(self.bias, x2, self.weight.t(), use_gelu=True)
        return y.view(*x.shape[:-1], y.shape[-1])


class RMSNorm:
    def __init__(self, n, eps, gen, device):
        self.weight = (1 + 0.1 * torch.randn(n, generator=gen, device=device)).to(torch.bfloat16)
        self.eps = eps

    def __call__(self, x):
        return wan.rms_norm(x, self.weight, self.eps)


class Attention:
    """the attributes diffusers' Attention exposes to a processor: heads, to_q / to_k / to_v, to_out (projection and
    an identity in place of dropout), norm_q / norm_k (RMSNorm over all heads)"""

    def __init__(self, cfg: DiTConfig, gen, device):
        d = cfg.dim
        self.heads = cfg.heads
        self.to_q, self.to_k, self.to_v = (Linear(d, d, cfg.std, gen, device) for _ in range(3))
        self.to_out = [Linear(d, d, cfg.std, gen, device), lambda x: x]
        self.norm_q, self.norm_k = RMSNorm(d, cfg.eps, gen, device), RMSNorm(d, cfg.eps, gen, device)


class Block:
    """one Wan transformer block: modulated self-attention, cross-attention, modulated GELU feed forward"""

    def __init__(self, cfg: DiTConfig, gen, device):
        d = cfg.dim
        self.cfg = cfg
        self.attn1, self.attn2 = Attention(cfg, gen, device), Attention(cfg, gen, device)
        self.norm2_w = (1 + 0.1 * torch.randn(d, generator=gen, device=device)).float()
        self.norm2_b = (0.1 * torch.randn(d, generator=gen, device=device)).float()
        self.ffn_in = Linear(d, cfg.ffn, cfg.std, gen, device)
        self.ffn_out = Linear(cfg.ffn, d, cfg.std, gen, device)
        self.scale_shift_table = torch.randn(6, d, generator=gen, device=device) / d ** 0.5

    def modulation(self, temb6):
        """(shift, scale, gate, c_shift, c_scale, c_gate), each [1, dim] fp32"""
        return (self.scale_shift_table + temb6).chunk(6, 0)

    def __call__(self, x, n, mod, text, rotary, p_self, p_cross):
        """x [1, S, dim] bf16, updated in place; n: LayerNorm(x) * (1 + scale) + shift of this block's modulation
        `mod`; text [1, L, dim] bf16. Returns the feed forward's output and its gate: the caller adds them to x
        together with the next LayerNorm (the block's own residual adds run with the norms that follow them)."""
        eps = self.cfg.eps
        shift, scale, gate, c_shift, c_scale, c_gate = mod
        n = residual_layernorm_modulate_(x, p_self(self.attn1, n, rotary_emb=rotary), eps, gate=gate,
                                         weight=self.norm2_w, bias=self.norm2_b)
        n = residual_layernorm_modulate_(x, p_cross(self.attn2, n, encoder_hidden_states=text), eps, scale=c_scale,
                                         shift=c_shift)
        return self.ffn_out(self.ffn_in.gelu_tanh(n)), c_gate


def timestep_features(t: float, n: int, device) -> torch.Tensor:
    """sinusoidal features of timestep t: [cos(t f_i), sin(t f_i)] with f_i = 10000^(-i / (n / 2))"""
    f = torch.exp(-math.log(10000.0) * torch.arange(n // 2, device=device, dtype=torch.float32) / (n // 2))
    return torch.cat([torch.cos(t * f), torch.sin(t * f)])


class WanDiT:
    """random-init DiT over one multi-scene latent; `forward` is one transformer pass (one denoising step without
    classifier-free guidance)"""

    def __init__(self, cfg: DiTConfig, layout: SceneLayout, T: int, text_len: int, device, seed: int = 0):
        gen = torch.Generator(device=device).manual_seed(seed)
        d, self.cfg = cfg.dim, cfg
        self.patch_embed = Linear(cfg.in_channels * cfg.patch, d, cfg.std, gen, device)
        self.text_in, self.text_out = Linear(cfg.text_dim, d, cfg.std, gen, device), Linear(d, d, cfg.std, gen, device)
        self.time_in, self.time_out = Linear(cfg.freq_dim, d, cfg.std, gen, device), Linear(d, d, cfg.std, gen, device)
        self.time_proj = Linear(d, 6 * d, cfg.std, gen, device)
        self.blocks = [Block(cfg, gen, device) for _ in range(cfg.blocks)]
        self.scale_shift_table = torch.randn(2, d, generator=gen, device=device) / d ** 0.5
        self.proj_out = Linear(d, cfg.in_channels * cfg.patch, cfg.std, gen, device)
        self.ctx = wan.Context(layout=layout, T=T, text_len=text_len)
        self.p_self = wan.Processor(self.ctx, 'self')
        self.p_cross = wan.Processor(self.ctx, 'cross')

    def forward(self, tokens, t: float, text, rotary):
        """tokens [S, in_channels * patch] bf16 (the patchified latent, frame-major), text [n_scenes * text_len,
        text_dim] bf16 (sentence j in rows j * text_len ..), rotary (cos, sin) [1, S, 1, D] fp32 -> [S, in * patch]"""
        d = self.cfg.dim
        x = self.patch_embed(tokens)[None]
        temb = self.time_out(F.silu(self.time_in(timestep_features(t, self.cfg.freq_dim, tokens.device)
                                                 .to(torch.bfloat16))))
        temb6 = self.time_proj(F.silu(temb)).float().view(6, d)
        ctx_text = self.text_out(F.gelu(self.text_in(text), approximate='tanh'))[None]
        eps = self.cfg.eps
        mods = [blk.modulation(temb6) for blk in self.blocks]
        out_shift, out_scale = (self.scale_shift_table + temb.float()[None]).chunk(2, 0)
        n = layernorm_modulate(x, eps, scale=mods[0][1], shift=mods[0][0])
        for i, blk in enumerate(self.blocks):
            f, gate = blk(x, n, mods[i], ctx_text, rotary, self.p_self, self.p_cross)
            # the feed forward's residual add, with the next block's first norm (the output norm after the last)
            shift, scale = (mods[i + 1][0], mods[i + 1][1]) if i + 1 < len(self.blocks) else (out_shift, out_scale)
            n = residual_layernorm_modulate_(x, f, eps, gate=gate, scale=scale, shift=shift)
        return self.proj_out(n)[0]

    def flops(self, text_rows: int) -> dict:
        """useful FLOP of one forward: GEMMs (2 m n k each) and attention (4 Lq Lk H D per scope, self and cross)"""
        c, lay, T = self.cfg, self.ctx.layout, self.ctx.T
        S = lay.n_frames * T
        d, hd = c.dim, c.dim // c.heads
        per_block = (4 * 2 * S * d * d            # self q, k, v, out
                     + 2 * 2 * S * d * d          # cross q, out
                     + 2 * 2 * text_rows * d * d  # cross k, v
                     + 2 * 2 * S * d * c.ffn)     # feed forward
        attn_self = sum(4 * (hi - lo) * T * len(lay.key_frames(j)) * T * c.heads * hd
                        for j, (lo, hi) in enumerate(lay.ranges))
        attn_cross = sum(4 * (hi - lo) * T * self.ctx.text_len * c.heads * hd for lo, hi in lay.ranges)
        other = 2 * 2 * S * d * c.in_channels * c.patch + 2 * 2 * text_rows * d * (c.text_dim + d)
        return dict(gemm=c.blocks * per_block + other, attention_self=c.blocks * attn_self,
                    attention_cross=c.blocks * attn_cross)


def wan_rope_table(F_: int, Hh: int, Ww: int, D: int, theta: float = 10000.0):
    """Wan's 3D RoPE over (frame, row, column), split as diffusers' WanRotaryPosEmbed splits a head's D dims: height
    and width 2 * (D // 6) dims each, time the remaining D - 4 * (D // 6); interleaved real pairs (each angle twice).
    Returns cos / sin [1, F*Hh*Ww, 1, D] fp32."""
    hw = 2 * (D // 6)
    dims = [D - 2 * hw, hw, hw]
    f, y, x = torch.meshgrid(torch.arange(F_), torch.arange(Hh), torch.arange(Ww), indexing='ij')
    ang = torch.cat([p.reshape(-1, 1).double() * theta ** (-torch.arange(0, n, 2).double() / n)
                     for p, n in zip((f, y, x), dims)], 1)
    cos = ang.cos().float().repeat_interleave(2, 1)
    sin = ang.sin().float().repeat_interleave(2, 1)
    return cos[None, :, None], sin[None, :, None]
