"""GPU checks of the Wan-shaped DiT harness (onereel_amd.wan_dit): its scene processors against the oracle inside a
small random-init model, and a two-block forward against the same model run with oracle processors."""
import pytest
import torch

from helpers import assert_close
from onereel_amd import wan_dit as WD
from onereel_amd.layout import SceneLayout
from oracle import attention as OA
from oracle import layout as OL
from oracle import wan as OW

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]
DEV = 'cuda'

LENGTHS, T, TEXT_LEN = [2, 3, 2], 16, 8
EXTRA = {0: [3, 6], 1: [0], 2: [0, 4]}          # frame memory reps {0, 3, 4, 6} outside each scene


def _model(blocks):
    cfg = WD.DiTConfig(dim=512, heads=4, ffn=1024, blocks=blocks, in_channels=4, text_dim=256)
    lay = SceneLayout(LENGTHS, halo=0, extra=EXTRA)
    return WD.WanDiT(cfg, lay, T, TEXT_LEN, DEV, seed=3)


def _ref_self(model):
    """the processor's self-attention with the oracle's _qk and scope attention (fp32 attention on the CPU)"""
    sc = OL.hunyuan_scopes(OL.SceneLayout(LENGTHS, 0, 'adj', EXTRA), T, [0] * 3, 0, with_text=False)

    def run(attn, hidden_states, rotary_emb=None, **_):
        H, eps = attn.heads, attn.norm_q.eps
        cos, sin = (x[0, :, 0].cpu() for x in rotary_emb)
        q, k, v = attn.to_q(hidden_states), attn.to_k(hidden_states), attn.to_v(hidden_states)
        q = OW.qk_norm_rope(q[0].cpu(), attn.norm_q.weight.cpu(), eps, cos, sin, H)
        k = OW.qk_norm_rope(k[0].cpu(), attn.norm_k.weight.cpu(), eps, cos, sin, H)
        v = v[0].cpu().unflatten(1, (H, -1))
        qp, kp, vp = OA.pack(sc, q, k, v, q[:0], k[:0], v[:0], mode='none')
        o = OA.write_back(sc, OA.packed_attention(qp, kp, vp, sc.cu_q, sc.cu_k), 0)[0]
        return attn.to_out[0](o.flatten(1)[None].to(DEV).to(torch.bfloat16)), o
    return run


def _ref_cross(attn, hidden_states, encoder_hidden_states=None, **_):
    H = attn.heads
    q = attn.norm_q(attn.to_q(hidden_states))[0].cpu().unflatten(1, (H, -1))
    k = attn.norm_k(attn.to_k(encoder_hidden_states))[0].cpu().unflatten(1, (H, -1))
    v = attn.to_v(encoder_hidden_states)[0].cpu().unflatten(1, (H, -1))
    cq = [0]
    for n in LENGTHS:
        cq.append(cq[-1] + n * T)
    o = OA.packed_attention(q, k, v, cq, None, k_off=[j * TEXT_LEN for j in range(3)], k_len=[TEXT_LEN] * 3)
    return attn.to_out[0](o.flatten(1)[None].to(DEV).to(torch.bfloat16)), o


def _inputs(model):
    g = torch.Generator(device=DEV).manual_seed(5)
    S = sum(LENGTHS) * T
    tokens = torch.randn(S, 16, generator=g, device=DEV).to(torch.bfloat16)
    text = torch.randn(3 * TEXT_LEN, 256, generator=g, device=DEV).to(torch.bfloat16)
    rot = tuple(x.to(DEV) for x in WD.wan_rope_table(sum(LENGTHS), 4, 4, 128))
    return tokens, text, rot


def test_processors_match_the_oracle_inside_the_model():
    print('wan dit processors', flush=True)
    model = _model(1)
    tokens, text, rot = _inputs(model)
    blk = model.blocks[0]
    x = model.patch_embed(tokens)[None]
    got = model.p_self(blk.attn1, x, rotary_emb=rot)
    ref_out, ref_o = _ref_self(model)(blk.attn1, x, rotary_emb=rot)
    # the attention output itself (before the output projection), through the processor's own steps
    q, k, v = blk.attn1.to_q(x), blk.attn1.to_k(x), blk.attn1.to_v(x)
    from onereel_amd import wan
    qq, kk = wan._qk(q, k, blk.attn1.norm_q.weight, blk.attn1.norm_k.weight, blk.attn1.norm_q.eps, *rot, 4)
    o = wan.self_ranges(model.ctx, qq[0].contiguous(), kk[0].contiguous(), v[0].unflatten(1, (4, -1)).contiguous())
    assert_close(o.cpu(), ref_o, what='dit self-attention')
    assert (got.float() - ref_out.float()).abs().max() < 5e-2
    ctx_text = model.text_out(torch.nn.functional.gelu(model.text_in(text), approximate='tanh'))[None]
    got = model.p_cross(blk.attn2, x, encoder_hidden_states=ctx_text)
    ref_out, _ = _ref_cross(blk.attn2, x, encoder_hidden_states=ctx_text)
    assert (got.float() - ref_out.float()).abs().max() < 5e-2


def test_two_block_forward_matches_oracle_processors():
    print('wan dit forward', flush=True)
    model = _model(2)
    tokens, text, rot = _inputs(model)
    out = model.forward(tokens, 500.0, text, rot).float()
    ref_self = _ref_self(model)
    model.p_self = lambda attn, hs, rotary_emb=None: ref_self(attn, hs, rotary_emb=rotary_emb)[0]
    model.p_cross = lambda attn, hs, encoder_hidden_states=None: _ref_cross(attn, hs, encoder_hidden_states)[0]
    ref = model.forward(tokens, 500.0, text, rot).float()
    rel = ((out - ref).norm() / ref.norm()).item()
    print(f'two-block forward rel-L2 {rel:.2e}', flush=True)
    assert rel < 2e-2
    assert out.shape == (sum(LENGTHS) * T, 16) and torch.isfinite(out).all()


@pytest.mark.parametrize('S,C', [(257, 3072), (64, 512), (9, 1000)])
def test_fused_layernorm_modulate_and_residual_match_torch(S, C):
    """the block's fused passes against the torch expressions they replace: LayerNorm + modulation within one bf16
    step (and > 99% bit-equal), the gated residual bit-exact"""
    print(f'fused dit elementwise S={S} C={C}', flush=True)
    import torch.nn.functional as F
    g = torch.Generator(device=DEV).manual_seed(S)
    x = (torch.randn(S, C, generator=g, device=DEV) * 2 + 0.5).to(torch.bfloat16)
    a = torch.randn(S, C, generator=g, device=DEV).to(torch.bfloat16)
    scale, shift, gate = (0.3 * torch.randn(1, C, generator=g, device=DEV) for _ in range(3))
    w, b = 1 + 0.1 * torch.randn(C, generator=g, device=DEV), 0.1 * torch.randn(C, generator=g, device=DEV)
    cases = [(WD.layernorm_modulate(x, 1e-6, scale=scale, shift=shift),
              (F.layer_norm(x.float(), (C,), eps=1e-6) * (1 + scale) + shift).to(torch.bfloat16)),
             (WD.layernorm_modulate(x, 1e-6, weight=w, bias=b),
              F.layer_norm(x.float(), (C,), w, b, 1e-6).to(torch.bfloat16))]
    for got, ref in cases:
        diff = (got.float() - ref.float()).abs()
        assert (diff <= ref.float().abs() * 2 ** -7 + 1e-6).all(), diff.max()
        assert (got.view(torch.int16) == ref.view(torch.int16)).float().mean() > 0.99
    for gt in (gate, None):
        ref = (x.float() + a.float() * gt).to(torch.bfloat16) if gt is not None else x + a
        y = x.clone()
        WD.gated_residual_(y, a, gt)
        assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


@pytest.mark.parametrize('S,C', [(257, 3072), (64, 512), (9, 1000), (5, 4096), (3, 5120)])
def test_fused_residual_layernorm_matches_two_passes(S, C):
    """x += a [* gate] with the following LayerNorm in one pass: x and the normalised rows bit-equal to
    gated_residual_ then layernorm_modulate, with and without gate, modulation or affine weights; strided rows
    (a view of a wider buffer); C over 4096 takes the two-pass path"""
    print(f'fused residual + layernorm S={S} C={C}', flush=True)
    g = torch.Generator(device=DEV).manual_seed(C + S)
    x0 = (torch.randn(S, C + 64, generator=g, device=DEV) * 2 + 0.5).to(torch.bfloat16)
    a = torch.randn(S, C, generator=g, device=DEV).to(torch.bfloat16)
    scale, shift, gate = (0.3 * torch.randn(1, C, generator=g, device=DEV) for _ in range(3))
    w, b = 1 + 0.1 * torch.randn(C, generator=g, device=DEV), 0.1 * torch.randn(C, generator=g, device=DEV)
    for gt, prm in ((gate, dict(scale=scale, shift=shift)), (None, dict(weight=w, bias=b)), (gate, {})):
        ref_buf, buf = x0.clone(), x0.clone()
        x_ref, x = ref_buf[:, :C], buf[:, :C]          # rows of C inside rows of C + 64
        WD.gated_residual_(x_ref, a, gt)
        n_ref = WD.layernorm_modulate(x_ref, 1e-6, **prm)
        n = WD.residual_layernorm_modulate_(x, a, 1e-6, gate=gt, **prm)
        assert torch.equal(buf.view(torch.int16), ref_buf.view(torch.int16))    # the padding columns untouched too
        assert torch.equal(n.view(torch.int16), n_ref.view(torch.int16))


def test_linear_gelu_epilogue_matches_unfused():
    """the feed-forward's GEMM with GELU (tanh) in the epilogue against linear then GELU: as close to the fp32
    result as the unfused bf16 path, and within two bf16 steps of it"""
    print('linear gelu epilogue', flush=True)
    g = torch.Generator(device=DEV).manual_seed(11)
    lin = WD.Linear(512, 1024, 0.05, g, DEV)
    x = torch.randn(2, 300, 512, generator=g, device=DEV).to(torch.bfloat16)
    got = lin.gelu_tanh(x)
    ref = torch.nn.functional.gelu(lin(x), approximate='tanh')
    assert got.shape == ref.shape == (2, 300, 1024) and got.dtype == torch.bfloat16
    exact = torch.nn.functional.gelu(x.float() @ lin.weight.float().t() + lin.bias.float(), approximate='tanh')
    err_got, err_ref = (got.float() - exact).abs().max().item(), (ref.float() - exact).abs().max().item()
    assert err_got <= 1.5 * err_ref + 1e-3, (err_got, err_ref)
    assert ((got.float() - ref.float()).abs() <= ref.float().abs() * 2 ** -6 + 2e-3).all()


@pytest.mark.parametrize('S,C', [(300, 3072), (17, 512)])
def test_rms_norm_matches_torch(S, C):
    """the cross-attention's RMSNorm (or_rmsnorm_rope without tables) against torch's rms_norm: within one bf16 step
    and > 99% bit-equal"""
    print(f'rms_norm S={S} C={C}', flush=True)
    from onereel_amd import wan
    g = torch.Generator(device=DEV).manual_seed(C + S)
    x = (torch.randn(S, C, generator=g, device=DEV) * 3).to(torch.bfloat16)
    w = (1 + 0.1 * torch.randn(C, generator=g, device=DEV)).to(torch.bfloat16)
    got = wan.rms_norm(x, w, 1e-6)
    ref = torch.nn.functional.rms_norm(x.float(), (C,), w.float(), 1e-6).to(torch.bfloat16)
    diff = (got.float() - ref.float()).abs()
    assert (diff <= ref.float().abs() * 2 ** -7 + 1e-6).all(), diff.max()
    assert (got.view(torch.int16) == ref.view(torch.int16)).float().mean() > 0.99

