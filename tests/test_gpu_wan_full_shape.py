"""GPU parity of the Wan2.2-TI2V-5B path at the DiT step's own attention shape: 16 scenes x 15 latent frames x 880
tokens (22 x 40) = 211200 tokens, 24 heads x 128, frame memory 4 (src/onereel/models/wan.py:64-124,
src/onereel/attention.py:74-84):

- self-attention with the frame memory's extra frames (packed video-only scopes): at step 0 the fallback halo
  frames (2 on each side), from step 1 on the representatives {0, 80, 159, 239};
- per-scene cross-attention, scene j's queries over sentence j's 128 text rows;
- `_qk` (RMSNorm over 3072 features + interleaved RoPE) over all 211200 rows of q and k.

Inputs are bf16 N(0, 1) drawn on the GPU from a seeded generator and copied to the host for the reference. Attention
is compared on sampled query rows (every segment's first and last row and 24 more per segment) against fp32 softmax
attention of the same scopes: max-abs <= 2e-2, mean-abs <= 2e-3."""
import numpy as np
import pytest
import torch

from helpers import assert_close, attn_rows_reference, sample_rows, scope_rows_reference
from onereel_amd import wan as W
from onereel_amd.frame_memory import FrameMemory
from onereel_amd.layout import SceneLayout
from oracle import layout as OL

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]
DEV = 'cuda'
LENGTHS, T, H, D, TEXT = [15] * 16, 880, 24, 128, 128
REPS = [0, 80, 159, 239]


def _randn(shape, seed, scale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return (torch.randn(shape, generator=g, device=DEV) * scale).to(torch.bfloat16)


@pytest.fixture(scope='module')
def qkv():
    S = sum(LENGTHS) * T
    dq, dk, dv = (_randn((S, H, D), s) for s in (501, 502, 503))
    return (dq, dk, dv), tuple(x.cpu() for x in (dq, dk, dv))


def _frame_memory_layout(step):
    """the layout the Wan processor sees at `step`: halo 0, extra frames from a FrameMemory with budget 4"""
    lay = SceneLayout(list(LENGTHS), halo=0)
    fm = FrameMemory(budget=4)
    fm.reset(lay, 30)
    if step > 0:
        fm.set_representatives(REPS)
    fm.begin_step(step)
    return lay


@pytest.mark.parametrize('step', [0, 1])
def test_wan_self_attention_with_frame_memory(qkv, step):
    (dq, dk, dv), (q, k, v) = qkv
    lay = _frame_memory_layout(step)
    print(f'wan 16 x 15 x 880 self-attention, frame memory step {step}: extra[0] = {lay.extra[0]}', flush=True)
    if step == 0:
        assert lay.extra[1] == [13, 14, 30, 31]
    else:
        assert lay.extra[0] == [80, 159, 239] and lay.extra[5] == [0, 159, 239]
    ctx = W.Context(lay, T=T, text_len=TEXT)
    o = W.self_ranges(ctx, dq, dk, dv)
    sc = OL.hunyuan_scopes(OL.SceneLayout(list(LENGTHS), 0, 'adj', lay.extra), T, [0] * 16, 0, with_text=False)
    assert int(sc.cu_q[-1]) == q.shape[0]
    rows = sample_rows(sc.cu_q, 24, seed=step)
    empty = q[:0]
    ref = scope_rows_reference(sc, q, k, v, empty, empty, empty, rows, mode='none')
    assert_close(o.cpu()[torch.as_tensor(sc.q_src[rows])], ref, what=f'wan self-attention step {step}')


def test_wan_cross_attention_per_scene(qkv):
    (dq, _, _), (q, _, _) = qkv
    print('wan 16 x 15 x 880 cross-attention over 16 x 128 text rows', flush=True)
    lay = SceneLayout(list(LENGTHS), halo=0)
    ctx = W.Context(lay, T=T, text_len=TEXT)
    de, dev_ = _randn((16 * TEXT, H, D), 504), _randn((16 * TEXT, H, D), 505)
    o = W.cross_ranges(ctx, dq, de, dev_)
    cq = np.array([0] + [b * T for _, b in lay.ranges])
    rows = sample_rows(cq, 24, seed=9)
    ref = attn_rows_reference(q, de.cpu(), dev_.cpu(), cq, None, rows, k_off=[j * TEXT for j in range(16)],
                              k_len=[TEXT] * 16)
    assert_close(o.cpu()[torch.as_tensor(rows)], ref, what='wan cross-attention')


def test_wan_qk_at_full_shape():
    """_qk over 211200 x 3072 (q and k read as views of one fused projection), sampled rows against the oracle's
    fp32 restatement (at most one bf16 step apart, almost all bit-equal)"""
    from oracle import wan as OW
    S, C = sum(LENGTHS) * T, H * D
    print(f'wan _qk {S} x {C}', flush=True)
    qkv = _randn((S, 3 * C), 506, 3.0)
    g = torch.Generator(device=DEV).manual_seed(507)
    wq = (torch.rand(C, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    wk = (torch.rand(C, generator=g, device=DEV) + 0.5).to(torch.bfloat16)
    ang = torch.randn(S, D // 2, generator=g, device=DEV)
    cos, sin = ang.cos().repeat_interleave(2, 1), ang.sin().repeat_interleave(2, 1)
    qo, ko = W._qk(qkv[None, :, :C], qkv[None, :, C:2 * C], wq, wk, 1e-6, cos[None, :, None], sin[None, :, None], H)
    assert qo.shape == (1, S, H, D)
    rows = torch.as_tensor(np.unique(np.concatenate([[0, S - 1], np.random.default_rng(8).integers(0, S, 3000)])))
    x = qkv[rows.to(DEV)].cpu()
    c, s = cos[rows.to(DEV)].cpu(), sin[rows.to(DEV)].cpu()
    for got, xs, w in ((qo, x[:, :C], wq), (ko, x[:, C:2 * C], wk)):
        ref = OW.qk_norm_rope(xs, w.cpu(), 1e-6, c, s, H)
        got = got[0][rows.to(DEV)].cpu()
        diff = (got.float() - ref.float()).abs()
        assert (diff <= ref.float().abs() * 2 ** -7 + 1e-6).all(), diff.max()
        assert (got.view(torch.int16) == ref.view(torch.int16)).float().mean() > 0.99
