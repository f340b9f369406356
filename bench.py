"""Benchmark: one scene-structured attention layer at the HunyuanVideo-1.5 480p 4-scene shape on one MI355X.

Workload (one step = one pass of the hot path over one layer's synthetic inputs, already resident in HBM):
4 scenes x 8 latent frames x 1590 tokens (30 x 53 latent grid) + 128 text tokens per scene, frame memory of 4 frames
(representatives {0, 10, 21, 31}), shared frames at their adjacent positions (step >= shared_switch 5), scene RoPE
over a 3D table, 16 heads x 128, bf16 q / k / v ~ N(0, 1). A step runs the layout kernel, one pack launch (the keys
with RoPE, each scene's text segment reading its keys in place from its video segment's packed rows; the values the
attention does not read in place; the RoPE of the video queries, once, in token order), the varlen attention
(queries, each scope's own-frame values and the outputs in place) and the text-padding write-back (none here).

value = useful attention TFLOP/s of the whole step (sum over scopes of 4 * Lq * Lk * H * D per step time), timed
over `steps` steps after `warmup` untimed ones; before those, once per process, 0.3 s of untimed steps bring the GPU
to its steady clock (the first calls of a fresh process run up to 20% slower).
roofline: the attention kernel alone, timed with HIP events on the stream it runs on.
cpu_baseline: the oracle's packing plus torch SDPA per scope in fp32 on the host cores, on a sample of heads.
gemm_reference: torch.matmul (hipBLASLt) of two bf16 16384 x 16384 N(0, 1) matrices in the same run: what the
vendor's dense bf16 GEMM reaches on this GPU with data of the same distribution. MI355X throttles its clock under
MFMA load (power and current management), and MFMA power depends on the operand bits, so this is the practical MFMA
ceiling here.
mfma_ceiling: a loop of nothing but bf16 MFMAs on N(0, 1) operands held in registers (libonereel_bench.so), one
wavefront per SIMD on every CU, in the same run: what the matrix cores sustain at the throttled clock with no memory
traffic, LDS or softmax at all; and the same loop with an exact softmax's VALU work per MFMA beside it (the
exponential, its scale, the row sum, the bf16 conversion); attention_frac and attention_frac_of_softmax_valu are the
attention kernel's rate over each.
copy_reference: a device-to-device copy of the pack's size (torch copy_) with cold caches, in the same run: the
practical ceiling of the HBM-bound pack and scatter kernels.

    python bench.py [--gpus 1] [--steps 20] [--warmup 3] [--no-cpu] [--no-gemm-ref]

--share R/P runs one rank's share of the layer instead (rank R of P work-balanced video-token ranges): the step a
rank of a P-GPU run computes once its K/V rows are local, on this one GPU.
"""
from __future__ import annotations

import argparse
import ctypes
import hashlib
import json
import os
import platform
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = 'scene-attn TFLOP/s & % bf16 MFMA peak; ms/layer, HunyuanVideo-1.5 480p 4-scene'
PEAK_BF16_TFLOPS = 2516.6      # MI355X dense bf16 MFMA (256 CU x 2.4 GHz x 4096 FLOP/clk)
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E
# the sources of the attention kernel: profiles/attention_traffic.json holds their digest at the measured commit, and
# its HBM traffic is reported only while they are unchanged
ATTN_SOURCES = ['onereel_amd/csrc/attention.hip', 'onereel_amd/csrc/gen_attn_ring64.py', 'onereel_amd/csrc/common.h']


def attn_sources_digest():
    h = hashlib.sha256()
    for f in ATTN_SOURCES:
        h.update((ROOT / f).read_bytes())
    return h.hexdigest()[:16]

LENGTHS, T, COUNTS, H, D = [8, 8, 8, 8], 1590, [128] * 4, 16, 128
REPS = [0, 10, 21, 31]
GRID = (32, 30, 53)


UNEVEN = ['uneven2', 'uneven4', 'uneven8', 'uneven12']


def workload(name):
    """scene-attention layer shapes: the HunyuanVideo-1.5 480p layer (the default and headline), the Wan2.2 704x1280
    joint scopes, and the uneven sweep points with K = 2, 4, 8 or 12 scenes (lengths in [2, 16] frames and text counts
    in [64, 256] drawn from numpy's generator seeded K)"""
    if name == 'hunyuan480p':
        return dict(workload='hunyuan15-480p-4scene-scene-attention-layer', lengths=LENGTHS, T=T, counts=COUNTS, H=H,
                    D=D, halo=0, sides='adj', reps=REPS, grid=GRID, scene_rope=True, adjacent=True)
    if name == 'wan704':
        return dict(workload='wan22-704x1280-3scene-joint-scope-attention-layer', lengths=[11] * 3, T=880,
                    counts=[128] * 3, H=24, D=128, halo=2, sides='next', reps=None, grid=(33, 22, 40),
                    scene_rope=False, adjacent=False)
    if name in UNEVEN:
        import numpy as np
        K = int(name[len('uneven'):])
        rng = np.random.default_rng(K)
        lengths = rng.integers(2, 17, K).tolist()
        counts = rng.integers(64, 257, K).tolist()
        F = sum(lengths)
        reps = sorted({int(x) for x in np.linspace(0, F - 1, 4).round()})
        return dict(workload=f'uneven-{K}-scene-sweep-attention-layer', lengths=lengths, T=1590, counts=counts, H=16,
                    D=128, halo=0, sides='adj', reps=reps, grid=(F, 30, 53), scene_rope=True, adjacent=True)
    raise ValueError(name)


def rope_table(F, Hh, Ww, D, theta=1e4):
    """3D RoPE table (temporal / height / width pair groups, interleaved real pairs), fp32 [F*Hh*Ww, D]"""
    import torch
    f, y, x = torch.meshgrid(torch.arange(F), torch.arange(Hh), torch.arange(Ww), indexing='ij')
    nt, ny = D // 8, 3 * D // 16
    groups = [(f, nt), (y, ny), (x, D // 2 - nt - ny)]
    ang = torch.cat([p.reshape(-1, 1).float() * (theta ** (-torch.arange(n).float() / n)) for p, n in groups], 1)
    return ang.cos().repeat_interleave(2, 1).contiguous(), ang.sin().repeat_interleave(2, 1).contiguous()


def extra_from_reps(lengths, reps):
    out, lo = {}, 0
    for j, n in enumerate(lengths):
        out[j] = sorted(f for f in reps if not lo <= f < lo + n)
        lo += n
    return out


def time_events(fn, reps, stream):
    import torch
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for _ in range(reps):
        fn()
    b.record(stream)
    b.synchronize()
    return a.elapsed_time(b) / reps


def time_cold(fn, reps, stream, flush):
    """average duration of `reps` single calls, each after `flush` (not timed) evicted the L2 and the 256 MB last-level
    cache, so that an HBM-bound kernel reads its inputs from HBM rather than from data the previous call left"""
    import torch
    total = 0.0
    for _ in range(reps):
        flush()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        fn()
        b.record(stream)
        b.synchronize()
        total += a.elapsed_time(b)
    return total / reps


def gemm_reference(n=16384, reps=5):
    """TFLOP/s of torch.matmul on bf16 N(0, 1) n x n matrices (hipBLASLt), best of three timings of `reps` calls"""
    import torch
    g = torch.Generator(device='cuda').manual_seed(1)
    a = torch.randn(n, n, generator=g, device='cuda').to(torch.bfloat16)
    b = torch.randn(n, n, generator=g, device='cuda').to(torch.bfloat16)
    c = a @ b
    torch.cuda.synchronize()
    st = torch.cuda.current_stream()
    ms = min(time_events(lambda: torch.matmul(a, b, out=c), reps, st) for _ in range(3))
    tflops = 2.0 * n ** 3 / ms / 1e9
    del a, b, c
    torch.cuda.empty_cache()
    return dict(what=f'torch.matmul bf16 {n}x{n}x{n}, N(0,1) inputs (hipBLASLt), same run', ms=round(ms, 4),
                tflops=round(tflops, 1), frac_bf16_peak=round(tflops / PEAK_BF16_TFLOPS, 4))


def mfma_ceiling_call(mode=0, iters=80000):
    """(call, FLOP per call) of or_mfma_ceiling: one work-group of four wavefronts per CU, each running `iters`
    iterations of 8 bf16 MFMAs on N(0, 1) operands held in registers (~12-16 ms per call at the throttled clock);
    mode 2 adds an exact softmax's VALU work per MFMA"""
    import torch
    from onereel_amd import _lib as L
    blocks = torch.cuda.get_device_properties(0).multi_processor_count
    g = torch.Generator(device='cuda').manual_seed(2)
    ops = torch.randn(1 << 19, generator=g, device='cuda').to(torch.bfloat16)   # 65536 vectors of 8
    out = torch.empty(blocks * 256, dtype=torch.float32, device='cuda')
    st = torch.cuda.current_stream()

    def call():
        L.bench_check(L.bench_lib().or_mfma_ceiling(ops.data_ptr(), ops.numel() // 8, out.data_ptr(), blocks, iters,
                                                    mode, ctypes.c_void_p(st.cuda_stream)), 'or_mfma_ceiling')
    return call, float(blocks) * 4 * iters * 8 * 32768


def mfma_ceiling(reps=10):
    """TFLOP/s of the register-only MFMA loop (libonereel_bench.so) in both bf16 MFMA shapes, and in the attention
    kernel's shape beside an exact softmax's VALU work per MFMA (one v_mul_f32, one v_exp_f32, one v_add_f32, half a
    v_cvt_pk_bf16_f32: what the attention kernel does per score), best of three timings of `reps` calls after three
    warm-up calls: what the matrix cores sustain on this GPU at its throttled clock with N(0, 1) operands"""
    import torch
    st = torch.cuda.current_stream()
    res = {}
    for mode, name in ((0, '32x32x16'), (1, '16x16x32'), (2, 'softmax_valu')):
        call, fl = mfma_ceiling_call(mode)
        for _ in range(3):
            call()
        torch.cuda.synchronize()
        ms = min(time_events(call, reps, st) for _ in range(3))
        res[name] = (ms, fl / ms / 1e9)
    ms, tf = res['32x32x16']
    return dict(what='register-only loop of v_mfma_f32_32x32x16_bf16 (the attention kernel\'s MFMA) on N(0,1) bf16 '
                     'operands, one wavefront per SIMD on every CU, no memory traffic, same run',
                ms=round(ms, 4), tflops=round(tf, 1), frac_bf16_peak=round(tf / PEAK_BF16_TFLOPS, 4),
                tflops_16x16x32=round(res['16x16x32'][1], 1),
                tflops_with_softmax_valu=round(res['softmax_valu'][1], 1))


def copy_reference(nbytes, reps, stream, flush):
    """GB/s of a device-to-device copy of `nbytes` (torch copy_, the runtime's blit kernel), each call after a cache
    eviction: what a plain read + write stream of the pack's size reaches on this GPU"""
    import torch
    src = torch.ones(nbytes // 2, dtype=torch.int16, device='cuda')
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    ms = time_cold(lambda: dst.copy_(src), reps, stream, flush)
    gbs = 2 * (nbytes // 2) * 2 / ms / 1e6
    del src, dst
    torch.cuda.empty_cache()
    return dict(what=f'device copy of {nbytes / 1e9:.3f} GB (torch copy_), cold caches, same run', ms=round(ms, 4),
                gbs=round(gbs, 1), frac_hbm_peak=round(gbs / PEAK_HBM_GBS, 4))


def cpu_baseline(heads=16, runs=3):
    """the oracle's packing + per-scope fp32 SDPA on the host CPU, for `heads` of the 16 heads (median of runs)"""
    import numpy as np
    import torch
    from oracle import attention as OA
    from oracle import layout as OL
    torch.set_num_threads(os.cpu_count())
    lay = OL.SceneLayout(LENGTHS, halo=0, extra=extra_from_reps(LENGTHS, REPS))
    S, Le = sum(LENGTHS) * T, sum(COUNTS)
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(S, heads, D, generator=g) for _ in range(3))
    eq, ek, ev = (torch.randn(Le, heads, D, generator=g) for _ in range(3))
    cos, sin = rope_table(*GRID, D)

    def run():
        sc = OL.hunyuan_scopes(lay, T, COUNTS, Le, scene_rope=True, adjacent=True)
        qp, kp, vp = OA.pack(sc, q, k, v, eq, ek, ev, cos, sin, mode='raw')
        OA.packed_attention(qp, kp, vp, sc.cu_q, sc.cu_k)
        return sc

    sc = run()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        run()
        ts.append(time.perf_counter() - t0)
    t = float(np.median(ts))
    flops = OA.useful_flops(sc.lq, sc.lk, heads, D)
    cpu = platform.processor() or ''
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name'):
                cpu = line.split(':', 1)[1].strip()
                break
    except OSError:
        pass
    return dict(value=round(flops / t / 1e12, 4), unit='TFLOP/s', cores=torch.get_num_threads(), kind='port',
                sample=f'the full HunyuanVideo-1.5 480p 4-scene layer (layout, packing with RoPE, fp32 SDPA per scope) for {heads} of {H} heads; '
                       f'median of {runs} runs after 1 warm-up: {t:.2f} s on {os.cpu_count()} logical CPUs ({cpu})',
                seconds=round(t, 3))


def run_dit(args):
    """one forward of a random-init Wan2.2-TI2V-5B-shaped DiT (30 blocks, hidden 3072 = 24 x 128, FFN 14336, bf16
    weights N(0, 0.02)) over 16 scenes x 15 latent frames x 880 tokens (22 x 40 grid) with frame memory 4 and 128
    text tokens per scene: end-to-end ms per step (one transformer pass; classifier-free guidance would double it)"""
    import torch
    from onereel_amd import wan_dit as WD
    from onereel_amd.layout import SceneLayout
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    lengths, Tw, text_len, grid = [15] * 16, 880, 128, (240, 22, 40)
    F = sum(lengths)
    reps = sorted({int(round(x)) for x in [i * (F - 1) / 3 for i in range(4)]})
    lay = SceneLayout(lengths, halo=0, extra=extra_from_reps(lengths, reps))
    cfg = WD.DiTConfig()
    model = WD.WanDiT(cfg, lay, Tw, text_len, dev, seed=0)
    g = torch.Generator(device=dev).manual_seed(0)
    S = F * Tw
    tokens = torch.randn(S, cfg.in_channels * cfg.patch, generator=g, device=dev).to(torch.bfloat16)
    text = torch.randn(len(lengths) * text_len, cfg.text_dim, generator=g, device=dev).to(torch.bfloat16)
    rot = tuple(x.to(dev) for x in WD.wan_rope_table(*grid, cfg.dim // cfg.heads))
    steps = args.steps if args.steps is not None else 3
    warmup = args.warmup if args.warmup is not None else 1
    for _ in range(warmup):
        model.forward(tokens, 500.0, text, rot)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        model.forward(tokens, 500.0, text, rot)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    # one more pass with events around the attention processors (outside the timed steps)
    marks = {'self': [], 'cross': []}

    def timed(kind, fn):
        def run(*a, **kw):
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            out = fn(*a, **kw)
            e1.record()
            marks[kind].append((e0, e1))
            return out
        return run
    p_self, p_cross = model.p_self, model.p_cross
    model.p_self, model.p_cross = timed('self', p_self), timed('cross', p_cross)
    model.forward(tokens, 500.0, text, rot)
    torch.cuda.synchronize()
    model.p_self, model.p_cross = p_self, p_cross
    attn_ms = {k: sum(a.elapsed_time(b) for a, b in v) for k, v in marks.items()}
    fl = model.flops(len(lengths) * text_len)
    total = sum(fl.values())
    out = dict(metric='Wan2.2-TI2V-5B-shaped DiT forward, ms/step (16 scenes x 15 frames x 880 tokens, frame memory 4)',
               value=round(ms, 2), unit='ms', n_gpus=1, steps=steps, warmup=warmup, ms_per_step=round(ms, 2),
               higher_is_better=False, scaling='weak', vs_baseline=None, dtype='bf16',
               data='synthetic latent, text and timestep; random-init N(0, 0.02) bf16 weights',
               config=dict(workload='wan22-ti2v-5b-dit-forward-16scene', blocks=cfg.blocks, hidden=cfg.dim,
                           heads=cfg.heads, head_dim=cfg.dim // cfg.heads, ffn=cfg.ffn, scenes=len(lengths),
                           frames_per_scene=15, tokens_per_frame=Tw, tokens=S, text_per_scene=text_len,
                           frame_memory=reps, classifier_free_guidance=False),
               flop_per_step={k: float(v) for k, v in fl.items()}, tflops=round(total / ms / 1e9, 1),
               attention_ms=dict(self_processors=round(attn_ms['self'], 2), cross_processors=round(attn_ms['cross'], 2),
                                 what='processor calls: QKV / output projections, _qk, layout, pack and varlen '
                                      'kernels (self); projections and varlen (cross)'))
    print(json.dumps(out), flush=True)


def run_lse_merge(args):
    """the log-sum-exp merge of a partial attention result into a running one at the HunyuanVideo-1.5 480p layer's
    packed shape (51 392 rows x 16 heads x 128): o fp32 read and written, o_s bf16 read, lse / lse_s fp32; each call
    timed alone with the caches evicted before it"""
    import torch
    from onereel_amd import attention as A
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    N, H_, D_ = 51392, 16, 128
    g = torch.Generator(device=dev).manual_seed(0)
    o = torch.randn(N, H_, D_, generator=g, device=dev)
    o_s = torch.randn(N, H_, D_, generator=g, device=dev).to(torch.bfloat16)
    lse = torch.randn(H_, N, generator=g, device=dev) + 9.0
    lse_s = torch.randn(H_, N, generator=g, device=dev) + 9.0
    st = torch.cuda.current_stream(dev)
    evict = torch.ones(128 << 20, dtype=torch.int32, device=dev)
    flush = lambda: evict.sum()
    A.merge_lse(o, lse, o_s, lse_s)
    torch.cuda.synchronize()
    t = time_cold(lambda: A.merge_lse(o, lse, o_s, lse_s), args.kernel_reps, st, flush)
    nbytes = N * H_ * D_ * (4 + 4 + 2) + N * H_ * 4 * 3
    gbs = nbytes / t / 1e6
    out = dict(metric='LSE merge of a partial attention result: GB/s and % of HBM peak', value=round(gbs, 1),
               unit='GB/s', n_gpus=1, steps=args.kernel_reps, warmup=1, ms_per_step=round(t, 4), higher_is_better=True,
               scaling='weak', vs_baseline=None, dtype='fp32', data='synthetic',
               config=dict(workload='lse-merge-hunyuan15-480p-packed-rows', rows=N, heads=H_, head_dim=D_),
               roofline=dict(bound='hbm', achieved=round(gbs, 1), peak=PEAK_HBM_GBS, unit='GB/s',
                             frac=round(gbs / PEAK_HBM_GBS, 4), traffic=None, kernel='lse_merge_kernel + lse_update_kernel'),
               bytes=nbytes, timing='cold caches, single calls')
    print(json.dumps(out), flush=True)


def run_bounded_memory(args):
    """the bounded memory (per-head boundary-frame representatives, M = 128) at the HunyuanVideo-1.5 480p layer's
    shape: one layer call = representative choice (warm-started k-means) + the foreign representatives' index arrays +
    the pack of the local rows past each piece's in-place run and of the representatives + one multi-head varlen call
    (local keys and values of the leading run read in place), timed in steady state: after the first call, whose
    k-means runs 50 iterations, and `warmup` (default 3) more calls"""
    import torch
    import torch.nn.functional as F
    from onereel_amd.layout import SceneLayout
    from onereel_amd.memory import BoundaryMemory, MemoryAttention, frame_plan
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    lay = SceneLayout(LENGTHS, halo=0)
    S, Le = lay.n_frames * T, sum(COUNTS)
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn(S + Le, H, D, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    tr, c = [], 0
    for n in COUNTS:
        tr.append((c, c + n))
        c += n
    plan = frame_plan(lay, T, torch.arange(S), S, [(j, lo * T, hi * T) for j, (lo, hi) in enumerate(lay.ranges)], tr,
                      set(range(lay.n_scenes)), S, dev)
    M = 128
    mem = MemoryAttention(BoundaryMemory(M))
    key = ('layer', True)
    st = torch.cuda.current_stream(dev)
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(st)
    mem(key, q, k, v, plan)
    b.record(st)
    b.synchronize()
    t_first = a.elapsed_time(b)
    warm = 3 if args.warmup is None else args.warmup
    for _ in range(warm):
        mem(key, q, k, v, plan)
    reps = max(3, args.kernel_reps)
    t_call = time_events(lambda: mem(key, q, k, v, plan), reps, st)
    # useful FLOPs of the attention: each piece and head reads its local keys plus the foreign representatives
    rep, valid = BoundaryMemory(M).select(key, k[plan.cand])
    rep_scene = plan.owner[rep]
    foreign = valid[:, None, :] & (rep_scene[:, None, :] != plan.scene[None, :, None]) & plan.mem[None, :, None]
    lk = (plan.lens[None] + foreign.sum(-1)).double()
    flops = float((4.0 * plan.qlen[None].double() * lk * D).sum())
    out = dict(metric='bounded memory layer: ms per call and attention TFLOP/s', value=round(t_call, 4), unit='ms',
               n_gpus=1, steps=reps, warmup=1 + warm, ms_per_step=round(t_call, 4), higher_is_better=False,
               scaling='weak', vs_baseline=None, dtype='bf16', data='synthetic',
               config=dict(workload='bounded-memory-hunyuan15-480p-4scene', scenes=len(LENGTHS), tokens_per_frame=T,
                           text_per_scene=COUNTS, heads=H, head_dim=D, representatives=M),
               first_call_ms=round(t_first, 4), useful_flop=flops, tflops=round(flops / t_call / 1e9, 1))
    print(json.dumps(out), flush=True)


def run_power(args):
    """board power and clocks while the headline layer's attention kernel runs back to back (about 8 s), then while
    the bf16 GEMM reference does, then the attention kernel again on operands with two mantissa bits, then the
    register-only MFMA loop alone and beside an exact softmax's VALU work (or_mfma_ceiling modes 0 and 2), sampled
    with amd-smi every ~0.25 s: at what power and clock each runs. One JSON line: per phase the median socket power, the mean over samples of the XCDs' mean
    clock, and the kernel's ms per call and TFLOP/s over the phase."""
    import statistics
    import subprocess
    import threading
    import torch
    from onereel_amd import scene
    from onereel_amd.layout import SceneLayout
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    W = workload('hunyuan480p')
    lay = SceneLayout(W['lengths'], halo=0, extra=extra_from_reps(W['lengths'], W['reps']))
    S, Le = sum(W['lengths']) * W['T'], sum(W['counts'])
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn(S, H, D, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    eq, ek, ev = (torch.randn(Le, H, D, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    cos, sin = (x.to(dev) for x in rope_table(*W['grid'], D))
    plan = scene.ScopePlan(lay, W['T'], W['counts'], Le, True, None, True, True, dev, text_keys_in_place=True)
    kp, vp = scene.pack_rows(plan, k, ek, 'k', b_video=v, b_text=ev, cos=cos, sin=sin, mode='raw')
    ov = torch.empty_like(q)
    ot = torch.empty(Le, H, D, dtype=torch.bfloat16, device=dev)
    ws = plan.workspace(H, D)
    lq = [int(x) for x in (plan.cu_q[1:] - plan.cu_q[:-1]).tolist()]
    lk = [int(x) for x in plan.k_len.tolist()]
    flops = float(sum(4.0 * a * b * H * D for a, b in zip(lq, lk)))
    qr = scene.rotate_queries(plan, q, cos, sin)
    attn = lambda: scene.varlen(qr, kp, vp, plan.cu_q, plan.cu_k, plan.max_q, plan.max_k, k_off=plan.k_off,
                                k_len=plan.k_len, out=ov, seg_q_src=plan.seg_q_src, q_text=eq, o_text=ot,
                                n_q_video=plan.n_video, sum_q=plan.sum_q, workspace=ws)
    # the same call on operands with two mantissa bits (bf16 bits 4..0 cleared): the same FLOP and schedule, less
    # MFMA switching power, so the rate it reaches at the board's limit shows how much power bounds the kernel
    low = lambda x: (x.view(torch.int16) & -32).view(torch.bfloat16)
    qr2, kp2, vp2, eq2 = low(qr), low(kp), low(vp), low(eq)
    attn2 = lambda: scene.varlen(qr2, kp2, vp2, plan.cu_q, plan.cu_k, plan.max_q, plan.max_k, k_off=plan.k_off,
                                 k_len=plan.k_len, out=ov, seg_q_src=plan.seg_q_src, q_text=eq2, o_text=ot,
                                 n_q_video=plan.n_video, sum_q=plan.sum_q, workspace=ws)
    n_g = 16384
    a = torch.randn(n_g, n_g, generator=g, device=dev).to(torch.bfloat16)
    b = torch.randn(n_g, n_g, generator=g, device=dev).to(torch.bfloat16)
    c = a @ b
    gemm = lambda: torch.matmul(a, b, out=c)
    samples, phase, stop = [], ['idle'], threading.Event()

    def sample():
        while not stop.is_set():
            try:
                r = subprocess.run(['amd-smi', 'metric', '-g', '0', '-p', '-c', '--json'], capture_output=True,
                                   text=True, timeout=10)
                d = json.loads(r.stdout)
                d = d['gpu_data'][0] if isinstance(d, dict) else d[0]
                clk = [x['clk']['value'] for name, x in d['clock'].items() if name.startswith('gfx_')]
                samples.append((phase[0], float(d['power']['socket_power']['value']), sum(clk) / len(clk)))
            except Exception as e:      # no amd-smi, or a format this parser does not know: no samples
                samples.append((phase[0], None, repr(e)[:200]))
                return
            time.sleep(0.25)

    th = threading.Thread(target=sample, daemon=True)
    th.start()
    time.sleep(1.5)
    out = dict(metric='board power (W) and clock (MHz) while the attention kernel and the bf16 GEMM reference run',
               unit='W', n_gpus=1, data='synthetic',
               config=dict(workload='hunyuan15-480p-4scene-attention-kernel-vs-gemm16384', sampler='amd-smi metric '
                           '-p -c, every ~0.25 s'))
    ceil, ceil_fl = mfma_ceiling_call(0)
    ceil2, ceil2_fl = mfma_ceiling_call(2)
    for name, fn, fl in (('attention', attn, flops), ('gemm_reference', gemm, 2.0 * n_g ** 3),
                         ('attention_two_mantissa_bits', attn2, flops), ('mfma_ceiling', ceil, ceil_fl),
                         ('mfma_ceiling_with_softmax_valu', ceil2, ceil2_fl)):
        fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        phase[0] = 'warm'
        t_end, n = time.perf_counter() + 1.0, 0
        while time.perf_counter() < t_end:   # one second to reach the limit before sampling
            fn()
            torch.cuda.synchronize()
        phase[0] = name
        e0.record()
        t_end = time.perf_counter() + 8.0
        while time.perf_counter() < t_end:
            for _ in range(20):
                fn()
            n += 20
            torch.cuda.synchronize()
        e1.record()
        phase[0] = 'idle'
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / n
        got = [(p_, c_) for ph, p_, c_ in samples if ph == name and p_ is not None]
        out[name] = dict(ms=round(ms, 4), tflops=round(fl / ms / 1e9, 1), calls=n, samples=len(got),
                         socket_power_w=statistics.median([p_ for p_, _ in got]) if got else None,
                         mean_gfx_clock_mhz=round(sum(c_ for _, c_ in got) / len(got), 1) if got else None)
        time.sleep(1.5)
    stop.set()
    th.join(timeout=15)
    idle = [p_ for ph, p_, _ in samples if ph == 'idle' and p_ is not None]
    out['idle_socket_power_w'] = statistics.median(idle) if idle else None
    errs = [c_ for _, p_, c_ in samples if p_ is None]
    if errs:
        out['sampler_error'] = errs[0]
    out['value'] = out['attention']['socket_power_w']
    print(json.dumps(out), flush=True)


def run_frame_memory(args):
    """frame memory at the DiT-step shape: pooling of one observed layer (16 scenes x 15 frames x 880 tokens x 3072
    bf16, 1.3 GB) per frame, and the k-means choice of 4 representatives among the 240 frames; each call timed alone
    with the caches evicted before it"""
    import torch
    from onereel_amd.frame_memory import FrameMemory
    from onereel_amd.layout import SceneLayout
    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    lengths, Tw, C = [15] * 16, 880, 3072
    lay = SceneLayout(lengths, halo=0)
    S = lay.n_frames * Tw
    g = torch.Generator(device=dev).manual_seed(0)
    hs = torch.randn(S, C, generator=g, device=dev).to(torch.bfloat16)
    frame = torch.arange(S, device=dev) // Tw
    fm = FrameMemory(budget=4)
    fm.reset(lay, 30)
    st = torch.cuda.current_stream(dev)
    evict = torch.ones(128 << 20, dtype=torch.int32, device=dev)
    flush = lambda: evict.sum()
    reps = args.kernel_reps

    def pool():
        fm.sums, fm.counts = {}, {}
        fm.collect(frame, hs, layer=15)
    pool()
    torch.cuda.synchronize()
    # the sums buffers are allocated inside collect; time the kernel on preallocated buffers
    sums, counts = fm.sums[15], fm.counts[15]
    from onereel_amd import _lib as L
    row0, T_ = fm.frame_layout(frame)
    call = lambda: L.check(L.lib().or_frame_pool(hs.data_ptr(), S, C, hs.stride(0), row0, T_, lay.n_frames,
                                                 sums.data_ptr(), counts.data_ptr(), st.cuda_stream), 'or_frame_pool')
    t_pool = time_cold(call, reps, st, flush)
    feats = torch.nn.functional.normalize(torch.randn(lay.n_frames, C, generator=g, device=dev), dim=-1)
    fm.select(feats)
    torch.cuda.synchronize()
    t_sel = time_cold(lambda: fm.select(feats), reps, st, flush)
    nbytes = S * C * 2
    out = dict(metric='frame memory: per-frame pooling GB/s and k-means selection us (240 frames, 3072 features)',
               value=round(nbytes / t_pool / 1e6, 1), unit='GB/s', n_gpus=1, steps=reps, warmup=1,
               higher_is_better=True, dtype='bf16 in, fp32 sums', data='synthetic',
               config=dict(workload='frame-memory-16scene', tokens=S, features=C, frames=lay.n_frames, budget=4),
               pool=dict(ms=round(t_pool, 4), gbs=round(nbytes / t_pool / 1e6, 1),
                         frac_hbm_peak=round(nbytes / t_pool / 1e6 / PEAK_HBM_GBS, 4), bytes=nbytes),
               select=dict(us=round(t_sel * 1e3, 1), what='one or_frame_select launch plus the read-back of the 4 '
                                                          'chosen frames (host sync)'))
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=None, help='timed steps (default 20; 3 for wan-dit-step)')
    ap.add_argument('--warmup', type=int, default=None, help='untimed steps first (default 3; 1 for wan-dit-step)')
    ap.add_argument('--no-cpu', action='store_true', help='skip the CPU baseline leg')
    ap.add_argument('--kernel-reps', type=int, default=10)
    ap.add_argument('--no-gemm-ref', action='store_true', help='skip the bf16 GEMM reference')
    ap.add_argument('--workload', default='hunyuan480p',
                    choices=['hunyuan480p', 'wan704'] + UNEVEN + ['wan-dit-step', 'frame-memory', 'lse-merge',
                                                                   'bounded-memory', 'power'],
                    help='hunyuan480p (default, the headline): the HunyuanVideo-1.5 480p 4-scene layer; wan704 and '
                         'unevenK: the same layer at the Wan2.2 704x1280 shape and at the K-scene uneven sweep points '
                         '(K = 2, 4, 8, 12); wan-dit-step: '
                         'one forward of a random-init Wan2.2-TI2V-5B-shaped DiT over 16 scenes x 15 frames x 880 '
                         'tokens with frame memory 4 (end-to-end ms per step); frame-memory: the pooling and '
                         'selection kernels at that shape; lse-merge: the log-sum-exp merge at the 480p layer shape; '
                         'bounded-memory: the head-major bounded memory layer at that shape; power: board power and '
                         'clocks under the attention kernel and under the bf16 GEMM reference (amd-smi)')
    ap.add_argument('--share', default=None, metavar='R/P',
                    help="one rank's share of a layer workload: rank R of P work-balanced video-token ranges "
                         "(Algorithm 1 over the scenes' modelled query costs), its scenes' clipped queries and their "
                         "full keys, and the sentences whose scene starts in its range, run on this one GPU")
    ap.add_argument('--once', action='store_true',
                    help='profiling mode: a 1 GiB device copy (counter calibration), then the layout, pack-gather, '
                         'attention and scatter kernels once each, then one bf16 16384^3 torch.matmul (the GEMM '
                         'reference); prints nothing else')
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py measures the single-GPU scene-attention path only: run it with --gpus 1 '
              '(the multi-GPU K/V gathering and Ulysses paths are not implemented)', file=sys.stderr)
        sys.exit(2)
    if args.share:
        # argument errors before anything touches the GPU
        m = re.fullmatch(r'(\d+)/(\d+)', args.share)
        if not m or not 0 <= int(m.group(1)) < int(m.group(2)):
            raise SystemExit(f'--share {args.share}: give R/P with the rank R in [0, P)')

    if args.workload == 'wan-dit-step':
        return run_dit(args)
    if args.workload == 'frame-memory':
        return run_frame_memory(args)
    if args.workload == 'lse-merge':
        return run_lse_merge(args)
    if args.workload == 'bounded-memory':
        return run_bounded_memory(args)
    if args.workload == 'power':
        return run_power(args)
    args.steps = 20 if args.steps is None else args.steps
    args.warmup = 3 if args.warmup is None else args.warmup
    W = workload(args.workload)
    headline = args.workload == 'hunyuan480p' and args.share is None
    T_, H_, D_ = W['T'], W['H'], W['D']

    import torch
    from onereel_amd import comm, scene
    from onereel_amd.layout import SceneLayout

    dev = torch.device('cuda:0')
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    extra = extra_from_reps(W['lengths'], W['reps']) if W['reps'] else {}
    lay = SceneLayout(W['lengths'], halo=W['halo'], sides=W['sides'], extra=extra)
    q_range = None
    if args.share:
        r, P = (int(x) for x in args.share.split('/'))
        q_range = comm.partition(lay, P, T_, 'scene', W['counts'])[r]
        W['workload'] += f'-rank{r}of{P}'
    S, Le = sum(W['lengths']) * T_, sum(W['counts'])
    g = torch.Generator(device=dev).manual_seed(0)
    q, k, v = (torch.randn(S, H_, D_, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    eq, ek, ev = (torch.randn(Le, H_, D_, generator=g, device=dev).to(torch.bfloat16) for _ in range(3))
    cos, sin = (x.to(dev) for x in rope_table(*W['grid'], D_))
    # text segments read their keys in place from their scene's video segment (no packed copy)
    plan = scene.ScopePlan(lay, T_, W['counts'], Le, W['scene_rope'], None, W['adjacent'], True, dev,
                           text_keys_in_place=True, q_range=q_range)
    H, D = H_, D_
    lq = [int(x) for x in (plan.cu_q[1:] - plan.cu_q[:-1]).tolist()]
    lk = [int(x) for x in plan.k_len.tolist()]
    flops = float(sum(4.0 * a * b * H * D for a, b in zip(lq, lk)))
    kbuf = torch.empty(plan.sum_k, H, D, dtype=torch.bfloat16, device=dev)
    vbuf = torch.empty_like(kbuf)
    qbuf = torch.empty_like(q)                   # the video queries rotated once per layer

    if args.once:
        src = torch.empty(1 << 29, dtype=torch.int16, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)                           # 1 GiB read + 1 GiB written
        torch.cuda.synchronize()
        plan.build()
        ov, ot = scene.scene_attention(plan, q, k, v, eq, ek, ev, cos, sin, mode='raw', fused=True, kbuf=kbuf,
                                       vbuf=vbuf, qbuf=qbuf)
        scene.scatter(plan, torch.zeros(plan.sum_q, H, D, dtype=torch.bfloat16, device=dev), ov, ot)
        torch.cuda.synchronize()
        if headline:
            gemm_reference(reps=1)
        print('once: copy 1 GiB, layout, pack_layer, plan + attention, scatter, bf16 GEMM reference',
              flush=True)
        return

    def make_step(p):
        def step():
            p.build()
            return scene.scene_attention(p, q, k, v, eq, ek, ev, cos, sin, mode='raw', fused=True, kbuf=kbuf,
                                         vbuf=vbuf, qbuf=qbuf)
        return step

    prewarmed = []

    def time_steps(step):
        # once per process, before the first warm-up step: run the step for 0.3 s untimed. The first calls of a fresh
        # process run slower while the GPU's clock and power settle (6.4, 6.0, 5.6, 5.5 ms for the first attention
        # calls at 480p, then 5.3-5.4 ms), longer than the default warm-up of 3 steps
        if not prewarmed:
            torch.cuda.synchronize()
            t_end = time.perf_counter() + 0.3
            while time.perf_counter() < t_end:
                step()
                torch.cuda.synchronize()
            prewarmed.append(True)
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        return (time.perf_counter() - t0) * 1e3 / args.steps

    ms = time_steps(make_step(plan))
    # the other shared-frame layout of a frame-memory run: before shared_switch the shared keys keep their own
    # positions ('source'), from it on they sit next to the scene ('adjacent'); same scopes and FLOPs, other rotations
    other = None
    if W['reps'] and W['scene_rope']:
        plan_o = scene.ScopePlan(lay, T_, W['counts'], Le, W['scene_rope'], None, not W['adjacent'], True, dev,
                                 text_keys_in_place=True, q_range=q_range)
        ms_o = time_steps(make_step(plan_o))

    # per-kernel durations with HIP events on the launch stream
    R = args.kernel_reps
    ov = torch.empty_like(q)
    ot = torch.empty(Le, H, D, dtype=torch.bfloat16, device=dev)
    ws = plan.workspace(H, D)
    # the attention kernel as the step runs it: video queries already rotated (qbuf), read in place, the own-frame
    # values read in place from v
    attn_of = lambda p: (lambda: scene.varlen(qbuf, kbuf, vbuf, p.cu_q, p.cu_k, p.max_q, p.max_k, k_off=p.k_off,
                                              k_len=p.k_len, out=ov, seg_q_src=p.seg_q_src, q_text=eq, o_text=ot,
                                              n_q_video=p.n_video, sum_q=p.sum_q, workspace=ws, v_tok=v,
                                              v_lead=p.v_lead, v_row=p.v_row, v_runs=p.v_runs))
    # the step's one pack launch: K rows (rotated), the V rows not read in place, the video queries rotated once
    pack_of = lambda p: (lambda: scene.pack_layer(p, k, ek, v, ev, cos, sin, 'raw', kbuf, vbuf, q=q, qbuf=qbuf))
    attn, pack = attn_of(plan), pack_of(plan)
    qpk = torch.empty(plan.sum_q, H, D, dtype=torch.bfloat16, device=dev)
    scat = lambda: scene.scatter(plan, qpk, ov, ot)
    pack()
    attn()
    scat()
    torch.cuda.synchronize()
    t_attn = time_events(attn, R, stream)
    if W['reps'] and W['scene_rope']:
        attn_o = attn_of(plan_o)
        pack_of(plan_o)()
        attn_o()
        torch.cuda.synchronize()
        t_attn_o = time_events(attn_o, R, stream)
        pack()                                      # the adjacent layout's keys back in the buffers
        torch.cuda.synchronize()
        v_o = flops / (ms_o * 1e-3) / 1e12
        other = dict(shared_pos='source' if W['adjacent'] else 'adjacent',
                     when='denoising steps before shared_switch (5)' if W['adjacent'] else 'from shared_switch on',
                     ms_per_step=round(ms_o, 4), tflops_step=round(v_o, 2),
                     frac_bf16_peak_step=round(v_o / PEAK_BF16_TFLOPS, 4),
                     attention=dict(ms=round(t_attn_o, 4), tflops=round(flops / t_attn_o / 1e9, 1),
                                    frac_bf16_peak=round(flops / t_attn_o / 1e9 / PEAK_BF16_TFLOPS, 4)))
    # HBM-bound kernels: each call timed alone after the caches were evicted (cold), and back to back (warm: inputs
    # that fit the 256 MB last-level cache are then partly served from it)
    evict = torch.ones(128 << 20, dtype=torch.int32, device=dev)
    flush = lambda: evict.sum()   # reads 512 MB: the caches then hold clean lines of it, nothing to write back
    row = H * D * 2
    n_vq = sum(lq[0::2])                             # video query rows (the even segments)
    n_vcopy = int((plan.v_src >= 0).sum())           # value rows packed (the others are read in place)
    n_krot = int((plan.k_rope >= 0).sum())           # key rows rotated (video keys)
    # K rows, packed V rows and video Q rows each read + written, and the fp32 cos / sin rows of every rotated row
    pack_bytes = 2 * (plan.sum_k + n_vcopy + n_vq) * row + (n_krot + n_vq) * D * 8
    t_pack, t_pack_w = time_cold(pack, R, stream, flush), time_events(pack, R, stream)
    t_layout = time_cold(plan.build, R, stream, flush)
    t_scat, t_scat_w = time_cold(scat, R, stream, flush), time_events(scat, R, stream)
    copy_ref = copy_reference(pack_bytes // 2, R, stream, flush) if headline else None
    del evict
    scat_bytes = 2 * plan.sum_q * row                # packed rows read + written
    kernels = {
        'attention': dict(ms=round(t_attn, 4), tflops=round(flops / t_attn / 1e9, 1),
                          frac_bf16_peak=round(flops / t_attn / 1e9 / PEAK_BF16_TFLOPS, 4)),
        'pack_layer': dict(ms=round(t_pack, 4), gbs=round(pack_bytes / t_pack / 1e6, 1),
                           frac_hbm_peak=round(pack_bytes / t_pack / 1e6 / PEAK_HBM_GBS, 4), bytes=pack_bytes,
                           rows=dict(keys=plan.sum_k, values=n_vcopy, queries=n_vq), warm_ms=round(t_pack_w, 4),
                           timing='cold caches, single calls'),
        'layout': dict(us=round(t_layout * 1e3, 2), gbs=round(plan.index_bytes() / t_layout / 1e6, 1),
                       bytes=plan.index_bytes(),
                       bound=f'launch latency ({plan.index_bytes() / 1e6:.1f} MB of int32 indices)'),
        'scatter': dict(ms=round(t_scat, 4), gbs=round(scat_bytes / t_scat / 1e6, 1),
                        frac_hbm_peak=round(scat_bytes / t_scat / 1e6 / PEAK_HBM_GBS, 4), bytes=scat_bytes,
                        warm_ms=round(t_scat_w, 4), timing='cold caches, single calls'),
    }
    # the kernel or_varlen_fwd runs for an O-only call: the 64-query ring kernel at head_dim 128
    kname = 'attn8_kernel' if D == 128 else 'attn4_kernel<64>'
    traffic, traffic_src = None, None
    tf = ROOT / 'profiles' / 'attention_traffic.json'
    if headline and tf.exists():    # measured (PMC) on the headline layer only, for the kernel that runs
        rec = json.loads(tf.read_text())
        same = rec.get('sources_sha256') == attn_sources_digest()
        if rec.get('kernel') == kname and same:
            traffic = rec.get('hbm_bytes_per_launch')
        traffic_src = dict(commit=rec.get('commit'), sources_sha256=rec.get('sources_sha256'),
                           current_sources_sha256=attn_sources_digest(),
                           status='measured on these kernel sources' if same else
                           'kernel sources changed since the measurement: traffic not reported')
    value = flops / (ms * 1e-3) / 1e12
    metric = METRIC if headline else f'scene-attn TFLOP/s & % bf16 MFMA peak; ms/layer, {W["workload"]}'
    out = dict(metric=metric, value=round(value, 2), unit='TFLOP/s', n_gpus=1, steps=args.steps, warmup=args.warmup,
               ms_per_step=round(ms, 4), higher_is_better=True, scaling='weak', vs_baseline=None, dtype='bf16',
               data='synthetic',
               config=dict(workload=W['workload'], scenes=len(W['lengths']), frames_per_scene=W['lengths'],
                           tokens_per_frame=T_, text_per_scene=W['counts'], halo=W['halo'], sides=W['sides'],
                           frame_memory=W['reps'], shared_pos='adjacent' if W['adjacent'] else 'source',
                           scene_rope=W['scene_rope'], heads=H, head_dim=D, sum_q=plan.sum_q, sum_k=plan.sum_k,
                           video_token_range=list(q_range) if q_range else None,
                           useful_flop_per_step=flops, frac_bf16_peak_step=round(value / PEAK_BF16_TFLOPS, 4)),
               roofline=dict(bound='mfma', achieved=round(flops / t_attn / 1e9, 1), peak=PEAK_BF16_TFLOPS,
                             unit='TFLOP/s', frac=round(flops / t_attn / 1e9 / PEAK_BF16_TFLOPS, 4), traffic=traffic,
                             traffic_source=traffic_src, kernel=f'{kname} (+ plan_kernel, up to 8 blocks, ~11 us)'),
               kernels=kernels)
    if other:
        out['other_layout'] = other
    if copy_ref:
        out['copy_reference'] = copy_ref
    if headline and not args.no_gemm_ref:
        out['gemm_reference'] = gemm_reference()
        mc = out['mfma_ceiling'] = mfma_ceiling()
        mc['attention_frac'] = round(kernels['attention']['tflops'] / mc['tflops'], 4)
        mc['attention_frac_of_softmax_valu'] = round(kernels['attention']['tflops'] / mc['tflops_with_softmax_valu'], 4)
    if headline and not args.no_cpu:
        out['cpu_baseline'] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
