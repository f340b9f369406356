"""GPU check of bench.py's measurement kernel (libonereel_bench.so): the register-only MFMA loop really multiplies
the operands it loads, and its softmax mode really exponentiates its scores.

The sum of every element of an MFMA's output is sum_k colsum(A)[k] * rowsum(B)[k], and in both bf16 shapes a lane
holds A and B values at the same k (lane group g = lane // 32 for 32x32x16, lane // 16 for 16x16x32, element e at
k = 8 g + e), whatever rows and columns it holds. So the sum of the kernel's outputs over a wavefront is fixed by the
operand vectors each lane loads and the order in which the loop pairs them, independently of the output layout.
Mode 2 adds each thread's row sums of 2^(c s) over its scores."""
import ctypes

import pytest
import torch

from onereel_amd import _lib as L

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]


def _wave_total(a, b, group):
    """sum of all outputs of one MFMA over a wavefront: a, b [64, 8] float64 (lane, element)"""
    ca = a.view(64 // group, group, 8).sum(1)
    cb = b.view(64 // group, group, 8).sum(1)
    return float((ca * cb).sum())


def _row_sums(tid, iters):
    """mode 2's row sums of thread tid: sum over the loop of 2^(c s_i), s_i = -((7 tid + 13 i) mod 97) / 8, the score
    register i = k + 8 (r mod 2) at the k-th MFMA of pass r, each exponent argument rounded to fp32 as on the GPU"""
    c = torch.tensor(0.12752981, dtype=torch.float32)
    total = 0.0
    for r in range(8):
        for k in range(8):
            i = k + 8 * (r & 1)
            s = torch.tensor(-((tid * 7 + i * 13) % 97) * 0.125, dtype=torch.float32)
            total += 2.0 ** float(s * c)
    return total * (iters // 8)


@pytest.mark.parametrize('mode', [0, 1, 2])
def test_mfma_ceiling_sums_of_products(mode):
    blocks, iters = 2, 16
    n_vec = blocks * 256 * 16                     # every lane reads its own 16 vectors (no wrap)
    g = torch.Generator().manual_seed(5)
    ops = torch.randn(n_vec * 8, generator=g).to(torch.bfloat16)
    out = torch.full((blocks * 256,), float('nan'), device='cuda')
    d_ops = ops.cuda()
    st = torch.cuda.current_stream()
    print(f'or_mfma_ceiling mode {mode}, {blocks} blocks x {iters} iterations', flush=True)
    L.bench_check(L.bench_lib().or_mfma_ceiling(d_ops.data_ptr(), n_vec, out.data_ptr(), blocks, iters, mode,
                                                ctypes.c_void_p(st.cuda_stream)), 'or_mfma_ceiling')
    torch.cuda.synchronize()
    got = out.cpu().double().view(blocks * 4, 64).sum(1)
    v = ops.double().view(blocks * 4, 64, 16, 8)  # wave, lane, vector (a[0..7], b[0..7]), element
    group, per_r = (16, 16) if mode == 1 else (32, 8)
    for w in range(blocks * 4):
        a, b = v[w, :, :8], v[w, :, 8:]
        want, scale = 0.0, 0.0
        if mode == 2:
            want = scale = sum(_row_sums(64 * w + lane, iters) for lane in range(64))
        for _ in range(iters // 8):
            for r in range(8):
                for k in range(per_r):
                    t = _wave_total(a[:, k & 7], b[:, (k + r) & 7], group)
                    want += t
                    scale += _wave_total(a[:, k & 7].abs(), b[:, (k + r) & 7].abs(), group)
        # fp32 accumulation in another order: a few ulps of the absolute sum (operands paired in another order would
        # move the total by about 1% of it)
        assert abs(got[w].item() - want) <= 1e-4 * scale, (w, got[w].item(), want, scale)
