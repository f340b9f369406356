"""The allocation-free attention entry point (or_varlen_fwd_noalloc) against or_varlen_fwd, through the C ABI: two
calls in a row, the second smaller, each compared with the workspace entry point's output (bit-identical when that
call's workspace fits the library's array, so both plan the same key splits; within the bf16 tolerance and against
the fp32 oracle otherwise), and a call too large for the array rejected before any launch."""
import ctypes

import numpy as np
import pytest
import torch

from helpers import assert_close, rand_bf16
from onereel_amd import _lib as L
from onereel_amd import scene
from oracle import attention as OA

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not torch.cuda.is_available(), reason='needs the GPU')]
DEV = 'cuda'
SCRATCH = 32 << 20          # OR_NOALLOC_SCRATCH_BYTES


def _case(lq, lk, H, D, seed):
    q = rand_bf16((sum(lq), H, D), seed)
    k = rand_bf16((sum(lk), H, D), seed + 1)
    v = rand_bf16((sum(lk), H, D), seed + 2)
    cq = torch.tensor(np.cumsum([0] + lq), dtype=torch.int32)
    ck = torch.tensor(np.cumsum([0] + lk), dtype=torch.int32)
    return q, k, v, cq, ck


@pytest.mark.parametrize('calls', [
    # (lq, lk, H, D) of the first call, then of a smaller second call
    [([1000, 300, 2000, 0, 77], [3000, 500, 4000, 20, 900], 8, 128), ([100, 7], [900, 50], 2, 128)],
    [([12720, 128] * 2, [17618, 12848] * 2, 16, 128), ([300, 45, 129], [700, 130, 33], 3, 64)],
])
def test_noalloc_matches_workspace_entry(calls):
    for n, (lq, lk, H, D) in enumerate(calls):
        print(f'noalloc call {n}: lq={lq} lk={lk} H={H} D={D}', flush=True)
        q, k, v, cq, ck = _case(lq, lk, H, D, 70 + 5 * n)
        g = [x.to(DEV) for x in (q, k, v, cq, ck)]
        ref_out = scene.varlen(*g, max(lq), max(lk))
        # stale contents in the output rows must not survive: prefill with a value attention cannot produce
        out = torch.full_like(ref_out, 9.0)
        got = scene.varlen(*g, max(lq), max(lk), out=out, noalloc=True)
        torch.cuda.synchronize()
        assert got.data_ptr() == out.data_ptr()
        need = int(L.lib().or_varlen_workspace_size(len(lq), sum(lq), H, D))
        if need <= SCRATCH:
            assert torch.equal(got.view(torch.int16), ref_out.view(torch.int16)), 'same plan, same bits'
        else:
            assert_close(got.cpu(), ref_out.cpu().float(), what='noalloc vs workspace entry')
        rows = np.unique(np.linspace(0, sum(lq) - 1, 64).round().astype(int)) if sum(lq) > 4096 else None
        if rows is None:
            assert_close(got.cpu(), OA.packed_attention(q, k, v, cq.numpy(), ck.numpy()), what='noalloc vs oracle')
        else:
            from helpers import attn_rows_reference
            assert_close(got.cpu()[rows], attn_rows_reference(q, k, v, cq.numpy(), ck.numpy(), rows),
                         what='noalloc vs oracle (sampled rows)')


def test_noalloc_rejects_a_call_beyond_the_array():
    """4096 segments of 65536 queries x 256 heads would need a work-item queue far beyond the array: rejected with
    the library's message before anything is launched (the buffers named are small and never read)"""
    x = torch.zeros(8, 256, 128, dtype=torch.bfloat16, device=DEV)
    cu = torch.zeros(4097, dtype=torch.int32, device=DEV)
    a = L.VarlenArgs()
    a.q = a.k = a.v = a.o = x.data_ptr()
    a.cu_q = a.cu_k = cu.data_ptr()
    a.n_q_video = 8
    a.q_row_stride = a.k_row_stride = a.o_row_stride = 256 * 128
    a.n_seg, a.sum_q, a.max_q, a.max_k, a.H, a.D = 4096, 1 << 28, 1 << 16, 8, 256, 128
    a.scale = 128 ** -0.5
    rc = L.lib().or_varlen_fwd_noalloc(ctypes.byref(a), L.stream_handle(x.device))
    assert rc == -1
    assert 'library array' in L.lib().or_last_error().decode()
    torch.cuda.synchronize()
