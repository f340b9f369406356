"""CPU checks of the built code itself (no GPU): register invariants of the 64-query attention kernel that only its
assembly shows.

attn8_kernel keeps each work item's queries in the AGPRs a128..a191 from the load that fills them (the previous item's
key loop at its exit, or the kernel's own Q load) to the key loop that reads them, and the O accumulators in
a0..a127 inside the key loop. The loads and the key loop are inline asm; the C++ code between them (claims, item
records, the ring head's DMA, the lse stores) does not know that a128..a191 are live, so it must not touch them. The
compiler spills into AGPRs above a191 here; if register pressure or a compiler change made it use a0..a191 outside
the asm blocks, the queries would be overwritten on some item paths only, which no parity test would reliably catch.
This test compiles attention.hip with the build's flags to device assembly and fails on any such reference.
"""
import re
import shutil
import subprocess

import pytest

from onereel_amd import build as B

KERNEL = '_ZN7onereel12_GLOBAL__N_112attn8_kernelENS0_8AttnArgsEPi'


def _agpr_refs(line):
    code = line.split(';')[0]
    out = []
    for m in re.finditer(r'\ba(\d+)\b|\ba\[(\d+):(\d+)\]', code):
        lo = int(m.group(1) or m.group(2))
        hi = int(m.group(1) or m.group(3))
        out.append((lo, hi))
    return out


def test_agpr_reference_parser():
    assert _agpr_refs('v_accvgpr_write_b32 a130, v5') == [(130, 130)]
    assert _agpr_refs('global_load_dwordx4 a[128:131], v[2:3], off offset:32') == [(128, 131)]
    assert _agpr_refs('v_accvgpr_read_b32 v3, a197 ; a5 in a comment') == [(197, 197)]
    assert _agpr_refs('s_add_u32 s64, s64, s2') == []


@pytest.mark.skipif(shutil.which(B.HIPCC) is None and not B.Path(B.HIPCC).exists(), reason='needs hipcc')
def test_attn8_q_and_accumulator_agprs_untouched_outside_asm(tmp_path):
    # the in-tree key loop is what the generator writes now (the build regenerates it; the source includes it)
    subprocess.run([B.sys.executable, str(B.CSRC / 'gen_attn_ring64.py'), '--out', str(tmp_path / 'attn_ring64.inc')],
                   check=True, capture_output=True)
    assert (tmp_path / 'attn_ring64.inc').read_text() == (B.CSRC / 'attn_ring64.inc').read_text()
    asm = tmp_path / 'attention.s'
    flags = B.FLAGS + B.SOURCE_FLAGS.get('attention.hip', [])
    r = subprocess.run([B.HIPCC, *flags, '--cuda-device-only', '-S', str(B.CSRC / 'attention.hip'), '-o', str(asm)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    lines = asm.read_text().splitlines()
    start = next(i for i, l in enumerate(lines) if l.startswith(KERNEL + ':'))
    end = next(i for i in range(start, len(lines)) if lines[i].strip().startswith('.Lfunc_end'))
    in_asm, n_asm, bad = False, 0, []
    for i in range(start, end):
        l = lines[i]
        if ';;#ASMSTART' in l:
            in_asm, n_asm = True, n_asm + 1
            continue
        if ';;#ASMEND' in l:
            in_asm = False
            continue
        if in_asm:
            continue
        if any(lo <= 191 for lo, hi in _agpr_refs(l)):
            bad.append(l.strip())
    assert n_asm > 10, 'the kernel body was not found or has no inline asm'
    assert not bad, f'{len(bad)} compiler instructions touch a0..a191 outside the asm blocks: {bad[:5]}'
