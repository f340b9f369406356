"""Build libonereel_hip.so (gfx950) in-tree with hipcc: one object per HIP source, then one shared library; and,
linked against it, libonereel_dit.so (the DiT harness's elementwise kernels) and libonereel_bench.so (bench.py's
measurement kernels).

    python -m onereel_amd.build            # or __graft_entry__.build()
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / 'csrc'
INCLUDE = PKG.parent / 'include'
LIB = PKG / 'libonereel_hip.so'
DIT_LIB = PKG / 'libonereel_dit.so'
BENCH_LIB = PKG / 'libonereel_bench.so'
OBJ = PKG / 'csrc' / '_obj'
SOURCES = ['layout.hip', 'gather.hip', 'attention.hip', 'merge.hip', 'norm_rope.hip', 'frame_memory.hip', 'memory.hip']
DIT_SOURCES = ['dit_fused.hip']
BENCH_SOURCES = ['mfma_ceiling.hip']
# attention: no NaN operands reach the softmax max, so fmax needs no quieting of its inputs (v_max3_f32 directly)
SOURCE_FLAGS = {'attention.hip': ['-fno-honor-nans']}
ARCH = os.environ.get('ONEREEL_ARCH', 'gfx950')

HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
FLAGS = [f'--offload-arch={ARCH}', '-O3', '-std=c++17', '-fPIC', '-I', str(INCLUDE),
         # packed-FP32 VALU ops are disabled on purpose; hipcc's host pass warns that it does not know the feature
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
         # MFMA accumulators in VGPRs: the softmax rescales them with VALU ops, which cannot address AGPRs
         '-mllvm', '-amdgpu-mfma-vgpr-form=1',
         '-Wno-unused-result']


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = '\n'.join(l for l in r.stderr.splitlines() if noise not in l)
    if r.returncode != 0:
        raise RuntimeError(f'build failed: {" ".join(cmd)}\n{err}')
    return err


def build(verbose: bool = False) -> Path:
    OBJ.mkdir(exist_ok=True)
    # the key loop of the 64-query attention kernel is generated asm
    _run([sys.executable, str(CSRC / 'gen_attn_ring64.py'), '--out', str(CSRC / 'attn_ring64.inc')])
    objs = [OBJ / (s.replace('.hip', '.o')) for s in SOURCES]
    dit_objs = [OBJ / (s.replace('.hip', '.o')) for s in DIT_SOURCES]
    bench_objs = [OBJ / (s.replace('.hip', '.o')) for s in BENCH_SOURCES]

    def one(src_obj):
        src, obj = src_obj
        return _run([HIPCC, *FLAGS, *SOURCE_FLAGS.get(src, []), '-c', str(CSRC / src), '-o', str(obj)])

    srcs = SOURCES + DIT_SOURCES + BENCH_SOURCES
    with ThreadPoolExecutor(max_workers=len(srcs)) as ex:
        logs = list(ex.map(one, zip(srcs, objs + dit_objs + bench_objs)))
    tmp = LIB.with_suffix('.so.tmp')
    logs.append(_run([HIPCC, f'--offload-arch={ARCH}', '-shared', '-fPIC', *map(str, objs), '-o', str(tmp)]))
    os.replace(tmp, LIB)
    # the harness and measurement libraries resolve the error helpers from libonereel_hip.so, found beside them at
    # run time
    for out, lib_objs in ((DIT_LIB, dit_objs), (BENCH_LIB, bench_objs)):
        tmp = out.with_suffix('.so.tmp')
        logs.append(_run([HIPCC, f'--offload-arch={ARCH}', '-shared', '-fPIC', *map(str, lib_objs), '-L', str(PKG),
                          '-l:libonereel_hip.so', "-Wl,-rpath,$ORIGIN", '-o', str(tmp)]))
        os.replace(tmp, out)
    if verbose:
        for l in logs:
            if l.strip():
                print(l, file=sys.stderr)
    return LIB


if __name__ == '__main__':
    print(build(verbose=True))
