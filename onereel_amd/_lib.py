"""ctypes binding of libonereel_hip.so (declared in include/onereel_hip.h).

torch is imported first so that the library binds to the HIP runtime torch already loaded (one runtime per process;
torch's streams are then valid handles for the library). There is no fallback: without the built library every entry
point raises.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime the library binds to)

LIB_PATH = Path(os.environ.get('ONEREEL_HIP_LIB', Path(__file__).resolve().parent / 'libonereel_hip.so'))
# the DiT harness's elementwise kernels (include/onereel_dit.h), not on the scene-attention path
DIT_LIB_PATH = Path(__file__).resolve().parent / 'libonereel_dit.so'
# bench.py's measurement kernels (include/onereel_bench.h), not on the scene-attention path
BENCH_LIB_PATH = Path(__file__).resolve().parent / 'libonereel_bench.so'

OR_MAX_SCENES = 64
OR_MAX_EXTRA = 512

i32, i64, vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_void_p


class LayoutDesc(ctypes.Structure):
    _fields_ = [('n_scenes', i32), ('T', i32), ('halo', i32), ('sides', i32), ('with_text', i32),
                ('scene_rope', i32), ('adjacent', i32), ('n_rope_lengths', i32), ('text_rows', i32),
                ('text_keys_in_place', i32), ('q_lo', i32), ('q_hi', i32), ('lengths', i32 * OR_MAX_SCENES), ('rope_lengths', i32 * OR_MAX_SCENES),
                ('counts', i32 * OR_MAX_SCENES), ('extra_ptr', i32 * (OR_MAX_SCENES + 1)),
                ('extra', i32 * OR_MAX_EXTRA)]


class LayoutSizes(ctypes.Structure):
    _fields_ = [('n_seg', i64), ('sum_q', i64), ('sum_k', i64), ('max_q', i64), ('max_k', i64), ('n_video', i64),
                ('max_rope_row', i64)]


class LayoutOut(ctypes.Structure):
    _fields_ = [(n, vp) for n in ('cu_q', 'cu_k', 'seg_q_src', 'q_src', 'q_rope', 'k_src', 'k_rope', 'k_move_a',
                                  'k_move_b', 'k_off', 'k_len', 'v_lead', 'v_row', 'v_src', 'v_runs')]

# keys per block of the attention kernels' K/V stream (OR_VARLEN_KEY_BLOCK): in-place value rows come in whole blocks
KEY_BLOCK = 32
# value runs per segment past its leading one (OR_VALUE_RUNS)
VALUE_RUNS = 4


class VarlenArgs(ctypes.Structure):
    _fields_ = [('q', vp), ('q_text', vp), ('k', vp), ('v', vp), ('o', vp), ('o_text', vp), ('lse', vp),
                ('cu_q', vp), ('cu_k', vp), ('k_off', vp), ('k_len', vp), ('seg_q_src', vp), ('q_rope', vp),
                ('cos_table', vp), ('sin_table', vp), ('n_rope_rows', i64), ('n_q_video', i64),
                ('q_row_stride', i64), ('k_row_stride', i64), ('o_row_stride', i64), ('n_seg', i32), ('sum_q', i32),
                ('max_q', i32), ('max_k', i32), ('H', i32), ('D', i32), ('scale', ctypes.c_float),
                ('workspace', vp), ('workspace_bytes', i64), ('q_row_step', i32), ('v_tok', vp), ('v_lead', vp),
                ('v_row', vp), ('v_tok_rows', i64), ('k_len_head', vp), ('k_tok', vp), ('k_lead', vp),
                ('k_tok_rows', i64), ('v_runs', vp)]


class PackArgs(ctypes.Structure):
    _fields_ = [('k_video', vp), ('k_text', vp), ('v_video', vp), ('v_text', vp), ('video_row_stride', i64),
                ('text_row_stride', i64), ('n_video', i64), ('k_src', vp), ('k_rope', vp), ('k_move_from', vp),
                ('v_src', vp), ('n_keys', i64), ('k_dst', vp), ('k_out', vp), ('v_out', vp), ('q', vp),
                ('q_row_stride', i64),
                ('q_src', vp), ('q_rope', vp), ('n_queries', i64), ('q_out', vp), ('q_out_row_stride', i64),
                ('cos_table', vp), ('sin_table', vp), ('n_rope_rows', i64), ('H', i32), ('D', i32)]


# every exported symbol with its ctypes signature: include/onereel_hip.h
SIGNATURES = {
    'or_layout_plan': (i32, [ctypes.POINTER(LayoutDesc), ctypes.POINTER(LayoutSizes)]),
    'or_layout_build': (i32, [ctypes.POINTER(LayoutDesc), ctypes.POINTER(LayoutOut), vp]),
    'or_pack_gather': (i32, [vp, vp, vp, vp, i64, i64, i64, vp, vp, vp, vp, vp, i64, i64, i32, i32, vp, vp, vp]),
    'or_scatter': (i32, [vp, vp, i64, i64, vp, vp, i64, i64, i64, i64, i32, i32, vp]),
    'or_rotate_rows': (i32, [vp, i64, i64, vp, vp, vp, vp, i64, i64, i32, i32, vp, i64, vp]),
    'or_pack_layer': (i32, [ctypes.POINTER(PackArgs), vp]),
    'or_varlen_workspace_size': (i64, [i32, i32, i32, i32]),
    'or_varlen_fwd': (i32, [ctypes.POINTER(VarlenArgs), vp]),
    'or_varlen_fwd_noalloc': (i32, [ctypes.POINTER(VarlenArgs), vp]),
    'or_lse_merge': (i32, [vp, vp, vp, vp, i64, i32, i32, i64, i64, vp]),
    'or_rmsnorm_rope': (i32, [vp, vp, vp, vp, i64, i64, i64, i32, i32, ctypes.c_float, vp, vp, vp, i64, vp, vp, i64,
                              i64, vp]),
    'or_frame_pool': (i32, [vp, i64, i32, i64, i64, i32, i32, vp, vp, vp]),
    'or_frame_select': (i32, [vp, i32, i32, vp, i32, i32, i32, vp, vp, vp]),
    'or_memory_select_workspace_size': (i64, [i32, i32, i32, i32, i32]),
    'or_memory_select': (i32, [vp, i32, vp, i64, i32, i32, i32, i32, vp, vp, i32, vp, vp, vp, i64, vp]),
    'or_memory_index': (i32, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, vp, vp, vp]),
    'or_memory_foreign': (i32, [vp, vp, vp, vp, vp, vp, vp, vp, i32, i32, i32, vp, vp, vp, vp]),
    'or_last_error': (ctypes.c_char_p, []),
    'or_version': (ctypes.c_char_p, []),
}

# libonereel_dit.so: include/onereel_dit.h
DIT_SIGNATURES = {
    'or_layernorm_modulate': (i32, [vp, vp, i64, i32, i64, i64, ctypes.c_float, vp, vp, vp, vp, vp]),
    'or_gated_residual': (i32, [vp, vp, vp, i64, i32, i64, i64, vp]),
    'or_residual_layernorm_modulate': (i32, [vp, vp, vp, vp, i64, i32, i64, i64, i64, ctypes.c_float, vp, vp, vp, vp,
                                             vp]),
}

# libonereel_bench.so: include/onereel_bench.h
BENCH_SIGNATURES = {
    'or_mfma_ceiling': (i32, [vp, i64, vp, i32, i32, i32, vp]),
}

_lib = None
_dit_lib = None
_bench_lib = None


class HipPathError(RuntimeError):
    """a library call failed (bad argument or HIP error); the message is the library's"""


class HipValueError(HipPathError, ValueError):
    """an argument the host layer rejects before calling the library (shape, size, layout): a RuntimeError, as
    FlashAttention's argument errors are, and a ValueError"""


class HipTypeError(HipPathError, TypeError):
    """a tensor of the wrong dtype or device: a RuntimeError, as FlashAttention's dtype errors are, and a TypeError"""


def lib():
    """the loaded library; raises if it was not built (no CPU fallback exists)"""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f'{LIB_PATH} is not built: run python -m onereel_amd.build (the HIP path has no '
                               f'fallback)')
        h = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(h, name)
            f.restype, f.argtypes = res, args
        _lib = h
    return _lib


def dit_lib():
    """the DiT harness's library (it loads libonereel_hip.so beside it and reports errors through its or_last_error,
    which dit_check reads through this handle)"""
    global _dit_lib
    if _dit_lib is None:
        lib()
        if not DIT_LIB_PATH.exists():
            raise RuntimeError(f'{DIT_LIB_PATH} is not built: run python -m onereel_amd.build')
        h = ctypes.CDLL(str(DIT_LIB_PATH))
        for name, (res, args) in DIT_SIGNATURES.items():
            f = getattr(h, name)
            f.restype, f.argtypes = res, args
        h.or_last_error.restype, h.or_last_error.argtypes = ctypes.c_char_p, []
        _dit_lib = h
    return _dit_lib


def bench_lib():
    """the measurement library (it loads libonereel_hip.so beside it and reports errors through its or_last_error,
    which bench_check reads through this handle)"""
    global _bench_lib
    if _bench_lib is None:
        lib()
        if not BENCH_LIB_PATH.exists():
            raise RuntimeError(f'{BENCH_LIB_PATH} is not built: run python -m onereel_amd.build')
        h = ctypes.CDLL(str(BENCH_LIB_PATH))
        for name, (res, args) in BENCH_SIGNATURES.items():
            f = getattr(h, name)
            f.restype, f.argtypes = res, args
        h.or_last_error.restype, h.or_last_error.argtypes = ctypes.c_char_p, []
        _bench_lib = h
    return _bench_lib


def check(rc: int, what: str):
    if rc != 0:
        msg = lib().or_last_error().decode()
        raise HipPathError(f'{what} failed ({rc}): {msg}')


def dit_check(rc: int, what: str):
    if rc != 0:
        msg = dit_lib().or_last_error().decode()
        raise HipPathError(f'{what} failed ({rc}): {msg}')


def bench_check(rc: int, what: str):
    if rc != 0:
        msg = bench_lib().or_last_error().decode()
        raise HipPathError(f'{what} failed ({rc}): {msg}')


def ptr(t):
    """device pointer of a tensor, or None"""
    return None if t is None else t.data_ptr()


def stream_handle(device=None):
    return torch.cuda.current_stream(device).cuda_stream
