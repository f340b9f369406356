"""onereel_amd: OneReel's scene-structured attention hot path, rebuilt for one MI355X (gfx950).

Drop-in modules (same names and semantics as the reference's):
    onereel_amd.layout.SceneLayout          src/onereel/layout.py
    onereel_amd.frame_memory.FrameMemory    src/onereel/frame_memory.py (the layout-facing part)
    onereel_amd.comm                        runs / frame_tokens / merge / clip of src/onereel/parallel/comm.py
    onereel_amd.attention                   src/onereel/attention.py on the HIP varlen kernel
    onereel_amd.hunyuan15                   Context / Processor / RoPE positions of src/onereel/models/hunyuan15.py
    onereel_amd.wan                         Context / Processor of src/onereel/models/wan.py
Engine: onereel_amd.scene (ScopePlan, pack_rows, varlen, scatter, scene_attention) over libonereel_hip.so.
"""
from .layout import SceneLayout

__all__ = ['SceneLayout']
