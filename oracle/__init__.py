"""CPU oracle for the scene-attention hot path: TEST INFRASTRUCTURE ONLY.

This package restates, in plain Python / numpy / torch-on-CPU, the reference's algorithm for one scene-structured
attention layer (layout, scope packing, scene RoPE, per-scope attention, write-back). It is the checker that the HIP
path is compared against. Only `tests/`, `__graft_entry__.smoke()` and the `cpu_baseline` leg of `bench.py` may import
it; the product package `onereel_amd` never does, and has no CPU fallback.

How each function is pinned (besides the GPU comparison) is stated in its docstring; every function here is checked by
`tests/test_oracle.py` against the reference's own known answers (copied as fixtures under `tests/golden/`),
hand-derived values, closed forms, brute force on tiny layouts, or invariants that a plausible slip would break.
"""
