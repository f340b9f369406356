/*
 * onereel_bench.h: C ABI of libonereel_bench.so, the measurement kernels bench.py times beside the scene-attention
 * path. They have no counterpart in the reference (which ships no native code): they measure what this GPU sustains,
 * so that the path's kernels can be read against it. The library links against libonereel_hip.so and reports errors
 * through its or_last_error.
 *
 * Conventions as in onereel_hip.h: caller-owned device memory, bf16 as uint16_t bits, every launch on the given
 * stream (a hipStream_t, NULL = the null stream); 0 on success, -1 for a bad argument, -2 for a HIP error.
 */
#ifndef ONEREEL_BENCH_H
#define ONEREEL_BENCH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The matrix cores' own ceiling at the board's throttled clock, alone and beside an exact softmax's VALU work:
 * `blocks` work-groups of four wavefronts (one wavefront per SIMD when blocks is the CU count) each load 8 A and 8 B
 * operand registers of 8 bf16 from `operands` (n_vec vectors of 8 bf16, read at lane-dependent indices modulo n_vec)
 * and then run `iters` iterations of 8 dense bf16 MFMAs with no memory access and no LDS, cycling through the
 * operands so that consecutive MFMAs read different registers.
 *   mode 0: v_mfma_f32_32x32x16_bf16 (the attention kernel's), four accumulators, no other work;
 *   mode 1: v_mfma_f32_16x16x32_bf16, 16 per iteration (the same FLOP), eight accumulators, no other work;
 *   mode 2: mode 0 plus, per MFMA, the VALU work of an exact softmax per score: p = 2^(c s) (v_mul_f32, v_exp_f32),
 *           l[k] += p (v_add_f32) and every second MFMA a v_cvt_pk_bf16_f32 of two p, where s = -((7 t + 13 i) mod 97)
 *           / 8 for thread t and i = k + 8 (r mod 2) at the k-th MFMA of the r-th pass over the B rotation, and
 *           c = 128^-0.5 log2(e).
 * Each thread writes the sum of its accumulators (and row sums) to out[thread] (blocks * 256 floats), so that no
 * MFMA is dead code. Useful FLOP per call: blocks * 4 * iters * 8 * 32768. iters must be a positive multiple of 8. */
int or_mfma_ceiling(const void* operands, int64_t n_vec, float* out, int32_t blocks, int32_t iters, int32_t mode,
                    void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ONEREEL_BENCH_H */
