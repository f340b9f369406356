/*
 * onereel_dit.h: C ABI of libonereel_dit.so, the fused elementwise kernels of the Wan-shaped DiT block harness
 * (onereel_amd/wan_dit.py): a random-init model that runs the scene-attention processors end to end so that a
 * denoising step's time can be measured. These kernels are not on the scene-attention path (libonereel_hip.so,
 * include/onereel_hip.h); the library links against libonereel_hip.so and reports errors through its or_last_error.
 *
 * Conventions as in onereel_hip.h: caller-owned device memory, bf16 as uint16_t bits, rows with a row stride in
 * elements, every launch on the given stream (a hipStream_t, NULL = the null stream); 0 on success, -1 for a bad
 * argument, -2 for a HIP error.
 */
#ifndef ONEREEL_DIT_H
#define ONEREEL_DIT_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces the LayerNorm + modulation chains of the Wan transformer block the reference's processors run in
 * (diffusers' WanTransformerBlock, third-party; installed at src/onereel/models/wan.py:77-108): per bf16 row of C
 * elements, y = (x - mean) * rstd, then * weight, + bias, * (1 + scale), + shift for each of those fp32 [C] vectors
 * that is not NULL, in that order and in fp32; out = bf16(y). */
int or_layernorm_modulate(const void* x, void* out, int64_t n_rows, int32_t C, int64_t x_row_stride,
                          int64_t out_row_stride, float eps, const float* weight, const float* bias, const float* scale,
                          const float* shift, void* stream);

/* Replaces the block's residual adds (same block): x = bf16(float(x) + float(a) * gate), gate fp32 [C], or
 * x = bf16(float(x) + float(a)) when gate is NULL; in place on x. */
int or_gated_residual(void* x, const void* a, const float* gate, int64_t n_rows, int32_t C, int64_t x_row_stride,
                      int64_t a_row_stride, void* stream);

/* Replaces a residual add of the block followed by the next LayerNorm + modulation (the same block, or the next
 * block's first norm): or_gated_residual on x, then or_layernorm_modulate of the updated x into out, with the same
 * results bit for bit, in one pass over the rows when C <= 4096 (two passes above). out must be neither x nor a. */
int or_residual_layernorm_modulate(void* x, const void* a, const float* gate, void* out, int64_t n_rows, int32_t C,
                                   int64_t x_row_stride, int64_t a_row_stride, int64_t out_row_stride, float eps,
                                   const float* weight, const float* bias, const float* scale, const float* shift,
                                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* ONEREEL_DIT_H */
