// Register-only bf16 MFMA loop: what the matrix cores sustain on this GPU when nothing else runs (no HBM or L2
// traffic, no LDS, no softmax). Built as libonereel_bench.so (include/onereel_bench.h) for bench.py. On MI355X the
// board's power and current management lowers the clock under MFMA load, and MFMA power depends on the operand bits,
// so with N(0, 1) operands this rate, not the nominal 2.4 GHz peak, bounds every bf16 kernel; the attention kernel is
// read against it. The operands stay in registers and rotate so that consecutive MFMAs read different registers, as a
// kernel's K / Q and V / P operands do. Mode 2 adds, per MFMA, the VALU work an exact softmax does per score in a
// kernel that computes 64 queries x 32 keys per 32 MFMAs of this shape: p = 2^(c s) (one v_mul_f32 and one
// v_exp_f32), the row sum l += p (one v_add_f32) and every second MFMA one v_cvt_pk_bf16_f32 of two p; on independent
// registers, so that the MFMA issue never waits on them.
#include "../../include/onereel_bench.h"
#include "common.h"

namespace onereel {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kCeilThreads = 256;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// the scores mode 2 exponentiates: -((7 t + 13 i) mod 97) / 8 for thread t and register i, in [-12, 0]
__device__ __forceinline__ float ceiling_score(int64_t tid, int i) {
  return -(float)((tid * 7 + i * 13) % 97) * 0.125f;
}

// every operand index is taken modulo n_vec, so the loads stay inside the caller's buffer
template <int MODE>
__global__ __launch_bounds__(kCeilThreads) void mfma_ceiling_kernel(const bf16x8* __restrict__ in, int64_t n_vec,
                                                                    float* __restrict__ out, int iters) {
  const int64_t tid = (int64_t)blockIdx.x * kCeilThreads + threadIdx.x;
  bf16x8 a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = in[(tid * 16 + i) % n_vec];
    b[i] = in[(tid * 16 + 8 + i) % n_vec];
  }
  float s = 0.0f;
  if constexpr (MODE != 1) {
    constexpr float kC = 0.12752981f;   // 128^-0.5 * log2(e)
    float x[16], l[8];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = ceiling_score(tid, i);
#pragma unroll
    for (int i = 0; i < 8; ++i) l[i] = 0.0f;
    f32x16 c[4] = {};
    for (int it = 0; it < iters; it += 8) {
      // the rotation of B is unrolled, so that every operand is a fixed register
#pragma unroll
      for (int r = 0; r < 8; ++r) {
        float pp = 0.0f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          c[k & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[k], b[(k + r) & 7], c[k & 3], 0, 0, 0);
          if constexpr (MODE == 2) {
            const float p = __builtin_amdgcn_exp2f(x[k + 8 * (r & 1)] * kC);
            l[k] += p;
            if (k & 1) {
              const bf16x2 pk = {(__bf16)pp, (__bf16)p};
              asm volatile("" ::"v"(pk));
            }
            pp = p;
          }
        }
        if constexpr (MODE == 2) {
          // the scores are new values for the compiler, so that nothing is hoisted out of the loop
#pragma unroll
          for (int i = 0; i < 16; ++i) asm volatile("" : "+v"(x[i]));
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int e = 0; e < 16; ++e) s += c[i][e];
#pragma unroll
    for (int i = 0; i < 8; ++i) s += l[i];
  } else {
    f32x4 c[8] = {};
    for (int it = 0; it < iters; it += 8) {
#pragma unroll
      for (int r = 0; r < 8; ++r)
#pragma unroll
        for (int k = 0; k < 16; ++k)
          c[k & 7] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[k & 7], b[(k + r) & 7], c[k & 7], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int e = 0; e < 4; ++e) s += c[i][e];
  }
  out[tid] = s;
}

}  // namespace

}  // namespace onereel

extern "C" int or_mfma_ceiling(const void* operands, int64_t n_vec, float* out, int32_t blocks, int32_t iters,
                               int32_t mode, void* stream) {
  using namespace onereel;
  if (!operands || !out) return fail_arg("or_mfma_ceiling: operands and out are required");
  if (n_vec < 1) return fail_arg("or_mfma_ceiling: n_vec must be positive (got %lld)", (long long)n_vec);
  if (((uintptr_t)operands & 15) || ((uintptr_t)out & 3))
    return fail_arg("or_mfma_ceiling: operands must be 16-byte aligned and out 4-byte aligned");
  if (blocks < 1 || blocks > 65536) return fail_arg("or_mfma_ceiling: blocks must be in [1, 65536] (got %d)", blocks);
  if (iters < 8 || iters % 8)
    return fail_arg("or_mfma_ceiling: iters must be a positive multiple of 8 (got %d)", iters);
  if (mode < 0 || mode > 2)
    return fail_arg("or_mfma_ceiling: mode must be 0 (32x32x16), 1 (16x16x32) or 2 (32x32x16 with softmax VALU work)");
  const bf16x8* in = (const bf16x8*)operands;
  hipStream_t st = (hipStream_t)stream;
  if (mode == 0)
    hipLaunchKernelGGL(mfma_ceiling_kernel<0>, dim3(blocks), dim3(kCeilThreads), 0, st, in, n_vec, out, iters);
  else if (mode == 1)
    hipLaunchKernelGGL(mfma_ceiling_kernel<1>, dim3(blocks), dim3(kCeilThreads), 0, st, in, n_vec, out, iters);
  else
    hipLaunchKernelGGL(mfma_ceiling_kernel<2>, dim3(blocks), dim3(kCeilThreads), 0, st, in, n_vec, out, iters);
  return check_hip(hipGetLastError(), "mfma_ceiling_kernel launch");
}
