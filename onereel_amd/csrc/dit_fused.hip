// Fused elementwise work of a Wan transformer block: LayerNorm with modulation, and gated residual adds.
//
// The reference runs diffusers' WanTransformerBlock (third-party, not vendored; OneReel installs its attention
// processors into it, src/onereel/models/wan.py:77-108, and xDiT's Wan example applies the same shift / scale
// modulation at its output norm, third_party/xDiT/examples/wan_example.py:162-167). Per block that model does, in
// fp32 on bf16 activations x:
//   n = LayerNorm(x) * (1 + scale) + shift                (norm1 / norm3 with the AdaLN modulation)
//   n = LayerNorm(x) * w + b                              (norm2, the affine cross-attention norm)
//   x = x + a * gate, x = x + a                           (the gated and plain residual adds)
// each a chain of torch kernels over [tokens, hidden] fp32 temporaries (x.float(), layer_norm, *, +, .to(bf16)).
// Here each is one pass: bf16 in, fp32 math in torch's order (no contraction), bf16 out.
//
// HBM-bound: LayerNorm + modulation reads and writes one bf16 row (4 B per element); the residual reads two rows
// and writes one (6 B per element). LayerNorm: one wavefront per row, 8 consecutive elements per lane and chunk.
#include <math.h>

#include "common.h"

namespace onereel {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxChunks = 16;   // rows up to 64 lanes * 16 chunks * 8 = 8192 elements

struct LnArgs {
  const uint16_t* x;
  uint16_t* out;
  int64_t n_rows, x_stride, out_stride;
  const float* weight;   // [C] or NULL
  const float* bias;     // [C] or NULL
  const float* scale;    // [C] or NULL: * (1 + scale)
  const float* shift;    // [C] or NULL
  int C;
  float eps;
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

__device__ __forceinline__ void unpack8(u32x4 v, float (&f)[8]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    f[2 * p] = bf2f((uint16_t)(v[p] & 0xffffu));
    f[2 * p + 1] = bf2f((uint16_t)(v[p] >> 16));
  }
}

// The per-column parameters (weight, bias, scale, shift: those given) are staged in LDS once per block; each
// wavefront loads its next row while it reduces and writes the current one.
template <int NCH>
__global__ __launch_bounds__(kThreads) void layernorm_modulate_kernel(LnArgs g) {
#pragma clang fp contract(off)
  extern __shared__ __attribute__((aligned(16))) float prm[];
  const int lane = threadIdx.x & 63;
  const int C = g.C;
  const float* src[4] = {g.weight, g.bias, g.scale, g.shift};
  int at[4];
  int n_prm = 0;
#pragma unroll
  for (int a = 0; a < 4; ++a) at[a] = src[a] ? C * n_prm++ : -1;
#pragma unroll
  for (int a = 0; a < 4; ++a)
    if (src[a])
      for (int e = 4 * threadIdx.x; e < C; e += 4 * kThreads) *(f32x4*)(prm + at[a] + e) = *(const f32x4*)(src[a] + e);
  __syncthreads();

  const int64_t stride = (int64_t)gridDim.x * kWaves;
  auto load = [&](u32x4 (&raw)[NCH], int64_t row) {
    const uint16_t* xp = g.x + row * g.x_stride;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int e = 8 * (lane + 64 * i);
      if (e < C) raw[i] = *(const u32x4*)(xp + e);
    }
  };
  // the row's elements are unpacked from the raw bf16 words in each pass, so that only raw words stay live
  auto process = [&](const u32x4 (&raw)[NCH], int64_t row) {
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      if (8 * (lane + 64 * i) < C) {
        float v[8];
        unpack8(raw[i], v);
#pragma unroll
        for (int t = 0; t < 8; ++t) s += v[t];
      }
    }
    const float mean = wave_sum(s) / (float)C;
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      if (8 * (lane + 64 * i) < C) {
        float v[8];
        unpack8(raw[i], v);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const float d = v[t] - mean;
          q += d * d;
        }
      }
    }
    const float rstd = 1.0f / sqrtf(wave_sum(q) / (float)C + g.eps);
    uint16_t* op = g.out + row * g.out_stride;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int e = 8 * (lane + 64 * i);
      if (e >= C) continue;
      float y[8];
      unpack8(raw[i], y);
#pragma unroll
      for (int t = 0; t < 8; ++t) y[t] = (y[t] - mean) * rstd;
#pragma unroll
      for (int a = 0; a < 4; ++a) {
        if (at[a] < 0) continue;
        const f32x4 p0 = *(const f32x4*)(prm + at[a] + e), p1 = *(const f32x4*)(prm + at[a] + e + 4);
        const float pv[8] = {p0[0], p0[1], p0[2], p0[3], p1[0], p1[1], p1[2], p1[3]};
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          if (a == 0) y[t] = y[t] * pv[t];                  // weight
          else if (a == 1) y[t] = y[t] + pv[t];             // bias
          else if (a == 2) y[t] = y[t] * (1.0f + pv[t]);    // scale
          else y[t] = y[t] + pv[t];                         // shift
        }
      }
      u32x4 o;
#pragma unroll
      for (int p = 0; p < 4; ++p) o[p] = pack2(y[2 * p], y[2 * p + 1]);
      *(u32x4*)(op + e) = o;
    }
  };
  // two rows in flight per wavefront: the next row loads while the current one is reduced and written
  u32x4 ra[NCH], rb[NCH];
  int64_t r = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  if (r < g.n_rows) load(ra, r);
  while (r < g.n_rows) {
    if (r + stride < g.n_rows) load(rb, r + stride);
    process(ra, r);
    r += stride;
    if (r >= g.n_rows) break;
    if (r + stride < g.n_rows) load(ra, r + stride);
    process(rb, r);
    r += stride;
  }
}

struct ResArgs {
  uint16_t* x;
  const uint16_t* a;
  const float* gate;     // [C] or NULL
  int64_t n_rows, x_stride, a_stride;
  int C;
};

// x = bf16(float(x) + float(a) * gate): 8 elements per thread, grid-stride over rows * C / 8
__global__ __launch_bounds__(kThreads) void gated_residual_kernel(ResArgs g) {
#pragma clang fp contract(off)
  const int per = g.C >> 3;
  const int64_t total = g.n_rows * per;
  for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (int64_t)gridDim.x * kThreads) {
    const int64_t r = t / per;
    const int e = 8 * (int)(t - r * per);
    uint16_t* xp = g.x + r * g.x_stride + e;
    float xv[8], av[8];
    unpack8(*(const u32x4*)xp, xv);
    unpack8(*(const u32x4*)(g.a + r * g.a_stride + e), av);
    u32x4 o;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      float y0, y1;
      if (g.gate) {
        y0 = xv[2 * p] + av[2 * p] * g.gate[e + 2 * p];
        y1 = xv[2 * p + 1] + av[2 * p + 1] * g.gate[e + 2 * p + 1];
      } else {
        y0 = xv[2 * p] + av[2 * p];
        y1 = xv[2 * p + 1] + av[2 * p + 1];
      }
      o[p] = pack2(y0, y1);
    }
    *(u32x4*)xp = o;
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace onereel

using namespace onereel;

extern "C" int or_layernorm_modulate(const void* x, void* out, int64_t n_rows, int32_t C, int64_t x_row_stride,
                                     int64_t out_row_stride, float eps, const float* weight, const float* bias,
                                     const float* scale, const float* shift, void* stream) {
  if (n_rows < 0 || C < 8 || C % 8 || C > 64 * 8 * kMaxChunks || x_row_stride < C || out_row_stride < C)
    return fail_arg("or_layernorm_modulate: need C a multiple of 8 up to %d and row strides covering C (C=%d)",
                    64 * 8 * kMaxChunks, C);
  if (n_rows == 0) return 0;
  if (!x || !out) return fail_arg("or_layernorm_modulate: x and out are required");
  if (!aligned16(x) || !aligned16(out) || x_row_stride % 8 || out_row_stride % 8)
    return fail_arg("or_layernorm_modulate: x and out must be 16-byte aligned rows");
  const float* prm[4] = {weight, bias, scale, shift};
  int n_prm = 0;
  for (const float* a : prm) {
    if (a && !aligned16(a)) return fail_arg("or_layernorm_modulate: weight, bias, scale and shift must be 16-byte aligned");
    n_prm += a != nullptr;
  }
  LnArgs g{(const uint16_t*)x, (uint16_t*)out, n_rows, x_row_stride, out_row_stride, weight, bias, scale, shift, C,
           eps};
  int64_t blocks = (n_rows + kWaves - 1) / kWaves;
  if (blocks > 256 * 8) blocks = 256 * 8;
  hipStream_t st = (hipStream_t)stream;
  const int nch = (C + 511) / 512;
  const dim3 grid((unsigned)blocks), block(kThreads);
  const size_t lds = (size_t)n_prm * C * sizeof(float);   // at most 4 x 8192 x 4 B = 128 KiB
  if (nch <= 2) hipLaunchKernelGGL(layernorm_modulate_kernel<2>, grid, block, lds, st, g);
  else if (nch <= 4) hipLaunchKernelGGL(layernorm_modulate_kernel<4>, grid, block, lds, st, g);
  else if (nch <= 6) hipLaunchKernelGGL(layernorm_modulate_kernel<6>, grid, block, lds, st, g);
  else if (nch <= 8) hipLaunchKernelGGL(layernorm_modulate_kernel<8>, grid, block, lds, st, g);
  else hipLaunchKernelGGL(layernorm_modulate_kernel<16>, grid, block, lds, st, g);
  return check_hip(hipGetLastError(), "layernorm_modulate_kernel launch");
}

extern "C" int or_gated_residual(void* x, const void* a, const float* gate, int64_t n_rows, int32_t C,
                                 int64_t x_row_stride, int64_t a_row_stride, void* stream) {
  if (n_rows < 0 || C < 8 || C % 8 || x_row_stride < C || a_row_stride < C)
    return fail_arg("or_gated_residual: need C a multiple of 8 and row strides covering C (C=%d)", C);
  if (n_rows == 0) return 0;
  if (!x || !a) return fail_arg("or_gated_residual: x and a are required");
  if (!aligned16(x) || !aligned16(a) || x_row_stride % 8 || a_row_stride % 8)
    return fail_arg("or_gated_residual: x and a must be 16-byte aligned rows");
  ResArgs g{(uint16_t*)x, (const uint16_t*)a, gate, n_rows, x_row_stride, a_row_stride, C};
  const int64_t total = n_rows * (C / 8);
  int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 256 * 16) blocks = 256 * 16;
  hipLaunchKernelGGL(gated_residual_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream, g);
  return check_hip(hipGetLastError(), "gated_residual_kernel launch");
}
