// Fused RMSNorm + interleaved RoPE of the Wan self-attention's queries and keys, one launch for both.
//
// Reference: _qk (src/onereel/models/wan.py:64-74), compiled there with torch.compile: per token row x [C] (C = H * D,
// the norm spans every head, diffusers' 'rms_norm_across_heads'):
//   y = x / sqrt(mean(x^2) + eps) * w
// then per head, for the interleaved pairs (2i, 2i+1) of its D dims, with c = cos[row, 2i] and s = sin[row, 2i+1]
// (cos[..., 0::2], sin[..., 1::2]):
//   out[2i] = y[2i] c - y[2i+1] s,   out[2i+1] = y[2i] s + y[2i+1] c,
// cast to bf16 (type_as(x)). Here the whole chain is fp32 with one rounding at the end, as the compiled graph computes
// it; the bf16 input is read once and the bf16 output written once.
//
// HBM-bound: 2 * C * 2 bytes per row and tensor, plus the row's cos / sin entries (2 * D * 4 bytes, shared by its
// heads). One wavefront per row: each lane holds C / 512 16-byte chunks, the sum of squares is reduced across the
// wavefront, and every lane's chunks sit at the same dims of their heads (512 elements = a whole number of heads for
// D dividing 512), so each lane loads its cos / sin entries once per row.
#include <math.h>

#include "common.h"

namespace onereel {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxChunks = 16;   // rows up to 64 lanes * 16 chunks * 8 = 8192 elements

struct NormRopeArgs {
  const uint16_t* x[2];
  uint16_t* out[2];
  const uint16_t* w[2];          // bf16 [C]
  int64_t x_stride[2], out_stride[2];
  const float* cos_t;
  const float* sin_t;
  const int32_t* rope_row;       // per token row, or NULL: the token row itself
  int64_t n_rows, n_rope_rows;
  int C, D;
  float eps;
};

// One row's inputs: its bf16 words, and this lane's cos / sin entries (d0 = 8 lane mod D, pairs 2p, 2p + 1).
template <int NCH>
struct RowIn {
  u32x4 x[NCH];
  float c[4], s[4];
};

template <int NCH>
__device__ __forceinline__ void load_row(const NormRopeArgs& g, int which, int64_t r, int lane, RowIn<NCH>& in) {
  const uint16_t* xp = g.x[which] + r * g.x_stride[which];
#pragma unroll
  for (int i = 0; i < NCH; ++i) in.x[i] = *(const u32x4*)(xp + 8 * (lane + 64 * i));
  const int rr = g.rope_row ? g.rope_row[r] : (int)r;
  const int d0 = (8 * lane) % g.D;
  const bool rot = rr >= 0 && rr < g.n_rope_rows;   // rows outside the table (or no table) are not rotated
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    in.c[p] = rot ? g.cos_t[(int64_t)rr * g.D + d0 + 2 * p] : 1.0f;
    in.s[p] = rot ? g.sin_t[(int64_t)rr * g.D + d0 + 2 * p + 1] : 0.0f;
  }
}

template <int NCH>
__device__ __forceinline__ void norm_rope_row(const NormRopeArgs& g, int which, int64_t r, int lane,
                                              const RowIn<NCH>& in, const uint16_t* w) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const float a = bf2f((uint16_t)(in.x[i][p] & 0xffffu)), b = bf2f((uint16_t)(in.x[i][p] >> 16));
      ss += a * a + b * b;
    }
  }
  const float inv = 1.0f / sqrtf(wave_sum(ss) / (float)g.C + g.eps);
  uint16_t* op = g.out[which] + r * g.out_stride[which];
#pragma unroll
  for (int i = 0; i < NCH; ++i) {
    const int e = 8 * (lane + 64 * i);
    const u32x4 wv = *(const u32x4*)(w + e);
    u32x4 o;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma clang fp contract(off)
      const float y0 = bf2f((uint16_t)(in.x[i][p] & 0xffffu)) * inv * bf2f((uint16_t)(wv[p] & 0xffffu));
      const float y1 = bf2f((uint16_t)(in.x[i][p] >> 16)) * inv * bf2f((uint16_t)(wv[p] >> 16));
      o[p] = pack2(y0 * in.c[p] - y1 * in.s[p], y0 * in.s[p] + y1 * in.c[p]);
    }
    __builtin_nontemporal_store(o, (u32x4*)(op + e));
  }
}

// blockIdx.y picks q or k. The block stages its weight row in LDS; each wavefront takes one row at a time, and the
// other wavefronts of its SIMD cover the load latency.
template <int NCH>
__global__ __launch_bounds__(kThreads) void norm_rope_kernel(NormRopeArgs g) {
  __shared__ __attribute__((aligned(16))) uint16_t wl[64 * 8 * NCH];
  const int lane = threadIdx.x & 63;
  const int which = blockIdx.y;
  for (int e = 8 * threadIdx.x; e < g.C; e += 8 * kThreads) *(u32x4*)(wl + e) = *(const u32x4*)(g.w[which] + e);
  __syncthreads();
  const int64_t stride = (int64_t)gridDim.x * kWaves;
  for (int64_t r = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); r < g.n_rows; r += stride) {
    RowIn<NCH> a;
    load_row<NCH>(g, which, r, lane, a);
    norm_rope_row<NCH>(g, which, r, lane, a, wl);
  }
}

}  // namespace
}  // namespace onereel

using namespace onereel;

extern "C" int or_rmsnorm_rope(const void* q, const void* k, const void* wq, const void* wk, int64_t q_row_stride,
                               int64_t k_row_stride, int64_t n_rows, int32_t C, int32_t D, float eps,
                               const float* cos_table, const float* sin_table, const int32_t* rope_row,
                               int64_t n_rope_rows, void* q_out, void* k_out, int64_t qo_row_stride,
                               int64_t ko_row_stride, void* stream) {
  if (n_rows < 0) return fail_arg("or_rmsnorm_rope: n_rows < 0");
  if (D < 8 || D % 8 || 512 % D || C % 512 || C < 512 || C > 64 * 8 * kMaxChunks)
    return fail_arg("or_rmsnorm_rope: need D a multiple of 8 dividing 512 and C a multiple of 512 up to %d "
                    "(C=%d D=%d)", 64 * 8 * kMaxChunks, C, D);
  if (n_rows == 0) return 0;
  if (!q || !wq || !q_out) return fail_arg("or_rmsnorm_rope: q, wq and q_out are required");
  if (n_rope_rows > 0 && (!cos_table || !sin_table))
    return fail_arg("or_rmsnorm_rope: n_rope_rows > 0 needs the cos / sin tables");
  if (n_rope_rows < 0) return fail_arg("or_rmsnorm_rope: n_rope_rows < 0");
  if (k && (!wk || !k_out)) return fail_arg("or_rmsnorm_rope: k needs wk and k_out");
  if (q_row_stride < C || qo_row_stride < C || (k && (k_row_stride < C || ko_row_stride < C)))
    return fail_arg("or_rmsnorm_rope: row strides must cover C elements");
  const uintptr_t al = (uintptr_t)q | (uintptr_t)wq | (uintptr_t)q_out | (uintptr_t)(k ? k : q) |
                       (uintptr_t)(wk ? wk : wq) | (uintptr_t)(k_out ? k_out : q_out);
  if ((al & 15u) || q_row_stride % 8 || qo_row_stride % 8 || (k && (k_row_stride % 8 || ko_row_stride % 8)))
    return fail_arg("or_rmsnorm_rope: pointers must be 16-byte aligned and row strides multiples of 8 elements");
  NormRopeArgs g;
  g.x[0] = (const uint16_t*)q;
  g.x[1] = (const uint16_t*)(k ? k : q);
  g.out[0] = (uint16_t*)q_out;
  g.out[1] = (uint16_t*)(k ? k_out : q_out);
  g.w[0] = (const uint16_t*)wq;
  g.w[1] = (const uint16_t*)(k ? wk : wq);
  g.x_stride[0] = q_row_stride;
  g.x_stride[1] = k ? k_row_stride : q_row_stride;
  g.out_stride[0] = qo_row_stride;
  g.out_stride[1] = k ? ko_row_stride : qo_row_stride;
  g.cos_t = cos_table;
  g.sin_t = sin_table;
  g.rope_row = rope_row;
  g.n_rows = n_rows;
  g.n_rope_rows = n_rope_rows;
  g.C = C;
  g.D = D;
  g.eps = eps;
  int64_t blocks = (n_rows + kWaves - 1) / kWaves;
  if (blocks > 256 * 8) blocks = 256 * 8;
  const dim3 grid((unsigned)blocks, k ? 2 : 1);
  hipStream_t st = (hipStream_t)stream;
  switch (C / 512) {
    case 1: hipLaunchKernelGGL(norm_rope_kernel<1>, grid, dim3(kThreads), 0, st, g); break;
    case 2: hipLaunchKernelGGL(norm_rope_kernel<2>, grid, dim3(kThreads), 0, st, g); break;
    case 3: hipLaunchKernelGGL(norm_rope_kernel<3>, grid, dim3(kThreads), 0, st, g); break;
    case 4: hipLaunchKernelGGL(norm_rope_kernel<4>, grid, dim3(kThreads), 0, st, g); break;
    case 5: hipLaunchKernelGGL(norm_rope_kernel<5>, grid, dim3(kThreads), 0, st, g); break;
    case 6: hipLaunchKernelGGL(norm_rope_kernel<6>, grid, dim3(kThreads), 0, st, g); break;
    case 8: hipLaunchKernelGGL(norm_rope_kernel<8>, grid, dim3(kThreads), 0, st, g); break;
    case 12: hipLaunchKernelGGL(norm_rope_kernel<12>, grid, dim3(kThreads), 0, st, g); break;
    case 16: hipLaunchKernelGGL(norm_rope_kernel<16>, grid, dim3(kThreads), 0, st, g); break;
    default: return fail_arg("or_rmsnorm_rope: C=%d not instantiated (512 x {1..6, 8, 12, 16})", C);
  }
  return check_hip(hipGetLastError(), "norm_rope_kernel launch");
}
