// Fused elementwise work of a Wan transformer block: LayerNorm with modulation, and gated residual adds. Built as
// libonereel_dit.so (include/onereel_dit.h) for the DiT harness; it uses libonereel_hip.so's error reporting.
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
// A residual add and the LayerNorm that follows it also run as one pass (x += a [* gate], then the LayerNorm of the
// updated x): the rows of x are read once instead of twice.
//
// HBM-bound: LayerNorm + modulation reads and writes one bf16 row (4 B per element); the residual reads two rows
// and writes one (6 B per element); the fused pair reads two rows and writes two (8 B per element). LayerNorm: one
// wavefront per row, 8 consecutive elements per lane and chunk.
#include <math.h>

#include <vector>

#include "../../include/onereel_dit.h"
#include "common.h"

namespace onereel {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxChunks = 16;   // rows up to 64 lanes * 16 chunks * 8 = 8192 elements

struct LnArgs {
  uint16_t* x;           // read only, except in the residual form
  uint16_t* out;
  int64_t n_rows, x_stride, out_stride;
  const float* weight;   // [C] or NULL
  const float* bias;     // [C] or NULL
  const float* scale;    // [C] or NULL: * (1 + scale)
  const float* shift;    // [C] or NULL
  int C;
  float eps;
  // residual form: x = bf16(float(x) + float(a) * gate) (gate NULL: + float(a)) is written back, and the LayerNorm
  // reads that updated row
  const uint16_t* a;
  const float* gate;     // [C] or NULL
  int64_t a_stride;
};

__device__ __forceinline__ void unpack8(u32x4 v, float (&f)[8]) {
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    f[2 * p] = bf2f((uint16_t)(v[p] & 0xffffu));
    f[2 * p + 1] = bf2f((uint16_t)(v[p] >> 16));
  }
}

// x + a * gate as gated_residual_kernel rounds it, 8 elements
__device__ __forceinline__ u32x4 residual8(u32x4 xr, u32x4 ar, const float* gate, int e) {
#pragma clang fp contract(off)
  float xv[8], av[8];
  unpack8(xr, xv);
  unpack8(ar, av);
  u32x4 o;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float y0, y1;
    if (gate) {
      y0 = xv[2 * p] + av[2 * p] * gate[e + 2 * p];
      y1 = xv[2 * p + 1] + av[2 * p + 1] * gate[e + 2 * p + 1];
    } else {
      y0 = xv[2 * p] + av[2 * p];
      y1 = xv[2 * p + 1] + av[2 * p + 1];
    }
    o[p] = pack2(y0, y1);
  }
  return o;
}

// The per-column parameters (weight, bias, scale, shift: those given) are staged in LDS once per block; each
// wavefront takes one row at a time, and the other wavefronts of its SIMD cover the load latency (one row in flight
// per wavefront leaves room for more wavefronts than two would: 13% faster in the residual form at C = 3072). RES: the
// residual form (LnArgs).
template <int NCH, bool RES>
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
  auto load = [&](u32x4 (&raw)[NCH], u32x4 (&araw)[NCH], int64_t row) {
    const uint16_t* xp = g.x + row * g.x_stride;
#pragma unroll
    for (int i = 0; i < NCH; ++i) {
      const int e = 8 * (lane + 64 * i);
      if (e < C) {
        raw[i] = *(const u32x4*)(xp + e);
        if constexpr (RES) araw[i] = *(const u32x4*)(g.a + row * g.a_stride + e);
      }
    }
  };
  // the row's elements are unpacked from the raw bf16 words in each pass, so that only raw words stay live
  auto process = [&](u32x4 (&raw)[NCH], const u32x4 (&araw)[NCH], int64_t row) {
    if constexpr (RES) {
      uint16_t* xp = g.x + row * g.x_stride;
#pragma unroll
      for (int i = 0; i < NCH; ++i) {
        const int e = 8 * (lane + 64 * i);
        if (e < C) {
          raw[i] = residual8(raw[i], araw[i], g.gate, e);
          __builtin_nontemporal_store(raw[i], (u32x4*)(xp + e));
        }
      }
    }
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
      __builtin_nontemporal_store(o, (u32x4*)(op + e));
    }
  };
  u32x4 ra[NCH], aa[NCH];
  for (int64_t r = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6); r < g.n_rows; r += stride) {
    load(ra, aa, r);
    process(ra, aa, r);
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
  const int per = g.C >> 3;
  const int64_t total = g.n_rows * per;
  for (int64_t t = (int64_t)blockIdx.x * kThreads + threadIdx.x; t < total; t += (int64_t)gridDim.x * kThreads) {
    const int64_t r = t / per;
    const int e = 8 * (int)(t - r * per);
    uint16_t* xp = g.x + r * g.x_stride + e;
    __builtin_nontemporal_store(residual8(*(const u32x4*)xp, *(const u32x4*)(g.a + r * g.a_stride + e), g.gate, e),
                                (u32x4*)xp);
  }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace
}  // namespace onereel

using namespace onereel;

namespace {

// checks shared by both LayerNorm entries; returns the number of parameter vectors given, or -1 after fail_arg
int check_ln(const char* fn, const void* x, const void* out, int64_t n_rows, int32_t C, int64_t x_row_stride,
             int64_t out_row_stride, const float* const (&prm)[4]) {
  if (n_rows < 0 || C < 8 || C % 8 || C > 64 * 8 * kMaxChunks || x_row_stride < C || out_row_stride < C) {
    fail_arg("%s: need C a multiple of 8 up to %d and row strides covering C (C=%d)", fn, 64 * 8 * kMaxChunks, C);
    return -1;
  }
  if (n_rows == 0) return 0;
  if (!x || !out) {
    fail_arg("%s: x and out are required", fn);
    return -1;
  }
  if (!aligned16(x) || !aligned16(out) || x_row_stride % 8 || out_row_stride % 8) {
    fail_arg("%s: x and out must be 16-byte aligned rows", fn);
    return -1;
  }
  int n_prm = 0;
  for (const float* a : prm) {
    if (a && !aligned16(a)) {
      fail_arg("%s: weight, bias, scale and shift must be 16-byte aligned", fn);
      return -1;
    }
    n_prm += a != nullptr;
  }
  return n_prm;
}

// blocks of `kernel` (with `lds` bytes of dynamic LDS) resident on the current device at once: CUs x blocks per CU,
// cached per device, kernel and LDS size
int resident_blocks(const void* kernel, size_t lds, int* out) {
  struct Entry {
    int dev;
    const void* kernel;
    size_t lds;
    int blocks;
  };
  static thread_local std::vector<Entry> cache;
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  for (const Entry& c : cache)
    if (c.dev == dev && c.kernel == kernel && c.lds == lds) {
      *out = c.blocks;
      return 0;
    }
  int cus = 0, per_cu = 0;
  if (int rc = check_hip(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev), "hipDeviceGetAttribute"))
    return rc;
  if (int rc = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kThreads, lds),
                         "hipOccupancyMaxActiveBlocksPerMultiprocessor"))
    return rc;
  *out = cus * (per_cu > 0 ? per_cu : 1);
  cache.push_back({dev, kernel, lds, *out});
  return 0;
}

// one launch over all rows with as many blocks as are resident at once (each wavefront strides over the rows, so
// no partly filled last round of blocks)
template <int NCH, bool RES>
int launch_ln_nch(const LnArgs& g, size_t lds, hipStream_t st) {
  const void* kernel = (const void*)layernorm_modulate_kernel<NCH, RES>;
  int resident = 0;
  if (int rc = resident_blocks(kernel, lds, &resident)) return rc;
  int64_t blocks = (g.n_rows + kWaves - 1) / kWaves;
  if (blocks > resident) blocks = resident;
  hipLaunchKernelGGL((layernorm_modulate_kernel<NCH, RES>), dim3((unsigned)blocks), dim3(kThreads), lds, st, g);
  return check_hip(hipGetLastError(), "layernorm_modulate_kernel launch");
}

template <bool RES>
int launch_ln(const LnArgs& g, int n_prm, hipStream_t st) {
  const int nch = (g.C + 511) / 512;
  const size_t lds = (size_t)n_prm * g.C * sizeof(float);   // at most 4 x 8192 x 4 B = 128 KiB
  if (nch <= 2) return launch_ln_nch<2, RES>(g, lds, st);
  if (nch <= 4) return launch_ln_nch<4, RES>(g, lds, st);
  if (nch <= 6) return launch_ln_nch<6, RES>(g, lds, st);
  if (nch <= 8) return launch_ln_nch<8, RES>(g, lds, st);
  if constexpr (!RES) return launch_ln_nch<16, false>(g, lds, st);
  return fail_arg("layernorm_modulate: the residual form takes rows up to 4096 elements");
}

int launch_residual(uint16_t* x, const uint16_t* a, const float* gate, int64_t n_rows, int32_t C, int64_t x_row_stride,
                    int64_t a_row_stride, hipStream_t st) {
  ResArgs g{x, a, gate, n_rows, x_row_stride, a_row_stride, C};
  const int64_t total = n_rows * (C / 8);
  int64_t blocks = (total + kThreads - 1) / kThreads;
  if (blocks > 256 * 16) blocks = 256 * 16;
  hipLaunchKernelGGL(gated_residual_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, st, g);
  return check_hip(hipGetLastError(), "gated_residual_kernel launch");
}

}  // namespace

extern "C" int or_layernorm_modulate(const void* x, void* out, int64_t n_rows, int32_t C, int64_t x_row_stride,
                                     int64_t out_row_stride, float eps, const float* weight, const float* bias,
                                     const float* scale, const float* shift, void* stream) {
  const float* const prm[4] = {weight, bias, scale, shift};
  const int n_prm = check_ln("or_layernorm_modulate", x, out, n_rows, C, x_row_stride, out_row_stride, prm);
  if (n_prm < 0) return -1;
  if (n_rows == 0) return 0;
  LnArgs g{(uint16_t*)x, (uint16_t*)out, n_rows, x_row_stride, out_row_stride, weight, bias, scale, shift, C, eps,
           nullptr, nullptr, 0};
  return launch_ln<false>(g, n_prm, (hipStream_t)stream);
}

extern "C" int or_residual_layernorm_modulate(void* x, const void* a, const float* gate, void* out, int64_t n_rows,
                                              int32_t C, int64_t x_row_stride, int64_t a_row_stride,
                                              int64_t out_row_stride, float eps, const float* weight,
                                              const float* bias, const float* scale, const float* shift,
                                              void* stream) {
  const float* const prm[4] = {weight, bias, scale, shift};
  const int n_prm = check_ln("or_residual_layernorm_modulate", x, out, n_rows, C, x_row_stride, out_row_stride, prm);
  if (n_prm < 0) return -1;
  if (n_rows == 0) return 0;
  if (!a || !aligned16(a) || a_row_stride < C || a_row_stride % 8)
    return fail_arg("or_residual_layernorm_modulate: a must be 16-byte aligned rows covering C");
  if (out == x || out == a) return fail_arg("or_residual_layernorm_modulate: out must not be x or a");
  hipStream_t st = (hipStream_t)stream;
  if (C > 64 * 8 * 8) {
    // rows over 4096 elements: two passes (two rows of x and a in flight would not fit the registers)
    const int rc = launch_residual((uint16_t*)x, (const uint16_t*)a, gate, n_rows, C, x_row_stride, a_row_stride, st);
    if (rc) return rc;
    LnArgs g{(uint16_t*)x, (uint16_t*)out, n_rows, x_row_stride, out_row_stride, weight, bias, scale, shift, C, eps,
             nullptr, nullptr, 0};
    return launch_ln<false>(g, n_prm, st);
  }
  LnArgs g{(uint16_t*)x, (uint16_t*)out, n_rows, x_row_stride, out_row_stride, weight, bias, scale, shift, C, eps,
           (const uint16_t*)a, gate, a_row_stride};
  return launch_ln<true>(g, n_prm, st);
}

extern "C" int or_gated_residual(void* x, const void* a, const float* gate, int64_t n_rows, int32_t C,
                                 int64_t x_row_stride, int64_t a_row_stride, void* stream) {
  if (n_rows < 0 || C < 8 || C % 8 || x_row_stride < C || a_row_stride < C)
    return fail_arg("or_gated_residual: need C a multiple of 8 and row strides covering C (C=%d)", C);
  if (n_rows == 0) return 0;
  if (!x || !a) return fail_arg("or_gated_residual: x and a are required");
  if (!aligned16(x) || !aligned16(a) || x_row_stride % 8 || a_row_stride % 8)
    return fail_arg("or_gated_residual: x and a must be 16-byte aligned rows");
  return launch_residual((uint16_t*)x, (const uint16_t*)a, gate, n_rows, C, x_row_stride, a_row_stride,
                         (hipStream_t)stream);
}
