// Frame memory on the device: per-frame pooling of hidden states, and the k-means (cosine) choice of representative
// frames with their medoids.
//
// Reference: FrameMemory.collect (src/onereel/frame_memory.py:76-85): the per-frame sums and counts of one layer's
// video rows (index_add_), and FrameMemory.select (frame_memory.py:114-132): farthest-point initialisation, k-means
// on L2-normalised features with the dot product as similarity, then per cluster the member most similar to its
// centre (the first on ties). Here:
//
// - frame_pool_kernel: rows are frame-major (frame of row r = (row0 + r) / T, as the one-GPU processors build
//   them), so a frame's rows are contiguous. One wavefront per (frame, 512-column block) adds them in row order:
//   deterministic, unlike an atomic index_add_. Per lane, 8 consecutive columns in fp32.
// - frame_select_kernel: the whole selection in one workgroup of 1024 threads, centres in LDS (k * C floats); no
//   host round trip per iteration. Ties are broken towards the lower index, as torch.argmax does. A pass stops when
//   the new centres equal the old ones exactly (torch.equal).
#include <math.h>

#include "common.h"

namespace onereel {

namespace {

constexpr int kPoolThreads = 256;
constexpr int kSelThreads = 1024;
constexpr int kSelWaves = kSelThreads / 64;
constexpr int kMaxCand = 1024;
constexpr int kMaxCentreFloats = 32768;   // k * C: the centres, 128 KiB of LDS
constexpr int kMaxK = 64;

struct PoolArgs {
  const uint16_t* hs;
  int64_t n_rows, row_stride, row0;
  int C, T, n_frames;
  float* sums;       // [n_frames, C]
  float* counts;     // [n_frames]
};

// grid: (groups of four 512-column blocks, frames); each wavefront covers 512 columns (64 lanes x 8) of one frame
__global__ __launch_bounds__(kPoolThreads) void frame_pool_kernel(PoolArgs g) {
  const int lane = threadIdx.x & 63;
  const int cb = blockIdx.x * (kPoolThreads / 64) + (threadIdx.x >> 6);   // 512-column block
  const int f = blockIdx.y;
  const int col = cb * 512 + 8 * lane;
  if (col >= g.C) return;
  int64_t r0 = (int64_t)f * g.T - g.row0, r1 = r0 + g.T;
  r0 = r0 < 0 ? 0 : r0;
  r1 = r1 > g.n_rows ? g.n_rows : r1;
  float acc[8] = {};
  int64_t r = r0;
  // four rows in flight per lane, added in row order
  for (; r + 4 <= r1; r += 4) {
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = *(const u32x4*)(g.hs + (r + u) * g.row_stride + col);
#pragma unroll
    for (int u = 0; u < 4; ++u)
#pragma unroll
      for (int p = 0; p < 4; ++p) {
        acc[2 * p] += bf2f((uint16_t)(v[u][p] & 0xffffu));
        acc[2 * p + 1] += bf2f((uint16_t)(v[u][p] >> 16));
      }
  }
  for (; r < r1; ++r) {
    const u32x4 v = *(const u32x4*)(g.hs + r * g.row_stride + col);
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      acc[2 * p] += bf2f((uint16_t)(v[p] & 0xffffu));
      acc[2 * p + 1] += bf2f((uint16_t)(v[p] >> 16));
    }
  }
  if (r1 <= r0) return;
  float* sp = g.sums + (int64_t)f * g.C + col;
#pragma unroll
  for (int e = 0; e < 8; ++e) sp[e] += acc[e];
  if (cb == 0 && lane == 0) g.counts[f] += (float)(r1 - r0);
}

struct SelectArgs {
  const float* feats;      // [n_frames, C], rows L2-normalised
  const int32_t* cand;     // [n_cand] candidate frames
  int n_cand, C, k, iters;
  int32_t* reps;           // [k] out: chosen frames ascending, -1 after them
  float* work;             // [8, C] workspace
};

// butterfly sum over the 64 lanes by xor shuffles, the same in every lane
__device__ __forceinline__ float wave_sum_xor(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// first index of the maximum of v[0 .. n) (n <= kMaxCand); every thread of the block calls it
__device__ int block_argmax(const float* v, int n, float* sv, int* si) {
  const int tid = threadIdx.x;
  float best = -INFINITY;
  int bi = 0x7fffffff;
  for (int i = tid; i < n; i += kSelThreads)
    if (bi == 0x7fffffff || v[i] > best) {   // ascending i per thread: its first maximum
      best = v[i];
      bi = i;
    }
  sv[tid] = best;
  si[tid] = bi;
  __syncthreads();
  for (int o = kSelThreads / 2; o > 0; o >>= 1) {
    if (tid < o) {
      const float b = sv[tid + o];
      const int j = si[tid + o];
      if (b > sv[tid] || (b == sv[tid] && j < si[tid])) {
        sv[tid] = b;
        si[tid] = j;
      }
    }
    __syncthreads();
  }
  const int r = si[0];
  __syncthreads();
  return r;
}

// dot product of candidate row n with a centre (LDS or global), reduced over the wavefront
__device__ __forceinline__ float row_dot(const SelectArgs& g, int n, const float* cv, int lane) {
  const float* x = g.feats + (int64_t)g.cand[n] * g.C;
  float acc = 0.0f;
  for (int e = lane; e < g.C; e += 64) acc += x[e] * cv[e];
  return wave_sum_xor(acc);
}

__global__ __launch_bounds__(kSelThreads) void frame_select_kernel(SelectArgs g) {
  extern __shared__ float smem[];
  float* c = smem;                  // [k, C] centres
  float* mrow = g.work;             // [8, C] means of the eight clusters being updated (global workspace)
  __shared__ float dv[kMaxCand];    // per-candidate scores
  __shared__ int z[kMaxCand];       // assignment
  __shared__ float sv[kSelThreads];
  __shared__ int si[kSelThreads];
  __shared__ int centre[kMaxK];
  __shared__ int cnt[kMaxK];
  __shared__ int changed;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int nc = g.n_cand, C = g.C, k = g.k;

  // farthest-point initialisation: centre 0 is candidate 0, then each time the candidate whose nearest chosen
  // centre is farthest (largest 1 - dot)
  for (int n = tid; n < nc; n += kSelThreads) dv[n] = INFINITY;
  if (tid == 0) centre[0] = 0;
  __syncthreads();
  for (int m = 1; m < k; ++m) {
    const float* xc = g.feats + (int64_t)g.cand[centre[m - 1]] * C;
    for (int n = w; n < nc; n += kSelWaves) {
      const float d = 1.0f - row_dot(g, n, xc, lane);
      if (lane == 0) dv[n] = fminf(dv[n], d);
    }
    __syncthreads();
    const int a = block_argmax(dv, nc, sv, si);
    if (tid == 0) centre[m] = a;
    __syncthreads();
  }
  for (int e = tid; e < k * C; e += kSelThreads) c[e] = g.feats[(int64_t)g.cand[centre[e / C]] * C + e % C];
  __syncthreads();

  // k-means: z = the most similar centre (first on ties); centre i = normalize(mean of its members), unchanged when
  // it has none; stop when no centre changed. After the loop z belongs to the final centres. Centres are taken eight
  // at a time, so that a candidate row is read once per eight dot products and the member sums of eight clusters
  // accumulate in one pass over the rows (in row order).
  for (int it = 0;; ++it) {
    for (int n = w; n < nc; n += kSelWaves) {
      const float* x = g.feats + (int64_t)g.cand[n] * C;
      float best = 0.0f;
      int bi = 0;
      for (int i0 = 0; i0 < k; i0 += 8) {
        float acc[8] = {};
        for (int e = lane; e < C; e += 64) {
          const float xv = x[e];
#pragma unroll
          for (int q = 0; q < 8; ++q)
            if (i0 + q < k) acc[q] += xv * c[(i0 + q) * C + e];
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          if (i0 + q >= k) break;
          const float d = wave_sum_xor(acc[q]);
          if (i0 + q == 0 || d > best) {
            best = d;
            bi = i0 + q;
          }
        }
      }
      if (lane == 0) z[n] = bi;
    }
    if (tid < k) cnt[tid] = 0;
    if (tid == 0) changed = 0;
    __syncthreads();
    if (it == g.iters) break;
    for (int n = tid; n < nc; n += kSelThreads) atomicAdd(&cnt[z[n]], 1);
    __syncthreads();
    for (int i0 = 0; i0 < k; i0 += 8) {
      float part[8] = {};
      for (int e = tid; e < C; e += kSelThreads) {
        float sum[8] = {};
        for (int n = 0; n < nc; ++n) {
          const int zi = z[n] - i0;     // the same for every thread: a uniform branch
          if (zi < 0 || zi >= 8) continue;
          const float v = g.feats[(int64_t)g.cand[n] * C + e];
#pragma unroll
          for (int q = 0; q < 8; ++q)
            if (zi == q) sum[q] += v;
        }
#pragma unroll
        for (int q = 0; q < 8; ++q) {
          if (i0 + q >= k) break;
          const float mean = cnt[i0 + q] ? sum[q] / (float)cnt[i0 + q] : 0.0f;
          mrow[q * C + e] = mean;
          part[q] += mean * mean;
        }
      }
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const float p = wave_sum_xor(part[q]);
        if (lane == 0) sv[q * kSelWaves + w] = p;
      }
      __syncthreads();
      for (int q = 0; q < 8 && i0 + q < k; ++q) {
        if (cnt[i0 + q] == 0) continue;   // no members: the centre stays
        float t = 0.0f;
        for (int u = 0; u < kSelWaves; ++u) t += sv[q * kSelWaves + u];
        const float nrm = fmaxf(sqrtf(t), 1e-12f);
        float* ci = c + (i0 + q) * C;
        for (int e = tid; e < C; e += kSelThreads) {
          const float nv = mrow[q * C + e] / nrm;
          if (nv != ci[e]) changed = 1;
          ci[e] = nv;
        }
      }
      __syncthreads();
    }
    if (!changed) break;   // z was computed from these (unchanged) centres
    __syncthreads();
  }

  // medoid of each non-empty cluster: the member most similar to its centre, the first on ties
  for (int i = 0; i < k; ++i) {
    for (int n = w; n < nc; n += kSelWaves) {
      float d = -INFINITY;
      if (z[n] == i) d = row_dot(g, n, c + i * C, lane);
      if (lane == 0) dv[n] = d;
    }
    if (tid == 0) changed = 0;
    __syncthreads();
    for (int n = tid; n < nc; n += kSelThreads)
      if (z[n] == i) changed = 1;
    __syncthreads();
    const int any = changed;
    const int a = block_argmax(dv, nc, sv, si);
    if (tid == 0) centre[i] = any ? g.cand[a] : -1;
    __syncthreads();
  }
  if (tid == 0) {
    int out[kMaxK];
    int n = 0;
    for (int i = 0; i < k; ++i)
      if (centre[i] >= 0) out[n++] = centre[i];
    for (int a = 1; a < n; ++a)
      for (int b = a; b > 0 && out[b - 1] > out[b]; --b) {
        const int t = out[b];
        out[b] = out[b - 1];
        out[b - 1] = t;
      }
    for (int i = 0; i < k; ++i) g.reps[i] = i < n ? out[i] : -1;
  }
}

}  // namespace
}  // namespace onereel

using namespace onereel;

extern "C" int or_frame_pool(const void* hs, int64_t n_rows, int32_t C, int64_t row_stride, int64_t row0, int32_t T,
                             int32_t n_frames, float* sums, float* counts, void* stream) {
  if (n_rows < 0 || C < 8 || C % 8 || T < 1 || n_frames < 1 || row0 < 0 || row_stride < C)
    return fail_arg("or_frame_pool: need n_rows >= 0, C a multiple of 8, T >= 1, n_frames >= 1, row0 >= 0 and a row "
                    "stride covering C (C=%d T=%d frames=%d)", C, T, n_frames);
  if (n_rows == 0) return 0;
  if (!hs || !sums || !counts) return fail_arg("or_frame_pool: hs, sums and counts are required");
  if ((row0 + n_rows + T - 1) / T > n_frames)
    return fail_arg("or_frame_pool: rows %lld..%lld reach past frame %d", (long long)row0, (long long)(row0 + n_rows),
                    n_frames);
  if (((uintptr_t)hs & 15u) || row_stride % 8) return fail_arg("or_frame_pool: hs must be 16-byte aligned rows");
  PoolArgs g{(const uint16_t*)hs, n_rows, row_stride, row0, C, T, n_frames, sums, counts};
  const int col_blocks = (C + 512 - 1) / 512;
  const dim3 grid((unsigned)((col_blocks + 3) / 4), (unsigned)n_frames);
  hipLaunchKernelGGL(frame_pool_kernel, grid, dim3(kPoolThreads), 0, (hipStream_t)stream, g);
  return check_hip(hipGetLastError(), "frame_pool_kernel launch");
}

extern "C" int or_frame_select(const float* feats, int32_t n_frames, int32_t C, const int32_t* cand, int32_t n_cand,
                               int32_t k, int32_t iters, int32_t* reps, float* work, void* stream) {
  if (C < 1 || n_frames < 1 || n_cand < 1 || n_cand > kMaxCand || k < 1 || k > kMaxK || k > n_cand || iters < 0)
    return fail_arg("or_frame_select: need C >= 1, 1 <= n_cand <= %d and 1 <= k <= min(n_cand, %d) (n_cand=%d k=%d)",
                    kMaxCand, kMaxK, n_cand, k);
  if ((int64_t)k * C > kMaxCentreFloats)
    return fail_arg("or_frame_select: k * C = %lld floats of centres exceed %d of LDS", (long long)k * C,
                    kMaxCentreFloats);
  if (!feats || !cand || !reps || !work) return fail_arg("or_frame_select: feats, cand, reps and work are required");
  SelectArgs g{feats, cand, n_cand, C, k, iters, reps, work};
  const size_t lds = (size_t)k * C * sizeof(float);
  static thread_local bool attr = false;
  if (!attr) {
    if (int rc = check_hip(hipFuncSetAttribute((const void*)frame_select_kernel,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, kMaxCentreFloats * 4),
                           "hipFuncSetAttribute"))
      return rc;
    attr = true;
  }
  hipLaunchKernelGGL(frame_select_kernel, dim3(1), dim3(kSelThreads), lds, (hipStream_t)stream, g);
  return check_hip(hipGetLastError(), "frame_select_kernel launch");
}
