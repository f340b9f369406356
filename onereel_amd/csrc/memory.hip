// Bounded cross-scene memory on the GPU: the per-head choice of representatives among the boundary-frame keys
// (k-means over L2-normalised keys, one medoid per non-empty cluster) and the per-(head, piece) key lists of the
// head-major attention that reads them.
//
// Reference: BoundaryMemory.select (src/onereel/memory.py:58-93) and the index building of MemoryAttention.__call__
// (memory.py:152-168). The reference runs torch ops: batched fp32 matmuls for the distances, one-hot matmuls for the
// cluster sums, a host read per iteration for the convergence test, stable sorts for the tie-break.
//
// Here, per call:
//   prep     one wavefront per (candidate, head): the key row (bf16 or fp32) in fp32, x = row / max(|row|, 1e-12),
//            |x|^2; x stored [H, B, D] fp32. A cold start copies the evenly spaced candidates into the centroids.
//   assign   per (64-candidate tile, head): dot products x . c by fp32 MFMA (v_mfma_f32_16x16x4_f32, the centroids
//            in LDS), d = |x|^2 - 2 x . c + |c|^2, the nearest centroid (the lowest index on equal distances).
//   group    one workgroup per head: a stable counting sort of the candidates by cluster (ascending candidate
//            within a cluster), so that every later sum has a fixed order.
//   update   per (cluster, head): the mean of the members in that order (fp32), or the old centroid when the
//            cluster is empty; a flag records whether any centroid moved.
//   medoid   one workgroup per head: per non-empty cluster, in cluster order, the member nearest its centroid (the
//            lowest candidate on equal distances) -> rep[h, r] (int64) and valid[h, r] = 1, then zeros.
// assign / group / update of iteration it > 0 return at once when iteration it - 1 moved no centroid (a fixed point:
// every later iteration would give the same assignment), so the host launches all passes without reading anything
// back, and the result equals a loop that stops at convergence.
#include <math.h>

#include "common.h"

namespace onereel {

namespace {

constexpr int kMaxClusters = 1024;  // M of one call (counting-sort table in LDS)
constexpr int kAssignThreads = 256;  // 4 wavefronts
constexpr int kAssignRows = 64;      // candidates per assign block: 4 wavefronts x 16
constexpr int kCChunk = 128;        // centroids per LDS chunk in assign
constexpr int kCPitch = 132;        // floats per centroid row in LDS (padding spreads 16 rows over the banks)

typedef float f32x4v __attribute__((ext_vector_type(4)));

struct SelArgs {
  const void* keys;         // candidate key rows: bf16 or fp32
  const int32_t* rows;      // [B] row of each candidate in keys (NULL: candidate b is row b)
  int64_t stride;           // elements between consecutive rows of keys
  int B, H, D, M, fp32_in, iters;
  float* X;                 // [H, B, D] normalised keys
  float* xx;                // [H, B] |x|^2
  float* C;                 // [H, M, D] centroids (in / out)
  float* cc;                // [H, M] |c|^2 of the current centroids
  int32_t* z;               // [H, B] cluster of each candidate
  float* dist;              // [H, B] its squared distance to that centroid
  int32_t* order;           // [H, B] candidates grouped by cluster, ascending within a cluster
  int32_t* start;           // [H, M + 1] group offsets into order
  int32_t* moved;           // [iters + 1] moved[it] != 0: iteration it changed a centroid
  int64_t* rep;             // [H, M]
  uint8_t* valid;           // [H, M]
};

__device__ __forceinline__ float wave_sum64(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// ------------------------------------------------------------------------------------------------------------------
// prep: one wavefront per (candidate b, group of 64 / LPH heads); LPH = D / 32 lanes per head, 32 consecutive elements
// per lane (4 x 16-byte loads of bf16, or 8 of fp32), the head's |row|^2 summed over its lanes by shuffles
template <int D>
__global__ __launch_bounds__(256) void mem_prep_kernel(SelArgs g, int n_moved) {
  constexpr int LPH = D / 32, HPW = 64 / LPH;   // lanes per head, heads per wavefront
  const int lane = threadIdx.x & 63;
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int h = blockIdx.y * HPW + lane / LPH, part = lane % LPH;
  if (blockIdx.x == 0 && blockIdx.y == 0)
    for (int i = threadIdx.x; i < n_moved; i += 256) g.moved[i] = 1;   // until an update says otherwise
  if (b >= g.B) return;
  const bool live = h < g.H;
  const int64_t row = g.rows ? g.rows[b] : b;
  float v[32];
  const int64_t off = row * g.stride + (int64_t)min(h, g.H - 1) * D + 32 * part;
  if (g.fp32_in) {
    const f32x4v* p = (const f32x4v*)((const float*)g.keys + off);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const f32x4v t = p[k];
#pragma unroll
      for (int j = 0; j < 4; ++j) v[4 * k + j] = t[j];
    }
  } else {
    const u32x4* p = (const u32x4*)((const uint16_t*)g.keys + off);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const u32x4 t = p[k];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[8 * k + 2 * j] = bf2f((uint16_t)(t[j] & 0xffffu));
        v[8 * k + 2 * j + 1] = bf2f((uint16_t)(t[j] >> 16));
      }
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e) ss += v[e] * v[e];
#pragma unroll
  for (int o = 1; o < LPH; o <<= 1) ss += __shfl_xor(ss, o, 64);
  const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
  float q = 0.0f;
#pragma unroll
  for (int e = 0; e < 32; ++e) {
    v[e] *= inv;
    q += v[e] * v[e];
  }
#pragma unroll
  for (int o = 1; o < LPH; o <<= 1) q += __shfl_xor(q, o, 64);
  if (!live) return;
  f32x4v* x = (f32x4v*)(g.X + ((int64_t)h * g.B + b) * D + 32 * part);
#pragma unroll
  for (int k = 0; k < 8; ++k) x[k] = f32x4v{v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]};
  if (part == 0) g.xx[(int64_t)h * g.B + b] = q;
}

// |c|^2 of a centroid held one element per thread (threads 0..D-1 of a 128-thread group), summed by a fixed tree in
// LDS: the same bits wherever it is computed
__device__ __forceinline__ float centroid_norm2(float c, int d, int D, float* red) {
  if (d < 128) red[d] = d < D ? c * c : 0.0f;   // threads with d >= 128 only take part in the barriers
  __syncthreads();
  for (int o = 64; o >= 1; o >>= 1) {
    if (d < o) red[d] += red[d + o];
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

// start of a call: a cold start copies x of candidate init[i] into centroid i; every start computes |c|^2
__global__ __launch_bounds__(128) void mem_start_kernel(SelArgs g, const int32_t* init) {
  __shared__ float red[128];
  const int i = blockIdx.x, h = blockIdx.y, d = threadIdx.x;
  float* dst = g.C + ((int64_t)h * g.M + i) * g.D;
  float c = 0.0f;
  if (d < g.D) {
    c = init ? g.X[((int64_t)h * g.B + init[i]) * g.D + d] : dst[d];
    if (init) dst[d] = c;
  }
  const float n2 = centroid_norm2(c, d, g.D, red);
  if (d == 0) g.cc[(int64_t)h * g.M + i] = n2;
}

// ------------------------------------------------------------------------------------------------------------------
// assign: block (tile, h) takes candidates [64 tile, 64 tile + 64); wavefront w the 16 from 64 tile + 16 w. Two
// blocks per CU (68 KB of LDS each), two wavefronts per SIMD.
// MFMA 16x16x4 f32: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16] and holds D[4 (l / 16) + r][l % 16].
// The reduction dimension is visited in the order d = (l / 16) * (D / 4) + s at step s (any order of the same
// products is the same dot product), so that every lane reads D / 4 consecutive floats of its row and centroid. The
// eight 16-centroid tiles of a 128-centroid chunk accumulate side by side (eight independent MFMA chains); centroids
// past M are zeros in LDS and their distances are skipped.
template <int D>
__global__ __launch_bounds__(kAssignThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void mem_assign_kernel(SelArgs g, int it) {
  if (it > 0 && g.moved[it - 1] == 0) return;
  constexpr int KS = D / 4;   // MFMA steps per dot product
  __shared__ float cl[kCChunk * kCPitch];
  __shared__ float ccl[kCChunk];
  const int h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int kq = lane >> 4, c16 = lane & 15;
  const int b0 = blockIdx.x * kAssignRows + w * 16;
  // A operands: candidate b0 + c16, dims kq * KS .. + KS - 1 (rows past B are zeros)
  // every load below reads a valid row (indices clamped) and is issued before any of them is waited for; values of
  // rows past B are then replaced by zeros
  float a[KS];
  {
    const int b = b0 + c16;
    const float keep = b < g.B ? 1.0f : 0.0f;
    const float* xr = g.X + ((int64_t)h * g.B + min(b, g.B - 1)) * D + kq * KS;
    f32x4v t[KS / 4];
#pragma unroll
    for (int s = 0; s < KS / 4; ++s) t[s] = *(const f32x4v*)(xr + 4 * s);
#pragma unroll
    for (int s = 0; s < KS / 4; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) a[4 * s + j] = t[s][j] * keep;
  }
  float xxr[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) xxr[r] = g.xx[(int64_t)h * g.B + min(b0 + 4 * kq + r, g.B - 1)];
  float best[4];
  int besti[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    best[r] = __builtin_inff();
    besti[r] = 0;   // stays 0 only if no distance is finite (non-finite keys): still a valid cluster
  }
  const float* Ch = g.C + (int64_t)h * g.M * D;
  for (int c0 = 0; c0 < g.M; c0 += kCChunk) {
    const int nc = min(kCChunk, g.M - c0);
    __syncthreads();
    {
      constexpr int PER = kCChunk * (D / 4) / kAssignThreads;   // float4 per thread
      f32x4v t[PER];
      float ccv = 0.0f;
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int e = tid + k * kAssignThreads, i = e / (D / 4), d4 = e % (D / 4);
        t[k] = *(const f32x4v*)(Ch + (int64_t)(c0 + min(i, nc - 1)) * D + 4 * d4);
      }
      if (tid < kCChunk) ccv = g.cc[(int64_t)h * g.M + c0 + min(tid, nc - 1)];
#pragma unroll
      for (int k = 0; k < PER; ++k) {
        const int e = tid + k * kAssignThreads, i = e / (D / 4), d4 = e % (D / 4);
        const float keep = i < nc ? 1.0f : 0.0f;
        *(f32x4v*)(cl + i * kCPitch + 4 * d4) = t[k] * keep;
      }
      if (tid < kCChunk) ccl[tid] = tid < nc ? ccv : 0.0f;
    }
    __syncthreads();
    f32x4v acc[8];
#pragma unroll
    for (int t = 0; t < 8; ++t) acc[t] = f32x4v{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int s = 0; s < KS; s += 4) {
#pragma unroll
      for (int th = 0; th < 8; th += 4) {   // four tiles' operands at a time
        f32x4v bv[4];
#pragma unroll
        for (int t = 0; t < 4; ++t) bv[t] = *(const f32x4v*)(cl + (16 * (th + t) + c16) * kCPitch + kq * KS + s);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int t = 0; t < 4; ++t)
            acc[th + t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s + j], bv[t][j], acc[th + t], 0, 0, 0);
      }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int i = 16 * t + c16;
      if (i < nc) {
        const float cc = ccl[i];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float dd = (xxr[r] - 2.0f * acc[t][r]) + cc;
          if (dd < best[r]) {    // centroids visited in ascending order: the first minimum stays
            best[r] = dd;
            besti[r] = c0 + i;
          }
        }
      }
    }
  }
  // across the 16 lanes that hold the same 4 candidates: the smallest distance, then the lowest centroid
#pragma unroll
  for (int o = 1; o < 16; o <<= 1) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float od = __shfl_xor(best[r], o, 64);
      const int oi = __shfl_xor(besti[r], o, 64);
      if (od < best[r] || (od == best[r] && oi < besti[r])) {
        best[r] = od;
        besti[r] = oi;
      }
    }
  }
  if (c16 == 0) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int b = b0 + 4 * kq + r;
      if (b < g.B) {
        g.z[(int64_t)h * g.B + b] = besti[r];
        g.dist[(int64_t)h * g.B + b] = best[r];
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------------------------
// group: one workgroup of 16 wavefronts per head, a stable counting sort of the candidates by cluster. Wavefront w
// owns the contiguous candidates [w n / 16, (w + 1) n / 16) rounded to 64; it counts them per cluster, the counts
// are scanned cluster by cluster and, within a cluster, wavefront by wavefront, and then every wavefront places its
// candidates in order: lanes with the same cluster find each other through ballots over the cluster's bits, so a
// candidate's place is its wavefront's running count for the cluster plus its rank among the earlier lanes.
__global__ __launch_bounds__(1024) void mem_group_kernel(SelArgs g, int it, int bits) {
  // the moved flag of this iteration starts at 0 (prep set every flag to 1, so that iteration 0 always runs); the
  // update after this kernel raises it
  if (blockIdx.x == 0 && threadIdx.x == 0 && it < g.iters) g.moved[it] = 0;
  if (it > 0 && g.moved[it - 1] == 0) return;
  __shared__ int cnt[16 * kMaxClusters];   // cnt[w * M + c]
  __shared__ int wsum[16];
  const int h = blockIdx.x, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int32_t* zh = g.z + (int64_t)h * g.B;
  const int per = ((g.B + 16 * 64 - 1) / (16 * 64)) * 64;
  const int lo = min(g.B, w * per), hi = min(g.B, lo + per);
  for (int i = tid; i < 16 * g.M; i += 1024) cnt[i] = 0;
  __syncthreads();
  for (int b = lo + lane; b < hi; b += 64) atomicAdd(&cnt[w * g.M + zh[b]], 1);
  __syncthreads();
  // per cluster c (thread c, and c + 1024 ... past 1024 clusters, which kMaxClusters excludes): its total and the
  // exclusive prefix over the wavefronts
  const int c = tid;
  int tot = 0;
  if (c < g.M)
    for (int x = 0; x < 16; ++x) {
      const int n = cnt[x * g.M + c];
      cnt[x * g.M + c] = tot;
      tot += n;
    }
  // exclusive scan of the totals over the clusters: within each wavefront by shuffles, then over the wavefronts
  int incl = tot;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int y = __shfl_up(incl, o, 64);
    if (lane >= o) incl += y;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  int before = 0;
  for (int x = 0; x < w; ++x) before += wsum[x];
  const int start = before + incl - tot;
  int32_t* st = g.start + (int64_t)h * (g.M + 1);
  if (c < g.M) {
    st[c] = start;
    for (int x = 0; x < 16; ++x) cnt[x * g.M + c] += start;
  }
  if (c == 0) st[g.M] = g.B;
  __syncthreads();
  int32_t* oh = g.order + (int64_t)h * g.B;
  const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  int* mine = cnt + w * g.M;
  for (int b0 = lo; b0 < hi; b0 += 64) {   // the same trip count in every lane of the wavefront
    const int b = b0 + lane;
    const bool in = b < hi;
    const int cl = in ? zh[b] : -1;
    uint64_t same = __ballot(in);
    for (int k = 0; k < bits; ++k) {
      const uint64_t ones = __ballot(in && ((cl >> k) & 1));
      same &= ((cl >> k) & 1) ? ones : ~ones;
    }
    const int rank = __popcll(same & below);
    const int base = in ? mine[cl] : 0;
    if (in) oh[base + rank] = b;
    // every lane has read its base before the group's last lane moves the count on (one wavefront, in order)
    __builtin_amdgcn_wave_barrier();
    if (in && (same >> lane) == 1ull) mine[cl] = base + rank + 1;
    __builtin_amdgcn_wave_barrier();
  }
}

// ------------------------------------------------------------------------------------------------------------------
// update: block (i, h) averages cluster i's members in their fixed order: four groups of 128 threads take the members
// j = q, q + 4, ... (group q), one element of D per thread, and the four partial sums are added in group order
__global__ __launch_bounds__(512) void mem_update_kernel(SelArgs g, int it) {
  if (it > 0 && g.moved[it - 1] == 0) return;
  __shared__ float part[4][128];
  __shared__ float red[128];
  const int i = blockIdx.x, h = blockIdx.y, d = threadIdx.x & 127, q = threadIdx.x >> 7;
  const int32_t* st = g.start + (int64_t)h * (g.M + 1);
  const int a = st[i], e = st[i + 1];
  if (a == e) return;   // empty: the centroid (and its |c|^2) stays
  const int32_t* oh = g.order + (int64_t)h * g.B;
  const float* Xh = g.X + (int64_t)h * g.B * g.D;
  float s = 0.0f;
  if (d < g.D) {
    int j = a + q;
    for (; j + 12 < e; j += 16) {
      const int r0 = oh[j], r1 = oh[j + 4], r2 = oh[j + 8], r3 = oh[j + 12];
      const float x0 = Xh[(int64_t)r0 * g.D + d], x1 = Xh[(int64_t)r1 * g.D + d];
      const float x2 = Xh[(int64_t)r2 * g.D + d], x3 = Xh[(int64_t)r3 * g.D + d];
      s += x0;
      s += x1;
      s += x2;
      s += x3;
    }
    for (; j < e; j += 4) s += Xh[(int64_t)oh[j] * g.D + d];
  }
  part[q][d] = s;
  __syncthreads();
  float c = 0.0f;
  bool change = false;
  if (q == 0 && d < g.D) {
    c = ((part[0][d] + part[1][d]) + part[2][d]) + part[3][d];
    c = c / (float)(e - a);
    float* cp = g.C + ((int64_t)h * g.M + i) * g.D + d;
    change = *cp != c;
    *cp = c;
  }
  // |c|^2 by the fixed tree (every thread takes part in the barriers; group 0 holds the values)
  const float n2 = centroid_norm2(q == 0 ? c : 0.0f, q == 0 ? d : 128, g.D, red);
  if (threadIdx.x == 0) g.cc[(int64_t)h * g.M + i] = n2;
  if (__syncthreads_or(change) && threadIdx.x == 0) atomicOr(&g.moved[it], 1);
}

// ------------------------------------------------------------------------------------------------------------------
// medoid: one workgroup per head; wavefront w takes clusters w, w + 16, ...; rep / valid compacted in cluster order
__global__ __launch_bounds__(1024) void mem_medoid_kernel(SelArgs g) {
  __shared__ int pick[kMaxClusters];
  __shared__ int slot[kMaxClusters];
  const int h = blockIdx.x, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int32_t* st = g.start + (int64_t)h * (g.M + 1);
  const int32_t* oh = g.order + (int64_t)h * g.B;
  const float* dh = g.dist + (int64_t)h * g.B;
  for (int i = w; i < g.M; i += 16) {
    const int a = st[i], e = st[i + 1];
    float bd = __builtin_inff();
    int bb = 0x7fffffff;
    for (int j = a + lane; j < e; j += 64) {
      const int b = oh[j];
      const float dd = dh[b];
      if (dd < bd || (dd == bd && b < bb)) {
        bd = dd;
        bb = b;
      }
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
      const float od = __shfl_xor(bd, o, 64);
      const int ob = __shfl_xor(bb, o, 64);
      if (od < bd || (od == bd && ob < bb)) {
        bd = od;
        bb = ob;
      }
    }
    if (lane == 0) pick[i] = a < e ? bb : -1;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int r = 0;
    for (int i = 0; i < g.M; ++i) slot[i] = pick[i] >= 0 ? r++ : -1;
  }
  __syncthreads();
  int64_t* rp = g.rep + (int64_t)h * g.M;
  uint8_t* vp = g.valid + (int64_t)h * g.M;
  for (int i = threadIdx.x; i < g.M; i += 1024) {
    rp[i] = 0;
    vp[i] = 0;
  }
  __syncthreads();
  for (int i = threadIdx.x; i < g.M; i += 1024)
    if (slot[i] >= 0) {
      rp[slot[i]] = pick[i];
      vp[slot[i]] = 1;
    }
}

// ------------------------------------------------------------------------------------------------------------------
// foreign keys of the head-major attention: block (piece i, head h) appends, after piece i's local keys, the rows of
// head h's valid representatives that belong to another scene (when the piece reads the memory), in rep order
__global__ __launch_bounds__(256) void mem_index_kernel(const int64_t* rep, const uint8_t* valid, const int64_t* cand_row,
                                                        const int64_t* cand_scene, const int64_t* piece_scene,
                                                        const uint8_t* piece_mem, const int32_t* piece_len,
                                                        const int32_t* k_off, int32_t* kidx, int32_t* k_len, int n,
                                                        int H, int M) {
  __shared__ int wave_cnt[4];
  const int i = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int seg = h * n + i;
  const int base = k_off[seg] + piece_len[i];
  const int64_t scene = piece_scene[i];
  const bool reads = piece_mem[i] != 0;
  int total = 0;
  for (int r0 = 0; r0 < M; r0 += 256) {
    const int r = r0 + tid;
    bool f = false;
    int64_t row = 0;
    if (reads && r < M && valid[(int64_t)h * M + r]) {
      const int64_t c = rep[(int64_t)h * M + r];
      f = cand_scene[c] != scene;
      row = cand_row[c];
    }
    const uint64_t bal = __ballot(f);
    if (lane == 0) wave_cnt[w] = __popcll(bal);
    __syncthreads();
    int before = total;
    for (int x = 0; x < w; ++x) before += wave_cnt[x];
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    if (f) kidx[base + before + __popcll(bal & below)] = (int32_t)(row * H + h);
    total += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    __syncthreads();
  }
  if (tid == 0) k_len[seg] = piece_len[i] + total;
}

// The multi-head form of the per-call key lists (the packed K / V hold every head of a row, and each head's
// representatives sit in its own head slot after the piece's local keys): block (i, h) writes, for slot r < M of piece
// i and head h, src = cand_row[c] * H + h (the representative's row in the [rows * H, 1, D] view of the key buffer, or
// -1 for an unused slot) and dst = (k_off[i] + piece_len[i] + r) * H + h (its row in that view of the packed buffer),
// in the representatives' order, and k_len_head[i * H + h] = piece_len[i] + the count. Pieces that do not read the
// memory get no representatives.
__global__ __launch_bounds__(256) void mem_foreign_kernel(const int64_t* rep, const uint8_t* valid,
                                                          const int64_t* cand_row, const int64_t* cand_scene,
                                                          const int64_t* piece_scene, const uint8_t* piece_mem,
                                                          const int32_t* piece_len, const int32_t* k_off,
                                                          int32_t* fsrc, int32_t* fdst, int32_t* k_len_head, int n,
                                                          int H, int M) {
  __shared__ int wave_cnt[4];
  const int i = blockIdx.x, h = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int64_t slot0 = ((int64_t)i * H + h) * M;
  const int64_t dst0 = (int64_t)k_off[i] + piece_len[i];
  const int64_t scene = piece_scene[i];
  const bool reads = piece_mem[i] != 0;
  for (int r = tid; r < M; r += 256) {
    fsrc[slot0 + r] = -1;
    fdst[slot0 + r] = (int32_t)((dst0 + r) * H + h);
  }
  __syncthreads();
  int total = 0;
  for (int r0 = 0; r0 < M; r0 += 256) {
    const int r = r0 + tid;
    bool f = false;
    int64_t row = 0;
    if (reads && r < M && valid[(int64_t)h * M + r]) {
      const int64_t c = rep[(int64_t)h * M + r];
      f = cand_scene[c] != scene;
      row = cand_row[c];
    }
    const uint64_t bal = __ballot(f);
    if (lane == 0) wave_cnt[w] = __popcll(bal);
    __syncthreads();
    int before = total;
    for (int x = 0; x < w; ++x) before += wave_cnt[x];
    const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    if (f) fsrc[slot0 + before + __popcll(bal & below)] = (int32_t)(row * H + h);
    total += wave_cnt[0] + wave_cnt[1] + wave_cnt[2] + wave_cnt[3];
    __syncthreads();
  }
  if (tid == 0) k_len_head[(int64_t)i * H + h] = piece_len[i] + total;
}

struct WsParts {
  int64_t X, xx, cc, z, dist, order, start, moved, total;
};

WsParts ws_parts(int B, int H, int D, int M, int iters) {
  WsParts p;
  int64_t o = 0;
  auto take = [&](int64_t bytes) {
    const int64_t at = o;
    o += (bytes + 255) / 256 * 256;
    return at;
  };
  p.X = take((int64_t)H * B * D * 4);
  p.xx = take((int64_t)H * B * 4);
  p.cc = take((int64_t)H * M * 4);
  p.z = take((int64_t)H * B * 4);
  p.dist = take((int64_t)H * B * 4);
  p.order = take((int64_t)H * B * 4);
  p.start = take((int64_t)H * (M + 1) * 4);
  p.moved = take((int64_t)(iters + 1) * 4);
  p.total = o;
  return p;
}

}  // namespace
}  // namespace onereel

using namespace onereel;

extern "C" int64_t or_memory_select_workspace_size(int32_t B, int32_t H, int32_t D, int32_t M, int32_t iters) {
  if (B < 1 || H < 1 || M < 1 || iters < 0 || (D != 64 && D != 128)) return -1;
  return ws_parts(B, H, D, M, iters).total;
}

extern "C" int or_memory_select(const void* keys, int32_t fp32_keys, const int32_t* rows, int64_t key_row_stride,
                                int32_t B, int32_t H, int32_t D, int32_t M, float* centroids, const int32_t* init,
                                int32_t iters, int64_t* rep, uint8_t* valid, void* workspace, int64_t workspace_bytes,
                                void* stream) {
  if (B < 1 || H < 1 || (D != 64 && D != 128))
    return fail_arg("or_memory_select: need B >= 1, H >= 1 and D 64 or 128 (B=%d H=%d D=%d)", B, H, D);
  if (M < 1 || M > B || M > kMaxClusters)
    return fail_arg("or_memory_select: M=%d outside [1, min(B=%d, %d)]", M, B, kMaxClusters);
  if (iters < 0 || iters > 1000) return fail_arg("or_memory_select: iters=%d outside [0, 1000]", iters);
  if (!keys || !centroids || !rep || !valid || key_row_stride < (int64_t)H * D)
    return fail_arg("or_memory_select: keys, centroids, rep and valid are required, rows of at least H*D elements");
  const WsParts wp = ws_parts(B, H, D, M, iters);
  if (!workspace || workspace_bytes < wp.total || ((uintptr_t)workspace & 255u))
    return fail_arg("or_memory_select: a 256-byte aligned workspace of %lld bytes is needed", (long long)wp.total);
  if (((uintptr_t)centroids & 15u) || ((uintptr_t)keys & 15u) || key_row_stride % (fp32_keys ? 4 : 8))
    return fail_arg("or_memory_select: centroids and keys must be 16-byte aligned and the key row stride a multiple "
                    "of 16 bytes");
  char* w = (char*)workspace;
  SelArgs g;
  g.keys = keys;
  g.rows = rows;
  g.stride = key_row_stride;
  g.B = B;
  g.H = H;
  g.D = D;
  g.M = M;
  g.fp32_in = fp32_keys ? 1 : 0;
  g.iters = iters;
  g.X = (float*)(w + wp.X);
  g.xx = (float*)(w + wp.xx);
  g.cc = (float*)(w + wp.cc);
  g.C = centroids;
  g.z = (int32_t*)(w + wp.z);
  g.dist = (float*)(w + wp.dist);
  g.order = (int32_t*)(w + wp.order);
  g.start = (int32_t*)(w + wp.start);
  g.moved = (int32_t*)(w + wp.moved);
  g.rep = rep;
  g.valid = valid;
  hipStream_t st = (hipStream_t)stream;
  if (D == 128) hipLaunchKernelGGL(mem_prep_kernel<128>, dim3((B + 3) / 4, (H + 15) / 16), dim3(256), 0, st, g, iters + 1);
  else hipLaunchKernelGGL(mem_prep_kernel<64>, dim3((B + 3) / 4, (H + 31) / 32), dim3(256), 0, st, g, iters + 1);
  if (int rc = check_hip(hipGetLastError(), "mem_prep_kernel launch")) return rc;
  hipLaunchKernelGGL(mem_start_kernel, dim3(M, H), dim3(128), 0, st, g, init);
  if (int rc = check_hip(hipGetLastError(), "mem_start_kernel launch")) return rc;
  int bits = 0;
  while ((1 << bits) < M) ++bits;
  const dim3 agrid((B + kAssignRows - 1) / kAssignRows, H);
  for (int it = 0; it <= iters; ++it) {
    if (D == 128) hipLaunchKernelGGL(mem_assign_kernel<128>, agrid, dim3(kAssignThreads), 0, st, g, it);
    else hipLaunchKernelGGL(mem_assign_kernel<64>, agrid, dim3(kAssignThreads), 0, st, g, it);
    hipLaunchKernelGGL(mem_group_kernel, dim3(H), dim3(1024), 0, st, g, it, bits);
    if (it < iters) hipLaunchKernelGGL(mem_update_kernel, dim3(M, H), dim3(512), 0, st, g, it);
    if (int rc = check_hip(hipGetLastError(), "k-means launch")) return rc;
  }
  hipLaunchKernelGGL(mem_medoid_kernel, dim3(H), dim3(1024), 0, st, g);
  return check_hip(hipGetLastError(), "mem_medoid_kernel launch");
}

extern "C" int or_memory_index(const int64_t* rep, const uint8_t* valid, const int64_t* cand_row,
                               const int64_t* cand_scene, const int64_t* piece_scene, const uint8_t* piece_mem,
                               const int32_t* piece_len, const int32_t* k_off, int32_t n_pieces, int32_t H, int32_t M,
                               int32_t* kidx, int32_t* k_len, void* stream) {
  if (n_pieces < 1 || H < 1 || M < 1 || n_pieces > 65535 || H > 65535)
    return fail_arg("or_memory_index: need 1 <= pieces, heads <= 65535 and M >= 1 (n=%d H=%d M=%d)", n_pieces, H, M);
  if (!rep || !valid || !cand_row || !cand_scene || !piece_scene || !piece_mem || !piece_len || !k_off || !kidx || !k_len)
    return fail_arg("or_memory_index: every array is required");
  hipLaunchKernelGGL(mem_index_kernel, dim3(n_pieces, H), dim3(256), 0, (hipStream_t)stream, rep, valid, cand_row,
                     cand_scene, piece_scene, piece_mem, piece_len, k_off, kidx, k_len, n_pieces, H, M);
  return check_hip(hipGetLastError(), "mem_index_kernel launch");
}

extern "C" int or_memory_foreign(const int64_t* rep, const uint8_t* valid, const int64_t* cand_row,
                                 const int64_t* cand_scene, const int64_t* piece_scene, const uint8_t* piece_mem,
                                 const int32_t* piece_len, const int32_t* k_off, int32_t n_pieces, int32_t H,
                                 int32_t M, int32_t* fsrc, int32_t* fdst, int32_t* k_len_head, void* stream) {
  if (n_pieces < 1 || H < 1 || M < 1 || n_pieces > 65535 || H > 65535)
    return fail_arg("or_memory_foreign: need 1 <= pieces, heads <= 65535 and M >= 1 (n=%d H=%d M=%d)", n_pieces, H, M);
  if (!rep || !valid || !cand_row || !cand_scene || !piece_scene || !piece_mem || !piece_len || !k_off || !fsrc ||
      !fdst || !k_len_head)
    return fail_arg("or_memory_foreign: every array is required");
  hipLaunchKernelGGL(mem_foreign_kernel, dim3(n_pieces, H), dim3(256), 0, (hipStream_t)stream, rep, valid, cand_row,
                     cand_scene, piece_scene, piece_mem, piece_len, k_off, fsrc, fdst, k_len_head, n_pieces, H, M);
  return check_hip(hipGetLastError(), "mem_foreign_kernel launch");
}
