// Scene layout on the device: one launch emits cu_seqlens, per-row gather indices, scene-RoPE rows and the table
// rows of _move_shared for every packed scope of one layer.
//
// Reference: _segments (src/onereel/models/hunyuan15.py:153-170) as Processor.scene calls it on one GPU (:212-251),
// SceneLayout (src/onereel/layout.py:43-78), comm.runs / frame_tokens (src/onereel/parallel/comm.py:84-85,115-123),
// cu_seqlens (src/onereel/attention.py:28-29), scene_rope_rows (hunyuan15.py:443-454), frame_position /
// adjacent_positions / shared_positions (hunyuan15.py:92-124), _move_shared's rows a, a + d (hunyuan15.py:136-145).
//
// Every block first derives the per-scene quantities in LDS: its first wavefront does it alone, one lane per scene
// (at most 64 scenes, 128 segments), with cross-lane prefix sums and no block barrier until the tables are complete.
// Then the grid writes the per-row arrays with a grid-stride loop: int32 stores, fully coalesced.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace onereel {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxSeg = 2 * OR_MAX_SCENES;

// segment s: with text, V_j = 2j and T_j = 2j + 1; without, V_j = j
struct SegTable {
  int n_seg;
  int cu_q[kMaxSeg + 1];
  int cu_k[kMaxSeg + 1];
};

__host__ __device__ inline int seg_scene(int with_text, int s) { return with_text ? s >> 1 : s; }
__host__ __device__ inline bool seg_is_text(int with_text, int s) { return with_text && (s & 1); }

// query / key counts of segment s
__host__ __device__ inline void seg_lengths(const LayoutDerived& L, int s, int* lq, int* lk) {
  const int j = seg_scene(L.with_text, s);
  const int own = (L.hi[j] - L.lo[j]) * L.T;
  const int txt = L.t1[j] - L.t0[j];
  if (seg_is_text(L.with_text, s)) {
    *lq = txt;
    *lk = own + txt;
  } else {
    *lq = own;
    *lk = own + (L.sh_ptr[j + 1] - L.sh_ptr[j]) * L.T + txt;
  }
}

// host: sequential derivation (the device runs the same helpers, one thread per scene)
int derive_host(const or_layout_desc& d, LayoutDerived& L) {
  L.n_scenes = d.n_scenes;
  L.T = d.T;
  L.with_text = d.with_text;
  L.scene_rope = d.scene_rope;
  L.adjacent = d.adjacent;
  L.text_rows = d.text_rows;
  int f = 0, t = 0;
  for (int j = 0; j < d.n_scenes; ++j) {
    L.lo[j] = f;
    f += d.lengths[j];
    L.hi[j] = f;
    L.t0[j] = t;
    if (d.with_text) t += d.counts[j];
    L.t1[j] = t;
  }
  L.F = f;
  const int nr = d.n_rope_lengths > 0 ? d.n_rope_lengths : d.n_scenes;
  const int* rl = d.n_rope_lengths > 0 ? d.rope_lengths : d.lengths;
  L.n_rope = nr;
  L.rope_start[0] = 0;
  for (int s = 0; s < nr; ++s) L.rope_start[s + 1] = L.rope_start[s] + rl[s];
  int n = 0;
  for (int j = 0; j < d.n_scenes; ++j) {
    L.sh_ptr[j] = n;
    int c = scene_shared_frames(d, L.lo, L.hi, j, L.sh + n, kMaxShared - n);
    if (c < 0) return -1;
    n += c;
  }
  L.sh_ptr[d.n_scenes] = n;
  for (int j = 0; j < d.n_scenes; ++j) {
    const int a = L.sh_ptr[j], c = L.sh_ptr[j + 1] - a;
    for (int i = 0; i < c; ++i) L.sh_dst[a + i] = shared_dst(L, j, L.sh + a, c, L.sh[a + i]);
  }
  return 0;
}

// ---------------------------------------------------------------------------------------------------------------
// device

// inclusive prefix sum over the 64 lanes of a wavefront
__device__ inline int wave_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int x = __shfl_up(v, o, 64);
    if (lane >= o) v += x;
  }
  return v;
}

// LDS writes of this wavefront's lanes become visible to its other lanes (no block barrier)
__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ inline int upper_bound(const int* a, int n, int x) {  // first i in [0, n) with a[i] > x
  int lo = 0, hi = n;
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if (a[mid] <= x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

struct RowOut {
  int32_t *q_src, *q_rope, *k_src, *k_rope, *k_move_a, *k_move_b;
};

__global__ __launch_bounds__(kThreads) void layout_kernel(const or_layout_desc d, RowOut out, int32_t* cu_q_out,
                                                          int32_t* cu_k_out, int32_t* seg_q_src_out,
                                                          int64_t sum_q, int64_t sum_k) {
  __shared__ LayoutDerived L;
  __shared__ SegTable S;
  __shared__ int sh_tmp[kMaxShared];
  const int tid = threadIdx.x;
  const int ns = d.n_scenes;
  const int n_seg = d.with_text ? 2 * ns : ns;

  if (tid < 64) {
    const int lane = tid;
    // 1. frame / text / rope prefix sums (lane j: scene j)
    const int len = lane < ns ? d.lengths[lane] : 0;
    const int lo = wave_scan(len) - len;
    const int cnt = (lane < ns && d.with_text) ? d.counts[lane] : 0;
    const int t0 = wave_scan(cnt) - cnt;
    const int nr = d.n_rope_lengths > 0 ? d.n_rope_lengths : ns;
    const int rl = lane < nr ? (d.n_rope_lengths > 0 ? d.rope_lengths[lane] : d.lengths[lane]) : 0;
    const int rs = wave_scan(rl) - rl;
    if (lane < ns) {
      L.lo[lane] = lo;
      L.hi[lane] = lo + len;
      L.t0[lane] = t0;
      L.t1[lane] = t0 + cnt;
    }
    if (lane < nr) L.rope_start[lane] = rs;
    if (lane == nr - 1) L.rope_start[nr] = rs + rl;
    if (lane == 0) {
      L.n_scenes = ns;
      L.T = d.T;
      L.with_text = d.with_text;
      L.scene_rope = d.scene_rope;
      L.adjacent = d.adjacent;
      L.text_rows = d.text_rows;
      L.n_rope = nr;
    }
    if (lane == ns - 1) L.F = lo + len;
    wave_lds_sync();

    // 2. shared frames per scene: upper-bound slots, then compaction (host validation keeps them within kMaxShared)
    int ub = 0;
    if (lane < ns) {
      const int k = d.halo;
      if (k > 0 && lane > 0 && (d.sides == 0 || d.sides == 1)) ub += min(k, d.lengths[lane - 1]);
      if (k > 0 && lane + 1 < ns && (d.sides == 0 || d.sides == 2)) ub += min(k, d.lengths[lane + 1]);
      ub += d.extra_ptr[lane + 1] - d.extra_ptr[lane];
    }
    const int off = wave_scan(ub) - ub;
    int n = 0;
    if (lane < ns) n = scene_shared_frames(d, L.lo, L.hi, lane, sh_tmp + off, ub);
    const int ptr = wave_scan(n) - n;
    if (lane < ns) {
      L.sh_ptr[lane] = ptr;
      for (int i = 0; i < n; ++i) L.sh[ptr + i] = sh_tmp[off + i];
    }
    if (lane == ns - 1) L.sh_ptr[ns] = ptr + n;
    wave_lds_sync();
    if (lane < ns && d.adjacent) {
      for (int i = 0; i < n; ++i) L.sh_dst[ptr + i] = shared_dst(L, lane, L.sh + ptr, n, L.sh[ptr + i]);
    }
    wave_lds_sync();

    // 3. segments and cu_seqlens: lane l holds segments l and 64 + l
    int lq0 = 0, lk0 = 0, lq1 = 0, lk1 = 0;
    if (lane < n_seg) seg_lengths(L, lane, &lq0, &lk0);
    if (64 + lane < n_seg) seg_lengths(L, 64 + lane, &lq1, &lk1);
    const int cq0 = wave_scan(lq0), ck0 = wave_scan(lk0);
    const int tq = __shfl(cq0, 63, 64), tk = __shfl(ck0, 63, 64);
    const int cq1 = wave_scan(lq1) + tq, ck1 = wave_scan(lk1) + tk;
    if (lane < n_seg) {
      S.cu_q[lane] = cq0 - lq0;
      S.cu_k[lane] = ck0 - lk0;
    }
    if (64 + lane < n_seg) {
      S.cu_q[64 + lane] = cq1 - lq1;
      S.cu_k[64 + lane] = ck1 - lk1;
    }
    if (lane == 63) {
      S.cu_q[n_seg] = cq1;
      S.cu_k[n_seg] = ck1;
      S.n_seg = n_seg;
    }
  }
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int s = tid; s <= n_seg; s += kThreads) {
      if (cu_q_out) cu_q_out[s] = S.cu_q[s];
      if (cu_k_out) cu_k_out[s] = S.cu_k[s];
      if (seg_q_src_out && s < n_seg) {
        const int j = seg_scene(L.with_text, s);
        seg_q_src_out[s] = seg_is_text(L.with_text, s) ? L.F * L.T + L.t0[j] : L.lo[j] * L.T;
      }
    }
  }

  // 4. per-row arrays
  const int T = L.T;
  const int n_video = L.F * T;
  const int64_t total = sum_q + sum_k;
  for (int64_t r = (int64_t)blockIdx.x * kThreads + tid; r < total; r += (int64_t)gridDim.x * kThreads) {
    if (r < sum_q) {
      const int rq = (int)r;
      const int s = upper_bound(S.cu_q, n_seg + 1, rq) - 1;
      const int o = rq - S.cu_q[s];
      const int j = seg_scene(L.with_text, s);
      int src, rope;
      if (seg_is_text(L.with_text, s)) {
        src = n_video + L.t0[j] + o;
        rope = -1;
      } else {
        src = L.lo[j] * T + o;
        rope = rope_row_of_token(L, src);
      }
      if (out.q_src) out.q_src[rq] = src;
      if (out.q_rope) out.q_rope[rq] = rope;
    } else {
      const int rk = (int)(r - sum_q);
      const int s = upper_bound(S.cu_k, n_seg + 1, rk) - 1;
      const int o = rk - S.cu_k[s];
      const int j = seg_scene(L.with_text, s);
      const bool text_seg = seg_is_text(L.with_text, s);
      const int own = L.hi[j] - L.lo[j];
      const int nsh = text_seg ? 0 : L.sh_ptr[j + 1] - L.sh_ptr[j];
      const int nvid = (own + nsh) * T;
      int src, rope = -1, ma = -1, mb = -1;
      if (o < nvid) {
        const int i = o / T, sp = o - (o / T) * T;
        if (i < own) {
          src = (L.lo[j] + i) * T + sp;
          rope = rope_row_of_token(L, src);
        } else {
          const int e = L.sh_ptr[j] + (i - own);
          const int f = L.sh[e];
          src = f * T + sp;
          if (L.adjacent) {
            const int dst = L.sh_dst[e];
            const int dd = dst - frame_position(L, f);
            const int a = dd >= 0 ? 0 : -dd;
            rope = dst * T + sp;
            ma = a * T + sp;
            mb = (a + dd) * T + sp;
          } else {
            rope = rope_row_of_token(L, src);
          }
        }
      } else {
        src = n_video + L.t0[j] + (o - nvid);
      }
      if (out.k_src) out.k_src[rk] = src;
      if (out.k_rope) out.k_rope[rk] = rope;
      if (out.k_move_a) out.k_move_a[rk] = ma;
      if (out.k_move_b) out.k_move_b[rk] = mb;
    }
  }
}

}  // namespace

// ---------------------------------------------------------------------------------------------------------------
// errors (thread-local message)

static thread_local char g_err[512];

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int fail_arg(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return -1;
}

int check_hip(hipError_t e, const char* what) {
  if (e == hipSuccess) return 0;
  set_error("%s: %s", what, hipGetErrorString(e));
  return -2;
}

}  // namespace onereel

using namespace onereel;

extern "C" const char* or_last_error(void) { return g_err; }

extern "C" const char* or_version(void) { return "onereel_hip 0.1 gfx950"; }

// validation + sizes (host); the same derivation the kernel runs
static int plan_impl(const or_layout_desc* dp, or_layout_sizes* sz, LayoutDerived* Lout) {
  if (!dp) return fail_arg("or_layout_plan: desc is NULL");
  const or_layout_desc& d = *dp;
  if (d.n_scenes < 1 || d.n_scenes > OR_MAX_SCENES)
    return fail_arg("n_scenes %d outside [1, %d]", d.n_scenes, OR_MAX_SCENES);
  if (d.T < 1) return fail_arg("T must be positive (got %d)", d.T);
  if (d.halo < 0) return fail_arg("halo must be >= 0 (got %d)", d.halo);
  if (d.sides < 0 || d.sides > 2) return fail_arg("sides must be 0 'adj', 1 'prev' or 2 'next' (got %d)", d.sides);
  if (d.n_rope_lengths < 0 || d.n_rope_lengths > OR_MAX_SCENES)
    return fail_arg("n_rope_lengths %d outside [0, %d]", d.n_rope_lengths, OR_MAX_SCENES);
  int64_t F = 0, ctext = 0;
  for (int j = 0; j < d.n_scenes; ++j) {
    if (d.lengths[j] <= 0) return fail_arg("scene %d has %d frames: lengths must be positive", j, d.lengths[j]);
    F += d.lengths[j];
    if (d.with_text) {
      if (d.counts[j] < 0) return fail_arg("sentence %d has a negative token count", j);
      ctext += d.counts[j];
    }
  }
  if (d.with_text && ctext > d.text_rows)
    return fail_arg("text counts sum to %lld but only %d text rows are given", (long long)ctext, d.text_rows);
  if (d.extra_ptr[0] != 0) return fail_arg("extra_ptr[0] must be 0");
  for (int j = 0; j < d.n_scenes; ++j)
    if (d.extra_ptr[j + 1] < d.extra_ptr[j]) return fail_arg("extra_ptr must be non-decreasing");
  if (d.extra_ptr[d.n_scenes] > OR_MAX_EXTRA)
    return fail_arg("%d extra frames exceed the maximum %d", d.extra_ptr[d.n_scenes], OR_MAX_EXTRA);
  for (int e = 0; e < d.extra_ptr[d.n_scenes]; ++e)
    if (d.extra[e] < 0 || d.extra[e] >= F) return fail_arg("extra frame %d outside [0, %lld)", d.extra[e], (long long)F);
  int64_t rope_frames = F;
  if (d.n_rope_lengths > 0) {
    rope_frames = 0;
    for (int s = 0; s < d.n_rope_lengths; ++s) {
      if (d.rope_lengths[s] <= 0) return fail_arg("rope_lengths must be positive");
      rope_frames += d.rope_lengths[s];
    }
  }
  if (d.scene_rope && rope_frames < F)
    return fail_arg("rope_lengths cover %lld frames, fewer than the layout's %lld", (long long)rope_frames, (long long)F);
  // upper bound of the device's slot allocation
  int64_t ub = 0;
  for (int j = 0; j < d.n_scenes; ++j) {
    if (d.halo > 0 && j > 0 && (d.sides == 0 || d.sides == 1)) ub += d.halo < d.lengths[j - 1] ? d.halo : d.lengths[j - 1];
    if (d.halo > 0 && j + 1 < d.n_scenes && (d.sides == 0 || d.sides == 2))
      ub += d.halo < d.lengths[j + 1] ? d.halo : d.lengths[j + 1];
    ub += d.extra_ptr[j + 1] - d.extra_ptr[j];
  }
  if (ub > kMaxShared) return fail_arg("%lld shared-frame entries exceed the maximum %d", (long long)ub, kMaxShared);
  if (F * (int64_t)d.T + d.text_rows >= (int64_t)1 << 31) return fail_arg("layout rows exceed int32");

  static thread_local LayoutDerived Lh;
  LayoutDerived& L = Lout ? *Lout : Lh;
  if (derive_host(d, L) != 0) return fail_arg("shared-frame lists overflow");
  const int n_seg = d.with_text ? 2 * d.n_scenes : d.n_scenes;
  int64_t sq = 0, sk = 0, mq = 0, mk = 0, max_rope = -1;
  for (int s = 0; s < n_seg; ++s) {
    int lq, lk;
    seg_lengths(L, s, &lq, &lk);
    sq += lq;
    sk += lk;
    mq = lq > mq ? lq : mq;
    mk = lk > mk ? lk : mk;
  }
  if (sq >= ((int64_t)1 << 31) || sk >= ((int64_t)1 << 31)) return fail_arg("packed rows exceed int32");
  // rotary rows: own tokens, shared frames at their source or adjacent position, move rows
  for (int f = 0; f < L.F; ++f) {
    int64_t p = L.scene_rope ? frame_position(L, f) : f;
    if (p * d.T + d.T - 1 > max_rope) max_rope = p * d.T + d.T - 1;
  }
  if (d.adjacent) {
    for (int j = 0; j < d.n_scenes; ++j)
      for (int e = L.sh_ptr[j]; e < L.sh_ptr[j + 1]; ++e) {
        int64_t dst = L.sh_dst[e];
        int64_t dd = dst - frame_position(L, L.sh[e]);
        int64_t a = dd >= 0 ? 0 : -dd;
        int64_t m = dst > a + dd ? dst : a + dd;
        m = m > a ? m : a;
        if (m * d.T + d.T - 1 > max_rope) max_rope = m * d.T + d.T - 1;
        if (dst < 0) return fail_arg("shared frame %d of scene %d moves to negative position %lld", L.sh[e], j, (long long)dst);
      }
  }
  if (sz) {
    sz->n_seg = n_seg;
    sz->sum_q = sq;
    sz->sum_k = sk;
    sz->max_q = mq;
    sz->max_k = mk;
    sz->n_video = (int64_t)L.F * d.T;
    sz->max_rope_row = max_rope;
  }
  return 0;
}

extern "C" int or_layout_plan(const or_layout_desc* desc, or_layout_sizes* sizes) {
  return plan_impl(desc, sizes, nullptr);
}

extern "C" int or_layout_build(const or_layout_desc* desc, const or_layout_out* out, void* stream) {
  or_layout_sizes sz;
  int rc = plan_impl(desc, &sz, nullptr);
  if (rc) return rc;
  if (!out) return fail_arg("or_layout_build: out is NULL");
  RowOut ro{out->q_src, out->q_rope, out->k_src, out->k_rope, out->k_move_a, out->k_move_b};
  const int64_t total = sz.sum_q + sz.sum_k;
  int64_t blocks = (total + kThreads * 2 - 1) / (kThreads * 2);  // about 2 rows per thread
  if (blocks < 1) blocks = 1;
  if (blocks > 2048) blocks = 2048;
  hipLaunchKernelGGL(layout_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream, *desc, ro,
                     out->cu_q, out->cu_k, out->seg_q_src, sz.sum_q, sz.sum_k);
  return check_hip(hipGetLastError(), "layout_kernel launch");
}
