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
// The packed rows then split into runs that share every index but the spatial offset: one run per (segment, frame)
// and one per (segment, sentence). A block takes one run at a time, derives its bases once, and writes its rows as
// base + offset with coalesced int32 stores, so no per-row search or division is left.
//
// One rank's share (q_lo, q_hi): V_j's queries are scene j's tokens inside [q_lo, q_hi) with the scene's full keys,
// T_j runs only when scene j's first token lies in the range, and every other segment is empty.
//
// T_j's keys (own frames, then the sentence) are the rows of V_j's own frames and sentence. With text_keys_in_place
// V_j's keys are packed as own frames, sentence, shared frames, so T_j's keys are the first rows of V_j's: T_j packs
// none and its key range (k_off / k_len) points there. The attention result does not depend on the order of a
// segment's keys.
//
// Every segment's keys start with its scene's own frames, which are consecutive token rows: the attention call can
// read their values in place from the token-order V (v_lead / v_row, whole key blocks of them), and the pack copies
// only the other value rows (v_src = -1 for the rows read in place). A video segment's shared frames are T consecutive
// token rows each: with v_runs, up to OR_VALUE_RUNS of them per segment are listed as further runs, whose whole key
// blocks are read in place too.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include "common.h"

namespace onereel {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxSeg = 2 * OR_MAX_SCENES;

// segment s: with text, V_j = 2j and T_j = 2j + 1; without, V_j = j. A segment's packed rows are runs: one per
// frame (T rows of one source frame) and one for its text rows. cu_uq / cu_uk count the runs of the query and key
// sides.
struct SegTable {
  int n_seg;
  int cu_q[kMaxSeg + 1];
  int cu_k[kMaxSeg + 1];
  int cu_uq[kMaxSeg + 1];
  int cu_uk[kMaxSeg + 1];
};

__host__ __device__ inline int seg_scene(int with_text, int s) { return with_text ? s >> 1 : s; }
__host__ __device__ inline bool seg_is_text(int with_text, int s) { return with_text && (s & 1); }

// the rank's video queries of scene j: tokens [*a, *b), the scene's clipped to [qa, qb) (mine, hunyuan15.py:221);
// empty when the scene lies outside the range
__host__ __device__ inline void scene_queries(const LayoutDerived& L, int j, int* a, int* b) {
  const int lo = L.lo[j] * L.T, hi = L.hi[j] * L.T;
  *a = lo > L.qa ? lo : L.qa;
  *b = hi < L.qb ? hi : L.qb;
  if (*b < *a) *b = *a;
}

// the rank runs scene j's sentence queries: the scene's first token lies in its range (text_for, hunyuan15.py:223)
__host__ __device__ inline bool owns_text(const LayoutDerived& L, int j) {
  const int lo = L.lo[j] * L.T;
  return L.qa <= lo && lo < L.qb;
}

// key count of segment s (the rows its queries attend to; none for a segment the rank does not run)
__host__ __device__ inline int seg_keys(const LayoutDerived& L, int s) {
  const int j = seg_scene(L.with_text, s);
  const int own = (L.hi[j] - L.lo[j]) * L.T, txt = L.t1[j] - L.t0[j];
  if (seg_is_text(L.with_text, s)) return owns_text(L, j) ? own + txt : 0;
  int a, b;
  scene_queries(L, j, &a, &b);
  return b > a ? own + (L.sh_ptr[j + 1] - L.sh_ptr[j]) * L.T + txt : 0;
}

// keys at the head of segment s whose values the attention call reads in place from the token-order rows: every
// segment's keys start with its scene's own frames (tokens lo * T ..), whole key blocks of them
__host__ __device__ inline int seg_v_lead(const LayoutDerived& L, int s) {
  const int j = seg_scene(L.with_text, s);
  return seg_keys(L, s) > 0 ? ((L.hi[j] - L.lo[j]) * L.T) / OR_VARLEN_KEY_BLOCK * OR_VARLEN_KEY_BLOCK : 0;
}

// key offset in segment s (a video segment with keys) of its i-th shared frame: after the own frames, and after the
// sentence when the text keys are read in place (the order the run loop below writes)
__host__ __device__ inline int seg_shared_key0(const LayoutDerived& L, int s, int i) {
  const int j = seg_scene(L.with_text, s);
  const int own = (L.hi[j] - L.lo[j]) * L.T, txt = L.t1[j] - L.t0[j];
  return own + (L.text_in_place ? txt : 0) + i * L.T;
}

// query count and packed key rows of segment s (T_j packs no keys when they are read in place from V_j's)
__host__ __device__ inline void seg_lengths(const LayoutDerived& L, int s, int* lq, int* lk) {
  const int j = seg_scene(L.with_text, s);
  const bool text = seg_is_text(L.with_text, s);
  int a, b;
  scene_queries(L, j, &a, &b);
  *lq = text ? (owns_text(L, j) ? L.t1[j] - L.t0[j] : 0) : b - a;
  *lk = text && L.text_in_place ? 0 : seg_keys(L, s);
}

// runs of segment s: query side (the frames its clipped video queries touch, or its sentence) and key side (own
// frames, shared frames, sentence)
__host__ __device__ inline void seg_runs(const LayoutDerived& L, int s, int* uq, int* uk) {
  const int j = seg_scene(L.with_text, s);
  const int own = L.hi[j] - L.lo[j];
  const int txt = L.t1[j] - L.t0[j] > 0 ? 1 : 0;
  if (seg_is_text(L.with_text, s)) {
    const bool mine = owns_text(L, j);
    *uq = mine ? txt : 0;
    *uk = L.text_in_place || !mine ? 0 : own + txt;
  } else {
    int a, b;
    scene_queries(L, j, &a, &b);
    *uq = b > a ? (b - 1) / L.T - a / L.T + 1 : 0;
    *uk = b > a ? own + (L.sh_ptr[j + 1] - L.sh_ptr[j]) + txt : 0;
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
  L.text_in_place = d.with_text && d.text_keys_in_place;
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
  L.qa = d.q_hi > 0 ? d.q_lo : 0;
  L.qb = d.q_hi > 0 ? d.q_hi : f * d.T;
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
  int32_t *q_src, *q_rope, *k_src, *k_rope, *k_move_a, *k_move_b, *k_off, *k_len, *v_lead, *v_row, *v_src, *v_runs;
};

__global__ __launch_bounds__(kThreads) void layout_kernel(const or_layout_desc d, RowOut out, int32_t* cu_q_out,
                                                          int32_t* cu_k_out, int32_t* seg_q_src_out) {
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
      L.text_in_place = d.with_text && d.text_keys_in_place;
      L.n_rope = nr;
    }
    if (lane == ns - 1) {
      L.F = lo + len;
      L.qa = d.q_hi > 0 ? d.q_lo : 0;
      L.qb = d.q_hi > 0 ? d.q_hi : (lo + len) * d.T;
    }
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
    int uq0 = 0, uk0 = 0, uq1 = 0, uk1 = 0;
    if (lane < n_seg) seg_runs(L, lane, &uq0, &uk0);
    if (64 + lane < n_seg) seg_runs(L, 64 + lane, &uq1, &uk1);
    const int rq0 = wave_scan(uq0), rk0 = wave_scan(uk0);
    const int rq1 = wave_scan(uq1) + __shfl(rq0, 63, 64), rk1 = wave_scan(uk1) + __shfl(rk0, 63, 64);
    if (lane < n_seg) {
      S.cu_uq[lane] = rq0 - uq0;
      S.cu_uk[lane] = rk0 - uk0;
    }
    if (64 + lane < n_seg) {
      S.cu_uq[64 + lane] = rq1 - uq1;
      S.cu_uk[64 + lane] = rk1 - uk1;
    }
    if (lane == 63) {
      S.cu_uq[n_seg] = rq1;
      S.cu_uk[n_seg] = rk1;
    }
  }
  __syncthreads();
  if (blockIdx.x == 0) {
    for (int s = tid; s <= n_seg; s += kThreads) {
      if (cu_q_out) cu_q_out[s] = S.cu_q[s];
      if (cu_k_out) cu_k_out[s] = S.cu_k[s];
      if (s < n_seg) {
        const int j = seg_scene(L.with_text, s);
        const bool text = seg_is_text(L.with_text, s);
        int qa, qb;
        scene_queries(L, j, &qa, &qb);
        if (seg_q_src_out) seg_q_src_out[s] = text ? L.F * L.T + L.t0[j] : qa;
        if (out.k_off) out.k_off[s] = text && L.text_in_place ? S.cu_k[s - 1] : S.cu_k[s];
        if (out.k_len) out.k_len[s] = seg_keys(L, s);
        if (out.v_lead) out.v_lead[s] = seg_v_lead(L, s);
        if (out.v_row) out.v_row[s] = L.lo[j] * L.T;
        if (out.v_runs) {
          // the segment's first OR_VALUE_RUNS shared frames (a video segment with keys)
          const int nsh = !text && seg_keys(L, s) > 0 ? L.sh_ptr[j + 1] - L.sh_ptr[j] : 0;
          for (int r = 0; r < OR_VALUE_RUNS; ++r) {
            int32_t* e = out.v_runs + ((int64_t)s * OR_VALUE_RUNS + r) * 3;
            const bool on = r < nsh;
            e[0] = on ? seg_shared_key0(L, s, r) : 0;
            e[1] = on ? L.T : 0;
            e[2] = on ? L.sh[L.sh_ptr[j] + r] * L.T : 0;
          }
        }
      }
    }
  }

  // 4. per-row arrays, one run at a time
  const int T = L.T;
  const int n_video = L.F * T;
  const int n_uq = S.cu_uq[n_seg], n_runs = n_uq + S.cu_uk[n_seg];
  for (int u = blockIdx.x; u < n_runs; u += gridDim.x) {
    // run bases (block-uniform): rows [row0, row0 + count) get src0 + x, and rope0 + x / ma0 + x / mb0 + x where
    // those apply (-1 elsewhere)
    const bool qside = u < n_uq;
    const int* cu_u = qside ? S.cu_uq : S.cu_uk;
    const int uu = qside ? u : u - n_uq;
    const int s = upper_bound(cu_u, n_seg + 1, uu) - 1;
    const int slot = uu - cu_u[s];
    const int j = seg_scene(L.with_text, s);
    const bool tseg = seg_is_text(L.with_text, s);
    const int own = L.hi[j] - L.lo[j];
    const int nsh = tseg ? 0 : L.sh_ptr[j + 1] - L.sh_ptr[j];
    const int txt = L.t1[j] - L.t0[j];
    const int base = qside ? S.cu_q[s] : S.cu_k[s];
    // the run's place in the segment: queries are V_j's own-frame tokens (clipped to the rank's range; a run per frame
    // they touch) or T_j's sentence; keys are the own frames, then the shared frames and the sentence (or, with the
    // text keys in place, the sentence and the shared frames)
    int kind, idx = 0, row0;   // kind 0: own frame idx, 1: shared frame idx, 2: sentence
    int qa = 0, qb = 0;   // video query runs: frame qa / T + slot of the scene's clipped query tokens [qa, qb)
    scene_queries(L, j, &qa, &qb);
    if (qside) {
      kind = tseg ? 2 : 0;
      idx = slot;
      row0 = base;
    } else if (slot < own) {
      kind = 0;
      idx = slot;
      row0 = base + slot * T;
    } else if (L.text_in_place && !tseg) {
      const int has_txt = txt > 0 ? 1 : 0;
      kind = slot == own && has_txt ? 2 : 1;
      idx = slot - own - has_txt;
      row0 = base + own * T + (kind == 2 ? 0 : txt + idx * T);
    } else {
      kind = slot < own + nsh ? 1 : 2;
      idx = slot - own;
      row0 = base + (kind == 1 ? slot : own + nsh) * T;
    }
    // values of the run's rows x < lead0 are read in place (own-frame rows inside the segment's v_lead), and with
    // v_runs those of rows [in0, in1) (the whole key blocks of one of the segment's first OR_VALUE_RUNS shared frames)
    const int lead0 = !qside && kind == 0 ? seg_v_lead(L, s) - idx * T : 0;
    int in0 = 0, in1 = 0;
    if (!qside && kind == 1 && out.v_runs && idx < OR_VALUE_RUNS) {
      const int x0 = row0 - base;   // the frame's key offset in the segment (= seg_shared_key0(L, s, idx))
      in0 = (x0 + OR_VARLEN_KEY_BLOCK - 1) / OR_VARLEN_KEY_BLOCK * OR_VARLEN_KEY_BLOCK - x0;
      in1 = (x0 + T) / OR_VARLEN_KEY_BLOCK * OR_VARLEN_KEY_BLOCK - x0;
    }
    int count, src0, rope0 = -1, ma0 = -1, mb0 = -1;
    bool rope = false, move = false;
    if (qside && kind == 0) {
      const int f = qa / T + slot;
      const int t0 = f * T > qa ? f * T : qa, t1 = (f + 1) * T < qb ? (f + 1) * T : qb;
      row0 = base + (t0 - qa);
      count = t1 - t0;
      rope = true;
      src0 = t0;
      rope0 = (L.scene_rope ? frame_position(L, f) * T : f * T) + (t0 - f * T);
    } else if (kind != 2) {
      count = T;
      rope = true;
      int f;
      if (kind == 0) {
        f = L.lo[j] + idx;
        rope0 = L.scene_rope ? frame_position(L, f) * T : f * T;
      } else {
        const int e = L.sh_ptr[j] + idx;
        f = L.sh[e];
        if (L.adjacent) {
          const int dst = L.sh_dst[e];
          const int dd = dst - frame_position(L, f);
          const int a = dd >= 0 ? 0 : -dd;
          rope0 = dst * T;
          ma0 = a * T;
          mb0 = (a + dd) * T;
          move = true;
        } else {
          rope0 = L.scene_rope ? frame_position(L, f) * T : f * T;
        }
      }
      src0 = f * T;
    } else {
      count = txt;
      src0 = n_video + L.t0[j];
    }
    if (qside) {
      for (int x = tid; x < count; x += kThreads) {
        if (out.q_src) out.q_src[row0 + x] = src0 + x;
        if (out.q_rope) out.q_rope[row0 + x] = rope ? rope0 + x : -1;
      }
    } else {
      for (int x = tid; x < count; x += kThreads) {
        if (out.k_src) out.k_src[row0 + x] = src0 + x;
        if (out.k_rope) out.k_rope[row0 + x] = rope ? rope0 + x : -1;
        if (out.k_move_a) out.k_move_a[row0 + x] = move ? ma0 + x : -1;
        if (out.k_move_b) out.k_move_b[row0 + x] = move ? mb0 + x : -1;
        if (out.v_src) out.v_src[row0 + x] = x < lead0 || (x >= in0 && x < in1) ? -1 : src0 + x;
      }
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
  if (d.q_hi < 0 || (d.q_hi == 0 && d.q_lo != 0))
    return fail_arg("q_lo / q_hi: q_hi = 0 (the whole layer) or 0 <= q_lo < q_hi (got %d, %d)", d.q_lo, d.q_hi);
  if (d.text_keys_in_place != 0 && (d.text_keys_in_place != 1 || !d.with_text))
    return fail_arg("text_keys_in_place must be 0, or 1 with text scopes (got %d, with_text %d)", d.text_keys_in_place,
                    d.with_text);
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
  if (d.q_hi > 0 && (d.q_lo < 0 || d.q_lo >= d.q_hi || d.q_hi > F * (int64_t)d.T))
    return fail_arg("query range [%d, %d) outside the layout's %lld video tokens", d.q_lo, d.q_hi,
                    (long long)(F * (int64_t)d.T));

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
    mk = seg_keys(L, s) > mk ? seg_keys(L, s) : mk;
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
  static thread_local LayoutDerived L;
  int rc = plan_impl(desc, &sz, &L);
  if (rc) return rc;
  if (!out) return fail_arg("or_layout_build: out is NULL");
  RowOut ro{out->q_src, out->q_rope, out->k_src, out->k_rope, out->k_move_a, out->k_move_b, out->k_off, out->k_len,
            out->v_lead, out->v_row, out->v_src, out->v_runs};
  // one block per run (frame or sentence of a segment), at most 2048
  int64_t runs = 0;
  for (int s = 0; s < sz.n_seg; ++s) {
    int uq, uk;
    seg_runs(L, s, &uq, &uk);
    runs += uq + uk;
  }
  int64_t blocks = runs < 1 ? 1 : runs > 2048 ? 2048 : runs;
  hipLaunchKernelGGL(layout_kernel, dim3((unsigned)blocks), dim3(kThreads), 0, (hipStream_t)stream, *desc, ro,
                     out->cu_q, out->cu_k, out->seg_q_src);
  return check_hip(hipGetLastError(), "layout_kernel launch");
}
