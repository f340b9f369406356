// K/V (or Q) pack-gather with RoPE on the way, and the scatter of packed outputs back to token order.
//
// Reference: the copies that pack each scope (src/onereel/models/hunyuan15.py:164,168,225; src/onereel/attention.py:69),
// diffusers apply_rotary_emb on the video q / k rows (hunyuan15.py:189-190), _move_shared (hunyuan15.py:148-150), and
// the write-back ov[lo:hi] = o / ot[t0:t1] = o after o.split (hunyuan15.py:226,231-235; attention.py:71).
//
// Both kernels are HBM-bound row copies: one wavefront moves one row of H*D bf16 (4 KiB at 16 x 128) per step in
// 16-byte lanes, all loads of a row issued before its stores (the pack loads the next row's index words ahead);
// rows under 1 KiB share a wavefront. Stores are non-temporal: the packed rows and the token-order outputs are
// written once and read by the next kernel from HBM, so they bypass the caches (about 10% and 25% faster than
// cached stores for the pack and the scatter). The rotation is done in
// fp32 as two rounded products and a rounded sum per element (no fused multiply-add), then rounded to bf16 to
// nearest even: the same bits as torch's x.float() * cos + rot(x).float() * sin followed by .to(bfloat16).
#include "common.h"

namespace onereel {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxChunksPerLane = 8;  // rows up to 64 lanes * 8 * 8 elements = 4096 elements (H*D)

// 16-byte store that bypasses the caches (global_store_dwordx4 ... nt)
__device__ __forceinline__ void store_nt(uint16_t* p, u32x4 v) { __builtin_nontemporal_store(v, (u32x4*)p); }

// One job of the row kernel: n_rows rows, row r read from src_idx[r] of [video ; text] (none where src_idx[r] < 0),
// rotated per rope_row / move_from, written to packed row dst_idx[r] (r without dst_idx) of a_out (in_place: to its
// own source row of a_out, row stride out_stride, and text rows skipped); the second source's row b_idx[r] (src_idx[r]
// without b_idx; none where b_idx[r] < 0) copied to the same packed row of b_out.
struct RowJob {
  const uint16_t* a_video;
  const uint16_t* a_text;
  const uint16_t* b_video;
  const uint16_t* b_text;
  int64_t src_stride, text_stride;
  const int32_t* src_idx;
  const int32_t* b_idx;
  const int32_t* dst_idx;
  const int32_t* rope_row;
  const int32_t* move_from;
  uint16_t* a_out;
  uint16_t* b_out;
  int64_t out_stride;
  int64_t n_rows;
  int in_place;
};

// rows [0, job[0].n_rows) run job 0, the next job[1].n_rows rows job 1 (one launch for the K/V pack and the query
// rotation of a layer)
struct GatherArgs {
  RowJob job[2];
  int64_t n_video;
  const float* cos_t;
  const float* sin_t;
  int64_t n_rope_rows;
  int H, D;
  int shared_d0;        // every chunk of a lane has the same offset within its head: (8 * lanes per row) % D == 0
};

// Rows narrower than 64 chunks (e.g. the single-head rows of the bounded memory, 16 chunks) share a wavefront: lane
// group `sub` of `per` = 64 / cp lanes (cp: the chunk count rounded up to a power of two) moves row r0 + sub.
struct RowLanes {
  int cp, per, sub, cl;
};

template <bool NARROW>
__device__ __forceinline__ RowLanes row_lanes(int chunks, int lane) {
  if constexpr (!NARROW) return RowLanes{64, 1, 0, lane};
  int cp = 1;
  while (cp < chunks) cp <<= 1;
  return RowLanes{cp, 64 / cp, lane / cp, lane % cp};
}

// One row of a job in flight: its loads issued by row_load, its rotation and stores done by row_store. CPL: 16-byte
// chunks per lane (the row's chunks over the lanes of its lane group, rounded up to a power of two).
template <int CPL>
struct RowWork {
  uint16_t* ao;
  uint16_t* bo;
  int rope, mfrom;
  bool live, rot;
  Tab8 tr, tm;
  u32x4 va[CPL], vb[CPL];
};

// The index words of row rr of the launch (source, second source, table rows, destination), loaded one row ahead of
// the row's data so that their latency overlaps the previous row's loads and stores
struct RowIdx {
  int src, bsrc, rope, mfrom;
  int64_t dst;
};

// MOVE: some job rotates with move_from (a second, inverse rotation first); without it no register holds its table
template <bool MOVE>
__device__ __forceinline__ RowIdx row_index(const GatherArgs& g, int64_t rr, int64_t total) {
  RowIdx x{-1, -1, -1, -1, 0};
  if (rr >= total) return x;
  const bool second = rr >= g.job[0].n_rows;
  const RowJob& J = second ? g.job[1] : g.job[0];
  const int64_t r = second ? rr - g.job[0].n_rows : rr;
  x.src = J.src_idx[r];
  x.bsrc = J.b_out ? (J.b_idx ? J.b_idx[r] : x.src) : -1;
  x.rope = J.rope_row ? J.rope_row[r] : -1;
  x.mfrom = MOVE && J.move_from ? J.move_from[r] : -1;
  x.dst = J.dst_idx ? J.dst_idx[r] : r;
  return x;
}

template <int CPL, bool MOVE>
__device__ __forceinline__ void row_load(const GatherArgs& g, int64_t rr, int64_t total, const RowLanes& rl,
                                         int chunks, const RowIdx& x, RowWork<CPL>& w) {
  w.live = false;
  if (rr >= total) return;
  const bool second = rr >= g.job[0].n_rows;
  const RowJob& J = second ? g.job[1] : g.job[0];
  const int src = x.src;
  const bool text = src >= g.n_video;
  if (src < 0 || (J.in_place && text)) return;
  w.live = true;
  const int64_t off = text ? (int64_t)(src - g.n_video) * J.text_stride : (int64_t)src * J.src_stride;
  const uint16_t* a = (text ? J.a_text : J.a_video) + off;
  const uint16_t* b = nullptr;
  if (J.b_out && x.bsrc >= 0) {
    const int bs = x.bsrc;
    const bool bt = bs >= g.n_video;
    b = bt ? J.b_text + (int64_t)(bs - g.n_video) * J.text_stride : J.b_video + (int64_t)bs * J.src_stride;
  }
  // table rows outside the table leave the row unrotated (the host validates them; this only keeps reads in bounds)
  int rope = x.rope;
  int mfrom = x.mfrom;
  if (rope >= g.n_rope_rows || mfrom >= g.n_rope_rows) rope = mfrom = -1;
  w.rope = rope;
  w.mfrom = mfrom;
  const int row_elems = g.H * g.D;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = rl.cl + rl.cp * i;
    if (c < chunks) {
      w.va[i] = *(const u32x4*)(a + 8 * c);
      if (b) w.vb[i] = *(const u32x4*)(b + 8 * c);
    }
  }
  // every chunk of a lane sits at the same offset within its head (8 cp a multiple of D): the lane's table entries
  // are loaded once per row, next to the row's loads, instead of once per chunk
  w.rot = MOVE && J.move_from ? (mfrom >= 0 && rope >= 0) : rope >= 0;
  if (g.shared_d0 && w.rot) {
    const int d0 = (8 * rl.cl) % g.D;
    w.tr = load_tab8(g.cos_t, g.sin_t, (int64_t)rope * g.D + d0);
    if (MOVE && J.move_from) w.tm = load_tab8(g.cos_t, g.sin_t, (int64_t)mfrom * g.D + d0);
  }
  const int64_t dst = x.dst;
  w.ao = J.in_place ? J.a_out + (int64_t)src * J.out_stride : J.a_out + dst * row_elems;
  w.bo = b ? J.b_out + dst * row_elems : nullptr;
}

template <int CPL, bool MOVE>
__device__ __forceinline__ void row_store(const GatherArgs& g, const RowLanes& rl, int chunks, RowWork<CPL>& w) {
  if (!w.live) return;
  const bool move = MOVE && w.mfrom >= 0;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = rl.cl + rl.cp * i;
    if (c < chunks) {
      u32x4 x = w.va[i];
      if (w.rot) {
        if (!g.shared_d0) {
          const int d0 = (8 * c) % g.D;
          w.tr = load_tab8(g.cos_t, g.sin_t, (int64_t)w.rope * g.D + d0);
          if (move) w.tm = load_tab8(g.cos_t, g.sin_t, (int64_t)w.mfrom * g.D + d0);
        }
        if (move) x = rotate8(x, w.tm, -1.0f);
        x = rotate8(x, w.tr, 1.0f);
      }
      store_nt(w.ao + 8 * c, x);
      if (w.bo) store_nt(w.bo + 8 * c, w.vb[i]);
    }
  }
}

// one row per wavefront (lane group) at a time; the register count per row (CPL chunks, no move table without MOVE)
// sets how many waves a SIMD holds. The wavefront index is made uniform (readfirstlane), so that a wide row's index
// words are scalar loads into SGPRs: 70 instead of 98 VGPRs, 7 waves per SIMD, and with the indices loaded one row
// ahead the layer's pack took 0.204 ms instead of 0.234 (index words loaded with the row: 0.224 ms; two or three rows
// ahead, or grids of 1792 or 3584 blocks: within 1%). Two rows per wavefront, the next row's data loaded before the
// current row's stores, measured 0.178 against 0.181 ms at 120 VGPRs and 4 waves per SIMD (with vector index loads
// at 94 VGPRs it had been 15% slower): too little for the second row's registers.
template <bool NARROW, int CPL, bool MOVE>
__global__ __launch_bounds__(kThreads) void pack_gather_kernel(GatherArgs g) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)__builtin_amdgcn_readfirstlane((int)(blockIdx.x * kWaves + (threadIdx.x >> 6)));
  const int64_t n_waves = (int64_t)gridDim.x * kWaves;
  const int chunks = (g.H * g.D) >> 3;
  const RowLanes rl = row_lanes<NARROW>(chunks, lane);
  const int64_t total = g.job[0].n_rows + g.job[1].n_rows;
  const int64_t step = n_waves * rl.per;
  RowIdx next = row_index<MOVE>(g, wave * rl.per + rl.sub, total);
  for (int64_t r0 = wave * rl.per; r0 < total; r0 += step) {
    const RowIdx cur = next;
    RowWork<CPL> w;
    row_load<CPL, MOVE>(g, r0 + rl.sub, total, rl, chunks, cur, w);
    next = row_index<MOVE>(g, r0 + step + rl.sub, total);
    row_store<CPL, MOVE>(g, rl, chunks, w);
  }
}

struct ScatterArgs {
  const uint16_t* packed;
  const int32_t* dst_idx;
  int64_t n_rows, n_video;
  uint16_t* o_video;
  uint16_t* o_text;
  int64_t dst_stride, text_stride, zero_from, text_rows;
  int H, D;
};

constexpr int kScatterRows = 1;   // rows per wavefront step: one 4 KiB row per wavefront, one step per wavefront

// rows r < n_rows: packed row r -> token-order row dst_idx[r]; rows n_rows .. n_rows + n_zero: zeroed text rows
template <bool NARROW>
__global__ __launch_bounds__(kThreads) void scatter_kernel(ScatterArgs g) {
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * kWaves + (threadIdx.x >> 6);
  const int64_t n_waves = (int64_t)gridDim.x * kWaves;
  const int row_elems = g.H * g.D;
  const int chunks = row_elems >> 3;
  const int64_t n_zero = g.text_rows > g.zero_from ? g.text_rows - g.zero_from : 0;
  const int64_t total = g.n_rows + n_zero;
  const RowLanes rl = row_lanes<NARROW>(chunks, lane);
  const int64_t step = (int64_t)kScatterRows * rl.per;
  for (int64_t r0 = wave * step; r0 < total; r0 += n_waves * step) {
    u32x4 v[kScatterRows][kMaxChunksPerLane];
    uint16_t* o[kScatterRows];
#pragma unroll
    for (int k = 0; k < kScatterRows; ++k) {
      const int64_t r = r0 + k * rl.per + rl.sub;
      o[k] = nullptr;
      if (r < g.n_rows) {
        const int dst = g.dst_idx[r];
        o[k] = dst >= g.n_video ? g.o_text + (int64_t)(dst - g.n_video) * g.text_stride
                                : g.o_video + (int64_t)dst * g.dst_stride;
        const uint16_t* p = g.packed + r * (int64_t)row_elems;
#pragma unroll
        for (int i = 0; i < kMaxChunksPerLane; ++i) {
          const int c = rl.cl + rl.cp * i;
          if (c < chunks) v[k][i] = *(const u32x4*)(p + 8 * c);
        }
      } else if (r < total) {
        o[k] = g.o_text + (g.zero_from + (r - g.n_rows)) * g.text_stride;
#pragma unroll
        for (int i = 0; i < kMaxChunksPerLane; ++i) v[k][i] = u32x4{0u, 0u, 0u, 0u};
      }
    }
#pragma unroll
    for (int k = 0; k < kScatterRows; ++k) {
      if (o[k]) {
#pragma unroll
        for (int i = 0; i < kMaxChunksPerLane; ++i) {
          const int c = rl.cl + rl.cp * i;
          if (c < chunks) store_nt(o[k] + 8 * c, v[k][i]);
        }
      }
    }
  }
}

int row_grid(int64_t rows) {
  // enough waves to keep every CU's memory pipes busy; the kernels loop over the rest
  int64_t blocks = (rows + kWaves - 1) / kWaves;
  if (blocks > 256 * 16) blocks = 256 * 16;
  return (int)(blocks < 1 ? 1 : blocks);
}

// the scatter: one wavefront per row (group of narrow rows), no loop; a cold 421 MB scatter measured 0.073 ms this
// way against 0.078 ms with two rows per step on a grid capped at 4096 blocks
int scatter_grid(int64_t rows, int rows_per_wave) {
  int64_t blocks = (rows + (int64_t)kWaves * rows_per_wave - 1) / ((int64_t)kWaves * rows_per_wave);
  if (blocks > 0x7fffffffLL) blocks = 0x7fffffffLL;
  return (int)(blocks < 1 ? 1 : blocks);
}

int check_row_shape(int H, int D, const char* who) {
  if (H < 1 || D < 8 || D % 8 != 0) return fail_arg("%s: need H >= 1 and D a multiple of 8 (H=%d D=%d)", who, H, D);
  if ((int64_t)H * D > 64 * 8 * kMaxChunksPerLane)
    return fail_arg("%s: rows of H*D=%d elements exceed the maximum %d", who, H * D, 64 * 8 * kMaxChunksPerLane);
  return 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// lanes per row as pack_gather_kernel lays them out (64 for rows of 64 chunks or more), times 8 elements per chunk,
// a multiple of D: then every chunk a lane moves starts at the same element within its head
int shared_d0(int H, int D) {
  const int chunks = H * D / 8;
  int cp = 64;
  if (chunks < 64) {
    cp = 1;
    while (cp < chunks) cp <<= 1;
  }
  return (8 * cp) % D == 0 ? 1 : 0;
}

}  // namespace
}  // namespace onereel

using namespace onereel;

namespace onereel {
namespace {

template <bool MOVE>
int launch_rows_t(const GatherArgs& g, int64_t rows, hipStream_t st) {
  const int chunks = g.H * g.D / 8;
  const dim3 grid(row_grid(rows)), block(kThreads);
  // rows under 64 chunks share a wavefront (one chunk per lane); wider rows take 2, 4 or 8 chunks per lane
  if (chunks <= 64)
    hipLaunchKernelGGL((pack_gather_kernel<true, 1, MOVE>), grid, block, 0, st, g);
  else if (chunks <= 128)
    hipLaunchKernelGGL((pack_gather_kernel<false, 2, MOVE>), grid, block, 0, st, g);
  else if (chunks <= 256)
    hipLaunchKernelGGL((pack_gather_kernel<false, 4, MOVE>), grid, block, 0, st, g);
  else
    hipLaunchKernelGGL((pack_gather_kernel<false, kMaxChunksPerLane, MOVE>), grid, block, 0, st, g);
  return check_hip(hipGetLastError(), "pack_gather_kernel launch");
}

int launch_rows(const GatherArgs& g, hipStream_t st) {
  const int64_t rows = g.job[0].n_rows + g.job[1].n_rows;
  if (rows == 0) return 0;
  return g.job[0].move_from || g.job[1].move_from ? launch_rows_t<true>(g, rows, st) : launch_rows_t<false>(g, rows, st);
}

int check_pack_job(const void* a_video, const void* a_text, const void* b_video, const void* b_text,
                   int64_t src_row_stride, int64_t text_row_stride, const int32_t* src_idx, const int32_t* rope_row,
                   const int32_t* move_from, const float* cos_table, const float* sin_table, int64_t n_rope_rows,
                   const void* a_out, const void* b_out, const char* fn) {
  if (!a_video || !src_idx || !a_out) return fail_arg("%s: the key rows, src_idx and the key output are required", fn);
  if (b_out && !b_video) return fail_arg("%s: a value output without value rows", fn);
  if ((rope_row || move_from) && (!cos_table || !sin_table || n_rope_rows < 1))
    return fail_arg("%s: rotation needs cos / sin tables", fn);
  if (move_from && !rope_row) return fail_arg("%s: move_from needs rope_row (the second rotation)", fn);
  if (!aligned16(a_video) || !aligned16(a_out) || (a_text && !aligned16(a_text)) || (b_video && !aligned16(b_video)) ||
      (b_text && !aligned16(b_text)) || (b_out && !aligned16(b_out)) || src_row_stride % 8 || text_row_stride % 8)
    return fail_arg("%s: pointers must be 16-byte aligned and row strides multiples of 8 elements", fn);
  return 0;
}

RowJob pack_job(const void* a_video, const void* a_text, const void* b_video, const void* b_text,
                int64_t src_row_stride, int64_t text_row_stride, const int32_t* src_idx, const int32_t* b_idx,
                const int32_t* dst_idx, const int32_t* rope_row, const int32_t* move_from, int64_t n_rows, void* a_out,
                void* b_out) {
  return RowJob{(const uint16_t*)a_video, (const uint16_t*)(a_text ? a_text : a_video), (const uint16_t*)b_video,
                (const uint16_t*)(b_text ? b_text : b_video), src_row_stride, text_row_stride, src_idx, b_idx, dst_idx,
                rope_row, move_from, (uint16_t*)a_out, (uint16_t*)b_out, 0, n_rows, 0};
}

}  // namespace
}  // namespace onereel

extern "C" int or_pack_gather(const void* a_video, const void* a_text, const void* b_video, const void* b_text,
                              int64_t src_row_stride, int64_t text_row_stride, int64_t n_video,
                              const int32_t* src_idx, const int32_t* rope_row, const int32_t* move_from,
                              const float* cos_table, const float* sin_table, int64_t n_rope_rows, int64_t n_rows,
                              int32_t H, int32_t D, void* a_out, void* b_out, void* stream) {
  if (int rc = check_row_shape(H, D, "or_pack_gather")) return rc;
  if (n_rows < 0) return fail_arg("or_pack_gather: n_rows < 0");
  if (n_rows == 0) return 0;
  if (int rc = check_pack_job(a_video, a_text, b_video, b_text, src_row_stride, text_row_stride, src_idx, rope_row,
                              move_from, cos_table, sin_table, n_rope_rows, a_out, b_out, "or_pack_gather"))
    return rc;
  GatherArgs g{};
  g.job[0] = pack_job(a_video, a_text, b_video, b_text, src_row_stride, text_row_stride, src_idx, nullptr, nullptr,
                      rope_row, move_from, n_rows, a_out, b_out);
  g.n_video = n_video;
  g.cos_t = cos_table;
  g.sin_t = sin_table;
  g.n_rope_rows = n_rope_rows;
  g.H = H;
  g.D = D;
  g.shared_d0 = shared_d0(H, D);
  return launch_rows(g, (hipStream_t)stream);
}

extern "C" int or_rotate_rows(const void* x, int64_t x_row_stride, int64_t n_video, const int32_t* src_idx,
                              const int32_t* rope_row, const float* cos_table, const float* sin_table,
                              int64_t n_rope_rows, int64_t n_rows, int32_t H, int32_t D, void* out,
                              int64_t out_row_stride, void* stream) {
  if (int rc = check_row_shape(H, D, "or_rotate_rows")) return rc;
  if (n_rows < 0) return fail_arg("or_rotate_rows: n_rows < 0");
  if (n_rows == 0) return 0;
  if (!x || !src_idx || !rope_row || !out || !cos_table || !sin_table || n_rope_rows < 1)
    return fail_arg("or_rotate_rows: x, src_idx, rope_row, out and the cos / sin tables are required");
  if (x_row_stride < (int64_t)H * D || out_row_stride < (int64_t)H * D)
    return fail_arg("or_rotate_rows: row strides must cover H * D elements");
  if (!aligned16(x) || !aligned16(out) || x_row_stride % 8 || out_row_stride % 8)
    return fail_arg("or_rotate_rows: pointers must be 16-byte aligned and row strides multiples of 8 elements");
  GatherArgs g{};
  g.job[0] = RowJob{(const uint16_t*)x, (const uint16_t*)x, nullptr, nullptr, x_row_stride, x_row_stride, src_idx,
                    nullptr, nullptr, rope_row, nullptr, (uint16_t*)out, nullptr, out_row_stride, n_rows, 1};
  g.n_video = n_video;
  g.cos_t = cos_table;
  g.sin_t = sin_table;
  g.n_rope_rows = n_rope_rows;
  g.H = H;
  g.D = D;
  g.shared_d0 = shared_d0(H, D);
  return launch_rows(g, (hipStream_t)stream);
}

extern "C" int or_pack_layer(const or_pack_args* p, void* stream) {
  if (!p) return fail_arg("or_pack_layer: args is NULL");
  const or_pack_args& x = *p;
  if (int rc = check_row_shape(x.H, x.D, "or_pack_layer")) return rc;
  if (x.n_keys < 0 || x.n_queries < 0) return fail_arg("or_pack_layer: negative row count");
  if (x.n_keys > 0) {
    if (int rc = check_pack_job(x.k_video, x.k_text, x.v_video, x.v_text, x.video_row_stride, x.text_row_stride,
                                x.k_src, x.k_rope, x.k_move_from, x.cos_table, x.sin_table, x.n_rope_rows, x.k_out,
                                x.v_out, "or_pack_layer"))
      return rc;
  }
  if (x.n_queries > 0) {
    if (!x.q || !x.q_src || !x.q_rope || !x.q_out || !x.cos_table || !x.sin_table || x.n_rope_rows < 1)
      return fail_arg("or_pack_layer: the query rotation needs q, q_src, q_rope, q_out and the cos / sin tables");
    if (x.q_row_stride < (int64_t)x.H * x.D || x.q_out_row_stride < (int64_t)x.H * x.D)
      return fail_arg("or_pack_layer: query row strides must cover H * D elements");
    if (!aligned16(x.q) || !aligned16(x.q_out) || x.q_row_stride % 8 || x.q_out_row_stride % 8)
      return fail_arg("or_pack_layer: pointers must be 16-byte aligned and row strides multiples of 8 elements");
  }
  GatherArgs g{};
  if (x.n_keys > 0)
    g.job[0] = pack_job(x.k_video, x.k_text, x.v_video, x.v_text, x.video_row_stride, x.text_row_stride, x.k_src,
                        x.v_src, x.k_dst, x.k_rope, x.k_move_from, x.n_keys, x.k_out, x.v_out);
  if (x.n_queries > 0)
    g.job[1] = RowJob{(const uint16_t*)x.q, (const uint16_t*)x.q, nullptr, nullptr, x.q_row_stride, x.q_row_stride,
                      x.q_src, nullptr, nullptr, x.q_rope, nullptr, (uint16_t*)x.q_out, nullptr, x.q_out_row_stride,
                      x.n_queries, 1};
  g.n_video = x.n_video;
  g.cos_t = x.cos_table;
  g.sin_t = x.sin_table;
  g.n_rope_rows = x.n_rope_rows;
  g.H = x.H;
  g.D = x.D;
  g.shared_d0 = shared_d0(x.H, x.D);
  return launch_rows(g, (hipStream_t)stream);
}

extern "C" int or_scatter(const void* packed, const int32_t* dst_idx, int64_t n_rows, int64_t n_video,
                          void* o_video, void* o_text, int64_t dst_row_stride, int64_t text_row_stride,
                          int64_t text_zero_from, int64_t text_rows, int32_t H, int32_t D, void* stream) {
  if (int rc = check_row_shape(H, D, "or_scatter")) return rc;
  if (n_rows < 0 || text_zero_from < 0) return fail_arg("or_scatter: negative row count");
  const int64_t n_zero = text_rows > text_zero_from ? text_rows - text_zero_from : 0;
  if (n_rows + n_zero == 0) return 0;
  if ((n_rows && (!packed || !dst_idx)) || (!o_video && !o_text))
    return fail_arg("or_scatter: packed, dst_idx and an output are required");
  if (n_zero && !o_text) return fail_arg("or_scatter: zeroing text rows needs o_text");
  if ((packed && !aligned16(packed)) || (o_video && !aligned16(o_video)) || (o_text && !aligned16(o_text)) ||
      dst_row_stride % 8 || text_row_stride % 8)
    return fail_arg("or_scatter: pointers must be 16-byte aligned and row strides multiples of 8 elements");
  ScatterArgs g{(const uint16_t*)packed, dst_idx, n_rows, n_video, (uint16_t*)o_video,
                (uint16_t*)(o_text ? o_text : o_video), dst_row_stride, text_row_stride, text_zero_from, text_rows,
                H, D};
  if ((int64_t)H * D < 64 * 8) {
    int cp = 1;   // lanes per narrow row (as row_lanes), so 64 / cp rows per wavefront
    while (cp < H * D / 8) cp <<= 1;
    hipLaunchKernelGGL(scatter_kernel<true>, dim3(scatter_grid(n_rows + n_zero, kScatterRows * (64 / cp))),
                       dim3(kThreads), 0, (hipStream_t)stream, g);
  } else {
    hipLaunchKernelGGL(scatter_kernel<false>, dim3(scatter_grid(n_rows + n_zero, kScatterRows)), dim3(kThreads), 0,
                       (hipStream_t)stream, g);
  }
  return check_hip(hipGetLastError(), "scatter_kernel launch");
}
