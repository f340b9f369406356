// Packed varlen attention forward for gfx950: non-causal softmax(q k^T * scale) v per segment, bf16 in and out, fp32
// accumulation. Replaces flash_attn_varlen_func as src/onereel/attention.py:39-53,78-83 calls it.
//
// Design (CDNA4, 64-wide wavefronts, v_mfma_f32_32x32x16_bf16):
// - A work item is (segment, head, query tile); a persistent block of 4 wavefronts takes one item at a time from a
//   queue. A planner kernel orders the items longest segment first (LPT over the uneven scene lengths) into eight
//   queues, one per XCD, by head: the blocks of one XCD work on the same segment-head together and share its K/V in
//   that XCD's L2. A block whose queue is empty takes items from the other queues.
// - Scores are computed transposed, S^T = K Q^T (keys on the MFMA rows, queries on the columns), so a lane holds one
//   query's scores: the max, the exponentials and the row sum are in-lane apart from one exchange with lane ^ 32.
//   The K rows of the A operand are permuted (pi32) so that lane half h holds keys 16h .. 16h+15 of each 32-key block
//   in register order, which makes P^T usable as the B operand of O^T = V^T P^T and each V^T operand 8 consecutive
//   keys of one transposing LDS read pair.
// - K and V stream in blocks of 32 keys through rings of LDS slots, filled by LDS DMA (buffer_load ... lds) several
//   blocks ahead; rows past a segment's end read as zeros.
// - head_dim 128: attn8_kernel, 64 queries per wavefront (one wavefront per SIMD), O in AGPRs, key loop in generated
//   asm. head_dim 64: attn4_kernel, 32 queries per wavefront, two wavefronts per SIMD.
// - Softmax in base 2, p = 2^(c (s - m)) with c = scale * log2(e), and a running max m raised only when needed.
// - Optional RoPE on the Q load (table row per packed query), with the rounding of diffusers apply_rotary_emb.
#include <math.h>
#include <stdlib.h>

#include <algorithm>
#include <mutex>

#include "common.h"
#include "attn_ring64.inc"

// work-item queue and key-split partials of or_varlen_fwd_noalloc (see scratch_of_current_device)
static __device__ __align__(256) unsigned char scratch[OR_NOALLOC_SCRATCH_BYTES];

namespace onereel {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kThreads = 256;   // 4 wavefronts
constexpr int kMinBQ = 128;     // smallest work-item query tile of the two kernels (sizes the item list)
constexpr int kQueues = 8;      // item queues: one per XCD
constexpr int kQueueWords = 32; // words per queue header (head counter, item count, first item), one 128-byte line
constexpr int kWsHeader = kQueues * kQueueWords;   // int32 words before the item list
// an item record: tile << 8 | head, part | ways << 8 (0: whole item), split index, and the segment's first query,
// query count, first source row, first key and key count, then the token row of its first in-place key / value, the
// number of keys whose values and whose keys are read there (0 without them) and the first value event of its
// segment (an index in units of 16 bytes into the event table, -1 without value runs) (three 16-byte loads)
constexpr int kItemWords = 12;
// value events of a segment with value runs (or_varlen_args.v_runs): the key blocks at which its value stream moves
// to another base, (block, base lo, base hi, 0) for head 0 in increasing block order, then sentinels (block
// 0x7fffffff): at most 1 + 2 * OR_VALUE_RUNS events and at least two sentinels, which the key loop's prefetch of the
// event after the next may read
constexpr int kVEvents = 2 * OR_VALUE_RUNS + 3;
constexpr int kNoEvent = 0x7fffffff;
constexpr int kPlanThreads = 1024;
constexpr int kMaxPlanSeg = 4096;
constexpr int kMaxSplitWays = 8;      // key parts of a split work item
constexpr int kMaxSplitParts = 1024;  // parts of all split items of one call (sizes their partial results)
constexpr int kSplitRows = 256;       // query rows of a split item (the 64-query kernel's tile)
constexpr int kSplitMaxRounds = 4;    // items are split only when there are fewer than this many rounds of them

struct AttnArgs {
  const uint16_t* q;
  const uint16_t* q_text;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* o;
  uint16_t* o_text;
  float* lse;
  const int32_t* cu_q;
  const int32_t* cu_k;
  const int32_t* k_off;
  const int32_t* k_len;
  const int32_t* seg_q_src;
  const int32_t* q_rope;
  const float* cos_t;
  const float* sin_t;
  int64_t n_rope_rows;
  int64_t n_q_video;
  int64_t qs, ks, os;   // row strides (elements)
  int64_t qstep;        // query i of a segment is source row (first source row) + i * qstep
  int32_t sum_q, H;
  float c;              // scale * log2(e)
  float scale;
  // key-split work items (workspace regions after the item list): per split item its segment, tile << 8 | head and
  // part count; per part the lse [kSplitRows] and O / l in fp32 [kSplitRows][128] of its key range
  int32_t* split_tab;
  float* split_lse;
  float* split_o;
  // in-place values and keys: token-order rows (row stride ks) and their row counts
  const uint16_t* v_tok;
  int64_t n_vtok;
  const uint16_t* k_tok;
  int64_t n_ktok;
  // value events of the segments with value runs (kVEvents int4 per segment, written by the planner)
  const int4* v_events;
};

// the list a work item without further value events points its key loop at: sentinels only
__device__ const int4 kNoEvents[4] = {{kNoEvent, 0, 0, 0}, {kNoEvent, 0, 0, 0}, {kNoEvent, 0, 0, 0},
                                      {kNoEvent, 0, 0, 0}};

// the value runs past the leading one, for the planner: per segment OR_VALUE_RUNS (key offset, count, token row)
// entries, and the addresses the events point at
struct VRunArgs {
  const int32_t* runs;
  uint64_t v_tok, v;       // token-order values and packed values, head 0
  int64_t rsb;             // row stride in bytes
  int64_t n_vtok;
  int4* events;            // [n_seg * kVEvents]
};


// A-operand row permutation of the S^T MFMA: row i = 8g + 4h + c reads key 16h + 4g + c
__device__ __forceinline__ int pi32(int i) { return ((i >> 2) & 1) * 16 + (i >> 3) * 4 + (i & 3); }

// ------------------------------------------------------------------------------------------------------------------
// planner: up to 8 blocks, each deriving the same queues (sort and scans repeated per block) and writing its share
// of the item records, about 1024 per block (one block wrote all 3264 items of the 480p layer in 13.5 us). Segments
// sorted by key count (descending), then index. Queue q holds the heads h with h % 8 == q: for every sorted segment,
// those heads in order, each head's query tiles in order. Queue q's header at
// ws[32 q]: [0] head counter, [1] item count, [2] index of its first item in the item list. Each item record carries
// its segment's query and key ranges, so a kernel needs no further lookups to start an item.
//
// Last round: with `slots` persistent blocks, the rem = items % slots items past the last full round would leave
// blocks idle at the end. When split_keys is set, the last items of every queue (rem in all, in proportion to the
// queue sizes) are each cut into W parts by key blocks, W minimising ceil(rem W / slots) / W: the parts of an item
// run on different blocks, each writes O / l and lse of its keys, and merge_kernel combines them afterwards
// (log-sum-exp weights). ws[3] holds the number of split items, the split table their (segment, tile, head, W).
__device__ inline int plan_upper_bound(const int* a, int n, int x) {
  int lo = 0, hi = n;
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if (a[mid] <= x) lo = mid + 1;
    else hi = mid;
  }
  return lo;
}

__global__ __launch_bounds__(kPlanThreads) void plan_kernel(const int32_t* cu_q, const int32_t* cu_k,
                                                            const int32_t* k_off, const int32_t* k_len,
                                                            const int32_t* seg_q_src, const int32_t* v_lead,
                                                            const int32_t* v_row, const int32_t* k_lead,
                                                            const int32_t* k_len_head,
                                                            int n_seg, int H, int bq,
                                                            int max_items, int slots, int split_keys, int parts_cap,
                                                            VRunArgs vra, int32_t* ws) {
  __shared__ unsigned long long key[kMaxPlanSeg];
  __shared__ int off[kMaxPlanSeg + 1];
  __shared__ int part[kPlanThreads];
  __shared__ int min_nb, split_w;
  __shared__ int q_n[kQueues], q_s[kQueues], q_first[kQueues], q_sb[kQueues], q_tot[kQueues];
  const int tid = threadIdx.x;
  if (tid == 0) min_nb = 0x7fffffff;
  int n2 = 1;
  while (n2 < n_seg) n2 <<= 1;
  for (int i = tid; i < n2; i += kPlanThreads) {
    if (i < n_seg) {
      int lk = k_len ? k_len[i] : cu_k[i + 1] - cu_k[i];
      lk = lk < 0 ? 0 : lk;
      key[i] = ((unsigned long long)(0x7fffffffu - (unsigned)lk) << 32) | (unsigned)i;
    } else {
      key[i] = ~0ull;
    }
  }
  __syncthreads();
  for (int k = 2; k <= n2; k <<= 1) {
    for (int j = k >> 1; j > 0; j >>= 1) {
      for (int i = tid; i < n2; i += kPlanThreads) {
        int ixj = i ^ j;
        if (ixj > i) {
          unsigned long long x = key[i], y = key[ixj];
          bool up = (i & k) == 0;
          if ((x > y) == up) {
            key[i] = y;
            key[ixj] = x;
          }
        }
      }
      __syncthreads();
    }
  }
  // items per sorted segment, exclusive scan (each thread owns a run of consecutive entries)
  const int per = (n_seg + kPlanThreads - 1) / kPlanThreads;
  int local = 0;
  for (int e = 0; e < per; ++e) {
    int i = tid * per + e;
    if (i < n_seg) {
      int s = (int)(key[i] & 0xffffffffu);
      int lq = cu_q[s + 1] - cu_q[s];
      int tiles = lq > 0 ? (lq + bq - 1) / bq : 0;
      off[i] = tiles * H;
      local += tiles * H;
      if (tiles > 0) {
        // the fewest key blocks of any item (a key-split item keeps at least one block per part)
        int lk_min = (int)(0x7fffffffu - (unsigned)(key[i] >> 32));
        if (k_len_head)
          for (int h = 0; h < H; ++h) lk_min = min(lk_min, max(k_len_head[(int64_t)s * H + h], 0));
        atomicMin(&min_nb, (lk_min + 31) / 32);
      }
    }
  }
  part[tid] = local;
  __syncthreads();
  for (int o = 1; o < kPlanThreads; o <<= 1) {
    int x = tid >= o ? part[tid - o] : 0;
    __syncthreads();
    part[tid] += x;
    __syncthreads();
  }
  int run = part[tid] - local;
  for (int e = 0; e < per; ++e) {
    int i = tid * per + e;
    if (i < n_seg) {
      int c = off[i];
      off[i] = run;
      run += c;
    }
  }
  if (tid == kPlanThreads - 1) off[n_seg] = part[tid];
  __syncthreads();
  // the host's bound guarantees that the items fit; if they did not, every queue stays empty and no item is written
  const bool fits = off[n_seg] <= max_items;
  const int total = fits ? off[n_seg] : 0;
  // off[i] / H: query tiles of the sorted segments before i, each counted once
  const int all_tiles = total / H;
  auto heads_of = [&](int q) { return (H - q + kQueues - 1) / kQueues; };   // heads h < H with h % 8 == q
  // With H not a multiple of 8 (single-head views of the bounded memory: H = 1) dealing by head would leave queues
  // empty or uneven: there the unit u = i H + h (sorted segment i, head h) goes to queue u mod 8, so that every
  // queue holds whole segment-heads in LPT order. Its place in the queue is the sum of the tiles of the units before
  // it there: rows of 8 consecutive units, per-queue exclusive scans over the rows.
  const bool by_unit = H % kQueues != 0;
  const int n_units = by_unit && fits ? n_seg * H : 0;
  const int n_rows8 = (n_units + kQueues - 1) / kQueues;
  const int rpt = (n_rows8 + kPlanThreads - 1) / kPlanThreads;   // rows of units per thread
  const int r_lo = min(tid * rpt, n_rows8), r_hi = min(r_lo + rpt, n_rows8);
  auto unit_tiles = [&](int u) {
    const int i = u / H;
    return (off[i + 1] - off[i]) / H;
  };
  int uexcl[kQueues];
  if (by_unit) {
    int loc[kQueues];
#pragma unroll
    for (int q = 0; q < kQueues; ++q) loc[q] = 0;
    for (int r = r_lo; r < r_hi; ++r)
#pragma unroll
      for (int q = 0; q < kQueues; ++q)
        if (r * kQueues + q < n_units) loc[q] += unit_tiles(r * kQueues + q);
#pragma unroll
    for (int q = 0; q < kQueues; ++q) {
      part[tid] = loc[q];
      __syncthreads();
      for (int o = 1; o < kPlanThreads; o <<= 1) {
        const int x = tid >= o ? part[tid - o] : 0;
        __syncthreads();
        part[tid] += x;
        __syncthreads();
      }
      uexcl[q] = part[tid] - loc[q];
      if (tid == kPlanThreads - 1) q_tot[q] = part[tid];
      __syncthreads();
    }
  }
  if (tid == 0) {
    int W = 1;
    const int rem = slots > 0 ? total % slots : 0;
    // with many rounds of items the GPU is at its power limit through the last one too, and blocks left idle at the
    // end let the busy ones clock higher: splitting pays only for a few rounds (measured: none at 12.75 rounds,
    // 7% at 3 rounds, 2.5-3x below one round)
    if (split_keys && rem > 0 && total < kSplitMaxRounds * slots) {
      float best = 1.0f;   // length of the last round in items: ceil(rem W / slots) / W
      for (int w = 2; w <= kMaxSplitWays && w <= min_nb && (rem + kQueues) * w <= parts_cap; ++w) {
        const float v = (float)((rem * w + slots - 1) / slots) / (float)w;
        if (v < best - 1e-6f) {
          best = v;
          W = w;
        }
      }
    }
    int first = 0, sb = 0;
    for (int q = 0; q < kQueues; ++q) {
      const int n = by_unit ? (fits ? q_tot[q] : 0) : all_tiles * heads_of(q);
      const int sq = W > 1 ? min(n, (int)(((int64_t)rem * n + total - 1) / total)) : 0;
      q_n[q] = n;
      q_s[q] = sq;
      q_first[q] = first;
      q_sb[q] = sb;
      first += n + sq * (W - 1);
      sb += sq;
    }
    split_w = W;
  }
  __syncthreads();
  const int W = split_w;
  // every block derives the same queues; block 0 writes their headers, and each block writes its share of the items
  if (blockIdx.x == 0 && tid < kQueues) {
    ws[kQueueWords * tid] = 0;
    ws[kQueueWords * tid + 1] = q_n[tid] + q_s[tid] * (W - 1);
    ws[kQueueWords * tid + 2] = q_first[tid];
  }
  int32_t* tab = ws + kWsHeader + (int64_t)kItemWords * (max_items + parts_cap);
  if (blockIdx.x == 0 && tid == 0) ws[3] = W > 1 ? q_sb[kQueues - 1] + q_s[kQueues - 1] : 0;
  // value events of every segment (block 0): the leading run's end, then each further run's whole key blocks (its
  // start and its end), clipped as the key loop's in-place blocks are (inside the segment's whole blocks and the
  // token rows, past the leading run and the run before); a run starting where the stream would return to the
  // packed rows replaces that event
  if (blockIdx.x == 0 && vra.runs) {
    for (int s = tid; s < n_seg; s += kPlanThreads) {
      int4* L = vra.events + (int64_t)s * kVEvents;
      const int lk_seg = max(k_len ? k_len[s] : cu_k[s + 1] - cu_k[s], 0);
      const int64_t k_beg = k_off ? k_off[s] : cu_k[s];
      const int bmax = lk_seg / 32;
      const int row = v_row ? v_row[s] : -1, lead = v_lead ? v_lead[s] : 0;
      int64_t la = row >= 0 && lead > 0 ? min((int64_t)lead, (int64_t)lk_seg) / 32 : 0;
      if (row >= 0) la = min(la, (vra.n_vtok - row) / 32);
      la = la < 0 ? 0 : la;
      int n = 0;
      auto add = [&](int blk, uint64_t at) {
        if (n > 0 && L[n - 1].x == blk) --n;   // superseded at the same block
        L[n++] = make_int4(blk, (int)(uint32_t)at, (int)(uint32_t)(at >> 32), 0);
      };
      auto packed_at = [&](int blk) { return vra.v + (uint64_t)((k_beg + 32 * (int64_t)blk) * vra.rsb); };
      if (la > 0) add((int)la, packed_at((int)la));
      int prev = (int)la;
      for (int r = 0; r < OR_VALUE_RUNS; ++r) {
        const int32_t* e = vra.runs + ((int64_t)s * OR_VALUE_RUNS + r) * 3;
        const int x0 = e[0], cnt = e[1], t = e[2];
        if (cnt <= 0 || x0 < 0 || t < 0) continue;
        int bs = (x0 + 31) / 32, be = (int)min((int64_t)(x0 + (int64_t)cnt) / 32, (int64_t)bmax);
        be = (int)min((int64_t)be, (vra.n_vtok - t + x0) / 32);   // token rows t + 32 B - x0 + i < n_vtok
        bs = max(bs, prev);
        if (be <= bs) continue;
        add(bs, vra.v_tok + (uint64_t)(((int64_t)t + 32 * (int64_t)bs - x0) * vra.rsb));
        add(be, packed_at(be));
        prev = be;
      }
      for (; n < kVEvents; ++n) L[n] = make_int4(kNoEvent, 0, 0, 0);
    }
  }
  // the record(s) of tile t of head `head` of sorted segment i, at position pos of queue q (the last q_s[q] positions
  // of a queue are items split into W key parts)
  auto emit = [&](int i, int head, int t, int q, int pos) {
    const int s = (int)(key[i] & 0xffffffffu);
    const int lq = cu_q[s + 1] - cu_q[s];
    const int keep = q_n[q] - q_s[q];
    const int q_beg = cu_q[s];
    const int k_beg = k_off ? k_off[s] : cu_k[s];
    const int lk_seg = k_len ? k_len[s] : cu_k[s + 1] - cu_k[s];
    const int lk = k_len_head ? min(k_len_head[(int64_t)s * H + head], lk_seg) : lk_seg;   // this head's keys
    const int q_src0 = seg_q_src ? seg_q_src[s] : q_beg;
    const int vl = v_lead ? v_lead[s] : 0, vr = v_row ? v_row[s] : 0, kl = k_lead ? k_lead[s] : 0;
    auto put = [&](int64_t entry, int pw, int sidx) {
      int32_t* e = ws + kWsHeader + kItemWords * entry;
      *(int4*)e = make_int4((t << 8) | head, pw, sidx, q_beg);
      *(int4*)(e + 4) = make_int4(lq, q_src0, k_beg, lk < 0 ? 0 : lk);
      *(int4*)(e + 8) = make_int4(vr, vl, kl, vra.runs ? s * kVEvents : -1);
    };
    if (pos < keep) {
      put(q_first[q] + pos, 0, 0);
    } else {
      const int k = pos - keep, sidx = q_sb[q] + k;
      for (int p = 0; p < W; ++p) put(q_first[q] + keep + k * W + p, p | (W << 8), sidx);
      tab[3 * sidx] = s;
      tab[3 * sidx + 1] = (t << 8) | head;
      tab[3 * sidx + 2] = W;
    }
  };
  if (by_unit) {
    for (int r = r_lo; r < r_hi; ++r)
#pragma unroll
      for (int q = 0; q < kQueues; ++q) {
        const int u = r * kQueues + q;
        if (u >= n_units) break;
        const int tiles = unit_tiles(u);
        if ((int)(u % gridDim.x) == (int)blockIdx.x)
          for (int t = 0; t < tiles; ++t) emit(u / H, u % H, t, q, uexcl[q] + t);
        uexcl[q] += tiles;
      }
    return;
  }
  for (int it = tid + blockIdx.x * kPlanThreads; it < total; it += kPlanThreads * gridDim.x) {
    const int i = plan_upper_bound(off, n_seg + 1, it) - 1;
    const int tiles = (off[i + 1] - off[i]) / H;
    const int local_it = it - off[i];
    const int head = local_it / tiles, t = local_it - head * tiles;
    const int q = head % kQueues;
    emit(i, head, t, q, (off[i] / H) * heads_of(q) + (head / kQueues) * tiles + t);   // position within queue q
  }
}

// Item count and first item of every queue, as the planner wrote them (constant while the kernel runs), copied to
// LDS once per block so that a claim takes one memory round trip: the atomic on the queue's counter.
struct QueueInfo {
  int n[kQueues], first[kQueues];
};

// the record of item `it`, read through the constant address space: the planner writes the records before the
// attention kernel starts and nothing writes them while it runs, and `it` is wave-uniform, so they load with scalar
// loads (counted by lgkmcnt: a record does not wait behind earlier O stores in the in-order vmcnt)
typedef __attribute__((address_space(4))) const int ItemWord;
struct ItemRec {
  int4 r0, r1, r2;
};
__device__ inline ItemRec item_record(const int32_t* ws, int it) {
  const ItemWord* x = (const ItemWord*)(ws + kWsHeader + kItemWords * it);
  return ItemRec{make_int4(x[0], x[1], x[2], x[3]), make_int4(x[4], x[5], x[6], x[7]),
                 make_int4(x[8], x[9], x[10], x[11])};
}


__device__ inline void load_queues(const int32_t* ws, QueueInfo* qi, int tid) {
  if (tid < kQueues) {
    qi->n[tid] = ws[kQueueWords * tid + 1];
    qi->first[tid] = ws[kQueueWords * tid + 2];
  }
}

// next work item of a block (thread 0 calls it): from the queue of the block's XCD (read from HW_REG_XCC_ID) with one
// atomic, then from the others in turn; -1 when every queue is empty. Another XCD's counter is read before its atomic
// so that exhausted queues are not incremented further; the block's own queue is taken directly (a counter past the
// count only reads as empty).
__device__ inline int next_item(int32_t* ws, int xcc, const QueueInfo* qi) {
  for (int r = 0; r < kQueues; ++r) {
    const int q = (xcc + r) & (kQueues - 1);
    const int n = qi->n[q];
    if (n <= 0) continue;
    int32_t* hq = ws + kQueueWords * q;
    if (r > 0 && __hip_atomic_load(hq, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= n) continue;
    const int x = atomicAdd(hq, 1);
    if (x < n) return qi->first[q] + x;
  }
  return -1;
}

__device__ __forceinline__ int xcc_id() { return __builtin_amdgcn_s_getreg(0xf814) & (kQueues - 1); }  // HW_REG_XCC_ID

// ------------------------------------------------------------------------------------------------------------------
// attention

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// max over the 32 keys of a query: in-lane over 16, then with lane ^ 32 (v_permlane32_swap)
__device__ __forceinline__ float pair_max(float x) {
  const int xi = __builtin_bit_cast(int, x);
  auto sw = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
  return fmaxf(__builtin_bit_cast(float, (int)sw[0]), __builtin_bit_cast(float, (int)sw[1]));
}

__device__ __forceinline__ float pair_sum(float x) {
  const int xi = __builtin_bit_cast(int, x);
  auto sw = __builtin_amdgcn_permlane32_swap(xi, xi, false, false);
  return __builtin_bit_cast(float, (int)sw[0]) + __builtin_bit_cast(float, (int)sw[1]);
}

// ------------------------------------------------------------------------------------------------------------------
// Ring kernel with 32 queries per wavefront (attn4_kernel, run for head_dim 64): software-pipelined over blocks of
// 32 keys. K and V blocks stream through two rings of four LDS slots each, filled by buffer loads straight into LDS (LDS DMA) three iterations ahead; rows past a
// segment's end read as zeros. Iteration j of a wavefront runs the softmax of block j on the VALU while the MFMA unit
// computes S of block j + 1 (QK^T) and O += V P^T of block j - 1, so the exponentials overlap the matrix work inside
// one wavefront as well as across the two wavefronts that share a SIMD.
//
// Running max: P(j) is computed with the running max m as it stands; only when some probability of the block
// exceeds 2^16 (its row-half sum exceeds 2^20, or overflows) does the wavefront take the max of the block, rescale O
// and l by 2^((m_old - m_new) c) and recompute P(j). The first block of every item takes that path (m starts at
// -1e30, a finite stand-in for -inf so that masked scores still give exactly 0).

constexpr int kBKB = 32;   // keys per ring slot
constexpr int kRing = 4;   // slots per ring (K ring and V ring)
constexpr float kRescaleSum = 1048576.0f;   // 2^20
constexpr float kMInit = -1e30f;

template <int D>
struct R4 {
  static constexpr int CH = D / 8;                     // 16-byte chunks per row
  static constexpr int KS = D / 16;                    // MFMA k-steps of S^T
  static constexpr int DB = D / 32;                    // 32-row blocks of O^T
  static constexpr int LPB = kBKB * CH / kThreads;     // loads per lane for one K (or V) block
  static constexpr int SLOT = kBKB * D;                // bf16 elements per slot
  static constexpr int GROUP = 2 * LPB;                // loads per lane issued by one iteration (a K and a V block)
};

// s_waitcnt immediate that waits until at most n vector-memory operations of this wavefront are outstanding
constexpr int vmcnt_imm(int n) { return (n & 0xF) | (0x7 << 4) | (0xF << 8) | ((n >> 4) << 14); }

// K slot swizzle (XOR on the 16-byte chunk index of block-local row r): the 16 lanes that one b128 read services
// together read 16 distinct chunk positions. V slot swizzle: the 32 lanes of one transposing b64 read cover the 64
// banks once.
template <int CH>
__device__ __forceinline__ int swz4_k(int r) {
  if constexpr (CH == 16) return (r & 3) | (((r >> 4) & 1) << 2) | (((r >> 2) & 1) << 3);
  else return ((r >> 1) & 3) | (((r >> 4) & 1) << 2);
}
template <int CH>
__device__ __forceinline__ int swz4_v(int r) {
  if constexpr (CH == 16) return 4 * (r & 3);
  else return 4 * ((r >> 1) & 1);
}

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

__device__ __forceinline__ uint32_t lds_addr(const void* p) { return (uint32_t)(uintptr_t)(const lds_void*)p; }

// the slots are distinct __shared__ arrays, addressed by compile-time index
struct Ring {
  uint16_t* k[kRing];
  uint16_t* v[kRing];
};

// One K or V block into an LDS slot: lane i of load n fetches 16 bytes at voff[n] from the block's first row into
// LDS byte m0 + n * 4096 + 16 * lane (m0: the slot plus this wavefront's 1 KiB). The buffer descriptor's record
// count ends at the segment's last row, so rows past it read 0. Inline asm: the compiler does not see these LDS
// writes, so it adds no waits on them before unrelated LDS reads; the kernel waits with vmcnt and a barrier itself.
// gfx9 needs one wait state between an SALU write of M0 and the LDS DMA that reads it (the s_nop).
template <int LPB>
__device__ __forceinline__ void dma_block(uint64_t base, int32_t nrec, const uint32_t* voff, uint32_t m0) {
  const i32x4 r = {(int32_t)(uint32_t)base, (int32_t)(uint32_t)(base >> 32), nrec, 0x00020000};
#pragma unroll
  for (int n = 0; n < LPB; ++n)
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff[n]), "s"(r),
                 "s"(m0 + n * kThreads * 16)
                 : "memory");
}

// wait until at most N of this wavefront's loads are in flight, then synchronise the block
template <int N>
__device__ __forceinline__ void wait_loads_barrier() {
  if constexpr (N == 0) asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
  else if constexpr (N == 4) asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory");
  else if constexpr (N == 6) asm volatile("s_waitcnt vmcnt(6)\n\ts_barrier" ::: "memory");
  else if constexpr (N == 8) asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");
  else asm volatile("s_waitcnt vmcnt(12)\n\ts_barrier" ::: "memory");
}

// Per-item stream of one segment-head's K or V rows: block b starts at base + b * bb bytes (abase + b * bb for the
// in-place value blocks b < nba) and holds rem0 - b * bb valid bytes (clamped at 0).
struct Stream {
  uint64_t base;
  int32_t rem0;
  int32_t bb;
  uint64_t abase;
  int32_t nba;
  __device__ __forceinline__ uint64_t at(int b) const {
    return (b < nba ? abase : base) + (uint64_t)(int64_t)b * (uint32_t)bb;
  }
  __device__ __forceinline__ int32_t nrec(int b) const { return max(rem0 - b * bb, 0); }
};

// K or V stream of a work item (or of one key part of it): key blocks b < nba read the token-order rows from base a,
// the others the packed rows from base p; either way block b starts b * bb bytes past its base.
struct VRange {
  uint64_t a, p;
  int32_t nba;
};

// the in-place blocks of key blocks [b0, b0 + nb) of a segment whose first `lead` keys are token rows row.. of tok
// (whole blocks only, none past the n_tok token rows or the item's last whole block); p: packed rows of block b0
__device__ inline VRange tok_range(const uint16_t* tok, int64_t n_tok, int64_t rs, int row, int lead, int lk_seg,
                                   int b0, int nb, int64_t head_off, uint64_t p) {
  VRange r{p, p, 0};
  if (!tok || lead <= 0 || row < 0) return r;
  int64_t nba = min((int64_t)lead, (int64_t)lk_seg) / kBKB;
  const int64_t fit = (n_tok - row) / kBKB;   // blocks that lie inside the token rows
  nba = min(nba, fit) - b0;
  nba = nba < 0 ? 0 : (nba > nb ? nb : nba);
  r.nba = (int32_t)nba;
  if (nba > 0) r.a = (uint64_t)(tok + ((int64_t)row + (int64_t)kBKB * b0) * rs + head_off);
  return r;
}

template <int D>
__device__ __forceinline__ bf16x8 ring_vt(const uint16_t* slot, uint32_t vaddr, int half) {
  u32x2 lo, hi;
#pragma unroll
  for (int t = 0; t < 2; ++t) {
    const char* p = (const char*)slot + vaddr + (8 * half + 4 * t) * D * 2;
    bf16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4*)p);
    (t == 0 ? lo : hi) = __builtin_bit_cast(u32x2, x);
  }
  u32x4 v = {lo[0], lo[1], hi[0], hi[1]};
  return as_bf16x8(v);
}

template <int D>
struct St4 {
  bf16x8 q[R4<D>::KS];
  f32x16 acc[R4<D>::DB];
  f32x16 s[2];
  bf16x8 p[2][2];     // [parity][half]
  float m, mc, lsum;
  uint32_t kaddr[R4<D>::KS];
  uint32_t vaddr[R4<D>::DB];
};

__device__ __forceinline__ float max16(const f32x16& s) {
  float x = fmaxf(fmaxf(s[0], s[1]), s[2]);
#pragma unroll
  for (int r = 3; r < 15; r += 2) x = fmaxf(fmaxf(x, s[r]), s[r + 1]);
  return fmaxf(x, s[15]);
}

// P = 2^(s c - mc) rounded to bf16 pairs, and the fp32 sum of the unrounded values (as FlashAttention sums its fp32
// P before the PV product). The sum uses v_add_f32, which issues under a running MFMA: v_dot2_f32_bf16 does not
// (measured on gfx950: each dot2 between 32x32x16 MFMAs holds the matrix pipe for ~18 cycles).
__device__ __forceinline__ float exp_pack(const f32x16& s, float c, float mc, bf16x8 (&p)[2]) {
  f32x16 e;
#pragma unroll
  for (int r = 0; r < 16; ++r) e[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[r], c, -mc));
  float t[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) t[i] = (e[4 * i] + e[4 * i + 1]) + (e[4 * i + 2] + e[4 * i + 3]);
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    u32x4 pk;
#pragma unroll
    for (int i = 0; i < 4; ++i) pk[i] = pack2(e[8 * half + 2 * i], e[8 * half + 2 * i + 1]);
    p[half] = as_bf16x8(pk);
  }
  return (t[0] + t[1]) + (t[2] + t[3]);
}

// iteration j (J = j mod 4, compile-time: the slots it touches are compile-time)
template <int D, int J>
__device__ __forceinline__ void iter4(St4<D>& st, const Ring& rg, int j, int nb, int Lk, bool active,
                                      const Stream& ks, const Stream& vs, const uint32_t* voffk,
                                      const uint32_t* voffv, uint32_t m0w, int h, float c) {
  using C = R4<D>;
  constexpr int PAR = J & 1;
  // blocks K(j+1) and V(j-1) have landed (the loads of the last two iterations may still be in flight), and every
  // wavefront is done with iteration j-1's slots
  wait_loads_barrier<2 * C::GROUP>();
  dma_block<C::LPB>(ks.at(j + kRing), ks.nrec(j + kRing), voffk, lds_addr(rg.k[J]) + m0w);
  dma_block<C::LPB>(vs.at(j + 2), vs.nrec(j + 2), voffv, lds_addr(rg.v[(J + 2) % kRing]) + m0w);
  if (!active) return;

  bf16x8 kop[C::KS];
#pragma unroll
  for (int k = 0; k < C::KS; ++k) kop[k] = *(const bf16x8*)((const char*)rg.k[(J + 1) % kRing] + st.kaddr[k]);
  bf16x8 vop[2][C::DB];
#pragma unroll
  for (int half = 0; half < 2; ++half)
#pragma unroll
    for (int db = 0; db < C::DB; ++db) vop[half][db] = ring_vt<D>(rg.v[(J + 3) % kRing], st.vaddr[db], half);

  f32x16& s = st.s[PAR];
  if (j == nb - 1 && (Lk & (kBKB - 1))) {
    int valid = Lk - j * kBKB - 16 * h;
    asm volatile("" : "+v"(valid));   // computed here, not hoisted out of the loop as 16 lane masks in SGPRs
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = r < valid ? s[r] : -__builtin_inff();
  }

  // matrix work: S(j+1) = K(j+1) Q^T, O += V(j-1) P(j-1)
  f32x16& sn = st.s[PAR ^ 1];
  const f32x16 zero = {};
#pragma unroll
  for (int k = 0; k < C::KS; ++k) {
    sn = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kop[k], st.q[k], k == 0 ? zero : sn, 0, 0, 0);
    const int half = k / C::DB, db = k % C::DB;
    st.acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vop[half][db], st.p[PAR ^ 1][half], st.acc[db], 0, 0, 0);
  }
  // vector work: P(j) with the running max
  float ls = exp_pack(s, c, st.mc, st.p[PAR]);
#pragma unroll
  for (int i = 0; i < 2 * C::KS; ++i) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);
  }
  // keeps P(j) in this scheduling region (next to the MFMAs) instead of being sunk past the branch
  asm volatile("" ::"v"(st.p[PAR][0]), "v"(st.p[PAR][1]), "v"(ls));
  if (__any(!(ls <= kRescaleSum))) {
    const float mx = pair_max(max16(s));
    const float mn = fmaxf(st.m, mx);
    const float alpha = __builtin_amdgcn_exp2f((st.m - mn) * c);
    st.m = mn;
    st.mc = mn * c;
    ls = exp_pack(s, c, st.mc, st.p[PAR]);
#pragma unroll
    for (int db = 0; db < C::DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[db][r] *= alpha;
    st.lsum *= alpha;
  }
  st.lsum += ls;
}

template <int D>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2)))
void attn4_kernel(AttnArgs a, int32_t* ws) {
  using C = R4<D>;
  constexpr int WQ = 32, BQ = 4 * WQ;
  __shared__ __attribute__((aligned(16))) uint16_t k0[C::SLOT], k1[C::SLOT], k2[C::SLOT], k3[C::SLOT];
  __shared__ __attribute__((aligned(16))) uint16_t v0[C::SLOT], v1[C::SLOT], v2[C::SLOT], v3[C::SLOT];
  __shared__ int item_sh;
  __shared__ QueueInfo qinfo;
  const Ring rg = {{k0, k1, k2, k3}, {v0, v1, v2, v3}};
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t rs = a.ks;
  const uint32_t m0w = (uint32_t)w * 64 * 16;   // this wavefront's 1 KiB of each load's destination

  // per-lane constants: byte offsets of this lane's loads within a block, and of its LDS operand reads
  uint32_t voffk[C::LPB], voffv[C::LPB];
#pragma unroll
  for (int n = 0; n < C::LPB; ++n) {
    const int slot = n * kThreads + w * 64 + lane;
    const int row = slot / C::CH, phys = slot % C::CH;
    voffk[n] = (uint32_t)(row * rs * 2 + (phys ^ swz4_k<C::CH>(row)) * 16);
    voffv[n] = (uint32_t)(row * rs * 2 + (phys ^ swz4_v<C::CH>(row)) * 16);
  }
  St4<D> st;
  {
    const int row = pi32(l32);
#pragma unroll
    for (int k = 0; k < C::KS; ++k) st.kaddr[k] = (uint32_t)(row * D * 2 + (((2 * k + h) ^ swz4_k<C::CH>(row)) * 16));
    const int r = lane & 15, g = lane >> 4;
    const int cp = 2 * (g & 1) + ((r >> 1) & 1);
    const int mv = C::CH == 16 ? ((r >> 2) & 3) : ((r >> 3) & 1);
#pragma unroll
    for (int db = 0; db < C::DB; ++db)
      st.vaddr[db] = (uint32_t)((16 * h + (r >> 2)) * D * 2 + (4 * (db ^ mv) + cp) * 16 + (r & 1) * 8);
  }

  const int xcc = xcc_id();
  load_queues(ws, &qinfo, tid);
  __syncthreads();
  for (;;) {
    if (tid == 0) item_sh = next_item(ws, xcc, &qinfo);
    __syncthreads();
    const int it = __builtin_amdgcn_readfirstlane(item_sh);
    __syncthreads();
    if (it < 0) break;
    const int4 r0 = *(const int4*)(ws + kWsHeader + kItemWords * it);
    const int4 r1 = *(const int4*)(ws + kWsHeader + kItemWords * it + 4);
    const int4 r2 = *(const int4*)(ws + kWsHeader + kItemWords * it + 8);
    const int head = r0.x & 255, qt = r0.x >> 8;
    const int q_beg = r0.w, Lq = r1.x, q_src0 = r1.y, k_beg = r1.z, Lk = r1.w;
    const int q0 = qt * BQ + w * WQ;
    const bool active = q0 < Lq;
    const int nb = (Lk + kBKB - 1) / kBKB;
    const int32_t rb = (int32_t)rs * 2;
    const VRange vr = tok_range(a.v_tok, a.n_vtok, rs, r2.x, r2.y, Lk, 0, nb, head * D,
                                (uint64_t)(a.v + (int64_t)k_beg * rs + head * D));
    const VRange kr = tok_range(a.k_tok, a.n_ktok, rs, r2.x, r2.z, Lk, 0, nb, head * D,
                                (uint64_t)(a.k + (int64_t)k_beg * rs + head * D));
    const Stream ks = {kr.p, Lk * rb - rb + D * 2, kBKB * rb, kr.a, kr.nba};
    const Stream vs = {vr.p, Lk * rb - rb + D * 2, kBKB * rb, vr.a, vr.nba};

    // prologue: K(0) and the group {K(1), V(-1)} (V(-1) fills its slot with zeros: iteration 0 multiplies it by
    // P(-1) = 0) are in flight while Q loads; every load so far is waited for (so the compiler's own waits for Q do
    // not fall inside the loop), then the groups {K(2), V(0)} and {K(3), V(1)} go out
    dma_block<C::LPB>(ks.at(0), ks.nrec(0), voffk, lds_addr(rg.k[0]) + m0w);
    dma_block<C::LPB>(ks.at(1), ks.nrec(1), voffk, lds_addr(rg.k[1]) + m0w);
    dma_block<C::LPB>(vs.at(0), 0, voffv, lds_addr(rg.v[3]) + m0w);
    if (active) {
      const int i = q0 + l32 < Lq ? q0 + l32 : Lq - 1;
      const int64_t row = q_src0 + (int64_t)i * a.qstep;
      const uint16_t* qp = (row < a.n_q_video ? a.q + row * a.qs : a.q_text + (row - a.n_q_video) * a.qs) + head * D;
      int rr = a.q_rope ? a.q_rope[q_beg + i] : -1;
      if (rr >= a.n_rope_rows) rr = -1;
#pragma unroll
      for (int k = 0; k < C::KS; ++k) {
        const int d = 16 * k + 8 * h;
        u32x4 x = *(const u32x4*)(qp + d);
        if (rr >= 0) x = rotate8(x, a.cos_t, a.sin_t, (int64_t)rr * D + d, 1.0f);
        st.q[k] = as_bf16x8(x);
      }
    }
    __builtin_amdgcn_s_waitcnt(vmcnt_imm(0));
    dma_block<C::LPB>(ks.at(2), ks.nrec(2), voffk, lds_addr(rg.k[2]) + m0w);
    dma_block<C::LPB>(vs.at(0), vs.nrec(0), voffv, lds_addr(rg.v[0]) + m0w);
    dma_block<C::LPB>(ks.at(3), ks.nrec(3), voffk, lds_addr(rg.k[3]) + m0w);
    dma_block<C::LPB>(vs.at(1), vs.nrec(1), voffv, lds_addr(rg.v[1]) + m0w);

#pragma unroll
    for (int db = 0; db < C::DB; ++db)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[db][r] = 0.0f;
    {
      const u32x4 z = {0u, 0u, 0u, 0u};
      st.p[1][0] = as_bf16x8(z);
      st.p[1][1] = as_bf16x8(z);
    }
    st.m = kMInit;
    st.mc = kMInit * a.c;
    st.lsum = 0.0f;
    const float c = a.c;

    asm volatile("s_barrier" ::: "memory");
    if (active) {
      const f32x16 zero = {};
#pragma unroll
      for (int k = 0; k < C::KS; ++k)
        st.s[0] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*(const bf16x8*)((const char*)rg.k[0] + st.kaddr[k]),
                                                         st.q[k], k == 0 ? zero : st.s[0], 0, 0, 0);
    }
    for (int j = 0; j < nb; j += kRing) {
      iter4<D, 0>(st, rg, j, nb, Lk, active, ks, vs, voffk, voffv, m0w, h, c);
      if (j + 1 < nb) iter4<D, 1>(st, rg, j + 1, nb, Lk, active, ks, vs, voffk, voffv, m0w, h, c);
      if (j + 2 < nb) iter4<D, 2>(st, rg, j + 2, nb, Lk, active, ks, vs, voffk, voffv, m0w, h, c);
      if (j + 3 < nb) iter4<D, 3>(st, rg, j + 3, nb, Lk, active, ks, vs, voffk, voffv, m0w, h, c);
    }
    // epilogue: O += V(nb-1) P(nb-1), then normalise and store
    wait_loads_barrier<0>();
    if (active) {
      const int last = nb - 1;
      const int vsl = (last + kRing) % kRing;
      const uint16_t* vslot = vsl == 0 ? rg.v[0] : vsl == 1 ? rg.v[1] : vsl == 2 ? rg.v[2] : rg.v[3];
      const bool odd = (last & 1) != 0;
#pragma unroll
      for (int half = 0; half < 2; ++half) {
        const bf16x8 pp = odd ? st.p[1][half] : st.p[0][half];
#pragma unroll
        for (int db = 0; db < C::DB; ++db)
          st.acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ring_vt<D>(vslot, st.vaddr[db], half), pp,
                                                              st.acc[db], 0, 0, 0);
      }
      const float ltot = pair_sum(st.lsum);
      const int i = q0 + l32;
      if (i < Lq) {
        const float inv = nb > 0 ? 1.0f / ltot : 0.0f;
        const int64_t row = q_src0 + (int64_t)i * a.qstep;
        uint16_t* op = (row < a.n_q_video ? a.o + row * a.os : a.o_text + (row - a.n_q_video) * a.os) + head * D;
#pragma unroll
        for (int db = 0; db < C::DB; ++db)
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int d = db * 32 + 8 * g + 4 * h;
            uint32_t lo = pack2(st.acc[db][4 * g] * inv, st.acc[db][4 * g + 1] * inv);
            uint32_t hi = pack2(st.acc[db][4 * g + 2] * inv, st.acc[db][4 * g + 3] * inv);
            *(uint2*)(op + d) = make_uint2(lo, hi);
          }
        if (a.lse && h == 0)
          a.lse[(int64_t)head * a.sum_q + q_beg + i] = nb > 0 ? st.m * a.scale + logf(ltot) : -__builtin_inff();
      }
    }
  }
}

// ------------------------------------------------------------------------------------------------------------------
// Ring kernel with 64 queries per wavefront (D = 128): every K and V operand read from LDS feeds two MFMAs (two
// 32-query column blocks), so LDS reads per FLOP halve, and a block of four wavefronts covers 256 queries, so the K/V
// stream per FLOP halves too. One wavefront per SIMD, one block per CU. The O accumulators (128 registers per lane)
// live in AGPRs for the whole key loop, which is generated inline asm (gen_attn_ring64.py -> attn_ring64.inc): K and
// V blocks of 32 keys stream through rings of ONEREEL_RING64 LDS slots each, the barrier sits in the middle of an
// iteration so that the next iteration's operands are read during this one's MFMAs, and the epilogue normalises O and
// stores it (rows past the segment masked off). Q sits in a128..a191: at its loop's exit, where Q is no longer read,
// an item loads the next item's queries there ahead of its O stores (the block claims one item ahead while its XCD's
// queue holds plenty), so that the next item does not wait for the stores to drain before its Q lands. The item
// queue, the first two K blocks of an item, the first item's Q load (and any Q rotated on the load) and the lse store
// are C++.

constexpr int kRing64 = ONEREEL_RING64;
constexpr int kSlot64 = kBKB * 128;   // bf16 elements per slot

__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(1, 1)))
void attn8_kernel(AttnArgs a, int32_t* ws) {
  constexpr int D = 128, CH = 16, KS = 8, WQ = 64, BQ = 4 * WQ;
  __shared__ __attribute__((aligned(1024))) uint16_t ring[2 * kRing64 * kSlot64];
  __shared__ int item_sh;
  __shared__ QueueInfo qinfo;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, h = lane >> 5;
  const int64_t rs = a.ks;
  const uint32_t lds0 = lds_addr(ring);
  const uint32_t sbase = lds0 + (uint32_t)w * 64 * 16;

  // LDS read addresses: K step k reads row pi(l32), 16-byte chunk (2k + h) ^ swz(row), i.e. kb ^ 32k; V^T step
  // (half, db) reads from vb ^ 64 db (the generated code forms both from these bases)
  const int krow = pi32(l32), ksw = swz4_k<CH>(krow);
  const uint32_t kb = lds0 + krow * D * 2 + (uint32_t)((h ^ (ksw & 1)) * 16 + 32 * (ksw >> 1));
  const int r = lane & 15, g = lane >> 4;
  const int cp = 2 * (g & 1) + ((r >> 1) & 1), mv = (r >> 2) & 3;
  const uint32_t vb = lds0 + (uint32_t)(kRing64 * kSlot64 * 2) + (16 * h + (r >> 2)) * D * 2 + cp * 16 + (r & 1) * 8 +
                      64 * mv;
  // DMA lane offsets within a block (row * stride + swizzled chunk), as attn4_kernel
  uint32_t voff[4];
#pragma unroll
  for (int n = 0; n < 2; ++n) {
    const int slot = n * kThreads + w * 64 + lane;
    const int row = slot / CH, phys = slot % CH;
    voff[n] = (uint32_t)(row * rs * 2 + (phys ^ swz4_k<CH>(row)) * 16);
    voff[2 + n] = (uint32_t)(row * rs * 2 + (phys ^ swz4_v<CH>(row)) * 16);
  }

  // While its XCD's queue holds more than kAheadMin items, the block claims its next item before running the current
  // one, so that the current item's key loop can load the next item's queries at its exit (into a128..a191, ahead of
  // its O stores); have_q says they are there. Near the end of the queue it claims after each item, as a block that
  // holds two items cannot take work that another block left: the last rounds stay balanced.
  constexpr int kAheadMin = 64, kLater = -2;
  const int xcc = xcc_id(), own = xcc & (kQueues - 1);
  load_queues(ws, &qinfo, tid);
  __syncthreads();
  auto claim = [&](bool ahead) {
    if (tid == 0) {
      // (the counter is read for every claim: skipping the read for the claims after an item measured 0.2% slower)
      const int taken = __hip_atomic_load(ws + kQueueWords * own, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      item_sh = !ahead || qinfo.n[own] - taken > kAheadMin ? next_item(ws, xcc, &qinfo) : kLater;
    }
    __syncthreads();
    const int x = __builtin_amdgcn_readfirstlane(item_sh);
    __syncthreads();
    return x;
  };
  int it = claim(false);
  bool have_q = false;
  while (it >= 0) {
    const ItemRec rec = item_record(ws, it);
    const int4 r0 = rec.r0, r1 = rec.r1, r2 = rec.r2;
    const int head = r0.x & 255, qt = r0.x >> 8, part = r0.y & 255, ways = r0.y >> 8, sidx = r0.z;
    const int q_beg = r0.w, Lq = r1.x, q_src0 = r1.y;
    const int lk_seg = r1.w;
    int k_beg = r1.z, Lk = r1.w, b0 = 0;
    if (ways > 1) {
      // part `part` of `ways`: key blocks [nb_all part / ways, nb_all (part + 1) / ways), at least one each
      const int nb_all = (Lk + kBKB - 1) / kBKB;
      const int b1 = nb_all * (part + 1) / ways;
      b0 = nb_all * part / ways;
      k_beg += kBKB * b0;
      Lk = min(kBKB * b1, Lk) - kBKB * b0;
    }
    const int q0 = qt * BQ + w * WQ;
    const int nb = (Lk + kBKB - 1) / kBKB;
    float* part_o = ways > 1 ? a.split_o + (int64_t)(sidx * ways + part) * kSplitRows * D : nullptr;
    const int32_t rb = (int32_t)rs * 2;
    const int32_t rem0 = Lk * rb - rb + D * 2;
    const int32_t bb = kBKB * rb;
    // keys and values: blocks [0, nba) from the token-order rows, the others from the packed rows (the key loop moves
    // each stream's base once, to ksw / vsw: the packed rows of block nba)
    const VRange vr = tok_range(a.v_tok, a.n_vtok, rs, r2.x, r2.y, lk_seg, b0, nb, head * D,
                                (uint64_t)(a.v + (int64_t)k_beg * rs + head * D));
    const VRange kr = tok_range(a.k_tok, a.n_ktok, rs, r2.x, r2.z, lk_seg, b0, nb, head * D,
                                (uint64_t)(a.k + (int64_t)k_beg * rs + head * D));
    uint64_t vaddr = vr.nba > 0 ? vr.a : vr.p;
    uint64_t vsw = vr.p + (uint64_t)vr.nba * (uint32_t)bb;
    int vnext = vr.nba;   // the block (from b0) at which the value stream moves to vsw, 0: never
    // with value runs the stream moves at every event of the segment's list (the leading run's end among them,
    // merged with a run that starts on that block): the item walks the list to its first block (the events up to b0
    // give that block's base), and the key loop takes the events after the first one from vlist
    const int4* vlist = kNoEvents;
    const uint32_t hoff = (uint32_t)(head * D * 2);
    if (r2.w >= 0) {
      const int4* L = a.v_events + r2.w;
      int i = 0;
      int4 e = L[0];
      while (e.x <= b0) {   // the sentinels end the walk
        vaddr = (((uint64_t)(uint32_t)e.z << 32) | (uint32_t)e.y) + hoff + (uint64_t)(b0 - e.x) * (uint32_t)bb;
        e = L[++i];
      }
      vnext = e.x - b0 < nb ? e.x - b0 : 0;
      vsw = (((uint64_t)(uint32_t)e.z << 32) | (uint32_t)e.y) + hoff;
      vlist = L + i + 1;
    }
    // wave-uniform (scalar operands of the key loop)
    auto uni64 = [](uint64_t x) {
      return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(x >> 32)) << 32) |
             (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)x);
    };
    vaddr = uni64(vaddr);
    vsw = uni64(vsw);
    vnext = __builtin_amdgcn_readfirstlane(vnext);
    const uint64_t vlist_u = uni64((uint64_t)vlist);
    const uint64_t ksw = kr.p + (uint64_t)kr.nba * (uint32_t)bb;
    // K block b of the ring head (b = 0, 1) and the block the key loop's descriptor starts at (2)
    auto kblock = [&](int b) { return (b < kr.nba ? kr.a : kr.p) + (uint64_t)b * (uint32_t)bb; };
    const uint64_t kaddr = kblock(0);
    // every wavefront is done with the previous item's ring: a wavefront without live queries leaves its key loop
    // while the others' epilogues still read the last V block, and its refill below would overwrite a slot
    __syncthreads();
    if (nb > 0) {
      // the head of the ring, ahead of the Q loads so that both latencies overlap: K blocks 0 and 1 into slots 0
      // and 1, and zeros (record count 0) into the last V slot, the V operand of the key loop's first PV step; the
      // generated prologue fetches the rest of the ring
      const uint32_t vring = sbase + (uint32_t)(kRing64 * kSlot64 * 2);
      dma_block<2>(kaddr, max(rem0, 0), voff, sbase);
      dma_block<2>(kblock(1), max(rem0 - bb, 0), voff, sbase + kSlot64 * 2);
      dma_block<2>(vaddr, 0, voff + 2, vring + (kRing64 - 1) * kSlot64 * 2);
    }

    // the next item, now or (kLater) after this one
    const int nit = claim(true);
    const ItemRec nrec = item_record(ws, max(nit, 0));
    const int4 n0 = nrec.r0, n1 = nrec.r1;

    // Q operands (unless the previous item's key loop loaded them) and output rows. Rows past the segment take the
    // queries of the segment's last row (the key loop's loads are unconditional); their outputs are not stored.
    uint64_t op[2], qa[2], qc[2];
    int ok[2];
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const int i0 = q0 + qb * 32 + l32;
      const bool live = i0 < Lq;
      const int i = min(i0, Lq - 1);
      const int64_t row = q_src0 + (int64_t)i * a.qstep;
      const uint16_t* qp = (row < a.n_q_video ? a.q + row * a.qs : a.q_text + (row - a.n_q_video) * a.qs) + head * D;
      qc[qb] = (uint64_t)(qp + 8 * h);
      if (!have_q && a.q_rope) {
        // rotated on the load (rows past the segment get zero queries)
        int rr = live ? a.q_rope[q_beg + i] : -1;
        if (rr >= a.n_rope_rows) rr = -1;
#pragma unroll
        for (int k = 0; k < KS; ++k) {
          const int d = 16 * k + 8 * h;
          u32x4 x = {0u, 0u, 0u, 0u};
          if (live) x = *(const u32x4*)(qp + d);
          if (rr >= 0) x = rotate8(x, a.cos_t, a.sin_t, (int64_t)rr * D + d, 1.0f);
          ONEREEL_RING64_QSET_STEP(qb, k, x);
        }
      }
      // the lane's query row of the next item (its last row past the end), or this one's when it is not claimed yet
      qa[qb] = qc[qb];
      if (nit >= 0) {
        const int nLq = n1.x;
        const int ni = min((n0.x >> 8) * BQ + w * WQ + qb * 32 + l32, nLq - 1);
        const int64_t nrow = n1.y + (int64_t)ni * a.qstep;
        qa[qb] = (uint64_t)((nrow < a.n_q_video ? a.q + nrow * a.qs : a.q_text + (nrow - a.n_q_video) * a.qs) +
                            (n0.x & 255) * D + 8 * h);
      }
      uint16_t* o = (row < a.n_q_video ? a.o + row * a.os : a.o_text + (row - a.n_q_video) * a.os) + head * D + 4 * h;
      // a split item's part writes O / l of its keys in fp32 to its partial rows instead
      op[qb] = part_o ? (uint64_t)(part_o + (w * WQ + qb * 32 + l32) * D + 4 * h) : (uint64_t)o;
      ok[qb] = live;
    }
    if (!have_q && !a.q_rope)
      asm volatile(ONEREEL_RING64_QLOAD :: [qa0] "v"(qc[0]), [qa1] "v"(qc[1]) : ONEREEL_RING64_QCLOBBERS);
    if (nb == 0) {
      // no keys: O = 0 and lse = -inf, as attn4_kernel
#pragma unroll
      for (int qb = 0; qb < 2; ++qb)
        if (ok[qb]) {
          uint16_t* o = (uint16_t*)op[qb];
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int gg = 0; gg < 4; ++gg) *(uint2*)(o + db * 32 + 8 * gg) = make_uint2(0u, 0u);
          if (a.lse && h == 0) a.lse[(int64_t)head * a.sum_q + q_beg + q0 + qb * 32 + l32] = -__builtin_inff();
        }
      have_q = false;
      it = nit == kLater ? claim(false) : nit;
      continue;
    }
    const int valid = Lk - (nb - 1) * kBKB - 16 * h;
    const uint64_t kaddr2 = kblock(2);   // K block 2, where the prologue's ring fill starts
    float mo0, mo1, lo0, lo1;   // per query: the running max of q k^T, and the row sum relative to it
    asm volatile(ONEREEL_RING64_ASM
                 : [mo0] "=&v"(mo0), [mo1] "=&v"(mo1), [lo0] "=&v"(lo0), [lo1] "=&v"(lo1)
                 : [qa0] "v"(qa[0]), [qa1] "v"(qa[1]), [c] "s"(a.c), [nb] "s"(nb), [valid] "v"(valid), [kb] "v"(kb),
                   [vb] "v"(vb), [vk0] "v"(voff[0]), [vk1] "v"(voff[1]), [vv0] "v"(voff[2]), [vv1] "v"(voff[3]),
                   [sbase] "s"(sbase), [bb] "s"(bb), [kb_lo] "s"((uint32_t)kaddr2), [kb_hi] "s"((uint32_t)(kaddr2 >> 32)),
                   [vb_lo] "s"((uint32_t)vaddr), [vb_hi] "s"((uint32_t)(vaddr >> 32)), [rem0] "s"(rem0), [remk] "s"(rem0 - 2 * bb),
                   [op0] "v"(op[0]), [op1] "v"(op[1]), [ok0] "v"(ok[0]), [ok1] "v"(ok[1]),
                   [f32] "s"(__builtin_amdgcn_readfirstlane(ways > 1 ? 1 : 0)),
                   [dead] "s"(__builtin_amdgcn_readfirstlane(q0 >= Lq ? 1 : 0)), [vsw] "s"(vsw), [nbav] "s"(vnext),
                   [ksw] "s"(ksw), [nbak] "s"(kr.nba), [vlist] "s"(vlist_u), [hoff] "s"(hoff), [b0] "s"(b0)
                 : ONEREEL_RING64_CLOBBERS);
    // the next item's queries are in a128..a191 unless they must be rotated on the load
    have_q = nit >= 0 && !a.q_rope;
    it = nit == kLater ? claim(false) : nit;
    if (ways <= 1) {
      if (a.lse && h == 0) {
        if (ok[0]) a.lse[(int64_t)head * a.sum_q + q_beg + q0 + l32] = mo0 * a.scale + logf(lo0);
        if (ok[1]) a.lse[(int64_t)head * a.sum_q + q_beg + q0 + 32 + l32] = mo1 * a.scale + logf(lo1);
      }
      continue;
    }
    // a part of a split item: its lse next to its O / l (merge_kernel combines the parts)
    float* part_lse = a.split_lse + (int64_t)(sidx * ways + part) * kSplitRows;
    if (h == 0) {
      if (ok[0]) part_lse[w * WQ + l32] = mo0 * a.scale + logf(lo0);
      if (ok[1]) part_lse[w * WQ + 32 + l32] = mo1 * a.scale + logf(lo1);
    }
  }
}

// Merge of the key-split items, one block per split item (blocks past the count in ws[3] return): query r of the
// item gets O = sum_p e^(lse_p - M) O_p / sum_p e^(lse_p - M) over its parts p, M = max_p lse_p, and
// lse = M + log(sum_p e^(lse_p - M)); 4 dims per thread.
__global__ __launch_bounds__(kThreads) void merge_kernel(AttnArgs a, const int32_t* ws) {
  constexpr int D = 128;
  const int sidx = blockIdx.x;
  if (sidx >= ws[3]) return;
  const int32_t* tab = a.split_tab + 3 * sidx;
  const int seg = tab[0], head = tab[1] & 255, qt = tab[1] >> 8, ways = tab[2];
  const int q_beg = a.cu_q[seg], i_beg = qt * kSplitRows;
  const int n_rows = min(kSplitRows, a.cu_q[seg + 1] - q_beg - i_beg);
  const int q_src0 = a.seg_q_src ? a.seg_q_src[seg] : q_beg;
  const float* lse0 = a.split_lse + (int64_t)sidx * ways * kSplitRows;
  const float* o0 = a.split_o + (int64_t)sidx * ways * kSplitRows * D;
  for (int idx = threadIdx.x; idx < n_rows * (D / 4); idx += kThreads) {
    const int r = idx / (D / 4), d = 4 * (idx % (D / 4));
    float m = -__builtin_inff();
    for (int p = 0; p < ways; ++p) m = fmaxf(m, lse0[p * kSplitRows + r]);
    float wsum = 0.0f, acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int p = 0; p < ways; ++p) {
      const float wt = expf(lse0[p * kSplitRows + r] - m);
      const f32x4 o = *(const f32x4*)(o0 + ((int64_t)p * kSplitRows + r) * D + d);
      wsum += wt;
#pragma unroll
      for (int t = 0; t < 4; ++t) acc[t] += wt * o[t];
    }
    const float inv = 1.0f / wsum;
    const int64_t row = q_src0 + (int64_t)(i_beg + r) * a.qstep;
    uint16_t* out = (row < a.n_q_video ? a.o + row * a.os : a.o_text + (row - a.n_q_video) * a.os) + head * D + d;
    *(uint2*)out = make_uint2(pack2(acc[0] * inv, acc[1] * inv), pack2(acc[2] * inv, acc[3] * inv));
    if (a.lse && d == 0) a.lse[(int64_t)head * a.sum_q + q_beg + i_beg + r] = m + logf(wsum);
  }
}

typedef void (*AttnFn)(AttnArgs, int32_t*);

// head_dim 128 runs the 64-query kernel (256-query items), head_dim 64 the 32-query kernel (128-query items)
AttnFn attn_fn(int D) { return D == 128 ? attn8_kernel : attn4_kernel<64>; }
int item_bq(int D) { return D == 128 ? 256 : 128; }

struct DevInfo {
  int cus = 0;
  int occ[2] = {};  // resident blocks per CU, [D == 128]
};

int dev_info(DevInfo& info) {
  static thread_local int cached_dev = -1;
  static thread_local DevInfo cached;
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev != cached_dev) {
    DevInfo di;
    if (int rc = check_hip(hipDeviceGetAttribute(&di.cus, hipDeviceAttributeMultiprocessorCount, dev),
                           "hipDeviceGetAttribute"))
      return rc;
    for (int d = 0; d < 2; ++d)
      if (int rc = check_hip(hipOccupancyMaxActiveBlocksPerMultiprocessor(&di.occ[d], attn_fn(d ? 128 : 64), kThreads, 0),
                             "hipOccupancyMaxActiveBlocksPerMultiprocessor"))
        return rc;
    cached = di;
    cached_dev = dev;
  }
  info = cached;
  return 0;
}

int64_t max_items_of(int32_t n_seg, int32_t sum_q, int32_t H) {
  return ((int64_t)(sum_q + kMinBQ - 1) / kMinBQ + n_seg) * H;
}

// fewest work items a call can have: every query in one segment
int64_t min_items_of(int32_t sum_q, int32_t H, int32_t D) {
  return (int64_t)H * ((sum_q + item_bq(D) - 1) / item_bq(D));
}

// persistent blocks of an attention launch on the current device: one per resident slot (CUs x blocks per CU, one
// block per CU for the 64-query kernel), or fewer when ONEREEL_ATTN_MAX_BLOCKS (a test setting, read at every call)
// caps the grid so that each block walks many work items
int64_t grid_slots(const DevInfo& di, int32_t D) {
  int64_t grid = (int64_t)di.cus * di.occ[D == 128];
  if (const char* e = getenv("ONEREEL_ATTN_MAX_BLOCKS")) {
    const long cap = strtol(e, nullptr, 10);
    if (cap > 0 && cap < grid) grid = cap;
  }
  return grid;
}

// parts of key-split items a call may hold: only the 64-query kernel (head_dim 128) splits items, and only calls that
// can have fewer than kSplitMaxRounds rounds of items on the device's persistent blocks get room for them. Without a
// device (a size query on a host with no GPU) the count is that of MI355X, 256 blocks.
int64_t split_parts_cap(int32_t n_seg, int32_t sum_q, int32_t H, int32_t D) {
  if (D != 128) return 0;
  DevInfo di;
  const int64_t slots = dev_info(di) == 0 ? grid_slots(di, D) : 256;
  if (min_items_of(sum_q, H, D) >= (int64_t)kSplitMaxRounds * slots) return 0;
  const int64_t mi = max_items_of(n_seg, sum_q, H);
  return mi * kMaxSplitWays < kMaxSplitParts ? mi * kMaxSplitWays : kMaxSplitParts;
}

// workspace layout (bytes): queue headers and the item list, the split table (3 words per split item, at most cap / 2
// of them), then (16-byte aligned) the parts' lse and O / l, for at most `cap` key-split parts
struct WsLayout {
  int64_t tab, lse, o, ev, total;
};

WsLayout ws_layout(int32_t n_seg, int32_t sum_q, int32_t H, int64_t cap) {
  const int64_t mi = max_items_of(n_seg, sum_q, H);
  WsLayout l;
  l.tab = (kWsHeader + kItemWords * (mi + cap)) * 4;
  l.lse = (l.tab + (cap / 2) * 3 * 4 + 15) / 16 * 16;
  l.o = l.lse + cap * kSplitRows * 4;
  l.ev = l.o + cap * kSplitRows * 128 * 4;
  l.total = l.ev + (int64_t)n_seg * kVEvents * 16;
  return l;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// argument checks shared by both entry points (everything but the workspace)
int check_args(const or_varlen_args& x, const char* fn) {
  if (x.D != 64 && x.D != 128) return fail_arg("%s: head_dim %d not supported (64 or 128)", fn, x.D);
  if (x.H < 1 || x.H > 256) return fail_arg("%s: H=%d outside [1, 256]", fn, x.H);
  if (x.n_seg < 1 || x.n_seg > kMaxPlanSeg) return fail_arg("%s: n_seg=%d outside [1, %d]", fn, x.n_seg, kMaxPlanSeg);
  if (x.sum_q < 0) return fail_arg("%s: sum_q < 0", fn);
  if (!x.q || !x.k || !x.v || !x.o || !x.cu_q) return fail_arg("%s: q, k, v, o and cu_q are required", fn);
  if (!x.cu_k && !(x.k_off && x.k_len)) return fail_arg("%s: need cu_k, or k_off with k_len", fn);
  if (x.k_off && !x.k_len) return fail_arg("%s: k_off needs k_len (the per-segment key counts)", fn);
  if (x.q_row_step < 0 || (x.q_row_step > 1 && !x.seg_q_src))
    return fail_arg("%s: q_row_step %d needs seg_q_src (and must not be negative)", fn, x.q_row_step);
  if (x.q_rope && (!x.cos_table || !x.sin_table || x.n_rope_rows < 1))
    return fail_arg("%s: q_rope needs cos / sin tables", fn);
  if (x.q_row_stride < (int64_t)x.H * x.D || x.k_row_stride < (int64_t)x.H * x.D || x.o_row_stride < (int64_t)x.H * x.D)
    return fail_arg("%s: row strides must cover H * D elements", fn);
  if (x.q_row_stride % 8 || x.k_row_stride % 8 || x.o_row_stride % 8 || !aligned16(x.q) || !aligned16(x.k) ||
      !aligned16(x.v) || !aligned16(x.o) || (x.q_text && !aligned16(x.q_text)) || (x.o_text && !aligned16(x.o_text)))
    return fail_arg("%s: pointers must be 16-byte aligned and row strides multiples of 8 elements", fn);
  if (x.cos_table && (((uintptr_t)x.cos_table | (uintptr_t)x.sin_table) & 15u))
    return fail_arg("%s: rotary tables must be 16-byte aligned", fn);
  if ((int64_t)(x.max_k + 8 * 32) * x.k_row_stride * 2 > 0x7fffffffLL)
    return fail_arg("%s: a segment's keys span more than 2 GiB (max_k %d x row stride %lld)", fn, x.max_k,
                    (long long)x.k_row_stride);
  if (x.k_len_head && !x.k_len) return fail_arg("%s: k_len_head needs k_len (each segment's largest key count)", fn);
  if (x.v_tok && (!x.v_lead || !x.v_row || x.v_tok_rows < 0 || !aligned16(x.v_tok)))
    return fail_arg("%s: v_tok needs v_lead, v_row, v_tok_rows >= 0 and 16-byte alignment", fn);
  if (x.k_tok && (!x.k_lead || !x.v_row || x.k_tok_rows < 0 || !aligned16(x.k_tok)))
    return fail_arg("%s: k_tok needs k_lead, v_row, k_tok_rows >= 0 and 16-byte alignment", fn);
  if (x.v_runs && (!x.v_tok || x.D != 128 || x.k_len_head))
    return fail_arg("%s: v_runs needs v_tok and head_dim 128 (and no k_len_head)", fn);
  return 0;
}

// planner + attention kernel (+ merge of key-split parts) on workspace `wsp`, laid out by ws_layout(..., cap)
int launch_varlen(const or_varlen_args& x, void* wsp, int64_t cap, hipStream_t st) {
  if (x.sum_q == 0) return 0;
  DevInfo di;
  if (int rc = dev_info(di)) return rc;
  const int occ = di.occ[x.D == 128];
  if (occ < 1) return fail_arg("or_varlen_fwd: attention kernel cannot be resident (occupancy 0)");
  const int64_t max_items = max_items_of(x.n_seg, x.sum_q, x.H);
  // persistent blocks: one per resident slot, but no more than the work entries (items, or their key parts when
  // the planner may split items: only when even the fewest items the call can have come in few rounds)
  int64_t grid = grid_slots(di, x.D);
  const bool may_split = cap > 0 && min_items_of(x.sum_q, x.H, x.D) < kSplitMaxRounds * grid;
  const int64_t entries = max_items * (may_split ? kMaxSplitWays : 1);
  if (grid > entries) grid = entries;
  AttnArgs a;
  a.q = (const uint16_t*)x.q;
  a.q_text = (const uint16_t*)(x.q_text ? x.q_text : x.q);
  a.k = (const uint16_t*)x.k;
  a.v = (const uint16_t*)x.v;
  a.o = (uint16_t*)x.o;
  a.o_text = (uint16_t*)(x.o_text ? x.o_text : x.o);
  a.lse = x.lse;
  a.cu_q = x.cu_q;
  a.cu_k = x.cu_k;
  a.k_off = x.k_off;
  a.k_len = x.k_len;
  a.seg_q_src = x.seg_q_src;
  a.q_rope = x.q_rope;
  a.cos_t = x.cos_table;
  a.sin_t = x.sin_table;
  a.n_rope_rows = x.q_rope ? x.n_rope_rows : 0;
  a.n_q_video = x.seg_q_src ? x.n_q_video : ((int64_t)1 << 62);
  a.qs = x.q_row_stride;
  a.ks = x.k_row_stride;
  a.os = x.o_row_stride;
  a.qstep = x.q_row_step > 1 ? x.q_row_step : 1;
  a.sum_q = x.sum_q;
  a.H = x.H;
  a.scale = x.scale;
  a.c = x.scale * 1.4426950408889634f;
  int32_t* ws = (int32_t*)wsp;
  const WsLayout wl = ws_layout(x.n_seg, x.sum_q, x.H, cap);
  a.v_tok = (const uint16_t*)x.v_tok;
  a.n_vtok = x.v_tok ? x.v_tok_rows : 0;
  a.k_tok = (const uint16_t*)x.k_tok;
  a.n_ktok = x.k_tok ? x.k_tok_rows : 0;
  a.split_tab = (int32_t*)((char*)wsp + wl.tab);
  a.split_lse = (float*)((char*)wsp + wl.lse);
  a.split_o = (float*)((char*)wsp + wl.o);
  a.v_events = (const int4*)((char*)wsp + wl.ev);
  VRunArgs vra;
  vra.runs = x.v_tok ? x.v_runs : nullptr;
  vra.v_tok = (uint64_t)x.v_tok;
  vra.v = (uint64_t)x.v;
  vra.rsb = x.k_row_stride * 2;
  vra.n_vtok = x.v_tok ? x.v_tok_rows : 0;
  vra.events = (int4*)((char*)wsp + wl.ev);
  // the planner needs key counts only: k_len when given, else the cu_k differences. It writes every word of the
  // workspace the other kernels read (queue headers, item list, split table) before they run.
  // the item records are written by up to 8 blocks (each derives the same queues), about 1024 items per block
  const int plan_blocks = (int)std::min<int64_t>(8, std::max<int64_t>(1, (max_items + 1023) / 1024));
  hipLaunchKernelGGL(plan_kernel, dim3(plan_blocks), dim3(kPlanThreads), 0, st, x.cu_q, x.cu_k,
                     x.k_len ? x.k_off : nullptr,
                     x.k_len, x.seg_q_src, x.v_tok ? x.v_lead : nullptr, x.v_tok || x.k_tok ? x.v_row : nullptr,
                     x.k_tok ? x.k_lead : nullptr, x.k_len_head,
                     x.n_seg, x.H,
                     item_bq(x.D), (int)max_items, (int)grid,
                     may_split ? 1 : 0, (int)cap, vra, ws);
  if (int rc = check_hip(hipGetLastError(), "plan_kernel launch")) return rc;
  hipLaunchKernelGGL(attn_fn(x.D), dim3((unsigned)grid), dim3(kThreads), 0, st, a, ws);
  if (int rc = check_hip(hipGetLastError(), "attn_kernel launch")) return rc;
  // at most rem + 8 < grid + 8 items are split (the planner's rule), and at most cap / 2
  const int64_t n_merge = cap / 2 < grid + kQueues ? cap / 2 : grid + kQueues;
  if (may_split && n_merge > 0) {
    hipLaunchKernelGGL(merge_kernel, dim3((unsigned)n_merge), dim3(kThreads), 0, st, a, ws);
    return check_hip(hipGetLastError(), "merge_kernel launch");
  }
  return 0;
}

// ------------------------------------------------------------------------------------------------------------------
// Library-held workspace of or_varlen_fwd_noalloc: one array per GPU, created with the code object on that GPU and
// held until the process ends. The host name `scratch` is only a stand-in for the symbol: its device address on the
// current GPU comes from hipGetSymbolAddress, once per device, and only that address is passed to kernels.
constexpr int64_t kScratchBytes = OR_NOALLOC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

int scratch_of_current_device(void** out) {
  int dev = 0;
  if (int rc = check_hip(hipGetDevice(&dev), "hipGetDevice")) return rc;
  if (dev < 0 || dev >= kMaxDevices) return fail_arg("or_varlen_fwd_noalloc: device %d beyond %d", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (int rc = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)")) return rc;
    if (!p) return fail_arg("or_varlen_fwd_noalloc: no device address for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return 0;
}

}  // namespace
}  // namespace onereel

using namespace onereel;

extern "C" int64_t or_varlen_workspace_size(int32_t n_seg, int32_t sum_q, int32_t H, int32_t D) {
  if (n_seg < 0 || sum_q < 0 || H < 1) return -1;
  return ws_layout(n_seg, sum_q, H, split_parts_cap(n_seg, sum_q, H, D)).total;
}

extern "C" int or_varlen_fwd(const or_varlen_args* p, void* stream) {
  if (!p) return fail_arg("or_varlen_fwd: args is NULL");
  const or_varlen_args& x = *p;
  if (int rc = check_args(x, "or_varlen_fwd")) return rc;
  const int64_t need = or_varlen_workspace_size(x.n_seg, x.sum_q, x.H, x.D);
  if (!x.workspace || x.workspace_bytes < need || !aligned16(x.workspace))
    return fail_arg("or_varlen_fwd: a 16-byte aligned workspace of %lld bytes is needed", (long long)need);
  return launch_varlen(x, x.workspace, split_parts_cap(x.n_seg, x.sum_q, x.H, x.D), (hipStream_t)stream);
}

extern "C" int or_varlen_fwd_noalloc(const or_varlen_args* p, void* stream) {
  if (!p) return fail_arg("or_varlen_fwd_noalloc: args is NULL");
  const or_varlen_args& x = *p;
  if (int rc = check_args(x, "or_varlen_fwd_noalloc")) return rc;
  // key-split parts: as many as or_varlen_fwd would use, fewer when their partial results do not fit the array
  int64_t cap = split_parts_cap(x.n_seg, x.sum_q, x.H, x.D);
  const int64_t base = ws_layout(x.n_seg, x.sum_q, x.H, 0).total;
  if (base > kScratchBytes)
    return fail_arg("or_varlen_fwd_noalloc: the call needs %lld bytes of work-item queue, more than the %lld-byte "
                    "library array (fewer packed queries, segments or heads per call, or or_varlen_fwd with a "
                    "caller workspace)", (long long)base, (long long)kScratchBytes);
  while (cap > 0 && ws_layout(x.n_seg, x.sum_q, x.H, cap).total > kScratchBytes) cap = cap * 3 / 4;
  if (x.sum_q == 0) return 0;
  void* ws = nullptr;
  if (int rc = scratch_of_current_device(&ws)) return rc;
  return launch_varlen(x, ws, cap, (hipStream_t)stream);
}
