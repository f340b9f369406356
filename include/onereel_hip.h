/*
 * onereel_hip.h: C ABI of libonereel_hip.so, the MI355X (gfx950) scene-structured attention hot path.
 *
 * One DiT attention layer of OneReel's scene attention on one GPU runs as:
 *   or_layout_build   scope layout on the device: cu_seqlens, key ranges, per-row gather indices and scene-RoPE rows
 *   or_pack_gather    K/V (or Q) rows of every scope packed densely, RoPE applied on the way (optionally the text
 *                     scopes read their keys in place from their video scopes' packed rows)
 *   or_rotate_rows    the video queries rotated once, in token order (RoPE ahead of in-place attention)
 *   or_pack_layer     or_pack_gather (K, and the values not read in place) and or_rotate_rows in one launch
 *   or_varlen_fwd     packed varlen attention (bf16 MFMA), optional RoPE on the Q load, optional in-place Q / O,
 *                     each segment's leading keys and values optionally read in place from token-order rows
 *   or_scatter        packed output rows written back to token order, text padding rows zeroed
 *   or_lse_merge      log-sum-exp merge of two partial attention results (attention split over key sets)
 *   or_rmsnorm_rope   fused RMSNorm + interleaved RoPE of the Wan self-attention's queries and keys
 *   or_frame_pool     frame memory: per-frame sums of hidden states (deterministic)
 *   or_frame_select   frame memory: k-means (cosine) representatives and their medoids, one workgroup
 *   or_memory_select, or_memory_foreign,
 *   or_memory_index                            bounded memory: per-head k-means representatives, each piece's foreign
 *                                              representatives (multi-head form) or key lists (single-head form)
 *
 * The fused elementwise kernels of the Wan-shaped DiT block harness (a measurement harness around the scene path,
 * not part of it) are a separate library, libonereel_dit.so (include/onereel_dit.h).
 *
 * Conventions: every tensor is caller-owned device memory passed as a raw pointer; rows are [row][head][dim] with a
 * row stride in elements; bf16 is IEEE bfloat16 stored as uint16_t; index arrays are int32. Every launch goes on the
 * given stream (a hipStream_t, NULL = the null stream) and nothing synchronises the device. Entry points return 0 on
 * success and a negative code on a bad argument (-1) or a HIP error (-2); or_last_error() returns the message of the
 * calling thread's last failure. The library allocates no device memory: or_varlen_fwd takes a caller workspace of
 * or_varlen_workspace_size() bytes.
 *
 * Row space of the layout's index arrays: the virtual concatenation [video tokens ; text rows]. A video token row is
 * frame * T + spatial (frame-major, F*T rows); text row t of the valid-first text sequence is encoded as F*T + t.
 */
#ifndef ONEREEL_HIP_H
#define ONEREEL_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_MAX_SCENES 64
#define OR_MAX_EXTRA 512

/* Scene layout of one request, host memory. Mirrors SceneLayout(lengths, halo, sides, extra)
 * (src/onereel/layout.py:10-22) plus the scope options of the HunyuanVideo-1.5 processor: text counts per sentence
 * (Context.counts / text_ranges, src/onereel/models/hunyuan15.py:64,87-89), scene_rope / rope_lengths (:47-48) and
 * shared_pos resolved for the current step (:162: 'adjacent', or 'switch' at step >= shared_switch). */
typedef struct or_layout_desc {
  int32_t n_scenes;                      /* 1..OR_MAX_SCENES */
  int32_t T;                             /* video tokens per latent frame */
  int32_t halo;                          /* halo frames per neighbouring side */
  int32_t sides;                         /* 0 'adj', 1 'prev', 2 'next' */
  int32_t with_text;                     /* 1: joint scopes V_j, T_j (hunyuan15.py:153-170); 0: video-only scopes
                                            (wan.py:113-119) */
  int32_t scene_rope;                    /* temporal RoPE index restarts at every scene (+1 after scene 0) */
  int32_t adjacent;                      /* shared frames' keys at their adjacent positions (_move_shared) */
  int32_t n_rope_lengths;                /* 0: the scene lengths; else the rope_lengths entries */
  int32_t text_rows;                     /* Le: rows of the text q/k/v (valid tokens first, padding after) */
  int32_t text_keys_in_place;            /* with text: 0 packs every segment's keys in _segments' order (V_j: own
                                            frames, shared frames, sentence; T_j: own frames, sentence); 1 orders
                                            V_j's keys as own frames, sentence, shared frames, so that T_j's keys
                                            (hunyuan15.py:167-168: the same rows) are a prefix of V_j's: T_j packs
                                            no rows and reads that range in place (k_off / k_len) */
  int32_t q_lo, q_hi;                    /* q_hi > 0: one rank's share of the layer (Processor.scene with several
                                            ranks, hunyuan15.py:219-224): only the video queries in tokens
                                            [q_lo, q_hi) (each scene's clipped to the range, with the scene's full
                                            keys) and the sentences of the scenes whose first token lies in it; the
                                            other scenes' segments are empty. q_hi = 0: the whole layer */
  int32_t lengths[OR_MAX_SCENES];        /* latent frames per scene, each > 0 */
  int32_t rope_lengths[OR_MAX_SCENES];
  int32_t counts[OR_MAX_SCENES];         /* valid text tokens of sentence j */
  int32_t extra_ptr[OR_MAX_SCENES + 1];  /* CSR of SceneLayout.extra: frames extra[extra_ptr[j] .. extra_ptr[j+1]) */
  int32_t extra[OR_MAX_EXTRA];
} or_layout_desc;

/* Sizes of a layout, computed on the host from the descriptor (validates it). */
typedef struct or_layout_sizes {
  int64_t n_seg;       /* 2 * n_scenes with text, n_scenes without */
  int64_t sum_q;       /* packed query rows */
  int64_t sum_k;       /* packed key / value rows */
  int64_t max_q;
  int64_t max_k;       /* largest key count of a segment (k_len) */
  int64_t n_video;     /* F * T */
  int64_t max_rope_row;/* largest rotary-table row any index array names (-1 if none) */
} or_layout_sizes;

/* Outputs of or_layout_build, caller-allocated int32 device arrays; any pointer may be NULL to skip it. */
typedef struct or_layout_out {
  int32_t* cu_q;       /* [n_seg + 1] */
  int32_t* cu_k;       /* [n_seg + 1] */
  int32_t* seg_q_src;  /* [n_seg] source row of the segment's first query (its queries are contiguous there) */
  int32_t* q_src;      /* [sum_q] query row of every packed query (= the row its output is written back to) */
  int32_t* q_rope;     /* [sum_q] rotary-table row of a raw (unrotated) query, -1 for text rows */
  int32_t* k_src;      /* [sum_k] key / value row of every packed key */
  int32_t* k_rope;     /* [sum_k] rotary-table row of a raw key: own frames at their (scene) position, shared frames
                          at their adjacent position when moved, else their own; -1 for text rows */
  int32_t* k_move_a;   /* [sum_k] already-rotated keys: _move_shared's inverse-rotation row a*T+s, -1 if not moved */
  int32_t* k_move_b;   /* [sum_k] already-rotated keys: _move_shared's rotation row (a+d)*T+s, -1 if not moved */
  int32_t* k_off;      /* [n_seg] first packed key row of segment s (cu_k[s], or V_j's first row for T_j with
                          text_keys_in_place) */
  int32_t* k_len;      /* [n_seg] its key count (the varlen call's k_off / k_len) */
  int32_t* v_lead;     /* [n_seg] keys at the head of segment s whose value rows the attention call can read in place
                          from the token-order values: the scene's own-frame keys (every segment's keys start with
                          them), rounded down to a multiple of OR_VARLEN_KEY_BLOCK; 0 for a segment without keys */
  int32_t* v_row;      /* [n_seg] token row of segment s's first key (the first own-frame token of its scene) */
  int32_t* v_src;      /* [sum_k] value row to pack for packed key row r: k_src[r], or -1 when r lies in the first
                          v_lead keys of its segment, or (with v_runs) in a whole key block of one of its value runs
                          (read in place, not packed) */
  int32_t* v_runs;     /* optional [n_seg * OR_VALUE_RUNS * 3]: the value runs of segment s after its leading run, up
                          to OR_VALUE_RUNS of them: entry r = (key offset in the segment, key count, first token row)
                          of its r-th shared frame (T consecutive token rows), (0, 0, 0) past the last; the attention
                          call reads their whole key blocks in place (or_varlen_args.v_runs). NULL: none, and v_src
                          packs every value past v_lead */
} or_layout_out;

/* Keys per block of the attention kernels' K/V stream: a segment's in-place value rows (or_varlen_args.v_lead) come
 * in whole blocks. */
#define OR_VARLEN_KEY_BLOCK 32
/* Value runs per segment past its leading one (or_layout_out.v_runs, or_varlen_args.v_runs). */
#define OR_VALUE_RUNS 4

/* Replaces the host-side layout logic of SceneLayout.shared_frames / key_frames (src/onereel/layout.py:54-78),
 * comm.runs / frame_tokens (src/onereel/parallel/comm.py:84-85,115-123) and the sizes of attention.packed's
 * cu_seqlens (src/onereel/attention.py:28-29,67-70). Host only, no device work. */
int or_layout_plan(const or_layout_desc* desc, or_layout_sizes* sizes);

/* Replaces _segments' scope order and rows (src/onereel/models/hunyuan15.py:153-170, :225 own_rows), cu_seqlens
 * (src/onereel/attention.py:28-29), scene_rope_rows (hunyuan15.py:443-454), frame_position / adjacent_positions /
 * shared_positions (hunyuan15.py:92-124) and _move_shared's table rows (hunyuan15.py:136-145). One kernel launch. */
int or_layout_build(const or_layout_desc* desc, const or_layout_out* out, void* stream);

/* Replaces the pack copies of Processor.scene / _segments / attention.packed (hunyuan15.py:164,168,225;
 * attention.py:69) and, with rope, diffusers apply_rotary_emb on the keys (hunyuan15.py:189-190) and _move_shared
 * (hunyuan15.py:148-150).
 * For every packed row r: src = src_idx[r]; row = src < n_video ? a_video[src] : a_text[src - n_video] (and the same
 * for b when b_out != NULL); a_out[r] = rotate(row), b_out[r] = row.
 * rotate: rope_row[r] >= 0 and move_from == NULL: RoPE at table row rope_row[r];
 *         move_from != NULL and move_from[r] >= 0: x = bf16(R(-move_from[r]) row), then bf16(R(rope_row[r]) x);
 *         else: a copy. cos / sin: fp32 [n_rope_rows, D] (may be NULL when no row is rotated). */
int or_pack_gather(const void* a_video, const void* a_text, const void* b_video, const void* b_text,
                   int64_t src_row_stride, int64_t text_row_stride, int64_t n_video,
                   const int32_t* src_idx, const int32_t* rope_row, const int32_t* move_from,
                   const float* cos_table, const float* sin_table, int64_t n_rope_rows,
                   int64_t n_rows, int32_t H, int32_t D, void* a_out, void* b_out, void* stream);

/* Replaces the RoPE of the video queries in Processor.__call__ (src/onereel/models/hunyuan15.py:183-191, diffusers
 * apply_rotary_emb on q): for every r < n_rows with src = src_idx[r] < n_video, row src of out = row src of x
 * rotated at table row rope_row[r] (not rotated when rope_row[r] < 0 or past the table), with the rounding of
 * or_pack_gather; rows src >= n_video are skipped. With a layout's q_src / q_rope it rotates every video query once,
 * in token order, ahead of an attention call that reads the queries in place. x, out: bf16 rows of H * D elements
 * (row strides in elements); out may not alias x. */
int or_rotate_rows(const void* x, int64_t x_row_stride, int64_t n_video, const int32_t* src_idx,
                   const int32_t* rope_row, const float* cos_table, const float* sin_table, int64_t n_rope_rows,
                   int64_t n_rows, int32_t H, int32_t D, void* out, int64_t out_row_stride, void* stream);

/* Arguments of or_pack_layer: the K/V pack of or_pack_gather (keys as its a rows, values as its b rows) and the query
 * rotation of or_rotate_rows, one launch. */
typedef struct or_pack_args {
  const void* k_video;        /* bf16 key rows [video ; text], as or_pack_gather's a_video / a_text */
  const void* k_text;
  const void* v_video;        /* bf16 value rows, same strides (NULL with v_out NULL: keys only) */
  const void* v_text;
  int64_t video_row_stride;   /* elements between video rows (keys and values) */
  int64_t text_row_stride;
  int64_t n_video;            /* rows of the video part: source rows >= n_video are text rows */
  const int32_t* k_src;       /* [n_keys] source row of packed key r (-1: nothing written for r) */
  const int32_t* k_rope;      /* optional [n_keys] as or_pack_gather's rope_row */
  const int32_t* k_move_from; /* optional [n_keys] as or_pack_gather's move_from */
  const int32_t* v_src;       /* optional [n_keys] source row of packed value r, -1: not packed (its row of v_out is
                                 not written; the attention call reads it in place); NULL: k_src */
  int64_t n_keys;
  const int32_t* k_dst;       /* optional [n_keys]: the row of k_out / v_out that packed key r is written to (r when
                                 NULL) */
  void* k_out;                /* bf16 [rows, H, D]: n_keys rows, or the rows k_dst names */
  void* v_out;                /* bf16, as k_out, or NULL */
  const void* q;              /* video queries rotated in token order, as or_rotate_rows(q, .., q_out) */
  int64_t q_row_stride;
  const int32_t* q_src;       /* [n_queries] */
  const int32_t* q_rope;      /* [n_queries] */
  int64_t n_queries;          /* 0: no query rotation */
  void* q_out;
  int64_t q_out_row_stride;
  const float* cos_table;     /* fp32 [n_rope_rows, D] */
  const float* sin_table;
  int64_t n_rope_rows;
  int32_t H;
  int32_t D;
} or_pack_args;

/* Replaces the same code as or_pack_gather and or_rotate_rows together (hunyuan15.py:164,168,183-191,225;
 * attention.py:69): one layer's K/V pack and query rotation in one launch, with the results of those two calls, except
 * that rows whose v_src is -1 are left out of v_out. */
int or_pack_layer(const or_pack_args* args, void* stream);

/* Replaces the write-back of Processor.scene (hunyuan15.py:226,231-235) after attention.packed's split
 * (attention.py:71): o_video[dst] / o_text[dst - n_video] = packed[r] for dst = dst_idx[r]; then the text rows
 * [text_zero_from, text_rows) of o_text are zeroed (the padding rows of ot = eq.new_zeros). */
int or_scatter(const void* packed, const int32_t* dst_idx, int64_t n_rows, int64_t n_video,
               void* o_video, void* o_text, int64_t dst_row_stride, int64_t text_row_stride,
               int64_t text_zero_from, int64_t text_rows, int32_t H, int32_t D, void* stream);

/* Arguments of or_varlen_fwd. Segment s has queries [cu_q[s], cu_q[s+1]) of the packed query space and keys
 * k[k_start .. k_start + k_len) with k_start = k_off ? k_off[s] : cu_k[s] and k_len = k_len ? k_len[s] :
 * cu_k[s+1] - cu_k[s]. Query i of segment s is read from (and its output written to) source row
 * (seg_q_src ? seg_q_src[s] : cu_q[s]) + i * max(q_row_step, 1), a row of q / o when below n_q_video, else of
 * q_text / o_text. */
typedef struct or_varlen_args {
  const void* q;            /* bf16 [.., H, D] rows with stride q_row_stride */
  const void* q_text;       /* bf16 text query rows (may equal q when n_q_video covers every row) */
  const void* k;            /* bf16 [Nk, H, D] */
  const void* v;            /* bf16 [Nk, H, D] */
  void* o;                  /* bf16 output rows, same row space as q */
  void* o_text;
  float* lse;               /* optional fp32 [H, sum_q]: natural-log log-sum-exp of the scaled scores */
  const int32_t* cu_q;      /* [n_seg + 1] */
  const int32_t* cu_k;      /* [n_seg + 1] or NULL with k_off and k_len */
  const int32_t* k_off;     /* optional [n_seg] */
  const int32_t* k_len;     /* optional [n_seg] (seqused_k) */
  const int32_t* seg_q_src; /* optional [n_seg] */
  const int32_t* q_rope;    /* optional [sum_q] rotary-table row per packed query (-1: none) */
  const float* cos_table;   /* fp32 [n_rope_rows, D] when q_rope != NULL */
  const float* sin_table;
  int64_t n_rope_rows;
  int64_t n_q_video;
  int64_t q_row_stride;     /* elements between consecutive rows of q / q_text */
  int64_t k_row_stride;     /* of k and v */
  int64_t o_row_stride;     /* of o / o_text */
  int32_t n_seg;
  int32_t sum_q;
  int32_t max_q;
  int32_t max_k;
  int32_t H;
  int32_t D;                /* 64 or 128 */
  float scale;              /* softmax scale, D^-0.5 in the reference */
  void* workspace;          /* device scratch of or_varlen_workspace_size() bytes */
  int64_t workspace_bytes;
  int32_t q_row_step;       /* 0 or 1: a segment's queries are consecutive source rows; s > 1 (with seg_q_src):
                               query i of segment s is source row seg_q_src[s] + i * s, and its output row too
                               (e.g. one head of [tokens, H, D] rows viewed as [tokens * H, 1, D]: s = H) */
  const void* v_tok;        /* optional token-order value rows, row stride k_row_stride, read in place: the first
                               v_lead[s] keys of segment s take their values from rows v_row[s] .. v_row[s] +
                               v_lead[s] - 1 of v_tok, its other keys from v as without v_tok (rows k_start +
                               v_lead[s] ..). v_lead[s]: a multiple of OR_VARLEN_KEY_BLOCK, at most k_len; blocks past
                               v_tok_rows are taken from v. NULL: every value from v. (A layout's v_lead / v_row, with
                               the values packed per its v_src, read the own-frame values in place.) */
  const int32_t* v_lead;    /* [n_seg], with v_tok */
  const int32_t* v_row;     /* [n_seg], with v_tok */
  int64_t v_tok_rows;       /* rows of v_tok */
  const int32_t* k_len_head;/* optional [n_seg * H] (with k_len): head h of segment s attends to the first
                               min(k_len_head[s * H + h], k_len[s]) keys of the segment's range, e.g. a shared prefix
                               followed by rows that differ per head (the bounded memory's representatives) */
  const void* k_tok;        /* optional token-order key rows, row stride k_row_stride, read in place as v_tok is: the
                               first k_lead[s] keys of segment s are rows v_row[s] .. of k_tok, its other keys from k
                               (rows k_start + k_lead[s] ..); k_lead[s] a multiple of OR_VARLEN_KEY_BLOCK */
  const int32_t* k_lead;    /* [n_seg], with k_tok (and v_row) */
  int64_t k_tok_rows;       /* rows of k_tok */
  const int32_t* v_runs;    /* optional, with v_tok, head_dim 128 only: [n_seg * OR_VALUE_RUNS * 3] further runs of
                               segment s's values in v_tok: entry r = (key offset x0, key count n, token row t), keys
                               x0 .. x0 + n - 1 of the segment taking their values from rows t .. t + n - 1 of v_tok;
                               runs past the leading v_lead keys, in increasing x0, not overlapping it or each other
                               (n = 0: unused). Only their whole key blocks (inside the segment, its key count and
                               v_tok_rows) are read in place, the other keys' values from v (a layout's v_runs, with
                               the values packed per its v_src) */
} or_varlen_args;

/* Bytes of device workspace or_varlen_fwd needs for this many segments, packed queries and heads: the work-item
 * queues, plus, for head_dim 128 calls with few query tiles, room for the fp32 partial results of items split by
 * keys (up to 135 MB). */
int64_t or_varlen_workspace_size(int32_t n_seg, int32_t sum_q, int32_t H, int32_t D);

/* Replaces attention.varlen / flash_attn_varlen_func (src/onereel/attention.py:39-43), varlen_lse (:46-53) and
 * overlapping_ranges' FA3 call with seqused_k (:78-83): non-causal softmax(q k^T * scale) v per segment, bf16 in and
 * out, fp32 accumulation. Two launches: a tile planner and the attention kernel (64 queries per wavefront at
 * D = 128, 32 at D = 64). */
int or_varlen_fwd(const or_varlen_args* args, void* stream);

/* Bytes of the device array that or_varlen_fwd_noalloc uses in place of a caller workspace (one per GPU). */
#define OR_NOALLOC_SCRATCH_BYTES (32ll << 20)

/* No counterpart in the reference: or_varlen_fwd for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc). Same arguments and results; args->workspace and
 * args->workspace_bytes are ignored. The work-item queue (and the key-split partials) live in a fixed array of
 * OR_NOALLOC_SCRATCH_BYTES bytes inside the library, one per GPU, held until the process ends; no call allocates or
 * frees memory. A call whose queue alone exceeds the array is rejected (-1). Calls with few work items split fewer
 * of them by keys when the partials would not fit (the same results within the kernel's rounding). Every call on a
 * GPU shares that GPU's array: calls that overlap on one GPU (other streams, other threads) race and must be
 * serialised by the caller; calls on one stream are ordered. */
int or_varlen_fwd_noalloc(const or_varlen_args* args, void* stream);

/* Replaces the log-sum-exp merge of partial attention results: ring._merge (src/onereel/parallel/ring.py:63-70) and
 * the merge in Processor._far_lse (src/onereel/models/hunyuan15.py:270-275). o: fp32 [n_rows, H, D] (row stride
 * o_row_stride elements), lse: fp32 [H, n_rows], both updated in place with the partial result o_s: bf16
 * [n_rows, H, D] (row stride os_row_stride), lse_s: fp32 [H, n_rows] (as or_varlen_fwd writes them). Per (row, head):
 * m = max(lse, lse_s) (0 if infinite), w1 = exp(lse - m), w2 = exp(lse_s - m), o = o * (w1 / (w1 + w2)) +
 * o_s * (w2 / (w1 + w2)), lse = m + log(w1 + w2). Two kernel launches. */
int or_lse_merge(float* o, float* lse, const void* o_s, const float* lse_s, int64_t n_rows, int32_t H, int32_t D,
                 int64_t o_row_stride, int64_t os_row_stride, void* stream);

/* Replaces _qk of the Wan self-attention (src/onereel/models/wan.py:64-74): RMSNorm over each token row's C = H * D
 * elements with weight w (bf16 [C]) and eps, then diffusers' interleaved RoPE per head with c = cos[row, 2i],
 * s = sin[row, 2i + 1] (cos[..., 0::2], sin[..., 1::2]): out[2i] = y[2i] c - y[2i+1] s, out[2i+1] = y[2i] s +
 * y[2i+1] c; fp32 throughout, one rounding to bf16. q and k (k may be NULL) in one launch. Rows: bf16 with the given
 * strides (elements); cos / sin: fp32 [n_rope_rows, D], table row rope_row[r] (rope_row NULL: row r; out of range:
 * no rotation). With n_rope_rows = 0 and no tables it is the RMSNorm alone (the norm_q / norm_k of diffusers'
 * Wan cross-attention processor, which wan.py:83-87 calls per scene). D must divide 512 and C be a multiple of 512. */
int or_rmsnorm_rope(const void* q, const void* k, const void* wq, const void* wk, int64_t q_row_stride,
                    int64_t k_row_stride, int64_t n_rows, int32_t C, int32_t D, float eps, const float* cos_table,
                    const float* sin_table, const int32_t* rope_row, int64_t n_rope_rows, void* q_out, void* k_out,
                    int64_t qo_row_stride, int64_t ko_row_stride, void* stream);

/* Replaces the pooling of FrameMemory.collect (src/onereel/frame_memory.py:76-85, index_add_ of one layer's video rows
 * into per-frame sums and counts): for the frame-major rows r of hs (bf16, row stride row_stride elements, C wide),
 * frame (row0 + r) / T, sums[frame] += the row (fp32 [n_frames, C]) and counts[frame] += 1 (fp32 [n_frames]). Rows
 * are added in row order: the result does not depend on scheduling. */
int or_frame_pool(const void* hs, int64_t n_rows, int32_t C, int64_t row_stride, int64_t row0, int32_t T,
                  int32_t n_frames, float* sums, float* counts, void* stream);

/* Replaces FrameMemory.select (src/onereel/frame_memory.py:114-132): k-means with the dot product as similarity over
 * the L2-normalised feature rows feats[cand[n]] (fp32 [n_frames, C]; cand: int32 [n_cand] device, each < n_frames):
 * farthest-point initialisation from candidate 0, at most iters passes (stop when the centres do not change), then
 * per non-empty cluster the member most similar to its centre (the first on ties). reps: int32 [k] device, the chosen
 * frames ascending, -1 after them. work: fp32 [8, C] device scratch. One workgroup; k * C <= 32768. */
int or_frame_select(const float* feats, int32_t n_frames, int32_t C, const int32_t* cand, int32_t n_cand, int32_t k,
                    int32_t iters, int32_t* reps, float* work, void* stream);

/* Bytes of device workspace or_memory_select needs: the normalised keys [H, B, D] fp32 and per-candidate arrays. */
int64_t or_memory_select_workspace_size(int32_t B, int32_t H, int32_t D, int32_t M, int32_t iters);

/* Replaces BoundaryMemory.select (src/onereel/memory.py:58-93): per head h, k-means over the B candidate keys
 * x_b = key_b / max(|key_b|, 1e-12) (key_b: row rows[b] (or b) of keys, head h, D elements; bf16, or fp32 when
 * fp32_keys) into M clusters with squared Euclidean distance |x|^2 - 2 x.c + |c|^2 (fp32; the nearest centroid, the
 * lowest index on equal distances), centroids (fp32 [H, M, D], 16-byte aligned) updated in place: from the
 * candidates init[i] (int32 [M]) when init != NULL, else from their current values; `iters` update passes, an empty
 * cluster keeping its centroid, stopping early once no centroid moves (device-side: no host read). Then per head,
 * for every non-empty cluster in cluster order, the member nearest its centroid (the lowest candidate on equal
 * distances): rep (int64 [H, M]) = those candidates, valid (uint8 [H, M]) = 1, zeros after them. M <= min(B, 1024),
 * D 64 or 128; keys and centroids 16-byte aligned, key rows a multiple of 16 bytes apart. Sums are taken in a fixed
 * order (deterministic). */
int or_memory_select(const void* keys, int32_t fp32_keys, const int32_t* rows, int64_t key_row_stride, int32_t B,
                     int32_t H, int32_t D, int32_t M, float* centroids, const int32_t* init, int32_t iters,
                     int64_t* rep, uint8_t* valid, void* workspace, int64_t workspace_bytes, void* stream);

/* Replaces the key-list building of MemoryAttention.__call__ (src/onereel/memory.py:152-168), the per-call part: for
 * every piece i and head h (segment h * n_pieces + i), after the piece's piece_len[i] local keys at
 * kidx[k_off[seg] ..], the single-head rows cand_row[rep[h, r]] * H + h of head h's valid representatives r (in
 * order) whose scene cand_scene[rep[h, r]] differs from piece_scene[i], when piece_mem[i]; k_len[seg] = piece_len[i]
 * + their count. kidx must hold piece_len[i] + M entries from k_off[seg]. One launch. */
int or_memory_index(const int64_t* rep, const uint8_t* valid, const int64_t* cand_row, const int64_t* cand_scene,
                    const int64_t* piece_scene, const uint8_t* piece_mem, const int32_t* piece_len,
                    const int32_t* k_off, int32_t n_pieces, int32_t H, int32_t M, int32_t* kidx, int32_t* k_len,
                    void* stream);

/* Replaces the same key-list building (memory.py:152-168) for the multi-head form of the bounded memory's attention,
 * where the packed K / V rows hold every head and each head's foreign representatives sit in its own head slot after
 * the piece's piece_len[i] local keys (packed rows k_off[i] ..): for piece i, head h and slot r < M, fsrc / fdst
 * [n_pieces * H * M] (index (i * H + h) * M + r) get the source row cand_row[rep[h, x]] * H + h of head h's x-th
 * valid representative whose scene differs from piece_scene[i] (in order; -1 past the last, and for pieces with
 * piece_mem[i] = 0) and the packed row (k_off[i] + piece_len[i] + r) * H + h, both rows of [rows * H, 1, D] views
 * (an or_pack_layer job with H = 1 moves them); k_len_head[i * H + h] = piece_len[i] + their count. One launch. */
int or_memory_foreign(const int64_t* rep, const uint8_t* valid, const int64_t* cand_row, const int64_t* cand_scene,
                      const int64_t* piece_scene, const uint8_t* piece_mem, const int32_t* piece_len,
                      const int32_t* k_off, int32_t n_pieces, int32_t H, int32_t M, int32_t* fsrc, int32_t* fdst,
                      int32_t* k_len_head, void* stream);

/* Message of the calling thread's last failed call ("" if none). */
const char* or_last_error(void);

/* Library version string. */
const char* or_version(void);

#ifdef __cplusplus
}
#endif

#endif /* ONEREEL_HIP_H */
