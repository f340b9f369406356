// Shared helpers of libonereel_hip: error reporting, bf16 conversion and the per-scene layout logic that both the
// host planner (or_layout_plan) and the device layout kernel run, so that sizes and indices come from one code.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/onereel_hip.h"

namespace onereel {

// ---------------------------------------------------------------------------------------------------------------
// errors
void set_error(const char* fmt, ...);
int fail_arg(const char* fmt, ...);   // records the message, returns -1
int check_hip(hipError_t e, const char* what);  // 0 or -2 with the HIP error string

// ---------------------------------------------------------------------------------------------------------------
// bf16 (stored as uint16_t); conversions round to nearest even, as torch's .to(torch.bfloat16) does
__host__ __device__ inline float bf2f(uint16_t h) {
  union { uint32_t u; float f; } x;
  x.u = (uint32_t)h << 16;
  return x.f;
}

__host__ __device__ inline uint16_t f2bf(float f) {
  union { uint32_t u; float f; } x;
  x.f = f;
  uint32_t u = x.u;
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // NaN stays a quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// ---------------------------------------------------------------------------------------------------------------
// scene layout: derived per-scene quantities, computed identically on host and device
constexpr int kMaxShared = 1024;  // shared-frame entries over all scenes (halo + extra)

struct LayoutDerived {
  int n_scenes, T, F, with_text, scene_rope, adjacent, text_rows, n_rope;
  int text_in_place;                               // T_j's keys read in place from V_j's (own frames, sentence first)
  int qa, qb;                                      // the rank's video query tokens [qa, qb) (all: [0, F T))
  int lo[OR_MAX_SCENES], hi[OR_MAX_SCENES];        // frame range of scene j (layout.py:43-45)
  int t0[OR_MAX_SCENES], t1[OR_MAX_SCENES];        // text range of sentence j (hunyuan15.py:87-89)
  int rope_start[OR_MAX_SCENES + 1];               // frame boundaries of the rope scenes
  int sh_ptr[OR_MAX_SCENES + 1];                   // shared frames of scene j: sh[sh_ptr[j] .. sh_ptr[j+1])
  int sh[kMaxShared];
  int sh_dst[kMaxShared];                          // their temporal position when moved (adjacent)
};

// temporal RoPE index of frame f (hunyuan15.py:103-113); -1 when f lies past the rope scenes (IndexError there)
__host__ __device__ inline int frame_position(const LayoutDerived& L, int f) {
  if (!L.scene_rope) return f;
  for (int s = 0; s < L.n_rope; ++s) {
    int start = L.rope_start[s];
    if (f < L.rope_start[s + 1]) return f - start + (start > 0 ? 1 : 0);
  }
  return -1;
}

// rotary-table row of video token `tok` under the scene's RoPE (scene_rope_rows, hunyuan15.py:443-454)
__host__ __device__ inline int rope_row_of_token(const LayoutDerived& L, int tok) {
  if (!L.scene_rope) return tok;
  int f = tok / L.T;
  return frame_position(L, f) * L.T + (tok - f * L.T);
}

// shared frames of scene j (layout.py:54-69) written to out (capacity cap); returns their count or -1 on overflow.
// Halo first (previous neighbour's last `halo` frames, then the next one's first), then sorted(extra[j]) keeping
// frames outside the scene that are not in the halo list (repeats inside extra[j] are kept, as the reference does).
__host__ __device__ inline int scene_shared_frames(const or_layout_desc& d, const int* lo, const int* hi, int j,
                                                   int* out, int cap) {
  int n = 0;
  const int k = d.halo;
  if (k > 0) {
    if (j > 0 && (d.sides == 0 || d.sides == 1)) {
      int a = hi[j - 1] - k;
      if (a < lo[j - 1]) a = lo[j - 1];
      for (int f = a; f < hi[j - 1]; ++f) {
        if (n >= cap) return -1;
        out[n++] = f;
      }
    }
    if (j + 1 < d.n_scenes && (d.sides == 0 || d.sides == 2)) {
      int b = lo[j + 1] + k;
      if (b > hi[j + 1]) b = hi[j + 1];
      for (int f = lo[j + 1]; f < b; ++f) {
        if (n >= cap) return -1;
        out[n++] = f;
      }
    }
  }
  const int nh = n;
  const int e0 = d.extra_ptr[j], e1 = d.extra_ptr[j + 1];
  // insertion of sorted(extra[j]) after the halo, filtered as it goes (filter does not depend on the order)
  for (int e = e0; e < e1; ++e) {
    const int f = d.extra[e];
    if (lo[j] <= f && f < hi[j]) continue;
    bool in_halo = false;
    for (int i = 0; i < nh; ++i) in_halo |= (out[i] == f);
    if (in_halo) continue;
    if (n >= cap) return -1;
    int p = n++;
    while (p > nh && out[p - 1] > f) {
      out[p] = out[p - 1];
      --p;
    }
    out[p] = f;
  }
  return n;
}

// temporal position of shared frame f of scene j when moved (shared_positions / adjacent_positions,
// hunyuan15.py:92-124). `sh` holds the scene's n shared frames. A dict keyed by frame keeps a repeated frame's last
// index, so the count of entries <= f (of the relevant group) fixes the position.
__host__ __device__ inline int shared_dst(const LayoutDerived& L, int j, const int* sh, int n, int f) {
  const int lo = L.lo[j], hi = L.hi[j];
  if (L.scene_rope) {
    // the largest position among frames lo..hi-1: positions rise within a rope scene, so each rope scene that
    // overlaps [lo, hi) peaks at its last overlapping frame (frames past the rope scenes have none)
    int last = -1;
    for (int s = 0; s < L.n_rope; ++s) {
      const int a = L.rope_start[s], b = L.rope_start[s + 1];
      const int e = (hi < b ? hi : b) - 1;
      if (e < a || e < lo) continue;
      const int p = e - a + (a > 0 ? 1 : 0);
      if (p > last) last = p;
    }
    int c = 0;
    for (int i = 0; i < n; ++i) c += (sh[i] <= f);
    return last + c;
  }
  if (f < lo) {
    int nb = 0, c = 0;
    for (int i = 0; i < n; ++i) {
      nb += (sh[i] < lo);
      c += (sh[i] <= f);
    }
    return lo - nb + c - 1;
  }
  int c = 0;
  for (int i = 0; i < n; ++i) c += (sh[i] >= hi && sh[i] <= f);
  return hi + c - 1;
}

// ---------------------------------------------------------------------------------------------------------------
// RoPE of 8 consecutive bf16 (diffusers apply_rotary_emb, interleaved pairs (2i, 2i+1)), bit-identical to torch's
// (x.float() * cos + rot(x).float() * sin).to(bfloat16) with rot(x) = (-x_odd, x_even)
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

// (x0, x1) -> (x0*c0 - x1*s0, x1*c1 + x0*s1), each product and the sum rounded to fp32 separately
__device__ __forceinline__ void rot_pair(float x0, float x1, float c0, float c1, float s0, float s1, float& y0, float& y1) {
#pragma clang fp contract(off)
  float a = x0 * c0;
  float b = (-x1) * s0;
  float c = x1 * c1;
  float e = x0 * s1;
  y0 = a + b;
  y1 = c + e;
}

// two floats -> packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32 on gfx950)
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  f32x2_t f = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2_t));
}

// the table entries of 8 consecutive elements: cos and sin of one table row at one element offset
struct Tab8 {
  f32x4 c0, c1, s0, s1;
};

__device__ __forceinline__ Tab8 load_tab8(const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                          int64_t off) {
  return Tab8{*(const f32x4*)(cos_t + off), *(const f32x4*)(cos_t + off + 4), *(const f32x4*)(sin_t + off),
              *(const f32x4*)(sin_t + off + 4)};
}

// 8 bf16 in `v` rotated with the table entries t (sign +1) or its inverse (-1)
__device__ __forceinline__ u32x4 rotate8(u32x4 v, const Tab8& t, float sign) {
  float c[8] = {t.c0[0], t.c0[1], t.c0[2], t.c0[3], t.c1[0], t.c1[1], t.c1[2], t.c1[3]};
  float s[8] = {t.s0[0], t.s0[1], t.s0[2], t.s0[3], t.s1[0], t.s1[1], t.s1[2], t.s1[3]};
  u32x4 r;
#pragma unroll
  for (int p = 0; p < 4; ++p) {
    float x0 = bf2f((uint16_t)(v[p] & 0xffffu)), x1 = bf2f((uint16_t)(v[p] >> 16));
    float y0, y1;
    rot_pair(x0, x1, c[2 * p], c[2 * p + 1], sign * s[2 * p], sign * s[2 * p + 1], y0, y1);
    r[p] = pack2(y0, y1);
  }
  return r;
}

// 8 bf16 in `v` rotated with the table entries at element offset `off` of rows `row` (sign +1) or its inverse (-1)
__device__ __forceinline__ u32x4 rotate8(u32x4 v, const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                                int64_t off, float sign) {
  return rotate8(v, load_tab8(cos_t, sin_t, off), sign);
}

// Sum over the 64 lanes of a wavefront, the same in every lane: DPP adds within rows of 16 lanes (pairs, quads,
// halves, rows), then the row pairs and the two halves through v_permlane16_swap / v_permlane32_swap (no LDS round
// trips).
__device__ __forceinline__ float wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xf, 0xf, false));   // quad_perm 1032
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xf, 0xf, false));   // quad_perm 2301
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xf, 0xf, false));  // row_half_mirror
  v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xf, 0xf, false));  // row_mirror
  auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(p[0]) + __uint_as_float(p[1]);
  auto q = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(q[0]) + __uint_as_float(q[1]);
}

}  // namespace onereel
