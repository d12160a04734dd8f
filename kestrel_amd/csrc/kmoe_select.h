// kmoe_select.h — one token's expert selection by one wave (softmax, top-k,
// renormalisation; transformer.rs:479-495), shared by the decode router's tail
// and the decode gate/up kernel that selects its own experts.
#pragma once

#include "kmoe_device.h"

namespace kmoe {

// Wave-uniform reductions: DPP inside each 16-lane row, then the four row
// results read into scalars (no LDS round trips).
__device__ __forceinline__ uint32_t wave_umax_u(uint32_t v) {
  v = max(v, (uint32_t)dpp_i<kDppXor1>((int)v));
  v = max(v, (uint32_t)dpp_i<kDppXor2>((int)v));
  v = max(v, (uint32_t)dpp_i<kDppHalfMirror>((int)v));
  v = max(v, (uint32_t)dpp_i<kDppMirror>((int)v));
  const uint32_t a = __builtin_amdgcn_readlane((int)v, 0), b = __builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = __builtin_amdgcn_readlane((int)v, 32), d = __builtin_amdgcn_readlane((int)v, 48);
  return max(max(a, b), max(c, d));
}
__device__ __forceinline__ uint32_t wave_umin_u(uint32_t v) {
  v = min(v, (uint32_t)dpp_i<kDppXor1>((int)v));
  v = min(v, (uint32_t)dpp_i<kDppXor2>((int)v));
  v = min(v, (uint32_t)dpp_i<kDppHalfMirror>((int)v));
  v = min(v, (uint32_t)dpp_i<kDppMirror>((int)v));
  const uint32_t a = __builtin_amdgcn_readlane((int)v, 0), b = __builtin_amdgcn_readlane((int)v, 16);
  const uint32_t c = __builtin_amdgcn_readlane((int)v, 32), d = __builtin_amdgcn_readlane((int)v, 48);
  return min(min(a, b), min(c, d));
}
__device__ __forceinline__ float wave_fmax_u(float v) {
  v = fmaxf(v, dpp_f<kDppXor1>(v));
  v = fmaxf(v, dpp_f<kDppXor2>(v));
  v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  v = fmaxf(v, dpp_f<kDppMirror>(v));
  const int iv = __builtin_bit_cast(int, v);
  const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
  const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
  const float c = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
  const float d = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
  return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

// Rank key of a routing probability p >= +0 (its bits, monotone in p). A
// NaN p ranks as +0: the reference's sort comparator treats NaN as equal to
// everything and falls back to index order (transformer.rs:484), and its
// softmax makes every p of a row NaN once one logit is NaN or +inf, so such a
// row selects experts 0..k-1 in index order.
__device__ __forceinline__ uint32_t p_rank_key(float p) { return p != p ? 0u : __float_as_uint(p); }

// One token, one whole wave. lv[i] holds the logit of expert lane + 64*i
// (E <= 64*NPER; entries past E are ignored). p is this wave's LDS scratch of
// at least E floats. K <= 16. On return lane j < K holds selection j in
// sel_l (expert id) and w_l (weight), selection order:
//   p_e = exp(l_e - max) / (sum in expert order), correctly rounded exp;
//   K rounds of the largest p (compared by p_rank_key), ties to the lower
//   index; if norm_topk, w /= max(sum of the selected p in selection order,
//   2^-14); then w *= wscale unless wscale is 0 or 1.
// The selections stay one per lane (no register arrays indexed at run time,
// which the target can only address through its slow indexing mode).
template <int NPER>
__device__ __forceinline__ void wave_route_one(float (&lv)[NPER], int E, int K, int norm_topk, float wscale, float *p,
                                               uint32_t &sel_l, float &w_l) {
  const int lane = threadIdx.x & 63;
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < NPER; ++i)
    if (lane + 64 * i < E) m = fmaxf(m, lv[i]);
  m = wave_fmax_u(m);
#pragma unroll
  for (int i = 0; i < NPER; ++i) {
    const int e = lane + 64 * i;
    lv[i] = expf_cr(lv[i] - m);
    if (e < E) p[e] = lv[i];
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  float sum = -0.0f;  // in expert order
  if (lane == 0) {
    int e = 0;
    for (; e + 4 <= E; e += 4) {
      const float4 v = *(const float4 *)(p + e);
      sum = sum + v.x;
      sum = sum + v.y;
      sum = sum + v.z;
      sum = sum + v.w;
    }
    for (; e < E; ++e) sum = sum + p[e];
  }
  sum = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, sum)));
#pragma unroll
  for (int i = 0; i < NPER; ++i) lv[i] = lv[i] / sum;
  uint32_t taken = 0;
  sel_l = 0;
  w_l = 0.0f;
  for (int j = 0; j < K; ++j) {
    uint32_t best = 0;
    int bi = NPER;
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const int e = lane + 64 * i;
      const uint32_t u = p_rank_key(lv[i]);
      if (e < E && !((taken >> i) & 1u) && (bi == NPER || u > best)) {
        best = u;
        bi = i;
      }
    }
    const uint32_t mx = wave_umax_u(bi == NPER ? 0u : best);
    const bool has = bi != NPER && best == mx;
    const uint32_t es = wave_umin_u(has ? (uint32_t)(64 * bi + lane) : 0xffffffffu);
    const int ib = (int)(es >> 6), lw = (int)(es & 63);
    if (lane == lw) taken |= 1u << ib;
    float mine = lv[0];
#pragma unroll
    for (int i = 1; i < NPER; ++i) mine = i == ib ? lv[i] : mine;
    const float wj = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine), lw));
    sel_l = lane == j ? es : sel_l;
    w_l = lane == j ? wj : w_l;
  }
  if (norm_topk) {
    float ss = -0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const float v = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w_l), j));
      const float t = ss + v;
      ss = j < K ? t : ss;
    }
    ss = fmaxf(ss, 6.103515625e-05f);
    w_l = w_l / ss;
  }
  if (wscale != 0.0f && wscale != 1.0f) w_l = w_l * wscale;
}

// Slot of the lane's selection (lanes j < K; all ids distinct): the number of
// selections with a smaller expert id, slots in ascending expert id.
__device__ __forceinline__ uint32_t selection_rank(uint32_t sel_l, int K) {
  uint32_t r = 0;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)sel_l, j);
    r += (j < K && v < sel_l) ? 1u : 0u;
  }
  return r;
}

// The expert in slot `slot` (the selection whose rank is slot), or -1 when
// slot >= K; uniform across the wave.
__device__ __forceinline__ int selection_in_slot(uint32_t sel_l, uint32_t rk_l, int K, int slot) {
  const int lane = threadIdx.x & 63;
  const uint64_t m = __ballot(lane < K && rk_l == (uint32_t)slot);
  return m ? __builtin_amdgcn_readlane((int)sel_l, (int)__builtin_ctzll(m)) : -1;
}

// The routing of one token from its selection, written by one wave: idx and
// weights in selection order, perm / inv between selection entry and slot,
// the active experts by slot, their count and the per-expert slot offsets
// [E + 1] (the dispatch of transformer.rs:525-531 for one token).
__device__ __forceinline__ void publish_selection(uint32_t sel_l, float w_l, uint32_t rk_l, int K, int E, int lane,
                                                  uint32_t *idx, float *wsel, uint32_t *perm, uint32_t *inv,
                                                  int32_t *active, int32_t *n_active, uint32_t *offsets) {
  if (lane < K) {
    idx[lane] = sel_l;
    wsel[lane] = w_l;
    perm[rk_l] = (uint32_t)lane;
    inv[lane] = rk_l;
    active[rk_l] = (int32_t)sel_l;
  }
  if (lane == 0) *n_active = K;
  for (int ee = lane; ee <= E; ee += 64) {
    uint32_t c = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const uint32_t v = (uint32_t)__builtin_amdgcn_readlane((int)sel_l, j);
      c += (j < K && v < (uint32_t)ee) ? 1u : 0u;
    }
    offsets[ee] = c;
  }
}

}  // namespace kmoe
