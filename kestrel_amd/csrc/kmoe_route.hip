// kmoe_route.hip — router logits, softmax/top-k, dispatch, slot quantization
// and the combine of Transformer::moe_ffn (transformer.rs:472-570).
//
// Router logits must be bit-identical to the reference's for the routing
// indices to be, so each logit is summed in the exact order quant::matmul
// (quant.rs:229) uses for an F32 [E, d] router at this s_rows:
//   s_rows < 4 (or d % 8 != 0): quant::dot (quant.rs:208-224): eight chains
//     acc_l += w*x (multiply, then add) over elements 8c+l, summed
//     acc_0..acc_7 in order, then the tail.
//   s_rows >= 4: gemm_f32 over 48-row tiles (quant.rs:243-257). In each tile
//     the first rows/3*3 rows of each group of 4 activation rows use the
//     3x4 register kernel (avx2.rs:238-273): eight FMA chains over 8c+l and
//     hsum; the other rows and the last s_rows % 4 activation rows use
//     dot_f32 (avx2.rs:289-308): two interleaved sets of eight FMA chains,
//     added lane-wise, hsum, then the tail.
// hsum (avx2.rs:20-27) = ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7)).
// One lane per chain (16 lanes per logit); lane 0 of the 16 combines them.
// Each chain reads its elements from LDS in the same order it would from
// global memory (k_router_logits below).
#include "kmoe_device.h"
#include "kmoe_launch.h"
#include "kmoe_logit.h"
#include "kmoe_select.h"

namespace kmoe {

namespace {

enum { ORD_GEMM = 0, ORD_DOTF32 = 1, ORD_QDOT = 2 };

__device__ __forceinline__ float hsum8(const float *v) {
  const float a = v[0] + v[4], b = v[2] + v[6], c = v[1] + v[5], d = v[3] + v[7];
  return (a + b) + (c + d);
}

// Work-group = TE weight rows and TT activation rows: 16 lanes per (row,
// token) logit as above, TE * TT <= 16 logits. Columns are staged through LDS
// CH at a time (a multiple of 16, so every element stays in its chain and
// every chain keeps its order); the chains read LDS, the tails past the last
// whole group of 8 (or 16) read global memory. Decode batches (S <= 8) take
// one row and two tokens (many small work-groups); larger batches take 4 x 4
// tiles, so a row is staged once per 4 tokens and a token once per 4 rows.
// Work-groups from nlog on quantize the activation rows for the int8 path
// instead (qkind 1: Q8_K, one wave per 256-block; 2: Q8, eight lanes per
// 32-block), with k_quant_q8k's / k_quant_q8's arithmetic.
template <int TE, int TT, int CH>
__global__ void __launch_bounds__(256) k_router_logits(const float *__restrict__ W, int32_t E, int64_t d,
                                                       const float *__restrict__ X, int64_t S,
                                                       float *__restrict__ logits, int qdot, int32_t nlog, int qkind,
                                                       int8_t *__restrict__ xq, float *__restrict__ xd,
                                                       int32_t *__restrict__ xs) {
  __shared__ __attribute__((aligned(16))) float Wc[TE][CH];
  __shared__ __attribute__((aligned(16))) float Xc[TT][CH];
  if ((int32_t)blockIdx.x >= nlog) {  // no block barriers on this path
    const int lane = threadIdx.x & 63;
    const int64_t u = (int64_t)(blockIdx.x - nlog) * 4 + (threadIdx.x >> 6);
    if (qkind == 1) {
      if (u < S * (d / 256)) wave_quant_q8k_block(X + u * 256, xq + u * 256, xd + u, xs + u * 16, lane);
    } else {
      const int64_t blk = u * 8 + (lane >> 3);
      if (blk < S * (d / 32)) group8_quant_q8_block(X + blk * 32, xq + blk * 32, xd + blk, xs + blk * 2, lane & 7);
    }
    return;
  }
  const bool vec = d % 4 == 0 && (((uintptr_t)W | (uintptr_t)X) & 15) == 0;
  const int tid = threadIdx.x;
  const int l16 = tid & 15, pair = tid >> 4;
  const int ee = pair / TT, tt = pair % TT;
  const int ntile_e = (E + TE - 1) / TE;
  const int e0 = (int)(blockIdx.x % (uint32_t)ntile_e) * TE;  // blocks: (token tile, row tile) pairs
  const int64_t s0 = (int64_t)(blockIdx.x / (uint32_t)ntile_e) * TT;
  const int ne = E - e0 < TE ? E - e0 : TE;
  const int ns = (int)(S - s0 < TT ? S - s0 : TT);
  const bool valid = ee < ne && tt < ns;
  const int e = e0 + (valid ? ee : 0);
  const int64_t s = s0 + (valid ? tt : 0);
  int ord;
  if (qdot || S < 4 || (d % 8) != 0) {
    ord = ORD_QDOT;
  } else {
    const int64_t s4 = S / 4 * 4;
    const int r0 = e / 48 * 48;
    const int trows = (E - r0 < 48 ? E - r0 : 48);
    const int rows3 = trows / 3 * 3;
    ord = (s < s4 && (e - r0) < rows3) ? ORD_GEMM : ORD_DOTF32;
  }
  const float *w = W + (int64_t)e * d;
  const float *x = X + s * d;
  const int64_t n8 = d / 8, n16 = d / 16;
  const int l = l16 & 7;
  const int off = l16 < 8 ? 0 : 8;
  float acc = 0.0f;
  for (int64_t c0 = 0; c0 < d; c0 += CH) {
    const int cw = (int)(d - c0 < CH ? d - c0 : CH);
    __syncthreads();  // the previous chunk has been read
    if (vec) {  // every 16-byte load of the chunk issued before any is stored
      constexpr int Q = CH / 4 / 256;
      float4 rv[TE + TT][Q];
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const int i = 4 * (q * 256 + tid);
#pragma unroll
        for (int r = 0; r < TE; ++r)
          rv[r][q] = i < cw && r < ne ? *(const float4 *)(W + (int64_t)(e0 + r) * d + c0 + i)
                                      : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int t = 0; t < TT; ++t)
          rv[TE + t][q] = i < cw && t < ns ? *(const float4 *)(X + (s0 + t) * d + c0 + i)
                                           : make_float4(0.f, 0.f, 0.f, 0.f);
      }
#pragma unroll
      for (int q = 0; q < Q; ++q) {
        const int i = 4 * (q * 256 + tid);
        if (i < cw) {
#pragma unroll
          for (int r = 0; r < TE; ++r) *(float4 *)&Wc[r][i] = rv[r][q];
#pragma unroll
          for (int t = 0; t < TT; ++t) *(float4 *)&Xc[t][i] = rv[TE + t][q];
        }
      }
    } else {
      for (int r = 0; r < ne; ++r)
        for (int i = tid; i < cw; i += 256) Wc[r][i] = W[(int64_t)(e0 + r) * d + c0 + i];
      for (int t = 0; t < ns; ++t)
        for (int i = tid; i < cw; i += 256) Xc[t][i] = X[(s0 + t) * d + c0 + i];
    }
    __syncthreads();
    if (!valid) continue;
    const float *wr = Wc[ee], *xr = Xc[tt];
    if (ord == ORD_GEMM || ord == ORD_QDOT) {
      if (l16 < 8) {
        const int64_t cb = c0 / 8, ce = (c0 + cw) / 8 < n8 ? (c0 + cw) / 8 : n8;
        if (ord == ORD_GEMM) {
#pragma unroll 8
          for (int64_t c = cb; c < ce; ++c) {
            const int o = (int)(8 * c - c0) + l16;
            acc = fmaf(wr[o], xr[o], acc);
          }
        } else {
#pragma unroll 8
          for (int64_t c = cb; c < ce; ++c) {
            const int o = (int)(8 * c - c0) + l16;
            const float p = wr[o] * xr[o];
            acc = acc + p;
          }
        }
      }
    } else {
      const int64_t cb = c0 / 16, ce = (c0 + cw) / 16 < n16 ? (c0 + cw) / 16 : n16;
#pragma unroll 8
      for (int64_t c = cb; c < ce; ++c) {
        const int o = (int)(16 * c - c0) + off + l;
        acc = fmaf(wr[o], xr[o], acc);
      }
    }
  }
  if (valid && ord == ORD_DOTF32 && l16 < 8 && (d - 16 * n16) >= 8) acc = fmaf(w[16 * n16 + l], x[16 * n16 + l], acc);
  // Gather the 16 chains of this logit in lane 0 of the group.
  float v[16];
  const int base = threadIdx.x & 63 & ~15;
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = __shfl(acc, base + i);
  if (!valid || l16 != 0) return;
  float r;
  if (ord == ORD_GEMM) {
    r = hsum8(v);
  } else if (ord == ORD_DOTF32) {
    float u[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) u[i] = v[i] + v[i + 8];
    r = hsum8(u);
    for (int64_t c = d / 8 * 8; c < d; ++c) {
      const float p = w[c] * x[c];
      r = r + p;
    }
  } else {
    r = -0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) r = r + v[i];
    for (int64_t c = n8 * 8; c < d; ++c) {
      const float p = w[c] * x[c];
      r = r + p;
    }
  }
  logits[s * E + e] = r;
}

// One wave per token: softmax, top-k, renormalisation (transformer.rs:479-495).
constexpr int kMaxExperts = 512;

// The same for E <= 64*NPER experts through the single-token selection of the
// decode kernels (wave_route_one: the logits in lane registers, the sum in
// expert order, the k rounds as wave reductions without block barriers): one
// wave per token, four tokens per work-group, the same bits as the kernel
// below.
template <int NPER>
__global__ void __launch_bounds__(256) k_route_topk_w(const float *__restrict__ logits, int64_t S, int32_t E,
                                                      int32_t k, int32_t norm_topk, float weights_scale,
                                                      uint32_t *__restrict__ idx, float *__restrict__ wout) {
  __shared__ __attribute__((aligned(16))) float P[4][64 * NPER];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t s = (int64_t)blockIdx.x * 4 + wave;
  if (s >= S) return;  // no block barriers below
  const float *row = logits + s * E;
  float lv[NPER];
#pragma unroll
  for (int i = 0; i < NPER; ++i) lv[i] = lane + 64 * i < E ? row[lane + 64 * i] : -INFINITY;
  uint32_t sel_l;
  float w_l;
  wave_route_one<NPER>(lv, E, k, norm_topk, weights_scale, P[wave], sel_l, w_l);
  if (lane < k) {
    idx[s * k + lane] = sel_l;
    wout[s * k + lane] = w_l;
  }
}

__global__ void __launch_bounds__(256) k_route_topk(const float *__restrict__ logits, int64_t S, int32_t E, int32_t k,
                                                    int32_t norm_topk, float weights_scale, uint32_t *__restrict__ idx,
                                                    float *__restrict__ wout) {
  __shared__ float P[4][kMaxExperts];
  __shared__ int taken[4][kMaxExperts];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t s = (int64_t)blockIdx.x * 4 + wave;
  const bool valid = s < S;  // no early return: the block barriers below stay uniform
  const float *row = logits + (valid ? s : 0) * E;
  float m = -INFINITY;
  for (int e = lane; e < E; e += 64) m = fmaxf(m, row[e]);
  m = group_max<64>(m);
  for (int e = lane; e < E; e += 64) {
    P[wave][e] = expf_cr(row[e] - m);
    taken[wave][e] = 0;
  }
  __syncthreads();
  float sum = 0.0f;
  if (lane == 0) {
    sum = -0.0f;
    for (int e = 0; e < E; ++e) sum = sum + P[wave][e];
  }
  sum = __shfl(sum, 0);
  for (int e = lane; e < E; e += 64) P[wave][e] = P[wave][e] / sum;
  __syncthreads();
  float wsel[16];
  uint32_t isel[16];
  for (int j = 0; j < k; ++j) {
    // Largest p, ties to the lower index: key = (p_rank_key(p) << 32) | ~index.
    uint64_t best = 0;
    for (int e = lane; e < E; e += 64) {
      if (taken[wave][e]) continue;
      const uint64_t key = ((uint64_t)p_rank_key(P[wave][e]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
      best = key > best ? key : best;
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const uint32_t hi = __shfl_xor((unsigned)(best >> 32), off), lo = __shfl_xor((unsigned)best, off);
      const uint64_t o = ((uint64_t)hi << 32) | lo;
      best = o > best ? o : best;
    }
    const uint32_t e = 0xffffffffu - (uint32_t)best;
    if (lane == 0) taken[wave][e] = 1;
    isel[j] = e;
    wsel[j] = P[wave][e];
    __syncthreads();
  }
  if (lane != 0 || !valid) return;
  if (norm_topk) {
    float ss = -0.0f;
    for (int j = 0; j < k; ++j) ss = ss + wsel[j];
    ss = fmaxf(ss, 6.103515625e-05f);
    for (int j = 0; j < k; ++j) wsel[j] = wsel[j] / ss;
  }
  if (weights_scale != 0.0f && weights_scale != 1.0f)
    for (int j = 0; j < k; ++j) wsel[j] = wsel[j] * weights_scale;
  for (int j = 0; j < k; ++j) {
    idx[s * k + j] = isel[j];
    wout[s * k + j] = wsel[j];
  }
}

// Stable counting sort of n flat (token, slot) entries by expert id, in one
// work-group of 1024 threads: every entry's rank among its expert's entries
// in flat order, the order BTreeMap<expert, Vec<(token, w)>> fills in. Each
// of the 16 waves owns a contiguous range of entries and walks it twice in
// steps of 64. In a step the lanes that share an expert are found with
// log2(E) ballots and ranked by popcount; pass 1 counts each wave's entries
// per expert, a prefix over the waves (in order) and over the experts gives
// each (wave, expert) its first position, and pass 2 places the entries.
// With up to 64*kDispRegs entries per wave the ids are loaded into registers
// once, all loads in flight together.
constexpr int kDispRegs = 32;
__global__ void __launch_bounds__(1024) k_dispatch(const uint32_t *__restrict__ idx, int64_t n, int32_t E,
                                                   uint32_t *__restrict__ perm, uint32_t *__restrict__ offsets,
                                                   uint32_t *__restrict__ inv, int32_t *__restrict__ n_active,
                                                   int32_t *__restrict__ active) {
  __shared__ uint32_t cnt[16][kMaxExperts];
  __shared__ uint32_t base[kMaxExperts];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  for (int w = 0; w < 16; ++w)
    for (int e = tid; e < E; e += 1024) cnt[w][e] = 0;
  __syncthreads();
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  const int64_t per = ((n + 15) / 16 + 63) / 64 * 64;
  const int64_t b0 = (int64_t)wave * per, b1 = b0 + per < n ? b0 + per : n;
  const bool in_regs = per <= 64 * kDispRegs;
  uint32_t ids[kDispRegs];
  if (in_regs) {
#pragma unroll
    for (int k = 0; k < kDispRegs; ++k) {
      const int64_t i = b0 + 64 * k + lane;
      ids[k] = i < b1 ? idx[i] : 0u;
    }
  }
  // the id of entry i = b0 + 64k + lane
  auto id_at = [&](int k, int64_t i) -> uint32_t {
    if (in_regs) {
      uint32_t v = 0;
#pragma unroll
      for (int kk = 0; kk < kDispRegs; ++kk) v = kk == k ? ids[kk] : v;
      return v;
    }
    return i < b1 ? idx[i] : 0u;
  };
  // lanes of this step sharing the lane's expert (ids >= E are dropped, never indexed)
  auto step = [&](int k, int64_t i, uint32_t &e, bool &valid, uint64_t &same) {
    const uint32_t ev = id_at(k, i);
    valid = i < b1 && ev < (uint32_t)E;
    e = valid ? ev : 0u;
    same = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1u;
      const uint64_t m = __ballot(valid && bit);
      same &= bit ? m : ~m;
    }
  };
  for (int64_t i0 = b0; i0 < b1; i0 += 64) {  // pass 1: this wave's count per expert
    uint32_t e;
    bool valid;
    uint64_t same;
    step((int)((i0 - b0) >> 6), i0 + lane, e, valid, same);
    if (valid && (same & lt) == 0) cnt[wave][e] += (uint32_t)__popcll(same);
  }
  __syncthreads();
  for (int ee = tid; ee < E; ee += 1024) {  // wave w's first rank per expert; expert totals
    uint32_t run = 0;
    for (int w = 0; w < 16; ++w) {
      const uint32_t c = cnt[w][ee];
      cnt[w][ee] = run;
      run += c;
    }
    base[ee] = run;
  }
  __syncthreads();
  if (wave == 0) {  // exclusive prefix over the experts; the active ones in ascending order
    constexpr int PER = kMaxExperts / 64;  // experts per lane
    uint32_t tot[PER], sum = 0, nz = 0;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int ee = PER * lane + k;
      tot[k] = ee < E ? base[ee] : 0u;
      sum += tot[k];
      nz += tot[k] > 0 ? 1u : 0u;
    }
    uint32_t isum = sum, inz = nz;  // inclusive scans over the lanes
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const uint32_t a = __shfl_up(isum, o), b = __shfl_up(inz, o);
      if (lane >= o) {
        isum += a;
        inz += b;
      }
    }
    uint32_t run = isum - sum, na = inz - nz;
#pragma unroll
    for (int k = 0; k < PER; ++k) {
      const int ee = PER * lane + k;
      if (ee < E) {
        offsets[ee] = run;
        base[ee] = run;
        if (tot[k] > 0 && active) active[na++] = ee;
        run += tot[k];
      }
    }
    if (lane == 63) {
      offsets[E] = isum;
      if (n_active) *n_active = (int32_t)inz;
    }
  }
  __syncthreads();
  for (int64_t i0 = b0; i0 < b1; i0 += 64) {  // pass 2: positions in flat order
    const int64_t i = i0 + lane;
    uint32_t e;
    bool valid;
    uint64_t same;
    step((int)((i0 - b0) >> 6), i, e, valid, same);
    const uint32_t wrank = (uint32_t)__popcll(same & lt);
    const uint32_t before = valid ? cnt[wave][e] : 0u;  // read by every lane before the leader adds
    __builtin_amdgcn_wave_barrier();
    if (valid) {
      const uint32_t p = base[e] + before + wrank;
      perm[p] = (uint32_t)i;
      if (inv) inv[i] = p;
      if (wrank == 0) cnt[wave][e] = before + (uint32_t)__popcll(same);
    }
    __builtin_amdgcn_wave_barrier();
  }
}

__device__ __forceinline__ bool slot_is_int(const Routing &rt, const uint32_t *idx_flat, int64_t p, int regime) {
  if (regime == REGIME_INT8) return true;
  if (regime == REGIME_EXACT) return false;
  const uint32_t e = idx_flat[rt.perm[p]];
  return rt.offsets[e + 1] - rt.offsets[e] < 4;
}

__global__ void __launch_bounds__(256) k_quant_slots_q8k(const float *__restrict__ h, int64_t n_slots, int64_t cols,
                                                         Routing rt, const uint32_t *__restrict__ idx_flat, int regime,
                                                         int8_t *__restrict__ q, float *__restrict__ d,
                                                         int32_t *__restrict__ bs) {
  const int lane = threadIdx.x & 63;
  const int64_t nb = cols / 256;
  const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= n_slots * nb) return;
  const int64_t p = blk / nb;
  if (!slot_is_int(rt, idx_flat, p, regime)) return;
  wave_quant_q8k_block(h + blk * 256, q + blk * 256, d + blk, bs + blk * 16, lane);
}

__global__ void __launch_bounds__(256) k_quant_slots_q8(const float *__restrict__ h, int64_t n_slots, int64_t cols,
                                                        Routing rt, const uint32_t *__restrict__ idx_flat, int regime,
                                                        int8_t *__restrict__ q, float *__restrict__ d,
                                                        int32_t *__restrict__ s16) {
  const int lane = threadIdx.x & 63;
  const int64_t nb = cols / 32;
  const int64_t blk = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
  if (blk >= n_slots * nb) return;
  const int64_t p = blk / nb;
  if (!slot_is_int(rt, idx_flat, p, regime)) return;
  group8_quant_q8_block(h + blk * 32, q + blk * 32, d + blk, s16 + blk * 2, lane & 7);
}

// The token's slots in ascending slot position (== ascending expert id) and
// their weights; every thread of the work-group computes the same.
__device__ __forceinline__ int token_slots(const Routing &rt, int64_t s, uint32_t (&p)[16], float (&w)[16]) {
  const int k = rt.topk;
  for (int j = 0; j < k; ++j) {
    p[j] = rt.inv[s * k + j];
    w[j] = rt.wsel[s * k + j];
  }
  for (int j = 1; j < k; ++j) {
    const uint32_t pj = p[j];
    const float wj = w[j];
    int i = j - 1;
    while (i >= 0 && p[i] > pj) {
      p[i + 1] = p[i];
      w[i + 1] = w[i];
      --i;
    }
    p[i + 1] = pj;
    w[i + 1] = wj;
  }
  return k;
}

// k_combine on 16-byte groups: one token per blockIdx.y, columns 4c..4c+3
// per thread, one wave per work-group (d % 4 == 0, y and out 16-byte
// aligned). Same arithmetic.
__global__ void __launch_bounds__(64) k_combine4(const float *__restrict__ y, Routing rt, int64_t s0, int64_t d,
                                                 float *__restrict__ out) {
  const int64_t s = s0 + blockIdx.y;
  uint32_t p[16];
  float w[16];
  const int k = token_slots(rt, s, p, w);
  const int64_t d4 = d / 4;
  for (int64_t c = (int64_t)blockIdx.x * 64 + threadIdx.x; c < d4; c += (int64_t)gridDim.x * 64) {
    float4 o = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int j = 0; j < k; ++j) {
      const float4 v = ((const float4 *)(y + (int64_t)p[j] * d))[c];
      float4 t;
      t.x = w[j] * v.x;
      t.y = w[j] * v.y;
      t.z = w[j] * v.z;
      t.w = w[j] * v.w;
      o.x = o.x + t.x;
      o.y = o.y + t.y;
      o.z = o.z + t.z;
      o.w = o.w + t.w;
    }
    ((float4 *)(out + s * d))[c] = o;
  }
}

// out[s, c] = sum over the token's slots in ascending expert id of w * y[slot, c]
// (multiply, then add; transformer.rs:566-570).
__global__ void __launch_bounds__(256) k_combine(const float *__restrict__ y, Routing rt, int64_t S, int64_t s0,
                                                 int64_t d, float *__restrict__ out) {
  const int64_t s = s0 + blockIdx.y;
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s >= S || c >= d) return;
  uint32_t p[16];
  float w[16];
  const int k = token_slots(rt, s, p, w);
  float o = 0.0f;
  for (int j = 0; j < k; ++j) {
    const float t = w[j] * y[(int64_t)p[j] * d + c];
    o = o + t;
  }
  out[s * d + c] = o;
}

// ---------------------------------------------------------------------------
// Decode routing in one work-group (s_rows < 4): logits in quant::dot order,
// softmax, top-k, renormalisation, dispatch, and the int8 quantization of the
// activation rows, fused.
//
// With s_rows < 4 the reference computes each F32 router logit with
// quant::dot (quant.rs:208-224): eight chains acc_l = sum of p_{8c+l} in
// order of c, where each product p = w*x is rounded on its own (no FMA). The
// products do not depend on the chains, so all 1024 threads form them with
// coalesced float4 loads and write them to LDS transposed per chain; each
// chain then reads its products four at a time. The chain additions stay in
// the reference's order, so the logits are bit-identical.
struct RouteDecArgs {
  const float *W;
  int32_t E;
  int64_t d;
  const float *X;
  int32_t S, k, norm_topk;
  float weights_scale;
  float *logits;  // [S, E]
  uint32_t *idx;
  float *wsel;
  uint32_t *perm, *offsets, *inv;
  int32_t *n_active, *active;
  int qtype;  // 0: none, T_Q4_K or T_Q6_K: Q8_K rows, T_Q8_0: Q8 rows
  int8_t *xq;
  float *xd;
  int32_t *xs;
  uint32_t *done;  // finished work-groups; 0 between calls (the last one resets it)
  int vec;         // W, X 16-byte aligned and d % 4 == 0
  RouteNorm norm;  // norm.w non-null: X = rmsnorm(norm.x (+= norm.y)) is computed here
};

// One token's FFN norm in front of the router (RouteNorm): every work-group
// forms x + y and the normed row in registers (wg_residual_rmsnorm: the bits
// of k_rmsnorm_regs); work-group 0 also stores the normed row and its int8
// rows (qtype) for the gate/up kernel, and the last work-group to count
// itself on n.done stores x + y back into x.
template <int NV>
__device__ __forceinline__ void route_norm_row(const RouteDecArgs &a, float4 (&h)[NV], bool store, float *red,
                                               int *xlast) {
  const int t = threadIdx.x;
  const int n4 = (int)(a.d / 4);
  const RouteNorm &n = a.norm;
  wg_residual_rmsnorm<NV>(n.x, n.y, n.w, a.d, n.eps, n.done, h, red, xlast);
  if (!store) return;
  float4 *frow = (float4 *)n.f;
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = t + 256 * k;
    if (i < n4) {
      frow[i] = h[k];
      if (is_kquant(a.qtype)) {
        const int64_t b = 4 * k + (t >> 6);
        wave_quant_q8k_vals(h[k], a.xq + 256 * b, a.xd + b, a.xs + 16 * b, t & 63);
      } else if (a.qtype == T_Q8_0) {
        const int64_t b = (4 * (int64_t)i) / 32;
        group8_quant_q8_vals(h[k], a.xq + 32 * b, a.xd + b, a.xs + 2 * b, t & 7);
      }
    }
  }
}


// Softmax, top-k and renormalisation (transformer.rs:479-495) for the S <= 3
// tokens whose logits the work-groups wrote, then the dispatch (the stable
// sort of the S*k flat slots by expert). Run by the last work-group to finish.
// Expert lane + 64*i is held by lane `lane`, i < NPER (E <= 64*NPER).
template <int NPER>
__device__ void route_dec_tail(const RouteDecArgs &a, float *P, uint32_t *sel, int *first) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int E = a.E, K = a.k, n = a.S * a.k;
  if (wave < a.S) {
    const int s = wave;
    float lv[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) {
      const int e = lane + 64 * i;
      // written by other work-groups of this launch: read past this CU's L1
      lv[i] = e < E ? __hip_atomic_load(a.logits + s * E + e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : -INFINITY;
    }
    uint32_t sl;
    float wl;
    wave_route_one<NPER>(lv, E, K, a.norm_topk, a.weights_scale, P + s * kMaxExperts, sl, wl);
    if (lane < K) {
      sel[s * K + lane] = sl;
      a.idx[s * K + lane] = sl;
      a.wsel[s * K + lane] = wl;
    }
  }
  __syncthreads();
  // dispatch of n <= 48 slots: position = #slots of lower experts + #earlier slots of the same expert
  uint32_t ej = 0;
  if (tid < n) {
    ej = sel[tid];
    uint32_t lt = 0, eq = 0;
    for (int i = 0; i < n; ++i) {
      const uint32_t ei = sel[i];
      lt += ei < ej ? 1u : 0u;
      eq += (i < tid && ei == ej) ? 1u : 0u;
    }
    const uint32_t pos = lt + eq;
    a.perm[pos] = (uint32_t)tid;
    a.inv[tid] = pos;
    first[tid] = eq == 0;
  }
  for (int e = tid; e <= E; e += blockDim.x) {
    uint32_t c = 0;
    for (int i = 0; i < n; ++i) c += sel[i] < (uint32_t)e ? 1u : 0u;
    a.offsets[e] = c;
  }
  __syncthreads();
  if (tid < n && first[tid]) {
    int rank = 0;
    for (int i = 0; i < n; ++i) rank += (first[i] && sel[i] < ej) ? 1 : 0;
    a.active[rank] = (int32_t)ej;
  }
  if (tid == 0) {
    int na = 0;
    for (int i = 0; i < n; ++i) na += first[i];
    *a.n_active = na;
  }
}

// Decode routing (S <= 3 tokens), one work-group per expert e:
//   logits[s][e] in quant::dot order (quant.rs:208-224): eight chains
//   acc_l = sum over c of p_{8c+l} in order, each p = w*x rounded on its own,
//   then -0.0 + acc_0 + ... + acc_7 and the d % 8 tail columns in order.
// The products of a token go to LDS chain-major; lanes 0..7 of wave 0 fold
// the chains with their LDS reads two stages ahead, while waves 1..3 quantize
// this work-group's share of the activation rows for the int path. The last
// work-group to finish (counter a.done) runs the softmax / top-k / dispatch
// tail; nothing waits on another work-group.
template <int NV>
__global__ void __launch_bounds__(256) k_route_dec(RouteDecArgs a) {
  __shared__ __attribute__((aligned(16))) float T[kLogitLds];
  __shared__ float P[3 * kMaxExperts];
  __shared__ uint32_t sel[64];
  __shared__ int first[64];
  __shared__ int last;
  __shared__ float red[4];
  __shared__ int xlast;
  const int tid = threadIdx.x, lane = tid & 63;
  const int e = blockIdx.x, G = gridDim.x;
  const int64_t d = a.d;
  const int nq = (int)(2 * (d / 8));  // float4 groups in the first 8*(d/8) columns
  const float *w = a.W + (int64_t)e * d;

  float4 wv[NV];
  logit_row_load<NV>(w, nq, a.vec, wv, tid);
  if (a.norm.w) {  // one token, d % 256 == 0: the normed row from registers
    float4 xr[NV];
    route_norm_row<NV>(a, xr, e == 0, red, &xlast);
    const float r = wg_logit_at<NV>(wv, w, [&](int v, int) { return xr[v]; }, a.norm.f, d, T, [](int) {});
    if (tid == 0) {
      if (a.done) st_agent(a.logits + e, r);  // read by the last work-group below
      else a.logits[e] = r;
    }
  }
  for (int s = 0; s < (a.norm.w ? 0 : a.S); ++s) {
    const float *x = a.X + (int64_t)s * d;
    __syncthreads();  // the previous token's fold has read T
    const float r = wg_logit<NV>(wv, w, x, d, a.vec, T, [&](int wv_) {
      if (s != 0) return;
      // int8 activation rows: this work-group's blocks, one wave (Q8_K) or
      // eight lanes (Q8) per block
      const int wid = e * 3 + (wv_ - 1), nw = 3 * G;
      if (is_kquant(a.qtype)) {
        const int64_t nb = (int64_t)a.S * (d / 256);
        for (int64_t b = wid; b < nb; b += nw)
          wave_quant_q8k_block(a.X + b * 256, a.xq + b * 256, a.xd + b, a.xs + b * 16, lane);
      } else if (a.qtype == T_Q8_0) {
        const int64_t nb = (int64_t)a.S * (d / 32);
        for (int64_t b = (int64_t)wid * 8 + (lane >> 3); b < nb; b += (int64_t)nw * 8)
          group8_quant_q8_block(a.X + b * 32, a.xq + b * 32, a.xd + b, a.xs + b * 2, lane & 7);
      }
    });
    if (tid == 0) {
      if (a.done) st_agent(a.logits + (int64_t)s * a.E + e, r);  // read by the last work-group below
      else a.logits[(int64_t)s * a.E + e] = r;
    }
  }
  if (!a.done) return;  // logits only: the selection happens in the next kernel
  __syncthreads();
  if (tid == 0) {
    // The logits went out with agent-scope stores, waited for here; the
    // release add orders them before the counter, and the work-group that
    // completes it acquires before its tail reads them (with agent-scope
    // loads). The int8 rows are read by later kernels only.
    vm_wait();
    last = add_release(a.done, 1u) == (uint32_t)(G - 1);
    if (last) acquire_agent();
  }
  __syncthreads();
  if (!last) return;
  if (a.E <= 64) route_dec_tail<1>(a, P, sel, first);
  else if (a.E <= 128) route_dec_tail<2>(a, P, sel, first);
  else if (a.E <= 256) route_dec_tail<4>(a, P, sel, first);
  else route_dec_tail<8>(a, P, sel, first);
  if (tid == 0) __hip_atomic_store(a.done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

hipError_t launch_router_logits(hipStream_t st, const float *router, int32_t n_expert, int64_t d, const float *x,
                                int64_t s_rows, float *logits, bool qdot, int qkind, int8_t *xq, float *xd,
                                int32_t *xs) {
  if (s_rows * n_expert == 0) return hipSuccess;
  int64_t qblocks = 0;  // work-groups of 4 waves for the int8 rows of x
  if (qkind == 1) qblocks = (s_rows * (d / 256) + 3) / 4;
  else if (qkind == 2) qblocks = ((s_rows * (d / 32) + 7) / 8 + 3) / 4;
  if (s_rows <= 8) {
    const int64_t blocks = (s_rows + 1) / 2 * n_expert;
    if (blocks + qblocks > (int64_t)INT32_MAX) return hipErrorInvalidValue;
    KMOE_LAUNCH((k_router_logits<1, 2, 4096>), dim3((unsigned)(blocks + qblocks)), dim3(256), 0, st, router,
                n_expert, d, x, s_rows, logits, qdot ? 1 : 0, (int32_t)blocks, qkind, xq, xd, xs);
    return hipGetLastError();
  }
  const int64_t blocks = (s_rows + 3) / 4 * ((n_expert + 3) / 4);
  if (blocks + qblocks > (int64_t)INT32_MAX) return hipErrorInvalidValue;
  KMOE_LAUNCH((k_router_logits<4, 4, 1024>), dim3((unsigned)(blocks + qblocks)), dim3(256), 0, st, router, n_expert,
              d, x, s_rows, logits, qdot ? 1 : 0, (int32_t)blocks, qkind, xq, xd, xs);
  return hipGetLastError();
}

hipError_t launch_route_topk(hipStream_t st, const float *logits, int64_t s_rows, int32_t n_expert, int32_t k,
                             int32_t norm_topk, float weights_scale, uint32_t *idx, float *w) {
  if (s_rows == 0) return hipSuccess;
  if (n_expert > kMaxExperts || k > 16 || k > n_expert || k <= 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((s_rows + 3) / 4));
  if (n_expert <= 64)
    KMOE_LAUNCH(k_route_topk_w<1>, grid, dim3(256), 0, st, logits, s_rows, n_expert, k, norm_topk, weights_scale,
                idx, w);
  else if (n_expert <= 128)
    KMOE_LAUNCH(k_route_topk_w<2>, grid, dim3(256), 0, st, logits, s_rows, n_expert, k, norm_topk, weights_scale,
                idx, w);
  else if (n_expert <= 256)
    KMOE_LAUNCH(k_route_topk_w<4>, grid, dim3(256), 0, st, logits, s_rows, n_expert, k, norm_topk, weights_scale,
                idx, w);
  else
    KMOE_LAUNCH(k_route_topk, grid, dim3(256), 0, st, logits, s_rows, n_expert, k, norm_topk, weights_scale, idx,
                w);
  return hipGetLastError();
}

hipError_t launch_dispatch(hipStream_t st, const uint32_t *idx, int64_t n_slots, int32_t n_expert, uint32_t *perm,
                           uint32_t *offsets, uint32_t *inv, int32_t *n_active, int32_t *active, uint32_t *rank_tmp) {
  if (n_expert > kMaxExperts || n_expert <= 0) return hipErrorInvalidValue;
  (void)rank_tmp;
  KMOE_LAUNCH(k_dispatch, dim3(1), dim3(1024), 0, st, idx, n_slots, n_expert, perm, offsets, inv, n_active,
                     active);
  return hipGetLastError();
}

// One unit per wave: a Q8_K block (KQ) or eight Q8 blocks; segment A's units
// first, then segment B's.
template <bool KA, bool KB>
__global__ void __launch_bounds__(256) k_quant_two(const float *__restrict__ ha, int64_t n_a, int8_t *__restrict__ qa,
                                                   float *__restrict__ da, int32_t *__restrict__ sa,
                                                   const float *__restrict__ hb, int64_t n_b, int8_t *__restrict__ qb,
                                                   float *__restrict__ db, int32_t *__restrict__ sb) {
  const int lane = threadIdx.x & 63;
  int64_t u = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t ua = KA ? n_a / 256 : (n_a / 32 + 7) / 8;
  const int64_t ub = KB ? n_b / 256 : (n_b / 32 + 7) / 8;
  if (u < ua) {
    if constexpr (KA) {
      wave_quant_q8k_block(ha + u * 256, qa + u * 256, da + u, sa + u * 16, lane);
    } else {
      const int64_t blk = u * 8 + (lane >> 3);
      if (blk < n_a / 32) group8_quant_q8_block(ha + blk * 32, qa + blk * 32, da + blk, sa + blk * 2, lane & 7);
    }
    return;
  }
  u -= ua;
  if (u >= ub) return;
  if constexpr (KB) {
    wave_quant_q8k_block(hb + u * 256, qb + u * 256, db + u, sb + u * 16, lane);
  } else {
    const int64_t blk = u * 8 + (lane >> 3);
    if (blk < n_b / 32) group8_quant_q8_block(hb + blk * 32, qb + blk * 32, db + blk, sb + blk * 2, lane & 7);
  }
}

hipError_t launch_quant_two(hipStream_t st, int type_a, const float *ha, int64_t n_a, int8_t *qa, float *da,
                            int32_t *sa, int type_b, const float *hb, int64_t n_b, int8_t *qb, float *db,
                            int32_t *sb) {
  const bool ka = is_kquant(type_a), kb = is_kquant(type_b);
  if ((type_a != T_Q8_0 && !ka) || (type_b != T_Q8_0 && !kb) || n_a % (ka ? 256 : 32) || n_b % (kb ? 256 : 32))
    return hipErrorNotSupported;
  const int64_t units = (ka ? n_a / 256 : (n_a / 32 + 7) / 8) + (kb ? n_b / 256 : (n_b / 32 + 7) / 8);
  if (units <= 0) return hipSuccess;
  const dim3 grid((unsigned)((units + 3) / 4));
  if (ka && kb) KMOE_LAUNCH((k_quant_two<true, true>), grid, dim3(256), 0, st, ha, n_a, qa, da, sa, hb, n_b, qb, db, sb);
  else if (ka) KMOE_LAUNCH((k_quant_two<true, false>), grid, dim3(256), 0, st, ha, n_a, qa, da, sa, hb, n_b, qb, db, sb);
  else if (kb) KMOE_LAUNCH((k_quant_two<false, true>), grid, dim3(256), 0, st, ha, n_a, qa, da, sa, hb, n_b, qb, db, sb);
  else KMOE_LAUNCH((k_quant_two<false, false>), grid, dim3(256), 0, st, ha, n_a, qa, da, sa, hb, n_b, qb, db, sb);
  return hipGetLastError();
}

hipError_t launch_quant_slots(hipStream_t st, int type, const float *h, int64_t n_slots, int64_t cols,
                              const Routing &rt, const uint32_t *idx_flat, int regime, int8_t *q, float *d,
                              int32_t *sums) {
  if (n_slots == 0) return hipSuccess;
  if (is_kquant(type)) {
    const int64_t nb = n_slots * (cols / 256);
    KMOE_LAUNCH(k_quant_slots_q8k, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, st, h, n_slots, cols, rt,
                       idx_flat, regime, q, d, sums);
  } else if (type == T_Q8_0) {
    const int64_t nb = n_slots * (cols / 32);
    const int64_t waves = (nb + 7) / 8;
    KMOE_LAUNCH(k_quant_slots_q8, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, h, n_slots, cols, rt,
                       idx_flat, regime, q, d, sums);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_combine(hipStream_t st, const float *y, const Routing &rt, int64_t s_rows, int64_t d, float *out) {
  if (s_rows == 0) return hipSuccess;
  if (rt.topk > 16) return hipErrorInvalidValue;
  const bool vec = d % 4 == 0 && (((uintptr_t)y | (uintptr_t)out) & 15) == 0;
  for (int64_t s0 = 0; s0 < s_rows; s0 += 65535) {  // tokens along grid y, at most 65535 per launch
    const unsigned ny = (unsigned)(s_rows - s0 < 65535 ? s_rows - s0 : 65535);
    if (vec) {
      // one wave per 64 float4 columns (at most 64 per token), so a small
      // batch still spreads over many CUs
      const int64_t d4 = d / 4, gx = (d4 + 63) / 64 < 64 ? (d4 + 63) / 64 : 64;
      KMOE_LAUNCH(k_combine4, dim3((unsigned)gx, ny), dim3(64), 0, st, y, rt, s0, d, out);
    } else {
      KMOE_LAUNCH(k_combine, dim3((unsigned)((d + 255) / 256), ny), dim3(256), 0, st, y, rt, s_rows, s0, d, out);
    }
  }
  return hipGetLastError();
}

}  // namespace kmoe

namespace kmoe {
bool route_norm_supported(const RouteNorm *n, int32_t S, int64_t d) {
  if (!n || !n->x || !n->w || !n->f || !n->done || S != 1 || d % 256 != 0 || d < 256 || d > kDecMaxD) return false;
  return (((uintptr_t)n->x | (uintptr_t)n->y | (uintptr_t)n->w | (uintptr_t)n->f) & 15) == 0;
}

hipError_t launch_route_decode(hipStream_t st, const float *router, int32_t E, int64_t d, const float *x, int32_t S,
                               int32_t k, int32_t norm_topk, float weights_scale, float *logits, uint32_t *idx,
                               float *w, uint32_t *perm, uint32_t *offsets, uint32_t *inv, int32_t *n_active,
                               int32_t *active, int qtype, int8_t *xq, float *xd, int32_t *xs, uint32_t *done,
                               const RouteNorm *norm) {
  if (S < 1 || S > 3 || E < 1 || E > kMaxExperts || k < 1 || k > 16 || k > E || S * k > 48) return hipErrorNotSupported;
  if (d < 8 || d > kDecMaxD) return hipErrorNotSupported;
  if (!logits) return hipErrorInvalidValue;
  if (norm && !route_norm_supported(norm, S, d)) return hipErrorNotSupported;
  const int vec = d % 4 == 0 && ((uintptr_t)router & 15) == 0 && ((uintptr_t)x & 15) == 0;
  RouteDecArgs a{router, E, d, x, S, k, norm_topk, weights_scale, logits, idx, w, perm, offsets, inv, n_active, active,
                 qtype, xq, xd, xs, done, vec, norm ? *norm : RouteNorm{}};
  const int64_t nq = 2 * (d / 8);
  if (nq <= 256) KMOE_LAUNCH(k_route_dec<1>, dim3(E), dim3(256), 0, st, a);
  else if (nq <= 512) KMOE_LAUNCH(k_route_dec<2>, dim3(E), dim3(256), 0, st, a);
  else if (nq <= 1024) KMOE_LAUNCH(k_route_dec<4>, dim3(E), dim3(256), 0, st, a);
  else KMOE_LAUNCH(k_route_dec<8>, dim3(E), dim3(256), 0, st, a);
  return hipGetLastError();
}
}  // namespace kmoe
