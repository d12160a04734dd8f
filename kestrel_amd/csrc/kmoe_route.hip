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
#include "kmoe_device.h"
#include "kmoe_launch.h"

namespace kmoe {

namespace {

enum { ORD_GEMM = 0, ORD_DOTF32 = 1, ORD_QDOT = 2 };

__device__ __forceinline__ float hsum8(const float *v) {
  const float a = v[0] + v[4], b = v[2] + v[6], c = v[1] + v[5], d = v[3] + v[7];
  return (a + b) + (c + d);
}

__global__ void __launch_bounds__(256) k_router_logits(const float *__restrict__ W, int32_t E, int64_t d,
                                                       const float *__restrict__ X, int64_t S,
                                                       float *__restrict__ logits) {
  const int l16 = threadIdx.x & 15;
  const int64_t pair = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const bool valid = pair < S * E;
  const int64_t s = valid ? pair / E : 0;
  const int e = valid ? (int)(pair % E) : 0;
  int ord;
  if (S < 4 || (d % 8) != 0) {
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
  const int64_t n8 = d / 8;
  float acc = 0.0f;
  if (valid) {
    if (ord == ORD_GEMM) {
      if (l16 < 8) {
#pragma unroll 8
        for (int64_t c = 0; c < n8; ++c) acc = fmaf(w[8 * c + l16], x[8 * c + l16], acc);
      }
    } else if (ord == ORD_QDOT) {
      if (l16 < 8) {
#pragma unroll 8
        for (int64_t c = 0; c < n8; ++c) {
          const float p = w[8 * c + l16] * x[8 * c + l16];
          acc = acc + p;
        }
      }
    } else {
      const int64_t n16 = d / 16;
      const int l = l16 & 7;
      const int64_t off = l16 < 8 ? 0 : 8;
#pragma unroll 8
      for (int64_t c = 0; c < n16; ++c) acc = fmaf(w[16 * c + off + l], x[16 * c + off + l], acc);
      if (l16 < 8 && (d - 16 * n16) >= 8) acc = fmaf(w[16 * n16 + l], x[16 * n16 + l], acc);
    }
  }
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
    // Largest p, ties to the lower index: key = (bits(p) << 32) | ~index.
    uint64_t best = 0;
    for (int e = lane; e < E; e += 64) {
      if (taken[wave][e]) continue;
      const uint64_t key = ((uint64_t)__float_as_uint(P[wave][e]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
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
// work-group of 1024 threads. Per chunk of 1024 entries, each wave finds the
// lanes that share its expert with log2(E) ballots, ranks within the wave by
// popcount, and a per-expert prefix over the 16 waves (plus a running base
// from earlier chunks) gives every entry its rank among its expert's entries
// in flat order — the order BTreeMap<expert, Vec<(token, w)>> fills in.
__global__ void __launch_bounds__(1024) k_dispatch(const uint32_t *__restrict__ idx, int64_t n, int32_t E,
                                                   uint32_t *__restrict__ perm, uint32_t *__restrict__ offsets,
                                                   uint32_t *__restrict__ inv, int32_t *__restrict__ n_active,
                                                   int32_t *__restrict__ active, uint32_t *__restrict__ rank) {
  __shared__ uint32_t hist[16][kMaxExperts];
  __shared__ uint32_t base[kMaxExperts];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int nbits = 0;
  while ((1 << nbits) < E) ++nbits;
  for (int e = tid; e < E; e += 1024) base[e] = 0;
  for (int w = 0; w < 16; ++w)
    for (int e = tid; e < E; e += 1024) hist[w][e] = 0;
  __syncthreads();
  const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int64_t c0 = 0; c0 < n; c0 += 1024) {
    const int64_t i = c0 + tid;
    const uint32_t ev = i < n ? idx[i] : 0u;
    const bool valid = i < n && ev < (uint32_t)E;  // ids >= E are dropped, never indexed
    const uint32_t e = valid ? ev : 0u;
    uint64_t same = __ballot(valid);
    for (int b = 0; b < nbits; ++b) {
      const bool bit = (e >> b) & 1u;
      const uint64_t m = __ballot(valid && bit);
      same &= bit ? m : ~m;
    }
    const uint32_t wrank = (uint32_t)__popcll(same & lt);
    if (valid && wrank == 0) hist[wave][e] = (uint32_t)__popcll(same);
    __syncthreads();
    for (int ee = tid; ee < E; ee += 1024) {
      uint32_t run = base[ee];
      for (int w = 0; w < 16; ++w) {
        const uint32_t c = hist[w][ee];
        hist[w][ee] = run;
        run += c;
      }
      base[ee] = run;
    }
    __syncthreads();
    if (valid) rank[i] = hist[wave][e] + wrank;
    __syncthreads();
    for (int w = 0; w < 16; ++w)
      for (int ee = tid; ee < E; ee += 1024) hist[w][ee] = 0;
    __syncthreads();
  }
  if (tid == 0) {
    uint32_t run = 0;
    int na = 0;
    for (int ee = 0; ee < E; ++ee) {
      offsets[ee] = run;
      if (base[ee] > 0 && active) active[na++] = ee;
      run += base[ee];
      base[ee] = offsets[ee];
    }
    offsets[E] = run;
    if (n_active) *n_active = na;
  }
  __syncthreads();
  for (int64_t i = tid; i < n; i += 1024) {
    if (idx[i] >= (uint32_t)E) continue;
    const uint32_t p = base[idx[i]] + rank[i];
    perm[p] = (uint32_t)i;
    if (inv) inv[i] = p;
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

// out[s, c] = sum over the token's slots in ascending expert id of w * y[slot, c]
// (multiply, then add; transformer.rs:566-570).
__global__ void __launch_bounds__(256) k_combine(const float *__restrict__ y, Routing rt, int64_t S, int64_t d,
                                                 float *__restrict__ out) {
  const int64_t s = blockIdx.y;
  const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (s >= S || c >= d) return;
  const int k = rt.topk;
  uint32_t p[16];
  float w[16];
  for (int j = 0; j < k; ++j) {
    p[j] = rt.inv[s * k + j];
    w[j] = rt.wsel[s * k + j];
  }
  for (int j = 1; j < k; ++j) {  // ascending slot position == ascending expert id
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
  float *logits;  // [S, E]: written when the logits are split over work-groups (or asked for)
  uint32_t *idx;
  float *wsel;
  uint32_t *perm, *offsets, *inv;
  int32_t *n_active, *active;
  int qtype;  // 0: none, T_Q4_K: Q8_K rows, T_Q8_0: Q8 rows
  int8_t *xq;
  float *xd;
  int32_t *xs;
};

constexpr int kDecEpw = 8;       // experts per work-group
constexpr int kDecMaxChunks = 16;  // columns per work-group <= 16 chunks of 512

// Softmax, top-k, renormalisation (transformer.rs:479-495) for S tokens whose
// logits are in lg[s*E + e] (LDS), then the dispatch and the int8 quantization
// of x. Runs in one work-group of 1024 threads.
__device__ void route_tail(const RouteDecArgs &a, const float *lg, float *Pn, int *taken, uint32_t *sel_e,
                           float *sel_w, uint32_t *cnt) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nthr = blockDim.x, nwaves = nthr >> 6;
  const int E = a.E;
  if (wave < a.S) {
    const int s = wave;
    const float *row = lg + s * E;
    float *P = Pn + s * E;
    int *tk = taken + s * E;
    float m = -INFINITY;
    for (int e = lane; e < E; e += 64) m = fmaxf(m, row[e]);
    m = group_max<64>(m);
    for (int e = lane; e < E; e += 64) {
      P[e] = expf_cr(row[e] - m);
      tk[e] = 0;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    float sum = 0.0f;
    if (lane == 0) {
      sum = -0.0f;
      for (int e = 0; e < E; ++e) sum = sum + P[e];
    }
    sum = __shfl(sum, 0);
    for (int e = lane; e < E; e += 64) P[e] = P[e] / sum;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    for (int j = 0; j < a.k; ++j) {
      uint64_t best = 0;
      for (int e = lane; e < E; e += 64) {
        if (tk[e]) continue;
        const uint64_t key = ((uint64_t)__float_as_uint(P[e]) << 32) | (uint64_t)(0xffffffffu - (uint32_t)e);
        best = key > best ? key : best;
      }
#pragma unroll
      for (int off = 32; off > 0; off >>= 1) {
        const uint32_t hi = __shfl_xor((unsigned)(best >> 32), off), lo = __shfl_xor((unsigned)best, off);
        const uint64_t o = ((uint64_t)hi << 32) | lo;
        best = o > best ? o : best;
      }
      const uint32_t e = 0xffffffffu - (uint32_t)best;
      if (lane == 0) {
        tk[e] = 1;
        sel_e[s * a.k + j] = e;
        sel_w[s * a.k + j] = P[e];
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    }
    if (lane == 0) {
      float *w = &sel_w[s * a.k];
      if (a.norm_topk) {
        float ss = -0.0f;
        for (int j = 0; j < a.k; ++j) ss = ss + w[j];
        ss = fmaxf(ss, 6.103515625e-05f);
        for (int j = 0; j < a.k; ++j) w[j] = w[j] / ss;
      }
      if (a.weights_scale != 0.0f && a.weights_scale != 1.0f)
        for (int j = 0; j < a.k; ++j) w[j] = w[j] * a.weights_scale;
      for (int j = 0; j < a.k; ++j) {
        a.idx[s * a.k + j] = sel_e[s * a.k + j];
        a.wsel[s * a.k + j] = w[j];
      }
    }
  }
  // dispatch: stable counting sort of the S*k <= 64 flat slots by expert
  const int n = a.S * a.k;
  for (int e = tid; e < E; e += nthr) cnt[e] = 0;
  __syncthreads();
  if (tid < n) atomicAdd(&cnt[sel_e[tid]], 1u);
  __syncthreads();
  if (tid == 0) {
    uint32_t run = 0;
    int na = 0;
    for (int e = 0; e < E; ++e) {
      const uint32_t c = cnt[e];
      a.offsets[e] = run;
      if (c) a.active[na++] = e;
      cnt[e] = run;
      run += c;
    }
    a.offsets[E] = run;
    *a.n_active = na;
  }
  __syncthreads();
  if (tid < n) {
    const uint32_t e = sel_e[tid];
    uint32_t r = 0;
    for (int j = 0; j < tid; ++j) r += sel_e[j] == e ? 1u : 0u;  // earlier slots of the same expert
    const uint32_t p = cnt[e] + r;
    a.perm[p] = (uint32_t)tid;
    a.inv[tid] = p;
  }
  // int8 activation rows for the int path
  const int64_t d = a.d;
  if (a.qtype == T_Q4_K) {
    const int64_t nb = (int64_t)a.S * (d / 256);
    for (int64_t b = wave; b < nb; b += nwaves)
      wave_quant_q8k_block(a.X + b * 256, a.xq + b * 256, a.xd + b, a.xs + b * 16, lane);
  } else if (a.qtype == T_Q8_0) {
    const int64_t nb = (int64_t)a.S * (d / 32);
    for (int64_t b = (int64_t)wave * 8 + (lane >> 3); b < nb; b += (int64_t)nwaves * 8)
      group8_quant_q8_block(a.X + b * 32, a.xq + b * 32, a.xd + b, a.xs + b * 2, lane & 7);
  }
}

// Logits of experts [8g, 8g+8) for the S (< 4) tokens in quant::dot order
// (quant.rs:208-224): eight chains acc_l = sum over c of p_{8c+l} in order,
// p = w*x rounded on its own. Each of the 1024 threads loads its share of W
// and x for every 512-column chunk at once (one memory latency) and forms
// the products in registers; chunk by chunk they are transposed into LDS so
// each chain reads its products four at a time. With a single work-group the
// tail (top-k, dispatch, quantization) follows in the same kernel.
template <int NCH>
__global__ void __launch_bounds__(512) k_route_decode(RouteDecArgs a) {
  constexpr int KC = 512;    // columns per chunk
  constexpr int L = KC / 8;  // chain steps per chunk
  constexpr int CS = L + 4;  // padded chain row (spreads LDS banks)
  __shared__ __attribute__((aligned(16))) float P[2][kDecEpw * 8 * CS];
  __shared__ float lg[3 * kMaxExperts];
  __shared__ float Pn[3 * kMaxExperts];
  __shared__ int taken[3 * kMaxExperts];
  __shared__ uint32_t sel_e[64];
  __shared__ float sel_w[64];
  __shared__ uint32_t cnt[kMaxExperts];
  const int tid = threadIdx.x, lane = tid & 63;
  const int E = a.E;
  const int64_t d = a.d;
  const int64_t n8 = d / 8;  // chain length
  const int e0 = blockIdx.x * kDecEpw;
  const int ne = E - e0 < kDecEpw ? E - e0 : kDecEpw;
  const int nchain = ne * 8;
  const int nch = (int)((n8 * 8 + KC - 1) / KC);
  const bool vec = (d % 4) == 0;
  // This thread's 8 products per chunk: expert e0 + te, columns 8c..8c+7 of
  // the chunk, i.e. step c of each of the expert's eight chains.
  const int te = tid >> 6, c = tid & 63;

  for (int s = 0; s < a.S; ++s) {
    const float *x = a.X + (int64_t)s * d;
    float4 pa[NCH], pb[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      pa[j] = pb[j] = make_float4(0.f, 0.f, 0.f, 0.f);
      const int64_t col = (int64_t)j * KC + 8 * c;
      if (j < nch && te < ne && col < n8 * 8) {
        const float *w = a.W + (int64_t)(e0 + te) * d;
        if (vec) {
          const float4 w0 = *(const float4 *)(w + col), w1 = *(const float4 *)(w + col + 4);
          const float4 x0 = *(const float4 *)(x + col), x1 = *(const float4 *)(x + col + 4);
          pa[j] = make_float4(w0.x * x0.x, w0.y * x0.y, w0.z * x0.z, w0.w * x0.w);
          pb[j] = make_float4(w1.x * x1.x, w1.y * x1.y, w1.z * x1.z, w1.w * x1.w);
        } else {
          float t[8];
#pragma unroll
          for (int m = 0; m < 8; ++m) t[m] = w[col + m] * x[col + m];
          pa[j] = make_float4(t[0], t[1], t[2], t[3]);
          pb[j] = make_float4(t[4], t[5], t[6], t[7]);
        }
      }
    }
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j < nch) {
        float *B = P[j & 1];
        float *dst = B + (te * 8) * CS + c;
        dst[0 * CS] = pa[j].x;
        dst[1 * CS] = pa[j].y;
        dst[2 * CS] = pa[j].z;
        dst[3 * CS] = pa[j].w;
        dst[4 * CS] = pb[j].x;
        dst[5 * CS] = pb[j].y;
        dst[6 * CS] = pb[j].z;
        dst[7 * CS] = pb[j].w;
        __syncthreads();
        if (tid < nchain) {
          const float *row = &B[tid * CS];
          const int64_t left = n8 - (int64_t)j * L;
          const int steps = left < L ? (int)left : L;
          if (steps == L) {
#pragma unroll 4
            for (int i = 0; i < L; i += 4) {
              const float4 v = *(const float4 *)(row + i);
              acc = acc + v.x;
              acc = acc + v.y;
              acc = acc + v.z;
              acc = acc + v.w;
            }
          } else {
            for (int i = 0; i < steps; ++i) acc = acc + row[i];
          }
        }
      }
    }
    // Sum each expert's eight chains in order, then the tail (quant.rs:219-222).
    float v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = __shfl(acc, (lane & ~7) + i);
    if (tid < nchain && (tid & 7) == 0) {
      const int e = e0 + (tid >> 3);
      float r = -0.0f;
#pragma unroll
      for (int i = 0; i < 8; ++i) r = r + v[i];
      for (int64_t cc = n8 * 8; cc < d; ++cc) {
        const float p = a.W[(int64_t)e * d + cc] * x[cc];
        r = r + p;
      }
      lg[s * E + e] = r;
      if (a.logits) a.logits[(int64_t)s * E + e] = r;
    }
    __syncthreads();
  }
  if (gridDim.x == 1) route_tail(a, lg, Pn, taken, sel_e, sel_w, cnt);
}

// The tail for logits computed by several work-groups.
__global__ void __launch_bounds__(1024) k_route_finish(RouteDecArgs a) {
  __shared__ float lg[3 * kMaxExperts];
  __shared__ float Pn[3 * kMaxExperts];
  __shared__ int taken[3 * kMaxExperts];
  __shared__ uint32_t sel_e[64];
  __shared__ float sel_w[64];
  __shared__ uint32_t cnt[kMaxExperts];
  for (int i = threadIdx.x; i < a.S * a.E; i += 1024) lg[i] = a.logits[i];
  __syncthreads();
  route_tail(a, lg, Pn, taken, sel_e, sel_w, cnt);
}

}  // namespace

hipError_t launch_router_logits(hipStream_t st, const float *router, int32_t n_expert, int64_t d, const float *x,
                                int64_t s_rows, float *logits) {
  const int64_t pairs = s_rows * n_expert;
  if (pairs == 0) return hipSuccess;
  hipLaunchKernelGGL(k_router_logits, dim3((unsigned)((pairs + 15) / 16)), dim3(256), 0, st, router, n_expert, d, x,
                     s_rows, logits);
  return hipGetLastError();
}

hipError_t launch_route_topk(hipStream_t st, const float *logits, int64_t s_rows, int32_t n_expert, int32_t k,
                             int32_t norm_topk, float weights_scale, uint32_t *idx, float *w) {
  if (s_rows == 0) return hipSuccess;
  if (n_expert > kMaxExperts || k > 16 || k > n_expert || k <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_route_topk, dim3((unsigned)((s_rows + 3) / 4)), dim3(256), 0, st, logits, s_rows, n_expert, k,
                     norm_topk, weights_scale, idx, w);
  return hipGetLastError();
}

hipError_t launch_dispatch(hipStream_t st, const uint32_t *idx, int64_t n_slots, int32_t n_expert, uint32_t *perm,
                           uint32_t *offsets, uint32_t *inv, int32_t *n_active, int32_t *active, uint32_t *rank_tmp) {
  if (n_expert > kMaxExperts || n_expert <= 0) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_dispatch, dim3(1), dim3(1024), 0, st, idx, n_slots, n_expert, perm, offsets, inv, n_active,
                     active, rank_tmp);
  return hipGetLastError();
}

hipError_t launch_quant_slots(hipStream_t st, int type, const float *h, int64_t n_slots, int64_t cols,
                              const Routing &rt, const uint32_t *idx_flat, int regime, int8_t *q, float *d,
                              int32_t *sums) {
  if (n_slots == 0) return hipSuccess;
  if (type == T_Q4_K) {
    const int64_t nb = n_slots * (cols / 256);
    hipLaunchKernelGGL(k_quant_slots_q8k, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, st, h, n_slots, cols, rt,
                       idx_flat, regime, q, d, sums);
  } else if (type == T_Q8_0) {
    const int64_t nb = n_slots * (cols / 32);
    const int64_t waves = (nb + 7) / 8;
    hipLaunchKernelGGL(k_quant_slots_q8, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, h, n_slots, cols, rt,
                       idx_flat, regime, q, d, sums);
  } else {
    return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_combine(hipStream_t st, const float *y, const Routing &rt, int64_t s_rows, int64_t d, float *out) {
  if (s_rows == 0) return hipSuccess;
  if (rt.topk > 16) return hipErrorInvalidValue;
  hipLaunchKernelGGL(k_combine, dim3((unsigned)((d + 255) / 256), (unsigned)s_rows), dim3(256), 0, st, y, rt, s_rows,
                     d, out);
  return hipGetLastError();
}

}  // namespace kmoe

namespace kmoe {
hipError_t launch_route_decode(hipStream_t st, const float *router, int32_t E, int64_t d, const float *x, int32_t S,
                               int32_t k, int32_t norm_topk, float weights_scale, float *logits, uint32_t *idx,
                               float *w, uint32_t *perm, uint32_t *offsets, uint32_t *inv, int32_t *n_active,
                               int32_t *active, int qtype, int8_t *xq, float *xd, int32_t *xs) {
  if (S < 1 || S > 3 || E < 1 || E > 512 || k < 1 || k > 16 || k > E || S * k > 64) return hipErrorNotSupported;
  const int64_t nch = (d / 8 * 8 + 511) / 512;
  if (nch > kDecMaxChunks || d < 8) return hipErrorNotSupported;
  const int groups = (E + kDecEpw - 1) / kDecEpw;
  if (groups > 1 && !logits) return hipErrorInvalidValue;  // the split path needs the logits buffer
  RouteDecArgs a{router, E, d, x, S, k, norm_topk, weights_scale, logits, idx, w, perm, offsets, inv, n_active, active,
                 qtype, xq, xd, xs};
  if (nch <= 4) hipLaunchKernelGGL(k_route_decode<4>, dim3(groups), dim3(512), 0, st, a);
  else if (nch <= 8) hipLaunchKernelGGL(k_route_decode<8>, dim3(groups), dim3(512), 0, st, a);
  else hipLaunchKernelGGL(k_route_decode<16>, dim3(groups), dim3(512), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || groups == 1) return e;
  hipLaunchKernelGGL(k_route_finish, dim3(1), dim3(1024), 0, st, a);
  return hipGetLastError();
}
}  // namespace kmoe
