// kmoe_mfma.hip — grouped Q4_K x Q8_K expert products on the int8 matrix
// cores (prefill and batched decode on the int8 path).
//
// Per expert e with n_e routed rows (token slots), per 32-row weight tile and
// 32-token tile, per superblock b (256 columns):
//   sumi(t, r) = sum_j sc_j(r) * sum_{x in sub-block j} q(r, x) * a(t, x)
//   mins(t, r) = sum_j m_j(r) * bsum_j(t)
//   y(t, r)   += (d(r) * ad(t, b)) * sumi - (dmin(r) * ad(t, b)) * mins
// (avx2.rs:351-379 for every row: the reference's int path). The integers are
// exact on the matrix cores:
//   * the 6-bit scale splits as sc = 8*hi + lo with hi, lo < 8, so q*hi and
//     q*lo (q < 16) are int8 values <= 105 and
//     sumi = 8 * mfma(a, q*hi) + mfma(a, q*lo), each an i32 dot over the
//     superblock's 256 columns (eight v_mfma_i32_32x32x32_i8 per tile);
//   * bsum_j (a sum of 32 int8, |bsum| <= 4064) splits as 64*bh + bl with
//     bl in [0, 64), so one v_mfma_f32_32x32x16_f16 over k = (j, half) of
//     (bh_j, bl_j) x (64*m_j, m_j) gives mins exactly (all products and partial
//     sums are integers below 2^24).
// Roles: A = activation rows (tokens, 32 per tile), B = weight rows, so in the
// 32x32 result each lane owns one weight row (lane % 32) and 16 tokens, and
// the per-row d, dmin, sc, m stay in the lane.
// The k order inside an MFMA only has to agree between A and B: lane half h
// holds columns 16h .. 16h+15 of the 32-column sub-block on both sides, which
// for the weights is exactly tiled chunk (b, j/2, h): lo nibbles for even j,
// hi nibbles for odd j.
// Work-group: 4 waves, one per SIMD. Each takes one 64-token half of a
// 128-token pass and one 32-row tile of one matrix (gate/up: 32 rows per
// group, SwiGLU, transformer.rs:558, after an LDS exchange between the gate
// and up waves; the single-matrix modes: 64 rows). More than 128 routed rows
// take more passes; the plain modes give each pass its own work-group.
// Modes: grouped gate/up and down over the expert tier's tiled Q4_K rows
// (routed token slots), and plain GGUF Q4_K rows [rows, cols] against s_rows
// activation rows: the matmul (quant.rs:229 on the int path) and the per-block
// integer accumulators (avx2.rs:361-374) exposed for parity checks.
// Superblock b+1's activation tile (LDS, double-buffered) and weight pieces
// are in flight while superblock b is multiplied.
#include "kmoe_device.h"
#include "kmoe_launch.h"

namespace kmoe {

namespace {

typedef int v4i32 __attribute__((ext_vector_type(4)));
typedef int v16i32 __attribute__((ext_vector_type(16)));
typedef float v16f32 __attribute__((ext_vector_type(16)));
typedef _Float16 v8f16 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kTokTile = 32, kTokPass = 128;  // token rows per pass (two halves of 64)

enum { MF_GATE_UP = 0, MF_DOWN = 1, MF_PLAIN = 2, MF_SUMS = 3 };

struct MfmaArgs {
  ExpertTier tier;
  Routing rt;
  const uint8_t *w0;   // plain modes: GGUF rows
  int64_t s_rows;      // plain modes: activation rows
  int64_t rows, cols;  // weight rows (F for gate/up, d for down), columns
  const int8_t *aq;    // int8 activation rows
  const float *ad;     // their block scales [.., cols/256]
  const int32_t *abs;  // their 16-sums [.., cols/16]
  float *out;          // [slots or s_rows, rows]
  int32_t *sumi, *mins;  // MF_SUMS: [(s*rows + r)*nb + b]
  int regime;
};

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

// One LDS stage (superblock b of the pass's 128 token rows):
//   int8 [8 sub-blocks][2 halves][128 tokens][16 bytes]    32 KB
//   f16  [2 halves][128 tokens][8] = (bh_0..7 | bl_0..7)    4 KB
//   f32  ad [128]                                           0.5 KB
constexpr int kStageQ = 8 * 2 * kTokPass * 16;
constexpr int kStageB = 2 * kTokPass * 16;
constexpr int kStageBytes = kStageQ + kStageB + kTokPass * 4;

__device__ __forceinline__ bool mfma_int_regime(int regime, int n) {
  return regime == REGIME_INT8 || (regime == REGIME_AVX2 && n < 4);
}

// scale_min_k4 (quant.rs:54-61) for all eight sub-blocks of a superblock head.
__device__ __forceinline__ void q4k_scales8(uint32_t s03, uint32_t s47, uint32_t s811, int (&sc)[8], int (&m)[8]) {
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sc[j] = (int)((s03 >> (8 * j)) & 63u);
    m[j] = (int)((s47 >> (8 * j)) & 63u);
    const uint32_t q8 = (s811 >> (8 * j)) & 0xffu;
    sc[j + 4] = (int)((q8 & 0xfu) | (((s03 >> (8 * j + 6)) & 3u) << 4));
    m[j + 4] = (int)((q8 >> 4) | (((s47 >> (8 * j + 6)) & 3u) << 4));
  }
}

// 4 waves, one per SIMD (the full register file each: accumulators, B
// operands and the next superblock's loads stay in registers). Wave w takes
// the 64-token half w & 1 of each 128-row pass and, for gate/up, matrix w >> 1
// of the group's 32-row tile; otherwise 32-row tile w >> 1 of the group's 64.
template <int MODE>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) k_moe_mfma(MfmaArgs a) {
  constexpr bool TILED = MODE == MF_GATE_UP || MODE == MF_DOWN;  // expert tier rows are tiled, plain rows GGUF
  __shared__ __attribute__((aligned(16))) uint8_t stage[2][kStageBytes];
  __shared__ int32_t srcs[kTokPass];
  const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t cols = a.cols, nb = cols / 256, row_bytes = nb * 144;
  const int mat = MODE == MF_GATE_UP ? (wave >> 1) : 2;
  const int64_t rtile = MODE == MF_GATE_UP ? (int64_t)blockIdx.x : (int64_t)blockIdx.x * 2 + (wave >> 1);
  const int th = wave & 1;  // token half of the pass
  const int64_t r = rtile * 32 + l32;  // this lane's weight row
  const bool rv = r < a.rows;
  const int64_t rr = rv ? r : a.rows - 1;
  int64_t p0 = 0;
  int n, t_begin, t_end;
  const uint8_t *W;
  if constexpr (TILED) {
    const int i_act = blockIdx.y;
    if (i_act >= *a.rt.n_active) return;
    const int e = a.rt.active[i_act];
    p0 = a.rt.offsets[e];
    n = (int)(a.rt.offsets[e + 1] - p0);
    if (!mfma_int_regime(a.regime, n)) return;
    W = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[mat] + rr * row_bytes;
    t_begin = 0;
    t_end = n;
  } else {
    n = (int)a.s_rows;
    W = a.w0 + rr * row_bytes;
    t_begin = (int)blockIdx.y * kTokPass;
    t_end = t_begin + kTokPass < n ? t_begin + kTokPass : n;
  }
  // staging roles: 16-byte piece pc (columns 16pc..) of tokens (tid >> 4) + 16k, k < 8
  const int pc = tid & 15, sj = pc >> 1, sh = pc & 1;

  for (int t0 = t_begin; t0 < t_end; t0 += kTokPass) {
    const int nt = t_end - t0 < kTokPass ? t_end - t0 : kTokPass;
    __syncthreads();  // the previous pass is done with srcs and the stages
    if (tid < kTokPass) {
      int32_t src = 0;
      if (tid < nt) {
        if constexpr (MODE == MF_GATE_UP) src = (int32_t)(a.rt.perm[p0 + t0 + tid] / a.rt.topk);
        else src = (int32_t)(p0 + t0 + tid);
      }
      srcs[tid] = src;
    }
    __syncthreads();
    int64_t qoff[8];
    bool qv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const int t = (tid >> 4) + 16 * k;
      qv[k] = t < nt;
      qoff[k] = (int64_t)srcs[qv[k] ? t : 0] * cols + 16 * pc;
    }
    const bool bt = tid < kTokPass && tid < nt;
    const int64_t src_b = bt ? srcs[tid] : 0;
    const int tq = tid >> 2, bq = tid & 3;  // 16-sum staging: tokens tq and tq + 64, sums 4bq .. 4bq+3
    const bool qt0 = tq < nt, qt1 = tq + 64 < nt;
    const int64_t src_q0 = qt0 ? srcs[tq] : 0, src_q1 = qt1 ? srcs[tq + 64] : 0;
    // prefetch registers: activation pieces, 16-sums, block scale, weight head and nibbles
    int4 SQ[8], SB0, SB1;
    float SD = 0.0f;
    u32x4 WH, WQ[4];
    auto fetch = [&](int64_t b) {
#pragma unroll
      for (int k = 0; k < 8; ++k) SQ[k] = *(const int4 *)(a.aq + qoff[k] + 256 * b);
      SB0 = *(const int4 *)(a.abs + src_q0 * (cols / 16) + 16 * b + 4 * bq);  // 16-sums 4bq .. 4bq+3
      SB1 = *(const int4 *)(a.abs + src_q1 * (cols / 16) + 16 * b + 4 * bq);
      if constexpr (MODE != MF_SUMS) {
        if (tid < kTokPass) SD = a.ad[src_b * nb + b];
      }
      if constexpr (TILED) {
        WH = __builtin_nontemporal_load((const u32x4 *)(W + 16 * b));
        const uint8_t *qp = W + tq4_qs_off(nb, b, 0, half);
#pragma unroll
        for (int i = 0; i < 4; ++i) WQ[i] = __builtin_nontemporal_load((const u32x4 *)(qp + 16 * i));
      } else {  // GGUF superblock: head, then qs chunk (k, half) at 16 + 32k + 16*half
        const uint8_t *sbp = W + 144 * b;
        WH = __builtin_nontemporal_load((const u32x4a4 *)sbp);
#pragma unroll
        for (int i = 0; i < 4; ++i)
          WQ[i] = __builtin_nontemporal_load((const u32x4a4 *)(sbp + 16 + 32 * i + 16 * half));
      }
    };
    auto put = [&](int buf) {
      uint8_t *S = stage[buf];
#pragma unroll
      for (int k = 0; k < 8; ++k) {
        const int t = (tid >> 4) + 16 * k;
        *(int4 *)(S + ((sj * 2 + sh) * kTokPass + t) * 16) = qv[k] ? SQ[k] : make_int4(0, 0, 0, 0);
      }
      _Float16 *hb = (_Float16 *)(S + kStageQ);
      auto put_sums = [&](int t, bool ok, const int4 &sb) {
        // sub-blocks 2bq, 2bq+1 of token t: 32-sums split as 64*bh + bl (bl in [0, 64))
        const int s0 = ok ? sb.x + sb.y : 0, s1 = ok ? sb.z + sb.w : 0;
        const int h0 = s0 >> 6, h1 = s1 >> 6;  // floor division
        hb[(0 * kTokPass + t) * 8 + 2 * bq] = (_Float16)h0;
        hb[(0 * kTokPass + t) * 8 + 2 * bq + 1] = (_Float16)h1;
        hb[(1 * kTokPass + t) * 8 + 2 * bq] = (_Float16)(s0 - 64 * h0);
        hb[(1 * kTokPass + t) * 8 + 2 * bq + 1] = (_Float16)(s1 - 64 * h1);
      };
      put_sums(tq, qt0, SB0);
      put_sums(tq + 64, qt1, SB1);
      if (tid < kTokPass) *(float *)(S + kStageQ + kStageB + 4 * tid) = bt ? SD : 0.0f;
    };
    v4i32 bhi[8], blo[8];
    v8f16 bm;
    float dw = 0.0f, dmw = 0.0f;
    auto build = [&]() {  // B operands of this lane's row from WH/WQ
      int sc[8], mn[8];
      q4k_scales8(WH.y, WH.z, WH.w, sc, mn);
      dw = f16_bits_to_f32(WH.x);
      dmw = f16_bits_to_f32(WH.x >> 16);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const u32x4 w = WQ[j >> 1];
        const uint32_t msk = 0x0f0f0f0fu;
        const int s4 = (j & 1) ? 4 : 0;
        const uint32_t n0 = (w.x >> s4) & msk, n1 = (w.y >> s4) & msk, n2 = (w.z >> s4) & msk,
                       n3 = (w.w >> s4) & msk;
        const uint32_t hi = (uint32_t)(sc[j] >> 3), lo = (uint32_t)(sc[j] & 7);
        // bytes times a factor < 8 stay below 106: no carries between bytes
        bhi[j] = v4i32{(int)(n0 * hi), (int)(n1 * hi), (int)(n2 * hi), (int)(n3 * hi)};
        blo[j] = v4i32{(int)(n0 * lo), (int)(n1 * lo), (int)(n2 * lo), (int)(n3 * lo)};
        bm[j] = (_Float16)(half ? mn[j] : 64 * mn[j]);
      }
    };
    float y[2][16];
#pragma unroll
    for (int T = 0; T < 2; ++T)
#pragma unroll
      for (int v = 0; v < 16; ++v) y[T][v] = 0.0f;
    const int ntiles_mine = (nt - 64 * th + kTokTile - 1) / kTokTile;  // this wave's tiles (may be <= 0)
    fetch(0);
    put(0);
    build();
    lds_barrier();
    for (int64_t b = 0; b < nb; ++b) {
      const uint8_t *S = stage[b & 1];
      if (b + 1 < nb) fetch(b + 1);
#pragma unroll
      for (int T = 0; T < 2; ++T) {
        if (T < ntiles_mine) {
          const int tl = 64 * th + T * kTokTile + l32;  // A-operand token row of this lane
          v16i32 ahi = {0}, alo = {0};
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const v4i32 av = *(const v4i32 *)(S + ((j * 2 + half) * kTokPass + tl) * 16);
            ahi = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, bhi[j], ahi, 0, 0, 0);
            alo = __builtin_amdgcn_mfma_i32_32x32x32_i8(av, blo[j], alo, 0, 0, 0);
          }
          const v8f16 am = *(const v8f16 *)(S + kStageQ + (half * kTokPass + tl) * 16);
          v16f32 mins = {0};
          mins = __builtin_amdgcn_mfma_f32_32x32x16_f16(am, bm, mins, 0, 0, 0);
          // result layout: token row 8*(v/4) + 4*half + v%4 of the tile, weight row l32
          if constexpr (MODE == MF_SUMS) {
            if (rv) {
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const int t = 64 * th + T * kTokTile + 8 * (v >> 2) + 4 * half + (v & 3);
                if (t < nt) {
                  const int64_t o = ((int64_t)(t0 + t) * a.rows + r) * nb + b;
                  a.sumi[o] = 8 * ahi[v] + alo[v];
                  a.mins[o] = (int)mins[v];
                }
              }
            }
            continue;
          }
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 adv =
                *(const float4 *)(S + kStageQ + kStageB + 4 * (64 * th + T * kTokTile + 8 * g + 4 * half));
            const float advs[4] = {adv.x, adv.y, adv.z, adv.w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              const int v = 4 * g + c;
              const int si = 8 * ahi[v] + alo[v];
              const float dd = dw * advs[c], dm = dmw * advs[c];
              y[T][v] = fmaf(dd, (float)si, y[T][v]);
              y[T][v] = fmaf(-dm, mins[v], y[T][v]);
            }
          }
        }
      }
      if (b + 1 < nb) {
        put((b + 1) & 1);
        build();
      }
      lds_barrier();
    }
    // ---- results: out[p0 + t0 + token, r]
    if constexpr (MODE == MF_SUMS) {
    } else if constexpr (MODE == MF_GATE_UP) {
      // the up waves (2, 3) hand their values to the gate waves (0, 1) of the same token half
      float *x = (float *)stage[0];  // [2 halves][32 rows][64 tokens + 1]
      constexpr int XS = 65;
      if (wave >= 2) {
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
          for (int v = 0; v < 16; ++v)
            x[((wave & 1) * 32 + l32) * XS + T * kTokTile + 8 * (v >> 2) + 4 * half + (v & 3)] = y[T][v];
      }
      lds_barrier();
      if (wave < 2 && rv) {
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int tt = T * kTokTile + 8 * (v >> 2) + 4 * half + (v & 3);
            const int t = 64 * th + tt;
            if (t < nt) {
              const float g = y[T][v], u = x[(th * 32 + l32) * XS + tt];
              const float den = 1.0f + expf_cr(-g);  // SwiGLU: g / (1 + exp(-g)) * u
              const float q = g / den;
              a.out[(p0 + t0 + t) * a.rows + r] = q * u;
            }
          }
      }
    } else {
      if (rv) {
#pragma unroll
        for (int T = 0; T < 2; ++T)
#pragma unroll
          for (int v = 0; v < 16; ++v) {
            const int t = 64 * th + T * kTokTile + 8 * (v >> 2) + 4 * half + (v & 3);
            if (t < nt) a.out[(p0 + t0 + t) * a.rows + r] = y[T][v];
          }
      }
    }
  }
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

// Launch knob, read once: KMOE_MFMA_MIN_ROWS, the token rows from which the
// matrix-core kernels are used (default 8).
int mfma_min_rows() {
  static const int v = [] {
    const char *e = getenv("KMOE_MFMA_MIN_ROWS");
    const int x = e && *e ? atoi(e) : 0;
    return x > 0 ? x : 8;
  }();
  return v;
}

bool moe_mfma_supported(int64_t rows, int64_t cols) {
  return rows > 0 && cols > 0 && cols % 256 == 0 && rows < (1ll << 31) / 32 && cols / 256 < (1ll << 24);
}

hipError_t launch_moe_mfma(hipStream_t st, int mode, const ExpertTier &tier, int64_t rows, int64_t cols,
                           const Routing &rt, int regime, int max_active, const int8_t *aq, const float *ad,
                           const int32_t *abs, float *out) {
  if (!moe_mfma_supported(rows, cols) || !aligned16(aq) || !aligned16(abs)) return hipErrorNotSupported;
  if (max_active == 0) return hipSuccess;
  MfmaArgs a{};
  a.tier = tier;
  a.rt = rt;
  a.rows = rows;
  a.cols = cols;
  a.aq = aq;
  a.ad = ad;
  a.abs = abs;
  a.out = out;
  a.regime = regime;
  const int64_t rows_per_wg = mode == MF_GATE_UP ? 32 : 64;
  const dim3 grid((unsigned)((rows + rows_per_wg - 1) / rows_per_wg), (unsigned)max_active);
  if (mode == MF_GATE_UP) KMOE_LAUNCH((k_moe_mfma<MF_GATE_UP>), grid, dim3(256), 0, st, a);
  else KMOE_LAUNCH((k_moe_mfma<MF_DOWN>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_plain_mfma(hipStream_t st, const uint8_t *w, int64_t rows, int64_t cols, const int8_t *aq,
                             const float *ad, const int32_t *abs, int64_t s_rows, float *out, int32_t *sumi,
                             int32_t *mins) {
  if (!moe_mfma_supported(rows, cols) || !aligned16(aq) || !aligned16(abs) || ((uintptr_t)w & 3u) ||
      s_rows > (int64_t)kTokPass * 65535)
    return hipErrorNotSupported;
  if (s_rows == 0) return hipSuccess;
  MfmaArgs a{};
  a.w0 = w;
  a.s_rows = s_rows;
  a.rows = rows;
  a.cols = cols;
  a.aq = aq;
  a.ad = ad;
  a.abs = abs;
  a.out = out;
  a.sumi = sumi;
  a.mins = mins;
  a.regime = REGIME_INT8;
  const dim3 grid((unsigned)((rows + 63) / 64), (unsigned)((s_rows + kTokPass - 1) / kTokPass));
  if (sumi) KMOE_LAUNCH((k_moe_mfma<MF_SUMS>), grid, dim3(256), 0, st, a);
  else KMOE_LAUNCH((k_moe_mfma<MF_PLAIN>), grid, dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace kmoe
