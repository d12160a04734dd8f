// kmoe_gemm_f32.hip — the reference's batched regime: weights dequantized to
// f32 and multiplied with f32 activations (quant.rs:242-260).
//
// Dequantization is dequant_row (quant.rs:82-89 for Q8_0: q * d; quant.rs:
// 138-155 for Q4_K: (d*sc)*q - (dmin*m), one multiply and one subtract, no
// FMA), so every weight value equals the reference's bit for bit. The dot
// products run on the fp32 matrix cores (exact products, fp32 sums) in a
// different order from gemm_f32's 8-lane chains (avx2.rs:230-286): results
// agree to a few f32 ulp of the sum.
//
// Tiling: a work-group computes 64 weight rows x 16 or 64 activation rows;
// the products run on the fp32 matrix cores (see k_gemm_f32). When the row tiles
// alone give few work-groups (decode batches), the columns are split: each
// split writes partial sums and a second kernel adds them in split order, so
// results do not depend on timing.
#include <type_traits>

#include "kmoe_device.h"
#include "kmoe_launch.h"

namespace kmoe {

namespace {

constexpr int TR = 64, KC = 64, PAD = 68;  // PAD: 16-byte aligned LDS rows

// f(std::integral_constant<int, 0>) ... f(std::integral_constant<int, N-1>), in order.
template <int I, int N>
struct Unroll {
  template <class F>
  __device__ __forceinline__ static void run(F &&f) {
    f(std::integral_constant<int, I>{});
    Unroll<I + 1, N>::run(f);
  }
};
template <int N>
struct Unroll<N, N> {
  template <class F>
  __device__ __forceinline__ static void run(F &&) {}
};
template <int N, class F>
__device__ __forceinline__ void unroll(F &&f) {
  Unroll<0, N>::run(f);
}


struct GArgs {
  const uint8_t *w;  // plain
  int64_t rows, cols;
  const float *x;
  int64_t s_rows;
  float *out;
  ExpertTier tier;
  Routing rt;
  int regime;
  int ntt;       // token tiles
  int ks;        // column splits (1: no partial sums)
  int64_t cps;   // column chunks per split
  float *part;      // [ks][n_slots][rows] partial sums when ks > 1
  int64_t n_slots;  // activation rows (plain) or slots (grouped)
  int min_rows;     // grouped: experts with fewer rows are another kernel's
};

enum { G_PLAIN = 0, G_GATE = 1, G_UP = 2, G_DOWN = 3 };

__device__ __forceinline__ bool f32_regime(int regime, int n) {
  return regime == REGIME_EXACT || (regime == REGIME_AVX2 && n >= 4);
}

// 16 consecutive dequantized weights of chunk kc, part p (0..3), of one row
// (Q4_K and Q6_K: GGUF bytes, or tiled rows of nb superblocks when TILED), in
// two steps: load16 issues the loads of the raw bytes, convert16 turns them
// into f32 (so the next chunk's bytes can be in flight meanwhile).
typedef uint32_t u32x4u2 __attribute__((ext_vector_type(4), aligned(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

template <int TYPE, bool TILED>
struct Raw16 {
  u32x4u2 a, b;    // Q4_K: header, nibbles; Q6_K: low bits, high bits; Q8_0: a = the 16 bytes
  uint32_t c, d;   // Q6_K: scale byte, f16 d; Q8_0: f16 d
};
template <bool TILED>
struct Raw16<T_F32, TILED> {
  float4 f[4];
};

template <int TYPE, bool TILED>
__device__ __forceinline__ Raw16<TYPE, TILED> load16(const uint8_t *row, int64_t kc, int p, int64_t nb) {
  Raw16<TYPE, TILED> r;
  if constexpr (TYPE == T_Q4_K) {
    const int64_t sbi = kc >> 2;
    const int k = (int)(kc & 3);
    const uint8_t *sb = row + sbi * (TILED ? 16 : 144);
    r.a = *(const u32x4u2 *)sb;
    r.b = *(const u32x4u2 *)(TILED ? row + tq4_qs_off(nb, sbi, k, p & 1) : sb + 16 + 32 * k + 16 * (p & 1));
  } else if constexpr (TYPE == T_Q6_K) {
    const int64_t sb = kc >> 2;
    const int k = (int)(kc & 3), h = k >> 1, np = k & 1, ri = 2 * np + (p >> 1), l0 = 16 * (p & 1);
    if constexpr (TILED) {  // tq6_piece_off: nibble piece p&1, high-bit piece
      const uint8_t *p0 = row + tq6_piece_off(nb, sb, k, 0);
      const int64_t js = tq6_j_stride(nb, sb);
      r.a = *(const u32x4u2 *)(p0 + (p & 1) * js);
      r.b = *(const u32x4u2 *)(p0 + 2 * js);
      r.c = row[192 * nb + 16 * sb + 4 * k + p];
      r.d = *(const uint16_t *)(row + 208 * nb + 2 * sb);
    } else {
      const uint8_t *blk = row + sb * 210;
      r.a = *(const u32x4u2 *)(blk + 64 * h + 32 * (ri & 1) + l0);
      r.b = *(const u32x4u2 *)(blk + 128 + 32 * h + l0);
      r.c = blk[192 + 8 * h + 2 * ri + (p & 1)];
      r.d = *(const uint16_t *)(blk + 208);
    }
  } else if constexpr (TYPE == T_Q8_0) {
    const uint8_t *blk = row + (2 * kc + (p >> 1)) * 34;
    r.a = *(const u32x4u2 *)(blk + 2 + 16 * (p & 1));
    r.d = *(const uint16_t *)blk;
  } else {  // F32
    const float4 *f = (const float4 *)((const float *)row + kc * 64 + 16 * p);
#pragma unroll
    for (int i = 0; i < 4; ++i) r.f[i] = f[i];
  }
  return r;
}

template <int TYPE, bool TILED>
__device__ __forceinline__ void convert16(const Raw16<TYPE, TILED> &r, int64_t kc, int p, float *o) {
  if constexpr (TYPE == T_Q4_K) {  // quant.rs:138-155: (d*sc)*q - (dmin*m)
    const int k = (int)(kc & 3);
    const float d = f16_bits_to_f32(r.a.x), dmin = f16_bits_to_f32(r.a.x >> 16);
    int sA, mA, sB, mB;
    q4k_scale_min_pair(r.a.y, r.a.z, r.a.w, k, sA, mA, sB, mB);
    const bool hi = p >= 2;
    const float dl = d * (float)(hi ? sB : sA);
    const float ml = dmin * (float)(hi ? mB : mA);
    const uint32_t qw[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t byte = (qw[i >> 2] >> (8 * (i & 3))) & 0xffu;
      const uint32_t nib = hi ? (byte >> 4) : (byte & 0xfu);
      const float t = dl * (float)nib;
      o[i] = t - ml;
    }
  } else if constexpr (TYPE == T_Q6_K) {  // quant.rs:180-201: y = (d * sc) * (q - 32)
    const int k = (int)(kc & 3), np = k & 1, ri = 2 * np + (p >> 1);
    const float ds = f16_bits_to_f32(r.d) * (float)(int8_t)r.c;
    const uint32_t lw[4] = {r.a.x, r.a.y, r.a.z, r.a.w}, hw[4] = {r.b.x, r.b.y, r.b.z, r.b.w};
    // tiled: nibble p>>1 of the nibble piece, bits 4*(p&1)+2*(p>>1) of the
    // high-bit piece; GGUF: nibble np of ql, bits 2*ri of qh
    const int nsh = TILED ? 4 * (p >> 1) : 4 * np;
    const int hsh = TILED ? 4 * (p & 1) + 2 * (p >> 1) : 2 * ri;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t lb = (lw[i >> 2] >> (8 * (i & 3))) & 0xffu, hb = (hw[i >> 2] >> (8 * (i & 3))) & 0xffu;
      const int q = (int)(((lb >> nsh) & 0xfu) | (((hb >> hsh) & 3u) << 4)) - 32;
      o[i] = ds * (float)q;
    }
  } else if constexpr (TYPE == T_Q8_0) {  // quant.rs:82-89: q * d
    const float d = f16_bits_to_f32(r.d);
    const uint32_t qw[4] = {r.a.x, r.a.y, r.a.z, r.a.w};
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = (float)(int8_t)((qw[i >> 2] >> (8 * (i & 3))) & 0xffu) * d;
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[4 * i] = r.f[i].x;
      o[4 * i + 1] = r.f[i].y;
      o[4 * i + 2] = r.f[i].z;
      o[4 * i + 3] = r.f[i].w;
    }
  }
}

// A work-group computes TR = 64 weight rows x TN activation rows (TN = 16 for
// batches below kLargeBatch rows, 64 from there: the weights are dequantized
// once per TN rows). Each K-step of KC = 64 columns dequantizes
// the weight tile into LDS (4 threads per row, 16 weights each; the raw bytes
// of the next PF steps are in flight) and stages the activation tile. Wave w
// then multiplies rows [16w, 16w+16) by the TN activation rows on the fp32
// matrix cores (v_mfma_f32_16x16x4f32, exact fp32 products, fp32 sums): MFMA
// s of the step takes column 16q + s for lane quad q, so each lane reads its
// 16 values with four ds_read_b128. blockIdx.z = ks * ntt + token tile: with
// split-K (ks > 1) the work-group covers column chunks [ks*cps, (ks+1)*cps)
// and writes its partial sums to a.part[ks][slot][r]; k_gemm_f32_reduce then
// adds the splits in ks order.
constexpr int kLargeBatch = 256;  // batches from this size take the TN = 64 kernel

template <int TYPE, int MODE, int TN>
__global__ void __launch_bounds__(256) k_gemm_f32(GArgs a) {
  constexpr bool TL = MODE != G_PLAIN;  // expert tier rows are tiled
  constexpr int PF = TN == 16 ? 4 : 2;
  constexpr int NX = TN / 16;  // activation float4 per thread and step; accumulator tiles per wave
  constexpr int NB = TN == 16 ? 2 : 1;  // LDS buffers
  __shared__ __attribute__((aligned(16))) float Ws[NB][TR][PAD];
  __shared__ __attribute__((aligned(16))) float Xs[NB][TN][PAD];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int64_t rows = a.rows, cols = a.cols;
  const int64_t row_bytes = TYPE == T_Q4_K   ? cols / 256 * 144
                            : TYPE == T_Q6_K ? cols / 256 * 210
                            : TYPE == T_Q8_0 ? cols / 32 * 34
                                             : cols * 4;

  int n;
  int64_t p0 = 0;
  const uint8_t *W = a.w;
  if constexpr (MODE == G_PLAIN) {
    n = (int)a.s_rows;
  } else {
    const int i = blockIdx.y;
    if (i >= *a.rt.n_active) return;
    const int e = a.rt.active[i];
    p0 = a.rt.offsets[e];
    n = (int)(a.rt.offsets[e + 1] - p0);
    if (!f32_regime(a.regime, n) || n < a.min_rows) return;
    W = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[MODE == G_GATE ? 0 : (MODE == G_UP ? 1 : 2)];
  }
  const int ntt = a.ntt, ksn = a.ks;
  const int64_t cps = a.cps;
  const int tile = (int)(blockIdx.z % ntt), ks = (int)(blockIdx.z / ntt);
  const int j0 = tile * TN;
  if (j0 >= n) return;
  const int64_t nchunk = cols / KC;
  const int64_t c_begin = (int64_t)ks * cps;
  const int64_t c_end = c_begin + cps < nchunk ? c_begin + cps : nchunk;
  if (c_begin >= c_end) return;
  const int64_t r0 = (int64_t)blockIdx.x * TR;
  const int64_t nb = cols / 256;

  // activation row of local token j (absolute row index into a.x)
  auto act_row = [&](int j) -> int64_t {
    if constexpr (MODE == G_GATE || MODE == G_UP) return a.rt.perm[p0 + j] / a.rt.topk;
    else if constexpr (MODE == G_DOWN) return p0 + j;
    else return j;
  };

  const int drow = tid >> 2, dpart = tid & 3;
  const int xcol = (tid & 15) * 4;
  const float *xrow[NX];
  f32x4 acc[NX][2];  // TN == 16: even and odd column quads, added at the end; TN == 64: [0] only
  if constexpr (TN == 16) {
    // Rows past the end repeat the last row, token rows past n the last
    // token row, chunks past the split's end its last chunk: every load is
    // unconditional, so the compiler's wait counts stay exact and the ring of
    // PF chunks stays in flight (results of the padding are never stored).
    const uint8_t *wrow = W + (r0 + drow < rows ? r0 + drow : rows - 1) * row_bytes;
    {
      const int xt = tid >> 4;
      xrow[0] = a.x + act_row(j0 + xt < n ? j0 + xt : n - 1) * cols + xcol;
    }
    Raw16<TYPE, TL> raw[PF];
    float4 xr[PF];
    auto fetch = [&](auto D, int64_t kc) {  // ring slot D <- chunk kc
      constexpr int d = decltype(D)::value;
      const int64_t kk = kc < c_end ? kc : c_end - 1;
      raw[d] = load16<TYPE, TL>(wrow, kk, dpart, nb);
      xr[d] = *(const float4 *)(xrow[0] + kk * KC);
    };
    unroll<PF>([&](auto D) { fetch(D, c_begin + decltype(D)::value); });
    // Two LDS buffers: chunk kc is multiplied from buffer (kc - c_begin) & 1
    // while the next chunk is converted into the other, one barrier per
    // chunk. stage: chunk kc (ring slot D) to buffer b, then slot D <- chunk
    // kc + PF.
    auto stage = [&](auto D, int64_t kc, int b) {
      constexpr int d = decltype(D)::value;
      float wv[16];
      convert16<TYPE, TL>(raw[d], kc < c_end ? kc : c_end - 1, dpart, wv);
      const float4 xc = xr[d];
      fetch(D, kc + PF);
      float4 *wd = (float4 *)&Ws[b][drow][dpart * 16];
#pragma unroll
      for (int i = 0; i < 4; ++i) wd[i] = make_float4(wv[4 * i], wv[4 * i + 1], wv[4 * i + 2], wv[4 * i + 3]);
      *(float4 *)&Xs[b][tid >> 4][xcol] = xc;
    };
    acc[0][0] = acc[0][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    stage(std::integral_constant<int, 0>{}, c_begin, 0);
    lds_barrier();
    for (int64_t k0 = c_begin; k0 < c_end; k0 += PF) {
      unroll<PF>([&](auto D) {
        constexpr int d = decltype(D)::value;
        constexpr int b = d & 1;  // (k0 - c_begin) is a multiple of PF, which is even
        if (k0 + d < c_end) {
          const float4 *wa = (const float4 *)&Ws[b][16 * wave + (lane & 15)][16 * (lane >> 4)];
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const float4 A = wa[m];
            const float4 B = ((const float4 *)&Xs[b][lane & 15][16 * (lane >> 4)])[m];
            f32x4 &c = acc[0][m & 1];
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(A.x, B.x, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(A.y, B.y, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(A.z, B.z, c, 0, 0, 0);
            c = __builtin_amdgcn_mfma_f32_16x16x4f32(A.w, B.w, c, 0, 0, 0);
          }
        }
        stage(std::integral_constant<int, (d + 1) % PF>{}, k0 + d + 1, b ^ 1);
        lds_barrier();
      });
    }
  } else {
    bool xvalid[NX];
#pragma unroll
    for (int u = 0; u < NX; ++u) {
      const int xt = (tid >> 4) + 16 * u;
      xvalid[u] = j0 + xt < n;
      xrow[u] = a.x + (xvalid[u] ? act_row(j0 + xt) : 0) * cols + xcol;
    }
    const bool wvalid = r0 + drow < rows;
    const uint8_t *wrow = W + (wvalid ? r0 + drow : 0) * row_bytes;

    // the raw bytes of the next PF column chunks are in flight (a ring of
    // registers, refilled as each chunk is converted)
    Raw16<TYPE, TL> raw[PF];
    float4 xr[PF][NX];
  #pragma unroll
    for (int d = 0; d < PF; ++d) {
  #pragma unroll
      for (int u = 0; u < NX; ++u) xr[d][u] = make_float4(0.f, 0.f, 0.f, 0.f);
      if (c_begin + d < c_end) {
        if (wvalid) raw[d] = load16<TYPE, TL>(wrow, c_begin + d, dpart, nb);
  #pragma unroll
        for (int u = 0; u < NX; ++u)
          if (xvalid[u]) xr[d][u] = *(const float4 *)(xrow[u] + (c_begin + d) * KC);
      }
    }
  #pragma unroll
    for (int u = 0; u < NX; ++u) acc[u][0] = acc[u][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    const float4 *wa = (const float4 *)&Ws[0][16 * wave + (lane & 15)][16 * (lane >> 4)];

    for (int64_t k0 = c_begin; k0 < c_end; k0 += PF) {
  #pragma unroll
      for (int d = 0; d < PF; ++d) {
        const int64_t kc = k0 + d;
        if (kc < c_end) {
          float wv[16];
          if (wvalid) {
            convert16<TYPE, TL>(raw[d], kc, dpart, wv);
          } else {
  #pragma unroll
            for (int i = 0; i < 16; ++i) wv[i] = 0.0f;
          }
          float4 xc[NX];
  #pragma unroll
          for (int u = 0; u < NX; ++u) xc[u] = xr[d][u];
          if (kc + PF < c_end) {  // refill this slot with chunk kc + PF
            if (wvalid) raw[d] = load16<TYPE, TL>(wrow, kc + PF, dpart, nb);
  #pragma unroll
            for (int u = 0; u < NX; ++u)
              if (xvalid[u]) xr[d][u] = *(const float4 *)(xrow[u] + (kc + PF) * KC);
          }
          float4 *wd = (float4 *)&Ws[0][drow][dpart * 16];
  #pragma unroll
          for (int i = 0; i < 4; ++i) wd[i] = make_float4(wv[4 * i], wv[4 * i + 1], wv[4 * i + 2], wv[4 * i + 3]);
  #pragma unroll
          for (int u = 0; u < NX; ++u) *(float4 *)&Xs[0][(tid >> 4) + 16 * u][xcol] = xc[u];
          __syncthreads();
  #pragma unroll
          for (int m = 0; m < 4; ++m) {
            const float4 A = wa[m];
  #pragma unroll
            for (int u = 0; u < NX; ++u) {
              const float4 B = ((const float4 *)&Xs[0][16 * u + (lane & 15)][16 * (lane >> 4)])[m];
              acc[u][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(A.x, B.x, acc[u][0], 0, 0, 0);
              acc[u][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(A.y, B.y, acc[u][0], 0, 0, 0);
              acc[u][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(A.z, B.z, acc[u][0], 0, 0, 0);
              acc[u][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(A.w, B.w, acc[u][0], 0, 0, 0);
            }
          }
          __syncthreads();
        }
      }
    }
  }

  // lane holds rows 4*(lane/16) + v of the wave's 16, activation row
  // 16u + lane%16 of the tile
#pragma unroll
  for (int u = 0; u < NX; ++u) {
    const int j = j0 + 16 * u + (lane & 15);
    if (j >= n) continue;
    const int64_t slot = MODE == G_PLAIN ? (int64_t)j : p0 + j;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t r = r0 + 16 * wave + 4 * (lane >> 4) + v;
      if (r >= rows) continue;
      const float y = TN == 16 ? acc[u][0][v] + acc[u][1][v] : acc[u][0][v];
      if (ksn > 1) {
        a.part[((int64_t)ks * a.n_slots + slot) * rows + r] = y;
      } else if constexpr (MODE == G_PLAIN || MODE == G_GATE || MODE == G_DOWN) {
        a.out[slot * rows + r] = y;
      } else {  // G_UP: SwiGLU with the gate value stored by G_GATE (transformer.rs:558)
        float *o = a.out + slot * rows + r;
        const float g = *o;
        const float den = 1.0f + expf_cr(-g);
        const float q = g / den;
        *o = q * y;
      }
    }
  }
}

// Sum of a group's a.ks partial results in split order, then the mode's store.
template <int MODE>
__global__ void __launch_bounds__(256) k_gemm_f32_reduce(GArgs a) {
  const int64_t rows = a.rows;
  const int64_t r = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (r >= rows) return;
  int n;
  int64_t p0 = 0;
  if constexpr (MODE == G_PLAIN) {
    n = (int)a.s_rows;
  } else {
    const int i = blockIdx.y;
    if (i >= *a.rt.n_active) return;
    const int e = a.rt.active[i];
    p0 = a.rt.offsets[e];
    n = (int)(a.rt.offsets[e + 1] - p0);
    if (!f32_regime(a.regime, n) || n < a.min_rows) return;
  }
  for (int j = 0; j < n; ++j) {
    const int64_t slot = p0 + j;
    float v = a.part[slot * rows + r];
    for (int k = 1; k < a.ks; ++k) v += a.part[((int64_t)k * a.n_slots + slot) * rows + r];
    if constexpr (MODE == G_UP) {
      float *o = a.out + slot * rows + r;
      const float g = *o;
      const float den = 1.0f + expf_cr(-g);
      const float q = g / den;
      *o = q * v;
    } else {
      a.out[slot * rows + r] = v;
    }
  }
}

// Split-K factor: enough work-groups (about 4096, counting the groups that
// exit at once) when the row tiles alone are few; 1 when they are many.
int splits_for(int64_t rows, int64_t cols, int64_t groups) {
  const int64_t tiles = (rows + TR - 1) / TR * groups;
  const int64_t nchunk = cols / KC;
  int64_t ks = (4096 + tiles - 1) / tiles;
  if (ks > nchunk / 8) ks = nchunk / 8;
  if (ks > 16) ks = 16;
  return ks < 1 ? 1 : (int)ks;
}

// Launch shape: tile width TN, token tiles, splits, chunks per split.
void shape_for(int64_t rows, int64_t cols, int groups, int64_t max_rows, int &tn, int &ntt, int &ks, int64_t &cps) {
  tn = max_rows >= kLargeBatch ? 64 : 16;
  ntt = (int)((max_rows + tn - 1) / tn);
  ks = splits_for(rows, cols, (int64_t)groups * ntt);
  const int64_t nchunk = cols / KC;
  cps = (nchunk + ks - 1) / ks;
}

template <int MODE>
hipError_t launch_type(hipStream_t st, int type, GArgs a, int64_t rows_x, int groups, int64_t max_rows,
                       int64_t part_floats) {
  int tn;
  shape_for(a.rows, a.cols, groups, max_rows, tn, a.ntt, a.ks, a.cps);
  if (!a.part || (int64_t)a.ks * a.n_slots * a.rows > part_floats) {
    a.ks = 1;
    a.cps = a.cols / KC;
  }
  const dim3 grid((unsigned)rows_x, (unsigned)groups, (unsigned)(a.ntt * a.ks));
#define KMOE_GEMM(TY)                                                               \
  do {                                                                              \
    if (tn == 16) KMOE_LAUNCH((k_gemm_f32<TY, MODE, 16>), grid, dim3(256), 0, st, a); \
    else KMOE_LAUNCH((k_gemm_f32<TY, MODE, 64>), grid, dim3(256), 0, st, a);         \
  } while (0)
  switch (type) {
    case T_Q4_K: KMOE_GEMM(T_Q4_K); break;
    case T_Q8_0: KMOE_GEMM(T_Q8_0); break;
    case T_Q6_K: KMOE_GEMM(T_Q6_K); break;
    case T_F32: KMOE_GEMM(T_F32); break;
    default: return hipErrorInvalidValue;
  }
#undef KMOE_GEMM
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || a.ks == 1) return e;
  KMOE_LAUNCH((k_gemm_f32_reduce<MODE>), dim3((unsigned)((a.rows + 255) / 256), (unsigned)groups), dim3(256), 0,
              st, a);
  return hipGetLastError();
}

}  // namespace

int64_t gemm_f32_part_floats(int64_t rows, int64_t cols, int64_t groups, int64_t max_rows, int64_t n_slots) {
  if (rows <= 0 || cols % KC != 0 || max_rows <= 0) return 0;
  int tn, ntt, ks;
  int64_t cps;
  shape_for(rows, cols, (int)groups, max_rows, tn, ntt, ks, cps);
  return ks > 1 ? (int64_t)ks * n_slots * rows : 0;
}

hipError_t launch_matmul_f32(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols, const float *x,
                             int64_t s_rows, float *out, float *part, int64_t part_floats) {
  if (rows == 0 || s_rows == 0) return hipSuccess;
  if (cols % KC != 0) return hipErrorInvalidValue;
  GArgs a{};
  a.w = w;
  a.rows = rows;
  a.cols = cols;
  a.x = x;
  a.s_rows = s_rows;
  a.out = out;
  a.part = part;
  a.n_slots = s_rows;
  return launch_type<G_PLAIN>(st, type, a, (rows + TR - 1) / TR, 1, s_rows, part_floats);
}

hipError_t launch_moe_f32(hipStream_t st, int mode, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                          const Routing &rt, int regime, int max_active, int64_t max_rows_per_expert,
                          int64_t n_slots, const float *x, float *out, float *part, int64_t part_floats,
                          int min_rows) {
  if (rows == 0 || max_active == 0 || max_rows_per_expert == 0 || max_rows_per_expert < min_rows) return hipSuccess;
  if (cols % KC != 0) return hipErrorInvalidValue;
  GArgs a{};
  a.min_rows = min_rows;
  a.rows = rows;
  a.cols = cols;
  a.x = x;
  a.out = out;
  a.tier = tier;
  a.rt = rt;
  a.regime = regime;
  a.part = part;
  a.n_slots = n_slots;
  const int64_t rx = (rows + TR - 1) / TR;
  switch (mode) {
    case 0: return launch_type<G_GATE>(st, type, a, rx, max_active, max_rows_per_expert, part_floats);
    case 1: return launch_type<G_UP>(st, type, a, rx, max_active, max_rows_per_expert, part_floats);
    case 2: return launch_type<G_DOWN>(st, type, a, rx, max_active, max_rows_per_expert, part_floats);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace kmoe
