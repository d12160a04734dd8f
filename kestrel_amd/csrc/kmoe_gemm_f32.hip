// kmoe_gemm_f32.hip — the reference's batched regime: weights dequantized to
// f32 and multiplied with f32 activations (quant.rs:242-260).
//
// Dequantization is dequant_row (quant.rs:82-89 for Q8_0: q * d; quant.rs:
// 138-155 for Q4_K: (d*sc)*q - (dmin*m), one multiply and one subtract, no
// FMA), so every weight value equals the reference's bit for bit. The dot
// products accumulate with FMA in a different order from gemm_f32's 8-lane
// chains (avx2.rs:230-286): results agree to a few f32 ulp of the sum.
//
// Tiling: a work-group computes 64 weight rows x 16 activation rows. Each
// K-step of 64 columns dequantizes the weight tile into LDS (4 threads per
// row, 16 weights each) and stages the activation tile; each thread then owns
// 4 rows x 1 activation row.
#include "kmoe_device.h"
#include "kmoe_launch.h"

namespace kmoe {

namespace {

constexpr int TR = 64, TT = 16, KC = 64, PAD = 65;

struct GArgs {
  const uint8_t *w;  // plain
  int64_t rows, cols;
  const float *x;
  int64_t s_rows;
  float *out;
  ExpertTier tier;
  Routing rt;
  int regime;
};

enum { G_PLAIN = 0, G_GATE = 1, G_UP = 2, G_DOWN = 3 };

__device__ __forceinline__ bool f32_regime(int regime, int n) {
  return regime == REGIME_EXACT || (regime == REGIME_AVX2 && n >= 4);
}

// 16 consecutive dequantized weights of chunk kc, part p (0..3), of one row
// (Q4_K and Q6_K: GGUF bytes, or tiled rows of nb superblocks when TILED).
template <int TYPE, bool TILED>
__device__ __forceinline__ void dequant16(const uint8_t *row, int64_t kc, int p, int64_t nb, float *o) {
  if constexpr (TYPE == T_Q4_K) {
    const int64_t sbi = kc >> 2;
    const uint8_t *sb = row + sbi * (TILED ? 16 : 144);
    const int k = (int)(kc & 3);
    const uint4 hdr = *(const uint4 *)sb;
    const float d = f16_bits_to_f32(hdr.x), dmin = f16_bits_to_f32(hdr.x >> 16);
    int sA, mA, sB, mB;
    q4k_scale_min_pair(hdr.y, hdr.z, hdr.w, k, sA, mA, sB, mB);
    const bool hi = p >= 2;
    const float dl = d * (float)(hi ? sB : sA);
    const float ml = dmin * (float)(hi ? mB : mA);
    const uint8_t *qp = TILED ? row + tq4_qs_off(nb, sbi, k, p & 1) : sb + 16 + 32 * k + 16 * (p & 1);
    const uint4 q = *(const uint4 *)qp;
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const uint32_t byte = (qw[i >> 2] >> (8 * (i & 3))) & 0xffu;
      const uint32_t nib = hi ? (byte >> 4) : (byte & 0xfu);
      const float t = dl * (float)nib;
      o[i] = t - ml;
    }
  } else if constexpr (TYPE == T_Q6_K) {  // quant.rs:180-201: y = (d * sc) * (q - 32)
    // chunk kc = quarter k of superblock kc/4 (half h, nibble np); part p is
    // weights 16*(p&1).. of row ri = 2*np + (p>>1) of the half
    typedef uint32_t u32x4u2 __attribute__((ext_vector_type(4), aligned(2)));
    const int64_t sb = kc >> 2;
    const int k = (int)(kc & 3), h = k >> 1, np = k & 1, ri = 2 * np + (p >> 1), l0 = 16 * (p & 1);
    if constexpr (TILED) {  // tq6_piece_off: nibble piece p&1 (nibble p>>1), high-bit piece (nibble p&1)
      const uint8_t *p0 = row + tq6_piece_off(nb, sb, k, 0);
      const int64_t js = tq6_j_stride(nb, sb);
      const float d = f16_bits_to_f32((uint32_t)row[208 * nb + 2 * sb] | ((uint32_t)row[208 * nb + 2 * sb + 1] << 8));
      const float ds = d * (float)(int8_t)row[192 * nb + 16 * sb + 4 * k + p];
      const u32x4u2 nv = *(const u32x4u2 *)(p0 + (p & 1) * js);
      const u32x4u2 hv = *(const u32x4u2 *)(p0 + 2 * js);
      const uint32_t nw[4] = {nv.x, nv.y, nv.z, nv.w}, hw[4] = {hv.x, hv.y, hv.z, hv.w};
      const int nsh = 4 * (p >> 1), hsh = 4 * (p & 1) + 2 * (p >> 1);
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t nb8 = (nw[i >> 2] >> (8 * (i & 3))) & 0xffu, hb8 = (hw[i >> 2] >> (8 * (i & 3))) & 0xffu;
        const int q = (int)(((nb8 >> nsh) & 0xfu) | (((hb8 >> hsh) & 3u) << 4)) - 32;
        o[i] = ds * (float)q;
      }
    } else {
      const uint8_t *blk = row + sb * 210;
      const float d = f16_bits_to_f32((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
      const float ds = d * (float)(int8_t)blk[192 + 8 * h + 2 * ri + (p & 1)];
      const u32x4u2 ql = *(const u32x4u2 *)(blk + 64 * h + 32 * (ri & 1) + l0);
      const u32x4u2 qh = *(const u32x4u2 *)(blk + 128 + 32 * h + l0);
      const uint32_t lw[4] = {ql.x, ql.y, ql.z, ql.w}, hw[4] = {qh.x, qh.y, qh.z, qh.w};
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const uint32_t lb = (lw[i >> 2] >> (8 * (i & 3))) & 0xffu, hb = (hw[i >> 2] >> (8 * (i & 3))) & 0xffu;
        const int q = (int)((np ? (lb >> 4) : (lb & 0xfu)) | (((hb >> (2 * ri)) & 3u) << 4)) - 32;
        o[i] = ds * (float)q;
      }
    }
  } else if constexpr (TYPE == T_Q8_0) {
    const int64_t b = 2 * kc + (p >> 1);
    const uint8_t *blk = row + b * 34;
    const float d = f16_bits_to_f32((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    const int8_t *qs = (const int8_t *)(blk + 2 + 16 * (p & 1));
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = (float)qs[i] * d;
  } else {  // F32
    const float *f = (const float *)row + kc * 64 + 16 * p;
#pragma unroll
    for (int i = 0; i < 16; ++i) o[i] = f[i];
  }
}

template <int TYPE, int MODE>
__global__ void __launch_bounds__(256) k_gemm_f32(GArgs a) {
  __shared__ float Ws[TR][PAD];
  __shared__ float Xs[TT][PAD];
  const int tid = threadIdx.x;
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
    if (!f32_regime(a.regime, n)) return;
    W = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[MODE == G_GATE ? 0 : (MODE == G_UP ? 1 : 2)];
  }
  const int j0 = blockIdx.z * TT;
  if (j0 >= n) return;
  const int64_t r0 = (int64_t)blockIdx.x * TR;

  // activation row of local token j (absolute row index into a.x)
  auto act_row = [&](int j) -> int64_t {
    if constexpr (MODE == G_GATE || MODE == G_UP) return a.rt.perm[p0 + j] / a.rt.topk;
    else if constexpr (MODE == G_DOWN) return p0 + j;
    else return j;
  };

  const int tok = tid & 15, rg = tid >> 4;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int drow = tid >> 2, dpart = tid & 3;
  const int xtok = tid >> 4, xcol = (tid & 15) * 4;
  const bool xvalid = j0 + xtok < n;
  const int64_t xr = xvalid ? act_row(j0 + xtok) : 0;
  const float *xrow = a.x + xr * cols;
  const bool wvalid = r0 + drow < rows;
  const uint8_t *wrow = W + (r0 + drow) * row_bytes;

  for (int64_t kc = 0; kc < cols / KC; ++kc) {
    float wv[16];
    if (wvalid) {
      dequant16<TYPE, MODE != G_PLAIN>(wrow, kc, dpart, cols / 256, wv);
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) wv[i] = 0.0f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Ws[drow][dpart * 16 + i] = wv[i];
    float4 xv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (xvalid) xv = *(const float4 *)(xrow + kc * KC + xcol);
    Xs[xtok][xcol + 0] = xv.x;
    Xs[xtok][xcol + 1] = xv.y;
    Xs[xtok][xcol + 2] = xv.z;
    Xs[xtok][xcol + 3] = xv.w;
    __syncthreads();
#pragma unroll 8
    for (int kk = 0; kk < KC; ++kk) {
      const float xk = Xs[tok][kk];
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = fmaf(Ws[4 * rg + i][kk], xk, acc[i]);
    }
    __syncthreads();
  }

  const int j = j0 + tok;
  if (j >= n) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t r = r0 + 4 * rg + i;
    if (r >= rows) continue;
    if constexpr (MODE == G_PLAIN) {
      a.out[(int64_t)j * rows + r] = acc[i];
    } else if constexpr (MODE == G_GATE || MODE == G_DOWN) {
      a.out[(p0 + j) * rows + r] = acc[i];
    } else {  // G_UP: SwiGLU with the gate value stored by G_GATE (transformer.rs:558)
      float *o = a.out + (p0 + j) * rows + r;
      const float g = *o;
      const float den = 1.0f + expf_cr(-g);
      const float q = g / den;
      *o = q * acc[i];
    }
  }
}

template <int MODE>
hipError_t launch_type(hipStream_t st, int type, const GArgs &a, dim3 grid) {
  switch (type) {
    case T_Q4_K:
      KMOE_LAUNCH((k_gemm_f32<T_Q4_K, MODE>), grid, dim3(256), 0, st, a);
      break;
    case T_Q8_0:
      KMOE_LAUNCH((k_gemm_f32<T_Q8_0, MODE>), grid, dim3(256), 0, st, a);
      break;
    case T_Q6_K:
      KMOE_LAUNCH((k_gemm_f32<T_Q6_K, MODE>), grid, dim3(256), 0, st, a);
      break;
    case T_F32:
      KMOE_LAUNCH((k_gemm_f32<T_F32, MODE>), grid, dim3(256), 0, st, a);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_matmul_f32(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols, const float *x,
                             int64_t s_rows, float *out) {
  if (rows == 0 || s_rows == 0) return hipSuccess;
  if (cols % KC != 0) return hipErrorInvalidValue;
  GArgs a{};
  a.w = w;
  a.rows = rows;
  a.cols = cols;
  a.x = x;
  a.s_rows = s_rows;
  a.out = out;
  dim3 grid((unsigned)((rows + TR - 1) / TR), 1, (unsigned)((s_rows + TT - 1) / TT));
  return launch_type<G_PLAIN>(st, type, a, grid);
}

hipError_t launch_moe_f32(hipStream_t st, int mode, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                          const Routing &rt, int regime, int max_active, int64_t max_rows_per_expert,
                          const float *x, float *out) {
  if (rows == 0 || max_active == 0 || max_rows_per_expert == 0) return hipSuccess;
  if (cols % KC != 0) return hipErrorInvalidValue;
  GArgs a{};
  a.rows = rows;
  a.cols = cols;
  a.x = x;
  a.out = out;
  a.tier = tier;
  a.rt = rt;
  a.regime = regime;
  dim3 grid((unsigned)((rows + TR - 1) / TR), (unsigned)max_active,
            (unsigned)((max_rows_per_expert + TT - 1) / TT));
  switch (mode) {
    case 0: return launch_type<G_GATE>(st, type, a, grid);
    case 1: return launch_type<G_UP>(st, type, a, grid);
    case 2: return launch_type<G_DOWN>(st, type, a, grid);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace kmoe
