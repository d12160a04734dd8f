// kmoe_f32rows.hip — the reference's f32 regime (quant.rs:242-260: weights
// dequantized to f32, multiplied with f32 activations; avx2.rs:230-308) for
// experts that hold a few token rows (decode batches), over the expert tier's
// tiled Q4_K rows.
//
// Streaming instead of staging: a work-group takes a block of 16*RT weight
// rows of one expert and runs over the whole rows once, its four waves taking
// a quarter of the superblocks each (split K). In a wave, lane l owns row
// 16*i + l % 16 of row tile i (i < RT) and, in every 64-column step (a
// quarter k of a superblock), the 16 columns 16*(l / 16) .. +15. Those 16
// weights are one tiled nibble chunk (quarter k, half (l / 16) & 1; low
// nibbles for the first two lane groups, high for the others), dequantized in
// registers as dequant_row does it (quant.rs:138-155: (d*sc)*q - dmin*m, a
// multiply and a subtract, so every weight equals the reference's f32 value;
// d*sc and dmin*m of the lane's four sub-blocks are formed once per
// superblock) and fed to v_mfma_f32_16x16x4f32 as its A operand: MFMA m of the
// step takes column 16*(l/16) + m for lane quad l/16. The B operand (the token
// rows, read from L2: token l % 16, the same 16 columns) is shared by the RT
// row tiles. The products are exact and the sums fp32 in the matrix core's
// order (a few ulp from gemm_f32's 8-lane chains); the four waves' partial
// sums are added in wave order through LDS at the end, so results do not
// depend on timing. Two steps' nibble chunks and token values and the next
// superblock's heads are in flight while a step is multiplied; loads are
// unconditional (rows, tokens and steps past the end are clamped, their
// results never used) and the last two steps issue none.
//
// gate/up: both matrices' rows per lane, so the lane that finishes a row tile
// holds gate and up of the same (row, token) elements and applies SwiGLU
// (transformer.rs:558) in registers. down: one matrix.
#include <type_traits>

#include "kmoe_device.h"
#include "kmoe_launch.h"
#include "kmoe_tq4.h"

namespace kmoe {

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));

struct F32RowsArgs {
  ExpertTier tier;
  Routing rt;
  int64_t rows, cols;  // weight rows and columns of one part
  const float *x;      // gate/up: the layer input [S, cols]; down: h [slots, cols]
  float *out;          // gate/up: h [slots, rows]; down: y [slots, rows]
  int regime;
  int min_rows, max_rows;  // experts with min_rows..max_rows rows on the f32 path
};

__device__ __forceinline__ bool rows_f32_regime(int regime, int n) {
  return regime == REGIME_EXACT || (regime == REGIME_AVX2 && n >= 4);
}

template <int MODE, int TT, int RT>
__global__ void __launch_bounds__(256, 2) k_f32_rows(F32RowsArgs a) {
  constexpr int NM = MODE == 0 ? 2 : 1;  // matrices per lane: gate and up, or down
  constexpr int NACC = RT * NM * TT;     // accumulator tiles per wave
  __shared__ __attribute__((aligned(16))) f32x4 red[3][NACC][64];  // waves 1..3's partial sums
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i_act = blockIdx.y;
  if (i_act >= *a.rt.n_active) return;
  const int e = a.rt.active[i_act];
  const int64_t p0 = a.rt.offsets[e];
  const int n = (int)(a.rt.offsets[e + 1] - p0);
  if (n < a.min_rows || n > a.max_rows || !rows_f32_regime(a.regime, n)) return;
  const int64_t cols = a.cols, nb = cols / 256, rows = a.rows, row_bytes = nb * 144;
  const int r16 = lane & 15, g = lane >> 4;
  const bool hi = g >= 2;  // high nibbles: the odd sub-block of each quarter
  const int64_t r0 = (int64_t)blockIdx.x * (16 * RT);
  const uint8_t *E = a.tier.base + (int64_t)e * a.tier.stride;
  const uint8_t *Wm[RT][NM];
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    const int64_t r = r0 + 16 * i + r16 < rows ? r0 + 16 * i + r16 : rows - 1;
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) Wm[i][mt] = E + a.tier.off[MODE == 0 ? mt : 2] + r * row_bytes;
  }
  // the token row of lane l in tile t (B operand column l % 16)
  const float *xr[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int tk = 16 * t + r16 < n ? 16 * t + r16 : n - 1;
    const int64_t src = MODE == 0 ? (int64_t)(a.rt.perm[p0 + tk] / (uint32_t)a.rt.topk) : p0 + tk;
    xr[t] = a.x + src * cols + 16 * g;
  }
  // this wave's superblocks [b0, b0 + nbw), its steps j = 4 * (b - b0) + k
  const int nbq = (int)((nb + 3) / 4);
  const int b0 = wave * nbq;
  const int nbw = b0 >= nb ? 0 : ((int)nb - b0 < nbq ? (int)nb - b0 : nbq);
  const int nsj = 4 * nbw;
  f32x4 acc[RT][NM][TT];
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
#pragma unroll
      for (int t = 0; t < TT; ++t) acc[i][mt][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  if (nbw > 0) {
    u32x4 q[2][RT][NM];
    float4 xv[2][TT][4];
    u32x4 hd[RT][NM];           // heads of the next superblock
    float dl[RT][NM][4], ml[RT][NM][4];  // d*sc, dmin*m of the lane's sub-block in each quarter
    auto load = [&](int j, int slot) {
      const int jc = j < nsj ? j : nsj - 1;
      const int64_t b = b0 + (jc >> 2);
      const int k = jc & 3;
      const int s = 4 * (int)b + k;
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) q[slot][i][mt] = *(const u32x4 *)(Wm[i][mt] + tq4_qs_off(nb, b, k, g & 1));
#pragma unroll
      for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) xv[slot][t][u] = *(const float4 *)(xr[t] + 64 * s + 4 * u);
    };
    auto load_heads = [&](int bl) {  // superblock b0 + bl (clamped)
      const int64_t b = b0 + (bl < nbw ? bl : nbw - 1);
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) hd[i][mt] = *(const u32x4 *)(Wm[i][mt] + 16 * b);
    };
    auto scales = [&]() {  // scale_min_k4 of the heads (quant.rs:54-61), per quarter
#pragma unroll
      for (int i = 0; i < RT; ++i)
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) {
          const u32x4 h = hd[i][mt];
          const float d = f16_bits_to_f32(h.x), dmin = f16_bits_to_f32(h.x >> 16);
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            int sA, mA, sB, mB;
            q4k_scale_min_pair(h.y, h.z, h.w, k, sA, mA, sB, mB);
            dl[i][mt][k] = d * (float)(hi ? sB : sA);
            ml[i][mt][k] = dmin * (float)(hi ? mB : mA);
          }
        }
    };
    auto step = [&](int slot, int k) {
#pragma unroll
      for (int i = 0; i < RT; ++i) {
        float w[NM][16];
#pragma unroll
        for (int mt = 0; mt < NM; ++mt) {
          const uint32_t qw[4] = {q[slot][i][mt].x, q[slot][i][mt].y, q[slot][i][mt].z, q[slot][i][mt].w};
          const float dk = dl[i][mt][k], mk = ml[i][mt][k];
#pragma unroll
          for (int c = 0; c < 16; ++c) {
            const uint32_t byte = (qw[c >> 2] >> (8 * (c & 3))) & 0xffu;
            const uint32_t nib = hi ? (byte >> 4) : (byte & 0xfu);
            const float tq = dk * (float)nib;
            w[mt][c] = tq - mk;
          }
        }
        // consecutive MFMAs alternate between independent accumulators
#pragma unroll
        for (int m = 0; m < 16; ++m)
#pragma unroll
          for (int t = 0; t < TT; ++t) {
            const float4 xq = xv[slot][t][m >> 2];
            const float b = (m & 3) == 0 ? xq.x : ((m & 3) == 1 ? xq.y : ((m & 3) == 2 ? xq.z : xq.w));
#pragma unroll
            for (int mt = 0; mt < NM; ++mt)
              acc[i][mt][t] = __builtin_amdgcn_mfma_f32_16x16x4f32(w[mt][m], b, acc[i][mt][t], 0, 0, 0);
          }
      }
    };
    // superblock loop: steps (k = 0, 1) from slots 0, 1, refilled with k = 2, 3,
    // then those; the next superblock's heads load during its predecessor
    load_heads(0);
    load(0, 0);
    load(1, 1);
    int bl = 0;
    for (; bl + 1 < nbw; ++bl) {
      const int j = 4 * bl;
      scales();
      load_heads(bl + 1);
      step(0, 0);
      load(j + 2, 0);
      step(1, 1);
      load(j + 3, 1);
      step(0, 2);
      load(j + 4, 0);
      step(1, 3);
      load(j + 5, 1);
    }
    // the last superblock: no loads after its quarters 2 and 3
    scales();
    step(0, 0);
    load(4 * bl + 2, 0);
    step(1, 1);
    load(4 * bl + 3, 1);
    step(0, 2);
    step(1, 3);
  }
  // partial sums of waves 1..3 to LDS; wave 0 adds them in wave order
  if (wave > 0) {
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int mt = 0; mt < NM; ++mt)
#pragma unroll
        for (int t = 0; t < TT; ++t) red[wave - 1][(i * NM + mt) * TT + t][lane] = acc[i][mt][t];
  }
  __syncthreads();
  if (wave != 0) return;
#pragma unroll
  for (int w = 0; w < 3; ++w)
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int mt = 0; mt < NM; ++mt)
#pragma unroll
        for (int t = 0; t < TT; ++t) acc[i][mt][t] += red[w][(i * NM + mt) * TT + t][lane];
  // lane l holds rows 4*(l/16) + v of each row tile, token 16t + l % 16
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int tk = 16 * t + r16;
    if (tk >= n) continue;
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t rw = r0 + 16 * i + 4 * g + v;
        if (rw >= rows) continue;
        if constexpr (MODE == 0) {  // SwiGLU: g / (1 + exp(-g)) * u
          const float gv = acc[i][0][t][v], uv = acc[i][1][t][v];
          const float den = 1.0f + expf_cr(-gv);
          const float qv = gv / den;
          a.out[(p0 + tk) * rows + rw] = qv * uv;
        } else {
          a.out[(p0 + tk) * rows + rw] = acc[i][0][t][v];
        }
      }
  }
}

}  // namespace

bool f32_rows_supported(int type, int64_t rows, int64_t cols) {
  return type == T_Q4_K && rows > 0 && cols > 0 && cols % 256 == 0;
}

hipError_t launch_f32_rows(hipStream_t st, int mode, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                           const Routing &rt, int regime, int max_active, int min_rows, int max_rows,
                           const float *x, float *out) {
  if (!f32_rows_supported(type, rows, cols) || max_rows > 32) return hipErrorNotSupported;
  if (rows == 0 || max_active == 0 || max_rows < min_rows) return hipSuccess;
  F32RowsArgs a{};
  a.tier = tier;
  a.rt = rt;
  a.rows = rows;
  a.cols = cols;
  a.x = x;
  a.out = out;
  a.regime = regime;
  // row tiles per work-group: gate/up 2 for one token tile over wide FFNs
  // (Mixtral's 14336 rows), else 1; down 1 (its rows are few and long:
  // 16-row work-groups keep every CU busy when a single expert is on this
  // path). Measured, Qwen3 shape at 16 tokens (768 rows): gate/up 35 -> 27 µs
  // with one row tile, the step 105 -> 100 µs.
#define KMOE_F32R(M, T, R)                                                                                 \
  KMOE_LAUNCH((k_f32_rows<M, T, R>), dim3((unsigned)((rows + 16 * R - 1) / (16 * R)), (unsigned)max_active), \
              dim3(256), 0, st, a)
  a.min_rows = min_rows;
  a.max_rows = max_rows < 16 ? max_rows : 16;
  if (a.min_rows <= a.max_rows) {
    if (mode == 0 && rows > 4096) KMOE_F32R(0, 1, 2);
    else if (mode == 0) KMOE_F32R(0, 1, 1);
    else KMOE_F32R(1, 1, 1);
  }
  if (max_rows > 16) {
    a.min_rows = min_rows > 17 ? min_rows : 17;
    a.max_rows = max_rows;
    if (mode == 0) KMOE_F32R(0, 2, 1);
    else KMOE_F32R(1, 2, 1);
  }
#undef KMOE_F32R
  return hipGetLastError();
}

}  // namespace kmoe
