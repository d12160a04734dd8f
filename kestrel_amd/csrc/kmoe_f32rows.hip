// kmoe_f32rows.hip — the reference's f32 regime (quant.rs:242-260: weights
// dequantized to f32, multiplied with f32 activations; avx2.rs:230-308) on
// Q4_K rows: the expert tier's tiled rows of the experts in the regime
// (blocks of up to 64 token rows per expert, each weight streamed once per
// block; gate and up in one launch with SwiGLU, transformer.rs:558, in the
// epilogue, down in another), and plain GGUF rows for quant::matmul itself and
// a shared expert's gate/up.
#include "kmoe_device.h"
#include "kmoe_launch.h"

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
  int ranked;              // blockIdx.y ranks the experts in that range, not the whole active list
  const uint8_t *pw;       // plain modes: GGUF rows [rows, cols] (16-byte aligned); mode 3: the gate rows
  const uint8_t *pw2;      // mode 3: the up rows
  int64_t s_rows;          // plain mode: activation rows of x
};

__device__ __forceinline__ bool rows_f32_regime(int regime, int n) {
  return regime == REGIME_EXACT || (regime == REGIME_AVX2 && n >= 4);
}

// The products run on the matrix cores' bf16 path, exactly.
// For sub-block j of a superblock, dequant_row's weights are w = A_j*q - B_j
// (A_j = d*sc_j, B_j = dmin*m_j, q the 4-bit value; quant.rs:138-155), so
// sum_k w_k x_k = A_j * sum_k q_k x_k - B_j * sum_k x_k. q is exact in bf16,
// and each x splits exactly into three bf16 pieces (x1 = x with its low 16
// bits cleared, x2 the same of x - x1, x3 = x - x1 - x2, which has at most 8
// significant bits), so v_mfma_f32_16x16x32_bf16 (K = 32, one sub-block)
// forms the exact products q*x1, q*x2, q*x3 and sums them in fp32; the
// sub-block's result then joins the row's sum as fma(A_j, P, y) and
// fma(-B_j, S_j, y), S_j the token's fp32 sum of the sub-block's x. The
// result is the f32 regime's within a few fp32 roundings (the reference's
// own sum runs in another order too).
//
// Work-group: 16 * (4 / KW) weight rows of one expert (or of the plain
// matrix) by a block of up to 16 * TT of its token rows (blockIdx.z); wave w
// takes row tile w / KW and, of every KW consecutive superblocks, the
// (w % KW)-th (KW = 1 for wide parts; narrow ones split the superblocks over
// the waves so that enough work-groups run). Per round of KW
// superblocks the 256 threads split the tokens' x into LDS (three bf16 planes
// per superblock, and the sub-block sums), each wave turns its rows' heads
// into A_j, B_j in LDS, and for every quarter k a lane converts its 8 nibble
// bytes of row 16 * tile + l % 16 (bytes 8*(l/16) .. +7 of the quarter's 32:
// elements 8*(l/16) .. +7 of sub-blocks 2k (low nibbles) and 2k+1 (high)) to
// the MFMA's A operand; the B operand of lane l is token l % 16's pieces of
// the same elements. Lane l ends with rows 16 * tile + 4*(l/16) + v, v < 4,
// of token l % 16 of each token tile; the KW waves of a tile add their sums
// through LDS in wave order at the end. The next round's x, nibbles and
// heads are loaded while the current one is multiplied.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
constexpr int kX3Pad = 264;           // bf16 per token row of a plane in LDS (256 + 8: two-way bank conflicts at most)

// Pairs of f32 whose low 16 bits are zero, as one dword of two bf16 (first low).
__device__ __forceinline__ uint32_t bf16_pair(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

// MODE 0: grouped gate/up + SwiGLU, 1: grouped down (the expert tier's tiled
// rows, routed token slots); 2: plain GGUF rows against s_rows activation rows
// (quant::matmul's f32 regime, quant.rs:242-260); 3: two plain GGUF matrices
// (gate, up) and SwiGLU (a shared expert's front, transformer.rs:572-587).
template <int MODE, int TT, int KW>
__global__ void __launch_bounds__(256, TT * KW > 2 ? 1 : 2) k_f32x3_rows(F32RowsArgs a) {
  constexpr bool PLAIN = MODE >= 2;
  constexpr int NM = MODE == 0 || MODE == 3 ? 2 : 1;
  constexpr int RT = 4 / KW;  // row tiles per work-group
  __shared__ __attribute__((aligned(16))) uint16_t xp[KW][3][TT * 16][kX3Pad];  // x pieces by token, column
  __shared__ float xs[KW][TT * 16][8];                                          // sub-block sums of x by token
  __shared__ __attribute__((aligned(16))) float ab[4][NM][2][8][16];             // wave, matrix, A|B, sub-block, row
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = wave / KW, kg = wave % KW;
  // blockIdx.y indexes the active list, or (ranked) ranks the experts this
  // launch takes (row count in min_rows..max_rows, f32 regime) in the list's
  // order: every wave finds the same one with ballots over the list.
  int e = -1;
  if (PLAIN) {
    e = 0;
  } else if (!a.ranked) {  // the grid covers the whole active list
    if ((int)blockIdx.y < *a.rt.n_active) e = a.rt.active[blockIdx.y];
  } else {
    const int na = *a.rt.n_active;
    int want = (int)blockIdx.y;
    for (int base = 0; base < na; base += 64) {
      const int i = base + lane;
      int ei = 0;
      bool in = false;
      if (i < na) {
        ei = a.rt.active[i];
        const int ni = (int)(a.rt.offsets[ei + 1] - a.rt.offsets[ei]);
        in = ni >= a.min_rows && ni <= a.max_rows && rows_f32_regime(a.regime, ni);
      }
      const uint64_t m = __ballot(in);
      const int cnt = __popcll(m);
      if (want < cnt) {
        const int below = (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
        const bool hit = in && below == want;
        const uint64_t hm = __ballot(hit);
        e = __builtin_amdgcn_readlane(ei, (int)__builtin_ctzll(hm));
        break;
      }
      want -= cnt;
    }
  }
  if (e < 0) return;
  const int64_t p0 = PLAIN ? 0 : a.rt.offsets[e];
  const int n = PLAIN ? (int)a.s_rows : (int)(a.rt.offsets[e + 1] - p0);
  if (!PLAIN && (n < a.min_rows || n > a.max_rows || !rows_f32_regime(a.regime, n))) return;
  const int tok0 = (int)blockIdx.z * 16 * TT;  // this work-group's block of the expert's token rows
  if (tok0 >= n) return;
  const int nbt = n - tok0 < 16 * TT ? n - tok0 : 16 * TT;
  const int ntt = (nbt + 15) / 16;  // token tiles of the block (<= TT; every tile is full below four)
  const int64_t cols = a.cols, nb = cols / 256, rows = a.rows, row_bytes = nb * 144;
  const int r16 = lane & 15, g = lane >> 4;
  const int64_t rbase = (int64_t)blockIdx.x * (16 * RT) + 16 * tile;
  const uint8_t *E = PLAIN ? a.pw : a.tier.base + (int64_t)e * a.tier.stride;
  const uint8_t *Wr[NM];  // this lane's A-operand row
#pragma unroll
  for (int mt = 0; mt < NM; ++mt) {
    const int64_t r = rbase + r16 < rows ? rbase + r16 : rows - 1;
    Wr[mt] = (PLAIN && mt == 1 ? a.pw2 : E) + (PLAIN ? 0 : a.tier.off[MODE == 0 ? mt : 2]) + r * row_bytes;
  }
  const uint8_t *Wh = Wr[NM == 2 ? g >> 1 : 0];
  // the split: thread tid takes token tid / 16 (+16t) and columns 16*(tid % 16) .. +15 of each of the round's superblocks
  const int stok = tid >> 4, sc16 = tid & 15;
  const float *xrow[TT];
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int tk = tok0 + (16 * t + stok < nbt ? 16 * t + stok : nbt - 1);
    const int64_t src = MODE == 0 ? (int64_t)(a.rt.perm[p0 + tk] / (uint32_t)a.rt.topk) : p0 + tk;
    xrow[t] = a.x + src * cols + 16 * sc16;
  }
  float4 xv[KW][TT][4];
  uint2 wq[NM][4];  // this wave's superblock: nibble bytes of the 4 quarters
  u32x4v hd;        // and the head of this lane's row of matrix g / 2 (gate/up) or of down
  auto load_round = [&](int64_t b0) {
#pragma unroll
    for (int q = 0; q < KW; ++q) {
      const int64_t b = b0 + q < nb ? b0 + q : nb - 1;
#pragma unroll
      for (int t = 0; t < TT; ++t)
#pragma unroll
        for (int u = 0; u < 4; ++u) xv[q][t][u] = *(const float4 *)(xrow[t] + 256 * b + 4 * u);
    }
    const int64_t b = b0 + kg < nb ? b0 + kg : nb - 1;
#pragma unroll
    for (int mt = 0; mt < NM; ++mt) {
#pragma unroll
      for (int k = 0; k < 4; ++k)  // bytes 8g .. 8g+7 of quarter k's 32 (GGUF: at 16 + 32k in the superblock)
        wq[mt][k] = *(const uint2 *)(Wr[mt] + (PLAIN ? 144 * b + 16 + 32 * k + 8 * g
                                                     : tq4_qs_off(nb, b, k, g >> 1) + 8 * (g & 1)));
    }
    hd = *(const u32x4v *)(Wh + (PLAIN ? 144 * b : 16 * b));
  };
  f32x4 acc[NM][TT];
#pragma unroll
  for (int mt = 0; mt < NM; ++mt)
#pragma unroll
    for (int t = 0; t < TT; ++t) acc[mt][t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
  load_round(0);
  for (int64_t b0 = 0; b0 < nb; b0 += KW) {
    // x of the round's superblocks -> three bf16 planes each and the sub-block sums
#pragma unroll
    for (int q = 0; q < KW; ++q)
#pragma unroll
      for (int t = 0; t < TT; ++t) {
        const float v[16] = {xv[q][t][0].x, xv[q][t][0].y, xv[q][t][0].z, xv[q][t][0].w,
                             xv[q][t][1].x, xv[q][t][1].y, xv[q][t][1].z, xv[q][t][1].w,
                             xv[q][t][2].x, xv[q][t][2].y, xv[q][t][2].z, xv[q][t][2].w,
                             xv[q][t][3].x, xv[q][t][3].y, xv[q][t][3].z, xv[q][t][3].w};
        uint32_t p1[8], p2[8], p3[8];
        float hs = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i += 2) {
          uint32_t u1[2], u2[2], u3[2];
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            const float x = v[i + h];
            const uint32_t b1 = __float_as_uint(x) & 0xffff0000u;
            const float r1 = x - __uint_as_float(b1);
            const uint32_t b2 = __float_as_uint(r1) & 0xffff0000u;
            const float r2 = r1 - __uint_as_float(b2);
            u1[h] = b1;
            u2[h] = b2;
            u3[h] = __float_as_uint(r2);
            hs = hs + x;
          }
          p1[i / 2] = bf16_pair(u1[0], u1[1]);
          p2[i / 2] = bf16_pair(u2[0], u2[1]);
          p3[i / 2] = bf16_pair(u3[0], u3[1]);
        }
        const float ss = hs + __shfl_xor(hs, 1);  // the two halves of sub-block sc16 / 2, low half first
        const int row = 16 * t + stok;
        uint32_t *d1 = (uint32_t *)&xp[q][0][row][16 * sc16], *d2 = (uint32_t *)&xp[q][1][row][16 * sc16],
                 *d3 = (uint32_t *)&xp[q][2][row][16 * sc16];
#pragma unroll
        for (int c = 0; c < 8; c += 4) {
          *(u32x4v *)(d1 + c) = u32x4v{p1[c], p1[c + 1], p1[c + 2], p1[c + 3]};
          *(u32x4v *)(d2 + c) = u32x4v{p2[c], p2[c + 1], p2[c + 2], p2[c + 3]};
          *(u32x4v *)(d3 + c) = u32x4v{p3[c], p3[c + 1], p3[c + 2], p3[c + 3]};
        }
        if ((sc16 & 1) == 0) xs[q][row][sc16 >> 1] = ss;
      }
    // the rows' A_j = d*sc_j and B_j = dmin*m_j (dequant_row's factors) of this wave's superblock:
    // lane (row l % 16, group g) takes matrix g / 2 and quarters 2(g % 2), +1 of gate/up,
    // quarter g of down
    {
      const u32x4v h = hd;
      const int mt = NM == 2 ? g >> 1 : 0;
      const float d = f16_bits_to_f32(h.x), dmin = f16_bits_to_f32(h.x >> 16);
#pragma unroll
      for (int kk = 0; kk < NM; ++kk) {
        const int k = NM == 2 ? 2 * (g & 1) + kk : g;
        int sA, mA, sB, mB;
        q4k_scale_min_pair(h.y, h.z, h.w, k, sA, mA, sB, mB);
        ab[wave][mt][0][2 * k][r16] = d * (float)sA;
        ab[wave][mt][1][2 * k][r16] = dmin * (float)mA;
        ab[wave][mt][0][2 * k + 1][r16] = d * (float)sB;
        ab[wave][mt][1][2 * k + 1][r16] = dmin * (float)mB;
      }
    }
    uint2 wc[NM][4];
#pragma unroll
    for (int mt = 0; mt < NM; ++mt)
#pragma unroll
      for (int k = 0; k < 4; ++k) wc[mt][k] = wq[mt][k];
    const bool live = b0 + kg < nb;  // this wave has a superblock in the round
    __syncthreads();
    if (b0 + KW < nb) load_round(b0 + KW);
    // quarter k's nibbles as the A operands: sub-blocks 2k (low nibbles), 2k+1 (high)
    auto a_ops = [&](int k, bf16x8 (&aop)[NM][2]) {
#pragma unroll
      for (int mt = 0; mt < NM; ++mt) {
        uint32_t lo[4], hi[4];
#pragma unroll
        for (int h = 0; h < 2; ++h) {  // each nibble q, exact in bf16 (the high half of (float)q)
          const uint32_t w = h ? wc[mt][k].y : wc[mt][k].x;
          uint32_t wl = w & 0x0f0f0f0fu, wh = (w >> 4) & 0x0f0f0f0fu;
          // opaque, so each byte converts with one v_cvt_f32_ubyteN rather than a
          // nibble extract and a conversion
          asm("" : "+v"(wl), "+v"(wh));
          lo[2 * h] = bf16_pair(__float_as_uint((float)(wl & 0xffu)), __float_as_uint((float)((wl >> 8) & 0xffu)));
          lo[2 * h + 1] = bf16_pair(__float_as_uint((float)((wl >> 16) & 0xffu)), __float_as_uint((float)(wl >> 24)));
          hi[2 * h] = bf16_pair(__float_as_uint((float)(wh & 0xffu)), __float_as_uint((float)((wh >> 8) & 0xffu)));
          hi[2 * h + 1] = bf16_pair(__float_as_uint((float)((wh >> 16) & 0xffu)), __float_as_uint((float)(wh >> 24)));
        }
        aop[mt][0] = __builtin_bit_cast(bf16x8, u32x4v{lo[0], lo[1], lo[2], lo[3]});
        aop[mt][1] = __builtin_bit_cast(bf16x8, u32x4v{hi[0], hi[1], hi[2], hi[3]});
      }
    };
    if (live && TT == 1 && KW == 2) {
      // One token tile, two K groups: quarter k + 1's LDS operands are read
      // while quarter k multiplies (two sets), the sub-block sums once per
      // round. With one K group the second set would cost the kernel its four
      // waves per SIMD (120 registers -> 183), which the 64-row work-groups
      // need when many run.
      struct QOps {
        bf16x8 b[2][3];    // x pieces of sub-blocks 2k, 2k+1
        float4 A[NM][2], B[NM][2];  // rows 4g..4g+3's factors
      };
      auto ld = [&](int k, QOps &o) {
#pragma unroll
        for (int sbh = 0; sbh < 2; ++sbh) {
          const int j = 2 * k + sbh, c0 = 32 * j + 8 * g;
#pragma unroll
          for (int pc = 0; pc < 3; ++pc) o.b[sbh][pc] = *(const bf16x8 *)&xp[kg][pc][r16][c0];
#pragma unroll
          for (int mt = 0; mt < NM; ++mt) {
            o.A[mt][sbh] = *(const float4 *)&ab[wave][mt][0][j][4 * g];
            o.B[mt][sbh] = *(const float4 *)&ab[wave][mt][1][j][4 * g];
          }
        }
      };
      const float4 s_lo = *(const float4 *)&xs[kg][r16][0], s_hi = *(const float4 *)&xs[kg][r16][4];
      const float sjv[8] = {s_lo.x, s_lo.y, s_lo.z, s_lo.w, s_hi.x, s_hi.y, s_hi.z, s_hi.w};
      QOps o[2];
      ld(0, o[0]);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if (k < 3) ld(k + 1, o[(k + 1) & 1]);
        bf16x8 aop[NM][2];
        a_ops(k, aop);
        const QOps &c = o[k & 1];
#pragma unroll
        for (int sbh = 0; sbh < 2; ++sbh) {
          const float sj = sjv[2 * k + sbh];
#pragma unroll
          for (int mt = 0; mt < NM; ++mt) {
            f32x4 P = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[mt][sbh], c.b[sbh][0], P, 0, 0, 0);
            P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[mt][sbh], c.b[sbh][1], P, 0, 0, 0);
            P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[mt][sbh], c.b[sbh][2], P, 0, 0, 0);
            const float Av[4] = {c.A[mt][sbh].x, c.A[mt][sbh].y, c.A[mt][sbh].z, c.A[mt][sbh].w};
            const float Bv[4] = {c.B[mt][sbh].x, c.B[mt][sbh].y, c.B[mt][sbh].z, c.B[mt][sbh].w};
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              float y = acc[mt][0][v];
              y = __builtin_fmaf(Av[v], P[v], y);
              y = __builtin_fmaf(-Bv[v], sj, y);
              acc[mt][0][v] = y;
            }
          }
        }
      }
    } else if (live) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        bf16x8 aop[NM][2];
        a_ops(k, aop);
#pragma unroll
        for (int t = 0; t < TT; ++t) {
          if (TT > 2 && t >= ntt) break;  // with one or two tiles the phase stays one block
          const int tok = 16 * t + r16;
#pragma unroll
          for (int sbh = 0; sbh < 2; ++sbh) {
            const int j = 2 * k + sbh, c0 = 32 * j + 8 * g;
            const bf16x8 b1 = *(const bf16x8 *)&xp[kg][0][tok][c0];
            const bf16x8 b2 = *(const bf16x8 *)&xp[kg][1][tok][c0];
            const bf16x8 b3 = *(const bf16x8 *)&xp[kg][2][tok][c0];
            const float sj = xs[kg][tok][j];
#pragma unroll
            for (int mt = 0; mt < NM; ++mt) {
              f32x4 P = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
              P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[mt][sbh], b1, P, 0, 0, 0);
              P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[mt][sbh], b2, P, 0, 0, 0);
              P = __builtin_amdgcn_mfma_f32_16x16x32_bf16(aop[mt][sbh], b3, P, 0, 0, 0);
              const float4 A4 = *(const float4 *)&ab[wave][mt][0][j][4 * g];
              const float4 B4 = *(const float4 *)&ab[wave][mt][1][j][4 * g];
              const float Av[4] = {A4.x, A4.y, A4.z, A4.w}, Bv[4] = {B4.x, B4.y, B4.z, B4.w};
#pragma unroll
              for (int v = 0; v < 4; ++v) {
                float y = acc[mt][t][v];
                y = __builtin_fmaf(Av[v], P[v], y);
                y = __builtin_fmaf(-Bv[v], sj, y);
                acc[mt][t][v] = y;
              }
            }
          }
        }
      }
    }
    __syncthreads();  // the planes and factors are read before the next round overwrites them
  }
  if constexpr (KW > 1) {  // the tile's K groups in wave order, through LDS (the planes are free now)
    f32x4 *red = (f32x4 *)&xp[0][0][0][0];  // [KW - 1][RT][NM][TT][64]
    if (kg > 0) {
#pragma unroll
      for (int mt = 0; mt < NM; ++mt)
#pragma unroll
        for (int t = 0; t < TT; ++t) red[(((kg - 1) * RT + tile) * NM + mt) * TT * 64 + t * 64 + lane] = acc[mt][t];
    }
    __syncthreads();
    if (kg == 0) {
#pragma unroll
      for (int q = 1; q < KW; ++q)
#pragma unroll
        for (int mt = 0; mt < NM; ++mt)
#pragma unroll
          for (int t = 0; t < TT; ++t) acc[mt][t] += red[(((q - 1) * RT + tile) * NM + mt) * TT * 64 + t * 64 + lane];
    }
  }
  // lane l of the tile's first wave: rows rbase + 4g + v, token 16t + l % 16
#pragma unroll
  for (int t = 0; t < TT; ++t) {
    const int tk = tok0 + 16 * t + r16;
    if (kg != 0 || 16 * t + r16 >= nbt) continue;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int64_t rw = rbase + 4 * g + v;
      if (rw >= rows) continue;
      if constexpr (NM == 2) {  // SwiGLU: g / (1 + exp(-g)) * u
        const float gv = acc[0][t][v], uv = acc[1][t][v];
        const float den = 1.0f + expf_cr(-gv);
        const float qv = gv / den;
        a.out[(p0 + tk) * rows + rw] = qv * uv;
      } else {
        a.out[(p0 + tk) * rows + rw] = acc[0][t][v];
      }
    }
  }
}

}  // namespace

bool f32_rows_supported(int type, int64_t rows, int64_t cols) {
  return type == T_Q4_K && rows > 0 && cols > 0 && cols % 256 == 0;
}

hipError_t launch_f32_rows(hipStream_t st, int mode, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                           const Routing &rt, int regime, int max_active, int64_t n_slots, int min_rows,
                           int max_rows, const float *x, float *out) {
  if (!f32_rows_supported(type, rows, cols)) return hipErrorNotSupported;
  if (rows == 0 || max_active == 0 || max_rows < min_rows) return hipSuccess;
  F32RowsArgs a{};
  a.tier = tier;
  a.rt = rt;
  a.rows = rows;
  a.cols = cols;
  a.x = x;
  a.out = out;
  a.regime = regime;
  // Experts of 4-16 rows take one token tile, 17-32 two, more blocks of four.
  // Superblock groups per work-group: parts of at most 4096 rows split the
  // superblocks over pairs of waves for one or two token tiles (32-row
  // work-groups, so that enough run); wider parts, and four token tiles,
  // give each wave its own 16 rows over all superblocks (64-row work-groups;
  // more groups would need more LDS than leaves one or two work-groups per CU).
  const int kw = rows <= 4096 && cols > 1024 ? 2 : 1;
  // At most n_slots / min_rows experts hold min_rows or more rows: when that
  // is fewer than the active experts, the grid's y ranks the experts in range
  // instead of covering the active list.
  auto ny = [&]() -> unsigned {
    const int64_t m = n_slots / (a.min_rows > 1 ? a.min_rows : 1);
    a.ranked = m < max_active;
    return (unsigned)(m < max_active ? m : max_active);
  };
#define KMOE_F32R(M, T, W, Z)                                                                                 \
  do {                                                                                                         \
    if (ny() > 0)                                                                                              \
      KMOE_LAUNCH((k_f32x3_rows<M, T, W>), dim3((unsigned)((rows + 64 / W - 1) / (64 / W)), ny(), (unsigned)(Z)), \
                  dim3(256), 0, st, a);                                                                        \
  } while (0)
#define KMOE_F32RW(M, T)                 \
  do {                                   \
    if (kw == 2) KMOE_F32R(M, T, 2, 1);  \
    else KMOE_F32R(M, T, 1, 1);          \
  } while (0)
  a.min_rows = min_rows;
  a.max_rows = max_rows < 16 ? max_rows : 16;
  if (a.min_rows <= a.max_rows) {
    if (mode == 0) KMOE_F32RW(0, 1);
    else KMOE_F32RW(1, 1);
  }
  a.min_rows = min_rows > 17 ? min_rows : 17;
  a.max_rows = max_rows < 32 ? max_rows : 32;
  if (a.min_rows <= a.max_rows) {
    if (mode == 0) KMOE_F32RW(0, 2);
    else KMOE_F32RW(1, 2);
  }
  a.min_rows = min_rows > 33 ? min_rows : 33;
  a.max_rows = max_rows;
  if (a.min_rows <= a.max_rows) {
    const int z = (max_rows + 63) / 64;
    if (mode == 0) KMOE_F32R(0, 4, 1, z);
    else KMOE_F32R(1, 4, 1, z);
  }
#undef KMOE_F32RW
#undef KMOE_F32R
  return hipGetLastError();
}

namespace {

template <int M>
hipError_t launch_plain_t(hipStream_t st, const F32RowsArgs &a, int64_t rows, int64_t cols, int64_t s_rows) {
  const int kw = rows <= 4096 && cols > 1024 ? 2 : 1;
  const int64_t gx2 = (rows + 31) / 32, gx1 = (rows + 63) / 64;
  // token blocks of 64, 32 or 16 rows: the largest that still gives at least
  // two work-groups per CU (smaller blocks re-read the weights, from L2)
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  const int64_t z4 = (s_rows + 63) / 64, z2 = (s_rows + 31) / 32, z1 = (s_rows + 15) / 16;
  const int64_t gx = kw == 2 ? gx2 : gx1;
  if (z1 > 65535 || gx1 * 2 > (int64_t)UINT32_MAX) return hipErrorNotSupported;
  if (s_rows > 32 && gx1 * z4 >= 2LL * cus) {
    KMOE_LAUNCH((k_f32x3_rows<M, 4, 1>), dim3((unsigned)gx1, 1, (unsigned)z4), dim3(256), 0, st, a);
  } else if (s_rows > 16 && gx * z2 >= 2LL * cus) {
    if (kw == 2) KMOE_LAUNCH((k_f32x3_rows<M, 2, 2>), dim3((unsigned)gx2, 1, (unsigned)z2), dim3(256), 0, st, a);
    else KMOE_LAUNCH((k_f32x3_rows<M, 2, 1>), dim3((unsigned)gx1, 1, (unsigned)z2), dim3(256), 0, st, a);
  } else {
    if (kw == 2) KMOE_LAUNCH((k_f32x3_rows<M, 1, 2>), dim3((unsigned)gx2, 1, (unsigned)z1), dim3(256), 0, st, a);
    else KMOE_LAUNCH((k_f32x3_rows<M, 1, 1>), dim3((unsigned)gx1, 1, (unsigned)z1), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace

hipError_t launch_f32_rows_plain(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                                 const float *x, int64_t s_rows, float *out, const uint8_t *w_up) {
  if (!f32_rows_supported(type, rows, cols) || ((uintptr_t)w & 15u) || ((uintptr_t)x & 15u) ||
      ((uintptr_t)w_up & 15u))
    return hipErrorNotSupported;
  if (s_rows <= 0) return hipSuccess;
  F32RowsArgs a{};
  a.rows = rows;
  a.cols = cols;
  a.x = x;
  a.out = out;
  a.pw = w;
  a.pw2 = w_up;
  a.s_rows = s_rows;
  if (w_up) return launch_plain_t<3>(st, a, rows, cols, s_rows);
  return launch_plain_t<2>(st, a, rows, cols, s_rows);
}

}  // namespace kmoe
