// kmoe_mfma.hip — grouped Q4_K x Q8_K expert products on the int8 matrix
// cores (prefill and batched decode on the int8 path).
//
// Per expert e with n_e routed rows (token slots), per 32-row weight tile and
// 32-token tile, per superblock b (256 columns):
//   sumi(t, r) = sum_j sc_j(r) * sum_{x in sub-block j} q(r, x) * a(t, x)
//   mins(t, r) = sum_j m_j(r) * bsum_j(t)
//   y(t, r)   += ad(t, b) * (d(r) * sumi - dmin(r) * mins)
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
// Roles: A = weight rows (32 per tile), B = activation rows (tokens, 32 per
// tile). In the 32x32 result lane l owns token column l % 32 and weight rows
// 8*(v/4) + 4*(l/32) + v%4, so the token's block scale is one value per lane
// and the 16 rows' (d, dmin) are read once per superblock.
// The k order inside an MFMA only has to agree between A and B: lane half h
// holds columns 16h .. 16h+15 of the 32-column sub-block on both sides, which
// for the weights is exactly tiled chunk (b, j/2, h): lo nibbles for even j,
// hi nibbles for odd j.
//
// Work-group: 4 waves, one per SIMD, each with the whole register file. A
// wave owns one 32-row weight tile and every token tile of a 128-row pass, so
// it decodes its rows' superblock into A operands once and multiplies them
// against up to 4 token tiles (gate/up: the group holds the same 64 rows of
// both matrices and applies SwiGLU, transformer.rs:558, after an LDS exchange
// between the gate and up waves; the single-matrix modes: 128 rows). An
// expert with more than 128 routed rows takes more passes; the plain modes
// give each pass its own work-group.
// Per superblock the activation tile (int8 pieces by direct global->LDS
// loads, the split 16-sums and the block scales through registers) goes to a
// double-buffered LDS stage while the previous superblock is multiplied; the
// weight pieces of the next superblock are loaded into registers meanwhile.
// Inside a superblock the B operands of token tile T+1 are read from LDS and
// the scale epilogue of tile T-1 runs while tile T's MFMAs execute.
// Modes: grouped gate/up and down over the expert tier's tiled Q4_K rows
// (routed token slots), and plain GGUF Q4_K rows [rows, cols] against s_rows
// activation rows: the matmul (quant.rs:229 on the int path) and the per-block
// integer accumulators (avx2.rs:361-374) exposed for parity checks.
#include <type_traits>

#include "kmoe_device.h"
#include "kmoe_launch.h"

namespace kmoe {

namespace {

typedef int v4i32 __attribute__((ext_vector_type(4)));
typedef int v16i32 __attribute__((ext_vector_type(16)));
typedef float v16f32 __attribute__((ext_vector_type(16)));
typedef float v4f32 __attribute__((ext_vector_type(4)));
typedef _Float16 v8f16 __attribute__((ext_vector_type(8)));
typedef _Float16 v4f16 __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int kTok = 128;  // token rows per pass
constexpr int kTiles = 4;  // 32-row token tiles per pass

enum { MF_GATE_UP = 0, MF_DOWN = 1, MF_PLAIN = 2, MF_SUMS = 3 };

struct MfmaArgs {
  ExpertTier tier;
  Routing rt;
  const uint8_t *w0;     // plain modes: GGUF rows
  int64_t s_rows;        // plain modes: activation rows
  int64_t rows, cols;    // weight rows (F for gate/up, d for down), columns
  const int8_t *aq;      // int8 activation rows
  const float *ad;       // their block scales [.., cols/256]
  const int32_t *abs;    // their 16-sums [.., cols/16]
  float *out;            // [slots or s_rows, rows]
  int32_t *sumi, *mins;  // MF_SUMS: [(s*rows + r)*nb + b]
  int regime;
  int min_rows;          // grouped modes: experts with fewer rows are another kernel's
  int max_rows;          // grouped modes: experts with more rows are another kernel's
  BlockDbg dbg;          // grouped modes with DBG: per-superblock integers (gate/down 0, up 1)
};

// One LDS stage (superblock b of the pass's 128 token rows):
//   int8 [16 pieces = (sub-block, half)][128 tokens][16 bytes]   32 KB
//   f16  [2 halves][128 tokens][8] = (bh_0..7 | bl_0..7)          4 KB
//   f32  ad [128]                                                 512 B
//   weights [row slots][5 chunks][64 lanes][16 bytes]: chunk 0 the head of
//   lane l's row (row l % 32 of the slot's tile), chunks 1..4 its nibble
//   bytes [32k + 16*half, +16), k < 4                   5 KB per row slot
constexpr int kStA = 16 * kTok * 16;
constexpr int kStM = 2 * kTok * 16;
constexpr int kStD = kTok * 4;
constexpr int kStW = kStA + kStM + kStD;
// Gate/up: 8 row slots (4 tiles of both matrices), every wave all token
// tiles. Other modes: 4 row slots, two waves per slot splitting the tiles.
template <int MODE>
constexpr int kSlots = MODE == 0 ? 8 : 4;
template <int MODE>
constexpr int kStage = kStW + kSlots<MODE> * 5 * 64 * 16;

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

// Each byte of n (< 16) times f (< 8), as two 16-bit products (no carry
// leaves a byte: 15 * 7 = 105).
__device__ __forceinline__ int mul_bytes(uint32_t n, uint32_t f) {
  const u16x2 nv = __builtin_bit_cast(u16x2, n);
  const u16x2 fv = {(unsigned short)f, (unsigned short)f};
  return __builtin_bit_cast(int, (u16x2)(nv * fv));
}

// 16 bytes per lane from g into LDS at lds_wave_base + 16*lane (the base is
// the same for the whole wave).
__device__ __forceinline__ void lds_dma16(const void *g, uint8_t *lds_wave_base) {
  __builtin_amdgcn_global_load_lds(g, (__attribute__((address_space(3))) void *)lds_wave_base, 16, 0, 0);
}

template <int MODE, bool DBG = false>
__global__ void __launch_bounds__(512) k_moe_mfma(MfmaArgs a) {
  constexpr bool TILED = MODE == MF_GATE_UP || MODE == MF_DOWN;  // expert tier rows are tiled, plain rows GGUF
  // Two stages as distinct objects: each access names its stage statically, so
  // reads of one are not ordered behind direct loads still filling the other.
  constexpr int SLOTS = kSlots<MODE>;
  constexpr int TSPLIT = 8 / SLOTS;  // waves per row slot, splitting the token tiles
  constexpr int TPW = kTiles / TSPLIT;  // token tiles per wave
  __shared__ __attribute__((aligned(16))) uint8_t st0[kStage<MODE>];
  __shared__ __attribute__((aligned(16))) uint8_t st1[kStage<MODE>];
  __shared__ int32_t srcs[kTok];
  const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave % SLOTS;  // the group's row slot (gate/up: matrix wr & 1, tile wr >> 1)
  const int th = wave / SLOTS;  // token tiles th, th + TSPLIT, ... of each pass
  const int64_t cols = a.cols, nb = cols / 256, row_bytes = nb * 144;
  const int mat = MODE == MF_GATE_UP ? (wr & 1) : 2;
  const int64_t rtile = MODE == MF_GATE_UP ? (int64_t)blockIdx.x * 4 + (wr >> 1) : (int64_t)blockIdx.x * 4 + wr;
  const int64_t r_lane = rtile * 32 + l32;  // the weight row this lane decodes (A operand row l32)
  const int64_t r_out = rtile * 32 + 4 * half;  // its output rows: r_out + 8g + c, g, c < 4
  const int64_t rows = a.rows;
  const uint8_t *W;
  int64_t p0 = 0;
  int t_begin, t_end;
  {
    const int64_t rr = r_lane < rows ? r_lane : rows - 1;
    if constexpr (TILED) {
      const int i_act = blockIdx.y;
      if (i_act >= *a.rt.n_active) return;
      const int e = a.rt.active[i_act];
      p0 = a.rt.offsets[e];
      const int n = (int)(a.rt.offsets[e + 1] - p0);
      if (n < a.min_rows || n > a.max_rows || !mfma_int_regime(a.regime, n)) return;
      W = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[mat] + rr * row_bytes;
      t_begin = 0;
      t_end = n;
    } else {
      W = a.w0 + rr * row_bytes;
      t_begin = (int)blockIdx.y * kTok;
      t_end = t_begin + kTok < (int)a.s_rows ? t_begin + kTok : (int)a.s_rows;
    }
  }

  for (int t0 = t_begin; t0 < t_end; t0 += kTok) {
    const int nt = t_end - t0 < kTok ? t_end - t0 : kTok;
    const int nT = (nt + 31) >> 5;  // token tiles of this pass
    __syncthreads();  // the previous pass is done with srcs and the stages
    if (tid < kTok) {
      int32_t src = 0;
      if (tid < nt) {
        if constexpr (MODE == MF_GATE_UP) src = (int32_t)(a.rt.perm[p0 + t0 + tid] / a.rt.topk);
        else src = (int32_t)(p0 + t0 + tid);
      }
      srcs[tid] = src;
    }
    __syncthreads();
    // Token rows past nt read token 0's row: their results are never stored.
    const int8_t *ap0 = a.aq + (int64_t)srcs[lane < nt ? lane : 0] * cols;  // direct-load sources:
    const int8_t *ap1 = a.aq + (int64_t)srcs[64 + lane < nt ? 64 + lane : 0] * cols;  // tokens lane, 64 + lane
    const bool two_q = nt > 64;
    // 16-sums: thread tid stages sums 4q .. 4q+3 (sub-blocks 2q, 2q+1) of
    // token tid % 128, q = tid / 128; threads < 128 also its block scale
    const int tok_me = tid & (kTok - 1), sq = tid >> 7;
    const int64_t src_me = srcs[tok_me < nt ? tok_me : 0];
    const int32_t *bsp = a.abs + src_me * (cols / 16) + 4 * sq;
    const float *adp = a.ad + src_me * nb;

    int4 SB;
    float SD = 0.0f;
    auto fetch = [&](int64_t b, uint8_t *A) {
#pragma unroll
      for (int i = 0; i < 2; ++i) {  // pieces 2*wave, 2*wave+1 of every token
        const int pc = 2 * wave + i;
        lds_dma16(ap0 + 256 * b + 16 * pc, A + pc * kTok * 16);
        if (two_q) lds_dma16(ap1 + 256 * b + 16 * pc, A + (pc * kTok + 64) * 16);
      }
      // weights of row slot wr (with two waves per slot: the th == 0 wave
      // takes the head and chunks 1, 2, the other chunks 3, 4)
      uint8_t *Wl = A + kStW + wr * 5 * 1024;
      const uint8_t *c0, *cq;  // head; nibble chunk k at cq + k*cs
      int64_t cs;
      if constexpr (TILED) {
        c0 = W + 16 * b;
        cq = W + tq4_qs_off(nb, b, 0, half);
        cs = 16;
      } else {  // GGUF superblock: head, then qs chunk (k, half) at 16 + 32k + 16*half
        c0 = W + 144 * b;
        cq = c0 + 16 + 16 * half;
        cs = 32;
      }
      if (TSPLIT == 1 || th == 0) {
        lds_dma16(c0, Wl);
        lds_dma16(cq, Wl + 1024);
        lds_dma16(cq + cs, Wl + 2048);
      }
      if (TSPLIT == 1 || th == 1) {
        lds_dma16(cq + 2 * cs, Wl + 3072);
        lds_dma16(cq + 3 * cs, Wl + 4096);
      }
      SB = *(const int4 *)(bsp + 16 * b);
      if constexpr (MODE != MF_SUMS) {
        if (tid < kTok) SD = adp[b];
      }
    };
    auto put = [&](uint8_t *S) {  // split 32-sums of sub-blocks 2q, 2q+1 of token tid % 128; block scale
      const int s0 = SB.x + SB.y, s1 = SB.z + SB.w;
      const int h0 = s0 >> 6, h1 = s1 >> 6;  // floor division: s = 64*h + l, l in [0, 64)
      h2 hv, lv;
      hv.x = (_Float16)h0;
      hv.y = (_Float16)h1;
      lv.x = (_Float16)(s0 - 64 * h0);
      lv.y = (_Float16)(s1 - 64 * h1);
      *(h2 *)(S + kStA + tok_me * 16 + 4 * sq) = hv;
      *(h2 *)(S + kStA + (kTok + tok_me) * 16 + 4 * sq) = lv;
      if (tid < kTok) *(float *)(S + kStA + kStM + 4 * tid) = SD;
    };
    v4i32 ahi[8], alo[8];
    v8f16 amn;
    auto build = [&](const uint8_t *S) {  // A operands of this lane's row
      const uint8_t *Wl = S + kStW + wr * 5 * 1024 + 16 * lane;
      const u32x4 WH = *(const u32x4 *)Wl;
      u32x4 WQ[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) WQ[i] = *(const u32x4 *)(Wl + (1 + i) * 1024);
      int sc[8], mn[8];
      q4k_scales8(WH.y, WH.z, WH.w, sc, mn);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const u32x4 w = WQ[j >> 1];
        const uint32_t msk = 0x0f0f0f0fu;
        const int s4 = (j & 1) ? 4 : 0;
        const uint32_t n0 = (w.x >> s4) & msk, n1 = (w.y >> s4) & msk, n2 = (w.z >> s4) & msk,
                       n3 = (w.w >> s4) & msk;
        const uint32_t hi = (uint32_t)(sc[j] >> 3), lo = (uint32_t)(sc[j] & 7);
        ahi[j] = v4i32{mul_bytes(n0, hi), mul_bytes(n1, hi), mul_bytes(n2, hi), mul_bytes(n3, hi)};
        alo[j] = v4i32{mul_bytes(n0, lo), mul_bytes(n1, lo), mul_bytes(n2, lo), mul_bytes(n3, lo)};
        amn[j] = (_Float16)(half ? mn[j] : 64 * mn[j]);
      }
    };

    float y[TPW][16];
#pragma unroll
    for (int i = 0; i < TPW; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) y[i][v] = 0.0f;

    fetch(0, st0);
    put(st0);
    __syncthreads();  // waits for the direct loads too
    // superblock b from stage S while superblock b+1 loads into stage Nx
    auto iter = [&](int64_t b, const uint8_t *S, uint8_t *Nx) {
      if (b + 1 < nb) fetch(b + 1, Nx);
      build(S);
      // (d, dmin) f16 pairs of the lane's 16 output rows 8g + 4*half + c: the
      // first dword of those rows' heads
      const uint8_t *hd = S + kStW + wr * 5 * 1024 + 16 * 4 * half;
#pragma unroll
      for (int i = 0; i < TPW; ++i) {
        const int T = TSPLIT * i + th;
        if (T < nT) {
          // B operands: pieces (j, half) of token 32T + l32; mins operand (bh | bl)
          const int tl = 32 * T + l32;
          v4i32 bv[8];
#pragma unroll
          for (int j = 0; j < 8; ++j) bv[j] = *(const v4i32 *)(S + ((2 * j + half) * kTok + tl) * 16);
          const v8f16 bm = *(const v8f16 *)(S + kStA + (half * kTok + tl) * 16);
          // sumi = 8 * (hi chain) + (lo chain): the lo chain accumulates onto the shifted hi sums
          v16i32 H = v16i32{0};
#pragma unroll
          for (int j = 0; j < 8; ++j) H = __builtin_amdgcn_mfma_i32_32x32x32_i8(ahi[j], bv[j], H, 0, 0, 0);
          H = H << 3;
#pragma unroll
          for (int j = 0; j < 8; ++j) H = __builtin_amdgcn_mfma_i32_32x32x32_i8(alo[j], bv[j], H, 0, 0, 0);
          const v16f32 N = __builtin_amdgcn_mfma_f32_32x32x16_f16(amn, bm, v16f32{0}, 0, 0, 0);
          // element v: token 32T + l32 of the pass, row r_out + 8*(v/4) + v%4
          if constexpr (MODE == MF_SUMS) {
            if (tl < nt) {
#pragma unroll
              for (int v = 0; v < 16; ++v) {
                const int64_t rw = r_out + 8 * (v >> 2) + (v & 3);
                if (rw < rows) {
                  const int64_t o = ((int64_t)(t0 + tl) * rows + rw) * nb + b;
                  a.sumi[o] = H[v];
                  a.mins[o] = (int)N[v];
                }
              }
            }
          } else {
            if constexpr (DBG) {  // the superblock's integers, complete in this lane
              int32_t *ds = a.dbg.s[mat == 1 ? 1 : 0], *dm = a.dbg.m[mat == 1 ? 1 : 0];
              if (tl < nt) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                  const int64_t rw = r_out + 8 * (v >> 2) + (v & 3);
                  if (rw < rows) {
                    const int64_t o = ((p0 + t0 + tl) * rows + rw) * nb + b;
                    ds[o] = H[v];
                    dm[o] = (int)N[v];
                  }
                }
              }
            }
            const float adt = *(const float *)(S + kStA + kStM + 4 * tl);
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const h2 dv = *(const h2 *)(hd + 16 * (8 * (v >> 2) + (v & 3)));
              const float m = fmaf(-(float)dv.y, N[v], 0.0f);  // - dmin * mins
              const float x = fmaf((float)dv.x, (float)H[v], m);
              y[i][v] = fmaf(adt, x, y[i][v]);
            }
          }
        }
      }
      if (b + 1 < nb) put(Nx);
      __syncthreads();  // next stage complete (direct loads included) and this one free
    };
    for (int64_t b = 0; b < nb; b += 2) {
      iter(b, st0, st1);
      if (b + 1 < nb) iter(b + 1, st1, st0);
    }
    // ---- results: out[p0 + t0 + token, row]
    auto store = [&](int T, int v, float val) {
      const int t = 32 * T + l32;
      const int64_t rw = r_out + 8 * (v >> 2) + (v & 3);
      if (t < nt && rw < rows) a.out[(p0 + t0 + t) * rows + rw] = val;
    };
    if constexpr (MODE == MF_GATE_UP) {
      // gate and up values to LDS ([128 tokens][128 rows + 1], gate in st0, up
      // in st1), then SwiGLU by every thread, row-contiguous stores
      constexpr int LD = 129;
      float *xm = mat == 0 ? (float *)st0 : (float *)st1;
#pragma unroll
      for (int i = 0; i < TPW; ++i)
        if (i < nT) {
#pragma unroll
          for (int v = 0; v < 16; ++v)
            xm[(32 * i + l32) * LD + 32 * (wr >> 1) + 8 * (v >> 2) + 4 * half + (v & 3)] = y[i][v];
        }
      lds_barrier();
      const float *xg = (const float *)st0, *xu = (const float *)st1;
      const int64_t rbase = (int64_t)blockIdx.x * 128;
      for (int e = tid; e < nt * 128; e += 512) {
        const int t = e >> 7, rl = e & 127;
        if (rbase + rl < rows) {
          const float g = xg[t * LD + rl], u = xu[t * LD + rl];
          const float den = 1.0f + expf_cr(-g);  // SwiGLU: g / (1 + exp(-g)) * u
          const float q = g / den;
          a.out[(p0 + t0 + t) * rows + rbase + rl] = q * u;
        }
      }
    } else if constexpr (MODE != MF_SUMS) {
#pragma unroll
      for (int i = 0; i < TPW; ++i)
        if (TSPLIT * i + th < nT) {
#pragma unroll
          for (int v = 0; v < 16; ++v) store(TSPLIT * i + th, v, y[i][v]);
        }
    }
  }
}


// ---- Experts with at most 32 routed rows (decode batches of a few dozen
// tokens). The kernel above keeps one superblock of loads in flight per
// work-group and waits for all of it at every barrier; with a single token
// tile per superblock its compute is short and HBM sits mostly idle. Here:
//   * work items are (expert, 32*TI weight rows) over the experts with
//     min_rows..32 rows on the int path; work-group w takes items w,
//     w + gridDim.x, ... as one chain of stages, so its pipeline does not
//     drain between items;
//   * a stage is two superblocks: each lane's weight bytes (the two 16-byte
//     heads and eight 16-byte nibble chunks of its row, 128 contiguous bytes
//     in the tiled row, the A operand pieces of the kernel above) go to
//     registers NS stages deep, with cached loads (a head line serves four
//     stages); the stage's token tile (int8 pieces, 16-sums and block scales
//     of the item's <= 32 rows) goes to LDS by direct loads. Every wave
//     issues the same vector memory instructions per stage, so one counted
//     wait and one barrier per stage cover the stage;
//   * gate/up: 4 waves = (row tile 0, 1) x (gate, up), the up waves hand
//     their sums to the gate waves through LDS for SwiGLU (transformer.rs:558).
//     Down: 8 waves = (row tile 0..3) x (first, second part of the
//     superblocks), the second part's sums handed to the first, added in
//     that order.
// Per superblock the integers are the kernel above's (sumi = 8 * hi chain +
// lo chain, here as two accumulators; mins on the f16 matrix cores).
constexpr int kRingTok = 32;
// A work-group barrier that orders the compiler's memory accesses around it
// but waits for nothing itself: a workgroup-scope LDS fence would also wait
// for every direct global->LDS load in flight, which would drain the ring.
// The callers issue the exact s_waitcnt the barrier needs first.
__device__ __forceinline__ void ring_barrier() {
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
  __builtin_amdgcn_s_barrier();
  __atomic_signal_fence(__ATOMIC_SEQ_CST);
}
// ds_write_b128 written out: the compiler's own 16-byte LDS stores lose their
// alias information, and it then waits for every direct load in flight before
// them (all of the ring) although none of those writes the stored-to array.
__device__ __forceinline__ void lds_store16(float *p, v4f32 v) {
  const uint32_t la = (uint32_t)(uintptr_t)(__attribute__((address_space(3))) float *)p;
  asm volatile("ds_write_b128 %0, %1" ::"v"(la), "v"(v) : "memory");
}
constexpr int kRingItems = 8;      // items per work-group at most (the launcher's grid guarantees it)
constexpr int kRingExperts = 256;  // experts with rows at most
template <int MODE>
constexpr int kRingWaves = MODE == MF_DOWN ? 8 : 4;

template <int MODE, int NS, bool DBG>
__global__ void __launch_bounds__(kRingWaves<MODE> * 64, 2) k_moe_mfma_ring(MfmaArgs a) {
  constexpr int NW = kRingWaves<MODE>;
  constexpr int TI = NW / 2;                   // row tiles per item
  constexpr int RI = 32 * TI;                  // rows per item
  constexpr int KS = MODE == MF_DOWN ? 2 : 1;  // superblock parts per item
  constexpr int G = NW / KS;                   // waves loading one part's token tile
  constexpr int kA8 = kRingTok * 256;          // int8 rows [32 tokens][16 pieces, swizzled]
  constexpr int kS16 = kRingTok * 64;          // 16-sums [32 tokens][16]
  constexpr int kSB = kA8 + kS16;              // one superblock's token tile
  constexpr int kAd = KS * kSB;                // then per wave: block scales [32 tokens] (twice)
  constexpr int kStg = kAd + NW * 256;
  constexpr int NA8 = 8 / G, NB16 = 8 / G;     // direct loads per wave and stage (1 KB and 256 B each)
  constexpr int OPS = 4 + 1 + 1 + NA8 + NB16;  // vector memory instructions per wave and stage
  static_assert(NS >= 2 && NS <= 3, "ring depth");
  // Distinct objects per stage: reads of one stage are not ordered behind the
  // direct loads still filling the other.
  __shared__ __attribute__((aligned(16))) uint8_t st0[kStg];
  __shared__ __attribute__((aligned(16))) uint8_t st1[kStg];
  __shared__ __attribute__((aligned(16))) uint8_t st2[NS > 2 ? kStg : 16];
  // per wave: the stage's nibble runs [64 runs][64 B, swizzled], then its heads [32 rows][16 B]
  __shared__ __attribute__((aligned(16))) uint8_t scr[NW][4096 + 512];
  __shared__ __attribute__((aligned(16))) float xch[RI][kRingTok + 4];  // the hand-over: [row][token]
  __shared__ int32_t it_e[kRingItems], it_n[kRingItems], it_rb[kRingItems], it_src[kRingItems][kRingTok];
  __shared__ uint32_t it_p0[kRingItems];
  __shared__ int32_t elig[kRingExperts];
  __shared__ int32_t n_elig;

  const int tid = threadIdx.x, lane = tid & 63, half = lane >> 5, l32 = lane & 31;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int tile = wave % TI, grp = wave / TI;  // grp: gate/up the matrix, down the part
  const int wig = MODE == MF_DOWN ? tile : wave;  // wave's index among the waves loading its part
  const int mat = MODE == MF_GATE_UP ? grp : 2;
  const int64_t rows = a.rows, cols = a.cols, nb = cols / 256, row_bytes = nb * 144;
  const int RB = KS == 1 ? (int)nb : (int)((nb + 1) / 2);  // superblocks per part
  const int SPI = RB;                                         // stages per item
  const int b_lo = grp * (KS == 1 ? 0 : RB);
  const int b_hi = KS == 1 ? (int)nb : (b_lo + RB < nb ? b_lo + RB : (int)nb);  // this part's end
  const int bpe = (int)((rows + RI - 1) / RI);  // items per expert

  // experts of this kernel, in active order
  if (wave == 0) {
    const int na = *a.rt.n_active;
    int cnt = 0;
    for (int i0 = 0; i0 < na; i0 += 64) {
      const int i = i0 + lane;
      bool ok = false;
      int e = 0;
      if (i < na) {
        e = a.rt.active[i];
        const int n = (int)(a.rt.offsets[e + 1] - a.rt.offsets[e]);
        ok = n >= a.min_rows && n <= a.max_rows && mfma_int_regime(a.regime, n);
      }
      const uint64_t m = __ballot(ok);
      if (ok) elig[cnt + __popcll(m & ((1ull << lane) - 1ull))] = e;
      cnt += __popcll(m);
    }
    if (lane == 0) n_elig = cnt;
  }
  __syncthreads();
  const int total = n_elig * bpe;
  const int nI = (int)blockIdx.x < total ? (total - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
  if (nI == 0) return;
  for (int x = tid; x < nI * kRingTok; x += NW * 64) {
    const int k = x / kRingTok, t = x % kRingTok;
    const int gi = (int)blockIdx.x + k * (int)gridDim.x;
    const int e = elig[gi / bpe];
    const uint32_t p0 = a.rt.offsets[e];
    const int n = (int)(a.rt.offsets[e + 1] - p0);
    const uint32_t tt = t < n ? (uint32_t)t : 0u;  // rows past n read the first row's data, never stored
    if constexpr (MODE == MF_GATE_UP) it_src[k][t] = (int32_t)(a.rt.perm[p0 + tt] / (uint32_t)a.rt.topk);
    else it_src[k][t] = (int32_t)(p0 + tt);
    if (t == 0) {
      it_e[k] = e;
      it_p0[k] = p0;
      it_n[k] = n;
      it_rb[k] = gi % bpe;
    }
  }
  __syncthreads();

  uint8_t *const stg[3] = {st0, st1, st2};
  uint8_t *const myscr = scr[wave];
  const int T = nI * SPI;
  const int part_off = MODE == MF_DOWN ? grp * kSB : 0;
  u32x4 wc[NS][4], wh[NS];
  int ik = 0, ib = 0;  // next stage to issue (item, stage in the item); clamped at the last
  // Per-lane base pointers of the item being issued, recomputed when the
  // issue cursor enters a new item; a stage then adds scalar offsets only.
  int ci = -1;
  const uint8_t *pWA = nullptr, *pWB = nullptr, *pH = nullptr;
  const float *pAd = nullptr;
  const int8_t *pA8[NA8];
  const int32_t *pS16[NB16];
  auto issue = [&](int slot) {
    const int k = ik < nI ? ik : nI - 1, b = ik < nI ? ib : SPI - 1;
    const bool adv = ik < nI, wrap = ib + 1 == SPI;  // selects, not branches: the cursor stays in registers
    ik = adv && wrap ? ik + 1 : ik;
    ib = adv ? (wrap ? 0 : ib + 1) : ib;
    if (k != ci) {
      ci = k;
      const uint8_t *E = a.tier.base + (int64_t)it_e[k] * a.tier.stride + a.tier.off[mat];
      const int64_t r0 = (int64_t)it_rb[k] * RI + tile * 32;
      auto rowp = [&](int r) {
        const int64_t rr = r0 + r < rows ? r0 + r : rows - 1;
        return E + rr * row_bytes;
      };
      pWA = rowp(lane >> 2) + 16 * (lane & 3);
      pWB = rowp(16 + (lane >> 2)) + 16 * (lane & 3);
      pH = rowp(l32);
      pAd = a.ad + (int64_t)it_src[k][l32] * nb;
#pragma unroll
      for (int i2 = 0; i2 < NA8; ++i2) {
        const int t = 4 * (wig * NA8 + i2) + (lane >> 4);
        pA8[i2] = a.aq + (int64_t)it_src[k][t] * cols + 16 * ((lane & 15) ^ (t & 7));
      }
#pragma unroll
      for (int i2 = 0; i2 < NB16; ++i2)
        pS16[i2] = a.abs + (int64_t)it_src[k][4 * (wig * NB16 + i2) + (lane >> 4)] * (cols / 16) + (lane & 15);
    }
    const int64_t bq = b_lo + b < nb ? b_lo + b : nb - 1;
    // Coalesced weight loads. Run rho = 32*h + r is half h of row r's nibble
    // chunks of the stage's superblock (64 contiguous bytes of the tiled
    // row); load i takes runs 16*i .. 16*i+15, four lanes per run. The heads
    // load takes row lane % 32's 16-byte head (the two halves of the wave
    // load the same rows).
#pragma unroll
    for (int i = 0; i < 4; ++i)  // runs 16*i + lane/4: row (i & 1)*16 + lane/4, half i/2
      wc[slot][i] = *(const u32x4 *)(((i & 1) ? pWB : pWA) + tq4_qs_off(nb, bq, 0, i >> 1));
    wh[slot] = *(const u32x4 *)(pH + 16 * bq);
    // block scales: lane -> row lane % 32
    __builtin_amdgcn_global_load_lds(pAd + bq, (__attribute__((address_space(3))) void *)(stg[slot] + kAd + wave * 256),
                                     4, 0, 0);
    uint8_t *S = stg[slot] + part_off;
#pragma unroll
    for (int i2 = 0; i2 < NA8; ++i2)  // rows 4i .. 4i+3, 16 lanes each (piece p at slot p ^ (t & 7))
      lds_dma16(pA8[i2] + 256 * bq, S + (wig * NA8 + i2) * 1024);
#pragma unroll
    for (int i2 = 0; i2 < NB16; ++i2)  // 16-sums of rows 4i .. 4i+3
      __builtin_amdgcn_global_load_lds(pS16[i2] + 16 * bq,
                                       (__attribute__((address_space(3))) void *)(S + kA8 + (wig * NB16 + i2) * 256),
                                       4, 0, 0);
  };

  float y[16];
#pragma unroll
  for (int v = 0; v < 16; ++v) y[v] = 0.0f;
  int ck = 0, cb = 0;  // stage being consumed
  auto consume = [&](int slot) {
    {
      const int64_t bb = b_lo + cb;
      if (bb < b_hi) {  // the second part of an odd superblock count ends one stage early
        // the runs through the wave's scratch (run rho at rho*64, piece p at
        // (p ^ ((rho >> 1) & 3))*16) into the operand layout: lane = run; heads likewise
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int rho = 16 * i + (lane >> 2), p = lane & 3;
          lds_store16((float *)(myscr + rho * 64 + ((p ^ ((rho >> 1) & 3)) * 16)),
                      __builtin_bit_cast(v4f32, wc[slot][i]));
        }
        lds_store16((float *)(myscr + 4096 + 16 * l32), __builtin_bit_cast(v4f32, wh[slot]));
        u32x4 wq[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) wq[p] = *(const u32x4 *)(myscr + lane * 64 + ((p ^ ((lane >> 1) & 3)) * 16));
        const u32x4 hd = *(const u32x4 *)(myscr + 4096 + 16 * l32);
        const uint8_t *S = stg[slot] + part_off;
        int sc[8], mn[8];
        q4k_scales8(hd.y, hd.z, hd.w, sc, mn);
        int s16[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int4 v4 = *(const int4 *)(S + kA8 + l32 * 64 + 16 * i);
          s16[4 * i] = v4.x;
          s16[4 * i + 1] = v4.y;
          s16[4 * i + 2] = v4.z;
          s16[4 * i + 3] = v4.w;
        }
        // Roles: A = the 32 rows' int8 pieces, B = the weight operands, so in
        // the 32x32 result lane l holds weight row l % 32 (its own head's d,
        // dmin) for the rows 8*(v/4) + 4*(l/32) + v%4 of the item.
        v8f16 bm, amn;
        v16i32 H = v16i32{0}, L = v16i32{0};
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int sj = s16[2 * j] + s16[2 * j + 1];
          const int hj = sj >> 6;  // floor: sj = 64*hj + (sj - 64*hj), the second part in [0, 64)
          bm[j] = (_Float16)(half ? sj - 64 * hj : hj);
          amn[j] = (_Float16)(half ? mn[j] : 64 * mn[j]);
          const v4i32 bv = *(const v4i32 *)(S + l32 * 256 + (((2 * j + half) ^ (l32 & 7)) * 16));
          const u32x4 w = wq[j >> 1];
          const uint32_t msk = 0x0f0f0f0fu;
          const int s4 = (j & 1) ? 4 : 0;
          const uint32_t n0 = (w.x >> s4) & msk, n1 = (w.y >> s4) & msk, n2 = (w.z >> s4) & msk,
                         n3 = (w.w >> s4) & msk;
          const uint32_t hi = (uint32_t)(sc[j] >> 3), lo = (uint32_t)(sc[j] & 7);
          const v4i32 ahi = v4i32{mul_bytes(n0, hi), mul_bytes(n1, hi), mul_bytes(n2, hi), mul_bytes(n3, hi)};
          const v4i32 alo = v4i32{mul_bytes(n0, lo), mul_bytes(n1, lo), mul_bytes(n2, lo), mul_bytes(n3, lo)};
          H = __builtin_amdgcn_mfma_i32_32x32x32_i8(bv, ahi, H, 0, 0, 0);
          L = __builtin_amdgcn_mfma_i32_32x32x32_i8(bv, alo, L, 0, 0, 0);
        }
        const v16f32 N = __builtin_amdgcn_mfma_f32_32x32x16_f16(bm, amn, v16f32{0}, 0, 0, 0);
        const v16i32 SI = (H << 3) + L;
        if constexpr (DBG) {
          const int k = ck, n = it_n[k];
          const int64_t rw = (int64_t)it_rb[k] * RI + tile * 32 + l32;
          if (rw < rows) {
            int32_t *ds = a.dbg.s[mat == 1 ? 1 : 0], *dm = a.dbg.m[mat == 1 ? 1 : 0];
#pragma unroll
            for (int v = 0; v < 16; ++v) {
              const int t = 8 * (v >> 2) + 4 * half + (v & 3);
              if (t < n) {
                const int64_t o = (((int64_t)it_p0[k] + t) * rows + rw) * nb + bb;
                ds[o] = SI[v];
                dm[o] = (int)N[v];
              }
            }
          }
        }
        const float d = f16_bits_to_f32(hd.x), dmin = f16_bits_to_f32(hd.x >> 16);
        const float *adl = (const float *)(stg[slot] + kAd + wave * 256);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 a4 = *(const float4 *)(adl + 8 * g + 4 * half);
          const float at[4] = {a4.x, a4.y, a4.z, a4.w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int v = 4 * g + c;
            const float x = fmaf(d, (float)SI[v], -(dmin * N[v]));
            y[v] = fmaf(at[c], x, y[v]);
          }
        }
      }
    }
    if (cb == SPI - 1) {  // the item is complete: hand-over, SwiGLU or the parts' sum, store
      const int k = ck;
      if (grp == 1) {
#pragma unroll
        for (int g = 0; g < 4; ++g)
          lds_store16(&xch[tile * 32 + l32][8 * g + 4 * half], v4f32{y[4 * g], y[4 * g + 1], y[4 * g + 2], y[4 * g + 3]});
      }
      __builtin_amdgcn_s_waitcnt((15 | (3 << 14)) | (7 << 4));  // lgkmcnt(0): the hand-over is written
      ring_barrier();
      if (grp == 0) {
        const int n = it_n[k];
        const int64_t p0 = it_p0[k], rw = (int64_t)it_rb[k] * RI + tile * 32 + l32;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 o4 = *(const float4 *)&xch[tile * 32 + l32][8 * g + 4 * half];
          const float ov[4] = {o4.x, o4.y, o4.z, o4.w};
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const int t = 8 * g + 4 * half + c;
            float o;
            if constexpr (MODE == MF_GATE_UP) {
              const float gv = y[4 * g + c];
              const float den = 1.0f + expf_cr(-gv);  // SwiGLU: g / (1 + exp(-g)) * u
              o = gv / den * ov[c];
            } else {
              o = y[4 * g + c] + ov[c];
            }
            if (t < n && rw < rows) a.out[(p0 + t) * rows + rw] = o;
          }
        }
      }
#pragma unroll
      for (int v = 0; v < 16; ++v) y[v] = 0.0f;
    }
    const bool wrap = cb == SPI - 1;
    ck = wrap ? ck + 1 : ck;
    cb = wrap ? 0 : cb + 1;
  };

  constexpr int kWait = (NS - 2) * OPS;
  // s_waitcnt: vmcnt(kWait), expcnt(7), lgkmcnt(0)
  constexpr int kWaitEnc = (kWait & 15) | ((kWait >> 4) << 14) | (7 << 4);
#pragma unroll
  for (int u = 0; u < NS - 1; ++u) issue(u);
  // Every pass of the body issues the same loads (stages past the last are
  // clamped re-loads), so the compiler's wait counts stay exact.
  for (int s0 = 0; s0 < T; s0 += NS) {
#pragma unroll
    for (int u = 0; u < NS; ++u) {
      __builtin_amdgcn_s_waitcnt(kWaitEnc);  // this wave's loads of stage s0+u are in, its LDS reads done
      ring_barrier();                        // every wave's, so the slot refilled next is free too
      issue((u + NS - 1) % NS);
      if (s0 + u < T) consume(u);
    }
  }
  __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8));  // vmcnt(0): no direct load outlives the work-group
}

int g_mfma_cus = 0;
int mfma_cus() {
  if (g_mfma_cus == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      g_mfma_cus = n;
    else
      g_mfma_cus = 256;
  }
  return g_mfma_cus;
}

bool aligned16(const void *p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

bool moe_mfma_supported(int64_t rows, int64_t cols) {
  return rows > 0 && cols > 0 && cols % 256 == 0 && rows < (1ll << 31) / 32 && cols / 256 < (1ll << 24);
}

template <int MODE, bool DBG>
hipError_t launch_ring(hipStream_t st, dim3 grid, const MfmaArgs &a) {
  // two stages: one in flight beside the one being multiplied
  KMOE_LAUNCH((k_moe_mfma_ring<MODE, 2, DBG>), grid, dim3(kRingWaves<MODE> * 64), 0, st, a);
  return hipGetLastError();
}

hipError_t launch_moe_mfma(hipStream_t st, int mode, const ExpertTier &tier, int64_t rows, int64_t cols,
                           const Routing &rt, int regime, int max_active, const int8_t *aq, const float *ad,
                           const int32_t *abs, float *out, int min_rows, int max_rows, int ring_rows,
                           const BlockDbg *dbg) {
  if (!moe_mfma_supported(rows, cols) || !aligned16(aq) || !aligned16(abs)) return hipErrorNotSupported;
  if (max_active == 0 || max_rows < min_rows) return hipSuccess;
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
  a.min_rows = min_rows;
  a.max_rows = max_rows;
  if (dbg) a.dbg = *dbg;
  ring_rows = ring_rows < kRingTok ? ring_rows : kRingTok;
  if (min_rows <= ring_rows && max_active <= kRingExperts) {
    // experts with min_rows..32 rows: the streaming kernel, (expert, 64- or 128-row) items,
    // eight waves per CU
    const int nw = mode == MF_GATE_UP ? kRingWaves<MF_GATE_UP> : kRingWaves<MF_DOWN>;
    const int64_t upper = (int64_t)max_active * ((rows + 16 * nw - 1) / (16 * nw));
    int64_t g = (int64_t)mfma_cus() * (8 / nw);
    g = g < upper ? g : upper;
    const int64_t gmin = (upper + kRingItems - 1) / kRingItems;
    g = g > gmin ? g : gmin;
    if (g > 0 && g < (1ll << 31)) {
      MfmaArgs r = a;
      r.max_rows = ring_rows;
      hipError_t e;
      if (mode == MF_GATE_UP) e = dbg ? launch_ring<MF_GATE_UP, true>(st, dim3((unsigned)g), r)
                                      : launch_ring<MF_GATE_UP, false>(st, dim3((unsigned)g), r);
      else e = dbg ? launch_ring<MF_DOWN, true>(st, dim3((unsigned)g), r)
                   : launch_ring<MF_DOWN, false>(st, dim3((unsigned)g), r);
      if (e != hipSuccess) return e;
      if (max_rows <= ring_rows) return hipSuccess;
      a.min_rows = ring_rows + 1;
    }
  }
  const int64_t rows_per_wg = 128;
  const dim3 grid((unsigned)((rows + rows_per_wg - 1) / rows_per_wg), (unsigned)max_active);
  if (mode == MF_GATE_UP) {
    if (dbg) KMOE_LAUNCH((k_moe_mfma<MF_GATE_UP, true>), grid, dim3(512), 0, st, a);
    else KMOE_LAUNCH((k_moe_mfma<MF_GATE_UP>), grid, dim3(512), 0, st, a);
  } else {
    if (dbg) KMOE_LAUNCH((k_moe_mfma<MF_DOWN, true>), grid, dim3(512), 0, st, a);
    else KMOE_LAUNCH((k_moe_mfma<MF_DOWN>), grid, dim3(512), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_plain_mfma(hipStream_t st, const uint8_t *w, int64_t rows, int64_t cols, const int8_t *aq,
                             const float *ad, const int32_t *abs, int64_t s_rows, float *out, int32_t *sumi,
                             int32_t *mins) {
  if (!moe_mfma_supported(rows, cols) || !aligned16(aq) || !aligned16(abs) || ((uintptr_t)w & 3u) ||
      s_rows > (int64_t)kTok * 65535)
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
  a.max_rows = 1 << 30;
  const dim3 grid((unsigned)((rows + 127) / 128), (unsigned)((s_rows + kTok - 1) / kTok));
  if (sumi) KMOE_LAUNCH((k_moe_mfma<MF_SUMS>), grid, dim3(512), 0, st, a);
  else KMOE_LAUNCH((k_moe_mfma<MF_PLAIN>), grid, dim3(512), 0, st, a);
  return hipGetLastError();
}

}  // namespace kmoe
