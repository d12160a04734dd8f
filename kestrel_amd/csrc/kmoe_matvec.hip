// kmoe_matvec.hip — int8-activation matvecs over GGUF blocks (the decode path).
//
// Arithmetic (per weight row r, activation row s):
//   Q4_K x Q8_K (avx2.rs:351-379): per superblock b,
//     sumi_b = sum_j sc_j * sum_{32 elems of j} q*x,  mins_b = sum_j m_j * (bsum pair of j)
//     y += (d_b * xd_b) * sumi_b - (dmin_b * xd_b) * mins_b
//   Q8_0 x Q8 (avx2.rs:49-58): per block b, p_b = sum q*x, y += (d_b * xd_b) * p_b
//   Q6_K x Q8_K (avx2.rs:384-419): per superblock b, with 6-bit q in 0..63 and
//     signed 16-element scales sc_g, t_b = sum_g sc_g * (sum_{16 elems} q*x - 32 * bsum_g)
//     y += (d_b * xd_b) * t_b
// The integers are exact (int32, no saturation: max |pair| is 2*15*127 for
// Q4_K and 2*128*127 for Q8_0), so sumi_b, mins_b and p_b equal the
// reference's bit for bit; the fp32 epilogue sums in a different order, which
// moves the result by a few ulp (checked against a 1e-3 relative L2 bound).
//
// Layout and mapping. Plain matvecs read GGUF bytes; the grouped (expert)
// kernels read the expert tier, whose Q4_K rows are tiled (tq4_qs_off in
// kmoe_device.h). A Q4_K "task" is one quarter of a 144-byte superblock: the
// 16-byte header (d, dmin, 12 scale bytes) plus 32 bytes of nibbles (64
// weights of sub-blocks 2k and 2k+1). Lanes take consecutive tasks, so in the
// tiled layout each wave load instruction covers one or two contiguous runs of
// bytes. A Q8_0 task is one 34-byte block, read as nine
// dwords from the dword-aligned address below it. LPR lanes share a row
// (LPR = 64 for 4096-wide Q4_K rows: one row per wave per step); they reduce
// with DPP and cross-row shuffles. Activations (int8 rows, their scales and
// 16-sums) are staged once per work-group in LDS; each lane reads its 64
// activation bytes with ds_read_b128.
#include "kmoe_device.h"
#include "kmoe_launch.h"
#include "kmoe_select.h"

#include <cstdlib>
#include <type_traits>
#include <cstring>

namespace kmoe {

namespace {

struct MvArgs {
  const uint8_t *w0;
  int64_t rows, cols;
  const int8_t *xq;
  const float *xd;
  const int32_t *xbs;
  int64_t s_rows;
  float *out;
  int32_t *isumi, *imins;
  ExpertTier tier;
  Routing rt;
  int regime;
  int rows_per_block;
  int min_rows;  // grouped modes: experts with fewer rows are another kernel's
  int max_rows;  // k_few_int: experts with more rows are another kernel's
  int sel_on;    // M_GATE_UP, one token: select the experts from sel.logits here
  DecSelect sel;
  QkvRope rope;  // M_QKV: the epilogue of the one-token q/k/v projection
  BlockDbg dbg;  // grouped modes: per-block integers of the part(s) computed
  int add;        // M_PLAIN: out[r] = out[r] + scale * y (AddEpi) instead of out[r] = y
  int32_t chunk;  // LDS-staged plain modes: activation rows per work-group (blockIdx.y picks the chunk)
  const float *add_logit;
  const float *xf;  // M_PLAIN_FX: the f32 activation row
  // M_GATE_UP, one token: the shared expert's gate rows (GGUF, sgu_rows of
  // them, its up rows right after) as extra items, SwiGLU into sgu_h
  const uint8_t *sgu_w;
  int64_t sgu_rows;
  float *sgu_h;
  // k_mv_down_exp with SHT != 0: the shared expert's down rows (GGUF, sh_cols
  // columns) against its int8 row, added after the routed combine
  const uint8_t *sh_w;
  int64_t sh_cols;
  const int8_t *sh_xq;
  const float *sh_xd;
  const int32_t *sh_xbs;
  const float *sh_logit;
  // M_QKV_NORM: the residual add and RMSNorm of the one-token row in front
  // (wg_residual_rmsnorm of nx + ny with weights nw); work-group 0 stores
  // nx + ny into nxo (another buffer: nx stays as it was) and the normed row
  // into nh
  const float *nx;
  const float *ny, *nw;
  float neps;
  float *nxo;
  float *nh;
};

enum { M_PLAIN = 0, M_GATE_UP = 1, M_DOWN = 2, M_SUMS = 3 };
enum { M_QKV = 5 };
// M_PLAIN with the f32 activation row (a.xf) quantized to Q8_K inside the
// kernel (K-quant rows of at most kRegFxBlocks superblocks)
enum { M_PLAIN_FX = 6 };
constexpr int kRegFxBlocks = 16;
// M_QKV whose activation row is the residual add and RMSNorm of nx (+ ny),
// formed and quantized to Q8_K inside the kernel as M_PLAIN_FX does
enum { M_QKV_NORM = 7 };

// The RoPE + KV store epilogue of a one-token q/k/v projection with
// interleaved pairs (rows 2i and 2i+1 of a head, dims below rope_dim) or
// neox pairs over the whole head (rows i and i + hd/2): row r
// of q rotates into q_out, of k into the f16 K cache at the position, of v
// goes to the f16 V cache; the raw projection is stored in out as well. The
// expressions are k_rope_kv's: x0*cos - x1*sin for the first of a pair,
// x0*sin + x1*cos for the second, sincosf of (float)position * inv_freq[i].
// With neox (rope_dim == head_dim) the kernel runs the rows of a head in the
// order qkv_row gives, so a wave step's two rows are a pair (i, i + hd/2).
__device__ __forceinline__ int64_t qkv_row(const QkvRope &q, int64_t r) {
  if (!q.neox || r >= (int64_t)(q.nh + q.nkv) * q.hd) return r;  // v rows keep their order
  const int64_t dd = r % q.hd, hb = r - dd;
  return hb + ((dd & 1) ? (dd >> 1) + q.hd / 2 : dd >> 1);
}
__device__ __forceinline__ void qkv_rope_store(const QkvRope &q, int64_t r, float v, float partner) {
  const int64_t nqr = (int64_t)q.nh * q.hd, kvw = (int64_t)q.nkv * q.hd;
  const int64_t p = q.pos0 + (q.pos_dev ? (int64_t)*q.pos_dev : 0);
  if (r < nqr + kvw) {
    const int dd = (int)(r % q.hd);
    float val = v;
    if (dd < q.rd) {
      // pairs (2i, 2i+1), or with neox (i, i + rd/2)
      const int hr = q.rd >> 1;
      const int i = q.neox ? (dd < hr ? dd : dd - hr) : dd >> 1;
      const bool first = q.neox ? dd < hr : (dd & 1) == 0;
      const float ang = (float)p * q.inv_freq[i];
      float sv, cv;
      sincosf(ang, &sv, &cv);
      const float x0 = first ? v : partner, x1 = first ? partner : v;
      val = first ? x0 * cv - x1 * sv : x0 * sv + x1 * cv;
    }
    if (r < nqr) q.q_out[r] = val;
    else if (p >= 0 && p < q.n_ctx) q.kc[p * kvw + (r - nqr)] = __builtin_bit_cast(uint16_t, (_Float16)val);
  } else if (p >= 0 && p < q.n_ctx) {
    q.vc[p * kvw + (r - nqr - kvw)] = __builtin_bit_cast(uint16_t, (_Float16)v);
  }
}

__device__ __forceinline__ bool int_regime(int regime, int n) {
  return regime == REGIME_INT8 || (regime == REGIME_AVX2 && n < 4);
}

// Block geometry per weight type: elements and bytes per block, tasks per
// block (a K-quant task is a quarter superblock, 64 weights).
template <int TYPE>
struct QT;
template <>
struct QT<T_Q4_K> {
  static constexpr int EL = 256, BYTES = 144, TPB = 4;
};
template <>
struct QT<T_Q6_K> {
  static constexpr int EL = 256, BYTES = 210, TPB = 4;
};
template <>
struct QT<T_Q8_0> {
  static constexpr int EL = 32, BYTES = 34, TPB = 1;
};

// Bytes per activation row in LDS, 16-byte aligned pieces: q, sums, scales.
template <int TYPE>
struct ActLayout {
  int64_t q, s, d, total;
  __host__ __device__ ActLayout(int64_t cols) {
    q = (cols + 15) & ~15ll;
    s = is_kquant(TYPE) ? ((cols / 16 * 4 + 15) & ~15ll) : 0;  // Q8_0 never reads the 16-sums
    const int64_t nd = cols / QT<TYPE>::EL;
    d = (nd * 4 + 15) & ~15ll;
    total = q + s + d;
  }
};

struct Q4kW {
  uint4 hdr, qa, qb;
};

// Weights are read once per token: non-temporal loads keep them from
// displacing the activations in the caches.
typedef uint32_t u32x4nt __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ld_nt(const uint8_t *p) {
  const u32x4nt v = __builtin_nontemporal_load((const u32x4nt *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Task t of a row of nb superblocks, GGUF bytes or tiled rows (expert tier).
template <bool TILED>
__device__ __forceinline__ Q4kW q4k_load(const uint8_t *row, int t, int64_t nb) {
  const int64_t sb = t >> 2;
  const int k = t & 3;
  Q4kW w;
  if constexpr (TILED) {
    const uint8_t *qa = row + tq4_qs_off(nb, sb, k, 0);
    w.hdr = ld_nt(row + 16 * sb);
    w.qa = ld_nt(qa);
    w.qb = ld_nt(qa + tq4_j_stride(nb, sb));
  } else {
    const uint8_t *s = row + sb * 144;
    w.hdr = ld_nt(s);
    w.qa = ld_nt(s + 16 + 32 * k);
    w.qb = ld_nt(s + 32 + 32 * k);
  }
  return w;
}

// Integer part of one Q4_K task against one Q8_K row (xq/xbs at the superblock).
__device__ __forceinline__ void q4k_ints(const Q4kW &w, int k, const int8_t *xq_sb, const int32_t *xbs_sb, int &sumi,
                                         int &mins) {
  int sA, mA, sB, mB;
  q4k_scale_min_pair(w.hdr.y, w.hdr.z, w.hdr.w, k, sA, mA, sB, mB);
  const int4 *xv = (const int4 *)(xq_sb + 64 * k);
  const int4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
  const uint32_t m = 0x0f0f0f0fu;
  int lo = 0, hi = 0;
  lo = sdot4(w.qa.x & m, (uint32_t)x0.x, lo);
  lo = sdot4(w.qa.y & m, (uint32_t)x0.y, lo);
  lo = sdot4(w.qa.z & m, (uint32_t)x0.z, lo);
  lo = sdot4(w.qa.w & m, (uint32_t)x0.w, lo);
  lo = sdot4(w.qb.x & m, (uint32_t)x1.x, lo);
  lo = sdot4(w.qb.y & m, (uint32_t)x1.y, lo);
  lo = sdot4(w.qb.z & m, (uint32_t)x1.z, lo);
  lo = sdot4(w.qb.w & m, (uint32_t)x1.w, lo);
  hi = sdot4((w.qa.x >> 4) & m, (uint32_t)x2.x, hi);
  hi = sdot4((w.qa.y >> 4) & m, (uint32_t)x2.y, hi);
  hi = sdot4((w.qa.z >> 4) & m, (uint32_t)x2.z, hi);
  hi = sdot4((w.qa.w >> 4) & m, (uint32_t)x2.w, hi);
  hi = sdot4((w.qb.x >> 4) & m, (uint32_t)x3.x, hi);
  hi = sdot4((w.qb.y >> 4) & m, (uint32_t)x3.y, hi);
  hi = sdot4((w.qb.z >> 4) & m, (uint32_t)x3.z, hi);
  hi = sdot4((w.qb.w >> 4) & m, (uint32_t)x3.w, hi);
  sumi = sA * lo + sB * hi;
  const int4 bs = *(const int4 *)(xbs_sb + 4 * k);
  mins = mA * (bs.x + bs.y) + mB * (bs.z + bs.w);
}

// Q6_K (quant.rs:180-201): 210-byte superblocks of ql[128] (low 4 bits),
// qh[64] (high 2 bits), sc[16] (signed scales of 16 elements) and the f16 d at
// byte 208. Task t is quarter k of superblock t/4: half h = k/2, nibble
// p = k%2. Its 64 weights are rows ri = 2p (weights 0-31) and 2p+1 (32-63) of
// half h; weight l of row ri is nibble p of ql[64h + 32*(ri&1) + l] with bits
// 2ri..2ri+1 of qh[32h + l] above it, scaled by sc[8h + 2ri + l/16]. Both
// tasks of a half need all 64 ql and 32 qh bytes of it: the two lanes holding
// tasks 2h and 2h+1 (adjacent lanes) each load one half of those bytes (lane
// p: ql[64h + 32p, +32) and qh[32h + 16p, +16)) and swap them at use with a
// DPP move. Superblocks start on 2-byte boundaries; the 16-byte loads rely on
// the target's unaligned global access.
struct Q6kW {
  uint4 l0, l1;  // ql[64h + 32p, 64h + 32p + 32)
  uint4 hq;      // qh[32h + 16p, 32h + 16p + 16)
  uint32_t sc;   // sc[8h+4p, 8h+4p+4)
  uint32_t d;    // f16 bits of d
};
typedef uint32_t u32x4u2 __attribute__((ext_vector_type(4), aligned(2)));
typedef uint32_t u32u2 __attribute__((aligned(2)));
__device__ __forceinline__ uint4 ld_nt_u2(const uint8_t *p) {
  const u32x4u2 v = __builtin_nontemporal_load((const u32x4u2 *)p);
  return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ Q6kW q6k_load(const uint8_t *row, int t) {
  const int64_t sb = t >> 2;
  const int k = t & 3, h = k >> 1, p = k & 1;
  const uint8_t *b = row + sb * 210;
  Q6kW w;
  w.l0 = ld_nt_u2(b + 64 * h + 32 * p);
  w.l1 = ld_nt_u2(b + 64 * h + 32 * p + 16);
  w.hq = ld_nt_u2(b + 128 + 32 * h + 16 * p);
  w.sc = __builtin_nontemporal_load((const u32u2 *)(b + 192 + 8 * h + 4 * p));
  w.d = __builtin_nontemporal_load((const uint16_t *)(b + 208));
  return w;
}
// Integer part of one Q6_K task: sumi = sum_g sc_g * sum q*x over its four
// 16-weight groups, offs = sum_g sc_g * bsum_g (avx2.rs:398-414). Every lane
// of the wave's active quads must call it together (the partner exchange).
__device__ __forceinline__ void q6k_ints(const Q6kW &w, int k, const int4 &x0, const int4 &x1, const int4 &x2,
                                         const int4 &x3, const int4 &bs, int &sumi, int &offs) {
  const bool p = (k & 1) != 0;
  const uint32_t own[12] = {w.l0.x, w.l0.y, w.l0.z, w.l0.w, w.l1.x, w.l1.y, w.l1.z, w.l1.w,
                            w.hq.x, w.hq.y, w.hq.z, w.hq.w};
  uint32_t L[16], H[8];
#pragma unroll
  for (int i = 0; i < 12; ++i) {
    const uint32_t o = (uint32_t)dpp_i<kDppXor1>((int)own[i]);  // the partner lane's half
    if (i < 8) {
      L[i] = p ? o : own[i];
      L[8 + i] = p ? own[i] : o;
    } else {
      H[i - 8] = p ? o : own[i];
      H[i - 4] = p ? own[i] : o;
    }
  }
  const int sn = p ? 4 : 0;  // nibble shift; the qh bits of row 2p sit at 4p, of row 2p+1 at 4p+2
  const uint32_t m4 = 0x0f0f0f0fu, m2 = 0x03030303u;
  const uint32_t X[16] = {(uint32_t)x0.x, (uint32_t)x0.y, (uint32_t)x0.z, (uint32_t)x0.w,
                          (uint32_t)x1.x, (uint32_t)x1.y, (uint32_t)x1.z, (uint32_t)x1.w,
                          (uint32_t)x2.x, (uint32_t)x2.y, (uint32_t)x2.z, (uint32_t)x2.w,
                          (uint32_t)x3.x, (uint32_t)x3.y, (uint32_t)x3.z, (uint32_t)x3.w};
  int g[4] = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t qa = ((L[i] >> sn) & m4) | (((H[i] >> sn) & m2) << 4);
    const uint32_t qb = ((L[8 + i] >> sn) & m4) | (((H[i] >> (sn + 2)) & m2) << 4);
    g[i >> 2] = sdot4(qa, X[i], g[i >> 2]);
    g[2 + (i >> 2)] = sdot4(qb, X[8 + i], g[2 + (i >> 2)]);
  }
  const int s0 = (int)(int8_t)(w.sc & 0xff), s1 = (int)(int8_t)((w.sc >> 8) & 0xff);
  const int s2 = (int)(int8_t)((w.sc >> 16) & 0xff), s3 = (int)(int8_t)(w.sc >> 24);
  sumi = s0 * g[0] + s1 * g[1] + s2 * g[2] + s3 * g[3];
  offs = s0 * bs.x + s1 * bs.y + s2 * bs.z + s3 * bs.w;
}

// Task t of a tiled Q6_K row of the expert tier (tq6_piece_off): nibbles
// n0/n1 (byte b: weight b of the first row low, of the second row high), high
// bits hb (byte b: weights b and b+16), the task's four scales and d.
struct Q6kT {
  uint4 n0, n1, hb;
  uint32_t sc;
  uint32_t d;
};
__device__ __forceinline__ Q6kT q6t_load(const uint8_t *row, int t, int64_t nb) {
  const int64_t sb = t >> 2;
  const int k = t & 3;
  const uint8_t *p0 = row + tq6_piece_off(nb, sb, k, 0);
  const int64_t js = tq6_j_stride(nb, sb);
  Q6kT w;
  w.n0 = ld_nt_u2(p0);
  w.n1 = ld_nt_u2(p0 + js);
  w.hb = ld_nt_u2(p0 + 2 * js);
  w.sc = __builtin_nontemporal_load((const u32u2 *)(row + 192 * nb + 16 * sb + 4 * k));
  w.d = __builtin_nontemporal_load((const uint16_t *)(row + 208 * nb + 2 * sb));
  return w;
}
__device__ __forceinline__ void q6t_ints(const Q6kT &w, const int4 &x0, const int4 &x1, const int4 &x2, const int4 &x3,
                                         const int4 &bs, int &sumi, int &offs) {
  const uint32_t m4 = 0x0f0f0f0fu, m2 = 0x03030303u;
  const uint32_t N[8] = {w.n0.x, w.n0.y, w.n0.z, w.n0.w, w.n1.x, w.n1.y, w.n1.z, w.n1.w};
  const uint32_t H[4] = {w.hb.x, w.hb.y, w.hb.z, w.hb.w};
  const uint32_t X[16] = {(uint32_t)x0.x, (uint32_t)x0.y, (uint32_t)x0.z, (uint32_t)x0.w,
                          (uint32_t)x1.x, (uint32_t)x1.y, (uint32_t)x1.z, (uint32_t)x1.w,
                          (uint32_t)x2.x, (uint32_t)x2.y, (uint32_t)x2.z, (uint32_t)x2.w,
                          (uint32_t)x3.x, (uint32_t)x3.y, (uint32_t)x3.z, (uint32_t)x3.w};
  int g[4] = {0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t hs = i < 4 ? H[i] : (H[i - 4] >> 4);  // weights 4i..4i+3: low nibbles, then high
    const uint32_t qa = (N[i] & m4) | ((hs & m2) << 4);
    const uint32_t qb = ((N[i] >> 4) & m4) | (((hs >> 2) & m2) << 4);
    g[i >> 2] = sdot4(qa, X[i], g[i >> 2]);
    g[2 + (i >> 2)] = sdot4(qb, X[8 + i], g[2 + (i >> 2)]);
  }
  const int s0 = (int)(int8_t)(w.sc & 0xff), s1 = (int)(int8_t)((w.sc >> 8) & 0xff);
  const int s2 = (int)(int8_t)((w.sc >> 16) & 0xff), s3 = (int)(int8_t)(w.sc >> 24);
  sumi = s0 * g[0] + s1 * g[1] + s2 * g[2] + s3 * g[3];
  offs = s0 * bs.x + s1 * bs.y + s2 * bs.z + s3 * bs.w;
}

struct Q80W {
  uint4 a, b;
  uint32_t c;
  int sh;  // 0: block starts on a dword, 2: two bytes past one
};

__device__ __forceinline__ Q80W q80_load(const uint8_t *row, int t) {
  const uintptr_t addr = (uintptr_t)(row + (int64_t)t * 34);
  const uint8_t *base = (const uint8_t *)(addr & ~(uintptr_t)3);
  Q80W w;
  w.sh = (int)(addr & 3);
  w.a = load_u4_a4(base);
  w.b = load_u4_a4(base + 16);
  w.c = *(const uint32_t *)(base + 32);
  return w;
}

__device__ __forceinline__ int q80_int(const Q80W &w, const int8_t *xq_b, float &dw) {
  const uint32_t v[9] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w, w.c};
  uint32_t q[8];
  if (w.sh == 0) {
    dw = f16_bits_to_f32(v[0]);
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], 2);
  } else {
    dw = f16_bits_to_f32(v[0] >> 16);
#pragma unroll
    for (int i = 0; i < 8; ++i) q[i] = v[i + 1];
  }
  const int4 *xv = (const int4 *)xq_b;
  const int4 x0 = xv[0], x1 = xv[1];
  int p = 0;
  p = sdot4(q[0], (uint32_t)x0.x, p);
  p = sdot4(q[1], (uint32_t)x0.y, p);
  p = sdot4(q[2], (uint32_t)x0.z, p);
  p = sdot4(q[3], (uint32_t)x0.w, p);
  p = sdot4(q[4], (uint32_t)x1.x, p);
  p = sdot4(q[5], (uint32_t)x1.y, p);
  p = sdot4(q[6], (uint32_t)x1.z, p);
  p = sdot4(q[7], (uint32_t)x1.w, p);
  return p;
}

// DBG: the grouped modes also add their per-block integers into a.dbg (the
// capture of kmoe_moe_ffn_dbg).
template <int TYPE, int LPR, int NT, int MODE, bool DBG>
__global__ void __launch_bounds__(256) k_matvec_int(MvArgs a) {
  extern __shared__ __attribute__((aligned(16))) char smem[];
  constexpr int RPW = 64 / LPR;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row_in_wave = lane / LPR, lr = lane % LPR;
  const int64_t cols = a.cols, rows = a.rows;
  const int64_t nblk = cols / QT<TYPE>::EL;
  const int ntasks = (int)(QT<TYPE>::TPB * nblk);
  const int64_t row_bytes = nblk * QT<TYPE>::BYTES;
  const int64_t xs_stride = cols / 16, xd_stride = nblk;
  const ActLayout<TYPE> L(cols);

  int n, c_begin = 0;
  int64_t p0 = 0;
  const uint8_t *W0 = a.w0, *W1 = nullptr;
  if constexpr (MODE == M_PLAIN || MODE == M_SUMS) {
    c_begin = (int)blockIdx.y * a.chunk;
    n = (int)(a.s_rows < (int64_t)c_begin + a.chunk ? a.s_rows : (int64_t)c_begin + a.chunk);
  } else {
    const int i = blockIdx.y;
    if (i >= *a.rt.n_active) return;
    const int e = a.rt.active[i];
    p0 = a.rt.offsets[e];
    n = (int)(a.rt.offsets[e + 1] - p0);
    if (n < a.min_rows || !int_regime(a.regime, n)) return;
    const uint8_t *eb = a.tier.base + (int64_t)e * a.tier.stride;
    if constexpr (MODE == M_GATE_UP) {
      W0 = eb + a.tier.off[0];
      W1 = eb + a.tier.off[1];
    } else {
      W0 = eb + a.tier.off[2];
    }
  }
  const int64_t r_begin = (int64_t)blockIdx.x * a.rows_per_block;
  const int64_t r_end = r_begin + a.rows_per_block < rows ? r_begin + a.rows_per_block : rows;

  for (int c0 = c_begin; c0 < n; c0 += NT) {
    const int nt = n - c0 < NT ? n - c0 : NT;
    // ---- stage the activation rows of tokens c0..c0+nt in LDS
    for (int t = 0; t < nt; ++t) {
      int64_t src;
      if constexpr (MODE == M_GATE_UP) src = a.rt.perm[p0 + c0 + t] / a.rt.topk;
      else if constexpr (MODE == M_DOWN) src = p0 + c0 + t;
      else src = c0 + t;
      char *dst = smem + t * L.total;
      const uint32_t *sq = (const uint32_t *)(a.xq + src * cols);
      for (int64_t i = threadIdx.x; i < cols / 4; i += 256) ((uint32_t *)dst)[i] = sq[i];
      if constexpr (is_kquant(TYPE)) {
        const int32_t *ss = a.xbs + src * xs_stride;
        for (int64_t i = threadIdx.x; i < xs_stride; i += 256) ((int32_t *)(dst + L.q))[i] = ss[i];
      }
      const float *sd = a.xd + src * xd_stride;
      for (int64_t i = threadIdx.x; i < xd_stride; i += 256) ((float *)(dst + L.q + L.s))[i] = sd[i];
    }
    __syncthreads();

    for (int64_t rb = r_begin + (int64_t)wave * RPW; rb < r_end; rb += 4 * RPW) {
      const int64_t r = rb + row_in_wave;
      const bool valid = r < r_end;
      float acc0[NT], acc1[NT];
#pragma unroll
      for (int t = 0; t < NT; ++t) acc0[t] = acc1[t] = 0.0f;
      if (valid) {
        const uint8_t *row0 = W0 + r * row_bytes;
        const uint8_t *row1 = MODE == M_GATE_UP ? W1 + r * row_bytes : nullptr;
        for (int t = lr; t < ntasks; t += LPR) {
          if constexpr (TYPE == T_Q4_K) {
            const int sb = t >> 2, k = t & 3;
            constexpr bool TL = MODE == M_GATE_UP || MODE == M_DOWN;  // expert tier rows are tiled
            const Q4kW w0 = q4k_load<TL>(row0, t, nblk);
            Q4kW w1;
            if constexpr (MODE == M_GATE_UP) w1 = q4k_load<TL>(row1, t, nblk);
            const float d0 = f16_bits_to_f32(w0.hdr.x), m0 = f16_bits_to_f32(w0.hdr.x >> 16);
#pragma unroll
            for (int tk = 0; tk < NT; ++tk) {
              if (tk < nt) {
                const char *act = smem + tk * L.total;
                const int8_t *xq_sb = (const int8_t *)act + sb * 256;
                const int32_t *xbs_sb = (const int32_t *)(act + L.q) + sb * 16;
                const float xd = ((const float *)(act + L.q + L.s))[sb];
                int si, mi;
                q4k_ints(w0, k, xq_sb, xbs_sb, si, mi);
                if constexpr (MODE == M_SUMS) {
                  const int ss = group_sum_i<4>(si), ms = group_sum_i<4>(mi);
                  if (k == 0) {
                    const int64_t o = ((int64_t)(c0 + tk) * rows + r) * nblk + sb;
                    a.isumi[o] = ss;
                    a.imins[o] = ms;
                  }
                } else {
                  const int64_t o = ((p0 + c0 + tk) * rows + r) * nblk + sb;  // grouped modes' capture
                  if (DBG && a.dbg.s[0]) {
                    atomicAdd(a.dbg.s[0] + o, si);
                    atomicAdd(a.dbg.m[0] + o, mi);
                  }
                  acc0[tk] = fmaf(d0 * xd, (float)si, acc0[tk]);
                  acc0[tk] = fmaf(-(m0 * xd), (float)mi, acc0[tk]);
                  if constexpr (MODE == M_GATE_UP) {
                    const float d1 = f16_bits_to_f32(w1.hdr.x), m1 = f16_bits_to_f32(w1.hdr.x >> 16);
                    q4k_ints(w1, k, xq_sb, xbs_sb, si, mi);
                    if (DBG && a.dbg.s[1]) {
                      atomicAdd(a.dbg.s[1] + o, si);
                      atomicAdd(a.dbg.m[1] + o, mi);
                    }
                    acc1[tk] = fmaf(d1 * xd, (float)si, acc1[tk]);
                    acc1[tk] = fmaf(-(m1 * xd), (float)mi, acc1[tk]);
                  }
                }
              }
            }
          } else if constexpr (TYPE == T_Q6_K) {
            const int sb = t >> 2, k = t & 3;
            constexpr bool TL = MODE == M_GATE_UP || MODE == M_DOWN;  // expert tier rows are tiled
            using W6 = typename std::conditional<TL, Q6kT, Q6kW>::type;
            auto ld6 = [&](const uint8_t *row) {
              if constexpr (TL) return q6t_load(row, t, nblk);
              else return q6k_load(row, t);
            };
            auto ints6 = [&](const W6 &w, const int4 &a0, const int4 &a1, const int4 &a2, const int4 &a3,
                             const int4 &b, int &si_, int &oi_) {
              if constexpr (TL) q6t_ints(w, a0, a1, a2, a3, b, si_, oi_);
              else q6k_ints(w, k, a0, a1, a2, a3, b, si_, oi_);
            };
            const W6 w0 = ld6(row0);
            W6 w1;
            if constexpr (MODE == M_GATE_UP) w1 = ld6(row1);
            const float d0 = f16_bits_to_f32(w0.d);
#pragma unroll
            for (int tk = 0; tk < NT; ++tk) {
              if (tk < nt) {
                const char *act = smem + tk * L.total;
                const int4 *xv = (const int4 *)((const int8_t *)act + sb * 256 + 64 * k);
                const int4 x0 = xv[0], x1 = xv[1], x2 = xv[2], x3 = xv[3];
                const int4 bs = *((const int4 *)(act + L.q) + sb * 4 + k);
                const float xd = ((const float *)(act + L.q + L.s))[sb];
                int si, oi;
                ints6(w0, x0, x1, x2, x3, bs, si, oi);
                if constexpr (MODE == M_SUMS) {
                  const int ss = group_sum_i<4>(si), os = group_sum_i<4>(oi);
                  if (k == 0) {
                    const int64_t o = ((int64_t)(c0 + tk) * rows + r) * nblk + sb;
                    a.isumi[o] = ss;
                    a.imins[o] = os;
                  }
                } else {
                  const int64_t o = ((p0 + c0 + tk) * rows + r) * nblk + sb;  // grouped modes' capture
                  if (DBG && a.dbg.s[0]) {
                    atomicAdd(a.dbg.s[0] + o, si);
                    atomicAdd(a.dbg.m[0] + o, oi);
                  }
                  acc0[tk] = fmaf(d0 * xd, (float)(si - 32 * oi), acc0[tk]);
                  if constexpr (MODE == M_GATE_UP) {
                    ints6(w1, x0, x1, x2, x3, bs, si, oi);
                    if (DBG && a.dbg.s[1]) {
                      atomicAdd(a.dbg.s[1] + o, si);
                      atomicAdd(a.dbg.m[1] + o, oi);
                    }
                    acc1[tk] = fmaf(f16_bits_to_f32(w1.d) * xd, (float)(si - 32 * oi), acc1[tk]);
                  }
                }
              }
            }
          } else {
            const Q80W w0 = q80_load(row0, t);
            Q80W w1;
            if constexpr (MODE == M_GATE_UP) w1 = q80_load(row1, t);
#pragma unroll
            for (int tk = 0; tk < NT; ++tk) {
              if (tk < nt) {
                const char *act = smem + tk * L.total;
                const int8_t *xq_b = (const int8_t *)act + t * 32;
                const float xd = ((const float *)(act + L.q + L.s))[t];
                float dw;
                const int p = q80_int(w0, xq_b, dw);
                if constexpr (MODE == M_SUMS) {
                  a.isumi[((int64_t)(c0 + tk) * rows + r) * nblk + t] = p;
                } else {
                  const int64_t o = ((p0 + c0 + tk) * rows + r) * nblk + t;  // grouped modes' capture
                  if (DBG && a.dbg.s[0]) atomicAdd(a.dbg.s[0] + o, p);
                  acc0[tk] = fmaf(dw * xd, (float)p, acc0[tk]);
                  if constexpr (MODE == M_GATE_UP) {
                    float dw1;
                    const int p1 = q80_int(w1, xq_b, dw1);
                    if (DBG && a.dbg.s[1]) atomicAdd(a.dbg.s[1] + o, p1);
                    acc1[tk] = fmaf(dw1 * xd, (float)p1, acc1[tk]);
                  }
                }
              }
            }
          }
        }
      }
      if constexpr (MODE != M_SUMS) {
#pragma unroll
        for (int tk = 0; tk < NT; ++tk) {
          acc0[tk] = group_sum<LPR>(acc0[tk]);
          if constexpr (MODE == M_GATE_UP) acc1[tk] = group_sum<LPR>(acc1[tk]);
        }
        if (valid && lr == 0) {
#pragma unroll
          for (int tk = 0; tk < NT; ++tk) {
            if (tk < nt) {
              if constexpr (MODE == M_PLAIN) {
                a.out[(int64_t)(c0 + tk) * rows + r] = acc0[tk];
              } else if constexpr (MODE == M_DOWN) {
                a.out[(p0 + c0 + tk) * rows + r] = acc0[tk];
              } else {  // SwiGLU (transformer.rs:558): g / (1 + exp(-g)) * u
                const float g = acc0[tk];
                const float den = 1.0f + expf_cr(-g);
                const float q = g / den;
                a.out[(p0 + c0 + tk) * rows + r] = q * acc1[tk];
              }
            }
          }
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// Decode kernel for one activation row per expert (single-token decode).
// Each lane always handles the same task slots t = lr + i*LPR of every row, so
// its slice of the Q8_K/Q8 activation row (64+16+4 bytes per Q4_K task, 32+4
// per Q8_0 block) is loaded once into registers and reused for every row: no
// LDS staging, no per-row activation traffic. Work-groups stride over a flat
// list of (expert, row-block) tasks, sized so every CU gets the same number.
// MODE M_GATE_UP: h[slot, r] = SwiGLU(gate_r . x, up_r . x) for each active expert.
// MODE M_DOWN_COMBINE: out[r] = sum over active experts in ascending id of
//   w_e * (down_e[r] . q8k(h[slot_e])) — the down projection and the combine
//   (transformer.rs:566-570) in one pass; valid when all slots belong to one token.
// MODE M_PLAIN: out[r] = W[r] . x for one activation row.
enum { M_DOWN_COMBINE = 4 };

template <int TYPE>
struct ActSlice;
template <>
struct ActSlice<T_Q4_K> {
  int4 x0, x1, x2, x3, bs;
  float d;
};
template <>
struct ActSlice<T_Q6_K> {
  int4 x0, x1, x2, x3, bs;
  float d;
};
template <>
struct ActSlice<T_Q8_0> {
  int4 x0, x1;
  float d;
};

template <int TYPE>
__device__ __forceinline__ void act_load(ActSlice<TYPE> &s, const int8_t *xq, const float *xd, const int32_t *xbs,
                                         int t) {
  if constexpr (is_kquant(TYPE)) {
    const int sb = t >> 2, k = t & 3;
    const int4 *v = (const int4 *)(xq + 256 * sb + 64 * k);
    s.x0 = v[0];
    s.x1 = v[1];
    s.x2 = v[2];
    s.x3 = v[3];
    s.bs = *(const int4 *)(xbs + 16 * sb + 4 * k);
    s.d = xd[sb];
  } else {
    const int4 *v = (const int4 *)(xq + 32 * t);
    s.x0 = v[0];
    s.x1 = v[1];
    s.d = xd[t];
  }
}

// One task's weight registers; TILED: a row of the expert tier (Q4_K and
// Q6_K tiled, Q8_0 GGUF bytes either way).
template <int TYPE, bool TILED>
struct WTask;
template <bool TL>
struct WTask<T_Q4_K, TL> {
  Q4kW w;
};
template <bool TL>
struct WTask<T_Q8_0, TL> {
  Q80W w;
};
template <>
struct WTask<T_Q6_K, false> {
  Q6kW w;
};
template <>
struct WTask<T_Q6_K, true> {
  Q6kT w;
};

// A GGUF row's task into the registers of a tier kernel (Q4_K: the same
// Q4kW as the tiled load, from the GGUF offsets; Q8_0 rows are GGUF either way).
template <int TYPE>
__device__ __forceinline__ auto wq_load_gguf(const uint8_t *row, int t, int64_t nblk) {
  if constexpr (TYPE == T_Q4_K) return q4k_load<false>(row, t, nblk);
  else return q80_load(row, t);
}

template <int TYPE, bool TILED>
__device__ __forceinline__ void w_load(WTask<TYPE, TILED> &w, const uint8_t *row, int t, int64_t nblk) {
  if constexpr (TYPE == T_Q4_K) w.w = q4k_load<TILED>(row, t, nblk);
  else if constexpr (TYPE == T_Q6_K && TILED) w.w = q6t_load(row, t, nblk);
  else if constexpr (TYPE == T_Q6_K) w.w = q6k_load(row, t);
  else w.w = q80_load(row, t);
}

// acc += (float) dot of one task against its activation slice. ds / dm
// (when non-null): the row's per-block integer accumulators, to which this
// task's integers are added (its block is t / tasks per block).
template <int TYPE, bool TILED>
__device__ __forceinline__ float task_dot(const WTask<TYPE, TILED> &wt, int t, const ActSlice<TYPE> &s, float acc,
                                          int32_t *ds = nullptr, int32_t *dm = nullptr) {
  if constexpr (TYPE == T_Q4_K) {
    const Q4kW &w = wt.w;
    const int k = t & 3;
    int sA, mA, sB, mB;
    q4k_scale_min_pair(w.hdr.y, w.hdr.z, w.hdr.w, k, sA, mA, sB, mB);
    const uint32_t m = 0x0f0f0f0fu;
    int lo = 0, hi = 0;
    lo = sdot4(w.qa.x & m, (uint32_t)s.x0.x, lo);
    lo = sdot4(w.qa.y & m, (uint32_t)s.x0.y, lo);
    lo = sdot4(w.qa.z & m, (uint32_t)s.x0.z, lo);
    lo = sdot4(w.qa.w & m, (uint32_t)s.x0.w, lo);
    lo = sdot4(w.qb.x & m, (uint32_t)s.x1.x, lo);
    lo = sdot4(w.qb.y & m, (uint32_t)s.x1.y, lo);
    lo = sdot4(w.qb.z & m, (uint32_t)s.x1.z, lo);
    lo = sdot4(w.qb.w & m, (uint32_t)s.x1.w, lo);
    hi = sdot4((w.qa.x >> 4) & m, (uint32_t)s.x2.x, hi);
    hi = sdot4((w.qa.y >> 4) & m, (uint32_t)s.x2.y, hi);
    hi = sdot4((w.qa.z >> 4) & m, (uint32_t)s.x2.z, hi);
    hi = sdot4((w.qa.w >> 4) & m, (uint32_t)s.x2.w, hi);
    hi = sdot4((w.qb.x >> 4) & m, (uint32_t)s.x3.x, hi);
    hi = sdot4((w.qb.y >> 4) & m, (uint32_t)s.x3.y, hi);
    hi = sdot4((w.qb.z >> 4) & m, (uint32_t)s.x3.z, hi);
    hi = sdot4((w.qb.w >> 4) & m, (uint32_t)s.x3.w, hi);
    const int sumi = sA * lo + sB * hi;
    const int mins = mA * (s.bs.x + s.bs.y) + mB * (s.bs.z + s.bs.w);
    if (ds) {
      atomicAdd(ds + (t >> 2), sumi);
      if (dm) atomicAdd(dm + (t >> 2), mins);
    }
    const float d = f16_bits_to_f32(w.hdr.x), dmin = f16_bits_to_f32(w.hdr.x >> 16);
    acc = fmaf(d * s.d, (float)sumi, acc);
    acc = fmaf(-(dmin * s.d), (float)mins, acc);
    return acc;
  } else if constexpr (TYPE == T_Q6_K) {
    int sumi, offs;
    if constexpr (TILED) q6t_ints(wt.w, s.x0, s.x1, s.x2, s.x3, s.bs, sumi, offs);
    else q6k_ints(wt.w, t & 3, s.x0, s.x1, s.x2, s.x3, s.bs, sumi, offs);
    if (ds) {
      atomicAdd(ds + (t >> 2), sumi);
      if (dm) atomicAdd(dm + (t >> 2), offs);
    }
    return fmaf(f16_bits_to_f32(wt.w.d) * s.d, (float)(sumi - 32 * offs), acc);
  } else {
    const Q80W &w = wt.w;
    const uint32_t v[9] = {w.a.x, w.a.y, w.a.z, w.a.w, w.b.x, w.b.y, w.b.z, w.b.w, w.c};
    uint32_t q[8];
    float dw;
    if (w.sh == 0) {
      dw = f16_bits_to_f32(v[0]);
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = __builtin_amdgcn_alignbyte(v[i + 1], v[i], 2);
    } else {
      dw = f16_bits_to_f32(v[0] >> 16);
#pragma unroll
      for (int i = 0; i < 8; ++i) q[i] = v[i + 1];
    }
    int p = 0;
    p = sdot4(q[0], (uint32_t)s.x0.x, p);
    p = sdot4(q[1], (uint32_t)s.x0.y, p);
    p = sdot4(q[2], (uint32_t)s.x0.z, p);
    p = sdot4(q[3], (uint32_t)s.x0.w, p);
    p = sdot4(q[4], (uint32_t)s.x1.x, p);
    p = sdot4(q[5], (uint32_t)s.x1.y, p);
    p = sdot4(q[6], (uint32_t)s.x1.z, p);
    p = sdot4(q[7], (uint32_t)s.x1.w, p);
    if (ds) atomicAdd(ds + t, p);
    return fmaf(dw * s.d, (float)p, acc);
  }
}

// One token's routing from its logits by wave 0 of a work-group (the
// selection of wave_route_one): slot_e[i] = the i-th smallest selected expert
// (the expert of slot i); work-group 0 also publishes the routing for the
// kernels that follow.
__device__ __forceinline__ void mv_select(const DecSelect &q, int lane, int32_t *slot_e, float *P, bool publish) {
  uint32_t sl;
  float wl;
  if (q.E <= 64) {
    float lv[1] = {lane < q.E ? q.logits[lane] : -INFINITY};
    wave_route_one<1>(lv, q.E, q.K, q.norm_topk, q.weights_scale, P, sl, wl);
  } else if (q.E <= 128) {
    float lv[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) lv[i] = lane + 64 * i < q.E ? q.logits[lane + 64 * i] : -INFINITY;
    wave_route_one<2>(lv, q.E, q.K, q.norm_topk, q.weights_scale, P, sl, wl);
  } else {
    float lv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) lv[i] = lane + 64 * i < q.E ? q.logits[lane + 64 * i] : -INFINITY;
    wave_route_one<4>(lv, q.E, q.K, q.norm_topk, q.weights_scale, P, sl, wl);
  }
  const uint32_t rk = selection_rank(sl, q.K);
  if (lane < q.K) slot_e[rk] = (int32_t)sl;
  if (publish)
    publish_selection(sl, wl, rk, q.K, q.E, lane, q.idx, q.wsel, q.perm, q.inv, q.active, q.n_active, q.offsets);
}

// DBG: the grouped modes also add their per-block integers into a.dbg (the
// capture of kmoe_moe_ffn_dbg); the product instantiation carries none of it.
template <int TYPE, int LPR, int TPLMAX, int RU, int MODE, bool DBG>
__global__ void __launch_bounds__(256) k_mv_reg(MvArgs a, int tpl) {
  constexpr int RPW = 64 / LPR;
  constexpr int RB = 4 * RPW * RU;  // rows per block-task
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row_in_wave = lane / LPR, lr = lane % LPR;
  const int64_t cols = a.cols, rows = a.rows;
  const int64_t nblk = cols / QT<TYPE>::EL;
  const int ntasks = (int)(QT<TYPE>::TPB * nblk);
  const int64_t row_bytes = nblk * QT<TYPE>::BYTES;
  const int64_t xs_stride = cols / 16;
  const int64_t bpe = (rows + RB - 1) / RB;
  int64_t total = bpe;
  __shared__ int32_t slot_e[16];
  __shared__ float selP[256];

  ActSlice<TYPE> act[TPLMAX];
  if constexpr (MODE == M_PLAIN_FX) {
    // The row's Q8_K blocks into LDS (block wave + 4i, four values per lane:
    // k_quant_q8k's arithmetic), then every lane's slices from there.
    __shared__ __attribute__((aligned(16))) int8_t fq[kRegFxBlocks * 256];
    __shared__ float fd[kRegFxBlocks];
    __shared__ __attribute__((aligned(16))) int32_t fbs[kRegFxBlocks * 16];
    float4 xv[kRegFxBlocks / 4];
#pragma unroll
    for (int i = 0; i < kRegFxBlocks / 4; ++i) {
      const int64_t bk = wave + 4 * i < nblk ? wave + 4 * i : nblk - 1;
      xv[i] = *(const float4 *)(a.xf + 256 * bk + 4 * lane);
    }
#pragma unroll
    for (int i = 0; i < kRegFxBlocks / 4; ++i) {
      const int bk = wave + 4 * i;
      if (bk < nblk) wave_quant_q8k_vals(xv[i], fq + 256 * bk, fd + bk, fbs + 16 * bk, lane);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TPLMAX; ++i) {
      const int t = lr + i * LPR;
      if (i < tpl && t < ntasks) act_load<TYPE>(act[i], fq, fd, fbs, t);
    }
  } else if constexpr (MODE == M_QKV_NORM) {
    // x (+ y), its RMSNorm (k_rmsnorm_regs' bits) and the Q8_K blocks into
    // LDS: thread t's float4 group t + 256i is element 4 * lane of block
    // wave + 4i, the layout of the wave quantizer
    __shared__ __attribute__((aligned(16))) int8_t fq[kRegFxBlocks * 256];
    __shared__ float fd[kRegFxBlocks];
    __shared__ __attribute__((aligned(16))) int32_t fbs[kRegFxBlocks * 16];
    __shared__ float red[4];
    __shared__ int xlast;
    float4 hv[kRegFxBlocks / 4];
    wg_residual_rmsnorm<kRegFxBlocks / 4>(const_cast<float *>(a.nx), a.ny, a.nw, cols, a.neps, nullptr, hv, red, &xlast,
                                          blockIdx.x == 0 ? a.nxo : nullptr);
#pragma unroll
    for (int i = 0; i < kRegFxBlocks / 4; ++i) {
      const int bk = wave + 4 * i;
      if (bk < nblk) {
        if (blockIdx.x == 0) *(float4 *)(a.nh + 256 * bk + 4 * lane) = hv[i];
        wave_quant_q8k_vals(hv[i], fq + 256 * bk, fd + bk, fbs + 16 * bk, lane);
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TPLMAX; ++i) {
      const int t = lr + i * LPR;
      if (i < tpl && t < ntasks) act_load<TYPE>(act[i], fq, fd, fbs, t);
    }
  } else if constexpr (MODE != M_DOWN_COMBINE) {  // one activation row: token 0 (or the plain row)
#pragma unroll
    for (int i = 0; i < TPLMAX; ++i) {
      const int t = lr + i * LPR;
      if (i < tpl && t < ntasks) act_load<TYPE>(act[i], a.xq, a.xd, a.xbs, t);
    }
  }
  int64_t routed_total = 0;
  if constexpr (MODE == M_GATE_UP) {  // after the activation loads are issued, so the two overlap
    if (a.sel_on) {
      if (wave == 0) mv_select(a.sel, lane, slot_e, selP, blockIdx.x == 0);
      __syncthreads();
      total = (int64_t)a.sel.K * bpe;
    } else {
      total = (int64_t)(*a.rt.n_active) * bpe;
    }
    routed_total = total;
    if (a.sgu_w) total += (a.sgu_rows + RB - 1) / RB;  // the shared expert's row blocks after the experts'
  }

  for (int64_t b = blockIdx.x; b < total; b += gridDim.x) {
    int64_t rblk = b;
    const uint8_t *W0 = a.w0, *W1 = nullptr;
    int64_t p0 = 0;
    bool shared_item = false;  // M_GATE_UP: a block of the shared expert's GGUF rows
    int64_t rows_i = rows;
    if constexpr (MODE == M_GATE_UP) {
      if (b >= routed_total) {
        shared_item = true;
        rblk = b - routed_total;
        rows_i = a.sgu_rows;
        W0 = a.sgu_w;
        W1 = a.sgu_w + a.sgu_rows * row_bytes;
      } else {
        const int i = (int)(b / bpe);
        rblk = b - (int64_t)i * bpe;
        const int e = a.sel_on ? slot_e[i] : a.rt.active[i];
        p0 = a.sel_on ? i : a.rt.offsets[e];
        const uint8_t *eb = a.tier.base + (int64_t)e * a.tier.stride;
        W0 = eb + a.tier.off[0];
        W1 = eb + a.tier.off[1];
      }
    }
    const int64_t r0 = rblk * RB + (int64_t)(wave * RU) * RPW + row_in_wave;

    if constexpr (MODE == M_DOWN_COMBINE) {
      float o[RU];
#pragma unroll
      for (int u = 0; u < RU; ++u) o[u] = 0.0f;
      const int na = *a.rt.n_active;
      for (int ia = 0; ia < na; ++ia) {  // ascending expert id
        const int e = a.rt.active[ia];
        const int64_t p = a.rt.offsets[e];
        const float wgt = a.rt.wsel[a.rt.perm[p]];
        const uint8_t *W = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[2];
#pragma unroll
        for (int i = 0; i < TPLMAX; ++i) {
          const int t = lr + i * LPR;
          if (i < tpl && t < ntasks)
            act_load<TYPE>(act[i], a.xq + p * cols, a.xd + p * nblk, a.xbs + p * xs_stride, t);
        }
        float acc[RU];
#pragma unroll
        for (int u = 0; u < RU; ++u) acc[u] = 0.0f;
#pragma unroll
        for (int i = 0; i < TPLMAX; ++i) {
          const int t = lr + i * LPR;
          if (i < tpl && t < ntasks) {
            WTask<TYPE, true> w[RU];
#pragma unroll
            for (int u = 0; u < RU; ++u) {
              const int64_t r = r0 + (int64_t)u * RPW;
              if (r < rows) w_load<TYPE, true>(w[u], W + r * row_bytes, t, nblk);
            }
#pragma unroll
            for (int u = 0; u < RU; ++u) {
              const int64_t r = r0 + (int64_t)u * RPW;
              if (r < rows) {
                if constexpr (DBG) {
                  const int64_t o = (p * rows + r) * nblk;
                  acc[u] = task_dot<TYPE>(w[u], t, act[i], acc[u], a.dbg.s[0] ? a.dbg.s[0] + o : nullptr,
                                          a.dbg.m[0] ? a.dbg.m[0] + o : nullptr);
                } else {
                  acc[u] = task_dot<TYPE>(w[u], t, act[i], acc[u]);
                }
              }
            }
          }
        }
#pragma unroll
        for (int u = 0; u < RU; ++u) {
          const float y = group_sum<LPR>(acc[u]);
          const float t = wgt * y;
          o[u] = o[u] + t;
        }
      }
      if (lr == 0) {
#pragma unroll
        for (int u = 0; u < RU; ++u) {
          const int64_t r = r0 + (int64_t)u * RPW;
          if (r < rows) a.out[r] = o[u];
        }
      }
    } else {
      float acc0[RU], acc1[RU];
#pragma unroll
      for (int u = 0; u < RU; ++u) acc0[u] = acc1[u] = 0.0f;
#pragma unroll
      for (int i = 0; i < TPLMAX; ++i) {
        const int t = lr + i * LPR;
        if (i < tpl && t < ntasks) {
          constexpr bool TLW = MODE == M_GATE_UP;  // expert tier rows are tiled, plain rows are GGUF
          WTask<TYPE, TLW> w0[RU], w1[RU];
#pragma unroll
          for (int u = 0; u < RU; ++u) {
            const int64_t r = r0 + (int64_t)u * RPW;
            if (r < rows_i) {
              constexpr bool TL = MODE == M_GATE_UP;  // expert tier rows are tiled, plain rows are GGUF
              int64_t rw = r;
              if constexpr (MODE == M_QKV || MODE == M_QKV_NORM) rw = qkv_row(a.rope, r);
              if constexpr (MODE == M_GATE_UP && (TYPE == T_Q4_K || TYPE == T_Q8_0)) {
                if (shared_item) {  // GGUF rows into the same registers (Q4_K and Q8_0 tasks alike)
                  w0[u].w = wq_load_gguf<TYPE>(W0 + r * row_bytes, t, nblk);
                  w1[u].w = wq_load_gguf<TYPE>(W1 + r * row_bytes, t, nblk);
                  continue;
                }
              }
              w_load<TYPE, TL>(w0[u], W0 + rw * row_bytes, t, nblk);
              if constexpr (MODE == M_GATE_UP) w_load<TYPE, TL>(w1[u], W1 + r * row_bytes, t, nblk);
            }
          }
#pragma unroll
          for (int u = 0; u < RU; ++u) {
            const int64_t r = r0 + (int64_t)u * RPW;
            if (r < rows_i) {
              if constexpr (MODE == M_GATE_UP && DBG) {  // (no shared items with DBG)
                const int64_t o = (p0 * rows + r) * nblk;
                const BlockDbg &g = a.dbg;
                acc0[u] = task_dot<TYPE>(w0[u], t, act[i], acc0[u], g.s[0] ? g.s[0] + o : nullptr,
                                         g.m[0] ? g.m[0] + o : nullptr);
                acc1[u] = task_dot<TYPE>(w1[u], t, act[i], acc1[u], g.s[1] ? g.s[1] + o : nullptr,
                                         g.m[1] ? g.m[1] + o : nullptr);
              } else {
                acc0[u] = task_dot<TYPE>(w0[u], t, act[i], acc0[u]);
                if constexpr (MODE == M_GATE_UP) acc1[u] = task_dot<TYPE>(w1[u], t, act[i], acc1[u]);
              }
            }
          }
        }
      }
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        acc0[u] = group_sum<LPR>(acc0[u]);
        if constexpr (MODE == M_GATE_UP) acc1[u] = group_sum<LPR>(acc1[u]);
      }
      float pair[RU];  // M_QKV: row r^1's sum, held by the lanes LPR away (RPW >= 2)
      if constexpr (MODE == M_QKV || MODE == M_QKV_NORM) {
        static_assert(RPW >= 2, "row pairs in one wave");
#pragma unroll
        for (int u = 0; u < RU; ++u) pair[u] = __shfl_xor(acc0[u], LPR);
      }
      if (lr == 0) {
#pragma unroll
        for (int u = 0; u < RU; ++u) {
          const int64_t r = r0 + (int64_t)u * RPW;
          if (r >= rows_i) continue;
          if constexpr (MODE == M_QKV || MODE == M_QKV_NORM) {
            const int64_t rw = qkv_row(a.rope, r);
            a.out[rw] = acc0[u];
            qkv_rope_store(a.rope, rw, acc0[u], pair[u]);
          } else if constexpr (MODE == M_GATE_UP) {  // SwiGLU (transformer.rs:558)
            const float g = acc0[u];
            const float den = 1.0f + expf_cr(-g);
            const float q = g / den;
            if (shared_item) a.sgu_h[r] = q * acc1[u];
            else a.out[p0 * rows + r] = q * acc1[u];
          } else if (a.add) {  // the shared expert's gated add (k_shared_add's arithmetic)
            float scale = 1.0f;
            if (a.add_logit) {
              const float den = 1.0f + expf_cr(-*a.add_logit);
              scale = 1.0f / den;
            }
            const float pv = scale * acc0[u];
            a.out[r] = a.out[r] + pv;
          } else {
            a.out[r] = acc0[u];
          }
        }
      }
    }
  }
}

constexpr int kSplitRbMax = 64;

template <int TYPE, int RU, int TPL, bool DBG>
__global__ void __launch_bounds__(256) k_down_splitk(MvArgs a, int rb_rows) {
  __shared__ float part[4][kSplitRbMax];
  __shared__ float outv[kSplitRbMax];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t cols = a.cols, rows = a.rows;
  const int64_t nblk = cols / QT<TYPE>::EL;
  const int ntasks = (int)(QT<TYPE>::TPB * nblk);
  const int64_t row_bytes = nblk * QT<TYPE>::BYTES;
  const int64_t xs_stride = cols / 16;
  const int tpw = (ntasks + 3) / 4;  // tasks per wave
  const int64_t r0 = (int64_t)blockIdx.x * rb_rows;
  const int nr = (int)(rows - r0 < rb_rows ? rows - r0 : rb_rows);
  if (nr <= 0) return;
  if (threadIdx.x < kSplitRbMax) outv[threadIdx.x] = 0.0f;
  int tk[TPL];
  bool tv[TPL];
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const int lt = lane + 64 * i;
    tk[i] = wave * tpw + lt;
    tv[i] = lt < tpw && tk[i] < ntasks;
  }
  // one token: its top-k experts are distinct, so k slots are active (no
  // dependent read of the count before the first weight loads)
  const int na = a.s_rows == 1 ? a.rt.topk : *a.rt.n_active;
  const int nb = (nr + RU - 1) / RU;  // row batches per expert
  const int items = na * nb;          // (expert, batch) in ascending expert id
  if (items == 0) {
    if (threadIdx.x < nr) a.out[r0 + threadIdx.x] = 0.0f;
    return;
  }
  struct Item {
    const uint8_t *W;
    int64_t p;
    int rr;
  };
  auto decode = [&](int it) {
    Item im;
    const int ia = it / nb;
    const int e = a.rt.active[ia];
    // one token: the ia-th active expert's single slot is at position ia
    im.p = a.s_rows == 1 ? ia : a.rt.offsets[e];
    im.W = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[2];
    im.rr = (it - ia * nb) * RU;
    return im;
  };
  WTask<TYPE, true> cur[RU][TPL], nxt[RU][TPL];
  ActSlice<TYPE> act[TPL], act_n[TPL];
  // Unconditional loads with clamped indices: a divergent branch around the
  // loads would make the compiler wait for all of them at the join.
  auto load_w = [&](const Item &im, WTask<TYPE, true> (&w)[RU][TPL]) {
#pragma unroll
    for (int u = 0; u < RU; ++u)
#pragma unroll
      for (int i = 0; i < TPL; ++i)
        w_load<TYPE, true>(w[u][i], im.W + (r0 + min(im.rr + u, nr - 1)) * row_bytes, min(tk[i], ntasks - 1), nblk);
  };
  auto load_act = [&](const Item &im, ActSlice<TYPE> (&s)[TPL]) {
#pragma unroll
    for (int i = 0; i < TPL; ++i)
      act_load<TYPE>(s[i], a.xq + im.p * cols, a.xd + im.p * nblk, a.xbs + im.p * xs_stride, min(tk[i], ntasks - 1));
  };
  // One (expert, row-batch) item; finishes the expert after its last batch.
  auto compute = [&](int it, const Item &ic, WTask<TYPE, true> (&w)[RU][TPL], ActSlice<TYPE> (&ac)[TPL]) {
    const bool last = (it + 1) % nb == 0;  // this expert's last row batch
    float wgt = 0.0f;
    if (last) wgt = a.rt.wsel[a.rt.perm[ic.p]];  // issued early, used after the dots
    float acc[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      acc[u] = 0.0f;
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        int32_t *ds = nullptr, *dm = nullptr;
        if constexpr (DBG) {
          if (tv[i] && ic.rr + u < nr) {
            const int64_t o = (ic.p * rows + r0 + ic.rr + u) * nblk;
            ds = a.dbg.s[0] + o;
            dm = a.dbg.m[0] ? a.dbg.m[0] + o : nullptr;
          }
        }
        const float v = task_dot<TYPE>(w[u][i], min(tk[i], ntasks - 1), ac[i], acc[u], ds, dm);
        acc[u] = tv[i] ? v : acc[u];
      }
      acc[u] = group_sum<64>(acc[u]);
    }
    if (lane == 0) {
#pragma unroll
      for (int u = 0; u < RU; ++u)
        if (ic.rr + u < nr) part[wave][ic.rr + u] = acc[u];
    }
    if (last) {  // y = sum of the wave partials, combine. LDS-only barriers: the
                 // next item's weight loads stay in flight.
      lds_barrier();
      if (threadIdx.x < nr) {
        const int t = threadIdx.x;
        const float y = ((part[0][t] + part[1][t]) + part[2][t]) + part[3][t];
        const float c = wgt * y;
        outv[t] = outv[t] + c;
      }
      lds_barrier();
    }
  };
  // Ping-pong register sets (weights and activation slices): item it+1's
  // loads are in flight while item it is computed.
  int it = 0;
  Item ia_ = decode(0);
  load_act(ia_, act);
  load_w(ia_, cur);
  for (;;) {
    Item ib;
    const bool hb = it + 1 < items;
    if (hb) {
      ib = decode(it + 1);
      if ((it + 1) % nb == 0) load_act(ib, act_n);
      else for (int i = 0; i < TPL; ++i) act_n[i] = act[i];
      load_w(ib, nxt);
    }
    compute(it, ia_, cur, act);
    if (!hb) break;
    ++it;
    const bool ha = it + 1 < items;
    if (ha) {
      ia_ = decode(it + 1);
      if ((it + 1) % nb == 0) load_act(ia_, act);
      else for (int i = 0; i < TPL; ++i) act[i] = act_n[i];
      load_w(ia_, cur);
    }
    compute(it, ib, nxt, act_n);
    if (!ha) break;
    ++it;
  }
  if (threadIdx.x < nr) a.out[r0 + threadIdx.x] = outv[threadIdx.x];
}

// Single-token down + combine with a ring of NS register sets: the weight loads
// of items i+1 .. i+NS-1 are in flight while item i is computed, and item
// i+NS's loads go out as soon as item i has been computed. Items are (slot,
// RU-row batch) pairs in ascending expert id, at most NIT of them (the host
// checks topk * ceil(rb_rows / RU) <= NIT and topk <= 2); the loop over them
// is unrolled, so every load is unconditional (clamped to the last item) and
// the compiler's wait counts stay exact. The routing weights come from two
// direct loads issued before the weight loads (wsel[j] and the slot inv[j] of
// selection j), so no wait for them sits between weight loads. Same
// arithmetic and combine order as k_down_splitk: y per row is the sum of the
// four wave partials ((w0 + w1) + w2) + w3, out = (0 + wgt_0*y_0) + wgt_1*y_1.
template <int TYPE, int RU, int NIT, int NS, bool DBG>
__global__ void __launch_bounds__(256) k_down_ring(MvArgs a, int rb_rows) {
  __shared__ float part[4][kSplitRbMax];
  __shared__ float outv[kSplitRbMax];
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t cols = a.cols, rows = a.rows;
  const int64_t nblk = cols / QT<TYPE>::EL;
  const int ntasks = (int)(QT<TYPE>::TPB * nblk);
  const int64_t row_bytes = nblk * QT<TYPE>::BYTES;
  const int64_t xs_stride = cols / 16;
  const int tpw = (ntasks + 3) / 4;  // tasks per wave (<= 64)
  const int64_t r0 = (int64_t)blockIdx.x * rb_rows;
  const int nr = (int)(rows - r0 < rb_rows ? rows - r0 : rb_rows);
  if (nr <= 0) return;
  if (threadIdx.x < kSplitRbMax) outv[threadIdx.x] = 0.0f;
  const int tk = wave * tpw + lane;
  const bool tv = lane < tpw && tk < ntasks;
  const int tc = min(tk, ntasks - 1);
  const int na = a.rt.topk;           // one token: topk distinct experts, slot p = p-th smallest id
  const int nb = (nr + RU - 1) / RU;  // row batches per expert
  const int items = na * nb;
  // selection j's expert slot and weight (lanes j < topk)
  const int jl = lane < na ? lane : 0;
  const int32_t e_l = a.rt.active[jl];
  const uint32_t inv_l = a.rt.inv[jl];
  const float w_l = a.rt.wsel[jl];
  const int e0 = __builtin_amdgcn_readfirstlane(e_l);
  const int e1 = __shfl(e_l, na > 1 ? 1 : 0);
  const uint8_t *W0 = a.tier.base + (int64_t)e0 * a.tier.stride + a.tier.off[2];
  const uint8_t *W1 = a.tier.base + (int64_t)__builtin_amdgcn_readfirstlane(e1) * a.tier.stride + a.tier.off[2];
  ActSlice<TYPE> act0, act1;
  act_load<TYPE>(act0, a.xq, a.xd, a.xbs, tc);
  const int p1 = na > 1 ? 1 : 0;
  act_load<TYPE>(act1, a.xq + p1 * cols, a.xd + p1 * nblk, a.xbs + p1 * xs_stride, tc);
  WTask<TYPE, true> w[NS][RU];
  auto issue = [&](int it, WTask<TYPE, true> (&ws)[RU]) {
    it = min(it, items - 1);
    const int ia = it / nb;
    const uint8_t *W = ia == 0 ? W0 : W1;
    const int rr = (it - ia * nb) * RU;
#pragma unroll
    for (int u = 0; u < RU; ++u) w_load<TYPE, true>(ws[u], W + (r0 + min(rr + u, nr - 1)) * row_bytes, tc, nblk);
  };
#pragma unroll
  for (int i = 0; i < NS; ++i) issue(i, w[i]);
  // the weights of slots 0 and 1: slot p's selection j has inv[j] == p
  const uint64_t m0 = __ballot(lane < na && inv_l == 0u), m1 = __ballot(lane < na && inv_l == 1u);
  const float wg0 = __shfl(w_l, m0 ? __builtin_ctzll(m0) : 0);
  const float wg1 = __shfl(w_l, m1 ? __builtin_ctzll(m1) : 0);
  // The dots run for every unrolled item, past `items` too (on clamped
  // duplicates, results dropped): a branch around them would let the compiler
  // sink the item's loads into it, behind the later items' loads.
#pragma unroll
  for (int i = 0; i < NIT; ++i) {
    const int ic = min(i, items - 1);
    const int ia = ic / nb;
    const int rr = (ic - ia * nb) * RU;
    const ActSlice<TYPE> &ac = ia == 0 ? act0 : act1;
    float acc[RU];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      int32_t *ds = nullptr, *dm = nullptr;
      if constexpr (DBG) {
        if (tv && rr + u < nr && i < items) {
          const int64_t o = ((int64_t)ia * rows + r0 + rr + u) * nblk;
          ds = a.dbg.s[0] + o;
          dm = a.dbg.m[0] ? a.dbg.m[0] + o : nullptr;
        }
      }
      const float v = task_dot<TYPE>(w[i % NS][u], tc, ac, 0.0f, ds, dm);
      acc[u] = group_sum<64>(tv ? v : 0.0f);
    }
    if (i < items) {
      if (lane == 0) {
#pragma unroll
        for (int u = 0; u < RU; ++u)
          if (rr + u < nr) part[wave][rr + u] = acc[u];
      }
      if ((i + 1) % nb == 0) {  // this expert's last row batch: y and the combine
        lds_barrier();
        if (threadIdx.x < nr) {
          const int t = threadIdx.x;
          const float y = ((part[0][t] + part[1][t]) + part[2][t]) + part[3][t];
          const float c = (ia == 0 ? wg0 : wg1) * y;
          outv[t] = outv[t] + c;
        }
        lds_barrier();
      }
    }
    if (i + NS < NIT) issue(i + NS, w[i % NS]);
  }
  if (threadIdx.x < nr) a.out[r0 + threadIdx.x] = outv[threadIdx.x];
}

// Single-token down + combine over narrow rows (one task slot per lane, LPR
// lanes per row): the arithmetic and order of k_mv_reg's M_DOWN_COMBINE mode
// (out[r] = sum over the token's experts in ascending id of w * (down_e[r] .
// q8(h_slot))), with the experts' loads software-pipelined: a ring of NS
// register sets (the slot's activation slice and the row's task) keeps the
// next NS-1 experts' loads in flight while one is reduced. The loop over the
// KMAX >= topk experts is unrolled and every load unconditional (indices
// clamped to the last expert), so the compiler's waits stay exact; the expert
// ids, slots and weights are read once per lane up front (lane j: selection
// j), so no dependent load sits between the weight loads. WPB waves per
// work-group, each RPW = 64 / LPR rows.
template <int TYPE, int LPR, int KMAX, int NS, int WPB, bool DBG, int SHT = 0>
__global__ void __launch_bounds__(64 * WPB) k_mv_down_exp(MvArgs a) {
  constexpr int RPW = 64 / LPR;
  constexpr int RB = WPB * RPW;  // rows per block-task
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row_in_wave = lane / LPR, lr = lane % LPR;
  const int64_t cols = a.cols, rows = a.rows;
  const int64_t nblk = cols / QT<TYPE>::EL;
  const int ntasks = (int)(QT<TYPE>::TPB * nblk);
  const int64_t row_bytes = nblk * QT<TYPE>::BYTES;
  const int64_t xs_stride = cols / 16;
  const bool tv = lr < ntasks;
  const int t = tv ? lr : ntasks - 1;
  // The shared expert (SHT): its row's task of this lane, its int8 slice
  // (loaded once) and its gate (k_shared_add's arithmetic: sigmoid of the
  // logit, 1 without a gate).
  constexpr int ST = SHT ? SHT : TYPE;
  const int64_t sh_nblk = SHT ? a.sh_cols / QT<ST>::EL : 0;
  const int sh_ntasks = (int)(QT<ST>::TPB * sh_nblk);
  const int64_t sh_row_bytes = sh_nblk * QT<ST>::BYTES;
  const bool sh_tv = lr < sh_ntasks;
  const int sh_t = sh_tv ? lr : (SHT ? sh_ntasks - 1 : 0);
  ActSlice<ST> sh_act;
  float sh_scale = 1.0f;
  if constexpr (SHT != 0) {
    act_load<ST>(sh_act, a.sh_xq, a.sh_xd, a.sh_xbs, sh_t);
    if (a.sh_logit) {
      const float den = 1.0f + expf_cr(-*a.sh_logit);
      sh_scale = 1.0f / den;
    }
  }
  const int K = a.rt.topk;
  const int jl = lane < K ? lane : 0;
  const int32_t e_l = a.rt.active[jl];  // expert of slot jl
  const uint32_t inv_l = a.rt.inv[jl];  // slot of selection jl
  const float w_l = a.rt.wsel[jl];      // weight of selection jl
  const int64_t bpe = (rows + RB - 1) / RB;
  for (int64_t blk = blockIdx.x; blk < bpe; blk += gridDim.x) {
    const int64_t r = blk * RB + (int64_t)wave * RPW + row_in_wave;
    const int64_t rc = r < rows ? r : rows - 1;
    ActSlice<TYPE> act[NS];
    WTask<TYPE, true> w[NS];
    auto issue = [&](int ia, int sl) {
      ia = ia < K ? ia : K - 1;
      const int e = __builtin_amdgcn_readlane(e_l, ia);
      const uint8_t *W = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[2];
      act_load<TYPE>(act[sl], a.xq + (int64_t)ia * cols, a.xd + (int64_t)ia * nblk, a.xbs + (int64_t)ia * xs_stride,
                     t);
      w_load<TYPE, true>(w[sl], W + rc * row_bytes, t, nblk);
    };
#pragma unroll
    for (int sl = 0; sl < NS; ++sl) issue(sl, sl);
    WTask<ST, false> sh_w;  // the shared row, in flight with the experts' first loads
    if constexpr (SHT != 0) w_load<ST, false>(sh_w, a.sh_w + rc * sh_row_bytes, sh_t, sh_nblk);
    float o = 0.0f;
#pragma unroll
    for (int ia = 0; ia < KMAX; ++ia) {  // ascending expert id: slot ia
      const int sl = ia % NS;
      const uint64_t m = __ballot(lane < K && inv_l == (uint32_t)ia);
      const float wgt = __builtin_bit_cast(
          float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w_l), m ? (int)__builtin_ctzll(m) : 0));
      int32_t *ds = nullptr, *dm = nullptr;
      if constexpr (DBG) {
        if (tv && r < rows && ia < K) {
          const int64_t oo = ((int64_t)ia * rows + r) * nblk;
          ds = a.dbg.s[0] + oo;
          dm = a.dbg.m[0] ? a.dbg.m[0] + oo : nullptr;
        }
      }
      const float v = task_dot<TYPE>(w[sl], t, act[sl], 0.0f, ds, dm);
      const float y = group_sum<LPR>(tv ? v : 0.0f);
      const float c = wgt * y;
      const float on = o + c;
      o = ia < K ? on : o;
      if (ia + NS < KMAX) issue(ia + NS, sl);
    }
    if constexpr (SHT != 0) {  // out[r] = combine + scale * shared (transformer.rs:572-587)
      const float v = task_dot<ST, false>(sh_w, sh_t, sh_act, 0.0f);
      const float y = group_sum<LPR>(sh_tv ? v : 0.0f);
      const float pv = sh_scale * y;
      o = o + pv;
    }
    if (lr == 0 && r < rows) a.out[r] = o;
  }
}

// Launch shapes (the measured best of the sweeps kept as measurements):
// register matvec work-groups capped at 4 per CU; split-K single-token down
// at 2 work-groups per CU with 4-row items; the single-token Q4_K / Q6_K down
// ring with 2 register sets.
constexpr int kGridMult = 4;
constexpr int kDownWgPerCu = 2;
constexpr int kDownRu = 4;
constexpr int kDownRingSets = 2;

int g_cu_count = 0;
int cu_count() {
  if (g_cu_count == 0) {
    int dev = 0, n = 0;
    if (hipGetDevice(&dev) == hipSuccess &&
        hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
      g_cu_count = n;
    else
      g_cu_count = 256;
  }
  return g_cu_count;
}

// Geometry of the register kernel for a row of `ntasks` tasks: lanes per row
// and task slots per lane. Returns false when the activation slice would not
// fit in registers.
bool reg_geometry(int type, int ntasks, int &lpr, int &tpl) {
  if (ntasks >= 64) {
    lpr = 64;
  } else {
    lpr = 16;
    while (lpr < ntasks) lpr *= 2;
  }
  tpl = (ntasks + lpr - 1) / lpr;
  return is_kquant(type) ? tpl <= 4 : tpl <= 8;
}

template <int TYPE, int LPR, int TPLMAX, int RU, int MODE>
hipError_t launch_reg(hipStream_t st, const MvArgs &a, int tpl, int64_t max_tasks) {
  constexpr int RB = 4 * (64 / LPR) * RU;
  (void)RB;
  const int64_t cap = (int64_t)cu_count() * kGridMult;
  int64_t grid = max_tasks;
  if (grid > cap) {
    const int64_t per = (max_tasks + cap - 1) / cap;  // equal task counts per work-group
    grid = (max_tasks + per - 1) / per;
  }
  if (grid < 1) grid = 1;
  if constexpr (MODE == M_GATE_UP || MODE == M_DOWN_COMBINE) {
    if (a.dbg.s[0] || a.dbg.s[1]) {
      KMOE_LAUNCH((k_mv_reg<TYPE, LPR, TPLMAX, RU, MODE, true>), dim3((unsigned)grid), dim3(256), 0, st, a, tpl);
      return hipGetLastError();
    }
  }
  KMOE_LAUNCH((k_mv_reg<TYPE, LPR, TPLMAX, RU, MODE, false>), dim3((unsigned)grid), dim3(256), 0, st, a, tpl);
  return hipGetLastError();
}

template <int TYPE, int MODE, int RU>
hipError_t dispatch_reg(hipStream_t st, const MvArgs &a, int n_groups) {
  const int64_t nblk = a.cols / QT<TYPE>::EL;
  const int ntasks = (int)(QT<TYPE>::TPB * nblk);
  int lpr, tpl;
  if (!reg_geometry(TYPE, ntasks, lpr, tpl)) return hipErrorNotSupported;
  const int64_t rb = 4 * (64 / lpr) * RU;
  const int64_t max_tasks = (a.rows + rb - 1) / rb * n_groups;
  constexpr int TM = is_kquant(TYPE) ? 4 : 8;
  switch (lpr) {
    case 64:
      if (tpl == 1) return launch_reg<TYPE, 64, 1, RU, MODE>(st, a, tpl, max_tasks);
      return launch_reg<TYPE, 64, TM, 1, MODE>(st, a, tpl, (a.rows + 3) / 4 * n_groups);
    case 32:
      return launch_reg<TYPE, 32, 1, RU, MODE>(st, a, tpl, max_tasks);
    case 16:
      return launch_reg<TYPE, 16, 1, RU, MODE>(st, a, tpl, max_tasks);
    default:
      return hipErrorNotSupported;
  }
}

template <int TYPE, int LPR, int NT, int MODE>
hipError_t launch_one(hipStream_t st, const MvArgs &a, dim3 grid) {
  const ActLayout<TYPE> L(a.cols);
  const size_t shmem = (size_t)NT * L.total;
  if constexpr (MODE == M_GATE_UP || MODE == M_DOWN) {
    if (a.dbg.s[0] || a.dbg.s[1]) {
      KMOE_LAUNCH((k_matvec_int<TYPE, LPR, NT, MODE, true>), grid, dim3(256), shmem, st, a);
      return hipGetLastError();
    }
  }
  KMOE_LAUNCH((k_matvec_int<TYPE, LPR, NT, MODE, false>), grid, dim3(256), shmem, st, a);
  return hipGetLastError();
}

// Lanes per row: the widest of 64/32/16/4 that keeps >= 85% of lanes busy.
int pick_lpr(int ntasks) {
  const int opts[4] = {64, 32, 16, 4};
  int best = 4;
  double best_eff = -1.0;
  for (int o : opts) {
    const int iters = (ntasks + o - 1) / o;
    const double eff = (double)ntasks / (double)(iters * o);
    if (eff >= 0.85) return o;
    if (eff > best_eff) {
      best_eff = eff;
      best = o;
    }
  }
  return best;
}

template <int TYPE, int MODE>
hipError_t dispatch_lpr_nt(hipStream_t st, const MvArgs &a, dim3 grid, int nt_max) {
  const int64_t nblk = a.cols / QT<TYPE>::EL;
  const int ntasks = (int)(QT<TYPE>::TPB * nblk);
  const int lpr = pick_lpr(ntasks);
#define KMOE_LPR_CASE(LPRV)                                                                          \
  case LPRV:                                                                                         \
    if constexpr (MODE == M_SUMS) return launch_one<TYPE, LPRV, 1, MODE>(st, a, grid);               \
    else if (nt_max == 1) return launch_one<TYPE, LPRV, 1, MODE>(st, a, grid);                       \
    else if (nt_max == 16) return launch_one<TYPE, LPRV, 16, MODE>(st, a, grid);                     \
    else if (nt_max == 8) return launch_one<TYPE, LPRV, 8, MODE>(st, a, grid);                       \
    else return launch_one<TYPE, LPRV, 3, MODE>(st, a, grid);
  switch (lpr) {
    KMOE_LPR_CASE(64)
    KMOE_LPR_CASE(32)
    KMOE_LPR_CASE(16)
    KMOE_LPR_CASE(4)
    default:
      return hipErrorInvalidValue;
  }
#undef KMOE_LPR_CASE
}

constexpr int kRowsPerBlock = 64;

// Plain-mode grid of the LDS-staged kernel: row blocks of 64 along x, and the
// activation rows split into chunks (a multiple of nt each) along y so that
// a launch has about 512 work-groups; each chunk re-reads the weights.
dim3 plain_grid(MvArgs &a, int64_t rows, int64_t s_rows, int nt) {
  const int64_t gx = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  int64_t chunks = (s_rows + nt - 1) / nt;
  const int64_t want = (512 + gx - 1) / gx;
  if (chunks > want) chunks = want;
  if (chunks < 1) chunks = 1;
  int64_t per = (s_rows + chunks - 1) / chunks;
  per = (per + nt - 1) / nt * nt;
  chunks = (s_rows + per - 1) / per;
  a.chunk = (int32_t)per;
  return dim3((unsigned)gx, (unsigned)chunks);
}

// Activation rows staged per pass of the LDS-staged kernel: every weight row
// is read once per pass, so batches take passes of 16 or 8 rows where the
// staging fits 64 KB of LDS (3 otherwise; 1 for a single row).
int pick_nt(int type, int64_t cols, int64_t rows_hint) {
  if (rows_hint <= 1) return 1;
  const int64_t per = is_kquant(type) ? ActLayout<T_Q4_K>(cols).total : ActLayout<T_Q8_0>(cols).total;
  if (rows_hint >= 24 && 16 * per <= 65536) return 16;
  if (rows_hint >= 6 && 8 * per <= 65536) return 8;
  return 3;
}

bool act_fits(int type, int64_t cols) {
  const int64_t per = is_kquant(type) ? ActLayout<T_Q4_K>(cols).total : ActLayout<T_Q8_0>(cols).total;
  return 3 * per <= 65536;
}

}  // namespace

hipError_t launch_decode_plain(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                               const int8_t *xq, const float *xd, const int32_t *xbs, float *out, const AddEpi *epi) {
  MvArgs a{};
  if (epi) {
    a.add = 1;
    a.add_logit = epi->logit;
  }
  a.w0 = w;
  a.rows = rows;
  a.cols = cols;
  a.xq = xq;
  a.xd = xd;
  a.xbs = xbs;
  a.s_rows = 1;
  a.out = out;
  if (type == T_Q4_K) {
    const hipError_t e = launch_dec_rows(st, w, rows, cols, xq, xd, xbs, out, epi);
    if (e != hipErrorNotSupported) return e;
    return dispatch_reg<T_Q4_K, M_PLAIN, 1>(st, a, 1);
  }
  if (type == T_Q6_K) return dispatch_reg<T_Q6_K, M_PLAIN, 1>(st, a, 1);
  if (type == T_Q8_0) return dispatch_reg<T_Q8_0, M_PLAIN, 1>(st, a, 1);
  return hipErrorInvalidValue;
}

hipError_t launch_decode_plain_fx(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                                  const float *xf, float *out) {
  if (!is_kquant(type) || cols % 256 != 0 || cols / 256 > kRegFxBlocks || ((uintptr_t)xf & 15u))
    return hipErrorNotSupported;
  MvArgs a{};
  a.w0 = w;
  a.rows = rows;
  a.cols = cols;
  a.xf = xf;
  a.s_rows = 1;
  a.out = out;
  if (type == T_Q4_K) return dispatch_reg<T_Q4_K, M_PLAIN_FX, 1>(st, a, 1);
  if (type == T_Q6_K) return dispatch_reg<T_Q6_K, M_PLAIN_FX, 1>(st, a, 1);
  return hipErrorNotSupported;
}

bool decode_gate_up_can_select(int type, int64_t cols, int32_t E, int32_t K) {
  if (E > 256 || K > 16 || K > E) return false;
  if (type == T_Q4_K && dec_gate_up_tq4_supported(cols)) return true;
  // the register kernels select too, where their geometry fits the row
  int lpr, tpl;
  const int64_t el = is_kquant(type) ? 256 : 32;
  if (cols % el) return false;
  return (type == T_Q4_K || type == T_Q6_K || type == T_Q8_0) &&
         reg_geometry(type, (int)((is_kquant(type) ? 4 : 1) * (cols / el)), lpr, tpl);
}

hipError_t launch_decode_gate_up(hipStream_t st, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                                 const Routing &rt, int max_active, const int8_t *xq, const float *xd,
                                 const int32_t *xbs, float *h, const DecSelect *sel, const BlockDbg *dbg,
                                 const SharedGateUp *sgu) {
  if (sgu) {  // the shared rows as extra items of the register kernel only (Q4_K and Q8_0 rows)
    if (dbg || (type != T_Q4_K && type != T_Q8_0) || (type == T_Q4_K && dec_gate_up_tq4_supported(cols)) ||
        sgu->rows <= 0)
      return hipErrorNotSupported;
  }
  MvArgs a{};
  if (dbg) a.dbg = *dbg;
  if (sgu) {
    a.sgu_w = sgu->w;
    a.sgu_rows = sgu->rows;
    a.sgu_h = sgu->h;
  }
  // the shared blocks ride on the grid of the experts' (at most one expert's
  // worth of groups per rows' worth of shared rows)
  const int sh_groups = sgu ? (int)((sgu->rows + rows - 1) / rows) : 0;
  a.rows = rows;
  a.cols = cols;
  a.xq = xq;
  a.xd = xd;
  a.xbs = xbs;
  a.out = h;
  a.tier = tier;
  a.rt = rt;
  if (sel) {  // one token: the kernel selects the experts from the logits
    if (sel->E > 256 || sel->K > 16 || sel->K > sel->E || sel->K != max_active) return hipErrorNotSupported;
    a.sel_on = 1;
    a.sel = *sel;
  }
  if (type == T_Q4_K) {
    const hipError_t e = launch_dec_gate_up_tq4(st, tier, rows, cols, rt, max_active, xq, xd, xbs, h, sel, dbg);
    if (e != hipErrorNotSupported) return e;
    return dispatch_reg<T_Q4_K, M_GATE_UP, 1>(st, a, max_active + sh_groups);
  }
  if (type == T_Q6_K) return dispatch_reg<T_Q6_K, M_GATE_UP, 2>(st, a, max_active);
  if (type == T_Q8_0) return dispatch_reg<T_Q8_0, M_GATE_UP, 2>(st, a, max_active + sh_groups);
  return hipErrorInvalidValue;
}

template <int TYPE>
static hipError_t launch_qkv_reg(hipStream_t st, const MvArgs &a) {
  const int ntasks = (int)(QT<TYPE>::TPB * (a.cols / QT<TYPE>::EL));
  int lpr, tpl;
  if (!reg_geometry(TYPE, ntasks, lpr, tpl)) return hipErrorNotSupported;
  // Rows 2i and 2i+1 sit in one wave at every step: a step's first row
  // r0 - row_in_wave is a multiple of 64 / LPR.
  const int64_t t32 = (a.rows + 4 * 2 - 1) / (4 * 2), t16 = (a.rows + 4 * 4 - 1) / (4 * 4);
  if (lpr == 32) return launch_reg<TYPE, 32, 1, 1, M_QKV>(st, a, tpl, t32);
  if (lpr == 16) return launch_reg<TYPE, 16, 1, 1, M_QKV>(st, a, tpl, t16);
  return hipErrorNotSupported;  // one row per wave step: pairs not in one wave
}

template <int TYPE>
static hipError_t launch_qkv_norm_reg(hipStream_t st, const MvArgs &a) {
  const int ntasks = (int)(QT<TYPE>::TPB * (a.cols / QT<TYPE>::EL));
  int lpr, tpl;
  if (!reg_geometry(TYPE, ntasks, lpr, tpl) || tpl != 1) return hipErrorNotSupported;
  const int64_t t32 = (a.rows + 4 * 2 - 1) / (4 * 2), t16 = (a.rows + 4 * 4 - 1) / (4 * 4);
  if (lpr == 32) return launch_reg<TYPE, 32, 1, 1, M_QKV_NORM>(st, a, tpl, t32);
  if (lpr == 16) return launch_reg<TYPE, 16, 1, 1, M_QKV_NORM>(st, a, tpl, t16);
  return hipErrorNotSupported;
}

hipError_t launch_matvec_qkv_rope_norm(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                                       const QkvNorm &nm, float *out, const QkvRope &rope) {
  if ((rope.neox && rope.rd != rope.hd) || rope.hd <= 0 || rope.hd % 2 || rope.rd % 2 || rope.rd > rope.hd ||
      rope.nh < 1 || rope.nkv < 0 || rows != (int64_t)(rope.nh + 2 * rope.nkv) * rope.hd)
    return hipErrorNotSupported;
  if (!is_kquant(type) || cols % 256 != 0 || cols / 256 > kRegFxBlocks || !nm.x || !nm.w || !nm.h || !nm.xo ||
      nm.xo == nm.x || (((uintptr_t)nm.x | (uintptr_t)nm.y | (uintptr_t)nm.w | (uintptr_t)nm.h | (uintptr_t)nm.xo) & 15u))
    return hipErrorNotSupported;
  MvArgs a{};
  a.w0 = w;
  a.rows = rows;
  a.cols = cols;
  a.s_rows = 1;
  a.out = out;
  a.rope = rope;
  a.nx = nm.x;
  a.ny = nm.y;
  a.nw = nm.w;
  a.neps = nm.eps;
  a.nxo = nm.xo;
  a.nh = nm.h;
  if (type == T_Q4_K) return launch_qkv_norm_reg<T_Q4_K>(st, a);
  if (type == T_Q6_K) return launch_qkv_norm_reg<T_Q6_K>(st, a);
  return hipErrorNotSupported;
}

hipError_t launch_matvec_qkv_rope(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                                  const int8_t *xq, const float *xd, const int32_t *xbs, float *out,
                                  const QkvRope &rope) {
  if ((rope.neox && rope.rd != rope.hd) || rope.hd <= 0 || rope.hd % 2 || rope.rd % 2 || rope.rd > rope.hd ||
      rope.nh < 1 || rope.nkv < 0 || rows != (int64_t)(rope.nh + 2 * rope.nkv) * rope.hd)
    return hipErrorNotSupported;
  if (!act_fits(type, cols)) return hipErrorNotSupported;
  MvArgs a{};
  a.w0 = w;
  a.rows = rows;
  a.cols = cols;
  a.xq = xq;
  a.xd = xd;
  a.xbs = xbs;
  a.s_rows = 1;
  a.out = out;
  a.rope = rope;
  if (type == T_Q4_K) return launch_qkv_reg<T_Q4_K>(st, a);
  if (type == T_Q6_K) return launch_qkv_reg<T_Q6_K>(st, a);
  if (type == T_Q8_0) return launch_qkv_reg<T_Q8_0>(st, a);
  return hipErrorNotSupported;
}

// Experts with 1..NT token rows on the int path (decode batches) over rows too
// narrow for the tiled few-rows kernels (kmoe_small.hip): the one-token
// register kernel's lane geometry (LPR lanes per row, one task per lane, RPW
// rows per wave) with the activation slices of the expert's NT rows in
// registers, so each weight task is loaded once and dotted with every row of
// the expert. MODE 0: gate and up rows, SwiGLU (transformer.rs:558), h[slot];
// the slices are the slots' token rows of the Q8_K/Q8 x. MODE 1: down rows,
// y[slot]; the slices are the slots' int8 h rows. Items are (active expert,
// block of 4*RPW rows) over the experts with min_rows..max_rows rows on the
// int path, in the active list's order (at most 256 experts). Slots past the
// expert's rows repeat its last (loads unconditional, results dropped).
// DBG: the per-block integers are added into a.dbg as the other int kernels do.
// NR row groups per wave and item: the weights of NR rows are in flight
// together, dotted with the one set of activation slices.
constexpr int kFewMaxExperts = 256;
template <int TYPE, int LPR, int NT, int MODE, bool DBG, int NR = 1>
__global__ void __launch_bounds__(256) k_few_int(MvArgs a) {
  constexpr int RPW = 64 / LPR;
  constexpr int RB = 4 * RPW * NR;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int row_in_wave = lane / LPR, lr = lane % LPR;
  const int64_t cols = a.cols, rows = a.rows;
  const int64_t nblk = cols / QT<TYPE>::EL;
  const int ntasks = (int)(QT<TYPE>::TPB * nblk);
  const int64_t row_bytes = nblk * QT<TYPE>::BYTES;
  const int64_t xs_stride = cols / 16;
  const bool tv = lr < ntasks;
  const int t = tv ? lr : ntasks - 1;
  const int64_t bpe = (rows + RB - 1) / RB;
  const int K = a.rt.topk;
  // the experts this kernel takes, in active-list order (wave 0 ballots over
  // the active list), so items are only theirs
  __shared__ int32_t qe[kFewMaxExperts];
  __shared__ int32_t nq_s;
  if (wave == 0) {
    const int na = *a.rt.n_active;
    int nq = 0;
    for (int j0 = 0; j0 < na; j0 += 64) {
      const int j = j0 + lane;
      bool ok = false;
      int e = 0;
      if (j < na) {
        e = a.rt.active[j];
        const int n = (int)(a.rt.offsets[e + 1] - a.rt.offsets[e]);
        ok = n >= a.min_rows && n <= a.max_rows && int_regime(a.regime, n);
      }
      const uint64_t m = __ballot(ok);
      if (ok) qe[nq + __popcll(m & ((1ull << lane) - 1))] = e;
      nq += __popcll(m);
    }
    if (lane == 0) nq_s = nq;
  }
  __syncthreads();
  const int64_t total = (int64_t)nq_s * bpe;
  for (int64_t b = blockIdx.x; b < total; b += gridDim.x) {
    const int i = (int)(b / bpe);
    const int64_t rblk = b - (int64_t)i * bpe;
    const int e = qe[i];
    const int64_t p0 = a.rt.offsets[e];
    const int n = (int)(a.rt.offsets[e + 1] - (uint32_t)p0);
    ActSlice<TYPE> act[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int64_t p = p0 + (j < n ? j : n - 1);
      const int64_t src = MODE == 0 ? (int64_t)(a.rt.perm[p] / (uint32_t)K) : p;  // token row, or the slot's h row
      act_load<TYPE>(act[j], a.xq + src * cols, a.xd + src * nblk, a.xbs + src * xs_stride, t);
    }
    const uint8_t *eb = a.tier.base + (int64_t)e * a.tier.stride;
    WTask<TYPE, true> w0s[NR], w1s[NR];
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      const int64_t r = rblk * RB + ((int64_t)wave * NR + q) * RPW + row_in_wave;
      const int64_t rc = r < rows ? r : rows - 1;
      w_load<TYPE, true>(w0s[q], eb + a.tier.off[MODE == 0 ? 0 : 2] + rc * row_bytes, t, nblk);
      if constexpr (MODE == 0) w_load<TYPE, true>(w1s[q], eb + a.tier.off[1] + rc * row_bytes, t, nblk);
    }
#pragma unroll
    for (int q = 0; q < NR; ++q) {
    const int64_t r = rblk * RB + ((int64_t)wave * NR + q) * RPW + row_in_wave;
    const WTask<TYPE, true> &w0 = w0s[q], &w1 = w1s[q];
    float g[NT], u[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      int32_t *ds0 = nullptr, *dm0 = nullptr, *ds1 = nullptr, *dm1 = nullptr;
      if constexpr (DBG) {
        if (tv && j < n && r < rows) {
          const int64_t o = ((p0 + j) * rows + r) * nblk;
          ds0 = a.dbg.s[0] ? a.dbg.s[0] + o : nullptr;
          dm0 = a.dbg.m[0] ? a.dbg.m[0] + o : nullptr;
          ds1 = a.dbg.s[1] ? a.dbg.s[1] + o : nullptr;
          dm1 = a.dbg.m[1] ? a.dbg.m[1] + o : nullptr;
        }
      }
      const float vg = task_dot<TYPE>(w0, t, act[j], 0.0f, ds0, dm0);
      g[j] = group_sum<LPR>(tv ? vg : 0.0f);
      if constexpr (MODE == 0) {
        const float vu = task_dot<TYPE>(w1, t, act[j], 0.0f, ds1, dm1);
        u[j] = group_sum<LPR>(tv ? vu : 0.0f);
      }
    }
    if (lr == 0 && r < rows) {
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (j >= n) break;
        if constexpr (MODE == 0) {  // SwiGLU: g / (1 + exp(-g)) * u
          const float den = 1.0f + expf_cr(-g[j]);
          const float q = g[j] / den;
          a.out[(p0 + j) * rows + r] = q * u[j];
        } else {
          a.out[(p0 + j) * rows + r] = g[j];
        }
      }
    }
    }
  }
}

constexpr int kFewNR = 2;  // row groups per wave and item of k_few_int

template <int TYPE, int MODE>
static hipError_t launch_few_int_t(hipStream_t st, const MvArgs &a, int lpr, int max_active, bool dbg) {
  const int rpw = 64 / lpr;
  const int64_t bpe = (a.rows + 4 * rpw * kFewNR - 1) / (4 * rpw * kFewNR);
  const int64_t items = (int64_t)max_active * bpe;
  // as many work-groups per CU as are resident at once (the kernel's
  // registers decide: 3 for the Q4_K gate/up, 4 or more for the others)
  auto grid_for = [&](const void *k, int &occ) -> unsigned {
    if (occ == 0) {
      int o = 0;
      if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&o, k, 256, 0) != hipSuccess || o < 1) o = kGridMult;
      occ = o < 8 ? o : 8;
    }
    const int64_t cap = (int64_t)cu_count() * occ;
    return (unsigned)(items < cap ? items : cap);
  };
#define KMOE_FEW_D(L, DB)                                                                               \
  do {                                                                                                  \
    static int occ = 0;                                                                                 \
    const unsigned grid = grid_for((const void *)k_few_int<TYPE, L, 3, MODE, DB, kFewNR>, occ);         \
    KMOE_LAUNCH((k_few_int<TYPE, L, 3, MODE, DB, kFewNR>), dim3(grid), dim3(256), 0, st, a);            \
  } while (0)
#define KMOE_FEW(L)                  \
  do {                               \
    if (dbg) KMOE_FEW_D(L, true);    \
    else KMOE_FEW_D(L, false);       \
    return hipGetLastError();        \
  } while (0)
  if (lpr == 16) KMOE_FEW(16);
  if (lpr == 32) KMOE_FEW(32);
  if (lpr == 64) KMOE_FEW(64);
#undef KMOE_FEW
#undef KMOE_FEW_D
  return hipErrorNotSupported;
}

hipError_t launch_few_int(hipStream_t st, int mode, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                          const Routing &rt, int regime, int max_active, const int8_t *xq, const float *xd,
                          const int32_t *xbs, float *out, int max_rows, const BlockDbg *dbg) {
  if (rows <= 0 || max_active <= 0) return hipSuccess;
  if (max_rows < 1 || max_rows > 3 || max_active > kFewMaxExperts || !act_fits(type, cols))
    return hipErrorNotSupported;
  const int ntasks = (int)((is_kquant(type) ? 4 : 1) * (cols / (is_kquant(type) ? 256 : 32)));
  int lpr, tpl;
  if (!reg_geometry(type, ntasks, lpr, tpl) || tpl != 1) return hipErrorNotSupported;
  MvArgs a{};
  if (dbg) a.dbg = *dbg;
  a.rows = rows;
  a.cols = cols;
  a.xq = xq;
  a.xd = xd;
  a.xbs = xbs;
  a.out = out;
  a.tier = tier;
  a.rt = rt;
  a.regime = regime;
  a.min_rows = 1;
  a.max_rows = max_rows;
  const bool g = dbg != nullptr;
  if (type == T_Q4_K)
    return mode == 0 ? launch_few_int_t<T_Q4_K, 0>(st, a, lpr, max_active, g)
                     : launch_few_int_t<T_Q4_K, 1>(st, a, lpr, max_active, g);
  if (type == T_Q6_K)
    return mode == 0 ? launch_few_int_t<T_Q6_K, 0>(st, a, lpr, max_active, g)
                     : launch_few_int_t<T_Q6_K, 1>(st, a, lpr, max_active, g);
  if (type == T_Q8_0)
    return mode == 0 ? launch_few_int_t<T_Q8_0, 0>(st, a, lpr, max_active, g)
                     : launch_few_int_t<T_Q8_0, 1>(st, a, lpr, max_active, g);
  return hipErrorNotSupported;
}

// k_mv_down_exp for rows of at most 64 task slots: lanes per row as the
// register kernel picks them, the smallest KMAX >= topk, 3 register sets, and
// waves per work-group so that the row blocks number at least two per CU.
template <int TYPE>
hipError_t launch_down_exp(hipStream_t st, const MvArgs &a, int ntasks, int topk, bool dbg) {
  int lpr, tpl;
  if (!reg_geometry(TYPE, ntasks, lpr, tpl) || tpl != 1) return hipErrorNotSupported;
  const int rpw = 64 / lpr;
  int wpb = 4;
  while (wpb > 1 && (a.rows + rpw * wpb - 1) / (rpw * wpb) < 2 * (int64_t)cu_count()) wpb >>= 1;
  const int64_t blocks = (a.rows + (int64_t)rpw * wpb - 1) / ((int64_t)rpw * wpb);
  const int64_t cap = (int64_t)cu_count() * kGridMult * (4 / wpb);
  const unsigned grid = (unsigned)(blocks < cap ? blocks : cap);
  const int kmax = topk <= 2 ? 2 : topk <= 4 ? 4 : topk <= 6 ? 6 : 8;
#define KMOE_DX(L, KM, WP)                                                                                         \
  do {                                                                                                             \
    if (dbg) KMOE_LAUNCH((k_mv_down_exp<TYPE, L, KM, 3, WP, true>), dim3(grid), dim3(64 * WP), 0, st, a);         \
    else KMOE_LAUNCH((k_mv_down_exp<TYPE, L, KM, 3, WP, false>), dim3(grid), dim3(64 * WP), 0, st, a);            \
    return hipGetLastError();                                                                                      \
  } while (0)
#define KMOE_DX_K(L, WP)             \
  do {                               \
    if (kmax == 2) KMOE_DX(L, 2, WP); \
    if (kmax == 4) KMOE_DX(L, 4, WP); \
    if (kmax == 6) KMOE_DX(L, 6, WP); \
    KMOE_DX(L, 8, WP);               \
  } while (0)
#define KMOE_DX_W(L)                  \
  do {                                \
    if (wpb == 1) KMOE_DX_K(L, 1);    \
    if (wpb == 2) KMOE_DX_K(L, 2);    \
    KMOE_DX_K(L, 4);                  \
  } while (0)
  if (lpr == 64) KMOE_DX_W(64);
  if (lpr == 32) KMOE_DX_W(32);
  if (lpr == 16) KMOE_DX_W(16);
#undef KMOE_DX_W
#undef KMOE_DX_K
#undef KMOE_DX
  return hipErrorNotSupported;
}

// The register down + combine over narrow rows with the shared expert's down
// row fused in (k_mv_down_exp<..., SHT>): the launch shape of launch_down_exp,
// for the shapes where both rows take the same lanes per row and one task
// slot per lane, the routed experts' top-k at most 8 and 4..8 experts' ring.
template <int TYPE, int SHT>
static hipError_t launch_down_shared_t(hipStream_t st, const MvArgs &a, int lpr, int topk) {
  const int rpw = 64 / lpr;
  int wpb = 4;
  while (wpb > 1 && (a.rows + rpw * wpb - 1) / (rpw * wpb) < 2 * (int64_t)cu_count()) wpb >>= 1;
  const int64_t blocks = (a.rows + (int64_t)rpw * wpb - 1) / ((int64_t)rpw * wpb);
  const int64_t cap = (int64_t)cu_count() * kGridMult * (4 / wpb);
  const unsigned grid = (unsigned)(blocks < cap ? blocks : cap);
  const int kmax = topk <= 4 ? 4 : topk <= 6 ? 6 : 8;
#define KMOE_DS(L, WP)                                                                                         \
  do {                                                                                                         \
    if (kmax == 4) KMOE_LAUNCH((k_mv_down_exp<TYPE, L, 4, 3, WP, false, SHT>), dim3(grid), dim3(64 * WP), 0, st, a); \
    else if (kmax == 6)                                                                                        \
      KMOE_LAUNCH((k_mv_down_exp<TYPE, L, 6, 3, WP, false, SHT>), dim3(grid), dim3(64 * WP), 0, st, a);     \
    else KMOE_LAUNCH((k_mv_down_exp<TYPE, L, 8, 3, WP, false, SHT>), dim3(grid), dim3(64 * WP), 0, st, a);  \
    return hipGetLastError();                                                                                  \
  } while (0)
  if (lpr == 64 && wpb == 4) KMOE_DS(64, 4);
  if (lpr == 32 && wpb == 2) KMOE_DS(32, 2);
  if (lpr == 16 && wpb == 1) KMOE_DS(16, 1);
#undef KMOE_DS
  return hipErrorNotSupported;
}

hipError_t launch_decode_down_shared(hipStream_t st, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                                     const Routing &rt, const int8_t *hq, const float *hd, const int32_t *hbs,
                                     float *out, const SharedDown &sh) {
  if (rt.topk < 1 || rt.topk > 8 || rows <= 0) return hipErrorNotSupported;
  const int ntasks = (int)((is_kquant(type) ? 4 : 1) * (cols / (is_kquant(type) ? 256 : 32)));
  const int sh_ntasks = (int)((is_kquant(sh.type) ? 4 : 1) * (sh.cols / (is_kquant(sh.type) ? 256 : 32)));
  int lpr, tpl, slpr, stpl;
  if (!act_fits(type, cols) || !act_fits(sh.type, sh.cols)) return hipErrorNotSupported;
  if (!reg_geometry(type, ntasks, lpr, tpl) || tpl != 1 || !reg_geometry(sh.type, sh_ntasks, slpr, stpl) ||
      stpl != 1 || slpr != lpr)
    return hipErrorNotSupported;
  MvArgs a{};
  a.s_rows = 1;
  a.rows = rows;
  a.cols = cols;
  a.xq = hq;
  a.xd = hd;
  a.xbs = hbs;
  a.out = out;
  a.tier = tier;
  a.rt = rt;
  a.sh_w = sh.w;
  a.sh_cols = sh.cols;
  a.sh_xq = sh.xq;
  a.sh_xd = sh.xd;
  a.sh_xbs = sh.xbs;
  a.sh_logit = sh.logit;
#define KMOE_DST(T)                                                                             \
  do {                                                                                          \
    if (sh.type == T_Q6_K) return launch_down_shared_t<T, T_Q6_K>(st, a, lpr, rt.topk);        \
    if (sh.type == T_Q4_K) return launch_down_shared_t<T, T_Q4_K>(st, a, lpr, rt.topk);        \
    return hipErrorNotSupported;                                                                \
  } while (0)
  if (type == T_Q8_0) KMOE_DST(T_Q8_0);
  if (type == T_Q4_K) KMOE_DST(T_Q4_K);
  if (type == T_Q6_K) KMOE_DST(T_Q6_K);
#undef KMOE_DST
  return hipErrorNotSupported;
}

hipError_t launch_decode_down_combine(hipStream_t st, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                                      const Routing &rt, const int8_t *hq, const float *hd, const int32_t *hbs,
                                      float *out, const BlockDbg *dbg) {
  MvArgs a{};
  if (dbg) a.dbg = *dbg;
  a.s_rows = 1;
  a.rows = rows;
  a.cols = cols;
  a.xq = hq;
  a.xd = hd;
  a.xbs = hbs;
  a.out = out;
  a.tier = tier;
  a.rt = rt;
  const int64_t nblk = cols / (is_kquant(type) ? 256 : 32);
  const int ntasks = (int)((is_kquant(type) ? 4 : 1) * nblk);
  // one token: its topk experts are distinct, so k slots are active
  if (ntasks >= 128 && ntasks <= 4 * 64 * 2) {
    // persistent split-K: one work-group per CU, rows split evenly
    const int64_t G = (int64_t)cu_count() * kDownWgPerCu;
    int rb = (int)((rows + G - 1) / G);
    if (rb <= kSplitRbMax) {
      const unsigned grid = (unsigned)((rows + rb - 1) / rb);
      const int tpl = (ntasks + 3) / 4 > 64 ? 2 : 1;
#define KMOE_SPLITK(T, RU, TP)                                                                        \
  do {                                                                                                \
    if (dbg) KMOE_LAUNCH((k_down_splitk<T, RU, TP, true>), dim3(grid), dim3(256), 0, st, a, rb);      \
    else KMOE_LAUNCH((k_down_splitk<T, RU, TP, false>), dim3(grid), dim3(256), 0, st, a, rb);         \
  } while (0)
      if (type == T_Q4_K) {
        if (tpl == 1 && rt.topk <= 2) {
          // the ring kernel: 2 rows per item, at most 8 items
          const int items = rt.topk * ((rb + 1) / 2);
          if (items <= 8) {
#define KMOE_RING(NIT_, NS_)                                                                                      \
  do {                                                                                                            \
    if (dbg) KMOE_LAUNCH((k_down_ring<T_Q4_K, 2, NIT_, NS_, true>), dim3(grid), dim3(256), 0, st, a, rb);        \
    else KMOE_LAUNCH((k_down_ring<T_Q4_K, 2, NIT_, NS_, false>), dim3(grid), dim3(256), 0, st, a, rb);           \
  } while (0)
            if (items <= 4) KMOE_RING(4, kDownRingSets);
            else KMOE_RING(8, kDownRingSets);
#undef KMOE_RING
            return hipGetLastError();
          }
        }
        if (tpl == 1) {
          KMOE_SPLITK(T_Q4_K, kDownRu, 1);
        } else {
          KMOE_SPLITK(T_Q4_K, 2, 2);
        }
      } else if (type == T_Q6_K) {  // 26 registers per task: fewer rows per item
        if (tpl == 1 && rt.topk <= 2 && rt.topk * ((rb + 1) / 2) <= 8) {
#define KMOE_RING6(NIT_)                                                                                     \
  do {                                                                                                       \
    if (dbg) KMOE_LAUNCH((k_down_ring<T_Q6_K, 2, NIT_, kDownRingSets, true>), dim3(grid), dim3(256), 0, st, a, rb);     \
    else KMOE_LAUNCH((k_down_ring<T_Q6_K, 2, NIT_, kDownRingSets, false>), dim3(grid), dim3(256), 0, st, a, rb);        \
  } while (0)
          if (rt.topk * ((rb + 1) / 2) <= 4) KMOE_RING6(4);
          else KMOE_RING6(8);
#undef KMOE_RING6
          return hipGetLastError();
        }
        if (tpl == 1) KMOE_SPLITK(T_Q6_K, 2, 1);
        else KMOE_SPLITK(T_Q6_K, 1, 2);
      } else {
        if (tpl == 1) KMOE_SPLITK(T_Q8_0, 4, 1);
        else KMOE_SPLITK(T_Q8_0, 2, 2);
      }
#undef KMOE_SPLITK
      return hipGetLastError();
    }
  }
  if (rt.topk <= 8) {
    hipError_t e = hipErrorNotSupported;
    if (type == T_Q4_K) e = launch_down_exp<T_Q4_K>(st, a, ntasks, rt.topk, dbg != nullptr);
    else if (type == T_Q6_K) e = launch_down_exp<T_Q6_K>(st, a, ntasks, rt.topk, dbg != nullptr);
    else if (type == T_Q8_0) e = launch_down_exp<T_Q8_0>(st, a, ntasks, rt.topk, dbg != nullptr);
    if (e != hipErrorNotSupported) return e;
  }
  if (type == T_Q4_K) return dispatch_reg<T_Q4_K, M_DOWN_COMBINE, 1>(st, a, 1);
  if (type == T_Q6_K) return dispatch_reg<T_Q6_K, M_DOWN_COMBINE, 1>(st, a, 1);
  if (type == T_Q8_0) return dispatch_reg<T_Q8_0, M_DOWN_COMBINE, 1>(st, a, 1);
  return hipErrorInvalidValue;
}

hipError_t launch_matvec_int(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols, const int8_t *xq,
                             const float *xd, const int32_t *xbs, int64_t s_rows, float *out) {
  if (rows == 0 || s_rows == 0) return hipSuccess;
  if (!act_fits(type, cols)) return hipErrorInvalidValue;
  MvArgs a{};
  a.w0 = w;
  a.rows = rows;
  a.cols = cols;
  a.xq = xq;
  a.xd = xd;
  a.xbs = xbs;
  a.s_rows = s_rows;
  a.out = out;
  a.rows_per_block = kRowsPerBlock;
  const int nt = pick_nt(type, cols, s_rows);
  const dim3 grid = plain_grid(a, rows, s_rows, nt);
  if (type == T_Q4_K) return dispatch_lpr_nt<T_Q4_K, M_PLAIN>(st, a, grid, nt);
  if (type == T_Q6_K) return dispatch_lpr_nt<T_Q6_K, M_PLAIN>(st, a, grid, nt);
  if (type == T_Q8_0) return dispatch_lpr_nt<T_Q8_0, M_PLAIN>(st, a, grid, nt);
  return hipErrorInvalidValue;
}

hipError_t launch_block_sums(hipStream_t st, int type, const uint8_t *w, int64_t rows, int64_t cols,
                             const int8_t *xq, const int32_t *xbs, int64_t s_rows, int32_t *sumi, int32_t *mins) {
  if (rows == 0 || s_rows == 0) return hipSuccess;
  if (!act_fits(type, cols)) return hipErrorInvalidValue;
  MvArgs a{};
  a.w0 = w;
  a.rows = rows;
  a.cols = cols;
  a.xq = xq;
  a.xbs = xbs;
  a.s_rows = s_rows;
  a.isumi = sumi;
  a.imins = mins;
  a.rows_per_block = kRowsPerBlock;
  const dim3 grid = plain_grid(a, rows, s_rows, 1);
  // The Q8_0 scales are not read by the sums; the K-quants' dw/xd are not either, but
  // the staging copies xd: give it a valid dummy of the right length.
  a.xd = (const float *)xq;  // nblk*4 bytes <= cols bytes are readable there
  if (type == T_Q4_K) return dispatch_lpr_nt<T_Q4_K, M_SUMS>(st, a, grid, 1);
  if (type == T_Q6_K) return dispatch_lpr_nt<T_Q6_K, M_SUMS>(st, a, grid, 1);
  if (type == T_Q8_0) return dispatch_lpr_nt<T_Q8_0, M_SUMS>(st, a, grid, 1);
  return hipErrorInvalidValue;
}

hipError_t launch_moe_int(hipStream_t st, int mode, int type, const ExpertTier &tier, int64_t rows, int64_t cols,
                          const Routing &rt, int regime, int max_active, int64_t s_rows, const int8_t *xq,
                          const float *xd, const int32_t *xbs, float *out, int min_rows, const BlockDbg *dbg) {
  if (rows == 0 || max_active == 0) return hipSuccess;
  if (!act_fits(type, cols)) return hipErrorInvalidValue;
  MvArgs a{};
  if (dbg) a.dbg = *dbg;
  a.rows = rows;
  a.cols = cols;
  a.xq = xq;
  a.xd = xd;
  a.xbs = xbs;
  a.out = out;
  a.tier = tier;
  a.rt = rt;
  a.regime = regime;
  a.min_rows = min_rows;
  a.rows_per_block = kRowsPerBlock;
  dim3 grid((unsigned)((rows + kRowsPerBlock - 1) / kRowsPerBlock), (unsigned)max_active);
  // A single token routes at most one row to each expert: the NT=1 kernel;
  // otherwise passes sized for the mean rows per active expert.
  const int nt = s_rows == 1 ? 1 : pick_nt(type, cols, (s_rows * rt.topk + max_active - 1) / max_active);
  if (type == T_Q4_K)
    return mode == 0 ? dispatch_lpr_nt<T_Q4_K, M_GATE_UP>(st, a, grid, nt)
                     : dispatch_lpr_nt<T_Q4_K, M_DOWN>(st, a, grid, nt);
  if (type == T_Q6_K)
    return mode == 0 ? dispatch_lpr_nt<T_Q6_K, M_GATE_UP>(st, a, grid, nt)
                     : dispatch_lpr_nt<T_Q6_K, M_DOWN>(st, a, grid, nt);
  if (type == T_Q8_0)
    return mode == 0 ? dispatch_lpr_nt<T_Q8_0, M_GATE_UP>(st, a, grid, nt)
                     : dispatch_lpr_nt<T_Q8_0, M_DOWN>(st, a, grid, nt);
  return hipErrorInvalidValue;
}

}  // namespace kmoe
