// kmoe_decode.hip — single-token (decode) gate/up + SwiGLU over the expert
// tier's tiled Q4_K rows.
//
// One wave owns RU consecutive rows of one expert per step and reads, for each
// row of gate and of up, three 16-byte pieces per lane: the head of superblock
// sb = t/4 and the two nibble chunks of quarter k = t%4 (t = lane + 64*i).
// In the tiled layout (tq4_qs_off) every such load instruction covers one
// contiguous run of bytes, and the lane's offsets inside a row are the same
// for every row, so they are computed once; the row base is wave-uniform
// (scalar registers). All 6*RU loads of a step are issued before any is used.
// Each lane keeps its slice of the Q8_K activation row (64 int8, the two
// 32-element sums and the block scale) in registers for the whole kernel.
// The dot products are the reference's (avx2.rs:351-379): per quarter,
// sumi = sA*sum(lo*x) + sB*sum(hi*x) and mins = mA*bsA + mB*bsB in int32,
// then acc += (d*xd)*sumi - (dmin*xd)*mins. After the 64-lane sums, lane u
// of the wave holds row u's gate and up sums and computes SwiGLU
// (transformer.rs:558) for it, so the exponential runs once per step.
#include "kmoe_device.h"
#include "kmoe_launch.h"
#include "kmoe_select.h"
#include "kmoe_tq4.h"

namespace kmoe {

namespace {

struct DecArgs {
  ExpertTier tier;
  Routing rt;
  int64_t rows, cols;  // rows = F (gate/up rows), cols = d
  const int8_t *xq;
  const float *xd;
  const int32_t *xbs;
  float *h;  // [slots, F]: h[p, r] for the slot p of expert e (one token)
  int32_t groups_per_expert;  // work-groups along the rows of one expert
  DecSelect sel;              // logits given: this kernel selects the experts
};

// TPL task slots per lane (a row has 4*nb <= 64*TPL quarters), RU rows per step.
// NPER = 0: the routing (active experts, slot offsets) is given. NPER > 0:
// every wave selects the token's experts from its E <= 64*NPER logits itself
// (softmax, top-k, renormalisation), work-group (0, 0) publishes the routing
// (idx, weights, permutation, offsets, active list), and the work-groups of
// grid row y take the y-th smallest selected expert, whose slot is y.
template <int TPL, int RU, int NPER>
__global__ void __launch_bounds__(256) k_dec_gate_up_tq4(DecArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nb = a.cols / 256, ntasks = 4 * nb;
  const int64_t row_bytes = nb * 144;

  // lane constants: offsets inside a row and the activation slice, whose loads
  // do not depend on the expert and are issued before the selection
  uint32_t oh[TPL], oa[TPL], ob[TPL];
  bool tv[TPL];
  Slice s[TPL];
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const int64_t t0 = lane + 64 * i;
    tv[i] = t0 < ntasks;
    const int64_t t = tv[i] ? t0 : ntasks - 1;
    const int64_t sb = t >> 2;
    const int k = (int)(t & 3);
    oh[i] = (uint32_t)(16 * sb);
    oa[i] = (uint32_t)tq4_qs_off(nb, sb, k, 0);
    ob[i] = oa[i] + (uint32_t)tq4_j_stride(nb, sb);
    const int4 *xv = (const int4 *)(a.xq + 256 * sb + 64 * k);
    s[i].x0 = xv[0];
    s[i].x1 = xv[1];
    s[i].x2 = xv[2];
    s[i].x3 = xv[3];
    const int4 bs = *(const int4 *)(a.xbs + 16 * sb + 4 * k);
    s[i].bsA = bs.x + bs.y;
    s[i].bsB = bs.z + bs.w;
    s[i].d = a.xd[sb];
  }
  const int slot_i = blockIdx.y;  // index into the active-expert list
  int e;
  int64_t p;
  if constexpr (NPER == 0) {
    if (slot_i >= *a.rt.n_active) return;
    e = a.rt.active[slot_i];
    p = slot_i;  // one token: the slot_i-th active expert's single slot is at position slot_i
  } else {
    __shared__ float P[4][64 * (NPER > 0 ? NPER : 1)];
    const DecSelect &q = a.sel;
    float lv[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) lv[i] = lane + 64 * i < q.E ? q.logits[lane + 64 * i] : -INFINITY;
    uint32_t sj[16];
    float wj[16];
    wave_route_one<NPER>(lv, q.E, q.K, q.norm_topk, q.weights_scale, P[wave], sj, wj);
    uint32_t rk[16];
    selection_ranks(sj, q.K, rk);
    e = -1;
    for (int j = 0; j < q.K; ++j)
      if ((int)rk[j] == slot_i) e = (int)sj[j];
    if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0)  // publish the routing of the token
      publish_selection(sj, wj, rk, q.K, q.E, lane, q.idx, q.wsel, q.perm, q.inv, q.active, q.n_active, q.offsets);
    if (e < 0) return;
    p = slot_i;
  }
  const uint8_t *G = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[0];
  const uint8_t *U = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[1];

  const int kq = lane & 3;  // quarter of every slot of this lane (64*i keeps it)

  const int64_t rows = a.rows;
  const int64_t rows_per_wg = 4 * RU;
  for (int64_t r0 = ((int64_t)blockIdx.x * 4 + wave) * RU; r0 < rows;
       r0 += (int64_t)a.groups_per_expert * rows_per_wg) {
    u32x4 hg[RU][TPL], ag[RU][TPL], bg[RU][TPL], hu[RU][TPL], au[RU][TPL], bu[RU][TPL];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int64_t r = r0 + u < rows ? r0 + u : rows - 1;
      const uint8_t *gr = G + r * row_bytes;
      const uint8_t *ur = U + r * row_bytes;
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        hg[u][i] = __builtin_nontemporal_load((const u32x4 *)(gr + oh[i]));
        ag[u][i] = __builtin_nontemporal_load((const u32x4 *)(gr + oa[i]));
        bg[u][i] = __builtin_nontemporal_load((const u32x4 *)(gr + ob[i]));
        hu[u][i] = __builtin_nontemporal_load((const u32x4 *)(ur + oh[i]));
        au[u][i] = __builtin_nontemporal_load((const u32x4 *)(ur + oa[i]));
        bu[u][i] = __builtin_nontemporal_load((const u32x4 *)(ur + ob[i]));
      }
    }
    float gsum = 0.0f, usum = 0.0f;  // lane u < RU: row r0+u
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      float ag_acc = 0.0f, au_acc = 0.0f;
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        int mg, mu;
        const int sg = q4k_quarter(hg[u][i], ag[u][i], bg[u][i], kq, s[i], mg);
        const int su = q4k_quarter(hu[u][i], au[u][i], bu[u][i], kq, s[i], mu);
        const float dg = f16_bits_to_f32(hg[u][i].x) * s[i].d, mgf = f16_bits_to_f32(hg[u][i].x >> 16) * s[i].d;
        const float du = f16_bits_to_f32(hu[u][i].x) * s[i].d, muf = f16_bits_to_f32(hu[u][i].x >> 16) * s[i].d;
        float vg = fmaf(dg, (float)sg, -(mgf * (float)mg));
        float vu = fmaf(du, (float)su, -(muf * (float)mu));
        vg = tv[i] ? vg : 0.0f;
        vu = tv[i] ? vu : 0.0f;
        ag_acc += vg;
        au_acc += vu;
      }
      ag_acc = group_sum<64>(ag_acc);
      au_acc = group_sum<64>(au_acc);
      gsum = lane == u ? ag_acc : gsum;
      usum = lane == u ? au_acc : usum;
    }
    if (lane < RU && r0 + lane < rows) {  // SwiGLU: g / (1 + exp(-g)) * u
      const float den = 1.0f + expf_cr(-gsum);
      const float q = gsum / den;
      a.h[p * rows + r0 + lane] = q * usum;
    }
  }
}

// Rows of one matrix against one Q8_K activation row (quant::matmul at one
// row on the int path, quant.rs:262-309: dot_q4_k_8k per row), with the
// structure of the gate/up kernel above: lane-constant offsets inside a row,
// the activation slice in registers, 3 loads per task and row, RU rows per
// wave step; lane u of the wave ends with row r0+u. Rows in GGUF order (head
// at 144*sb, nibble chunk (k, j) at 144*sb + 16 + 32k + 16j; rows need only
// 4-byte alignment) or tiled (tq4_qs_off).
struct RowsArgs {
  const uint8_t *W;
  int64_t rows, cols;
  const int8_t *xq;
  const float *xd;
  const int32_t *xbs;
  float *out;
  int32_t groups;  // work-groups striding over the rows
};

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

template <bool TILED, int TPL, int RU>
__global__ void __launch_bounds__(256) k_dec_rows(RowsArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nb = a.cols / 256, ntasks = 4 * nb;
  const int64_t row_bytes = nb * 144;
  uint32_t oh[TPL], oa[TPL], ob[TPL];
  bool tv[TPL];
  Slice s[TPL];
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const int64_t t0 = lane + 64 * i;
    tv[i] = t0 < ntasks;
    const int64_t t = tv[i] ? t0 : ntasks - 1;
    const int64_t sb = t >> 2;
    const int k = (int)(t & 3);
    if constexpr (TILED) {
      oh[i] = (uint32_t)(16 * sb);
      oa[i] = (uint32_t)tq4_qs_off(nb, sb, k, 0);
      ob[i] = oa[i] + (uint32_t)tq4_j_stride(nb, sb);
    } else {
      oh[i] = (uint32_t)(144 * sb);
      oa[i] = oh[i] + 16 + 32 * k;
      ob[i] = oa[i] + 16;
    }
    const int4 *xv = (const int4 *)(a.xq + 256 * sb + 64 * k);
    s[i].x0 = xv[0];
    s[i].x1 = xv[1];
    s[i].x2 = xv[2];
    s[i].x3 = xv[3];
    const int4 bs = *(const int4 *)(a.xbs + 16 * sb + 4 * k);
    s[i].bsA = bs.x + bs.y;
    s[i].bsB = bs.z + bs.w;
    s[i].d = a.xd[sb];
  }
  const int kq = lane & 3;
  const int64_t rows = a.rows;
  for (int64_t r0 = ((int64_t)blockIdx.x * 4 + wave) * RU; r0 < rows; r0 += (int64_t)a.groups * 4 * RU) {
    u32x4 hw[RU][TPL], aw[RU][TPL], bw[RU][TPL];
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const uint8_t *row = a.W + (r0 + u < rows ? r0 + u : rows - 1) * row_bytes;
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        if constexpr (TILED) {
          hw[u][i] = __builtin_nontemporal_load((const u32x4 *)(row + oh[i]));
          aw[u][i] = __builtin_nontemporal_load((const u32x4 *)(row + oa[i]));
          bw[u][i] = __builtin_nontemporal_load((const u32x4 *)(row + ob[i]));
        } else {
          hw[u][i] = __builtin_nontemporal_load((const u32x4a4 *)(row + oh[i]));
          aw[u][i] = __builtin_nontemporal_load((const u32x4a4 *)(row + oa[i]));
          bw[u][i] = __builtin_nontemporal_load((const u32x4a4 *)(row + ob[i]));
        }
      }
    }
    float res = 0.0f;  // lane u < RU: row r0+u
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      float acc = 0.0f;
#pragma unroll
      for (int i = 0; i < TPL; ++i) {
        int m;
        const int si = q4k_quarter(hw[u][i], aw[u][i], bw[u][i], kq, s[i], m);
        const float dd = f16_bits_to_f32(hw[u][i].x) * s[i].d, mf = f16_bits_to_f32(hw[u][i].x >> 16) * s[i].d;
        const float v = fmaf(dd, (float)si, -(mf * (float)m));
        acc += tv[i] ? v : 0.0f;
      }
      acc = group_sum<64>(acc);
      res = lane == u ? acc : res;
    }
    if (lane < RU && r0 + lane < rows) a.out[r0 + lane] = res;
  }
}

}  // namespace

bool dec_rows_supported(int64_t cols) {
  if (cols % 256 != 0) return false;
  const int64_t ntasks = 4 * (cols / 256);
  return ntasks >= 48 && ntasks <= 256;
}

hipError_t launch_dec_rows(hipStream_t st, bool tiled, const uint8_t *w, int64_t rows, int64_t cols, const int8_t *xq,
                           const float *xd, const int32_t *xbs, float *out) {
  if (rows <= 0) return hipSuccess;
  if (!dec_rows_supported(cols) || ((uintptr_t)w & 3u) || (tiled && ((uintptr_t)w & 15u)) || ((uintptr_t)xq & 15u) ||
      ((uintptr_t)xbs & 15u))
    return hipErrorNotSupported;
  const int tpl = (int)((4 * (cols / 256) + 63) / 64);
  const int ru = tpl <= 2 ? 2 : 1;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  RowsArgs a{w, rows, cols, xq, xd, xbs, out, 0};
  // work-group steps of 4*RU rows, spread evenly over about two groups per CU
  const int64_t need = (rows + 4 * ru - 1) / (4 * ru);
  const int64_t cap = 2LL * cus;
  const int64_t per = (need + cap - 1) / cap;
  a.groups = (int32_t)((need + per - 1) / per);
  const dim3 grid((unsigned)a.groups);
#define KMOE_DEC_ROWS(TL)                                                                      \
  do {                                                                                         \
    if (tpl == 1) KMOE_LAUNCH((k_dec_rows<TL, 1, 2>), grid, dim3(256), 0, st, a);              \
    else if (tpl == 2) KMOE_LAUNCH((k_dec_rows<TL, 2, 2>), grid, dim3(256), 0, st, a);         \
    else if (tpl == 3) KMOE_LAUNCH((k_dec_rows<TL, 3, 1>), grid, dim3(256), 0, st, a);         \
    else KMOE_LAUNCH((k_dec_rows<TL, 4, 1>), grid, dim3(256), 0, st, a);                       \
  } while (0)
  if (tiled) KMOE_DEC_ROWS(true);
  else KMOE_DEC_ROWS(false);
#undef KMOE_DEC_ROWS
  return hipGetLastError();
}

bool dec_gate_up_tq4_supported(int64_t cols, int ru) {
  if (cols % 256 != 0) return false;
  const int64_t ntasks = 4 * (cols / 256);
  const int tpl = (int)((ntasks + 63) / 64);
  // a row must fill most of the wave (narrower rows use the lanes-per-row kernels)
  return ntasks >= 48 && tpl <= 2 && !(tpl == 2 && ru > 2) && (ru == 1 || ru == 2 || ru == 4);
}

hipError_t launch_dec_gate_up_tq4(hipStream_t st, const ExpertTier &tier, int64_t rows, int64_t cols,
                                  const Routing &rt, int max_active, const int8_t *xq, const float *xd,
                                  const int32_t *xbs, float *h, int ru, int wg_per_cu_x16, const DecSelect *sel) {
  if (rows <= 0 || max_active <= 0 || !dec_gate_up_tq4_supported(cols, ru)) return hipErrorNotSupported;
  int nper = 0;
  if (sel) {
    if (sel->E > 256 || sel->K > 16 || sel->K > sel->E || sel->K != max_active) return hipErrorNotSupported;
    nper = sel->E <= 64 ? 1 : (sel->E <= 128 ? 2 : 4);
  }
  const int tpl = (int)((4 * (cols / 256) + 63) / 64);
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  DecArgs a{tier, rt, rows, cols, xq, xd, xbs, h, 0, sel ? *sel : DecSelect{}};
  // work-group steps of 4*RU rows per expert, spread evenly: every work-group
  // gets the same number of steps
  const int64_t rows_per_wg = 4LL * ru;
  const int64_t need = (rows + rows_per_wg - 1) / rows_per_wg;
  int64_t cap = (int64_t)cus * wg_per_cu_x16 / 16 / max_active;
  if (cap < 1) cap = 1;
  const int64_t per = (need + cap - 1) / cap;
  const int64_t gx = (need + per - 1) / per;
  a.groups_per_expert = (int32_t)gx;
  const dim3 grid((unsigned)gx, (unsigned)max_active);
#define KMOE_DEC_GU(TPLV, RUV)                                                                      \
  do {                                                                                             \
    if (nper == 0) KMOE_LAUNCH((k_dec_gate_up_tq4<TPLV, RUV, 0>), grid, dim3(256), 0, st, a);      \
    else if (nper == 1) KMOE_LAUNCH((k_dec_gate_up_tq4<TPLV, RUV, 1>), grid, dim3(256), 0, st, a); \
    else if (nper == 2) KMOE_LAUNCH((k_dec_gate_up_tq4<TPLV, RUV, 2>), grid, dim3(256), 0, st, a); \
    else KMOE_LAUNCH((k_dec_gate_up_tq4<TPLV, RUV, 4>), grid, dim3(256), 0, st, a);                \
  } while (0)
  if (tpl == 1) {
    if (ru == 1) KMOE_DEC_GU(1, 1);
    else if (ru == 2) KMOE_DEC_GU(1, 2);
    else KMOE_DEC_GU(1, 4);
  } else {
    if (ru == 1) KMOE_DEC_GU(2, 1);
    else KMOE_DEC_GU(2, 2);
  }
#undef KMOE_DEC_GU
  return hipGetLastError();
}


// ---------------------------------------------------------------------------
// Single-token down projection + combine over tiled Q4_K rows:
//   out[r] = sum over active experts e (ascending) of w_e * (down_e[r] . q8k(h_e))
// (transformer.rs:559-570; the combine multiplies, then adds, from 0).
// One 512-thread work-group per CU. The Q8_K rows of the K active slots are
// staged in LDS once, interleaved so that the 16-byte piece c of lane-slot t
// sits at (c*4*nb + t)*16: lane t reads its 64 activation bytes with four
// conflict-free ds_read_b128, plus its (sum of 32, sum of 32) pair and the
// block scale. Each wave then owns whole rows: TPL quarters per lane cover the
// row's 4*nb quarters, the experts follow one another (the next one's weights
// in flight while the current one is computed) and the combine stays in
// registers, so no work-group barrier is needed after the staging.
namespace {

struct DownArgs {
  ExpertTier tier;
  Routing rt;
  int64_t rows, cols;  // rows = d, cols = F
  const int8_t *hq;
  const float *hd;
  const int32_t *hbs;
  float *out;
  int32_t k;  // active slots (one token)
};

template <int TPL>
__global__ void __launch_bounds__(512) k_dec_down_tq4(DownArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  constexpr int NW = 8;  // waves per work-group
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t F = a.cols, nb = F / 256, nq = 4 * nb;  // quarters per row
  const int K = a.k;
  // LDS per slot: q [4][nq][16] int8, then (bsA, bsB) [nq] int2, then d [nq] float
  const int64_t slot_bytes = 16 * 4 * nq + 12 * nq;
  // lane constants
  uint32_t oh[TPL], oa[TPL], ob[TPL];
  bool tv[TPL];
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const int64_t t0 = lane + 64 * i;
    tv[i] = t0 < nq;
    const int64_t t = tv[i] ? t0 : nq - 1;
    const int64_t sb = t >> 2;
    oh[i] = (uint32_t)(16 * sb);
    oa[i] = (uint32_t)tq4_qs_off(nb, sb, (int)(t & 3), 0);
    ob[i] = oa[i] + (uint32_t)tq4_j_stride(nb, sb);
  }
  const int kq = lane & 3;
  const int64_t row_bytes = nb * 144;
  const int64_t nw = (int64_t)gridDim.x * NW;
  const int64_t r_first = (int64_t)blockIdx.x * NW + wave;
  const int64_t my_rows = r_first < a.rows ? (a.rows - 1 - r_first) / nw + 1 : 0;
  const int items = (int)my_rows * K;  // (row j, expert ia) with ia fastest, experts ascending
  auto row_ptr = [&](int it) {
    const int64_t r = r_first + (int64_t)(it / K) * nw;
    const int e = a.rt.active[it % K];
    return a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[2] + r * row_bytes;
  };
  u32x4 hA[TPL], qaA[TPL], qbA[TPL], hB[TPL], qaB[TPL], qbB[TPL];
  auto load = [&](int it, u32x4 (&h)[TPL], u32x4 (&qa)[TPL], u32x4 (&qb)[TPL]) {
    const uint8_t *row = row_ptr(it < items ? it : items - 1);
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      h[i] = __builtin_nontemporal_load((const u32x4 *)(row + oh[i]));
      qa[i] = __builtin_nontemporal_load((const u32x4 *)(row + oa[i]));
      qb[i] = __builtin_nontemporal_load((const u32x4 *)(row + ob[i]));
    }
  };
  // Prologue: stage the activation rows with all their loads in flight at
  // once (one round trip), then the first two items' weights.
  constexpr int SP = 4, SQ = 2;  // row pieces and (slot, quarter) pairs per thread (named below)
  const int P = (int)(F / 16), NQ = (int)nq;  // pieces per row, quarters per row (32-bit index math)
  const int npieces = K * P, npairs = K * NQ;
  const uint32_t sb_bytes = (uint32_t)slot_bytes, dummy = (uint32_t)K * sb_bytes;
  uint32_t pdst[SP], bdst[SQ], ddst[SQ];
  int psrc[SP], bsrc[SQ], dsrc[SQ];
#pragma unroll
  for (int j = 0; j < SP; ++j) {  // addresses first, all loads next, then the LDS writes
    const int c16 = tid + j * 64 * NW;
    const int ia = c16 / P, i = (c16 - ia * P) * 16;
    const int t = 4 * (i >> 8) + ((i >> 6) & 3), c = (i >> 4) & 3;
    const bool ok = c16 < npieces;
    psrc[j] = ok ? c16 : npieces - 1;
    pdst[j] = ok ? (uint32_t)ia * sb_bytes + (uint32_t)(c * NQ + t) * 16 : dummy;
  }
#pragma unroll
  for (int j = 0; j < SQ; ++j) {
    const int u = tid + j * 64 * NW;
    const bool ok = u < npairs;
    const int uc = ok ? u : npairs - 1;
    const int ia = uc / NQ, t = uc - ia * NQ;
    bsrc[j] = ia * P + 4 * t;  // int32 index into hbs (F/16 sums per slot)
    dsrc[j] = ia * (int)nb + (t >> 2);
    bdst[j] = ok ? (uint32_t)ia * sb_bytes + (uint32_t)(64 * NQ + 8 * t) : dummy;
    ddst[j] = ok ? (uint32_t)ia * sb_bytes + (uint32_t)(72 * NQ + 4 * t) : dummy + 8;
  }
  // named registers (not arrays) keep the staged values out of scratch
  const int4 p0 = *(const int4 *)(a.hq + (int64_t)psrc[0] * 16);
  const int4 p1 = *(const int4 *)(a.hq + (int64_t)psrc[1] * 16);
  const int4 p2 = *(const int4 *)(a.hq + (int64_t)psrc[2] * 16);
  const int4 p3 = *(const int4 *)(a.hq + (int64_t)psrc[3] * 16);
  const int4 b0 = *(const int4 *)(a.hbs + bsrc[0]);
  const int4 b1 = *(const int4 *)(a.hbs + bsrc[1]);
  const float d0 = a.hd[dsrc[0]], d1 = a.hd[dsrc[1]];
  *(int4 *)(lds + pdst[0]) = p0;
  *(int4 *)(lds + pdst[1]) = p1;
  *(int4 *)(lds + pdst[2]) = p2;
  *(int4 *)(lds + pdst[3]) = p3;
  *(int2 *)(lds + bdst[0]) = make_int2(b0.x + b0.y, b0.z + b0.w);
  *(int2 *)(lds + bdst[1]) = make_int2(b1.x + b1.y, b1.z + b1.w);
  *(float *)(lds + ddst[0]) = d0;
  *(float *)(lds + ddst[1]) = d1;
  // The barrier goes before the weight loads: a wave reaches it only once its
  // loads are accepted, and the memory queue accepts them at HBM speed.
  __syncthreads();
  if (items == 0) return;
  load(0, hA, qaA, qbA);
  if (items > 1) load(1, hB, qaB, qbB);
  auto dot = [&](int it, const u32x4 (&h)[TPL], const u32x4 (&qa)[TPL], const u32x4 (&qb)[TPL]) {
    const uint8_t *L = lds + (it % K) * slot_bytes;
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      const int t = tv[i] ? lane + 64 * i : (int)nq - 1;
      Slice s;
      s.x0 = *(const int4 *)(L + (0 * nq + t) * 16);
      s.x1 = *(const int4 *)(L + (1 * nq + t) * 16);
      s.x2 = *(const int4 *)(L + (2 * nq + t) * 16);
      s.x3 = *(const int4 *)(L + (3 * nq + t) * 16);
      const int2 bs = *(const int2 *)(L + 64 * nq + 8 * t);
      s.bsA = bs.x;
      s.bsB = bs.y;
      s.d = *(const float *)(L + 72 * nq + 4 * t);
      int mins;
      const int sumi = q4k_quarter(h[i], qa[i], qb[i], kq, s, mins);
      const float dw = f16_bits_to_f32(h[i].x) * s.d, mw = f16_bits_to_f32(h[i].x >> 16) * s.d;
      const float v = fmaf(dw, (float)sumi, -(mw * (float)mins));
      acc += tv[i] ? v : 0.0f;
    }
    return group_sum<64>(acc);
  };
  float o = 0.0f;
  auto finish = [&](int it, float y) {  // combine in ascending expert order, store after the last
    const float wgt = a.rt.wsel[a.rt.perm[it % K]];
    const float c = wgt * y;
    o = o + c;
    if (it % K == K - 1) {
      if (lane == 0) a.out[r_first + (int64_t)(it / K) * nw] = o;
      o = 0.0f;
    }
  };
  // ping-pong register sets: item it+1's weights are in flight while item it is computed
  for (int it = 0; it < items; it += 2) {
    if (it > 0) load(it + 1, hB, qaB, qbB);
    finish(it, dot(it, hA, qaA, qbA));
    if (it + 1 >= items) break;
    load(it + 2, hA, qaA, qbA);
    finish(it + 1, dot(it + 1, hB, qaB, qbB));
  }
}

}  // namespace

bool dec_down_tq4_supported(int64_t rows, int64_t cols, int k) {
  if (cols % 256 != 0 || rows <= 0 || k <= 0) return false;
  const int64_t nq = 4 * (cols / 256);
  const int64_t lds = (int64_t)k * (16 * 4 * nq + 12 * nq);
  // the staging holds 4 row pieces and 2 (slot, quarter) pairs per thread of 512
  return nq > 128 && nq <= 256 && lds <= 96 * 1024 && (int64_t)k * (cols / 16) <= 4 * 512 &&
         (int64_t)k * nq <= 2 * 512;
}

hipError_t launch_dec_down_tq4(hipStream_t st, const ExpertTier &tier, int64_t rows, int64_t cols, const Routing &rt,
                               int k, const int8_t *hq, const float *hd, const int32_t *hbs, float *out) {
  if (!dec_down_tq4_supported(rows, cols, k)) return hipErrorNotSupported;
  const int64_t nq = 4 * (cols / 256);
  const size_t lds = (size_t)k * (size_t)(16 * 4 * nq + 12 * nq) + 16;  // + the staging's dummy slot
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  int64_t grid = (rows + 7) / 8;
  if (grid > cus) grid = cus;
  DownArgs a{tier, rt, rows, cols, hq, hd, hbs, out, k};
  const int tpl = (int)((nq + 63) / 64);
#define KMOE_DEC_DN(TPLV)                                                                                   \
  do {                                                                                                     \
    hipError_t e_ = hipFuncSetAttribute((const void *)k_dec_down_tq4<TPLV>,                                \
                                        hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);             \
    if (e_ != hipSuccess) return e_;                                                                       \
    KMOE_LAUNCH((k_dec_down_tq4<TPLV>), dim3((unsigned)grid), dim3(512), lds, st, a);                      \
  } while (0)
  if (tpl == 3) KMOE_DEC_DN(3);
  else KMOE_DEC_DN(4);
#undef KMOE_DEC_DN
  return hipGetLastError();
}

}  // namespace kmoe
