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
  BlockDbg dbg;               // DBG: per-superblock integers of gate (0) and up (1)
};

// TPL task slots per lane (a row has 4*nb <= 64*TPL quarters), RU rows per step.
// NPER = 0: the routing (active experts, slot offsets) is given. NPER > 0:
// every wave selects the token's experts from its E <= 64*NPER logits itself
// (softmax, top-k, renormalisation), work-group (0, 0) publishes the routing
// (idx, weights, permutation, offsets, active list), and the work-groups of
// grid row y take the y-th smallest selected expert, whose slot is y.
// DBG: the per-superblock integers are also added into a.dbg.
template <int TPL, int RU, int NPER, bool DBG>
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
    uint32_t sl;
    float wl;
    wave_route_one<NPER>(lv, q.E, q.K, q.norm_topk, q.weights_scale, P[wave], sl, wl);
    const uint32_t rk = selection_rank(sl, q.K);
    e = selection_in_slot(sl, rk, q.K, slot_i);
    if (blockIdx.x == 0 && blockIdx.y == 0 && wave == 0)  // publish the routing of the token
      publish_selection(sl, wl, rk, q.K, q.E, lane, q.idx, q.wsel, q.perm, q.inv, q.active, q.n_active, q.offsets);
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
        if constexpr (DBG) {
          if (tv[i] && r0 + u < rows) {
            const int64_t o = (p * rows + r0 + u) * nb + ((lane + 64 * i) >> 2);
            dbg_add(a.dbg.s[0], o, sg);
            dbg_add(a.dbg.m[0], o, mg);
            dbg_add(a.dbg.s[1], o, su);
            dbg_add(a.dbg.m[1], o, mu);
          }
        }
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
  int32_t add;     // out[r] = out[r] + scale * y (AddEpi) instead of out[r] = y
  const float *add_logit;
  const float *xf;  // FX kernels: the f32 row, quantized to Q8_K inside the kernel
};

typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));

// FX: the f32 activation row is quantized to Q8_K inside the kernel instead
// of by a kernel before it (Q8KRow::quantize, qdot.rs:347-367, the same
// arithmetic as k_quant_q8k). Every work-group quantizes the whole row into
// LDS: thread t loads float4 t + 256*i (block wave + 4i, four values per
// lane), those loads issued before the first row step's weight loads, so the
// quantization runs while the weights are in flight.
constexpr int kFxMaxBlocks = 64;  // Q8_K blocks of the row (cols <= 16384)

template <bool TILED, int TPL, int RU, bool FX>
__global__ void __launch_bounds__(256) k_dec_rows(RowsArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nb = a.cols / 256, ntasks = 4 * nb;
  const int64_t row_bytes = nb * 144;
  constexpr int XB = FX ? 4 * TPL : 1;  // FX: blocks per wave (nb <= 16 * TPL)
  __shared__ __attribute__((aligned(16))) int8_t fq[FX ? kFxMaxBlocks * 256 : 16];
  __shared__ float fd[FX ? kFxMaxBlocks : 1];
  __shared__ __attribute__((aligned(16))) int32_t fbs[FX ? kFxMaxBlocks * 16 : 4];
  float4 xv4[XB];
  if constexpr (FX) {
#pragma unroll
    for (int i = 0; i < XB; ++i) {  // block wave + 4i (clamped to the last; only blocks < nb are kept)
      const int64_t b = wave + 4 * i < nb ? wave + 4 * i : nb - 1;
      xv4[i] = *(const float4 *)(a.xf + 256 * b + 4 * lane);
    }
  }
  uint32_t oh[TPL], oa[TPL], ob[TPL];
  bool tv[TPL];
  int64_t tsb[TPL];
  int tk[TPL];
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const int64_t t0 = lane + 64 * i;
    tv[i] = t0 < ntasks;
    const int64_t t = tv[i] ? t0 : ntasks - 1;
    const int64_t sb = t >> 2;
    const int k = (int)(t & 3);
    tsb[i] = sb;
    tk[i] = k;
    if constexpr (TILED) {
      oh[i] = (uint32_t)(16 * sb);
      oa[i] = (uint32_t)tq4_qs_off(nb, sb, k, 0);
      ob[i] = oa[i] + (uint32_t)tq4_j_stride(nb, sb);
    } else {
      oh[i] = (uint32_t)(144 * sb);
      oa[i] = oh[i] + 16 + 32 * k;
      ob[i] = oa[i] + 16;
    }
  }
  Slice s[TPL];
  auto slices = [&](const int8_t *xq, const float *xd, const int32_t *xbs) {
#pragma unroll
    for (int i = 0; i < TPL; ++i) {
      const int4 *xv = (const int4 *)(xq + 256 * tsb[i] + 64 * tk[i]);
      s[i].x0 = xv[0];
      s[i].x1 = xv[1];
      s[i].x2 = xv[2];
      s[i].x3 = xv[3];
      const int4 bs = *(const int4 *)(xbs + 16 * tsb[i] + 4 * tk[i]);
      s[i].bsA = bs.x + bs.y;
      s[i].bsB = bs.z + bs.w;
      s[i].d = xd[tsb[i]];
    }
  };
  if constexpr (!FX) slices(a.xq, a.xd, a.xbs);
  const int kq = lane & 3;
  const int64_t rows = a.rows;
  float add_scale = 1.0f;  // the shared expert's gate (k_shared_add's arithmetic)
  if (a.add && a.add_logit) {
    const float den = 1.0f + expf_cr(-*a.add_logit);
    add_scale = 1.0f / den;
  }
  auto load = [&](int64_t r0, u32x4 (&hw)[RU][TPL], u32x4 (&aw)[RU][TPL], u32x4 (&bw)[RU][TPL]) {
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
  };
  auto reduce_store = [&](int64_t r0, const u32x4 (&hw)[RU][TPL], const u32x4 (&aw)[RU][TPL],
                          const u32x4 (&bw)[RU][TPL]) {
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
    if (lane < RU && r0 + lane < rows) {
      if (a.add) {
        const float p = add_scale * res;
        a.out[r0 + lane] = a.out[r0 + lane] + p;
      } else {
        a.out[r0 + lane] = res;
      }
    }
  };
  const int64_t stride = (int64_t)a.groups * 4 * RU;
  int64_t r0 = ((int64_t)blockIdx.x * 4 + wave) * RU;
  if constexpr (FX) {
    // first row step's weights in flight (rows clamped), then the row's Q8_K
    // blocks into LDS, then the slices from there; every wave takes part
    u32x4 hw[RU][TPL], aw[RU][TPL], bw[RU][TPL];
    load(r0, hw, aw, bw);
#pragma unroll
    for (int i = 0; i < XB; ++i) {
      const int b = wave + 4 * i;
      if (b < nb) wave_quant_q8k_vals(xv4[i], fq + 256 * b, fd + b, fbs + 16 * b, lane);
    }
    __syncthreads();
    slices(fq, fd, fbs);
    if (r0 < rows) reduce_store(r0, hw, aw, bw);
    r0 += stride;
  }
  for (; r0 < rows; r0 += stride) {
    u32x4 hw[RU][TPL], aw[RU][TPL], bw[RU][TPL];
    load(r0, hw, aw, bw);
    reduce_store(r0, hw, aw, bw);
  }
}

}  // namespace

bool dec_rows_supported(int64_t cols) {
  if (cols % 256 != 0) return false;
  const int64_t ntasks = 4 * (cols / 256);
  return ntasks >= 48 && ntasks <= 256;
}

hipError_t launch_dec_rows(hipStream_t st, bool tiled, const uint8_t *w, int64_t rows, int64_t cols, const int8_t *xq,
                           const float *xd, const int32_t *xbs, float *out, const AddEpi *epi, const float *xf) {
  if (rows <= 0) return hipSuccess;
  if (!dec_rows_supported(cols) || ((uintptr_t)w & 3u) || (tiled && ((uintptr_t)w & 15u)))
    return hipErrorNotSupported;
  if (xf ? (((uintptr_t)xf & 15u) || cols / 256 > kFxMaxBlocks) : (((uintptr_t)xq & 15u) || ((uintptr_t)xbs & 15u)))
    return hipErrorNotSupported;
  const int tpl = (int)((4 * (cols / 256) + 63) / 64);
  const int ru = tpl <= 2 ? 2 : 1;
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  RowsArgs a{w, rows, cols, xq, xd, xbs, out, 0, epi ? 1 : 0, epi ? epi->logit : nullptr, xf};
  // work-group steps of 4*RU rows, spread evenly over about two groups per CU
  const int64_t need = (rows + 4 * ru - 1) / (4 * ru);
  const int64_t cap = 2LL * cus;
  const int64_t per = (need + cap - 1) / cap;
  a.groups = (int32_t)((need + per - 1) / per);
  const dim3 grid((unsigned)a.groups);
#define KMOE_DEC_ROWS(TL, FX)                                                                  \
  do {                                                                                         \
    if (tpl == 1) KMOE_LAUNCH((k_dec_rows<TL, 1, 2, FX>), grid, dim3(256), 0, st, a);          \
    else if (tpl == 2) KMOE_LAUNCH((k_dec_rows<TL, 2, 2, FX>), grid, dim3(256), 0, st, a);     \
    else if (tpl == 3) KMOE_LAUNCH((k_dec_rows<TL, 3, 1, FX>), grid, dim3(256), 0, st, a);     \
    else KMOE_LAUNCH((k_dec_rows<TL, 4, 1, FX>), grid, dim3(256), 0, st, a);                   \
  } while (0)
  if (xf) KMOE_DEC_ROWS(false, true);  // GGUF rows of kmoe_matmul
  else if (tiled) KMOE_DEC_ROWS(true, false);
  else KMOE_DEC_ROWS(false, false);
#undef KMOE_DEC_ROWS
  return hipGetLastError();
}

// Launch shape of the tiled gate/up kernel (measured best on the Mixtral and
// DeepSeek-V2-Lite shapes): 2 rows per wave step, 2 work-groups per CU.
constexpr int kGuRu = 2;
constexpr int kGuWgPerCu = 2;

bool dec_gate_up_tq4_supported(int64_t cols) {
  if (cols % 256 != 0) return false;
  const int64_t ntasks = 4 * (cols / 256);
  const int tpl = (int)((ntasks + 63) / 64);
  // a row must fill most of the wave (narrower rows use the lanes-per-row kernels)
  return ntasks >= 48 && tpl <= 2;
}

hipError_t launch_dec_gate_up_tq4(hipStream_t st, const ExpertTier &tier, int64_t rows, int64_t cols,
                                  const Routing &rt, int max_active, const int8_t *xq, const float *xd,
                                  const int32_t *xbs, float *h, const DecSelect *sel, const BlockDbg *dbg) {
  if (rows <= 0 || max_active <= 0 || !dec_gate_up_tq4_supported(cols)) return hipErrorNotSupported;
  int nper = 0;
  if (sel) {
    if (sel->E > 256 || sel->K > 16 || sel->K > sel->E || sel->K != max_active) return hipErrorNotSupported;
    nper = sel->E <= 64 ? 1 : (sel->E <= 128 ? 2 : 4);
  }
  const int tpl = (int)((4 * (cols / 256) + 63) / 64);
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  DecArgs a{tier, rt, rows, cols, xq, xd, xbs, h, 0, sel ? *sel : DecSelect{}, dbg ? *dbg : BlockDbg{}};
  // work-group steps of 4*RU rows per expert, spread evenly: every work-group
  // gets the same number of steps
  const int64_t rows_per_wg = 4LL * kGuRu;
  const int64_t need = (rows + rows_per_wg - 1) / rows_per_wg;
  int64_t cap = (int64_t)cus * kGuWgPerCu / max_active;
  if (cap < 1) cap = 1;
  const int64_t per = (need + cap - 1) / cap;
  const int64_t gx = (need + per - 1) / per;
  a.groups_per_expert = (int32_t)gx;
  const dim3 grid((unsigned)gx, (unsigned)max_active);
#define KMOE_DEC_GU_D(TPLV, RUV, DB)                                                                    \
  do {                                                                                                 \
    if (nper == 0) KMOE_LAUNCH((k_dec_gate_up_tq4<TPLV, RUV, 0, DB>), grid, dim3(256), 0, st, a);      \
    else if (nper == 1) KMOE_LAUNCH((k_dec_gate_up_tq4<TPLV, RUV, 1, DB>), grid, dim3(256), 0, st, a); \
    else if (nper == 2) KMOE_LAUNCH((k_dec_gate_up_tq4<TPLV, RUV, 2, DB>), grid, dim3(256), 0, st, a); \
    else KMOE_LAUNCH((k_dec_gate_up_tq4<TPLV, RUV, 4, DB>), grid, dim3(256), 0, st, a);                \
  } while (0)
#define KMOE_DEC_GU(TPLV, RUV)                     \
  do {                                             \
    if (dbg) KMOE_DEC_GU_D(TPLV, RUV, true);       \
    else KMOE_DEC_GU_D(TPLV, RUV, false);          \
  } while (0)
  if (tpl == 1) KMOE_DEC_GU(1, kGuRu);
  else KMOE_DEC_GU(2, kGuRu);
#undef KMOE_DEC_GU
#undef KMOE_DEC_GU_D
  return hipGetLastError();
}


}  // namespace kmoe
