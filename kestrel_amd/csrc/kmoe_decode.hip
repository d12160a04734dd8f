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
// task structure of the gate/up kernel above: lane-constant offsets inside a
// row, the activation slice in registers, RU rows per wave step; lane u of
// the wave ends with row r0+u. Rows in GGUF order (head at 144*sb, nibble
// chunk (k, j) at 144*sb + 16 + 32k + 16j; rows need only 4-byte alignment).
struct RowsArgs {
  const uint8_t *W;
  int64_t rows, cols;
  const int8_t *xq;
  const float *xd;
  const int32_t *xbs;
  float *out;
  int32_t groups;  // work-groups striding over the rows
  int32_t per;     // k_dec_rows_co: row steps of every wave (1, or even)
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
constexpr int kFxMaxBlocks = 16;  // Q8_K blocks of the row (cols <= 4096)

// The rows are read with contiguous loads: in the GGUF order a task's three
// 16-byte pieces sit at 144*sb, +16+32k and +32+32k, so a load instruction
// per piece touches 16-byte pieces scattered over its lines (that pattern
// streams at about 4.6 TB/s on MI355X against 6.85 for a linear read). A
// wave step covers RU consecutive rows, one contiguous span of RU*144*nb
// bytes: lane l loads its 16-byte chunks l, l+64, ... (each load instruction
// one contiguous KB), stores them into the wave's own LDS buffer, and reads
// its tasks' head and nibble chunks from there.
template <int TPL, int RU, int NL, bool FX, bool RING = true>
__global__ void __launch_bounds__(256, 2) k_dec_rows_co(RowsArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t nb = a.cols / 256, ntasks = 4 * nb;
  const int64_t row_bytes = nb * 144;
  constexpr int XB = FX ? 4 * TPL : 1;
  __shared__ __attribute__((aligned(16))) uint8_t stg[4][64 * NL * 16];
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
  uint32_t oh[TPL], oa[TPL];
  bool tv[TPL];
  int64_t tsb[TPL];
  int tk[TPL];
#pragma unroll
  for (int i = 0; i < TPL; ++i) {
    const int64_t t0 = lane + 64 * i;
    tv[i] = t0 < ntasks;
    const int64_t t = tv[i] ? t0 : ntasks - 1;
    tsb[i] = t >> 2;
    tk[i] = (int)(t & 3);
    oh[i] = (uint32_t)(144 * tsb[i]);
    oa[i] = oh[i] + 16 + 32 * tk[i];
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
  uint8_t *S = stg[wave];
  // The span of rows r0 .. min(r0 + RU, rows) - 1 into c: chunk indices past
  // the span's end repeat its last chunk (and a step past the last row reads
  // row rows - 1), so every load is unconditional and the compiler's counted
  // waits stay exact; those copies land in unused LDS bytes.
  auto issue = [&](int64_t r0, u32x4 (&c)[NL]) {
    const int64_t rb = r0 < rows ? r0 : rows - 1;
    const int64_t nr = rows - rb < RU ? rows - rb : RU;
    const int last = (int)(nr * row_bytes / 16) - 1;
    const uint8_t *base = a.W + rb * row_bytes;
#pragma unroll
    for (int n = 0; n < NL; ++n) {
      const int ci = lane + 64 * n < last ? lane + 64 * n : last;
      c[n] = __builtin_nontemporal_load((const u32x4a4 *)(base + 16 * ci));
    }
  };
  auto stage = [&](const u32x4 (&c)[NL]) {
#pragma unroll
    for (int n = 0; n < NL; ++n) *(u32x4 *)(S + 16 * (lane + 64 * n)) = c[n];
  };
  auto reduce_store = [&](int64_t r0) {
    float res = 0.0f;  // lane u < RU: row r0+u
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      float acc = 0.0f;
      if (r0 + u < rows) {  // wave-uniform
        const uint8_t *R = S + u * row_bytes;
#pragma unroll
        for (int i = 0; i < TPL; ++i) {
          const u32x4 hw = *(const u32x4 *)(R + oh[i]);
          const u32x4 aw = *(const u32x4 *)(R + oa[i]);
          const u32x4 bw = *(const u32x4 *)(R + oa[i] + 16);
          int m;
          const int si = q4k_quarter(hw, aw, bw, kq, s[i], m);
          const float dd = f16_bits_to_f32(hw.x) * s[i].d, mf = f16_bits_to_f32(hw.x >> 16) * s[i].d;
          const float v = fmaf(dd, (float)si, -(mf * (float)m));
          acc += tv[i] ? v : 0.0f;
        }
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
  auto prologue = [&]() {
    if constexpr (FX) {
      // the row's Q8_K blocks into LDS while the first spans are in flight,
      // then the slices from there; every wave takes part
#pragma unroll
      for (int i = 0; i < XB; ++i) {
        const int b = wave + 4 * i;
        if (b < nb) wave_quant_q8k_vals(xv4[i], fq + 256 * b, fd + b, fbs + 16 * b, lane);
      }
      __syncthreads();
      slices(fq, fd, fbs);
    }
  };
  // The wave's steps r_j = r_first + j * stride, j < a.per (the same count in
  // every wave: 1, or even with RING). With RING and two or more steps, two
  // spans are in flight: the main loop restages and refills both register
  // sets, the last pair is reduced without refills, so no wave ends with
  // loads it does not use. Without RING (the widest rows, whose second set
  // would not fit the registers) one span is in flight.
  const int64_t stride = (int64_t)a.groups * 4 * RU;
  const int64_t r_first = ((int64_t)blockIdx.x * 4 + wave) * RU;
  const int per = a.per;
  u32x4 c0[NL];
  if constexpr (!RING) {
    issue(r_first, c0);
    prologue();
    for (int j = 0; j < per; ++j) {
      stage(c0);
      if (j + 1 < per) issue(r_first + (j + 1) * stride, c0);
      reduce_store(r_first + j * stride);
    }
    return;
  }
  u32x4 c1[NL];
  if (per == 1) {
    issue(r_first, c0);
    prologue();
    stage(c0);
    reduce_store(r_first);
    return;
  }
  issue(r_first, c0);
  issue(r_first + stride, c1);
  prologue();
  for (int j = 0; j < per - 2; j += 2) {
    stage(c0);
    issue(r_first + (j + 2) * stride, c0);
    reduce_store(r_first + j * stride);
    stage(c1);
    issue(r_first + (j + 3) * stride, c1);
    reduce_store(r_first + (j + 1) * stride);
  }
  stage(c0);
  reduce_store(r_first + (per - 2) * stride);
  stage(c1);
  reduce_store(r_first + (per - 1) * stride);
}

}  // namespace

bool dec_rows_supported(int64_t cols) {
  if (cols % 256 != 0) return false;
  const int64_t ntasks = 4 * (cols / 256);
  return ntasks >= 48 && ntasks <= 256;
}

hipError_t launch_dec_rows(hipStream_t st, const uint8_t *w, int64_t rows, int64_t cols, const int8_t *xq,
                           const float *xd, const int32_t *xbs, float *out, const AddEpi *epi, const float *xf) {
  if (rows <= 0) return hipSuccess;
  if (!dec_rows_supported(cols) || ((uintptr_t)w & 3u)) return hipErrorNotSupported;
  if (xf ? (((uintptr_t)xf & 15u) || cols / 256 > 16) : (((uintptr_t)xq & 15u) || ((uintptr_t)xbs & 15u)))
    return hipErrorNotSupported;
  const int64_t nb = cols / 256;
  const int tpl = (int)((4 * nb + 63) / 64);
  int dev = 0, cus = 256;
  if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
  RowsArgs a{w, rows, cols, xq, xd, xbs, out, 0, 0, epi ? 1 : 0, epi ? epi->logit : nullptr, xf};
  // Rows per step: the larger choice (a step's span at most 576 chunks)
  // unless that leaves fewer than two work-groups per CU. Steps spread evenly
  // over at most one work-group per CU (measured best against two and three
  // at 4096x4096, 14336x4096 and 4096x14336); per wave 1 or an even count for
  // the ring kernels.
  const int ru_big = nb <= 16 ? 4 : (nb <= 32 ? 2 : 1);
  int ru = ru_big;
  if (ru_big > 1 && (rows + 4 * ru_big - 1) / (4 * ru_big) < 2LL * cus) ru = ru_big / 2;
  const int64_t need = (rows + 4 * ru - 1) / (4 * ru);
  const int64_t cap = cus;
  int64_t per = (need + cap - 1) / cap;
  if (per > 1 && nb <= 56) per = (per + 1) / 2 * 2;
  a.groups = (int32_t)((need + per - 1) / per);
  a.per = (int32_t)per;
  const dim3 grid((unsigned)a.groups);
#define KMOE_CO(TP, R, N, FX, RING) KMOE_LAUNCH((k_dec_rows_co<TP, R, N, FX, RING>), grid, dim3(256), 0, st, a)
  if (xf) {  // x quantized in the kernel: rows of at most 16 superblocks
    if (ru == 4) KMOE_CO(1, 4, 9, true, true);
    else KMOE_CO(1, 2, 5, true, true);
  } else if (tpl == 1) {
    if (ru == 4) KMOE_CO(1, 4, 9, false, true);
    else KMOE_CO(1, 2, 5, false, true);
  } else if (tpl == 2) {
    if (ru == 2) KMOE_CO(2, 2, 9, false, true);
    else KMOE_CO(2, 1, 5, false, true);
  } else if (tpl == 3) {
    KMOE_CO(3, 1, 7, false, true);
  } else if (nb <= 56) {
    KMOE_CO(4, 1, 8, false, true);
  } else {  // two spans of 64-superblock rows do not fit the registers
    KMOE_CO(4, 1, 9, false, false);
  }
#undef KMOE_CO
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
