// kmoe_fused.hip — the whole single-token MoE layer (Transformer::moe_ffn,
// transformer.rs:513-570, at one token) in one persistent kernel, for Q4_K
// experts in the tiled tier:
//   route   work-groups 0..E-1: logit e in quant::dot order (quant.rs:208-224),
//           their spare waves quantize x to Q8_K (qdot.rs:347-367);
//   select  every wave: softmax, top-k, renormalisation (transformer.rs:479-495)
//           from the E logits; one wave publishes the routing;
//   gate/up the other work-groups: 8-row steps of one selected expert's gate
//           and up rows, consecutive groups on consecutive steps, SwiGLU
//           (transformer.rs:551-558);
//           the work-group completing a 256-row block of h quantizes it to Q8_K;
//   down    every work-group: its rows of every selected expert's down part,
//           split-K over the four waves, combined in ascending expert id
//           (transformer.rs:559-570). The first two items' weights are loaded
//           before waiting for the quantized h.
// The arithmetic of every phase is the one of the separate kernels (the
// decode router, the selecting gate/up kernel, the slot quantizer and the
// split-K down kernel), so the results are the same bits.
//
// Work-groups wait for each other through counters in device memory (zero
// between calls): the grid is sized so that every work-group is resident. A
// wait is one thread polling with s_sleep, bounded: past the bound it sets a
// sticky flag and the work-group skips the remaining work, so the grid always
// drains (the host reports the flag). The last work-group to leave clears the
// counters for the next call. Everything one work-group hands to another
// (logits, the Q8_K of x, h and its Q8_K, the counters) is written and read
// with agent-scope accesses, which are coherent across the XCDs without
// writing back or invalidating the L2 caches; a counter is raised after the
// work-group barrier, which waits for the work-group's stores to complete.
#include "kmoe_device.h"
#include "kmoe_launch.h"
#include "kmoe_logit.h"
#include "kmoe_select.h"
#include "kmoe_tq4.h"

namespace kmoe {

namespace {

// sync[] words
enum { SY_LOGITS = 0, SY_QUANT = 1, SY_EXIT = 2, SY_TIMEOUT = 3, SY_ROWS = 16 };

constexpr int kSpinMax = 1 << 20;  // polls of up to ~1 us each: about a second at most

struct FusedArgs {
  const float *W;  // router [E, d], F32
  const float *X;  // the token [d]
  int32_t E, K, norm_topk, vec;
  float weights_scale;
  int64_t d, F;
  ExpertTier tier;
  float *logits;                                 // [E]
  int8_t *xq;                                    // Q8_K of x
  float *xd;
  int32_t *xs;
  float *h;                                      // [K, F], slot = rank of the expert among the selection
  int8_t *hq;                                    // Q8_K rows of h
  float *hd;
  int32_t *hs;
  float *out;                                    // [d]
  uint32_t *idx, *perm, *inv, *offsets;          // routing, published for the caller
  float *wsel;
  int32_t *active, *n_active;
  uint32_t *sync;
};

// Thread 0: wait until *c >= target. False past the bound.
__device__ __forceinline__ bool wait_count(const uint32_t *c, uint32_t target) {
  for (int i = 0; i < kSpinMax; ++i) {
    if (ld_agent(c) >= target) return true;
    __builtin_amdgcn_s_sleep(8);
  }
  return false;
}

// DC = 1: d <= 4096 (router rows in 4 float4 registers per thread, one gate/up
// task per lane); DC = 2: d <= 8192. NPER: logits per lane in the selection.
template <int DC, int NPER>
__global__ void __launch_bounds__(256) k_layer_dec(FusedArgs a) {
  constexpr int NV = 4 * DC, TPL = DC, RU = 2, DRU = 4;
  __shared__ __attribute__((aligned(16))) float T[kLogitLds];
  __shared__ float P[4][64 * NPER];
  __shared__ float part[4][64];
  __shared__ float outv[64];
  __shared__ int ok_s, nq_s, last_s;
  __shared__ int qlist[128];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int g = blockIdx.x, G = gridDim.x;
  const int E = a.E, K = a.K;
  const int64_t d = a.d, F = a.F;
  uint32_t *sync = a.sync;
  bool ok = true;

  // ---- route: logit g and this work-group's share of the Q8_K of x
  if (g < E) {
    const float *w = a.W + (int64_t)g * d;
    float4 wv[NV];
    logit_row_load<NV>(w, (int)(d / 4), a.vec, wv, tid);
    const float r = wg_logit<NV>(wv, w, a.X, d, a.vec, T, [&](int wv_) {
      const int64_t nbx = d / 256;
      for (int64_t b = g * 3 + (wv_ - 1); b < nbx; b += 3 * E)
        wave_quant_q8k_block<true>(a.X + b * 256, a.xq + b * 256, a.xd + b, a.xs + b * 16, lane);
    });
    if (tid == 0) st_agent(&a.logits[g], r);
    vm_wait();  // the logit and this group's int8 rows before the count
    __syncthreads();
    if (tid == 0) add_agent(&sync[SY_LOGITS], 1u);
  }
  if (tid == 0) ok_s = wait_count(&sync[SY_LOGITS], (uint32_t)E);
  __syncthreads();
  ok = ok_s;

  // ---- select (every wave; all compute the same)
  uint32_t sj[16], rk[16];
  float wj[16];
  {
    float lv[NPER];
#pragma unroll
    for (int i = 0; i < NPER; ++i) lv[i] = lane + 64 * i < E ? ld_agent(&a.logits[lane + 64 * i]) : -INFINITY;
    wave_route_one<NPER>(lv, E, K, a.norm_topk, a.weights_scale, P[wave], sj, wj);
    selection_ranks(sj, K, rk);
    if (g == 0 && wave == 0)
      publish_selection(sj, wj, rk, K, E, lane, a.idx, a.wsel, a.perm, a.inv, a.active, a.n_active, a.offsets);
  }
  auto slot_expert = [&](int i, float *wgt) {  // the expert of slot i (ascending id) and its weight
    int e = 0;
    float ww = 0.0f;
    for (int j = 0; j < K; ++j) {
      e = (int)rk[j] == i ? (int)sj[j] : e;
      ww = (int)rk[j] == i ? wj[j] : ww;
    }
    if (wgt) *wgt = ww;
    return e;
  };

  const int64_t nbd = d / 256, nbf = F / 256;
  // ---- gate/up + SwiGLU on the work-groups past the router's
  if (ok && g >= E) {
    const int q = g - E, GW = G - E;
    const int slot = q % K, m = q / K;
    const int Q = (GW - slot + K - 1) / K;  // work-groups of this slot
    const int64_t NS = F / (4 * RU);        // 8-row steps of the slot: m, m + Q, m + 2Q, ...
    const int e = slot_expert(slot, nullptr);
    const int64_t ntasks = 4 * nbd, row_bytes = nbd * 144;
    const uint8_t *Gw = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[0];
    const uint8_t *Uw = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[1];
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
      oa[i] = (uint32_t)tq4_qs_off(nbd, sb, k, 0);
      ob[i] = oa[i] + (uint32_t)tq4_j_stride(nbd, sb);
      const int8_t *xv = a.xq + 256 * sb + 64 * k;
      s[i].x0 = ld_agent4(xv);
      s[i].x1 = ld_agent4(xv + 16);
      s[i].x2 = ld_agent4(xv + 32);
      s[i].x3 = ld_agent4(xv + 48);
      const int4 bs = ld_agent4(a.xs + 16 * sb + 4 * k);
      s[i].bsA = bs.x + bs.y;
      s[i].bsB = bs.z + bs.w;
      s[i].d = ld_agent(&a.xd[sb]);
    }
    const int kq = lane & 3;
    for (int64_t j = m; j < NS; j += Q) {
      const int64_t r0 = (j * 4 + wave) * RU;
      u32x4 hg[RU][TPL], ag[RU][TPL], bg[RU][TPL], hu[RU][TPL], au[RU][TPL], bu[RU][TPL];
#pragma unroll
      for (int u = 0; u < RU; ++u) {
        const uint8_t *gr = Gw + (r0 + u) * row_bytes;
        const uint8_t *ur = Uw + (r0 + u) * row_bytes;
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
      if (lane < RU) {  // SwiGLU: g / (1 + exp(-g)) * u
        const float den = 1.0f + expf_cr(-gsum);
        const float qv = gsum / den;
        st_agent(&a.h[slot * F + r0 + lane], qv * usum);
      }
    }
    // each step wrote rows [8j, 8j+8) of the slot: count them per 256-row
    // block; the work-group completing a block quantizes it
    if (tid == 0) nq_s = 0;
    vm_wait();  // the h rows before their counts
    __syncthreads();
    if (wave == 0) {  // one lane per step: the counter updates travel together
      for (int64_t j = m + (int64_t)lane * Q; j < NS; j += 64 * (int64_t)Q) {
        const int64_t sb = (8 * j) / 256;
        const uint32_t prev = add_agent(&sync[SY_ROWS + slot * nbf + sb], 8u);
        if (prev + 8u == 256u) {
          const int n = atomicAdd(&nq_s, 1);
          if (n < 128) qlist[n] = (int)sb;
        }
      }
    }
    __syncthreads();
    const int nq = nq_s < 128 ? nq_s : 128;
    if (nq > 0) {
      for (int i = wave; i < nq; i += 4) {
        const int64_t b = (int64_t)slot * nbf + qlist[i];
        wave_quant_q8k_block<true>(a.h + b * 256, a.hq + b * 256, a.hd + b, a.hs + b * 16, lane);
      }
      vm_wait();  // the quantized blocks before their count
      __syncthreads();
      if (tid == 0) add_agent(&sync[SY_QUANT], (uint32_t)nq);
    }
  }

  // ---- down + combine: rows [g*rb, g*rb + nr) of every selected expert
  {
    const int64_t rb = (d + G - 1) / G;
    const int64_t r0 = (int64_t)g * rb;
    const int nr = (int)(d - r0 < rb ? d - r0 : rb);
    const int64_t ntasks = 4 * nbf, row_bytes = nbf * 144, xs_stride = F / 16;
    const int tpw = (int)((ntasks + 3) / 4);  // tasks per wave
    const int tk = wave * tpw + lane;
    const bool tvd = lane < tpw && tk < ntasks;
    const int tc = tvd ? tk : (int)ntasks - 1;
    const int64_t sbt = tc >> 2;
    const int kt = tc & 3;
    const uint32_t doh = (uint32_t)(16 * sbt), doa = (uint32_t)tq4_qs_off(nbf, sbt, kt, 0);
    const uint32_t dob = doa + (uint32_t)tq4_j_stride(nbf, sbt);
    const int nbt = nr > 0 ? (nr + DRU - 1) / DRU : 0;  // row batches per expert
    const int items = K * nbt;                          // (slot, batch), slots ascending
    if (tid < 64) outv[tid] = 0.0f;
    auto load_w = [&](int it, u32x4 (&h)[DRU], u32x4 (&qa)[DRU], u32x4 (&qb)[DRU]) {
      const int i = it / nbt;
      const int e = slot_expert(i, nullptr);
      const uint8_t *Wd = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[2];
      const int rr = (it - i * nbt) * DRU;
#pragma unroll
      for (int u = 0; u < DRU; ++u) {
        const uint8_t *row = Wd + (r0 + min(rr + u, nr - 1)) * row_bytes;
        h[u] = __builtin_nontemporal_load((const u32x4 *)(row + doh));
        qa[u] = __builtin_nontemporal_load((const u32x4 *)(row + doa));
        qb[u] = __builtin_nontemporal_load((const u32x4 *)(row + dob));
      }
    };
    auto load_act = [&](int i, Slice &sl) {
      const int8_t *v = a.hq + (int64_t)i * F + 256 * sbt + 64 * kt;
      sl.x0 = ld_agent4(v);
      sl.x1 = ld_agent4(v + 16);
      sl.x2 = ld_agent4(v + 32);
      sl.x3 = ld_agent4(v + 48);
      const int4 bs = ld_agent4(a.hs + (int64_t)i * xs_stride + 16 * sbt + 4 * kt);
      sl.bsA = bs.x + bs.y;
      sl.bsB = bs.z + bs.w;
      sl.d = ld_agent(&a.hd[(int64_t)i * nbf + sbt]);
    };
    auto compute = [&](int it, const u32x4 (&h)[DRU], const u32x4 (&qa)[DRU], const u32x4 (&qb)[DRU],
                       const Slice &sl) {
      const int i = it / nbt;
      const int rr = (it - i * nbt) * DRU;
      const bool lastb = (it + 1) % nbt == 0;  // this slot's last row batch
      float acc[DRU];
#pragma unroll
      for (int u = 0; u < DRU; ++u) {
        int mins;
        const int sumi = q4k_quarter(h[u], qa[u], qb[u], kt, sl, mins);
        const float dd = f16_bits_to_f32(h[u].x), dm = f16_bits_to_f32(h[u].x >> 16);
        float v = fmaf(dd * sl.d, (float)sumi, 0.0f);
        v = fmaf(-(dm * sl.d), (float)mins, v);
        acc[u] = tvd ? v : 0.0f;
        acc[u] = group_sum<64>(acc[u]);
      }
      if (lane == 0) {
#pragma unroll
        for (int u = 0; u < DRU; ++u)
          if (rr + u < nr) part[wave][rr + u] = acc[u];
      }
      if (lastb) {
        float wgt;
        (void)slot_expert(i, &wgt);
        lds_barrier();
        if (tid < nr) {
          const float y = ((part[0][tid] + part[1][tid]) + part[2][tid]) + part[3][tid];
          const float c = wgt * y;
          outv[tid] = outv[tid] + c;
        }
        lds_barrier();
      }
    };
    u32x4 hA[DRU], qaA[DRU], qbA[DRU], hB[DRU], qaB[DRU], qbB[DRU];
    if (items > 0) load_w(0, hA, qaA, qbA);
    if (items > 1) load_w(1, hB, qaB, qbB);
    if (tid == 0) ok_s = ok && wait_count(&sync[SY_QUANT], (uint32_t)(K * nbf));
    __syncthreads();
    ok = ok_s;
    if (ok && items > 0) {
      Slice sl;
      int cur_slot = -1;
      for (int it = 0; it < items; it += 2) {
        int i = it / nbt;
        if (i != cur_slot) {
          load_act(i, sl);
          cur_slot = i;
        }
        compute(it, hA, qaA, qbA, sl);
        if (it + 2 < items) load_w(it + 2, hA, qaA, qbA);
        if (it + 1 < items) {
          i = (it + 1) / nbt;
          if (i != cur_slot) {
            load_act(i, sl);
            cur_slot = i;
          }
          compute(it + 1, hB, qaB, qbB, sl);
          if (it + 3 < items) load_w(it + 3, hB, qaB, qbB);
        }
      }
      if (tid < nr) a.out[r0 + tid] = outv[tid];
    }
  }

  // ---- leave; the last work-group clears the counters
  vm_wait();
  __syncthreads();
  if (tid == 0) {
    if (!ok) st_agent(&sync[SY_TIMEOUT], 1u);
    last_s = add_agent(&sync[SY_EXIT], 1u) == (uint32_t)(G - 1);
  }
  __syncthreads();
  if (last_s) {
    const int nrows = K * (int)nbf;
    for (int i = tid; i < nrows; i += 256) st_agent(&sync[SY_ROWS + i], 0u);
    if (tid == 0) {
      st_agent(&sync[SY_LOGITS], 0u);
      st_agent(&sync[SY_QUANT], 0u);
      st_agent(&sync[SY_EXIT], 0u);
    }
  }
}

template <int DC, int NPER>
int fused_grid() {
  static const int v = [] {
    int dev = 0, cus = 0, occ = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, k_layer_dec<DC, NPER>, 256, 0) != hipSuccess) return 0;
    return cus * (occ < 2 ? occ : 2);
  }();
  return v;
}

}  // namespace

bool layer_dec_fused_supported(int64_t d, int64_t F, int32_t E, int32_t K) {
  return d % 256 == 0 && F % 256 == 0 && d >= 1024 && d <= 8192 && F >= 8192 && F <= 16384 && E >= 1 &&
         E <= 256 && K >= 1 && K <= 16 && K <= E && (int64_t)K * (F / 256) <= 4000;
}

hipError_t launch_layer_dec_fused(hipStream_t st, const float *router, int32_t E, int64_t d, const float *x, int32_t K,
                                  int32_t norm_topk, float weights_scale, const ExpertTier &tier, int64_t F,
                                  float *logits, int8_t *xq, float *xd, int32_t *xs, float *h, int8_t *hq, float *hd,
                                  int32_t *hs, float *out, const DecSelect &pub, uint32_t *sync) {
  if (!layer_dec_fused_supported(d, F, E, K)) return hipErrorNotSupported;
  FusedArgs a{};
  a.W = router;
  a.X = x;
  a.E = E;
  a.K = K;
  a.norm_topk = norm_topk;
  a.vec = ((uintptr_t)router % 16 == 0 && (uintptr_t)x % 16 == 0 && d % 4 == 0) ? 1 : 0;
  a.weights_scale = weights_scale;
  a.d = d;
  a.F = F;
  a.tier = tier;
  a.logits = logits;
  a.xq = xq;
  a.xd = xd;
  a.xs = xs;
  a.h = h;
  a.hq = hq;
  a.hd = hd;
  a.hs = hs;
  a.out = out;
  a.idx = pub.idx;
  a.wsel = pub.wsel;
  a.perm = pub.perm;
  a.inv = pub.inv;
  a.offsets = pub.offsets;
  a.active = pub.active;
  a.n_active = pub.n_active;
  a.sync = sync;
  const int dc = d <= 4096 ? 1 : 2;
  const int nper = E <= 64 ? 1 : (E <= 128 ? 2 : 4);
  int grid = 0;
#define KMOE_FUSED(DCV, NPV)                                                          \
  do {                                                                                \
    grid = fused_grid<DCV, NPV>();                                                    \
    /* every slot gets gate/up work-groups; down rows per group fit the LDS */        \
    if (grid < 2 * E || grid < 64 || (d + grid - 1) / grid > 64 ||                   \
        (F / 8 + (grid - E) / K - 1) / ((grid - E) / K) > 128)                        \
      return hipErrorNotSupported; /* steps per group fit its list of completed blocks */ \
    KMOE_LAUNCH((k_layer_dec<DCV, NPV>), dim3((unsigned)grid), dim3(256), 0, st, a);  \
  } while (0)
  if (dc == 1) {
    if (nper == 1) KMOE_FUSED(1, 1);
    else if (nper == 2) KMOE_FUSED(1, 2);
    else KMOE_FUSED(1, 4);
  } else {
    if (nper == 1) KMOE_FUSED(2, 1);
    else if (nper == 2) KMOE_FUSED(2, 2);
    else KMOE_FUSED(2, 4);
  }
#undef KMOE_FUSED
  return hipGetLastError();
}

}  // namespace kmoe
