// kmoe_small.hip — grouped expert products for experts that hold a few token
// rows (decode batches of 2..8 tokens: 1..4 rows per expert), over the tiled Q4_K rows of
// the expert tier, on the int path (transformer.rs:544-565 with
// quant::matmul's int8 activations, quant.rs:262-281; dot_q4_k_8k,
// avx2.rs:351-379).
//
// The single-token decode kernels' structure, widened to NT tokens: every lane
// owns one quarter-superblock task of a row and keeps the Q8_K slices of that
// task for all of the expert's token rows in registers (21 registers per
// token), so each weight byte is read once from HBM and used for every token.
// Per task and row the Q4_K scales and nibbles are unpacked once; only the
// int8 dot products (v_dot4_i32_i8) repeat per token. Work-groups exit unless
// their expert has 1..NT rows on the int path; larger experts take the
// matrix-core or LDS-staged kernels.
//
// k_small_gate_up: one wave per row step (RU rows of gate and up), lanes over
// the row's tasks (4*nb <= 64*TPL). h[p, r] = SwiGLU(gate_r . x_p, up_r . x_p)
// (transformer.rs:558).
// k_small_down: split-K, the four waves of a work-group take a quarter of the
// tasks each, rows in batches of RU; the wave partials meet in LDS.
// y[p, r] = down_r . q8k(h_p).
#include "kmoe_device.h"
#include "kmoe_launch.h"
#include "kmoe_tq4.h"

namespace kmoe {

namespace {

struct SmallArgs {
  ExpertTier tier;
  Routing rt;
  int64_t rows, cols;  // weight rows and columns of one part
  const int8_t *xq;    // int8 activation rows: x [S, cols] (gate/up) or h [slots, cols] (down)
  const float *xd;
  const int32_t *xbs;
  float *out;          // h [slots, rows] (gate/up) or y [slots, rows] (down)
  int regime;
  int32_t groups;      // gate/up: work-groups along one expert's rows
  int32_t rb;          // down: rows per work-group
  BlockDbg dbg;        // DBG kernels: per-superblock integers (gate/down 0, up 1)
};

__device__ __forceinline__ bool small_int_regime(int regime, int n) {
  return regime == REGIME_INT8 || (regime == REGIME_AVX2 && n < 4);
}

// Q4_K scales and nibbles of one task, unpacked once for all tokens.
struct TaskW {
  uint32_t lo[8], hi[8];  // nibbles of sub-block 2k (lo) and 2k+1 (hi), 4 per dword
  int sA, mA, sB, mB;
  float d, dmin;
};
__device__ __forceinline__ TaskW unpack_task(const u32x4 &hd, const u32x4 &qa, const u32x4 &qb, int k) {
  TaskW w;
  q4k_scale_min_pair(hd.y, hd.z, hd.w, k, w.sA, w.mA, w.sB, w.mB);
  const uint32_t m = 0x0f0f0f0fu;
  const uint32_t q[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    w.lo[i] = q[i] & m;
    w.hi[i] = (q[i] >> 4) & m;
  }
  w.d = f16_bits_to_f32(hd.x);
  w.dmin = f16_bits_to_f32(hd.x >> 16);
  return w;
}
// (d*xd) * sumi - (dmin*xd) * mins of one task against one token's slice;
// with ds non-null, sumi and mins are also added at ds[o] and dm[o].
__device__ __forceinline__ float task_value(const TaskW &w, const Slice &s, int32_t *ds = nullptr,
                                            int32_t *dm = nullptr, int64_t o = 0) {
  const int X[16] = {s.x0.x, s.x0.y, s.x0.z, s.x0.w, s.x1.x, s.x1.y, s.x1.z, s.x1.w,
                     s.x2.x, s.x2.y, s.x2.z, s.x2.w, s.x3.x, s.x3.y, s.x3.z, s.x3.w};
  int lo = 0, hi = 0;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    lo = sdot4(w.lo[i], (uint32_t)X[i], lo);
    hi = sdot4(w.hi[i], (uint32_t)X[8 + i], hi);
  }
  const int sumi = w.sA * lo + w.sB * hi;
  const int mins = w.mA * s.bsA + w.mB * s.bsB;
  if (ds) {
    atomicAdd(ds + o, sumi);
    atomicAdd(dm + o, mins);
  }
  return fmaf(w.d * s.d, (float)sumi, -((w.dmin * s.d) * (float)mins));
}

__device__ __forceinline__ void load_slice(Slice &s, const int8_t *xq, const float *xd, const int32_t *xbs,
                                           int64_t cols, int64_t row, int64_t sb, int k) {
  const int4 *v = (const int4 *)(xq + row * cols + 256 * sb + 64 * k);
  s.x0 = v[0];
  s.x1 = v[1];
  s.x2 = v[2];
  s.x3 = v[3];
  const int4 b = *(const int4 *)(xbs + row * (cols / 16) + 16 * sb + 4 * k);
  s.bsA = b.x + b.y;
  s.bsB = b.z + b.w;
  s.d = xd[row * (cols / 256) + sb];
}

template <int TPL, int NT, int RU, bool DBG>
__global__ void __launch_bounds__(256) k_small_gate_up(SmallArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = blockIdx.y;
  if (i >= *a.rt.n_active) return;
  const int e = a.rt.active[i];
  const int64_t p0 = a.rt.offsets[e];
  const int n = (int)(a.rt.offsets[e + 1] - p0);
  if (n < 1 || n > NT || !small_int_regime(a.regime, n)) return;
  const int64_t cols = a.cols, rows = a.rows;
  const int64_t nb = cols / 256, ntasks = 4 * nb, row_bytes = nb * 144;
  const uint8_t *G = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[0];
  const uint8_t *U = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[1];

  uint32_t oh[TPL], oa[TPL], ob[TPL];
  bool tv[TPL];
  Slice s[TPL][NT];
#pragma unroll
  for (int t = 0; t < TPL; ++t) {
    const int64_t t0 = lane + 64 * t;
    tv[t] = t0 < ntasks;
    const int64_t tk = tv[t] ? t0 : ntasks - 1;
    const int64_t sb = tk >> 2;
    const int k = (int)(tk & 3);
    oh[t] = (uint32_t)(16 * sb);
    oa[t] = (uint32_t)tq4_qs_off(nb, sb, k, 0);
    ob[t] = oa[t] + (uint32_t)tq4_j_stride(nb, sb);
#pragma unroll
    for (int j = 0; j < NT; ++j) {
      const int jj = j < n ? j : n - 1;  // rows past n repeat the last (their sums are not stored)
      load_slice(s[t][j], a.xq, a.xd, a.xbs, cols, a.rt.perm[p0 + jj] / a.rt.topk, sb, k);
    }
  }
  const int kq = lane & 3;

  // One task per lane: two register sets, the next step's rows load while
  // this step's are multiplied. Every load is unconditional (steps past the
  // last row reload the last row, never stored), so the compiler's wait
  // counts stay exact. Two tasks per lane keep one set (two would not leave
  // two waves per SIMD).
  struct WSet {
    u32x4 hg[RU][TPL], ag[RU][TPL], bg[RU][TPL], hu[RU][TPL], au[RU][TPL], bu[RU][TPL];
  };
  auto load = [&](int64_t r0, WSet &w) {
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int64_t r = r0 + u < rows ? r0 + u : rows - 1;
      const uint8_t *gr = G + r * row_bytes;
      const uint8_t *ur = U + r * row_bytes;
#pragma unroll
      for (int t = 0; t < TPL; ++t) {
        w.hg[u][t] = __builtin_nontemporal_load((const u32x4 *)(gr + oh[t]));
        w.ag[u][t] = __builtin_nontemporal_load((const u32x4 *)(gr + oa[t]));
        w.bg[u][t] = __builtin_nontemporal_load((const u32x4 *)(gr + ob[t]));
        w.hu[u][t] = __builtin_nontemporal_load((const u32x4 *)(ur + oh[t]));
        w.au[u][t] = __builtin_nontemporal_load((const u32x4 *)(ur + oa[t]));
        w.bu[u][t] = __builtin_nontemporal_load((const u32x4 *)(ur + ob[t]));
      }
    }
  };
  auto step = [&](int64_t r0, const WSet &w) {
    float gsum = 0.0f, usum = 0.0f;  // lane u*NT + j: row r0+u, token j
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      float gacc[NT], uacc[NT];
#pragma unroll
      for (int j = 0; j < NT; ++j) gacc[j] = uacc[j] = 0.0f;
#pragma unroll
      for (int t = 0; t < TPL; ++t) {
        const TaskW wg = unpack_task(w.hg[u][t], w.ag[u][t], w.bg[u][t], kq);
        const TaskW wu = unpack_task(w.hu[u][t], w.au[u][t], w.bu[u][t], kq);
#pragma unroll
        for (int j = 0; j < NT; ++j) {
          if (j < n) {  // uniform: the expert's row count
            float vg, vu;
            if constexpr (DBG) {
              const bool on = tv[t] && r0 + u < rows;
              const int64_t o = ((p0 + j) * rows + r0 + u) * nb + ((lane + 64 * t) >> 2);
              vg = task_value(wg, s[t][j], on ? a.dbg.s[0] : nullptr, a.dbg.m[0], o);
              vu = task_value(wu, s[t][j], on ? a.dbg.s[1] : nullptr, a.dbg.m[1], o);
            } else {
              vg = task_value(wg, s[t][j]);
              vu = task_value(wu, s[t][j]);
            }
            gacc[j] += tv[t] ? vg : 0.0f;
            uacc[j] += tv[t] ? vu : 0.0f;
          }
        }
      }
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (j < n) {
          const float g = group_sum<64>(gacc[j]), v = group_sum<64>(uacc[j]);
          gsum = lane == u * NT + j ? g : gsum;
          usum = lane == u * NT + j ? v : usum;
        }
      }
    }
    const int u = lane / NT, j = lane % NT;
    if (lane < RU * NT && j < n && r0 + u < rows) {  // SwiGLU: g / (1 + exp(-g)) * u
      const float den = 1.0f + expf_cr(-gsum);
      const float q = gsum / den;
      a.out[(p0 + j) * rows + r0 + u] = q * usum;
    }
  };
  const int64_t stride = (int64_t)a.groups * 4 * RU;
  int64_t r0 = ((int64_t)blockIdx.x * 4 + wave) * RU;
  if constexpr (TPL == 1) {
    WSet w0, w1;
    load(r0, w0);
    while (r0 < rows) {
      load(r0 + stride, w1);
      step(r0, w0);
      r0 += stride;
      if (r0 >= rows) break;
      load(r0 + stride, w0);
      step(r0, w1);
      r0 += stride;
    }
  } else {
    for (; r0 < rows; r0 += stride) {
      WSet w;
      load(r0, w);
      step(r0, w);
    }
  }
}

constexpr int kSmallRbMax = 32;
constexpr int kSmallBatchMax = 8;  // batches (tokens) up to this size use these kernels

template <int NT, int RU, bool DBG>
__global__ void __launch_bounds__(256) k_small_down(SmallArgs a) {
  __shared__ float part[4][kSmallRbMax][NT];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int i = blockIdx.y;
  if (i >= *a.rt.n_active) return;
  const int e = a.rt.active[i];
  const int64_t p0 = a.rt.offsets[e];
  const int n = (int)(a.rt.offsets[e + 1] - p0);
  if (n < 1 || n > NT || !small_int_regime(a.regime, n)) return;
  const int64_t cols = a.cols, rows = a.rows;
  const int64_t nb = cols / 256, ntasks = 4 * nb, row_bytes = nb * 144;
  const int64_t r0 = (int64_t)blockIdx.x * a.rb;
  const int nr = (int)(rows - r0 < a.rb ? rows - r0 : a.rb);
  if (nr <= 0) return;
  const uint8_t *W = a.tier.base + (int64_t)e * a.tier.stride + a.tier.off[2];

  // this wave's task: one of a quarter of the row's tasks
  const int64_t tpw = (ntasks + 3) / 4;
  const int64_t t0 = wave * tpw + lane;
  const bool tv = lane < tpw && t0 < ntasks;
  const int64_t tk = tv ? t0 : ntasks - 1;
  const int64_t sb = tk >> 2;
  const int k = (int)(tk & 3);
  const uint32_t oh = (uint32_t)(16 * sb), oa = (uint32_t)tq4_qs_off(nb, sb, k, 0);
  const uint32_t ob = oa + (uint32_t)tq4_j_stride(nb, sb);
  Slice s[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) load_slice(s[j], a.xq, a.xd, a.xbs, cols, p0 + (j < n ? j : n - 1), sb, k);

  // Two register sets: the next step's rows load while this step's are
  // dotted (loads past the block's last row repeat it, never stored).
  struct DSet {
    u32x4 hw[RU], aw[RU], bw[RU];
  };
  auto load = [&](int b0, DSet &d) {
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const int64_t r = r0 + (b0 + u < nr ? b0 + u : nr - 1);
      const uint8_t *row = W + r * row_bytes;
      d.hw[u] = __builtin_nontemporal_load((const u32x4 *)(row + oh));
      d.aw[u] = __builtin_nontemporal_load((const u32x4 *)(row + oa));
      d.bw[u] = __builtin_nontemporal_load((const u32x4 *)(row + ob));
    }
  };
  auto step = [&](int b0, const DSet &d) {
#pragma unroll
    for (int u = 0; u < RU; ++u) {
      const TaskW w = unpack_task(d.hw[u], d.aw[u], d.bw[u], k);
#pragma unroll
      for (int j = 0; j < NT; ++j) {
        if (j < n) {  // uniform: the expert's row count
          float v;
          if constexpr (DBG) {
            const bool on = tv && b0 + u < nr;
            v = task_value(w, s[j], on ? a.dbg.s[0] : nullptr, a.dbg.m[0],
                           ((p0 + j) * rows + r0 + b0 + u) * nb + sb);
          } else {
            v = task_value(w, s[j]);
          }
          v = group_sum<64>(tv ? v : 0.0f);
          if (lane == 0 && b0 + u < nr) part[wave][b0 + u][j] = v;
        }
      }
    }
  };
  DSet d0, d1;
  int b0 = 0;
  load(0, d0);
  while (b0 < nr) {
    load(b0 + RU, d1);
    step(b0, d0);
    b0 += RU;
    if (b0 >= nr) break;
    load(b0 + RU, d0);
    step(b0, d1);
    b0 += RU;
  }
  __syncthreads();
  for (int q = threadIdx.x; q < nr * NT; q += 256) {
    const int rr = q / NT, j = q % NT;
    if (j < n) {
      const float y = ((part[0][rr][j] + part[1][rr][j]) + part[2][rr][j]) + part[3][rr][j];
      a.out[(p0 + j) * rows + r0 + rr] = y;
    }
  }
}

int small_cus() {
  static int cus = 0;
  if (!cus) {
    int dev = 0, v = 0;
    cus = hipGetDevice(&dev) == hipSuccess &&
                  hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && v > 0
              ? v
              : 256;
  }
  return cus;
}

}  // namespace

bool small_supported(int64_t rows, int64_t cols, int mode) {
  if (cols % 256 != 0 || rows <= 0) return false;
  const int64_t ntasks = 4 * (cols / 256);
  // rows narrow enough for the registers, wide enough to keep most lanes busy
  if (mode == 0) return ntasks >= 48 && ntasks <= 128;  // gate/up: one or two tasks per lane
  return ntasks >= 128 && ntasks <= 256;                // down: a quarter of the tasks per wave
}

int small_rows_for(int64_t cols, int mode, int64_t max_rows) {
  (void)cols;
  (void)mode;
  // batches of up to 8 tokens: the experts mostly hold 1-3 rows, so slices
  // for 4 (the rare larger expert goes to the general kernels); 0 for larger
  // batches, whose experts are better served by the matrix-core kernels
  return max_rows <= 2 ? 2 : (max_rows <= kSmallBatchMax ? 4 : 0);
}

hipError_t launch_small(hipStream_t st, int mode, const ExpertTier &tier, int64_t rows, int64_t cols,
                        const Routing &rt, int regime, int max_active, int64_t max_rows, const int8_t *xq,
                        const float *xd, const int32_t *xbs, float *out, const BlockDbg *dbg) {
  if (rows <= 0 || max_active <= 0) return hipSuccess;
  const int nt = small_rows_for(cols, mode, max_rows);
  if (!small_supported(rows, cols, mode) || nt == 0) return hipErrorNotSupported;
  SmallArgs a{tier, rt, rows, cols, xq, xd, xbs, out, regime, 0, 0, dbg ? *dbg : BlockDbg{}};
  const int cus = small_cus();
  if (mode == 0) {
    const int tpl = 4 * (cols / 256) <= 64 ? 1 : 2;
    constexpr int RU = 1;
    // about two work-groups per CU in all, spread evenly over the experts' rows
    const int64_t need = (rows + 4 * RU - 1) / (4 * RU);
    int64_t cap = 2LL * cus / max_active;
    if (cap < 1) cap = 1;
    const int64_t per = (need + cap - 1) / cap;
    a.groups = (int32_t)((need + per - 1) / per);
    const dim3 grid((unsigned)a.groups, (unsigned)max_active);
#define KMOE_SGU(TP, N)                                                          \
  do {                                                                           \
    if (dbg) KMOE_LAUNCH((k_small_gate_up<TP, N, RU, true>), grid, dim3(256), 0, st, a);   \
    else KMOE_LAUNCH((k_small_gate_up<TP, N, RU, false>), grid, dim3(256), 0, st, a);      \
  } while (0)
    if (tpl == 1) {
      if (nt == 2) KMOE_SGU(1, 2);
      else KMOE_SGU(1, 4);
    } else {
      if (nt == 2) KMOE_SGU(2, 2);
      else KMOE_SGU(2, 4);
    }
#undef KMOE_SGU
  } else {
    constexpr int RU = 2;
    // rows per work-group: about two work-groups per CU in all
    int64_t rb = (rows * max_active + 2LL * cus - 1) / (2LL * cus);
    rb = (rb + RU - 1) / RU * RU;
    if (rb < RU) rb = RU;
    if (rb > kSmallRbMax) rb = kSmallRbMax;
    a.rb = (int32_t)rb;
    const dim3 grid((unsigned)((rows + rb - 1) / rb), (unsigned)max_active);
    if (nt == 2) {
      if (dbg) KMOE_LAUNCH((k_small_down<2, RU, true>), grid, dim3(256), 0, st, a);
      else KMOE_LAUNCH((k_small_down<2, RU, false>), grid, dim3(256), 0, st, a);
    } else {
      if (dbg) KMOE_LAUNCH((k_small_down<4, RU, true>), grid, dim3(256), 0, st, a);
      else KMOE_LAUNCH((k_small_down<4, RU, false>), grid, dim3(256), 0, st, a);
    }
  }
  return hipGetLastError();
}

}  // namespace kmoe
