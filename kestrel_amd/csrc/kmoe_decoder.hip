// kmoe_decoder.hip — the rest of the decoder layer around the MoE FFN
// (Transformer::forward_chunk_inner, transformer.rs:375-467): embedding rows,
// RMSNorm with the residual add, RoPE, the f16 KV cache store, causal GQA
// attention over that cache, SwiGLU for dense FFNs, bias rows and the greedy
// argmax.
//
// Positions: every position-dependent kernel takes pos0 and an optional
// device counter pos_dev; the position of row s is pos0 + s (+ *pos_dev). A
// decode step that reads its position from pos_dev can be captured once as a
// HIP graph and replayed, with k_pos_advance moving the counter.
//
// These kernels are latency-bound at decode (kilobytes per call); their
// sizes follow the data, not the 256 CUs.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "kmoe_device.h"
#include "kmoe_launch.h"

namespace kmoe {
namespace {

__device__ __forceinline__ float f16_at(const uint8_t *p) { return f16_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8)); }

// Element i of one GGUF row, in dequant_row's expression order
// (quant.rs:63-205): F32, F16, Q8_0, Q4_K, Q6_K.
__device__ float dq_elem(int t, const uint8_t *row, int64_t i) {
  switch (t) {
    case T_F32: return ((const float *)row)[i];
    case T_F16: return f16_at(row + 2 * i);
    case T_Q8_0: {
      const uint8_t *b = row + 34 * (i / 32);
      return (float)(int8_t)b[2 + i % 32] * f16_at(b);
    }
    case T_Q4_K: {
      const uint8_t *b = row + 144 * (i / 256);
      const int e = (int)(i % 256), k = e / 64, l = e % 32, hi = (e / 32) & 1;
      const int j = 2 * k + hi;  // sub-block
      const uint8_t *sc = b + 4;
      int s, m;
      if (j < 4) {
        s = sc[j] & 63;
        m = sc[j + 4] & 63;
      } else {
        s = (sc[j + 4] & 0xF) | ((sc[j - 4] >> 6) << 4);
        m = (sc[j + 4] >> 4) | ((sc[j] >> 6) << 4);
      }
      const uint8_t q = b[16 + 32 * k + l];
      const float d1 = f16_at(b) * (float)s, m1 = f16_at(b + 2) * (float)m;
      return d1 * (float)(hi ? (q >> 4) : (q & 0xF)) - m1;
    }
    case T_Q6_K: {
      const uint8_t *b = row + 210 * (i / 256);
      const int e = (int)(i % 256), h = e / 128, r = e % 128, qd = r / 32, l = r % 32;
      const uint8_t *ql = b + 64 * h, *qh = b + 128 + 32 * h, *sc = b + 192 + 8 * h;
      const uint8_t lo = (qd & 1) ? ql[l + 32] : ql[l];
      const int nib = (qd >= 2) ? (lo >> 4) : (lo & 0xF);
      const int q = (nib | (((qh[l] >> (2 * qd)) & 3) << 4)) - 32;
      return f16_at(b + 208) * (float)(int8_t)sc[l / 16 + 2 * qd] * (float)q;
    }
    default: return 0.0f;
  }
}

// quant::get_row (quant.rs:342-345) for s_rows token ids; ids >= n_rows give
// rows of zeros (the host entry point rejects them before launch).
__global__ void __launch_bounds__(256) k_get_rows(int t, const uint8_t *__restrict__ table, int64_t row_bytes,
                                                  int64_t n_rows, int64_t cols, const uint32_t *__restrict__ ids,
                                                  float *__restrict__ out) {
  const int64_t s = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= cols) return;
  const uint32_t id = ids[s];
  out[s * cols + i] = id < n_rows ? dq_elem(t, table + (int64_t)id * row_bytes, i) : 0.0f;
}

// Transformer::rmsnorm (transformer.rs:330-340) with the residual add of
// forward_chunk_inner (transformer.rs:427, :463) in front: when y is non-null,
// x += y is stored first and the norm is taken of the sum. out may alias x
// (each thread reads its elements before writing them).
__global__ void __launch_bounds__(256) k_add_rmsnorm(float *x, const float *__restrict__ y,
                                                     const float *__restrict__ w, int64_t dim, float eps,
                                                     float *out) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  float *xr = x + r * dim;
  float ss = 0.0f;
  for (int64_t j = threadIdx.x; j < dim; j += 256) {
    float v = xr[j];
    if (y) {
      v = v + y[r * dim + j];
      xr[j] = v;
    }
    ss += v * v;
  }
  ss = wg_sum256(ss, red);
  const float rr = 1.0f / sqrtf(ss / (float)dim + eps);
  for (int64_t j = threadIdx.x; j < dim; j += 256) {
    const float t = xr[j] * rr;
    out[r * dim + j] = t * w[j];
  }
}

// The same for rows with dim % 4 == 0 and dim <= 1024 * NCH, the row held in
// registers: thread t owns the float4 slots t + 256 k (elements 4t + 1024k
// .. +3), and every load is issued before the first use. QT 1 also writes
// the Q8_K quantization of the output (Q8KRow::quantize, qdot.rs:347-367;
// dim % 256 == 0: wave w of chunk k holds block 4k + w), QT 2 the Q8 one
// (Q8Row::quantize, qdot.rs:30-49; dim % 32 == 0: 8-lane groups hold blocks),
// for the integer matvec that follows.
template <int NCH, int QT>
__global__ void __launch_bounds__(256) k_rmsnorm_regs(float *x, const float *__restrict__ y,
                                                      const float *__restrict__ w, int64_t dim, float eps, float *out,
                                                      int8_t *__restrict__ q, float *__restrict__ qd,
                                                      int32_t *__restrict__ qs) {
  __shared__ float red[4];
  const int64_t r = blockIdx.x;
  const int t = threadIdx.x;
  const int n4 = (int)(dim / 4);
  float4 *xr = (float4 *)(x + r * dim);
  const float4 *yr = (const float4 *)(y + r * dim);
  const float4 *wr = (const float4 *)w;
  float4 v[NCH], ww[NCH];
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int i = t + 256 * k;
    if (i < n4) {
      v[k] = xr[i];
      ww[k] = wr[i];
    }
  }
  if (y) {
    float4 yy[NCH];
#pragma unroll
    for (int k = 0; k < NCH; ++k)
      if (t + 256 * k < n4) yy[k] = yr[t + 256 * k];
#pragma unroll
    for (int k = 0; k < NCH; ++k)
      if (t + 256 * k < n4) {
        v[k].x = v[k].x + yy[k].x;
        v[k].y = v[k].y + yy[k].y;
        v[k].z = v[k].z + yy[k].z;
        v[k].w = v[k].w + yy[k].w;
        xr[t + 256 * k] = v[k];
      }
  }
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NCH; ++k)
    if (t + 256 * k < n4) ss += ((v[k].x * v[k].x + v[k].y * v[k].y) + v[k].z * v[k].z) + v[k].w * v[k].w;
  ss = wg_sum256(ss, red);
  const float rr = 1.0f / sqrtf(ss / (float)dim + eps);
  float4 *orow = (float4 *)(out + r * dim);
#pragma unroll
  for (int k = 0; k < NCH; ++k) {
    const int i = t + 256 * k;
    if (i < n4) {
      float4 h;
      h.x = (v[k].x * rr) * ww[k].x;
      h.y = (v[k].y * rr) * ww[k].y;
      h.z = (v[k].z * rr) * ww[k].z;
      h.w = (v[k].w * rr) * ww[k].w;
      orow[i] = h;
      if constexpr (QT == 1) {
        const int64_t b = 4 * k + (t >> 6);
        wave_quant_q8k_vals(h, q + r * dim + 256 * b, qd + r * (dim / 256) + b, qs + r * (dim / 16) + 16 * b,
                            t & 63);
      } else if constexpr (QT == 2) {
        const int64_t b = (4 * (int64_t)i) / 32;
        group8_quant_q8_vals(h, q + r * dim + 32 * b, qd + r * (dim / 32) + b, qs + r * (dim / 16) + 2 * b, t & 7);
      }
    }
  }
}

__device__ __forceinline__ int64_t position(int64_t pos0, const int32_t *pos_dev) {
  return pos0 + (pos_dev ? (int64_t)*pos_dev : 0);
}

// Transformer::rope (transformer.rs:342-358), in place: one thread per
// (row, pair); sin and cos of the f32 angle from sincosf (within an ulp of
// the reference's f32::sin_cos).
__global__ void __launch_bounds__(256) k_rope(float *__restrict__ x, int64_t s_rows, int n_heads, int hd, int rd,
                                              int64_t pos0, const int32_t *__restrict__ pos_dev,
                                              const float *__restrict__ inv_freq, int neox) {
  const int half = rd / 2;
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= s_rows * half) return;
  const int64_t s = g / half;
  const int i = (int)(g % half);
  const float p = (float)(position(pos0, pos_dev) + s);
  const float ang = p * inv_freq[i];
  float sn, cs;
  sincosf(ang, &sn, &cs);
  const int a = neox ? i : 2 * i, b = neox ? i + half : 2 * i + 1;
  for (int h = 0; h < n_heads; ++h) {
    float *v = x + (s * n_heads + h) * (int64_t)hd;
    const float x0 = v[a], x1 = v[b];
    v[a] = x0 * cs - x1 * sn;
    v[b] = x0 * sn + x1 * cs;
  }
}

// KV cache store (transformer.rs:411-418): f32 -> f16, round to nearest even
// (half::f16::from_f32), at cache row position + s; rows past n_ctx are not
// written.
__global__ void __launch_bounds__(256) k_kv_store(const float *__restrict__ k, const float *__restrict__ v,
                                                  int64_t s_rows, int64_t kvw, int64_t pos0,
                                                  const int32_t *__restrict__ pos_dev, int64_t n_ctx,
                                                  uint16_t *__restrict__ kc, uint16_t *__restrict__ vc) {
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (g >= s_rows * kvw) return;
  const int64_t s = g / kvw, j = g % kvw;
  const int64_t p = position(pos0, pos_dev) + s;
  if (p < 0 || p >= n_ctx) return;
  kc[p * kvw + j] = __builtin_bit_cast(uint16_t, (_Float16)k[g]);
  vc[p * kvw + j] = __builtin_bit_cast(uint16_t, (_Float16)v[g]);
}

// ---------------------------------------------------------------------------
// RoPE of q and k and the KV cache store in one pass (transformer.rs:406-418):
// work-group (row s, group of 4 heads) builds the row's sin/cos table in LDS
// (sincosf of the f32 angle, within an ulp of glibc's), then one wave per
// head: q heads are rotated into q_out, k heads rotated and stored with the
// matching v head as f16 into the caches.
constexpr int kRopeHeads = 4;

__global__ void __launch_bounds__(256) k_rope_kv(const float *__restrict__ q, const float *__restrict__ k,
                                                 const float *__restrict__ v, int nh, int nkv, int hd, int rd,
                                                 int64_t pos0, const int32_t *__restrict__ pos_dev,
                                                 const float *__restrict__ inv_freq, int neox, int64_t n_ctx,
                                                 float *__restrict__ q_out, uint16_t *__restrict__ kc,
                                                 uint16_t *__restrict__ vc) {
  __shared__ float sn[128], cs[128];
  const int64_t s = blockIdx.x;
  const int half = rd / 2;
  const int64_t p = position(pos0, pos_dev) + s;
  for (int i = threadIdx.x; i < half; i += 256) {
    const float ang = (float)p * inv_freq[i];
    float sv, cv;
    sincosf(ang, &sv, &cv);
    sn[i] = sv;
    cs[i] = cv;
  }
  __syncthreads();
  const int head = blockIdx.y * kRopeHeads + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (head >= nh + nkv) return;
  const bool is_q = head < nh;
  const int kh = head - nh;
  if (!is_q && (p < 0 || p >= n_ctx)) return;
  const float *row = is_q ? q + (s * nh + head) * (int64_t)hd : k + (s * nkv + kh) * (int64_t)hd;
  const int64_t kvw = (int64_t)nkv * hd;
  for (int dd = lane; dd < hd; dd += 64) {
    float val = row[dd];
    if (dd < rd) {
      int i, a, b;
      bool first;
      if (neox) {
        first = dd < half;
        i = first ? dd : dd - half;
        a = i;
        b = i + half;
      } else {
        first = (dd & 1) == 0;
        i = dd >> 1;
        a = 2 * i;
        b = 2 * i + 1;
      }
      const float x0 = row[a], x1 = row[b];
      val = first ? x0 * cs[i] - x1 * sn[i] : x0 * sn[i] + x1 * cs[i];
    }
    if (is_q) {
      q_out[(s * nh + head) * (int64_t)hd + dd] = val;
    } else {
      kc[p * kvw + (int64_t)kh * hd + dd] = __builtin_bit_cast(uint16_t, (_Float16)val);
      vc[p * kvw + (int64_t)kh * hd + dd] =
          __builtin_bit_cast(uint16_t, (_Float16)v[(s * nkv + kh) * (int64_t)hd + dd]);
    }
  }
}

// ---------------------------------------------------------------------------
// Causal GQA attention (Transformer::attention, transformer.rs:591-631).
//
// One wave works one chunk of 64 cache positions for one query head:
// - loads: the chunk's K and V rows of kv head g as 16-byte pieces, coalesced
//   (load j of lane l reads piece l % (hd / 8) of row j * RPI + l / (hd / 8),
//   RPI = 64 / (hd / 8) rows per load); rows past the chunk's end are read
//   clamped to its last row;
// - scores: the K pieces turn through the wave's LDS tile so that lane l holds
//   position l's row; it is scored against the head's q (LDS, broadcast reads)
//   in quant::dot's eight-accumulator order (quant.rs:208-224), times
//   1/sqrt(hd), so the scores are bit-identical to the reference's; positions
//   past the end score -inf;
// - softmax: the chunk's max m, e = exp(score - m) (0 past the end), l = sum e;
// - weighted V: lane l keeps its V pieces (head dims 8p .. 8p + 7, p = l %
//   (hd / 8)) of rows j * RPI + l / (hd / 8) in registers, zeroed past the end,
//   sums e_r v_r over them in row order with e read from LDS, and the RPI row
//   classes of a piece are then added in class order across lanes.
// Chunk partials (m, l, acc) merge as out = sum acc e^(m - M) / sum l e^(m - M)
// over the chunks in order, M their max.
constexpr int kAttnChunk = 64;
constexpr int kMaxGroup = 16;
// Rows of at most this many chunks run in one work-group per head in the
// one-row kernel (one chunk per wave). Measured on MI355X with the caches read
// from HBM (16 heads of 128): 6.7 against 9.0 us at 128 positions, 8.2 against
// 9.7 us at 256, but 10.9 against 10.2 us at 384, where one CU's loads take
// longer than spreading the chunks and handing the partials over.
constexpr int kAttnSpanMax = 4;

// LDS written by lanes of a wave and read by other lanes of the same wave:
// orders the LDS accesses only, so global loads stay in flight.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// One chunk's K rows in LDS, each padded by a piece: the lane-per-row reads of
// eight lanes then cover the 32 banks once.
template <int HD>
struct AttnKTile {
  uint4 p[kAttnChunk][HD / 8 + 1];
};

// Load j of lane l: piece l % (HD / 8) of chunk row j * RPI + l / (HD / 8).
template <int HD>
__device__ __forceinline__ int64_t attn_piece_off(int64_t kvw, int g, int64_t p0, int np, int j, int lane) {
  constexpr int KV4 = HD / 8, RPI = 64 / KV4;
  const int r = j * RPI + lane / KV4;
  return (p0 + (r < np ? r : np - 1)) * kvw + (int64_t)g * HD + 8 * (lane % KV4);
}

// q of one head against lane-per-row K: the score of position lane.
template <int HD>
__device__ __forceinline__ float attn_score(const float *qh, const uint4 (&kr)[HD / 8], int lane, int np) {
  constexpr int KV4 = HD / 8;
  const float scale = 1.0f / sqrtf((float)HD);
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < KV4; ++j) {
    const uint32_t w4[4] = {kr[j].x, kr[j].y, kr[j].z, kr[j].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float a0 = qh[8 * j + 2 * i] * f16_bits_to_f32(w4[i]);
      const float a1 = qh[8 * j + 2 * i + 1] * f16_bits_to_f32(w4[i] >> 16);
      acc[2 * i] = acc[2 * i] + a0;
      acc[2 * i + 1] = acc[2 * i + 1] + a1;
    }
  }
  float t = -0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) t = t + acc[i];
  return lane < np ? t * scale : -INFINITY;
}

// sum e_r v_r over the chunk for head dims 8p .. 8p + 7, p = lane % (HD / 8)
// (every lane of piece p receives them); ws[r] = e_r, vp = this lane's pieces.
// Rows past np contribute +0 * +0 to sums that start at +0.
template <int HD>
__device__ __forceinline__ void attn_wv(const float *ws, const uint4 (&vp)[HD / 8], int lane, int np, float (&o8)[8]) {
  constexpr int KV4 = HD / 8, RPI = 64 / KV4;
  const int rc = lane / KV4, p = lane % KV4;
  float a[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < KV4; ++j) {
    const int r = j * RPI + rc;
    const float w = ws[r];
    const bool live = r < np;
    const uint32_t u[4] = {live ? vp[j].x : 0u, live ? vp[j].y : 0u, live ? vp[j].z : 0u, live ? vp[j].w : 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[2 * i] = a[2 * i] + w * f16_bits_to_f32(u[i]);
      a[2 * i + 1] = a[2 * i + 1] + w * f16_bits_to_f32(u[i] >> 16);
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    float t = __shfl(a[i], p);
#pragma unroll
    for (int c = 1; c < RPI; ++c) t = t + __shfl(a[i], p + c * KV4);
    o8[i] = t;
  }
}

// The int8 rows of the attention output for the projection after it: the
// group's group * HD outputs of row s (staged in LDS) are whole Q8_K blocks
// (qt 1, group * HD % 256 == 0: one wave per block) or Q8 blocks (qt 2, eight
// lanes per block), quantized as the matmul's own quantization kernel would.
template <int HD, int NW = 4>
__device__ __forceinline__ void attn_quant_group(const float *os, int group, int64_t s, int g, int nh, int qt,
                                                 int8_t *xq, float *xd, int32_t *xs) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int64_t row = (int64_t)nh * HD, gb = (int64_t)g * group * HD;
  const int nv = group * HD;
  if (qt == 1) {
    for (int b = wave; b < nv / 256; b += NW) {
      const float4 v = *(const float4 *)(os + 256 * b + 4 * lane);
      const int64_t blk = (gb / 256) + b;
      wave_quant_q8k_vals(v, xq + s * row + 256 * blk, xd + s * (row / 256) + blk, xs + s * (row / 16) + 16 * blk,
                          lane);
    }
  } else {
    for (int b = wave * 8 + (lane >> 3); b < nv / 32; b += 8 * NW) {
      const float4 v = *(const float4 *)(os + 32 * b + 4 * (lane & 7));
      const int64_t blk = (gb / 32) + b;
      group8_quant_q8_vals(v, xq + s * row + 32 * blk, xd + s * (row / 32) + blk, xs + s * (row / 16) + 2 * blk,
                           lane & 7);
    }
  }
}

// Work-group bid = (kv head g, query row s, chunk c) of 256 threads; wave w
// takes query heads w, w + 4, ... of the group over the chunk, whose K rows the
// work-group loads into its tile together. With one chunk the result is final;
// otherwise every work-group of the row hands (m, l, acc) over with agent-scope
// stores and a counter, and the last to arrive merges them and resets the
// counter. LDS: Qs and Os [kMaxGroup][HD], Ws [4][64], one K tile.
template <int HD>
__device__ __forceinline__ void attn_batch(int64_t bid, const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                           const uint16_t *__restrict__ vc, int64_t s_rows, int nh, int nkv,
                                           int64_t pos0, const int32_t *__restrict__ pos_dev, int64_t n_ctx,
                                           int nch_grid, float *part, uint32_t *counters, float *__restrict__ out,
                                           int qt, int8_t *__restrict__ xq, float *__restrict__ xd,
                                           int32_t *__restrict__ xs, float (*Qs)[HD], float (*Os)[HD],
                                           float (*Ws)[kAttnChunk], AttnKTile<HD> &Kt, uint32_t &last) {
  constexpr int KV4 = HD / 8;
  constexpr int DPL = HD / 64;  // head dims per lane in the merge
  constexpr int PW = HD + 2;    // one chunk partial: m, l, acc[HD]
  const int c = (int)(bid % nch_grid);
  const int64_t s = (bid / nch_grid) % s_rows;
  const int g = (int)(bid / nch_grid / s_rows);
  int64_t n = position(pos0, pos_dev) + s + 1;
  if (n > n_ctx) n = n_ctx;
  const int nch = (int)((n + kAttnChunk - 1) / kAttnChunk);
  if (c >= nch) return;
  const int group = nh / nkv;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int64_t kvw = (int64_t)nkv * HD;
  const int64_t p0 = (int64_t)c * kAttnChunk;
  const int np = (int)(n - p0 < kAttnChunk ? n - p0 : kAttnChunk);
  // q of the group's heads and the chunk's K rows into LDS, V pieces into the
  // registers of the waves that use them, all issued before any is used
  for (int e = threadIdx.x; e < group * HD; e += 256) Qs[e / HD][e % HD] = q[(s * nh + (int64_t)g * group) * HD + e];
  constexpr int NT = kAttnChunk * KV4 / 256;  // K pieces per thread
  uint4 kp[NT], vp[KV4];
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const int e = threadIdx.x + 256 * i, r = e / KV4;
    kp[i] = *(const uint4 *)(kc + (p0 + (r < np ? r : np - 1)) * kvw + (int64_t)g * HD + 8 * (e % KV4));
  }
  if (wave < group) {
#pragma unroll
    for (int j = 0; j < KV4; ++j) vp[j] = *(const uint4 *)(vc + attn_piece_off<HD>(kvw, g, p0, np, j, lane));
  }
#pragma unroll
  for (int i = 0; i < NT; ++i) {
    const int e = threadIdx.x + 256 * i;
    Kt.p[e / KV4][e % KV4] = kp[i];
  }
  lds_barrier();  // Qs, Kt
  if (wave < group) {
    uint4 kr[KV4];
#pragma unroll
    for (int j = 0; j < KV4; ++j) kr[j] = Kt.p[lane][j];
    for (int hh = wave; hh < group; hh += 4) {
      const int64_t h = (int64_t)g * group + hh;
      const float sc_ = attn_score<HD>(Qs[hh], kr, lane, np);
      const float m = group_max<64>(sc_);
      const float e = lane < np ? expf(sc_ - m) : 0.0f;
      const float l = group_sum<64>(e);
      Ws[wave][lane] = e;
      wave_lds_sync();
      float o8[8];
      attn_wv<HD>(Ws[wave], vp, lane, np, o8);
      wave_lds_sync();  // the weights are read before the next head writes them
      if (nch == 1) {
        const float inv = 1.0f / l;
        if (lane < KV4) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const float r = o8[i] * inv;
            out[(s * nh + h) * HD + 8 * lane + i] = r;
            Os[hh][8 * lane + i] = r;
          }
        }
      } else {
        float *pp = part + ((s * nh + h) * nch_grid + c) * PW;
        if (lane == 0) {
          st_agent(pp, m);
          st_agent(pp + 1, l);
        }
        if (lane < KV4) {
#pragma unroll
          for (int i = 0; i < 8; ++i) st_agent(pp + 2 + 8 * lane + i, o8[i]);
        }
      }
    }
  }
  if (nch == 1) {
    if (qt) {
      __syncthreads();
      attn_quant_group<HD>(Os[0], group, s, g, nh, qt, xq, xd, xs);
    }
    return;
  }
  vm_wait();  // this wave's partials are written before the counter moves
  __syncthreads();
  if (threadIdx.x == 0) {
    last = add_release(counters + s * nkv + g, 1u);
    if (last == (uint32_t)(nch - 1)) acquire_agent();
  }
  __syncthreads();
  if (last != (uint32_t)(nch - 1)) return;
  for (int hh = wave; hh < group; hh += 4) {
    const int64_t h = (int64_t)g * group + hh;
    const float *pb = part + (s * nh + h) * nch_grid * PW;
    // the partials of 8 chunks at a time, every load issued before any use
    constexpr int B = 8;
    float M = -INFINITY;
    for (int c0 = 0; c0 < nch; c0 += B) {
      float mv[B];
#pragma unroll
      for (int j = 0; j < B; ++j) mv[j] = c0 + j < nch ? ld_agent(pb + (c0 + j) * PW) : -INFINITY;
#pragma unroll
      for (int j = 0; j < B; ++j) M = fmaxf(M, mv[j]);
    }
    float L = 0.0f, O[DPL];
#pragma unroll
    for (int i = 0; i < DPL; ++i) O[i] = 0.0f;
    for (int c0 = 0; c0 < nch; c0 += B) {
      float mv[B], lv[B], ov[B][DPL];
#pragma unroll
      for (int j = 0; j < B; ++j) {
        if (c0 + j < nch) {
          const float *pc = pb + (c0 + j) * PW;
          mv[j] = ld_agent(pc);
          lv[j] = ld_agent(pc + 1);
#pragma unroll
          for (int i = 0; i < DPL; ++i) ov[j][i] = ld_agent(pc + 2 + lane * DPL + i);
        }
      }
#pragma unroll
      for (int j = 0; j < B; ++j) {
        if (c0 + j < nch) {
          const float f = expf(mv[j] - M);
          L += lv[j] * f;
#pragma unroll
          for (int i = 0; i < DPL; ++i) O[i] += ov[j][i] * f;
        }
      }
    }
    const float inv = 1.0f / L;
#pragma unroll
    for (int i = 0; i < DPL; ++i) {
      const float r = O[i] * inv;
      out[(s * nh + h) * HD + lane * DPL + i] = r;
      Os[hh][lane * DPL + i] = r;
    }
  }
  if (threadIdx.x == 0) st_agent(counters + s * nkv + g, 0u);  // ready for the next call
  if (qt) {
    __syncthreads();
    attn_quant_group<HD>(Os[0], group, s, g, nh, qt, xq, xd, xs);
  }
}

template <int HD>
__global__ void __launch_bounds__(256) k_attn_dec(const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                  const uint16_t *__restrict__ vc, int64_t s_rows, int nh, int nkv,
                                                  int64_t pos0, const int32_t *__restrict__ pos_dev, int64_t n_ctx,
                                                  int nch_grid, float *part, uint32_t *counters,
                                                  float *__restrict__ out, int qt, int8_t *__restrict__ xq,
                                                  float *__restrict__ xd, int32_t *__restrict__ xs) {
  __shared__ uint32_t last;
  __shared__ __attribute__((aligned(16))) float Qs[kMaxGroup][HD];
  __shared__ __attribute__((aligned(16))) float Os[kMaxGroup][HD];
  __shared__ float Ws[4][kAttnChunk];
  __shared__ AttnKTile<HD> Kt;
  attn_batch<HD>(blockIdx.x, q, kc, vc, s_rows, nh, nkv, pos0, pos_dev, n_ctx, nch_grid, part, counters, out, qt, xq,
                 xd, xs, Qs, Os, Ws, Kt, last);
}

// The same attention for one query row per call (decode), grid nh x nch_grid
// work-groups of 256 threads. Rows of at most kAttnSpanMax chunks: work-group
// h takes query head h, wave w chunk w over the rows of its kv head, with
// attn_batch's chunk arithmetic; the partials stay in LDS and wave 0 merges
// them in chunk order with attn_batch's merge expressions, so the output has
// a batch call's bits and nothing leaves the CU but the result. Longer rows:
// the work-groups below nkv x nch_grid run attn_batch, whose chunks spread
// over more CUs (one CU's loads would take longer than the merge's hand-off).
// QT 2 also writes the head's Q8 rows (32-blocks) for the projection after it;
// QT 1 (Q8_K, whose blocks span heads) is not taken.
template <int HD>
__global__ void __launch_bounds__(256) k_attn_one(const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                  const uint16_t *__restrict__ vc, int nh, int nkv, int64_t pos0,
                                                  const int32_t *__restrict__ pos_dev, int64_t n_ctx, int nch_grid,
                                                  float *part, uint32_t *counters, float *__restrict__ out, int qt,
                                                  int8_t *__restrict__ xq, float *__restrict__ xd,
                                                  int32_t *__restrict__ xs) {
  constexpr int KV4 = HD / 8;
  constexpr int DPL = HD / 64;
  constexpr int PW = HD + 2;  // one chunk partial: m, l, acc[HD]
  __shared__ uint32_t last;
  __shared__ __attribute__((aligned(16))) float Qs[kMaxGroup][HD];
  __shared__ __attribute__((aligned(16))) float Os[kMaxGroup][HD];
  __shared__ float Ws[4][kAttnChunk];
  __shared__ __attribute__((aligned(16))) float Lp[kAttnSpanMax][PW];
  __shared__ AttnKTile<HD> Kt[kAttnSpanMax];
  int64_t n = position(pos0, pos_dev) + 1;
  if (n > n_ctx) n = n_ctx;
  const int nch = (int)((n + kAttnChunk - 1) / kAttnChunk);
  if (nch > kAttnSpanMax) {
    if (blockIdx.x < nkv * nch_grid)
      attn_batch<HD>(blockIdx.x, q, kc, vc, 1, nh, nkv, pos0, pos_dev, n_ctx, nch_grid, part, counters, out, qt, xq,
                     xd, xs, Qs, Os, Ws, Kt[0], last);
    return;
  }
  if (blockIdx.x >= (unsigned)nh) return;
  const int h = blockIdx.x;
  const int g = h / (nh / nkv);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const int c = wave;
  const bool active = c < nch;
  const int64_t kvw = (int64_t)nkv * HD;
  const int64_t p0 = (int64_t)c * kAttnChunk;
  const int np = active ? (int)(n - p0 < kAttnChunk ? n - p0 : kAttnChunk) : 0;
  if (threadIdx.x < HD) Qs[0][threadIdx.x] = q[(int64_t)h * HD + threadIdx.x];
  uint4 kp[KV4], vp[KV4];
  if (active) {
#pragma unroll
    for (int j = 0; j < KV4; ++j) kp[j] = *(const uint4 *)(kc + attn_piece_off<HD>(kvw, g, p0, np, j, lane));
#pragma unroll
    for (int j = 0; j < KV4; ++j) vp[j] = *(const uint4 *)(vc + attn_piece_off<HD>(kvw, g, p0, np, j, lane));
#pragma unroll
    for (int j = 0; j < KV4; ++j) Kt[wave].p[j * (64 / KV4) + lane / KV4][lane % KV4] = kp[j];
  }
  lds_barrier();  // Qs, the K tiles
  if (active) {
    uint4 kr[KV4];
#pragma unroll
    for (int j = 0; j < KV4; ++j) kr[j] = Kt[wave].p[lane][j];
    const float sc_ = attn_score<HD>(Qs[0], kr, lane, np);
    const float m = group_max<64>(sc_);
    const float e = lane < np ? expf(sc_ - m) : 0.0f;
    const float l = group_sum<64>(e);
    Ws[wave][lane] = e;
    wave_lds_sync();
    float o8[8];
    attn_wv<HD>(Ws[wave], vp, lane, np, o8);
    if (lane == 0) {
      Lp[wave][0] = m;
      Lp[wave][1] = l;
    }
    if (lane < KV4) {
#pragma unroll
      for (int i = 0; i < 8; ++i) Lp[wave][2 + 8 * lane + i] = o8[i];
    }
  }
  lds_barrier();  // the chunk partials
  if (wave != 0) return;
  float M = -INFINITY, L = 0.0f, O[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) O[i] = 0.0f;
  for (int cc = 0; cc < nch; ++cc) M = fmaxf(M, Lp[cc][0]);
  for (int cc = 0; cc < nch; ++cc) {
    const float f = expf(Lp[cc][0] - M);
    L += Lp[cc][1] * f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) O[i] += Lp[cc][2 + lane * DPL + i] * f;
  }
  const float inv = 1.0f / L;
#pragma unroll
  for (int i = 0; i < DPL; ++i) {
    const float r = O[i] * inv;
    out[(int64_t)h * HD + lane * DPL + i] = r;
    Os[0][lane * DPL + i] = r;
  }
  if (qt == 2) {
    wave_lds_sync();  // the head's outputs are in LDS
    const int b = lane >> 3;  // HD / 32 blocks of 8 lanes
    if (b < HD / 32) {
      const float4 v = *(const float4 *)(&Os[0][0] + 32 * b + 4 * (lane & 7));
      const int64_t blk = (int64_t)h * (HD / 32) + b;
      group8_quant_q8_vals(v, xq + 32 * blk, xd + blk, xs + 2 * blk, lane & 7);
    }
  }
}

// Dense SwiGLU (transformer.rs:455): out = g / (1 + exp(-g)) * u.
__global__ void __launch_bounds__(256) k_swiglu(const float *__restrict__ g, const float *__restrict__ u, int64_t n,
                                                float *__restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const float gv = g[i];
  const float den = 1.0f + expf_cr(-gv);
  out[i] = gv / den * u[i];
}

// Bias rows (transformer.rs:394-401): x[r] += b.
__global__ void __launch_bounds__(256) k_add_rows(float *__restrict__ x, const float *__restrict__ b, int64_t rows,
                                                  int64_t cols) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * cols) return;
  x[i] = x[i] + b[i % cols];
}

// sampler::argmax (sampler.rs:104-112): the first index of the largest value
// (NaN never wins; a NaN at index 0 makes 0 the answer, as the scan's
// comparisons with it all fail). One work-group of 1024 threads.
__global__ void __launch_bounds__(1024) k_argmax(const float *__restrict__ l, int64_t n, uint32_t *__restrict__ out,
                                                 int32_t *pos_dev, int32_t advance) {
  __shared__ float bv[16];
  __shared__ int64_t bi[16];
  float v = -INFINITY;
  int64_t idx = -1;
  // each thread scans its values in ascending index order and keeps the first
  // largest: 16-byte pieces j = tid + 1024u (values 4j..4j+3), U4 pieces
  // loaded before any is compared, then the values past the last whole piece
  constexpr int U4 = 16;
  const int64_t n4 = (((uintptr_t)l & 15) == 0) ? n / 4 : 0;
  for (int64_t j0 = threadIdx.x; j0 < n4; j0 += 1024 * U4) {
    float4 xs[U4];
#pragma unroll
    for (int u = 0; u < U4; ++u) {
      const int64_t j = j0 + (int64_t)u * 1024;
      const float q = __builtin_nanf("");
      xs[u] = j < n4 ? ((const float4 *)l)[j] : make_float4(q, q, q, q);
    }
#pragma unroll
    for (int u = 0; u < U4; ++u) {
      const float xv[4] = {xs[u].x, xs[u].y, xs[u].z, xs[u].w};
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float x = xv[c];
        if (!isnan(x) && (idx < 0 || x > v)) {
          v = x;
          idx = 4 * (j0 + (int64_t)u * 1024) + c;
        }
      }
    }
  }
  for (int64_t i = 4 * n4 + threadIdx.x; i < n; i += 1024) {
    const float x = l[i];
    if (!isnan(x) && (idx < 0 || x > v)) {
      v = x;
      idx = i;
    }
  }
  // wave reduction: larger value wins, equal values keep the smaller index
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off);
    const int64_t oi = __shfl_xor(idx, off);
    if (oi >= 0 && (idx < 0 || ov > v || (ov == v && oi < idx))) {
      v = ov;
      idx = oi;
    }
  }
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    bv[w] = v;
    bi[w] = idx;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float V = bv[0];
    int64_t I = bi[0];
    for (int k = 1; k < 16; ++k)
      if (bi[k] >= 0 && (I < 0 || bv[k] > V || (bv[k] == V && bi[k] < I))) {
        V = bv[k];
        I = bi[k];
      }
    if (n > 0 && isnan(l[0])) I = 0;
    out[0] = (uint32_t)(I < 0 ? 0 : I);
    if (pos_dev) pos_dev[0] += advance;
  }
}

__global__ void k_pos_advance(int32_t *pos_dev, int32_t by) {
  if (threadIdx.x == 0) pos_dev[0] += by;
}

inline unsigned blocks(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

hipError_t launch_get_rows(hipStream_t st, int t, const uint8_t *table, int64_t row_bytes, int64_t n_rows,
                           int64_t cols, const uint32_t *ids, int64_t s_rows, float *out) {
  if (s_rows <= 0 || cols <= 0) return hipSuccess;
  KMOE_LAUNCH(k_get_rows, dim3(blocks(cols, 256), (unsigned)s_rows), dim3(256), 0, st, t, table, row_bytes, n_rows,
              cols, ids, out);
  return hipGetLastError();
}

// The register-resident kernel applies: dim % 4 == 0, dim <= 8192, 16-byte
// aligned rows, and the quantization's block size divides dim.
static bool rmsnorm_regs_ok(const void *x, const void *y, const void *w, const void *out, int64_t dim, int qt) {
  if (dim % 4 || dim > 8192 || dim < 4) return false;
  if ((((uintptr_t)x | (uintptr_t)y | (uintptr_t)w | (uintptr_t)out) & 15) != 0) return false;
  if (qt == 1 && dim % 256) return false;
  if (qt == 2 && dim % 32) return false;
  return true;
}

template <int QT>
static hipError_t launch_rmsnorm_regs(hipStream_t st, float *x, const float *y, const float *w, int64_t rows,
                                      int64_t dim, float eps, float *out, int8_t *q, float *qd, int32_t *qs) {
  const int nch = (int)((dim / 4 + 255) / 256);
  const dim3 g((unsigned)rows), b(256);
  if (nch <= 1) KMOE_LAUNCH((k_rmsnorm_regs<1, QT>), g, b, 0, st, x, y, w, dim, eps, out, q, qd, qs);
  else if (nch <= 2) KMOE_LAUNCH((k_rmsnorm_regs<2, QT>), g, b, 0, st, x, y, w, dim, eps, out, q, qd, qs);
  else if (nch <= 4) KMOE_LAUNCH((k_rmsnorm_regs<4, QT>), g, b, 0, st, x, y, w, dim, eps, out, q, qd, qs);
  else KMOE_LAUNCH((k_rmsnorm_regs<8, QT>), g, b, 0, st, x, y, w, dim, eps, out, q, qd, qs);
  return hipGetLastError();
}

hipError_t launch_add_rmsnorm(hipStream_t st, float *x, const float *y, const float *w, int64_t rows, int64_t dim,
                              float eps, float *out) {
  if (rows <= 0) return hipSuccess;
  if (rmsnorm_regs_ok(x, y, w, out, dim, 0))
    return launch_rmsnorm_regs<0>(st, x, y, w, rows, dim, eps, out, nullptr, nullptr, nullptr);
  KMOE_LAUNCH(k_add_rmsnorm, dim3((unsigned)rows), dim3(256), 0, st, x, y, w, dim, eps, out);
  return hipGetLastError();
}

hipError_t launch_rmsnorm_quant(hipStream_t st, float *x, const float *y, const float *w, int64_t rows, int64_t dim,
                                float eps, float *out, bool q8k, int8_t *q, float *qd, int32_t *qs) {
  if (rows <= 0) return hipSuccess;
  if (!rmsnorm_regs_ok(x, y, w, out, dim, q8k ? 1 : 2)) return hipErrorNotSupported;
  if (q8k) return launch_rmsnorm_regs<1>(st, x, y, w, rows, dim, eps, out, q, qd, qs);
  return launch_rmsnorm_regs<2>(st, x, y, w, rows, dim, eps, out, q, qd, qs);
}

hipError_t launch_rope(hipStream_t st, float *x, int64_t s_rows, int n_heads, int hd, int rd, int64_t pos0,
                       const int32_t *pos_dev, const float *inv_freq, int neox) {
  const int64_t n = s_rows * (rd / 2);
  if (n <= 0) return hipSuccess;
  KMOE_LAUNCH(k_rope, dim3(blocks(n, 256)), dim3(256), 0, st, x, s_rows, n_heads, hd, rd, pos0, pos_dev, inv_freq,
              neox);
  return hipGetLastError();
}

hipError_t launch_kv_store(hipStream_t st, const float *k, const float *v, int64_t s_rows, int64_t kvw,
                           int64_t pos0, const int32_t *pos_dev, int64_t n_ctx, uint16_t *kc, uint16_t *vc) {
  const int64_t n = s_rows * kvw;
  if (n <= 0) return hipSuccess;
  KMOE_LAUNCH(k_kv_store, dim3(blocks(n, 256)), dim3(256), 0, st, k, v, s_rows, kvw, pos0, pos_dev, n_ctx, kc, vc);
  return hipGetLastError();
}

int attn_supers(int64_t n_max) { return (int)((n_max + kAttnChunk - 1) / kAttnChunk); }

int64_t attn_part_floats(int64_t s_rows, int nh, int hd, int supers) {
  return supers <= 1 ? 0 : s_rows * nh * (int64_t)supers * (hd + 2);
}

bool attn_supported(int hd, int group) { return (hd == 64 || hd == 128) && group >= 1 && group <= kMaxGroup; }

hipError_t launch_attention(hipStream_t st, const float *q, const uint16_t *kc, const uint16_t *vc, int64_t s_rows,
                            int nh, int nkv, int hd, int64_t pos0, const int32_t *pos_dev, int64_t n_ctx, int supers,
                            float *part, uint32_t *counters, float *out, int qt, int8_t *xq, float *xd,
                            int32_t *xs) {
  if (s_rows <= 0) return hipSuccess;
  if (s_rows == 1) {  // decode
    if (qt == 1) return hipErrorNotSupported;  // a work-group per head writes no Q8_K blocks
    const unsigned g1 = (unsigned)((int64_t)nh * supers);
    if (hd == 64)
      KMOE_LAUNCH(k_attn_one<64>, dim3(g1), dim3(256), 0, st, q, kc, vc, nh, nkv, pos0, pos_dev, n_ctx, supers, part,
                  counters, out, qt, xq, xd, xs);
    else if (hd == 128)
      KMOE_LAUNCH(k_attn_one<128>, dim3(g1), dim3(256), 0, st, q, kc, vc, nh, nkv, pos0, pos_dev, n_ctx, supers, part,
                  counters, out, qt, xq, xd, xs);
    else
      return hipErrorInvalidValue;
    return hipGetLastError();
  }
  if (qt == 1 && ((nh / nkv) * hd) % 256 != 0) return hipErrorNotSupported;
  const unsigned grid = (unsigned)((int64_t)nkv * s_rows * supers);
  if (hd == 64)
    KMOE_LAUNCH(k_attn_dec<64>, dim3(grid), dim3(256), 0, st, q, kc, vc, s_rows, nh, nkv, pos0, pos_dev, n_ctx,
                supers, part, counters, out, qt, xq, xd, xs);
  else if (hd == 128)
    KMOE_LAUNCH(k_attn_dec<128>, dim3(grid), dim3(256), 0, st, q, kc, vc, s_rows, nh, nkv, pos0, pos_dev, n_ctx,
                supers, part, counters, out, qt, xq, xd, xs);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_rope_kv(hipStream_t st, const float *q, const float *k, const float *v, int64_t s_rows, int nh,
                          int nkv, int hd, int rd, int64_t pos0, const int32_t *pos_dev, const float *inv_freq,
                          int neox, int64_t n_ctx, float *q_out, uint16_t *kc, uint16_t *vc) {
  if (s_rows <= 0) return hipSuccess;
  const unsigned gy = (unsigned)((nh + nkv + kRopeHeads - 1) / kRopeHeads);
  KMOE_LAUNCH(k_rope_kv, dim3((unsigned)s_rows, gy), dim3(256), 0, st, q, k, v, nh, nkv, hd, rd, pos0, pos_dev,
              inv_freq, neox, n_ctx, q_out, kc, vc);
  return hipGetLastError();
}

hipError_t launch_swiglu(hipStream_t st, const float *g, const float *u, int64_t n, float *out) {
  if (n <= 0) return hipSuccess;
  KMOE_LAUNCH(k_swiglu, dim3(blocks(n, 256)), dim3(256), 0, st, g, u, n, out);
  return hipGetLastError();
}

hipError_t launch_add_rows(hipStream_t st, float *x, const float *b, int64_t rows, int64_t cols) {
  if (rows * cols <= 0) return hipSuccess;
  KMOE_LAUNCH(k_add_rows, dim3(blocks(rows * cols, 256)), dim3(256), 0, st, x, b, rows, cols);
  return hipGetLastError();
}

hipError_t launch_argmax(hipStream_t st, const float *l, int64_t n, uint32_t *out, int32_t *pos_dev,
                         int32_t advance) {
  KMOE_LAUNCH(k_argmax, dim3(1), dim3(1024), 0, st, l, n, out, pos_dev, advance);
  return hipGetLastError();
}

hipError_t launch_pos_advance(hipStream_t st, int32_t *pos_dev, int32_t by) {
  KMOE_LAUNCH(k_pos_advance, dim3(1), dim3(64), 0, st, pos_dev, by);
  return hipGetLastError();
}

}  // namespace kmoe
