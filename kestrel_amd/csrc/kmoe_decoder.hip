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

// Work-group sum of 256 threads, every thread receives the total. The order
// (per-thread strided partials, wave DPP tree, then four wave sums in order)
// is fixed, so results repeat exactly.
__device__ __forceinline__ float wg_sum256(float v, float *red) {
  v = group_sum<64>(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return ((red[0] + red[1]) + red[2]) + red[3];
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

__device__ __forceinline__ int64_t position(int64_t pos0, const int32_t *pos_dev) {
  return pos0 + (pos_dev ? (int64_t)*pos_dev : 0);
}

// Transformer::rope (transformer.rs:342-358), in place: one thread per
// (row, pair); sin and cos of the f32 angle are rounded from double
// precision (glibc's sinf/cosf are correctly rounded up to rare midpoints).
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
  const float sn = (float)sin((double)ang), cs = (float)cos((double)ang);
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
// Causal GQA attention (Transformer::attention, transformer.rs:591-631) as a
// split softmax over chunks of 64 cache positions.
//
// Work-group (kv head g, query row s, chunk c) stages the chunk's K and V
// rows (f16) in LDS, then each wave takes query heads of the group: lane l
// scores position 64c + l with quant::dot's eight-accumulator order
// (quant.rs:208-224) times 1/sqrt(hd), the wave takes the chunk's max m and
// e_p = exp(score - m), and lanes over head dims accumulate sum_p e_p V[p].
// The partial (m, sum e, acc) goes to the workspace; k_attn_combine merges
// the chunks of a (row, head): out = sum_c acc_c e^(m_c - M) / sum_c l_c e^(m_c - M).
constexpr int kAttnChunk = 64;

template <int HD>
__global__ void __launch_bounds__(256) k_attn_chunk(const float *__restrict__ q, const uint16_t *__restrict__ kc,
                                                    const uint16_t *__restrict__ vc, int64_t s_rows, int nh,
                                                    int nkv, int64_t pos0, const int32_t *__restrict__ pos_dev,
                                                    int64_t n_ctx, int chunks, float *__restrict__ part) {
  constexpr int RW = HD / 2 + 1;  // LDS row stride in dwords (odd: conflict-free column reads)
  __shared__ uint32_t Ks[kAttnChunk * RW];
  __shared__ uint32_t Vs[kAttnChunk * RW];
  __shared__ float Qs[4][HD];
  __shared__ float Ps[4][kAttnChunk];
  const int64_t bid = blockIdx.x;
  const int c = (int)(bid % chunks);
  const int64_t s = (bid / chunks) % s_rows;
  const int g = (int)(bid / chunks / s_rows);
  int64_t n = position(pos0, pos_dev) + s + 1;
  if (n > n_ctx) n = n_ctx;
  const int64_t p0 = (int64_t)c * kAttnChunk;
  if (p0 >= n) return;
  const int np = (int)(n - p0 < kAttnChunk ? n - p0 : kAttnChunk);
  const int64_t kvw = (int64_t)nkv * HD;
  // stage K and V rows [p0, p0 + np) of head g: HD/2 dwords per row
  for (int e = threadIdx.x; e < np * (HD / 2); e += 256) {
    const int r = e / (HD / 2), w = e % (HD / 2);
    const int64_t off = (p0 + r) * kvw + (int64_t)g * HD;
    Ks[r * RW + w] = ((const uint32_t *)(kc + off))[w];
    Vs[r * RW + w] = ((const uint32_t *)(vc + off))[w];
  }
  const int group = nh / nkv;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const float scale = 1.0f / sqrtf((float)HD);
  __syncthreads();
  for (int hh0 = 0; hh0 < group; hh0 += 4) {
    const int hh = hh0 + wave;
    const bool on = hh < group;
    const int h = g * group + hh;
    if (on)
      for (int j = lane; j < HD; j += 64) Qs[wave][j] = q[(s * nh + h) * (int64_t)HD + j];
    __syncthreads();
    if (on) {
      float sc = -INFINITY;
      if (lane < np) {
        float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        const uint32_t *kr = Ks + lane * RW;
#pragma unroll 4
        for (int c8 = 0; c8 < HD; c8 += 8) {
#pragma unroll
          for (int i = 0; i < 8; i += 2) {
            const uint32_t kw = kr[(c8 + i) / 2];
            const float k0 = f16_bits_to_f32(kw), k1 = f16_bits_to_f32(kw >> 16);
            const float a0 = Qs[wave][c8 + i] * k0, a1 = Qs[wave][c8 + i + 1] * k1;
            acc[i] = acc[i] + a0;
            acc[i + 1] = acc[i + 1] + a1;
          }
        }
        float t = -0.0f;
#pragma unroll
        for (int i = 0; i < 8; ++i) t = t + acc[i];
        sc = t * scale;
      }
      const float m = group_max<64>(sc);
      const float e = lane < np ? expf(sc - m) : 0.0f;
      const float l = group_sum<64>(e);
      Ps[wave][lane] = e;
      // lanes over dims: lane owns HD/64 consecutive dims
      constexpr int DPL = HD / 64;
      float o[DPL];
#pragma unroll
      for (int i = 0; i < DPL; ++i) o[i] = 0.0f;
      __builtin_amdgcn_wave_barrier();
      for (int p = 0; p < np; ++p) {
        const float wgt = Ps[wave][p];
        const uint32_t *vr = Vs + p * RW;
        if constexpr (DPL == 1) {
          const uint32_t vw = vr[lane >> 1];
          o[0] += wgt * f16_bits_to_f32((lane & 1) ? (vw >> 16) : vw);
        } else {
#pragma unroll
          for (int i = 0; i < DPL; i += 2) {
            const uint32_t vw = vr[(lane * DPL + i) / 2];
            o[i] += wgt * f16_bits_to_f32(vw);
            o[i + 1] += wgt * f16_bits_to_f32(vw >> 16);
          }
        }
      }
      const int64_t pi = ((s * nh + h) * (int64_t)chunks + c);
      float *pp = part + pi * (HD + 2);
      if (lane == 0) {
        pp[0] = m;
        pp[1] = l;
      }
#pragma unroll
      for (int i = 0; i < DPL; ++i) pp[2 + lane * DPL + i] = o[i];
    }
    __syncthreads();
  }
}

template <int HD>
__global__ void __launch_bounds__(256) k_attn_combine(const float *__restrict__ part, int64_t s_rows, int nh,
                                                      int64_t pos0, const int32_t *__restrict__ pos_dev,
                                                      int64_t n_ctx, int chunks, float *__restrict__ out) {
  constexpr int DPL = HD / 64;
  const int64_t pair = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= s_rows * nh) return;
  const int lane = threadIdx.x & 63;
  const int64_t s = pair / nh;
  int64_t n = position(pos0, pos_dev) + s + 1;
  if (n > n_ctx) n = n_ctx;
  const int nc = (int)((n + kAttnChunk - 1) / kAttnChunk);
  const float *pp = part + pair * chunks * (HD + 2);
  float M = -INFINITY;
  for (int c = 0; c < nc; ++c) M = fmaxf(M, pp[c * (HD + 2)]);
  float L = 0.0f, o[DPL];
#pragma unroll
  for (int i = 0; i < DPL; ++i) o[i] = 0.0f;
  for (int c = 0; c < nc; ++c) {
    const float *pc = pp + c * (HD + 2);
    const float f = expf(pc[0] - M);
    L += pc[1] * f;
#pragma unroll
    for (int i = 0; i < DPL; ++i) o[i] += pc[2 + lane * DPL + i] * f;
  }
  const float inv = 1.0f / L;
#pragma unroll
  for (int i = 0; i < DPL; ++i) out[pair * HD + lane * DPL + i] = o[i] * inv;
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
  for (int64_t i = threadIdx.x; i < n; i += 1024) {
    const float x = l[i];
    if (!isnan(x) && (idx < 0 || x > v)) {  // strided scan: ascending i, first max kept
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

hipError_t launch_add_rmsnorm(hipStream_t st, float *x, const float *y, const float *w, int64_t rows, int64_t dim,
                              float eps, float *out) {
  if (rows <= 0) return hipSuccess;
  KMOE_LAUNCH(k_add_rmsnorm, dim3((unsigned)rows), dim3(256), 0, st, x, y, w, dim, eps, out);
  return hipGetLastError();
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

int attn_chunks(int64_t n_max) { return (int)((n_max + kAttnChunk - 1) / kAttnChunk); }

int64_t attn_part_floats(int64_t s_rows, int nh, int hd, int chunks) {
  return s_rows * nh * (int64_t)chunks * (hd + 2);
}

bool attn_supported_hd(int hd) { return hd == 64 || hd == 128; }

hipError_t launch_attention(hipStream_t st, const float *q, const uint16_t *kc, const uint16_t *vc, int64_t s_rows,
                            int nh, int nkv, int hd, int64_t pos0, const int32_t *pos_dev, int64_t n_ctx, int chunks,
                            float *part, float *out) {
  if (s_rows <= 0) return hipSuccess;
  const unsigned g1 = (unsigned)((int64_t)nkv * s_rows * chunks);
  const unsigned g2 = blocks(s_rows * nh, 4);
#define KMOE_ATTN(HD)                                                                                          \
  do {                                                                                                         \
    KMOE_LAUNCH(k_attn_chunk<HD>, dim3(g1), dim3(256), 0, st, q, kc, vc, s_rows, nh, nkv, pos0, pos_dev, n_ctx, \
                chunks, part);                                                                                 \
    KMOE_LAUNCH(k_attn_combine<HD>, dim3(g2), dim3(256), 0, st, part, s_rows, nh, pos0, pos_dev, n_ctx, chunks,  \
                out);                                                                                          \
  } while (0)
  switch (hd) {
    case 64: KMOE_ATTN(64); break;
    case 128: KMOE_ATTN(128); break;
    default: return hipErrorInvalidValue;
  }
#undef KMOE_ATTN
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
