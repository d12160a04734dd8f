// kmoe_xtypes.hip — quant::matmul (quant.rs:229-328) for the other weight
// types the reference accepts: F16, BF16, Q4_0, Q4_1, Q5_0, Q5_1 and Q5_K.
//
// f32 regime (s_rows >= 4 on the AVX2 path, every row in the exact regime,
// F16/BF16 always): the weights are dequantized with dequant_row's own
// arithmetic (quant.rs:63-205) into an f32 matrix, which then takes the F32
// weights' kernel: the same summation orders (gemm_f32 / dot_f32 /
// quant::dot) as the reference, so the results are the reference's bits.
//
// int8 regime (Q8 activation rows, qdot.rs:30-49): qdot::unpack (qdot.rs:
// 74-200) and the AVX2 dot of an unpacked row with a Q8 row (avx2.rs:151-164),
// or for Q4_0 the fused dot_q4_0 (avx2.rs:61-75), replayed exactly: per
// 32-block the eight 4-element integer sums of mul_i8_i8 (lane l: elements
// 4l..4l+3) are converted to f32 and fused-multiply-added into eight chains
// with scale[2b] * d_x (lanes 0-3) or scale[2b+1] * d_x (lanes 4-7); the
// minimum terms run as one ordered chain; hsum of the chains, minus the mins.
#include "kmoe_device.h"
#include "kmoe_launch.h"

namespace kmoe {

namespace {

enum { X_F16 = 1, X_Q4_0 = 2, X_Q4_1 = 3, X_Q5_0 = 6, X_Q5_1 = 7, X_Q5_K = 13, X_BF16 = 30 };

__device__ __forceinline__ float f16at(const uint8_t *p) {
  return f16_bits_to_f32((uint32_t)p[0] | ((uint32_t)p[1] << 8));
}
__device__ __forceinline__ uint32_t le32(const uint8_t *p) {
  return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24);
}

template <int T>
struct XT;
template <>
struct XT<X_Q4_0> {
  static constexpr int EL = 32, BYTES = 18;
};
template <>
struct XT<X_Q4_1> {
  static constexpr int EL = 32, BYTES = 20;
};
template <>
struct XT<X_Q5_0> {
  static constexpr int EL = 32, BYTES = 22;
};
template <>
struct XT<X_Q5_1> {
  static constexpr int EL = 32, BYTES = 24;
};
template <>
struct XT<X_Q5_K> {
  static constexpr int EL = 256, BYTES = 176;
};

// scale_min_k4 (quant.rs:54-61)
__device__ __forceinline__ void scale_min_k4(int j, const uint8_t *q, int &sc, int &mn) {
  if (j < 4) {
    sc = q[j] & 63;
    mn = q[j + 4] & 63;
  } else {
    sc = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
    mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
  }
}

// One 32-element block b of a row as qdot::unpack leaves it: the integers of
// elements 4l..4l+3 and the block's 16-group scale and minimum (the same for
// both 16-groups of a 32-block in these types).
template <int T>
struct Blk32 {
  int q[4];
  float sc, mn;  // qdot::unpack's scale and min (min = -m for Q4_1 / Q5_1)
};

template <int T>
__device__ __forceinline__ Blk32<T> blk32(const uint8_t *row, int64_t b, int l) {
  Blk32<T> r;
  if constexpr (T == X_Q5_K) {
    const uint8_t *blk = row + (b >> 3) * 176;
    const int j = (int)(b & 7), k = j >> 1;
    const float d = f16at(blk), dmin = f16at(blk + 2);
    int s, m;
    scale_min_k4(j, blk + 4, s, m);
    r.sc = d * (float)s;
    r.mn = dmin * (float)m;
    const uint8_t *qh = blk + 16, *ql = blk + 48 + 32 * k;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * l + i;
      const int nib = (j & 1) ? (ql[e] >> 4) : (ql[e] & 0xF);
      r.q[i] = nib | (((qh[e] >> j) & 1) << 4);
    }
  } else {
    const uint8_t *blk = row + b * XT<T>::BYTES;
    const float d = f16at(blk);
    r.sc = d;
    r.mn = 0.0f;
    if constexpr (T == X_Q4_1 || T == X_Q5_1) r.mn = -f16at(blk + 2);
    constexpr int QH = T == X_Q5_0 ? 2 : (T == X_Q5_1 ? 4 : -1);
    constexpr int QS = T == X_Q4_0 ? 2 : (T == X_Q4_1 ? 4 : (T == X_Q5_0 ? 6 : 8));
    constexpr int BIAS = T == X_Q4_0 ? 8 : (T == X_Q5_0 ? 16 : 0);
    uint32_t qh = 0;
    if constexpr (QH >= 0) qh = le32(blk + QH);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * l + i;  // element of the block
      const uint8_t byte = blk[QS + (e & 15)];
      int v = e < 16 ? (byte & 0xF) : (byte >> 4);
      if constexpr (QH >= 0) v |= (int)((qh >> e) & 1u) << 4;  // bit e of qh is bit 4 of element e
      r.q[i] = v - BIAS;
    }
  }
  return r;
}

// dequant_row's values of block b (32 elements), for elements 4l..4l+3.
template <int T>
__device__ __forceinline__ void deq32(const uint8_t *row, int64_t b, int l, float (&y)[4]) {
  if constexpr (T == X_Q5_K) {
    const uint8_t *blk = row + (b >> 3) * 176;
    const int j = (int)(b & 7), k = j >> 1;
    const float d = f16at(blk), dmin = f16at(blk + 2);
    int s, m;
    scale_min_k4(j, blk + 4, s, m);
    const float d1 = d * (float)s, m1 = dmin * (float)m;  // quant.rs:165-166
    const uint8_t *qh = blk + 16, *ql = blk + 48 + 32 * k;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * l + i;
      const int nib = (j & 1) ? (ql[e] >> 4) : (ql[e] & 0xF);
      const int hi = ((qh[e] >> j) & 1) ? 16 : 0;
      const float t = d1 * (float)(nib + hi);
      y[i] = t - m1;
    }
  } else {
    const uint8_t *blk = row + b * XT<T>::BYTES;
    const float d = f16at(blk);
    float m = 0.0f;
    if constexpr (T == X_Q4_1 || T == X_Q5_1) m = f16at(blk + 2);
    constexpr int QH = T == X_Q5_0 ? 2 : (T == X_Q5_1 ? 4 : -1);
    constexpr int QS = T == X_Q4_0 ? 2 : (T == X_Q4_1 ? 4 : (T == X_Q5_0 ? 6 : 8));
    uint32_t qh = 0;
    if constexpr (QH >= 0) qh = le32(blk + QH);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int e = 4 * l + i;
      const uint8_t byte = blk[QS + (e & 15)];
      int v = e < 16 ? (byte & 0xF) : (byte >> 4);
      if constexpr (QH >= 0) v |= (int)((qh >> e) & 1u) << 4;
      if constexpr (T == X_Q4_0) {
        y[i] = (float)(v - 8) * d;  // quant.rs:95-96
      } else if constexpr (T == X_Q5_0) {
        y[i] = (float)(v - 16) * d;  // quant.rs:119-120
      } else {  // Q4_1 / Q5_1: q * d + m (quant.rs:107-108, :133-134)
        const float t = (float)v * d;
        y[i] = t + m;
      }
    }
  }
}

// out[r, c] = dequant_row(t, row r)[c] (quant.rs:63-205): the quantized types
// one thread per 4 elements of a 32-block, F16 / BF16 one per element.
template <int T>
__global__ void __launch_bounds__(256) k_dequant_x(const uint8_t *__restrict__ w, int64_t rows, int64_t cols,
                                                   int64_t row_bytes, float *__restrict__ out) {
  if constexpr (T == X_F16 || T == X_BF16) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < rows * cols; i += (int64_t)gridDim.x * 256) {
      const int64_t r = i / cols, c = i % cols;
      const uint8_t *p = w + r * row_bytes + 2 * c;
      const uint32_t h = (uint32_t)p[0] | ((uint32_t)p[1] << 8);
      out[i] = T == X_F16 ? f16_bits_to_f32(h) : __builtin_bit_cast(float, h << 16);  // quant.rs:72-81
    }
  } else {
    const int64_t n4 = cols / 4;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < rows * n4; i += (int64_t)gridDim.x * 256) {
      const int64_t r = i / n4, c4 = i % n4;
      float y[4];
      deq32<T>(w + r * row_bytes, (4 * c4) / 32, (int)((4 * c4) % 32) / 4, y);
      *(float4 *)(out + r * cols + 4 * c4) = make_float4(y[0], y[1], y[2], y[3]);
    }
  }
}

// out[s, r] = dot_unpacked(row r, Q8 row s) (dot_q4_0 for Q4_0). Eight lanes
// per (row, token): lane l runs chain l over the blocks in order.
template <int T>
__global__ void __launch_bounds__(256) k_mv_unpacked(const uint8_t *__restrict__ w, int64_t rows, int64_t cols,
                                                     int64_t row_bytes, const int8_t *__restrict__ xq,
                                                     const float *__restrict__ xd, const int32_t *__restrict__ s16,
                                                     int64_t s_rows, float *__restrict__ out) {
  const int l = threadIdx.x & 7;
  const int64_t pair = ((int64_t)blockIdx.x * 256 + threadIdx.x) >> 3;  // (row, token) pairs, token fastest
  if (pair >= rows * s_rows) return;  // whole groups of 8 leave together
  const int64_t r = pair / s_rows, s = pair % s_rows;
  const uint8_t *row = w + r * row_bytes;
  const int64_t nb = cols / 32;
  const int8_t *xs = xq + s * cols;
  const float *ds = xd + s * nb;
  const int32_t *ss = s16 + s * (cols / 16);
  float acc = 0.0f, mins = 0.0f;
  for (int64_t b = 0; b < nb; ++b) {
    const Blk32<T> u = blk32<T>(row, b, l);
    const uint32_t xv = *(const uint32_t *)(xs + 32 * b + 4 * l);
    int p = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) p += u.q[i] * (int)(int8_t)(xv >> (8 * i));
    const float ad = ds[b];
    const float sc = u.sc * ad;  // scale[2b] * d_x (lanes 0-3), scale[2b+1] * d_x (lanes 4-7): equal here
    acc = fmaf((float)p, sc, acc);
    if constexpr (T != X_Q4_0) {  // mins += d_x * (min[2b] * s16[2b] + min[2b+1] * s16[2b+1])
      const float t1 = u.mn * (float)ss[2 * b];
      const float t2 = u.mn * (float)ss[2 * b + 1];
      const float t = t1 + t2;
      mins = mins + ad * t;
    }
  }
  // hsum (avx2.rs:20-27): ((v0+v4)+(v2+v6)) + ((v1+v5)+(v3+v7))
  float v = acc;
  v = v + __shfl_xor(v, 4);
  v = v + __shfl_xor(v, 2);
  v = v + __shfl_xor(v, 1);
  if (l == 0) out[s * rows + r] = T == X_Q4_0 ? v : v - mins;
}

}  // namespace

bool xtype(int t) {
  return t == X_F16 || t == X_BF16 || t == X_Q4_0 || t == X_Q4_1 || t == X_Q5_0 || t == X_Q5_1 || t == X_Q5_K;
}

hipError_t launch_dequant_x(hipStream_t st, int t, const uint8_t *w, int64_t rows, int64_t cols, int64_t row_bytes,
                            float *out) {
  if (rows == 0) return hipSuccess;
  const bool flt = t == X_F16 || t == X_BF16;
  if (!flt && (cols % 32 || ((uintptr_t)out & 15))) return hipErrorInvalidValue;
  const int64_t n = flt ? rows * cols : rows * (cols / 4);
  const unsigned grid = (unsigned)((n + 255) / 256 < 65536 ? (n + 255) / 256 : 65536);
  switch (t) {
    case X_F16: KMOE_LAUNCH(k_dequant_x<X_F16>, dim3(grid), dim3(256), 0, st, w, rows, cols, row_bytes, out); break;
    case X_BF16: KMOE_LAUNCH(k_dequant_x<X_BF16>, dim3(grid), dim3(256), 0, st, w, rows, cols, row_bytes, out); break;
    case X_Q4_0: KMOE_LAUNCH(k_dequant_x<X_Q4_0>, dim3(grid), dim3(256), 0, st, w, rows, cols, row_bytes, out); break;
    case X_Q4_1: KMOE_LAUNCH(k_dequant_x<X_Q4_1>, dim3(grid), dim3(256), 0, st, w, rows, cols, row_bytes, out); break;
    case X_Q5_0: KMOE_LAUNCH(k_dequant_x<X_Q5_0>, dim3(grid), dim3(256), 0, st, w, rows, cols, row_bytes, out); break;
    case X_Q5_1: KMOE_LAUNCH(k_dequant_x<X_Q5_1>, dim3(grid), dim3(256), 0, st, w, rows, cols, row_bytes, out); break;
    case X_Q5_K: KMOE_LAUNCH(k_dequant_x<X_Q5_K>, dim3(grid), dim3(256), 0, st, w, rows, cols, row_bytes, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_mv_unpacked(hipStream_t st, int t, const uint8_t *w, int64_t rows, int64_t cols,
                              int64_t row_bytes, const int8_t *xq, const float *xd, const int32_t *s16, int64_t s_rows,
                              float *out) {
  if (rows == 0 || s_rows == 0) return hipSuccess;
  if (cols % 32 || ((uintptr_t)xq & 3)) return hipErrorInvalidValue;
  const int64_t threads = rows * s_rows * 8;
  const int64_t blocks = (threads + 255) / 256;
  if (blocks > (int64_t)UINT32_MAX) return hipErrorInvalidValue;
  const dim3 g((unsigned)blocks);
  switch (t) {
    case X_Q4_0: KMOE_LAUNCH(k_mv_unpacked<X_Q4_0>, g, dim3(256), 0, st, w, rows, cols, row_bytes, xq, xd, s16, s_rows, out); break;
    case X_Q4_1: KMOE_LAUNCH(k_mv_unpacked<X_Q4_1>, g, dim3(256), 0, st, w, rows, cols, row_bytes, xq, xd, s16, s_rows, out); break;
    case X_Q5_0: KMOE_LAUNCH(k_mv_unpacked<X_Q5_0>, g, dim3(256), 0, st, w, rows, cols, row_bytes, xq, xd, s16, s_rows, out); break;
    case X_Q5_1: KMOE_LAUNCH(k_mv_unpacked<X_Q5_1>, g, dim3(256), 0, st, w, rows, cols, row_bytes, xq, xd, s16, s_rows, out); break;
    case X_Q5_K: KMOE_LAUNCH(k_mv_unpacked<X_Q5_K>, g, dim3(256), 0, st, w, rows, cols, row_bytes, xq, xd, s16, s_rows, out); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

}  // namespace kmoe
