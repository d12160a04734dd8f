// kmoe_logit.h — one router logit per work-group in quant::dot order
// (the single-token router of the decode path).
#pragma once

#include "kmoe_device.h"

namespace kmoe {

constexpr int kDecMaxD = 8192;  // columns whose products one work-group holds in LDS
// LDS floats wg_logit needs for rows of up to kDecMaxD columns
constexpr int kLogitLds = 8 * (kDecMaxD / 8 + 8);

// The first 8*(d/8) columns of router row w as float4 groups q = tid + 256*v
// (zero past nq = d/4 groups), kept in registers.
template <int NV>
__device__ __forceinline__ void logit_row_load(const float *w, int nq, bool vec, float4 (&wv)[NV], int tid) {
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int q = tid + 256 * v;
    wv[v] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (q < nq) wv[v] = vec ? *(const float4 *)(w + 4 * q)
                            : make_float4(w[4 * q], w[4 * q + 1], w[4 * q + 2], w[4 * q + 3]);
  }
}

// logit = quant::dot(w, x) (quant.rs:208-224): eight strided partial sums of
// products over the first 8*(d/8) columns, each an ordered chain, folded in
// lane order, then the remaining columns in order. The work-group (256
// threads) writes the products into T (LDS, kLogitLds floats) and lanes 0..7
// of wave 0 run the chains with their LDS reads two stages ahead; waves 1..3
// call spare(wave) meanwhile. The caller synchronizes before reusing T. The
// logit is returned in thread 0.
// xat(v, q) gives x's float4 group q = tid + 256*v (from memory, or from
// registers when the caller computed x); x itself is read only for the
// d % 8 tail columns.
template <int NV, class XAt, class Spare>
__device__ __forceinline__ float wg_logit_at(const float4 (&wv)[NV], const float *w, XAt &&xat, const float *x,
                                             int64_t d, float *T, Spare &&spare) {
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t n8 = d / 8;
  const int cstr = (int)(((n8 + 3) & ~3ll) + 4);
  const int nq = (int)(2 * n8);
#pragma unroll
  for (int v = 0; v < NV; ++v) {
    const int q = tid + 256 * v;
    if (q < nq) {
      const float4 xv = xat(v, q);
      float *dst = T + (4 * (q & 1)) * cstr + (q >> 1);
      dst[0 * cstr] = wv[v].x * xv.x;
      dst[1 * cstr] = wv[v].y * xv.y;
      dst[2 * cstr] = wv[v].z * xv.z;
      dst[3 * cstr] = wv[v].w * xv.w;
    }
  }
  __syncthreads();
  float r = -0.0f;
  if (wave == 0) {
    float acc = 0.0f;
    if (lane < 8) {
      const float *row = T + lane * cstr;
      const int nst = (int)(n8 / 32);
      float4 A[8], B[8];
      auto ld = [&](float4 (&R)[8], int st) {
#pragma unroll
        for (int i = 0; i < 8; ++i) R[i] = *(const float4 *)(row + 32 * st + 4 * i);
      };
      auto add = [&](const float4 (&R)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          acc = acc + R[i].x;
          acc = acc + R[i].y;
          acc = acc + R[i].z;
          acc = acc + R[i].w;
        }
      };
      if (nst > 0) {
        // two register stages, the next one's LDS reads in flight while
        // the current one is added (no branches inside the loop body)
        ld(A, 0);
        int st = 0;
        for (; st + 2 < nst; st += 2) {
          ld(B, st + 1);
          add(A);
          ld(A, st + 2);
          add(B);
        }
        if (st + 1 < nst) {
          ld(B, st + 1);
          add(A);
          add(B);
        } else {
          add(A);
        }
      }
      for (int64_t c = (int64_t)nst * 32; c < n8; ++c) acc = acc + row[c];
    }
#pragma unroll
    for (int l = 0; l < 8; ++l) r = r + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), l));
    if (lane == 0) {
      for (int64_t c = n8 * 8; c < d; ++c) {
        const float pr = w[c] * x[c];
        r = r + pr;
      }
    }
  } else {
    spare(wave);
  }
  return r;
}

template <int NV, class Spare>
__device__ __forceinline__ float wg_logit(const float4 (&wv)[NV], const float *w, const float *x, int64_t d, bool vec,
                                          float *T, Spare &&spare) {
  auto xat = [&](int, int q) {
    return vec ? *(const float4 *)(x + 4 * q) : make_float4(x[4 * q], x[4 * q + 1], x[4 * q + 2], x[4 * q + 3]);
  };
  return wg_logit_at<NV>(wv, w, xat, x, d, T, spare);
}

}  // namespace kmoe
