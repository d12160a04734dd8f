// kmoe_tq4.h — one Q4_K quarter-superblock task against a Q8_K activation
// slice held in registers (the decode kernels over tiled rows).
#pragma once

#include "kmoe_device.h"

namespace kmoe {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct Slice {
  int4 x0, x1, x2, x3;  // 64 activation bytes: elements 64k .. 64k+63 of superblock sb
  int bsA, bsB;         // sums of the 32-element halves (sub-blocks 2k, 2k+1)
  float d;              // block scale
};

__device__ __forceinline__ int q4k_quarter(const u32x4 &hd, const u32x4 &qa, const u32x4 &qb, int k, const Slice &s,
                                           int &mins) {
  int sA, mA, sB, mB;
  q4k_scale_min_pair(hd.y, hd.z, hd.w, k, sA, mA, sB, mB);
  const uint32_t m = 0x0f0f0f0fu;
  int lo = 0, hi = 0;
  lo = sdot4(qa.x & m, (uint32_t)s.x0.x, lo);
  lo = sdot4(qa.y & m, (uint32_t)s.x0.y, lo);
  lo = sdot4(qa.z & m, (uint32_t)s.x0.z, lo);
  lo = sdot4(qa.w & m, (uint32_t)s.x0.w, lo);
  lo = sdot4(qb.x & m, (uint32_t)s.x1.x, lo);
  lo = sdot4(qb.y & m, (uint32_t)s.x1.y, lo);
  lo = sdot4(qb.z & m, (uint32_t)s.x1.z, lo);
  lo = sdot4(qb.w & m, (uint32_t)s.x1.w, lo);
  hi = sdot4((qa.x >> 4) & m, (uint32_t)s.x2.x, hi);
  hi = sdot4((qa.y >> 4) & m, (uint32_t)s.x2.y, hi);
  hi = sdot4((qa.z >> 4) & m, (uint32_t)s.x2.z, hi);
  hi = sdot4((qa.w >> 4) & m, (uint32_t)s.x2.w, hi);
  hi = sdot4((qb.x >> 4) & m, (uint32_t)s.x3.x, hi);
  hi = sdot4((qb.y >> 4) & m, (uint32_t)s.x3.y, hi);
  hi = sdot4((qb.z >> 4) & m, (uint32_t)s.x3.z, hi);
  hi = sdot4((qb.w >> 4) & m, (uint32_t)s.x3.w, hi);
  mins = mA * s.bsA + mB * s.bsB;
  return sA * lo + sB * hi;
}

}  // namespace kmoe
