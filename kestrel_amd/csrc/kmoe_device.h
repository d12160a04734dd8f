// kmoe_device.h — device helpers shared by the gfx950 kernels.
//
// Wave64 throughout. Cross-lane sums use DPP inside a 16-lane row
// (quad_perm xor1/xor2, row_half_mirror, row_mirror) and ds_swizzle/bpermute
// shuffles across rows. All float code is compiled with -ffp-contract=off:
// an FMA appears only where fmaf() is written.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kmoe {

constexpr int kWave = 64;

__device__ __forceinline__ float f16_bits_to_f32(uint32_t bits) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)(bits & 0xffffu));
}

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

// DPP controls (gfx9): quad_perm [1,0,3,2] = lane^1, [2,3,0,1] = lane^2,
// row_half_mirror (lane i <- 7-i within 8), row_mirror (lane i <- 15-i within 16).
constexpr int kDppXor1 = 0xb1;
constexpr int kDppXor2 = 0x4e;
constexpr int kDppHalfMirror = 0x141;
constexpr int kDppMirror = 0x140;

// Sum over aligned groups of W lanes (W in 1..64, power of two); every lane of
// the group receives the group sum.
template <int W>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (W >= 2) v += dpp_f<kDppXor1>(v);
  if constexpr (W >= 4) v += dpp_f<kDppXor2>(v);
  if constexpr (W >= 8) v += dpp_f<kDppHalfMirror>(v);
  if constexpr (W >= 16) v += dpp_f<kDppMirror>(v);
  if constexpr (W >= 32) v += __shfl_xor(v, 16);
  if constexpr (W >= 64) v += __shfl_xor(v, 32);
  return v;
}
template <int W>
__device__ __forceinline__ int group_sum_i(int v) {
  if constexpr (W >= 2) v += dpp_i<kDppXor1>(v);
  if constexpr (W >= 4) v += dpp_i<kDppXor2>(v);
  if constexpr (W >= 8) v += dpp_i<kDppHalfMirror>(v);
  if constexpr (W >= 16) v += dpp_i<kDppMirror>(v);
  if constexpr (W >= 32) v += __shfl_xor(v, 16);
  if constexpr (W >= 64) v += __shfl_xor(v, 32);
  return v;
}
// Max over groups of W lanes (exact in any order).
template <int W>
__device__ __forceinline__ float group_max(float v) {
  if constexpr (W >= 2) v = fmaxf(v, dpp_f<kDppXor1>(v));
  if constexpr (W >= 4) v = fmaxf(v, dpp_f<kDppXor2>(v));
  if constexpr (W >= 8) v = fmaxf(v, dpp_f<kDppHalfMirror>(v));
  if constexpr (W >= 16) v = fmaxf(v, dpp_f<kDppMirror>(v));
  if constexpr (W >= 32) v = fmaxf(v, __shfl_xor(v, 16));
  if constexpr (W >= 64) v = fmaxf(v, __shfl_xor(v, 32));
  return v;
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
  return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

__device__ __forceinline__ uint32_t byte_of(uint32_t w, int i) { return (w >> (8 * i)) & 0xffu; }

// scale_min_k4 (quant.rs:54-61) for sub-blocks j = 2k and 2k+1 of a Q4_K
// superblock whose 12 scale bytes are the little-endian words s03, s47, s811.
__device__ __forceinline__ void q4k_scale_min_pair(uint32_t s03, uint32_t s47, uint32_t s811, int k, int &sA,
                                                   int &mA, int &sB, int &mB) {
  // Branch-free: both forms are computed from byte index bi = 2*(k&1) and the
  // one for j = 2k (j < 4 or j >= 4) is selected, so lanes with different k
  // never diverge.
  const int bi = 2 * (k & 1);
  const bool hi = k >= 2;
  const uint32_t a0 = byte_of(s03, bi), a1 = byte_of(s03, bi + 1);
  const uint32_t b0 = byte_of(s47, bi), b1 = byte_of(s47, bi + 1);
  const uint32_t c0 = byte_of(s811, bi), c1 = byte_of(s811, bi + 1);
  sA = (int)(hi ? ((c0 & 0xfu) | ((a0 >> 6) << 4)) : (a0 & 63u));
  mA = (int)(hi ? ((c0 >> 4) | ((b0 >> 6) << 4)) : (b0 & 63u));
  sB = (int)(hi ? ((c1 & 0xfu) | ((a1 >> 6) << 4)) : (a1 & 63u));
  mB = (int)(hi ? ((c1 >> 4) | ((b1 >> 6) << 4)) : (b1 & 63u));
}

// Dword-aligned 16-byte load (global_load_dwordx4 accepts 4-byte alignment).
typedef uint32_t u32x4a4 __attribute__((ext_vector_type(4), aligned(4)));
__device__ __forceinline__ uint4 load_u4_a4(const void *p) {
  u32x4a4 v = *(const u32x4a4 *)p;
  return make_uint4(v.x, v.y, v.z, v.w);
}

// Work-group barrier ordering LDS only: unlike __syncthreads it does not wait
// for outstanding global loads, so loads issued for the next item stay in
// flight across it.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Tiled Q4_K rows: the expert tier's HBM layout for Q4_K parts. A row of nb
// superblocks keeps its 144*nb bytes, reordered:
//   [0, 16*nb)       the 16-byte head (f16 d, f16 dmin, 12 scale bytes) of
//                    superblock s at 16*s;
//   [16*nb, 144*nb)  the nibble bytes in groups of 8 superblocks: group g
//                    (superblocks 8g .. 8g+ns-1, ns = min(8, nb-8g)) starts at
//                    16*nb + 1024*g, and its 16-byte chunk j*4*ns + 4*sl + k
//                    holds nibble bytes [32k+16j, 32k+16j+16) of superblock 8g+sl.
// A wave whose lanes take consecutive (superblock, k) slots then reads each of
// its two nibble chunks from one or two contiguous 512-byte runs and its heads
// from one contiguous run, instead of touching every 144-byte superblock three
// times.
__host__ __device__ __forceinline__ int64_t tq4_qs_off(int64_t nb, int64_t sb, int k, int j) {
  const int64_t g = sb >> 3;
  const int64_t rem = nb - 8 * g;
  const int64_t ns = rem < 8 ? rem : 8;
  return 16 * nb + 1024 * g + 16 * (j * 4 * ns + 4 * (sb & 7) + k);
}
// Byte distance from chunk (sb, k, 0) to chunk (sb, k, 1).
__host__ __device__ __forceinline__ int64_t tq4_j_stride(int64_t nb, int64_t sb) {
  const int64_t rem = nb - 8 * (sb >> 3);
  return 64 * (rem < 8 ? rem : 8);
}

// Tiled Q6_K rows of the expert tier: the 210 bytes of each superblock
// regrouped per task (quarter k = 2h + p: rows 2p and 2p+1 of half h, 64
// weights; see quant.rs:180-201 for the GGUF order). Task (sb, k) owns three
// 16-byte pieces:
//   j = 0, 1  nibbles: byte b of the 32 holds weight b of the task's first
//             row in its low nibble and of its second row in its high nibble;
//   j = 2     high bits: byte b holds weight b (low nibble) and weight b+16
//             (high nibble), each nibble the first row's 2 bits then the
//             second row's.
// Pieces come in groups of 8 superblocks (1536 bytes); within a group all
// j = 0 pieces in task order, then j = 1, then j = 2. After the groups: the 16
// scale bytes of each superblock at 192*nb + 16*sb (the task's four at +4k),
// then the f16 d of each superblock at 208*nb + 2*sb.
__host__ __device__ __forceinline__ int64_t tq6_piece_off(int64_t nb, int64_t sb, int k, int j) {
  const int64_t g = sb >> 3;
  const int64_t rem = nb - 8 * g;
  const int64_t ns = rem < 8 ? rem : 8;
  return 1536 * g + 16 * (j * 4 * ns + 4 * (sb & 7) + k);
}
// Byte distance from piece (sb, k, j) to piece (sb, k, j + 1).
__host__ __device__ __forceinline__ int64_t tq6_j_stride(int64_t nb, int64_t sb) {
  const int64_t rem = nb - 8 * (sb >> 3);
  return 64 * (rem < 8 ? rem : 8);
}
// GGUF Q6_K superblock blk -> its bytes in the tiled row `row` (nb superblocks).
__host__ __device__ inline void tq6_pack_sb(const uint8_t *blk, uint8_t *row, int64_t nb, int64_t sb) {
  const int64_t js = tq6_j_stride(nb, sb);
  for (int k = 0; k < 4; ++k) {
    const int h = k >> 1, p = k & 1;
    uint8_t *n = row + tq6_piece_off(nb, sb, k, 0);
    for (int b = 0; b < 32; ++b) {
      const uint8_t lo = blk[64 * h + b], hi = blk[64 * h + 32 + b];
      const uint8_t a = p ? (uint8_t)(lo >> 4) : (uint8_t)(lo & 0xF);
      const uint8_t c = p ? (uint8_t)(hi >> 4) : (uint8_t)(hi & 0xF);
      n[(b >> 4) * js + (b & 15)] = (uint8_t)(a | (c << 4));
    }
    uint8_t *hb = n + 2 * js;
    for (int b = 0; b < 16; ++b)
      hb[b] = (uint8_t)(((blk[128 + 32 * h + b] >> (4 * p)) & 0xF) |
                        (((blk[128 + 32 * h + 16 + b] >> (4 * p)) & 0xF) << 4));
  }
  for (int i = 0; i < 16; ++i) row[192 * nb + 16 * sb + i] = blk[192 + i];
  row[208 * nb + 2 * sb] = blk[208];
  row[208 * nb + 2 * sb + 1] = blk[209];
}
// The inverse: tiled row bytes of superblock sb -> its GGUF block.
__host__ __device__ inline void tq6_unpack_sb(const uint8_t *row, uint8_t *blk, int64_t nb, int64_t sb) {
  const int64_t js = tq6_j_stride(nb, sb);
  for (int h = 0; h < 2; ++h) {
    const uint8_t *n0 = row + tq6_piece_off(nb, sb, 2 * h, 0), *n1 = row + tq6_piece_off(nb, sb, 2 * h + 1, 0);
    for (int b = 0; b < 32; ++b) {
      const uint8_t a = n0[(b >> 4) * js + (b & 15)], c = n1[(b >> 4) * js + (b & 15)];
      blk[64 * h + b] = (uint8_t)((a & 0xF) | ((c & 0xF) << 4));
      blk[64 * h + 32 + b] = (uint8_t)((a >> 4) | (c & 0xF0));
    }
    const uint8_t *h0 = n0 + 2 * js, *h1 = n1 + 2 * js;
    for (int b = 0; b < 16; ++b) {
      blk[128 + 32 * h + b] = (uint8_t)((h0[b] & 0xF) | ((h1[b] & 0xF) << 4));
      blk[128 + 32 * h + 16 + b] = (uint8_t)((h0[b] >> 4) | (h1[b] & 0xF0));
    }
  }
  for (int i = 0; i < 16; ++i) blk[192 + i] = row[192 * nb + 16 * sb + i];
  blk[208] = row[208 * nb + 2 * sb];
  blk[209] = row[208 * nb + 2 * sb + 1];
}

// Correctly rounded expf via double exp. glibc's expf (what the reference's
// f32::exp calls) is within 0.502 ulp, so the two agree except on inputs
// whose exact value lies within ~0.002 ulp of a rounding midpoint.
__device__ __forceinline__ float expf_cr(float x) { return (float)exp((double)x); }

// Rust `(v).round() as i32` clamped to [-127, 127] (qdot.rs:43, :360).
__device__ __forceinline__ int8_t q8_round(float v) {
  float r = roundf(v);  // half away from zero, like f32::round
  if (isnan(r)) return 0;
  r = fminf(fmaxf(r, -127.0f), 127.0f);
  return (int8_t)(int)r;
}

__device__ __forceinline__ uint32_t pack_i8x4(int8_t a, int8_t b, int8_t c, int8_t d) {
  return (uint32_t)(uint8_t)a | ((uint32_t)(uint8_t)b << 8) | ((uint32_t)(uint8_t)c << 16) | ((uint32_t)(uint8_t)d << 24);
}

// Loads and stores coherent across the device (agent scope, relaxed): data
// that work-groups of one kernel hand to each other without cache fences.
__device__ __forceinline__ uint32_t ld_agent(const uint32_t *p) {
  return __hip_atomic_load(const_cast<uint32_t *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float *p) {
  return __hip_atomic_load(const_cast<float *>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(uint32_t *p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_agent(float *p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Counter of a hand-off between the work-groups of one kernel. Each
// work-group adds once, with release semantics at agent scope, after every
// access it hands over (the agent-scope stores of its waves, each wave having
// waited for them); the add returns the count before it. The work-group that
// sees the final count then calls acquire_agent() before it reads what the
// others wrote (or writes what they read): every add continues the release
// sequence of the earlier ones, so all of their accesses happen before its
// own.
__device__ __forceinline__ uint32_t add_release(uint32_t *c, uint32_t v) {
  return __hip_atomic_fetch_add(c, v, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void acquire_agent() { __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent"); }

// Wait until this wave's vector memory operations have completed (s_waitcnt
// vmcnt(0): gfx9 encoding, expcnt and lgkmcnt left at their maxima). Agent-
// scope stores are then visible to every CU, so a counter update issued after
// this wait (by this wave, or by another wave of the work-group after a
// barrier) publishes them; a barrier alone waits only for LDS traffic.
__device__ __forceinline__ void vm_wait() { __builtin_amdgcn_s_waitcnt(0x0F70); }

__device__ __forceinline__ int4 ld_agent4(const void *p) {
  const uint32_t *u = (const uint32_t *)p;
  return make_int4((int)ld_agent(u), (int)ld_agent(u + 1), (int)ld_agent(u + 2), (int)ld_agent(u + 3));
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

// One row's residual add and RMSNorm by a work-group of 256 threads, as
// k_rmsnorm_regs computes it (transformer.rs:330-340, :427): thread t holds
// the float4 groups t + 256k of v = x (+ y), ss is the same sum over them then
// wg_sum256, and h[k] = (v * rr) * w per element, zero past the row (d % 4 ==
// 0, d <= 1024 * NV, 16-byte aligned rows). Every work-group of the launch
// calls it. With y and done, v goes back into x from the last work-group to
// count itself on *done, after every work-group's loads of x have returned
// (each counts after its reduction), so none can read the updated x; that
// work-group resets the counter. A non-null xo (another buffer) receives v.
template <int NV>
__device__ __forceinline__ void wg_residual_rmsnorm(float *x, const float *y, const float *w, int64_t d, float eps,
                                                    uint32_t *done, float4 (&h)[NV], float *red, int *xlast,
                                                    float *xo = nullptr) {
  const int t = threadIdx.x;
  const int n4 = (int)(d / 4);
  float4 *xr = (float4 *)x;
  const float4 *yr = (const float4 *)y;
  const float4 *wr = (const float4 *)w;
  float4 v[NV], ww[NV];
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    const int i = t + 256 * k;
    if (i < n4) {
      v[k] = xr[i];
      ww[k] = wr[i];
    }
  }
  if (yr) {
    float4 yy[NV];
#pragma unroll
    for (int k = 0; k < NV; ++k)
      if (t + 256 * k < n4) yy[k] = yr[t + 256 * k];
#pragma unroll
    for (int k = 0; k < NV; ++k)
      if (t + 256 * k < n4) {
        v[k].x = v[k].x + yy[k].x;
        v[k].y = v[k].y + yy[k].y;
        v[k].z = v[k].z + yy[k].z;
        v[k].w = v[k].w + yy[k].w;
      }
  }
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < NV; ++k)
    if (t + 256 * k < n4) ss += ((v[k].x * v[k].x + v[k].y * v[k].y) + v[k].z * v[k].z) + v[k].w * v[k].w;
  ss = wg_sum256(ss, red);  // its barriers: every thread's loads of x and y have returned
  if (xo) {
#pragma unroll
    for (int k = 0; k < NV; ++k)
      if (t + 256 * k < n4) ((float4 *)xo)[t + 256 * k] = v[k];
  }
  if (yr && done) {
    if (t == 0) {
      *xlast = add_release(done, 1u) == gridDim.x - 1;
      if (*xlast) acquire_agent();  // every other work-group has read x
    }
    __syncthreads();
    if (*xlast) {
#pragma unroll
      for (int k = 0; k < NV; ++k)
        if (t + 256 * k < n4) xr[t + 256 * k] = v[k];
      if (t == 0) __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  const float rr = 1.0f / sqrtf(ss / (float)d + eps);
#pragma unroll
  for (int k = 0; k < NV; ++k) {
    h[k] = make_float4(0.f, 0.f, 0.f, 0.f);
    if (t + 256 * k < n4) {
      h[k].x = (v[k].x * rr) * ww[k].x;
      h[k].y = (v[k].y * rr) * ww[k].y;
      h[k].z = (v[k].z * rr) * ww[k].z;
      h[k].w = (v[k].w * rr) * ww[k].w;
    }
  }
}

// Q8KRow::quantize of one 256-element block by one full wave (qdot.rs:353-365).
// The same from values already in registers: lane l holds elements
// 4l..4l+3 of the block in v.
template <bool COHERENT = false>
__device__ __forceinline__ void wave_quant_q8k_vals(float4 v, int8_t *q, float *d, int32_t *bsums, int lane) {
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  amax = group_max<64>(amax);
  const float scale = amax / 127.0f;
  const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  const int8_t a = q8_round(v.x * inv), b = q8_round(v.y * inv), c = q8_round(v.z * inv), e = q8_round(v.w * inv);
  int s = (int)a + (int)b + (int)c + (int)e;
  s = group_sum_i<4>(s);
  if constexpr (COHERENT) {
    st_agent((uint32_t *)(q + 4 * lane), pack_i8x4(a, b, c, e));
    if ((lane & 3) == 0) st_agent((uint32_t *)(bsums + (lane >> 2)), (uint32_t)s);
    if (lane == 0) st_agent(d, scale);
  } else {
    *(uint32_t *)(q + 4 * lane) = pack_i8x4(a, b, c, e);
    if ((lane & 3) == 0) bsums[lane >> 2] = s;
    if (lane == 0) *d = scale;
  }
}

// Lane l owns elements 4l..4l+3. Writes q[0..256), *d, bsums[0..16).
// COHERENT: x read and the results written with agent-scope accesses.
template <bool COHERENT = false>
__device__ __forceinline__ void wave_quant_q8k_block(const float *x, int8_t *q, float *d, int32_t *bsums, int lane) {
  float4 v;
  if constexpr (COHERENT) {
    const float *xp = x + 4 * lane;
    v = make_float4(ld_agent(xp), ld_agent(xp + 1), ld_agent(xp + 2), ld_agent(xp + 3));
  } else {
    v = *(const float4 *)(x + 4 * lane);
  }
  wave_quant_q8k_vals<COHERENT>(v, q, d, bsums, lane);
}

// Q8Row::quantize of one 32-element block by an aligned group of 8 lanes
// (qdot.rs:36-47). g = lane & 7 owns elements 4g..4g+3.
__device__ __forceinline__ void group8_quant_q8_vals(float4 v, int8_t *q, float *d, int32_t *s16, int g) {
  float amax = fmaxf(fmaxf(fabsf(v.x), fabsf(v.y)), fmaxf(fabsf(v.z), fabsf(v.w)));
  amax = group_max<8>(amax);
  const float scale = amax / 127.0f;
  const float inv = scale > 0.0f ? 1.0f / scale : 0.0f;
  const int8_t a = q8_round(v.x * inv), b = q8_round(v.y * inv), c = q8_round(v.z * inv), e = q8_round(v.w * inv);
  *(uint32_t *)(q + 4 * g) = pack_i8x4(a, b, c, e);
  int s = (int)a + (int)b + (int)c + (int)e;
  s = group_sum_i<4>(s);
  if ((g & 3) == 0) s16[g >> 2] = s;
  if (g == 0) *d = scale;
}
__device__ __forceinline__ void group8_quant_q8_block(const float *x, int8_t *q, float *d, int32_t *s16, int g) {
  group8_quant_q8_vals(*(const float4 *)(x + 4 * g), q, d, s16, g);
}

}  // namespace kmoe
