// kmoe_layout.hip — conversion between GGUF rows and the expert tier's tiled
// rows: Q4_K (tq4_qs_off in kmoe_device.h) and Q6_K (tq6_piece_off).
//
// A row of nb superblocks is 9*nb 16-byte chunks in both layouts: chunk c < nb
// is the head of superblock c, chunk nb + 8*sb + p is nibble piece p (bytes
// [16p, 16p+16) of the 128 nibble bytes) of superblock sb. Only their
// positions differ, so the conversion is a permutation of 16-byte chunks.
#include "kmoe_device.h"
#include "kmoe_launch.h"

namespace kmoe {

namespace {

// Byte offsets of chunk c of a row in the GGUF and the tiled layout.
__host__ __device__ __forceinline__ void tq4_chunk(int64_t nb, int64_t c, int64_t &gguf, int64_t &tiled) {
  if (c < nb) {
    gguf = 144 * c;
    tiled = 16 * c;
  } else {
    const int64_t q = c - nb, sb = q >> 3;
    const int p = (int)(q & 7);
    gguf = 144 * sb + 16 + 16 * p;
    tiled = tq4_qs_off(nb, sb, p >> 1, p & 1);
  }
}

// One thread per 16-byte chunk. ALIGNED: both buffers 16-byte aligned.
template <bool ALIGNED>
__global__ void __launch_bounds__(256) k_tq4_convert(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                     int64_t rows, int64_t nb, int to_tiled) {
  const int64_t per_row = 9 * nb;
  const int64_t n = rows * per_row;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / per_row, c = i - r * per_row;
    int64_t g, t;
    tq4_chunk(nb, c, g, t);
    const int64_t base = r * 144 * nb;
    const uint8_t *s = src + base + (to_tiled ? g : t);
    uint8_t *d = dst + base + (to_tiled ? t : g);
    if constexpr (ALIGNED) {
      *(uint4 *)d = *(const uint4 *)s;
    } else {
#pragma unroll
      for (int b = 0; b < 16; ++b) d[b] = s[b];
    }
  }
}

// One thread per Q6_K superblock: a byte-level regrouping (tq6_pack_sb /
// tq6_unpack_sb), not a chunk permutation.
__global__ void __launch_bounds__(256) k_tq6_convert(const uint8_t *__restrict__ src, uint8_t *__restrict__ dst,
                                                     int64_t rows, int64_t nb, int to_tiled) {
  const int64_t n = rows * nb;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / nb, sb = i - r * nb;
    const int64_t base = r * 210 * nb;
    if (to_tiled) tq6_pack_sb(src + base + 210 * sb, dst + base, nb, sb);
    else tq6_unpack_sb(src + base, dst + base + 210 * sb, nb, sb);
  }
}

}  // namespace

hipError_t launch_tq6_convert(hipStream_t st, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t nb,
                              bool to_tiled) {
  if (rows <= 0 || nb <= 0) return hipSuccess;
  int64_t grid = (rows * nb + 255) / 256;
  if (grid > 65536) grid = 65536;
  KMOE_LAUNCH(k_tq6_convert, dim3((unsigned)grid), dim3(256), 0, st, src, dst, rows, nb, to_tiled ? 1 : 0);
  return hipGetLastError();
}

void tq6_convert_host(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t nb, bool to_tiled) {
  for (int64_t r = 0; r < rows; ++r)
    for (int64_t sb = 0; sb < nb; ++sb) {
      const int64_t base = r * 210 * nb;
      if (to_tiled) tq6_pack_sb(src + base + 210 * sb, dst + base, nb, sb);
      else tq6_unpack_sb(src + base, dst + base + 210 * sb, nb, sb);
    }
}

hipError_t launch_tq4_convert(hipStream_t st, const uint8_t *src, uint8_t *dst, int64_t rows, int64_t nb,
                              bool to_tiled) {
  if (rows <= 0 || nb <= 0) return hipSuccess;
  const int64_t n = rows * 9 * nb;
  int64_t grid = (n + 255) / 256;
  if (grid > 65536) grid = 65536;
  const bool aligned = (((uintptr_t)src | (uintptr_t)dst) & 15) == 0;
  if (aligned)
    KMOE_LAUNCH((k_tq4_convert<true>), dim3((unsigned)grid), dim3(256), 0, st, src, dst, rows, nb,
                       to_tiled ? 1 : 0);
  else
    KMOE_LAUNCH((k_tq4_convert<false>), dim3((unsigned)grid), dim3(256), 0, st, src, dst, rows, nb,
                       to_tiled ? 1 : 0);
  return hipGetLastError();
}

void tq4_convert_host(const uint8_t *src, uint8_t *dst, int64_t rows, int64_t nb, bool to_tiled) {
  for (int64_t r = 0; r < rows; ++r) {
    const uint8_t *s = src + r * 144 * nb;
    uint8_t *d = dst + r * 144 * nb;
    for (int64_t c = 0; c < 9 * nb; ++c) {
      int64_t g, t;
      tq4_chunk(nb, c, g, t);
      const int64_t so = to_tiled ? g : t, dofs = to_tiled ? t : g;
      for (int b = 0; b < 16; ++b) d[dofs + b] = s[so + b];
    }
  }
}

}  // namespace kmoe
