// kmoe_quant.hip — activation quantizers on the device.
//
// Q8KRow::quantize (qdot.rs:347-367) and Q8Row::quantize (qdot.rs:30-49):
// scale = amax / 127, inv = scale > 0 ? 1 / scale : 0,
// q = clamp(round_half_away(x * inv), -127, 127), plus per-16 sums of q.
// Each step is one IEEE-rounded f32 operation (division and product are
// correctly rounded here and on the CPU; max is exact in any order), so the
// bytes, scales and sums are bit-identical to the reference's.
#include "kmoe_device.h"
#include "kmoe_launch.h"

namespace kmoe {

// One wave per 256-element block.
__global__ void __launch_bounds__(256) k_quant_q8k(const float *__restrict__ x, int64_t nblocks, int8_t *__restrict__ q,
                                                   float *__restrict__ d, int32_t *__restrict__ bsums) {
  const int lane = threadIdx.x & 63;
  const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (blk >= nblocks) return;
  wave_quant_q8k_block(x + blk * 256, q + blk * 256, d + blk, bsums + blk * 16, lane);
}

// One wave per 8 blocks of 32; whole 8-lane groups drop out past the end.
__global__ void __launch_bounds__(256) k_quant_q8(const float *__restrict__ x, int64_t nblocks, int8_t *__restrict__ q,
                                                  float *__restrict__ d, int32_t *__restrict__ s16) {
  const int lane = threadIdx.x & 63;
  const int64_t blk = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 8 + (lane >> 3);
  if (blk >= nblocks) return;
  group8_quant_q8_block(x + blk * 32, q + blk * 32, d + blk, s16 + blk * 2, lane & 7);
}

hipError_t launch_quant_q8k(hipStream_t st, const float *x, int64_t rows, int64_t cols, int8_t *q, float *d,
                            int32_t *bsums) {
  const int64_t nb = rows * (cols / 256);
  if (nb == 0) return hipSuccess;
  KMOE_LAUNCH(k_quant_q8k, dim3((unsigned)((nb + 3) / 4)), dim3(256), 0, st, x, nb, q, d, bsums);
  return hipGetLastError();
}

hipError_t launch_quant_q8(hipStream_t st, const float *x, int64_t rows, int64_t cols, int8_t *q, float *d,
                           int32_t *s16) {
  const int64_t nb = rows * (cols / 32);
  if (nb == 0) return hipSuccess;
  const int64_t waves = (nb + 7) / 8;
  KMOE_LAUNCH(k_quant_q8, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, x, nb, q, d, s16);
  return hipGetLastError();
}

}  // namespace kmoe
