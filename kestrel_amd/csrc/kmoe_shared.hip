// kmoe_shared.hip — elementwise pieces of the shared expert (qwen2moe,
// transformer.rs:572-587): SwiGLU over [S, F] and the gated add of its output.
#include "kmoe_device.h"
#include "kmoe_launch.h"

namespace kmoe {

namespace {

// g = g / (1 + exp(-g)) * u, elementwise (division, then multiplication).
__global__ void __launch_bounds__(256) k_swiglu(float *__restrict__ g, const float *__restrict__ u, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float gv = g[i];
    const float den = 1.0f + expf_cr(-gv);
    const float q = gv / den;
    g[i] = q * u[i];
  }
}

// out[s, c] = out[s, c] + scale_s * y[s, c], scale_s = 1 / (1 + exp(-logit_s))
// (logits null: scale 1).
__global__ void __launch_bounds__(256) k_shared_add(float *__restrict__ out, const float *__restrict__ y,
                                                    const float *__restrict__ logits, int64_t S, int64_t d) {
  const int64_t s = blockIdx.y;
  float scale = 1.0f;
  if (logits) {
    const float den = 1.0f + expf_cr(-logits[s]);
    scale = 1.0f / den;
  }
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c < d; c += (int64_t)gridDim.x * blockDim.x) {
    const float p = scale * y[s * d + c];
    out[s * d + c] = out[s * d + c] + p;
  }
}

// One row: gu[c] (gate) and gu[F + c] (up) -> g = gate / (1 + exp(-gate)) *
// up (k_swiglu's expressions), quantized as Q8KRow (QK: one wave per 256
// columns) or Q8Row (eight lanes per 32 columns), qdot.rs:30-49, :347-367.
template <bool QK>
__global__ void __launch_bounds__(256) k_swiglu_quant(const float *__restrict__ gu, int64_t F, int8_t *__restrict__ q,
                                                      float *__restrict__ d, int32_t *__restrict__ s) {
  const int lane = threadIdx.x & 63;
  const int64_t wv = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t blk = QK ? wv : wv * 8 + (lane >> 3);  // 256- or 32-column block
  const int64_t el = QK ? 256 : 32;
  if (blk * el >= F) return;  // whole waves (QK) or whole 8-lane groups leave together
  const int64_t c = blk * el + 4 * (QK ? lane : (lane & 7));
  const float4 gv = *(const float4 *)(gu + c), uv = *(const float4 *)(gu + F + c);
  float4 v;
  v.x = gv.x / (1.0f + expf_cr(-gv.x)) * uv.x;
  v.y = gv.y / (1.0f + expf_cr(-gv.y)) * uv.y;
  v.z = gv.z / (1.0f + expf_cr(-gv.z)) * uv.z;
  v.w = gv.w / (1.0f + expf_cr(-gv.w)) * uv.w;
  if constexpr (QK) wave_quant_q8k_vals(v, q + blk * 256, d + blk, s + blk * 16, lane);
  else group8_quant_q8_vals(v, q + blk * 32, d + blk, s + blk * 2, lane & 7);
}

}  // namespace

hipError_t launch_swiglu_quant(hipStream_t st, int type, const float *gu, int64_t F, int8_t *q, float *d,
                               int32_t *s) {
  if (F <= 0) return hipSuccess;
  if (((uintptr_t)gu & 15u) || (F % 4) || (F * 4) % 16) return hipErrorNotSupported;  // float4 loads of both halves
  if (is_kquant(type)) {
    if (F % 256) return hipErrorNotSupported;
    const int64_t waves = F / 256;
    KMOE_LAUNCH(k_swiglu_quant<true>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, gu, F, q, d, s);
  } else {
    if (F % 32) return hipErrorNotSupported;
    const int64_t waves = (F / 32 + 7) / 8;
    KMOE_LAUNCH(k_swiglu_quant<false>, dim3((unsigned)((waves + 3) / 4)), dim3(256), 0, st, gu, F, q, d, s);
  }
  return hipGetLastError();
}

hipError_t launch_swiglu(hipStream_t st, float *g, const float *u, int64_t n) {
  if (n <= 0) return hipSuccess;
  int64_t grid = (n + 255) / 256;
  if (grid > 8192) grid = 8192;
  KMOE_LAUNCH(k_swiglu, dim3((unsigned)grid), dim3(256), 0, st, g, u, n);
  return hipGetLastError();
}

hipError_t launch_shared_add(hipStream_t st, float *out, const float *y, const float *logits, int64_t S, int64_t d) {
  if (S <= 0 || d <= 0) return hipSuccess;
  if (S > 65535) return hipErrorInvalidValue;
  const int64_t gx = (d + 255) / 256 < 64 ? (d + 255) / 256 : 64;
  KMOE_LAUNCH(k_shared_add, dim3((unsigned)gx, (unsigned)S), dim3(256), 0, st, out, y, logits, S, d);
  return hipGetLastError();
}

}  // namespace kmoe
