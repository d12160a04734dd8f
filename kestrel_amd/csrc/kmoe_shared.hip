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

}  // namespace

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
