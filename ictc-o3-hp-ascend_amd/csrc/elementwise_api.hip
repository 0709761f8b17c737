// SiLU derivative forms for the radial MLP of force training (gfx950).
//
// The radial MLP applies silu between its layers; force training differentiates the first-order
// backward  y = g * silu'(x)  once more.  Given the cotangent h of y, one pass produces
//   dg = h * silu'(x)          (the cotangent of g)
//   dx = h * g * silu''(x)     (the cotangent of x)
// with s = 1 / (1 + exp(-x)), silu'(x) = s (1 + x (1 - s)), silu''(x) = s (1 - s) (2 + x (1 - 2 s)),
// where a composition of elementwise library ops takes about nine passes over the [E, 64]
// activations.  Replaces the silu derivative modes of the reference's fp32 elementwise kernel
// (ascendc/op_kernel/vector.cpp:6-136 via ascendc/elementwise.py:7-97).
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ictc_hip.h"

namespace ictc {
namespace {

constexpr int kEltBlock = 256;

__global__ void __launch_bounds__(kEltBlock)
silu_second_kernel(const float* __restrict__ x, const float* __restrict__ g, const float* __restrict__ h,
                   float* __restrict__ dg, float* __restrict__ dx, int64_t n) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kEltBlock;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kEltBlock + threadIdx.x; i < n; i += stride) {
    const float xv = x[i], hv = h[i];
    const float s = 1.0f / (1.0f + expf(-xv));
    const float q = 1.0f - s;
    if (dg != nullptr) dg[i] = hv * (s * fmaf(xv, q, 1.0f));
    if (dx != nullptr) dx[i] = hv * g[i] * (s * q * fmaf(xv, 1.0f - 2.0f * s, 2.0f));
  }
}

}  // namespace
}  // namespace ictc

extern "C" int ictc_hip_silu_second(const float* x, const float* grad, const float* cotangent, float* grad_grad,
                                    float* grad_x, int64_t n, hipStream_t stream) {
  if (n < 0) return ICTC_ERR_INVALID_ARGUMENT;
  if (n == 0 || (grad_grad == nullptr && grad_x == nullptr)) return ICTC_OK;
  if (x == nullptr || cotangent == nullptr || (grad_x != nullptr && grad == nullptr)) return ICTC_ERR_INVALID_ARGUMENT;
  const int64_t blocks = (n + ictc::kEltBlock - 1) / ictc::kEltBlock;
  const unsigned grid = static_cast<unsigned>(blocks < 16384 ? blocks : 16384);
  hipLaunchKernelGGL(ictc::silu_second_kernel, dim3(grid), dim3(ictc::kEltBlock), 0, stream, x, grad, cotangent,
                     grad_grad, grad_x, n);
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}
