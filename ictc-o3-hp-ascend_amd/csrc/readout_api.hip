// Atomic-energy readouts of the MACE model in one pass per derivative order (gfx950).
//
// Per node n, with x the last layer's scalar features and y an earlier layer's (optional):
//   VALUE: atomic[n] = w_lin . y[n] + sum_j w2[j] s silu(w1[j] . x[n])
//   VJP  : given g[n] = d/d atomic[n]:   grad_lin[n] = g[n] w_lin
//                                        grad_mlp[n] = sum_j w1[j] s w2[j] silu'(w1[j] . x[n]) g[n]
// the layer readout (a bias-free Linear(C, 1), reference EquivariantScalarReadoutSO3,
// pure_cartesian_ictd_layers.py:46-70) of one inner layer plus the last layer's MLP readout
// (Linear(C, H), normalised SiLU with constant s, Linear(H, 1); pure_cartesian_ictd_fix.py:1434-1449),
// summed as the model sums its per-layer energies.  Composed from library ops the two readouts and
// their adjoints take some ten small launches per step.
//
// One wave per node: lanes hold channels lane + 64 k; each hidden unit's pre-activation is a wave sum.
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "ictc_hip.h"

namespace ictc {
namespace {

constexpr int kRoWave = 64;
constexpr int kRoWaves = 4;
constexpr int kRoBlock = kRoWave * kRoWaves;
constexpr int kRoChunks = ICTC_READOUT_MAX_CHANNELS / kRoWave;

__device__ __forceinline__ float ro_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kRoWave);
  return v;
}

__device__ __forceinline__ float ro_sigmoid(float z) { return 1.f / (1.f + expf(-z)); }

struct ReadoutArgs {
  const float* y;      // [N, C] or null
  const float* wl;     // [C] (with y)
  const float* x;      // [N, C]
  const float* w1;     // [H, C]
  const float* w2;     // [H]
  float scale;
  const float* g;      // [N] (VJP)
  float* atomic;       // [N] (VALUE)
  float* grad_y;       // [N, C] (VJP, optional)
  float* grad_x;       // [N, C] (VJP, optional)
  int C, H;
  int64_t nodes;
};

template <int MODE>
__global__ void __launch_bounds__(kRoBlock) readout_kernel(const ReadoutArgs a) {
  const int lane = threadIdx.x & (kRoWave - 1);
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kRoWaves + threadIdx.x / kRoWave;
  if (n >= a.nodes) return;   // whole waves leave together (n is wave-uniform)
  const int C = a.C;
  const float* __restrict__ xr = a.x + n * C;
  float xv[kRoChunks];
#pragma unroll
  for (int k = 0; k < kRoChunks; ++k) {
    const int c = lane + k * kRoWave;
    xv[k] = c < C ? xr[c] : 0.f;
  }
  if constexpr (MODE == ICTC_READOUT_VALUE) {
    float e = 0.f;
    if (a.y != nullptr) {
      float p = 0.f;
      for (int c = lane; c < C; c += kRoWave) p = fmaf(a.wl[c], a.y[n * C + c], p);
      e = ro_wave_sum(p);
    }
    for (int j = 0; j < a.H; ++j) {
      const float* __restrict__ w1j = a.w1 + static_cast<int64_t>(j) * C;
      float p = 0.f;
#pragma unroll
      for (int k = 0; k < kRoChunks; ++k) {
        const int c = lane + k * kRoWave;
        if (c < C) p = fmaf(w1j[c], xv[k], p);
      }
      const float z = ro_wave_sum(p);
      e = fmaf(a.w2[j] * a.scale, z * ro_sigmoid(z), e);
    }
    if (lane == 0) a.atomic[n] = e;
  } else {
    const float gn = a.g[n];
    if (a.grad_y != nullptr)
      for (int c = lane; c < C; c += kRoWave) a.grad_y[n * C + c] = gn * a.wl[c];
    if (a.grad_x == nullptr) return;
    float dx[kRoChunks];
#pragma unroll
    for (int k = 0; k < kRoChunks; ++k) dx[k] = 0.f;
    for (int j = 0; j < a.H; ++j) {
      const float* __restrict__ w1j = a.w1 + static_cast<int64_t>(j) * C;
      float p = 0.f;
#pragma unroll
      for (int k = 0; k < kRoChunks; ++k) {
        const int c = lane + k * kRoWave;
        if (c < C) p = fmaf(w1j[c], xv[k], p);
      }
      const float z = ro_wave_sum(p);
      const float sg = ro_sigmoid(z);
      const float dz = gn * a.w2[j] * a.scale * (sg * (1.f + z * (1.f - sg)));
#pragma unroll
      for (int k = 0; k < kRoChunks; ++k) {
        const int c = lane + k * kRoWave;
        if (c < C) dx[k] = fmaf(w1j[c], dz, dx[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < kRoChunks; ++k) {
      const int c = lane + k * kRoWave;
      if (c < C) a.grad_x[n * C + c] = dx[k];
    }
  }
}

}  // namespace
}  // namespace ictc

extern "C" int ictc_hip_readout(int mode, const float* y, const float* w_lin, const float* x, const float* w1,
                                const float* w2, float scale, const float* grad_atomic, float* out_atomic,
                                float* grad_y, float* grad_x, int channels, int hidden, int64_t nodes,
                                hipStream_t stream) {
  using namespace ictc;
  if (mode != ICTC_READOUT_VALUE && mode != ICTC_READOUT_VJP) return ICTC_ERR_INVALID_ARGUMENT;
  if (nodes < 0 || channels < 1 || channels > ICTC_READOUT_MAX_CHANNELS || hidden < 1 ||
      hidden > ICTC_READOUT_MAX_HIDDEN)
    return ICTC_ERR_INVALID_ARGUMENT;
  if (nodes == 0) return ICTC_OK;
  if (!x || !w1 || !w2 || (y && !w_lin)) return ICTC_ERR_INVALID_ARGUMENT;
  if (mode == ICTC_READOUT_VALUE && !out_atomic) return ICTC_ERR_INVALID_ARGUMENT;
  if (mode == ICTC_READOUT_VJP) {
    if (!grad_atomic || (grad_y && !(y && w_lin))) return ICTC_ERR_INVALID_ARGUMENT;
    if (!grad_y && !grad_x) return ICTC_OK;
  }
  const int64_t blocks = (nodes + kRoWaves - 1) / kRoWaves;
  if (blocks > 0x7fffffff) return ICTC_ERR_INVALID_ARGUMENT;
  const ReadoutArgs a{y, w_lin, x, w1, w2, scale, grad_atomic, out_atomic, grad_y, grad_x, channels, hidden, nodes};
  if (mode == ICTC_READOUT_VALUE)
    hipLaunchKernelGGL(readout_kernel<ICTC_READOUT_VALUE>, dim3(static_cast<unsigned>(blocks)), dim3(kRoBlock), 0,
                       stream, a);
  else
    hipLaunchKernelGGL(readout_kernel<ICTC_READOUT_VJP>, dim3(static_cast<unsigned>(blocks)), dim3(kRoBlock), 0,
                       stream, a);
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}
