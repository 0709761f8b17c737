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
// One wave per node: lanes hold channels lane + 64 k; the hidden units' pre-activations are channel
// sums, reduced 16 units at a time (below).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "ictc_hip.h"
#include "ictc_common.hpp"

namespace ictc {
namespace {

constexpr int kRoWave = 64;
constexpr int kRoWaves = 4;
constexpr int kRoBlock = kRoWave * kRoWaves;
static_assert(ICTC_READOUT_MAX_CHANNELS <= 16 * 64, "at most 16 channel chunks per lane");

__device__ __forceinline__ float ro_wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kRoWave);
  return v;
}

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

// The hidden units are taken 16 at a time: every lane forms its partial dot products for the 16
// units first, and one transposing butterfly (WaveSums<16>) reduces them, leaving unit j's
// pre-activation on the lanes with (lane >> 2) & 15 == j (lane & 3 == 0 owns it once).
constexpr int kRoGroup = 16;
using RoSums = WaveSums<kRoGroup>;

// NK: channel chunks of 64 held per lane (ceil(C / 64) rounded up to a power of two), so the
// unrolled chunk loops carry no iterations for channels past C.
template <int MODE, int NK>
__global__ void __launch_bounds__(kRoBlock) readout_kernel(const ReadoutArgs a) {
  const int lane = threadIdx.x & (kRoWave - 1);
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kRoWaves + threadIdx.x / kRoWave;
  if (n >= a.nodes) return;   // whole waves leave together (n is wave-uniform)
  const int C = a.C;
  const float* __restrict__ xr = a.x + n * C;
  float xv[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) {
    const int c = lane + k * kRoWave;
    xv[k] = c < C ? xr[c] : 0.f;
  }
  const int own = RoSums::index(lane);          // the unit of the group this lane ends up holding
  const bool owner = RoSums::owner(lane);
  float gn = 0.f;
  if constexpr (MODE == ICTC_READOUT_VJP) {
    gn = a.g[n];
    if (a.grad_y != nullptr)
      for (int c = lane; c < C; c += kRoWave) a.grad_y[n * C + c] = gn * a.wl[c];
    if (a.grad_x == nullptr) return;
  }
  float e = 0.f;                                 // VALUE: this lane's share of the MLP readout
  float dx[NK];
#pragma unroll
  for (int k = 0; k < NK; ++k) dx[k] = 0.f;
  for (int j0 = 0; j0 < a.H; j0 += kRoGroup) {
    float p[kRoGroup];
#pragma unroll
    for (int q = 0; q < kRoGroup; ++q) {
      p[q] = 0.f;
      if (j0 + q < a.H) {                        // wave-uniform
        const float* __restrict__ w1j = a.w1 + static_cast<int64_t>(j0 + q) * C;
#pragma unroll
        for (int k = 0; k < NK; ++k) {
          const int c = lane + k * kRoWave;
          if (c < C) p[q] = fmaf(w1j[c], xv[k], p[q]);
        }
      }
    }
    const float z = RoSums::reduce(p, lane);     // unit j0 + own's pre-activation
    const int j = j0 + own;
    const bool live = owner && j < a.H;
    const float sg = 1.f / (1.f + expf(-z));
    if constexpr (MODE == ICTC_READOUT_VALUE) {
      if (live) e = fmaf(a.w2[j] * a.scale, z * sg, e);
    } else {
      const float dz = live ? gn * a.w2[j] * a.scale * (sg * (1.f + z * (1.f - sg))) : 0.f;
#pragma unroll
      for (int q = 0; q < kRoGroup; ++q) {
        if (j0 + q >= a.H) break;                // wave-uniform
        const float d = __shfl(dz, q << 2, kRoWave);   // lane 4q owns unit q of the group
        const float* __restrict__ w1j = a.w1 + static_cast<int64_t>(j0 + q) * C;
#pragma unroll
        for (int k = 0; k < NK; ++k) {
          const int c = lane + k * kRoWave;
          if (c < C) dx[k] = fmaf(w1j[c], d, dx[k]);
        }
      }
    }
  }
  if constexpr (MODE == ICTC_READOUT_VALUE) {
    float lin = 0.f;
    if (a.y != nullptr)
      for (int c = lane; c < C; c += kRoWave) lin = fmaf(a.wl[c], a.y[n * C + c], lin);
    const float tot = ro_wave_sum(lin + e);
    if (lane == 0) a.atomic[n] = tot;
  } else {
#pragma unroll
    for (int k = 0; k < NK; ++k) {
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
  const int chunks = (channels + kRoWave - 1) / kRoWave;
  const dim3 grid(static_cast<unsigned>(blocks));
#define ICTC_READOUT_LAUNCH(NK)                                                                             \
  if (mode == ICTC_READOUT_VALUE)                                                                           \
    hipLaunchKernelGGL((readout_kernel<ICTC_READOUT_VALUE, NK>), grid, dim3(kRoBlock), 0, stream, a);       \
  else                                                                                                      \
    hipLaunchKernelGGL((readout_kernel<ICTC_READOUT_VJP, NK>), grid, dim3(kRoBlock), 0, stream, a);
  if (chunks <= 1) {
    ICTC_READOUT_LAUNCH(1)
  } else if (chunks <= 2) {
    ICTC_READOUT_LAUNCH(2)
  } else if (chunks <= 4) {
    ICTC_READOUT_LAUNCH(4)
  } else if (chunks <= 8) {
    ICTC_READOUT_LAUNCH(8)
  } else {
    ICTC_READOUT_LAUNCH(16)
  }
#undef ICTC_READOUT_LAUNCH
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}
