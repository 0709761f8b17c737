// Element-conditioned linear map on a scalar block (the MACE interaction's self connection), gfx950.
//
//   APPLY    : out[n][o] = sum_i W[s_n][o][i] x[n][i]
//   TRANSPOSE: out[n][i] = sum_o W[s_n][o][i] x[n][o]      (the input adjoint of APPLY)
// W [S, C, C] holds one torch Linear weight per species (row o, column i), x and out [N, C], s the
// node's species.  ElementConditionedLinearSO3 (reference mace_ictc/models/pure_cartesian_ictd_fix.py:
// 335-390) applied to the l = 0 block; composed from library ops it is one [N, C] x [C, S*C] product
// (S times the useful work) and a gather of each node's block, and its adjoint a zero fill, a scatter
// and a second product.
//
// One wave per node.  The node's input row is staged in LDS and read as a wave-uniform broadcast;
// APPLY: lane o reads its weight row W[s][o][:] (float4 steps when C % 4 == 0), TRANSPOSE: lane i
// reads the column W[s][:][i], one contiguous row segment per step across the wave.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ictc_hip.h"

namespace ictc {
namespace {

constexpr int kSlWave = 64;
constexpr int kSlWaves = 4;
constexpr int kSlBlock = kSlWave * kSlWaves;

template <int MODE, bool VEC4>
__global__ void __launch_bounds__(kSlBlock)
species_linear_kernel(const float* __restrict__ w, const float* __restrict__ x, const int64_t* __restrict__ species,
                      float* __restrict__ out, int C, int num_species, int64_t nodes) {
  extern __shared__ float srow[];   // [kSlWaves][C]
  const int lane = threadIdx.x & (kSlWave - 1);
  const int wave = threadIdx.x / kSlWave;
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kSlWaves + wave;
  float* __restrict__ row = srow + wave * C;
  const bool node_live = n < nodes;
  if (node_live)
    for (int i = lane; i < C; i += kSlWave) row[i] = x[n * C + i];
  __syncthreads();
  if (!node_live) return;
  int64_t s = species[n];
  if (s < 0 || s >= num_species) s = 0;   // the caller validates; never read outside W
  const float* __restrict__ ws = w + s * C * C;
  for (int j = lane; j < C; j += kSlWave) {
    float acc = 0.f;
    if constexpr (MODE == ICTC_SPECIES_APPLY) {
      const float* __restrict__ wr = ws + static_cast<int64_t>(j) * C;
      if constexpr (VEC4) {
        for (int i = 0; i < C; i += 4) {
          const float4 v = *reinterpret_cast<const float4*>(wr + i);
          acc = fmaf(v.x, row[i], acc);
          acc = fmaf(v.y, row[i + 1], acc);
          acc = fmaf(v.z, row[i + 2], acc);
          acc = fmaf(v.w, row[i + 3], acc);
        }
      } else {
        for (int i = 0; i < C; ++i) acc = fmaf(wr[i], row[i], acc);
      }
    } else {
      for (int o = 0; o < C; ++o) acc = fmaf(ws[static_cast<int64_t>(o) * C + j], row[o], acc);
    }
    out[n * C + j] = acc;
  }
}

}  // namespace
}  // namespace ictc

extern "C" int ictc_hip_species_linear(int mode, const float* weight, const float* x, const int64_t* species,
                                       float* out, int channels, int num_species, int64_t nodes,
                                       hipStream_t stream) {
  using namespace ictc;
  if (mode != ICTC_SPECIES_APPLY && mode != ICTC_SPECIES_TRANSPOSE) return ICTC_ERR_INVALID_ARGUMENT;
  if (nodes < 0 || channels < 1 || channels > ICTC_SPECIES_MAX_CHANNELS || num_species < 1)
    return ICTC_ERR_INVALID_ARGUMENT;
  if (nodes == 0) return ICTC_OK;
  if (!weight || !x || !species || !out) return ICTC_ERR_INVALID_ARGUMENT;
  const int64_t blocks = (nodes + kSlWaves - 1) / kSlWaves;
  if (blocks > 0x7fffffff) return ICTC_ERR_INVALID_ARGUMENT;
  const dim3 grid(static_cast<unsigned>(blocks));
  const size_t lds = static_cast<size_t>(kSlWaves) * channels * sizeof(float);
  const bool vec4 = channels % 4 == 0 && (reinterpret_cast<uintptr_t>(weight) & 15) == 0;
  if (mode == ICTC_SPECIES_APPLY) {
    if (vec4)
      hipLaunchKernelGGL((species_linear_kernel<ICTC_SPECIES_APPLY, true>), grid, dim3(kSlBlock), lds, stream, weight,
                         x, species, out, channels, num_species, nodes);
    else
      hipLaunchKernelGGL((species_linear_kernel<ICTC_SPECIES_APPLY, false>), grid, dim3(kSlBlock), lds, stream,
                         weight, x, species, out, channels, num_species, nodes);
  } else {
    hipLaunchKernelGGL((species_linear_kernel<ICTC_SPECIES_TRANSPOSE, false>), grid, dim3(kSlBlock), lds, stream,
                       weight, x, species, out, channels, num_species, nodes);
  }
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}
