// Correlation <= 3 symmetric contraction with species-selected weights (gfx950).
//
//   out[n, c, l_out, m] = sum_p W[s_n, p, c] * chain_p(x[n, c, :])_m
// the MACE contraction recursion of reference
// ictc_o3/ops/_mace_symmetric_contraction.py:298-346 (_forward_selected_elements),
// evaluated through shared pair prefixes instead of dense U tensors (the factorisation
// idea of ictc_o3/ops/factorized_contraction.py:51-149).  One lane per (node, channel):
// the whole polynomial of a channel lives in registers, the weights of the node's
// species are read along the channel axis (coalesced), and nodes are independent.
//
// Layouts (mul_ir, the module's flat layout): x [N, C*(L+1)^2] with degree blocks
// [C, 2l+1]; out [N, C*(T+1)^2] with blocks [C, 2l+1]; W [S, KTOT, C].
#pragma once
#include "ictc_common.hpp"
#include "sc_plan.hpp"

namespace ictc {

constexpr int kScBlock = 256;
constexpr int kScWaves = kScBlock / kWave;

// Loads always read a valid channel (cc = c, or 0 for lanes past C) and are then
// selected, so the loads need no exec-mask branches.
template <int L>
__device__ __forceinline__ void sc_load_mul_ir(const float* __restrict__ row, int C, int cc, bool live,
                                               float* v) {
#pragma unroll
  for (int l = 0; l <= L; ++l) {
#pragma unroll
    for (int m = 0; m < 2 * l + 1; ++m) {
      const float t = row[C * l * l + cc * (2 * l + 1) + m];
      v[l * l + m] = live ? t : 0.f;
    }
  }
}

template <int L>
__device__ __forceinline__ void sc_store_mul_ir(float* __restrict__ row, int C, int c, const float* v) {
#pragma unroll
  for (int l = 0; l <= L; ++l) {
#pragma unroll
    for (int m = 0; m < 2 * l + 1; ++m) row[C * l * l + c * (2 * l + 1) + m] = v[l * l + m];
  }
}

// Directional modes take a tangent t [N, C*(L+1)^2] (mul_ir, like x) and evaluate the
// generated code on x + eps t:
//   mode 0: forward                           out [N, C*(T+1)^2]
//   mode 1: VJP to the node features          out [N, C*(L+1)^2]   = J(x)^T u
//   mode 2: weight features                   out [N, KTOT, C]     phi_p = <u, chain_p(x)>
//   mode 3: JVP                               out [N, C*(T+1)^2]   = J(x) t
//   mode 4: Hessian-vector product            out [N, C*(L+1)^2]   = d/dx <u, J(x) t>
//   mode 5: weight-feature JVP                out [N, KTOT, C]     <u, d chain_p(x)[t]>
// The straight-line float forward of the largest plans would take ~200 VGPRs (two waves per SIMD);
// it runs better at three (168 VGPRs, a few values spilled; cfg 3 forward 0.511 -> 0.494 ms, the
// VALU pairing more instructions with a third wave ready).  Every other mode keeps the compiler's
// own allocation.
constexpr int sc_min_waves(int l, int t, int k, int mode) { return (mode == 0 && l == 3 && k == 3 && t <= 1) ? 3 : 1; }

template <int L, int T, int K, int MODE>
__global__ void __launch_bounds__(kScBlock) __attribute__((amdgpu_waves_per_eu(sc_min_waves(L, T, K, MODE))))
sc_kernel(const float* __restrict__ x, const float* __restrict__ t, const int64_t* __restrict__ species,
          const float* __restrict__ w, const float* __restrict__ u, float* __restrict__ out, int C,
          int64_t nodes, int num_species, int nchunks) {
  using PL = sc::Plan<L, T, K>;
  using sc::Dual;
  constexpr int D = PL::D, NO = PL::NO;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kScWaves + wave;
  const int64_t node = item / nchunks;
  if (node >= nodes) return;
  const int chunk = static_cast<int>(item - node * nchunks);
  const int c = chunk * kWave + lane;
  const bool live = c < C;
  const int cc = live ? c : 0;
  int64_t s = species[node];
  if (s < 0 || s >= num_species) s = 0;  // host validates; never read outside W
  const float* __restrict__ wr = w + s * PL::KTOT * C + cc;
  float xv[D];
  sc_load_mul_ir<L>(x + node * D * C, C, cc, live, xv);
  float uv[NO];
  if constexpr (MODE != 0 && MODE != 3) sc_load_mul_ir<T>(u + node * NO * C, C, cc, live, uv);
  if constexpr (MODE <= 2) {
    if constexpr (MODE == 0) {
      float o[NO];
#pragma unroll
      for (int i = 0; i < NO; ++i) o[i] = 0.f;
      PL::forward(xv, wr, C, o);
      if (live) sc_store_mul_ir<T>(out + node * NO * C, C, c, o);
    } else if constexpr (MODE == 1) {
      float dx[D];
      PL::vjp(xv, wr, C, uv, dx);
      if (live) sc_store_mul_ir<L>(out + node * D * C, C, c, dx);
    } else {
      // only lanes with a real channel store (the per-node block is [KTOT, C])
      float* __restrict__ phi = out + node * PL::KTOT * C + cc;
      if (live) PL::weight_features(xv, C, uv, phi);
    }
  } else {
    float tv[D];
    sc_load_mul_ir<L>(t + node * D * C, C, cc, live, tv);
    Dual xd[D];
#pragma unroll
    for (int i = 0; i < D; ++i) xd[i] = Dual(xv[i], tv[i]);
    if constexpr (MODE == 3) {
      Dual o[NO];
#pragma unroll
      for (int i = 0; i < NO; ++i) o[i] = 0.f;
      PL::forward(xd, wr, C, o);
      float r[NO];
#pragma unroll
      for (int i = 0; i < NO; ++i) r[i] = o[i].d;
      if (live) sc_store_mul_ir<T>(out + node * NO * C, C, c, r);
    } else if constexpr (MODE == 4) {
      Dual dx[D];
      PL::vjp(xd, wr, C, uv, dx);
      float r[D];
#pragma unroll
      for (int i = 0; i < D; ++i) r[i] = dx[i].d;
      if (live) sc_store_mul_ir<L>(out + node * D * C, C, c, r);
    } else {
      float* __restrict__ phi = out + node * PL::KTOT * C + cc;
      if (live) PL::weight_features(xd, C, uv, phi);
    }
  }
}

template <int L, int T, int K>
int launch_sc(int mode, const float* x, const float* t, const int64_t* species, const float* w,
              const float* u, float* out, int C, int64_t nodes, int num_species, hipStream_t stream) {
  const int nchunks = (C + kWave - 1) / kWave;
  const dim3 grid(static_cast<unsigned>((nodes * nchunks + kScWaves - 1) / kScWaves));
  switch (mode) {
#define ICTC_SC_MODE(M)                                                                                   \
  case M:                                                                                                 \
    hipLaunchKernelGGL((sc_kernel<L, T, K, M>), grid, dim3(kScBlock), 0, stream, x, t, species, w, u, out, \
                       C, nodes, num_species, nchunks);                                                   \
    break;
    ICTC_SC_MODE(0)
    ICTC_SC_MODE(1)
    ICTC_SC_MODE(2)
    ICTC_SC_MODE(3)
    ICTC_SC_MODE(4)
    ICTC_SC_MODE(5)
#undef ICTC_SC_MODE
    default:
      return ICTC_ERR_INVALID_ARGUMENT;
  }
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}

}  // namespace ictc
