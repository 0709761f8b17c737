// Graph message: fused gather -> channelwise TP -> receiver segmented sum (gfx950).
//
//   out[n] = sum_{e : dst(e) = n} TP(x[src(e)], Y[e], g[e])
// which is the CPU semantics of reference backends/ascend/tensor_product.py:189-218
// (index_select(src) -> TP -> index_add(dst)) and of the MACE interaction
// (mace_ictc/models/pure_cartesian_ictd_fix.py:1801-1917), with the per-edge TP of
// tp_kernels.hpp.  An optional edge mask is folded into the gates by the caller.
//
// No atomics, deterministic order: edges are visited through a CSR over the
// receivers (rowptr_dst + slot->edge permutation), each destination node is owned by
// one wave per 64-channel chunk and accumulated in registers, so per-edge messages
// never touch HBM.  The VJP splits into
//   * msg_edge_grad_kernel (receiver CSR): per edge dY and dg, reading dout[n] once
//     per node (held in registers) and gathering x[src];
//   * msg_node_grad_kernel (source CSR): dx[s] = sum over the out-edges of s of the TP
//     feature adjoint, gathering dout[dst].
// Node-feature and cotangent gathers go through buffer descriptors spanning the whole
// node tensor, so an out-of-range index reads zeros instead of faulting; the host
// validates indices before launch.
#pragma once
#include "ictc_common.hpp"
#include "generated/ictc_cg_table.hpp"

namespace ictc {

constexpr int kMsgBlock = 256;
constexpr int kMsgWaves = kMsgBlock / kWave;

// LDS -> LDS visibility inside one wave: wait for this wave's LDS traffic.
__device__ __forceinline__ void wave_lds_sync() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
}

// Bond matrices of one edge, built by the 64 lanes of a wave into its LDS row.
// yv: wave-uniform harmonics of the edge.
template <int LIN, int LE, int LOUT>
__device__ __forceinline__ void wave_bond(const float* yv, float* __restrict__ row,
                                          const ictc_tp_desc& d, int lane) {
  using PS = Paths<LIN, LE, LOUT>;
  static_for<0, PS::N>([&](auto P) {
    constexpr int p = P;
    constexpr int l1 = PS::tab.l1[p], l2 = PS::tab.l2[p], l3 = PS::tab.l3[p];
    constexpr int ni = 2 * l1 + 1, nj = 2 * l2 + 1, no = 2 * l3 + 1;
    constexpr int boff = PS::tab.bond[p];
    constexpr int cgo = CGTab<l1, l2, l3>::offset;
    if (lane < ni * no) {
      const int k = lane / ni;
      const int i = lane - k * ni;
      float acc = 0.f;
      static_for<0, nj>([&](auto J) {
        acc = fmaf(yv[l2 * l2 + J], kCGFlat[cgo + (i * nj + J) * no + k], acc);
      });
      row[boff + lane] = acc * d.scale[p];
    }
  });
  wave_lds_sync();
}

// ----------------------------------------------------------------------------- forward
template <int LIN, int LE, int LOUT>
__global__ void __launch_bounds__(kMsgBlock)
msg_forward_kernel(const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ g,
                   const int64_t* __restrict__ src, const int64_t* __restrict__ rowptr,
                   const int64_t* __restrict__ perm, float* __restrict__ out, const ictc_tp_desc d,
                   int64_t nodes_src, int64_t nodes_dst, int nchunks) {
  using PS = Paths<LIN, LE, LOUT>;
  constexpr int NX = PS::NX, NY = PS::NY, NP = PS::N, NOC = PS::NOC;
  constexpr int NBS = PS::NB > 0 ? PS::NB : 1;
  __shared__ float sB[kMsgWaves][NBS];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kMsgWaves + wave;
  const int64_t node = item / nchunks;
  if (node >= nodes_dst) return;
  const int chunk = static_cast<int>(item - node * nchunks);
  const int C = d.channels;
  const int c = chunk * kWave + lane;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;
  const uint32_t vo = static_cast<uint32_t>(c) * 4u;
  const bool live = c < C;
  // whole-tensor descriptors: gathers are range checked
  const rsrc_t rx = make_rsrc(x, static_cast<uint32_t>(nodes_src * NX * row));
  float* bond = &sB[wave][0];
  float acc[NOC];
#pragma unroll
  for (int r = 0; r < NOC; ++r) acc[r] = 0.f;
  const int64_t s0 = rowptr[node], s1 = rowptr[node + 1];
  for (int64_t slot = s0; slot < s1; ++slot) {
    const int64_t e = perm ? perm[slot] : slot;
    const int64_t s = src[e];
    float yv[NY];
#pragma unroll
    for (int j = 0; j < NY; ++j) yv[j] = y[e * NY + j];
    wave_bond<LIN, LE, LOUT>(yv, bond, d, lane);
    const uint32_t xoff = static_cast<uint32_t>(s) * NX * row + vo;
    float xr[NX];
#pragma unroll
    for (int m = 0; m < NX; ++m) {
      const float v = buf_load<1>(rx, xoff + m * row).v[0];
      xr[m] = live ? v : 0.f;
    }
    const rsrc_t rg = make_rsrc(g + e * NP * C, NP * row);
    float gv[NP];
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      const float v = buf_load<1>(rg, vo + p * row).v[0];
      gv[p] = live ? v : 0.f;
    }
    static_for<0, NP>([&](auto P) {
      constexpr int p = P;
      constexpr int l1 = PS::tab.l1[p], l3 = PS::tab.l3[p];
      constexpr int ni = 2 * l1 + 1, no = 2 * l3 + 1;
      constexpr int boff = PS::tab.bond[p], oo = PS::tab.out[p];
      static_for<0, no>([&](auto K) {
        float t = 0.f;
        static_for<0, ni>([&](auto I) { t = fmaf(xr[l1 * l1 + I], bond[boff + K * ni + I], t); });
        acc[oo + K] = fmaf(t, gv[p], acc[oo + K]);
      });
    });
  }
  if (live) {
    float* __restrict__ on = out + node * NOC * C;
#pragma unroll
    for (int r = 0; r < NOC; ++r) __builtin_nontemporal_store(acc[r], on + r * C + c);
  }
}

// ----------------------------------------------------------------------------- VJP: per edge
// dg[e] (raw, unmasked) and dY partials per (edge, chunk): dyp[e*nchunks + chunk][NY].
template <int LIN, int LE, int LOUT>
__global__ void __launch_bounds__(kMsgBlock)
msg_edge_grad_kernel(const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ g,
                     const float* __restrict__ go, const int64_t* __restrict__ src,
                     const int64_t* __restrict__ rowptr, const int64_t* __restrict__ perm,
                     float* __restrict__ dyp, float* __restrict__ dg, const ictc_tp_desc d,
                     int64_t nodes_src, int64_t nodes_dst, int nchunks) {
  using PS = Paths<LIN, LE, LOUT>;
  constexpr int NX = PS::NX, NY = PS::NY, NP = PS::N, NOC = PS::NOC;
  constexpr int NBS = PS::NB > 0 ? PS::NB : 1;
  __shared__ float sB[kMsgWaves][NBS];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kMsgWaves + wave;
  const int64_t node = item / nchunks;
  if (node >= nodes_dst) return;
  const int chunk = static_cast<int>(item - node * nchunks);
  const int C = d.channels;
  const int c = chunk * kWave + lane;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;
  const uint32_t vo = static_cast<uint32_t>(c) * 4u;
  const bool live = c < C;
  const rsrc_t rx = make_rsrc(x, static_cast<uint32_t>(nodes_src * NX * row));
  float* bond = &sB[wave][0];
  float o[NOC];
  {
    const rsrc_t ron = make_rsrc(go + node * NOC * C, NOC * row);
#pragma unroll
    for (int r = 0; r < NOC; ++r) {
      const float v = buf_load<1>(ron, vo + r * row).v[0];
      o[r] = live ? v : 0.f;
    }
  }
  const int64_t s0 = rowptr[node], s1 = rowptr[node + 1];
  for (int64_t slot = s0; slot < s1; ++slot) {
    const int64_t e = perm ? perm[slot] : slot;
    const int64_t s = src[e];
    float yv[NY];
#pragma unroll
    for (int j = 0; j < NY; ++j) yv[j] = y[e * NY + j];
    wave_bond<LIN, LE, LOUT>(yv, bond, d, lane);
    const uint32_t xoff = static_cast<uint32_t>(s) * NX * row + vo;
    float xr[NX];
#pragma unroll
    for (int m = 0; m < NX; ++m) {
      const float v = buf_load<1>(rx, xoff + m * row).v[0];
      xr[m] = live ? v : 0.f;
    }
    const rsrc_t rg = make_rsrc(g + e * NP * C, NP * row);
    float* __restrict__ dge = dg ? dg + e * NP * C : nullptr;
    float dyl[NY];
#pragma unroll
    for (int j = 0; j < NY; ++j) dyl[j] = 0.f;
    static_for<0, NP>([&](auto P) {
      constexpr int p = P;
      constexpr int l1 = PS::tab.l1[p], l2 = PS::tab.l2[p], l3 = PS::tab.l3[p];
      constexpr int ni = 2 * l1 + 1, nj = 2 * l2 + 1, no = 2 * l3 + 1;
      constexpr int boff = PS::tab.bond[p], oo = PS::tab.out[p];
      using CG = CGTab<l1, l2, l3>;
      const float gl = buf_load<1>(rg, vo + p * row).v[0];
      const float gv = live ? gl : 0.f;
      float dgv = 0.f;
      static_for<0, no>([&](auto K) {
        float base = 0.f;
        static_for<0, ni>([&](auto I) { base = fmaf(xr[l1 * l1 + I], bond[boff + K * ni + I], base); });
        dgv = fmaf(base, o[oo + K], dgv);
      });
      if (dge != nullptr && live) __builtin_nontemporal_store(dgv, dge + p * C + c);
      float part[nj];
#pragma unroll
      for (int j = 0; j < nj; ++j) part[j] = 0.f;
      static_for<0, ni>([&](auto I) {
        static_for<0, no>([&](auto K) {
          const float t = xr[l1 * l1 + I] * (gv * o[oo + K]);
          static_for<0, nj>([&](auto J) {
            constexpr float cg = CG::v[(I * nj + J) * no + K];
            if constexpr (cg != 0.0f) part[J] = fmaf(cg, t, part[J]);
          });
        });
      });
      const float sc = d.scale[p];
#pragma unroll
      for (int j = 0; j < nj; ++j) dyl[l2 * l2 + j] = fmaf(sc, part[j], dyl[l2 * l2 + j]);
    });
    if (dyp != nullptr) {
      float mine = 0.f;
#pragma unroll
      for (int j = 0; j < NY; ++j) {
        const float tot = wave_sum(dyl[j]);
        if (lane == j) mine = tot;
      }
      if (lane < NY) dyp[(e * nchunks + chunk) * NY + lane] = mine;
    }
  }
}

// ----------------------------------------------------------------------------- VJP: per source node
// dx[s] = sum over edges with src(e) = s of sum_p sum_k M_p[e](:,k) g[e,p] dout[dst(e)]_k.
template <int LIN, int LE, int LOUT>
__global__ void __launch_bounds__(kMsgBlock)
msg_node_grad_kernel(const float* __restrict__ y, const float* __restrict__ g,
                     const float* __restrict__ go, const int64_t* __restrict__ dst,
                     const int64_t* __restrict__ rowptr_src, const int64_t* __restrict__ perm_src,
                     float* __restrict__ dx, const ictc_tp_desc d, int64_t nodes_src, int64_t nodes_dst,
                     int nchunks) {
  using PS = Paths<LIN, LE, LOUT>;
  constexpr int NX = PS::NX, NY = PS::NY, NP = PS::N, NOC = PS::NOC;
  constexpr int NBS = PS::NB > 0 ? PS::NB : 1;
  __shared__ float sB[kMsgWaves][NBS];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int64_t item = static_cast<int64_t>(blockIdx.x) * kMsgWaves + wave;
  const int64_t node = item / nchunks;
  if (node >= nodes_src) return;
  const int chunk = static_cast<int>(item - node * nchunks);
  const int C = d.channels;
  const int c = chunk * kWave + lane;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;
  const uint32_t vo = static_cast<uint32_t>(c) * 4u;
  const bool live = c < C;
  const rsrc_t rgo = make_rsrc(go, static_cast<uint32_t>(nodes_dst * NOC * row));
  float* bond = &sB[wave][0];
  float dxr[NX];
#pragma unroll
  for (int m = 0; m < NX; ++m) dxr[m] = 0.f;
  const int64_t s0 = rowptr_src[node], s1 = rowptr_src[node + 1];
  for (int64_t slot = s0; slot < s1; ++slot) {
    const int64_t e = perm_src ? perm_src[slot] : slot;
    const int64_t t = dst[e];
    float yv[NY];
#pragma unroll
    for (int j = 0; j < NY; ++j) yv[j] = y[e * NY + j];
    wave_bond<LIN, LE, LOUT>(yv, bond, d, lane);
    const uint32_t ooff = static_cast<uint32_t>(t) * NOC * row + vo;
    const rsrc_t rg = make_rsrc(g + e * NP * C, NP * row);
    static_for<0, NP>([&](auto P) {
      constexpr int p = P;
      constexpr int l1 = PS::tab.l1[p], l3 = PS::tab.l3[p];
      constexpr int ni = 2 * l1 + 1, no = 2 * l3 + 1;
      constexpr int boff = PS::tab.bond[p], oo = PS::tab.out[p];
      const float gl = buf_load<1>(rg, vo + p * row).v[0];
      const float gv = live ? gl : 0.f;
      float gov[no];
      static_for<0, no>([&](auto K) { gov[K] = gv * buf_load<1>(rgo, ooff + (oo + K) * row).v[0]; });
      static_for<0, ni>([&](auto I) {
        static_for<0, no>([&](auto K) {
          dxr[l1 * l1 + I] = fmaf(bond[boff + K * ni + I], gov[K], dxr[l1 * l1 + I]);
        });
      });
    });
  }
  if (live) {
    float* __restrict__ dxn = dx + node * NX * C;
#pragma unroll
    for (int m = 0; m < NX; ++m) __builtin_nontemporal_store(dxr[m], dxn + m * C + c);
  }
}

// ----------------------------------------------------------------------------- launchers
inline int msg_launch_status() { return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH; }

inline dim3 msg_grid(int64_t nodes, int nchunks) {
  return dim3(static_cast<unsigned>((nodes * nchunks + kMsgWaves - 1) / kMsgWaves));
}

template <int LIN, int LE, int LOUT>
int launch_msg_forward(const ictc_tp_desc& d, const float* x, const float* y, const float* g,
                       const int64_t* src, const int64_t* rowptr, const int64_t* perm, float* out,
                       int64_t nodes_src, int64_t nodes_dst, hipStream_t stream) {
  const int nchunks = (d.channels + kWave - 1) / kWave;
  hipLaunchKernelGGL((msg_forward_kernel<LIN, LE, LOUT>), msg_grid(nodes_dst, nchunks), dim3(kMsgBlock), 0,
                     stream, x, y, g, src, rowptr, perm, out, d, nodes_src, nodes_dst, nchunks);
  return msg_launch_status();
}

template <int LIN, int LE, int LOUT>
int launch_msg_edge_grad(const ictc_tp_desc& d, const float* x, const float* y, const float* g,
                         const float* go, const int64_t* src, const int64_t* rowptr, const int64_t* perm,
                         float* dyp, float* dg, int64_t nodes_src, int64_t nodes_dst, hipStream_t stream) {
  const int nchunks = (d.channels + kWave - 1) / kWave;
  hipLaunchKernelGGL((msg_edge_grad_kernel<LIN, LE, LOUT>), msg_grid(nodes_dst, nchunks), dim3(kMsgBlock),
                     0, stream, x, y, g, go, src, rowptr, perm, dyp, dg, d, nodes_src, nodes_dst, nchunks);
  return msg_launch_status();
}

template <int LIN, int LE, int LOUT>
int launch_msg_node_grad(const ictc_tp_desc& d, const float* y, const float* g, const float* go,
                         const int64_t* dst, const int64_t* rowptr_src, const int64_t* perm_src, float* dx,
                         int64_t nodes_src, int64_t nodes_dst, hipStream_t stream) {
  const int nchunks = (d.channels + kWave - 1) / kWave;
  hipLaunchKernelGGL((msg_node_grad_kernel<LIN, LE, LOUT>), msg_grid(nodes_src, nchunks), dim3(kMsgBlock),
                     0, stream, y, g, go, dst, rowptr_src, perm_src, dx, d, nodes_src, nodes_dst, nchunks);
  return msg_launch_status();
}

}  // namespace ictc
