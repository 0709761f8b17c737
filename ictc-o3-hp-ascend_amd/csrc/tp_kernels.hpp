// Channelwise path-preserving CG tensor product: forward and fused VJP (gfx950).
//
// Math (per instance e, path p = (l1,l2,l3), channel c, output component k):
//   M_p[e,i,k] = s_p * sum_j Y[e, l2^2+j] * Chat_p[i,j,k]            ("bond")
//   out[e, (o_p+k)*C + c] = g[e,p,c] * sum_i x[e, (l1^2+i)*C + c] * M_p[e,i,k]
// which is EdgeWeightedPathPreservingTensorProduct._forward_index_add
// (reference ictc_o3/basis/ictd_irreps.py:2669-2748) with the Y-side contracted
// first, as the reference's bond projection does (backends/ascend/tensor_product.py:30-55,
// structured_product.py:7-22).
//
// Launch shape: one 256-thread workgroup per tile of kFwdTile (forward) or kBwdTile (VJP)
// instances.
//   1. the tile's harmonics are staged in LDS and the bond matrices M_p of all
//      tile instances are built cooperatively into LDS (CG read from __constant__);
//   2. each wave then owns whole instances: lane l covers channels
//      [l*NV, l*NV+NV) (+64*NV per chunk), so every global access of a wave is one
//      contiguous run of 64*NV floats along the channel axis.  M_p is read from LDS
//      as a wave-uniform broadcast.
// The instance loop never round-trips intermediates through HBM: the forward reads
// x, Y, g once and writes out once; the VJP reads x, Y, g, dout once and writes
// dx, dY, dg once.
//
// Degree sets with an input degree of 4 take the VJP variant tp_backward_wide_kernel, which keeps
// only one input degree's x and dx rows in registers at a time (units compiled for those sets
// define ICTC_CG_WIDE and read the CG tables up to degree 4).
#pragma once
#include "ictc_common.hpp"
#ifdef ICTC_CG_WIDE
#include "generated/ictc_cg_table_wide.hpp"
#else
#include "generated/ictc_cg_table.hpp"
#endif

namespace ictc {

// instances per workgroup: one instance per wave in both kernels (a wave's next instance then
// starts in a fresh wave instead of behind this wave's output stores; measured best on gfx950
// at C128/lmax3: VJP 2.16 ms at 4 per workgroup, 2.18 at 8, 2.26 at 16, 2.28 at 32)
constexpr int kFwdTile = 4;
constexpr int kBwdTile = 4;
// The VJP requests the gate and dout rows of path p + kBwdPrefetch before it computes path p.
// Without that, each path's loads were issued behind the previous path's dg store and waited
// for together with it (gfx9's vmcnt counts loads and stores in one in-order counter, and the
// compiler cannot move a buffer load above a possibly aliasing buffer store), so every path
// paid a full memory round trip.  Measured at C128/lmax3 (16 instances per workgroup):
// 2.45 -> 2.26 ms (distance 1: 2.29 ms, 3 and 4: no further gain).
constexpr int kBwdPrefetch = 2;
constexpr int kBlock = 256;
constexpr int kWavesPerBlock = kBlock / kWave;

template <int LIN, int LE, int LOUT, int TILE, int NT = kBlock>
__device__ __forceinline__ void build_bond(const float (*sY)[Paths<LIN, LE, LOUT>::NY],
                                           float (*sM)[Paths<LIN, LE, LOUT>::NB > 0 ? Paths<LIN, LE, LOUT>::NB : 1],
                                           const ictc_tp_desc& d, int tid) {
  using PS = Paths<LIN, LE, LOUT>;
  static_for<0, PS::N>([&](auto P) {
    constexpr int p = P;
    constexpr int l1 = PS::tab.l1[p], l2 = PS::tab.l2[p], l3 = PS::tab.l3[p];
    constexpr int ni = 2 * l1 + 1, nj = 2 * l2 + 1, no = 2 * l3 + 1;
    constexpr int boff = PS::tab.bond[p];
    constexpr int cgo = CGTab<l1, l2, l3>::offset;
    const float s = d.scale[p];
    for (int t = tid; t < TILE * ni * no; t += NT) {
      const int e = t / (ni * no);
      const int r = t - e * (ni * no);  // M_p stored [k][i]: r = k*ni + i
      const int k = r / ni;
      const int i = r - k * ni;
      float acc = 0.f;
      static_for<0, nj>([&](auto J) {
        acc = fmaf(sY[e][l2 * l2 + J], kCGFlat[cgo + (i * nj + J) * no + k], acc);
      });
      sM[e][boff + r] = acc * s;
    }
  });
}

// Stage the tile's harmonics in LDS and build the bond matrices of all tile instances.
template <int LIN, int LE, int LOUT, int TILE, int NT = kBlock>
__device__ __forceinline__ void stage_tile(const float* __restrict__ y, int64_t e0, int64_t rows,
                                           float (*sY)[Paths<LIN, LE, LOUT>::NY],
                                           float (*sM)[Paths<LIN, LE, LOUT>::NB > 0 ? Paths<LIN, LE, LOUT>::NB : 1],
                                           const ictc_tp_desc& d, int tid) {
  constexpr int NY = Paths<LIN, LE, LOUT>::NY;
  for (int t = tid; t < TILE * NY; t += NT) {
    const int e = t / NY;
    sY[e][t - e * NY] = (e0 + e < rows) ? y[(e0 + e) * NY + (t - e * NY)] : 0.f;
  }
  __syncthreads();
  build_bond<LIN, LE, LOUT, TILE, NT>(sY, sM, d, tid);
  __syncthreads();
}

// Forward.  Per instance the wave issues every feature and gate load up front
// (NX + P row loads), then streams the NOC output rows; the path loop is fully
// unrolled with compile-time output offsets, so the instance body is branch-free.
template <int LIN, int LE, int LOUT, int NV>
__global__ void __launch_bounds__(kBlock)
tp_forward_kernel(const float* __restrict__ x, const float* __restrict__ y,
                  const float* __restrict__ g, float* __restrict__ out,
                  const ictc_tp_desc d, int64_t rows) {
  using PS = Paths<LIN, LE, LOUT>;
  constexpr int NX = PS::NX, NY = PS::NY, NP = PS::N, NOC = PS::NOC;
  constexpr int NBS = PS::NB > 0 ? PS::NB : 1;
  __shared__ float sY[kFwdTile][NY];
  __shared__ float sM[kFwdTile][NBS];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform (SGPR)
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kFwdTile;
  const int C = d.channels;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;  // bytes of one component row

  // The x rows of the wave's first instance and channel chunk are requested before the tile's
  // Y staging and bond build (two LDS barriers), so their latency overlaps that work; an
  // instance past the end gets an empty descriptor and its loads return zeros unread.
  // Holding them costs ~40 VGPRs (occupancy 4 -> 3 at lmax 3) and still measures 3% faster.
  const int64_t ew = e0 + wave;
  const rsrc_t rx0 = make_rsrc(ew < rows ? x + ew * NX * C : nullptr, NX * row);
  const uint32_t vo0 = static_cast<uint32_t>(lane * NV) * 4u;
  Vec<NV> xr0[NX];
#pragma unroll
  for (int m = 0; m < NX; ++m) xr0[m] = buf_load<NV>(rx0, vo0 + m * row);

  stage_tile<LIN, LE, LOUT, kFwdTile>(y, e0, rows, sY, sM, d, tid);

  for (int le = wave; le < kFwdTile; le += kWavesPerBlock) {
    const int64_t e = e0 + le;
    if (e >= rows) break;
    const rsrc_t rx = make_rsrc(x + e * NX * C, NX * row);
    const rsrc_t rg = make_rsrc(g + e * NP * C, NP * row);
    const rsrc_t ro = make_rsrc(out + e * NOC * C, NOC * row);
    for (int c = lane * NV; c < C; c += kWave * NV) {
      const uint32_t vo = static_cast<uint32_t>(c) * 4u;
      const float* __restrict__ bond = opaque_lds_row(&sM[le][0]);
      Vec<NV> xr[NX];
      Vec<NV> gv[NP];
      if (le == wave && c == lane * NV) {
#pragma unroll
        for (int m = 0; m < NX; ++m) xr[m] = xr0[m];
      } else {
#pragma unroll
        for (int m = 0; m < NX; ++m) xr[m] = buf_load<NV>(rx, vo + m * row);
      }
#pragma unroll
      for (int p = 0; p < NP; ++p) gv[p] = buf_load<NV>(rg, vo + p * row);
      static_for<0, NP>([&](auto P) {
        constexpr int p = P;
        constexpr int l1 = PS::tab.l1[p], l3 = PS::tab.l3[p];
        constexpr int ni = 2 * l1 + 1, no = 2 * l3 + 1;
        constexpr int boff = PS::tab.bond[p], oo = PS::tab.out[p];
        static_for<0, no>([&](auto K) {
          Vec<NV> acc;
#pragma unroll
          for (int v = 0; v < NV; ++v) acc.v[v] = 0.f;
          static_for<0, ni>([&](auto I) {
            const float m = bond[boff + K * ni + I];
#pragma unroll
            for (int v = 0; v < NV; ++v) acc.v[v] = fmaf(xr[l1 * l1 + I].v[v], m, acc.v[v]);
          });
#pragma unroll
          for (int v = 0; v < NV; ++v) acc.v[v] *= gv[p].v[v];
          buf_store<NV>(ro, vo + (oo + K) * row, acc);
        });
      });
    }
  }
}

// Fused VJP.  For each path:  go_k = g * dout_k
//   dx[l1,i]  += sum_k M_p[i,k] * go_k                        (structured_product.py:49-58)
//   dg[p]      = sum_k dout_k * sum_i x_i M_p[i,k]             (structured_product.py:75-87)
//   dY[l2,j]  += s_p * sum_{i,k} Chat_p[i,j,k] * sum_c x_i go_k  (structured_product.py:61-72
//                                                              composed with the bond adjoint)
// The dY channel sum is a per-lane partial followed by one wave reduction per instance.
// The path loop is software-pipelined: the gate and dout rows of path p + kBwdPrefetch are
// requested before path p is computed and its dg stored.
// The x, gate and dout rows are read exactly once and loaded with the non-temporal cache policy
// (measured at C128/lmax3: 2.16 -> 2.10 ms; the forward's loads measure slower with it).
// Outputs whose pointer is null get an empty buffer descriptor: their stores are
// dropped by the hardware range check, so the instance body has no branches.
// NV = 2 asks for three waves per SIMD (168 registers; the <3,3,3,2> instance needs 170 without
// the bound and measured 2.07 ms at two waves per SIMD, 2.04 ms at three).
template <int LIN, int LE, int LOUT, int NV>
__global__ void __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(NV == 2 ? 3 : 1)))
tp_backward_kernel(const float* __restrict__ x, const float* __restrict__ y,
                   const float* __restrict__ g, const float* __restrict__ go,
                   float* __restrict__ dx, float* __restrict__ dy, float* __restrict__ dg,
                   const ictc_tp_desc d, int64_t rows) {
  using PS = Paths<LIN, LE, LOUT>;
  constexpr int NX = PS::NX, NY = PS::NY, NP = PS::N, NOC = PS::NOC;
  constexpr int NBS = PS::NB > 0 ? PS::NB : 1;
  __shared__ float sY[kBwdTile][NY];
  __shared__ float sM[kBwdTile][NBS];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);  // wave-uniform (SGPR)
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kBwdTile;
  const int C = d.channels;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;
  // x rows of the wave's first instance and channel chunk requested before the tile's Y staging
  // and bond build, as in the forward (2.10 -> 2.06 ms at C128/lmax3, same occupancy, outputs
  // bit-identical); past the end, or without x, the descriptor is empty and the loads return 0
  const int64_t ew = e0 + wave;
  const rsrc_t rx0 = make_rsrc(ew < rows && x ? x + ew * NX * C : nullptr, NX * row);
  const uint32_t vo0 = static_cast<uint32_t>(lane * NV) * 4u;
  Vec<NV> xr0[NX];
#pragma unroll
  for (int m = 0; m < NX; ++m) xr0[m] = buf_load<NV, kNonTemporal>(rx0, vo0 + m * row);
  stage_tile<LIN, LE, LOUT, kBwdTile>(y, e0, rows, sY, sM, d, tid);

  for (int le = wave; le < kBwdTile; le += kWavesPerBlock) {
    const int64_t e = e0 + le;
    if (e >= rows) break;
    const rsrc_t rx = make_rsrc(x ? x + e * NX * C : nullptr, NX * row);
    const rsrc_t rg = make_rsrc(g + e * NP * C, NP * row);
    const rsrc_t rgo = make_rsrc(go + e * NOC * C, NOC * row);
    const rsrc_t rdx = make_rsrc(dx ? dx + e * NX * C : nullptr, NX * row);
    const rsrc_t rdg = make_rsrc(dg ? dg + e * NP * C : nullptr, NP * row);
    float dyl[NY];
#pragma unroll
    for (int j = 0; j < NY; ++j) dyl[j] = 0.f;
    for (int c = lane * NV; c < C; c += kWave * NV) {
      const uint32_t vo = static_cast<uint32_t>(c) * 4u;
      const float* __restrict__ bond = opaque_lds_row(&sM[le][0]);
      Vec<NV> xr[NX];
      Vec<NV> dxr[NX];
      if (le == wave && c == lane * NV) {
#pragma unroll
        for (int m = 0; m < NX; ++m) xr[m] = xr0[m];
      } else {
#pragma unroll
        for (int m = 0; m < NX; ++m) xr[m] = buf_load<NV, kNonTemporal>(rx, vo + m * row);
      }
#pragma unroll
      for (int m = 0; m < NX; ++m) {
#pragma unroll
        for (int v = 0; v < NV; ++v) dxr[m].v[v] = 0.f;
      }
      constexpr int D = kBwdPrefetch;
      Vec<NV> pre_g[D];                    // rows of the next D paths, in flight
      Vec<NV> pre_o[D][2 * LOUT + 1];
      auto request = [&](auto Q) {
        constexpr int q = Q;
        if constexpr (q < NP) {
          constexpr int nq = 2 * PS::tab.l3[q] + 1, oq = PS::tab.out[q];
          pre_g[q % D] = buf_load<NV, kNonTemporal>(rg, vo + q * row);
          static_for<0, nq>([&](auto K) { pre_o[q % D][K] = buf_load<NV, kNonTemporal>(rgo, vo + (oq + K) * row); });
        }
      };
      static_for<0, D>(request);
      static_for<0, NP>([&](auto P) {
        constexpr int p = P;
        constexpr int l1 = PS::tab.l1[p], l2 = PS::tab.l2[p], l3 = PS::tab.l3[p];
        constexpr int ni = 2 * l1 + 1, nj = 2 * l2 + 1, no = 2 * l3 + 1;
        constexpr int boff = PS::tab.bond[p];
        using CG = CGTab<l1, l2, l3>;
        const Vec<NV> gv = pre_g[p % D];
        Vec<NV> o[no];
        static_for<0, no>([&](auto K) { o[K] = pre_o[p % D][K]; });
        request(Int<p + D>{});             // issued ahead of this path's dg store
        // dg and dx in one pass over the bond entries: each M_p[i][k] is read once and used for
        // both (two passes kept the path's ni*no entries live in registers between them); every
        // dx row still accumulates in ascending k
        Vec<NV> dgv;
#pragma unroll
        for (int v = 0; v < NV; ++v) dgv.v[v] = 0.f;
        Vec<NV> gov[no];
        static_for<0, no>([&](auto K) {
#pragma unroll
          for (int v = 0; v < NV; ++v) gov[K].v[v] = gv.v[v] * o[K].v[v];
          Vec<NV> base;
#pragma unroll
          for (int v = 0; v < NV; ++v) base.v[v] = 0.f;
          static_for<0, ni>([&](auto I) {
            const float m = bond[boff + K * ni + I];
#pragma unroll
            for (int v = 0; v < NV; ++v) {
              base.v[v] = fmaf(xr[l1 * l1 + I].v[v], m, base.v[v]);
              dxr[l1 * l1 + I].v[v] = fmaf(m, gov[K].v[v], dxr[l1 * l1 + I].v[v]);
            }
          });
#pragma unroll
          for (int v = 0; v < NV; ++v) dgv.v[v] = fmaf(base.v[v], o[K].v[v], dgv.v[v]);
        });
        buf_store<NV>(rdg, vo + p * row, dgv);
        float part[nj];
#pragma unroll
        for (int j = 0; j < nj; ++j) part[j] = 0.f;
        static_for<0, ni>([&](auto I) {
          static_for<0, no>([&](auto K) {
            float t = 0.f;
#pragma unroll
            for (int v = 0; v < NV; ++v) t = fmaf(xr[l1 * l1 + I].v[v], gov[K].v[v], t);
            static_for<0, nj>([&](auto J) {
              constexpr float cg = CG::v[(I * nj + J) * no + K];
              if constexpr (cg != 0.0f) part[J] = fmaf(cg, t, part[J]);
            });
          });
        });
        const float s = d.scale[p];
#pragma unroll
        for (int j = 0; j < nj; ++j) dyl[l2 * l2 + j] = fmaf(s, part[j], dyl[l2 * l2 + j]);
      });
#pragma unroll
      for (int m = 0; m < NX; ++m) buf_store<NV>(rdx, vo + m * row, dxr[m]);
    }
    store_channel_sums<NY>(dyl, lane, make_rsrc(dy ? dy + e * NY : nullptr, NY * 4u));
  }
}

// First path of input degree a in the enumeration order (paths ascend in l1), or the path count.
template <int LIN, int LE, int LOUT>
constexpr int first_path_of_degree(int a) {
  constexpr PathTable t = Paths<LIN, LE, LOUT>::tab;
  for (int p = 0; p < t.n; ++p)
    if (t.l1[p] >= a) return p;
  return t.n;
}

// Fused VJP for wide degree sets (input degree 4: 25 x rows).  Same per-path arithmetic and
// output as tp_backward_kernel, reorganised by input degree: the x rows of degree a are
// requested while degree a - 1 is computed, and the dx rows of degree a are accumulated and
// stored with that degree, so x and dx occupy 2 (2a + 1) + (2a + 3) registers per channel
// instead of 2 NX.  One channel per lane (NV = 1), and one instance per single-wave workgroup:
// each wave builds its own bond rows, so no wave waits at a barrier for another's build.
// Measured at C64/(4,4,4), 65,536 instances: 300 registers with all x and dx rows resident (one
// wave per SIMD, 2.91 ms); 247 per degree (two waves, 1.89 ms); 118 with the single pass over
// the bond entries (four waves, 1.44 ms); one-wave workgroups 1.415 ms.
constexpr int kWideBlock = kWave;
template <int LIN, int LE, int LOUT>
__global__ void __launch_bounds__(kWideBlock)
tp_backward_wide_kernel(const float* __restrict__ x, const float* __restrict__ y,
                        const float* __restrict__ g, const float* __restrict__ go,
                        float* __restrict__ dx, float* __restrict__ dy, float* __restrict__ dg,
                        const ictc_tp_desc d, int64_t rows) {
  using PS = Paths<LIN, LE, LOUT>;
  constexpr int NX = PS::NX, NY = PS::NY, NP = PS::N, NOC = PS::NOC;
  constexpr int NBS = PS::NB > 0 ? PS::NB : 1;
  constexpr int WMAX = 2 * LIN + 1;
  __shared__ float sY[1][NY];
  __shared__ float sM[1][NBS];
  const int lane = threadIdx.x;
  const int64_t e = blockIdx.x;
  const int C = d.channels;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;
  stage_tile<LIN, LE, LOUT, 1, kWideBlock>(y, e, rows, sY, sM, d, lane);
  {
    const int le = 0;
    const rsrc_t rx = make_rsrc(x ? x + e * NX * C : nullptr, NX * row);
    const rsrc_t rg = make_rsrc(g + e * NP * C, NP * row);
    const rsrc_t rgo = make_rsrc(go + e * NOC * C, NOC * row);
    const rsrc_t rdx = make_rsrc(dx ? dx + e * NX * C : nullptr, NX * row);
    const rsrc_t rdg = make_rsrc(dg ? dg + e * NP * C : nullptr, NP * row);
    float dyl[NY];
#pragma unroll
    for (int j = 0; j < NY; ++j) dyl[j] = 0.f;
    for (int c = lane; c < C; c += kWave) {
      const uint32_t vo = static_cast<uint32_t>(c) * 4u;
      const float* __restrict__ bond = opaque_lds_row(&sM[le][0]);
      constexpr int D = kBwdPrefetch;
      float pre_g[D];                      // rows of the next D paths, in flight
      float pre_o[D][2 * LOUT + 1];
      auto request = [&](auto Q) {
        constexpr int q = Q;
        if constexpr (q < NP) {
          constexpr int nq = 2 * PS::tab.l3[q] + 1, oq = PS::tab.out[q];
          pre_g[q % D] = buf_load<1, kNonTemporal>(rg, vo + q * row).v[0];
          static_for<0, nq>([&](auto K) { pre_o[q % D][K] = buf_load<1, kNonTemporal>(rgo, vo + (oq + K) * row).v[0]; });
        }
      };
      float xn[WMAX];                      // the next input degree's x rows, in flight
      xn[0] = buf_load<1, kNonTemporal>(rx, vo).v[0];
      static_for<0, D>(request);
      static_for<0, LIN + 1>([&](auto A) {
        constexpr int a = A, ni = 2 * a + 1;
        constexpr int p0 = first_path_of_degree<LIN, LE, LOUT>(a), p1 = first_path_of_degree<LIN, LE, LOUT>(a + 1);
        float xr[ni], dxr[ni];
#pragma unroll
        for (int i = 0; i < ni; ++i) {
          xr[i] = xn[i];
          dxr[i] = 0.f;
        }
        if constexpr (a < LIN) {
#pragma unroll
          for (int i = 0; i < ni + 2; ++i) xn[i] = buf_load<1, kNonTemporal>(rx, vo + ((a + 1) * (a + 1) + i) * row).v[0];
        }
        static_for<p0, p1>([&](auto P) {
          constexpr int p = P;
          constexpr int l2 = PS::tab.l2[p], l3 = PS::tab.l3[p];
          constexpr int nj = 2 * l2 + 1, no = 2 * l3 + 1;
          constexpr int boff = PS::tab.bond[p];
          using CG = CGTab<a, l2, l3>;
          const float gv = pre_g[p % D];
          float o[no];
          static_for<0, no>([&](auto K) { o[K] = pre_o[p % D][K]; });
          request(Int<p + D>{});           // issued ahead of this path's dg store
          float dgv = 0.f;
          float gov[no];
          static_for<0, no>([&](auto K) {
            gov[K] = gv * o[K];
            float base = 0.f;
            static_for<0, ni>([&](auto I) {
              const float m = bond[boff + K * ni + I];
              base = fmaf(xr[I], m, base);
              dxr[I] = fmaf(m, gov[K], dxr[I]);
            });
            dgv = fmaf(base, o[K], dgv);
          });
          buf_store<1>(rdg, vo + p * row, Vec<1>{{dgv}});
          float part[nj];
#pragma unroll
          for (int j = 0; j < nj; ++j) part[j] = 0.f;
          static_for<0, ni>([&](auto I) {
            static_for<0, no>([&](auto K) {
              const float t = xr[I] * gov[K];
              static_for<0, nj>([&](auto J) {
                constexpr float cg = CG::v[(I * nj + J) * no + K];
                if constexpr (cg != 0.0f) part[J] = fmaf(cg, t, part[J]);
              });
            });
          });
          const float s = d.scale[p];
#pragma unroll
          for (int j = 0; j < nj; ++j) dyl[l2 * l2 + j] = fmaf(s, part[j], dyl[l2 * l2 + j]);
        });
#pragma unroll
        for (int i = 0; i < ni; ++i) buf_store<1>(rdx, vo + (a * a + i) * row, Vec<1>{{dxr[i]}});
      });
    }
    store_channel_sums<NY>(dyl, lane, make_rsrc(dy ? dy + e * NY : nullptr, NY * 4u));
  }
}

// ----------------------------------------------------------------------------- launchers
using FwdLaunch = int (*)(const ictc_tp_desc&, const float*, const float*, const float*, float*,
                          int64_t, hipStream_t);
using BwdLaunch = int (*)(const ictc_tp_desc&, const float*, const float*, const float*,
                          const float*, float*, float*, float*, int64_t, hipStream_t);

inline int launch_status() { return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH; }

template <int LIN, int LE, int LOUT>
int launch_forward(const ictc_tp_desc& d, const float* x, const float* y, const float* g, float* out,
                   int64_t rows, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((rows + kFwdTile - 1) / kFwdTile));
  if (d.channels % (2 * kWave) == 0)
    hipLaunchKernelGGL((tp_forward_kernel<LIN, LE, LOUT, 2>), grid, dim3(kBlock), 0, stream, x, y, g,
                       out, d, rows);
  else
    hipLaunchKernelGGL((tp_forward_kernel<LIN, LE, LOUT, 1>), grid, dim3(kBlock), 0, stream, x, y, g,
                       out, d, rows);
  return launch_status();
}

template <int LIN, int LE, int LOUT>
int launch_backward(const ictc_tp_desc& d, const float* x, const float* y, const float* g,
                    const float* go, float* dx, float* dy, float* dg, int64_t rows, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((rows + kBwdTile - 1) / kBwdTile));
  if constexpr (LIN >= 4) {
    if (rows > 0x7fffffff) return ICTC_ERR_INVALID_ARGUMENT;   // one workgroup per instance
    hipLaunchKernelGGL((tp_backward_wide_kernel<LIN, LE, LOUT>), dim3(static_cast<unsigned>(rows)),
                       dim3(kWideBlock), 0, stream, x, y, g, go, dx, dy, dg, d, rows);
  } else if (d.channels % (2 * kWave) == 0)
    hipLaunchKernelGGL((tp_backward_kernel<LIN, LE, LOUT, 2>), grid, dim3(kBlock), 0, stream, x, y, g,
                       go, dx, dy, dg, d, rows);
  else
    hipLaunchKernelGGL((tp_backward_kernel<LIN, LE, LOUT, 1>), grid, dim3(kBlock), 0, stream, x, y, g,
                       go, dx, dy, dg, d, rows);
  return launch_status();
}

}  // namespace ictc
