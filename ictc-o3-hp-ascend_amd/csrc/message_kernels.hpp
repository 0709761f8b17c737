// Graph message: fused gather -> channelwise TP -> receiver segmented sum (gfx950).
//
//   out[n] = sum_{e : dst(e) = n} TP(x[src(e)], Y[e], g[e])
// which is the CPU semantics of reference backends/ascend/tensor_product.py:189-218
// (index_select(src) -> TP -> index_add(dst)) and of the MACE interaction
// (mace_ictc/models/pure_cartesian_ictd_fix.py:1801-1917).  An optional edge mask is
// folded into the gates by the caller.
//
// Kernels (no atomics, deterministic order):
//   * msg_bond_kernel: per-edge bond matrices M_p[e][k][i] = s_p sum_j Y[e,j] C_p[i,j,k]
//     for every path (the reference's Y @ P bond projection, backends/ascend/
//     tensor_product.py:9-57 and structured_product.py:7-22), computed once per edge and
//     shared by every kernel below and by every channel chunk (for small degree sets the
//     kernels below build each row themselves from the harmonics instead: bond_inline);
//   * msg_forward_kernel (receiver CSR): one block per (node, 64-channel chunk); its waves
//     split the node's edges and accumulate in registers, then sum their partials in a
//     fixed order through LDS; per edge, the x[src] row, the gates and the bond row are
//     requested together (one round trip), the bond row is staged in the wave's LDS row,
//     and the kernel is kept small enough in registers that several waves per SIMD hide
//     the latency;
//   * msg_forward_degree_kernel (degree sets with a bond buffer): the forward and its tangent,
//     one launch per input degree with two channel chunks per lane;
//   * msg_edge_grad_degree_kernel (receiver CSR, every degree set): one block per (node, channel
//     chunk) contracts the node's dout rows with the CG tensors once, into LDS, and its waves
//     split the node's edges; per edge dg, dY partials and the edge's contribution to the
//     source-feature adjoint dxe[e] = sum_p g_p M_p^T dout[dst(e)] (so dout is never gathered
//     per edge), from the edge's harmonics row (no bond rows), in one pass per input degree
//     (first order or tangent);
//   * msg_node_grad_kernel (source CSR): dx[s] = sum over the out-edges of s of dxe[e],
//     a streaming segmented sum.
// Node-feature gathers go through buffer descriptors spanning the whole node tensor,
// so an out-of-range index reads zeros instead of faulting; the host validates indices
// before launch.
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

// Offset of CG(l1,l2,l3) in kCGFlat (generated table order: l1, l2, l3 ascending over
// the allowed triples with every degree <= 3).
constexpr int cg_flat_offset(int a, int b, int c) {
  int off = 0;
  for (int l1 = 0; l1 <= 3; ++l1)
    for (int l2 = 0; l2 <= 3; ++l2)
      for (int l3 = (l1 > l2 ? l1 - l2 : l2 - l1); l3 <= (l1 + l2 < 3 ? l1 + l2 : 3); ++l3) {
        if ((l1 + l2 + l3) & 1) continue;
        if (l1 == a && l2 == b && l3 == c) return off;
        off += (2 * l1 + 1) * (2 * l2 + 1) * (2 * l3 + 1);
      }
  return -1;
}
static_assert(cg_flat_offset(1, 2, 3) == CGTab<1, 2, 3>::offset, "CG table order");
static_assert(cg_flat_offset(3, 3, 2) == CGTab<3, 3, 2>::offset, "CG table order");

// Per bond entry (path p, row k, column i): the kCGFlat index of C_p[i, 0, k] and
// meta = p | nj << 6 | no << 9 | l2^2 << 12.
template <int LIN, int LE, int LOUT>
struct BondMap {
  static constexpr int NB = Paths<LIN, LE, LOUT>::NB;
  uint16_t cg[NB > 0 ? NB : 1];
  uint16_t meta[NB > 0 ? NB : 1];
};

template <int LIN, int LE, int LOUT>
constexpr BondMap<LIN, LE, LOUT> make_bond_map() {
  BondMap<LIN, LE, LOUT> m{};
  constexpr PathTable t = Paths<LIN, LE, LOUT>::tab;
  for (int p = 0; p < t.n; ++p) {
    const int ni = 2 * t.l1[p] + 1, nj = 2 * t.l2[p] + 1, no = 2 * t.l3[p] + 1;
    const int cgo = cg_flat_offset(t.l1[p], t.l2[p], t.l3[p]);
    for (int q = 0; q < ni * no; ++q) {
      const int k = q / ni, i = q - k * ni;
      m.cg[t.bond[p] + q] = static_cast<uint16_t>(cgo + i * nj * no + k);
      m.meta[t.bond[p] + q] = static_cast<uint16_t>(p | nj << 6 | no << 9 | (t.l2[p] * t.l2[p]) << 12);
    }
  }
  return m;
}

template <int LIN, int LE, int LOUT>
__constant__ BondMap<LIN, LE, LOUT> kBondMap = make_bond_map<LIN, LE, LOUT>();

// ----------------------------------------------------------------------------- bonds
// bonds[e, :] = Y[e, :] @ P with the constant projection P[j][entry] = s_p C_p[i, j - l2^2, k]
// on the entry's own degree block (zero elsewhere): a GEMM with K = (L_e+1)^2.  Thread t owns
// bond entries t, t + 256 (its P columns live in registers), the block stages kBondEdges
// harmonics rows in LDS and walks them: per edge the Y row is a wave-uniform LDS broadcast and
// every wave writes 64 consecutive entries of the row (coalesced, non-temporal).  Small tiles
// keep many workgroups' stores in flight: measured at lmax 3 over 105,634 edges, 91 us with a
// per-block LDS table of P and 64 edges per block, 60 us here (8 edges; 72 us at 16, 77 at 4),
// bit-identical (same products, same FMA order).
constexpr int kBondEdges = 8;

template <int LIN, int LE, int LOUT>
__global__ void __launch_bounds__(256)
msg_bond_kernel(const float* __restrict__ y, float* __restrict__ bonds, const ictc_tp_desc d, int64_t edges) {
  using PS = Paths<LIN, LE, LOUT>;
  constexpr int NB = PS::NB, NY = PS::NY;
  constexpr int NCOL = NB > 0 ? (NB + 255) / 256 : 1;
  __shared__ float sY[kBondEdges * NY];
  const int tid = threadIdx.x;
  float P[NCOL][NY];
#pragma unroll
  for (int c = 0; c < NCOL; ++c) {
    const int idx = tid + 256 * c;
    const bool live = idx < NB;
    const int cg = live ? kBondMap<LIN, LE, LOUT>.cg[idx] : 0;
    const int meta = live ? kBondMap<LIN, LE, LOUT>.meta[idx] : 0;
    const int p = meta & 63, nj = (meta >> 6) & 7, no = (meta >> 9) & 7, y0 = meta >> 12;
    const float sc = d.scale[p];
#pragma unroll
    for (int j = 0; j < NY; ++j) {
      const int jj = j - y0;
      P[c][j] = (live && jj >= 0 && jj < nj) ? kCGFlat[cg + jj * no] * sc : 0.f;
    }
  }
  const int64_t e0 = static_cast<int64_t>(blockIdx.x) * kBondEdges;
  const int ne = static_cast<int>(edges - e0 < kBondEdges ? edges - e0 : kBondEdges);
  for (int t = tid; t < ne * NY; t += 256) sY[t] = y[e0 * NY + t];
  __syncthreads();
  float* __restrict__ out = bonds + e0 * NB;
#pragma unroll 4
  for (int le = 0; le < ne; ++le) {
    float yv[NY];
#pragma unroll
    for (int j = 0; j < NY; ++j) yv[j] = sY[le * NY + j];
#pragma unroll
    for (int c = 0; c < NCOL; ++c) {
      const int idx = tid + 256 * c;
      if (idx < NB) {
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < NY; ++j) acc = fmaf(yv[j], P[c][j], acc);
        __builtin_nontemporal_store(acc, out + static_cast<int64_t>(le) * NB + idx);
      }
    }
  }
}

// Bond row of one edge staged by the wave: lane l holds entries l, l + 64, ...
template <int NB>
struct BondStage {
  static constexpr int NV = NB > 0 ? (NB + kWave - 1) / kWave : 1;
  float v[NV];
};

template <int NB>
__device__ __forceinline__ void bond_fetch(const float* __restrict__ bonds, int64_t e, int lane,
                                           BondStage<NB>& s) {
  const rsrc_t rb = make_rsrc(bonds + e * NB, NB * 4u);
#pragma unroll
  for (int r = 0; r < BondStage<NB>::NV; ++r) s.v[r] = buf_load<1>(rb, (lane + r * kWave) * 4u).v[0];
}

// In-kernel bond rows.  When a lane's share of the bond row (BondStage::NV entries) times the
// NY harmonics fits in 32 registers, the kernels form each edge's bond row themselves from its
// harmonics row, with the products and the accumulation order of msg_bond_kernel (so the rows
// are bit-identical), and no bond buffer exists: the caller passes the harmonics where the
// bond rows would go (ictc_hip_message_bond_width reports 0).  This saves the bond kernel and
// the bond-row traffic (115 floats per edge at lmax 2 against 9 harmonics).
constexpr bool bond_inline(int nb, int ny) { return nb > 0 && ((nb + kWave - 1) / kWave) * ny <= 32; }

template <int LIN, int LE, int LOUT>
struct BondInline {
  static constexpr bool value = bond_inline(Paths<LIN, LE, LOUT>::NB, Paths<LIN, LE, LOUT>::NY);
};

// Dense per-entry view of the projection for the in-kernel rows: cg[idx][j] = C_p[i, j - l2^2, k]
// on the entry's l2 block (0 elsewhere) and the entry's path, for every entry slot a wave's
// lanes own (slots past NB are all zero), so each lane loads its coefficients without branches.
template <int LIN, int LE, int LOUT>
struct BondDense {
  static constexpr int NB = Paths<LIN, LE, LOUT>::NB, NY = Paths<LIN, LE, LOUT>::NY;
  static constexpr int NS = BondStage<NB>::NV * kWave;
  float cg[NS][NY];
  uint8_t path[NS];
};

template <int LIN, int LE, int LOUT, int P = 0>
constexpr void fill_bond_dense(BondDense<LIN, LE, LOUT>& t) {
  if constexpr (P < Paths<LIN, LE, LOUT>::N) {
    constexpr PathTable tab = Paths<LIN, LE, LOUT>::tab;
    constexpr int l1 = tab.l1[P], l2 = tab.l2[P], l3 = tab.l3[P];
    constexpr int ni = 2 * l1 + 1, nj = 2 * l2 + 1, no = 2 * l3 + 1;
    using CG = CGTab<l1, l2, l3>;
    for (int q = 0; q < ni * no; ++q) {
      const int k = q / ni, i = q - k * ni, idx = tab.bond[P] + q;
      t.path[idx] = static_cast<uint8_t>(P);
      for (int jj = 0; jj < nj; ++jj) t.cg[idx][l2 * l2 + jj] = CG::v[(i * nj + jj) * no + k];
    }
    fill_bond_dense<LIN, LE, LOUT, P + 1>(t);
  }
}

template <int LIN, int LE, int LOUT>
constexpr BondDense<LIN, LE, LOUT> make_bond_dense() {
  BondDense<LIN, LE, LOUT> t{};
  fill_bond_dense<LIN, LE, LOUT>(t);
  return t;
}

template <int LIN, int LE, int LOUT>
__constant__ BondDense<LIN, LE, LOUT> kBondDense = make_bond_dense<LIN, LE, LOUT>();

// Per-lane projection coefficients of the lane's bond entries (the columns of Y @ P that the
// lane owns): c[r][j] = s_p C_p[i, j - l2^2, k] for entry lane + 64 r on its l2 block, +0
// elsewhere -- the values msg_bond_kernel puts in its LDS projection table.
template <int LIN, int LE, int LOUT, bool INLINE = BondInline<LIN, LE, LOUT>::value>
struct BondCoef {
  __device__ void init(const ictc_tp_desc&, int) {}
};

template <int LIN, int LE, int LOUT>
struct BondCoef<LIN, LE, LOUT, true> {
  static constexpr int NB = Paths<LIN, LE, LOUT>::NB, NY = Paths<LIN, LE, LOUT>::NY;
  static constexpr int NV = BondStage<NB>::NV;
  float c[NV][NY];
  __device__ __forceinline__ void init(const ictc_tp_desc& d, int lane) {
    const BondDense<LIN, LE, LOUT>& t = kBondDense<LIN, LE, LOUT>;
    // unconditional loads (issued together); off-block entries are stored zeros, and the path
    // scales are positive, so they stay +0 like the bond kernel's literal zeros
#pragma unroll
    for (int r = 0; r < NV; ++r) {
      const int idx = lane + r * kWave;
      const float sc = d.scale[t.path[idx]];
#pragma unroll
      for (int j = 0; j < NY; ++j) c[r][j] = t.cg[idx][j] * sc;
    }
  }
};

// Bond row of edge e into the wave's staging registers: fetched from the bond buffer, or
// formed from the harmonics row (one load, the NY values broadcast from lanes 0..NY-1).
template <int LIN, int LE, int LOUT>
__device__ __forceinline__ void bond_row(const float* __restrict__ bonds_or_y, int64_t e, int lane,
                                         const BondCoef<LIN, LE, LOUT>& bc,
                                         BondStage<Paths<LIN, LE, LOUT>::NB>& s) {
  constexpr int NB = Paths<LIN, LE, LOUT>::NB, NY = Paths<LIN, LE, LOUT>::NY;
  if constexpr (BondInline<LIN, LE, LOUT>::value) {
    const float yl = bonds_or_y[e * NY + (lane < NY ? lane : NY - 1)];
    float yv[NY];
#pragma unroll
    for (int j = 0; j < NY; ++j)
      yv[j] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, yl), j));
#pragma unroll
    for (int r = 0; r < BondStage<NB>::NV; ++r) {
      float acc = 0.f;
#pragma unroll
      for (int j = 0; j < NY; ++j) acc = fmaf(yv[j], bc.c[r][j], acc);
      s.v[r] = acc;
    }
  } else {
    bond_fetch<NB>(bonds_or_y, e, lane, s);
  }
}

template <int NB>
__device__ __forceinline__ void bond_commit(const BondStage<NB>& s, float* __restrict__ row, int lane) {
#pragma unroll
  for (int r = 0; r < BondStage<NB>::NV; ++r) row[lane + r * kWave] = s.v[r];
  wave_lds_sync();
}

// ----------------------------------------------------------------------------- forward
// One block per (receiver node, 64-channel chunk): its waves take every kMsgWaves-th edge
// of the node and accumulate partial outputs in registers, then the partials are summed
// in a fixed order (wave 0 + 1 + 2 + 3) through LDS, kMsgReduceRows output rows at a time.
// Four waves per receiver fill the GPU even for a few thousand receivers (the per-node
// wave count is what a one-wave-per-receiver launch is limited by).
constexpr int kMsgReduceRows = 16;

// Direction of the message inputs for the tangent (JVP) kernels: x [nodes_src, NX*C], g [edges,
// NP*C] and the harmonics direction, as bond rows (the harmonics direction itself when the rows
// are built in-kernel) for the forward tangent and as harmonics rows for the VJP tangent.
struct MsgTangent {
  const float* x;
  const float* bonds;   // forward tangent: the bond rows of the harmonics direction
  const float* g;
  const float* y;       // VJP tangent: the harmonics direction [edges, (L_e+1)^2]
};

// JVP = true computes the directional derivative of the message in direction t:
//   out[n] = sum_e g (.) [TP(tx, M) + TP(x, tM)] + tg (.) TP(x, M)
// (the sum of the three one-argument substitutions of the reference's bilinear second-order
// rule, structured_product.py:146-158, in one pass over the edges).
template <int LIN, int LE, int LOUT, bool JVP = false>
__global__ void __launch_bounds__(kMsgBlock)
msg_forward_kernel(const float* __restrict__ x, const float* __restrict__ bonds, const float* __restrict__ g,
                   const MsgTangent t, const int64_t* __restrict__ src, const int64_t* __restrict__ rowptr,
                   const int64_t* __restrict__ perm, float* __restrict__ out, const ictc_tp_desc d,
                   int64_t nodes_src, int64_t nodes_dst, int nchunks) {
  using PS = Paths<LIN, LE, LOUT>;
  constexpr int NX = PS::NX, NP = PS::N, NOC = PS::NOC, NB = PS::NB;
  constexpr int NBS = BondStage<NB>::NV * kWave;
  constexpr int NT = JVP ? 2 : 1;   // input sets per edge: primal (+ direction)
  constexpr int R = kMsgReduceRows;
  __shared__ float sB[kMsgWaves][NT][NBS];
  __shared__ float sR[kMsgWaves - 1][R][kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t item = xcd_block(blockIdx.x, gridDim.x);   // receivers contiguous per XCD
  const int64_t node = static_cast<int64_t>(item) / nchunks;
  const int chunk = static_cast<int>(item - node * nchunks);
  const int C = d.channels;
  const int c = chunk * kWave + lane;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;
  const bool live = c < C;
  const uint32_t xbytes = static_cast<uint32_t>(nodes_src * NX * row);
  const rsrc_t rx[2] = {make_rsrc(x, xbytes), make_rsrc(JVP ? t.x : x, xbytes)};   // range-checked gathers
  const float* gs[2] = {g, t.g};
  const float* bs_src[2] = {bonds, t.bonds};
  float acc[NOC];
#pragma unroll
  for (int r = 0; r < NOC; ++r) acc[r] = 0.f;
  // lanes past C read channel 0 (discarded): every access stays inside its row, so the
  // uniform row offsets can ride in soffset
  const uint32_t vc = static_cast<uint32_t>(live ? c : 0) * 4u;
  BondCoef<LIN, LE, LOUT> bc;
  bc.init(d, lane);
  // bond rows first: staging them into LDS then waits for those loads only, while the x and
  // gate loads issued after them are still in flight.  Gate rows are read exactly once and use
  // the non-temporal cache policy, which leaves L2 to the x[src] gathers that other edges of
  // nearby receivers re-read (C128/lmax-3 forward over 105,634 edges: 0.62 -> 0.55 ms measured,
  // bit-identical)
  auto fetch = [&](int64_t slot, float (*xo)[NX], float (*gvo)[NP], BondStage<NB>* bo) {
    const int64_t e = perm ? perm[slot] : slot;
#pragma unroll
    for (int q = 0; q < NT; ++q) bond_row<LIN, LE, LOUT>(bs_src[q], e, lane, bc, bo[q]);
    const uint32_t xoff = static_cast<uint32_t>(src[e]) * NX * row + vc;   // range-checked gather
#pragma unroll
    for (int q = 0; q < NT; ++q)
#pragma unroll
      for (int m = 0; m < NX; ++m) xo[q][m] = buf_load_vs(rx[q], xoff, m * row);
#pragma unroll
    for (int q = 0; q < NT; ++q) {
      const rsrc_t rg = make_rsrc(gs[q] + e * NP * C, NP * row);
#pragma unroll
      for (int p = 0; p < NP; ++p) gvo[q][p] = buf_load_vs<kNonTemporal>(rg, vc, p * row);
    }
  };

  auto compute = [&](const float (*xr)[NX], const float (*gv)[NP], const float* bond0, const float* bond1) {
    static_for<0, NP>([&](auto P) {
      constexpr int p = P;
      constexpr int l1 = PS::tab.l1[p], l3 = PS::tab.l3[p];
      constexpr int ni = 2 * l1 + 1, no = 2 * l3 + 1;
      constexpr int boff = PS::tab.bond[p], oo = PS::tab.out[p];
      // an opaque base per path plus a scheduling barrier keep the path's LDS reads next to
      // their use (otherwise the reads of the whole row are merged and hoisted into registers)
      const float* bp = opaque_lds_row(bond0 + boff);
      const float* tp = JVP ? opaque_lds_row(bond1 + boff) : bp;
      __builtin_amdgcn_sched_barrier(0);
      static_for<0, no>([&](auto K) {
        float u = 0.f;
        static_for<0, ni>([&](auto I) { u = fmaf(xr[0][l1 * l1 + I], bp[K * ni + I], u); });
        if constexpr (JVP) {
          float v = 0.f;   // TP(tx, M) + TP(x, tM)
          static_for<0, ni>([&](auto I) {
            v = fmaf(xr[1][l1 * l1 + I], bp[K * ni + I], v);
            v = fmaf(xr[0][l1 * l1 + I], tp[K * ni + I], v);
          });
          acc[oo + K] = fmaf(v, gv[0][p], fmaf(u, gv[1][p], acc[oo + K]));
        } else {
          acc[oo + K] = fmaf(u, gv[0][p], acc[oo + K]);
        }
      });
    });
  };

  // Every load of an edge is issued together.  The primal pass also requests the next edge's
  // loads before computing the current one (measured 5 % faster at lmax 3, where 158 VGPRs leave
  // 3 waves per SIMD to hide latency, 2 % at lmax 2; outputs bit-identical); the tangent pass,
  // with twice the per-edge inputs, relies on the other resident waves alone.
  const int64_t s0 = rowptr[node], s1 = rowptr[node + 1];
  if constexpr (!JVP) {
    int64_t slot = s0 + wave;
    if (slot < s1) {
      float xr[1][NX], gv[1][NP];
      BondStage<NB> bs[1];
      fetch(slot, xr, gv, bs);
#pragma clang loop unroll(disable)
      for (;;) {
        const int64_t nslot = slot + kMsgWaves;
        const bool more = nslot < s1;
        float xn[1][NX], gn[1][NP];
        BondStage<NB> bn[1];
        if (more) fetch(nslot, xn, gn, bn);
        bond_commit<NB>(bs[0], &sB[wave][0][0], lane);
        compute(xr, gv, &sB[wave][0][0], &sB[wave][0][0]);
        if (!more) break;
#pragma unroll
        for (int m = 0; m < NX; ++m) xr[0][m] = xn[0][m];
#pragma unroll
        for (int p = 0; p < NP; ++p) gv[0][p] = gn[0][p];
        bs[0] = bn[0];
        slot = nslot;
      }
    }
  } else {
#pragma clang loop unroll(disable)
    for (int64_t slot = s0 + wave; slot < s1; slot += kMsgWaves) {
      float xr[NT][NX], gv[NT][NP];
      BondStage<NB> bs[NT];
      fetch(slot, xr, gv, bs);
#pragma unroll
      for (int q = 0; q < NT; ++q) bond_commit<NB>(bs[q], &sB[wave][q][0], lane);
      compute(xr, gv, &sB[wave][0][0], &sB[wave][NT - 1][0]);
    }
  }
  const rsrc_t ro = make_rsrc(out + node * NOC * C, NOC * row);
  static_for<0, (NOC + R - 1) / R>([&](auto PIECE) {
    constexpr int r0 = PIECE * R;
    constexpr int nr = NOC - r0 < R ? NOC - r0 : R;
    if (wave > 0) {
#pragma unroll
      for (int r = 0; r < nr; ++r) sR[wave - 1][r][lane] = acc[r0 + r];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int r = 0; r < nr; ++r) {
        float v = acc[r0 + r];
#pragma unroll
        for (int w = 0; w < kMsgWaves - 1; ++w) v += sR[w][r][lane];
        buf_store_lane(ro, live, c * 4u + (r0 + r) * row, v);
      }
    }
    __syncthreads();
  });
}

inline int msg_launch_status() { return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH; }

// ----------------------------------------------------------------------------- forward by degree
// Forward (and tangent forward) for degree sets with a bond buffer (lmax 3): the receiver's
// work is split by input degree l1 into LIN + 1 launches.  Group l1 owns the x rows of degree
// l1, the paths with that l1 (their gates and bond entries) and those paths' output rows, so the
// groups partition every input and output: nothing is read twice.  Each lane carries CPL
// 64-channel chunks, so one LDS read of a bond entry -- the whole wave reads the same entry, and
// that broadcast is what bounds the one-chunk kernel above at lmax 3 -- serves CPL channels.
// Measured at C=128, lmax 3, 106,414 edges over 2,048 receivers: 557 -> 420 us (l1 groups and
// two chunks per lane; l1 groups alone 530 us, l3 groups 550 us), outputs bit-identical (same
// products in the same order).
struct DegreeGroup {
  int np = 0, noc = 0, nb = 0, nx = 0;
  int path[ICTC_MAX_PATHS] = {};   // the group's paths in enumeration order
  int out[ICTC_MAX_PATHS] = {};    // local first output row of each
  int bond[ICTC_MAX_PATHS] = {};   // local first bond entry of each
  int rowmap[128] = {};            // local output row -> output row
  int bidx[512] = {};              // local bond entry -> bond entry
};

template <int LIN, int LE, int LOUT, int L1>
constexpr DegreeGroup make_degree_group() {
  DegreeGroup t{};
  constexpr PathTable pt = Paths<LIN, LE, LOUT>::tab;
  t.nx = 2 * L1 + 1;
  for (int p = 0; p < pt.n; ++p) {
    if (pt.l1[p] != L1) continue;
    const int n = (2 * pt.l1[p] + 1) * (2 * pt.l3[p] + 1);
    t.path[t.np] = p;
    t.bond[t.np] = t.nb;
    for (int q = 0; q < n; ++q) t.bidx[t.nb + q] = pt.bond[p] + q;
    t.nb += n;
    ++t.np;
  }
  // output rows in their global order (ascending l3, enumeration order within one l3)
  for (int r = 0; r < pt.noc; ++r)
    for (int q = 0; q < t.np; ++q) {
      const int p = t.path[q];
      if (r == pt.out[p]) t.out[q] = t.noc;
      if (r >= pt.out[p] && r < pt.out[p] + 2 * pt.l3[p] + 1) t.rowmap[t.noc++] = r;
    }
  return t;
}

template <int LIN, int LE, int LOUT, int L1>
struct DegreeGroupOf {
  static constexpr DegreeGroup tab = make_degree_group<LIN, LE, LOUT, L1>();
};

template <int LIN, int LE, int LOUT, int L1>
__constant__ DegreeGroup kDegreeGroup = make_degree_group<LIN, LE, LOUT, L1>();

template <int LIN, int LE, int LOUT, int L1, int CPL, bool JVP>
__global__ void __launch_bounds__(kMsgBlock)
msg_forward_degree_kernel(const float* __restrict__ x, const float* __restrict__ bonds,
                          const float* __restrict__ g, const MsgTangent t, const int64_t* __restrict__ src,
                          const int64_t* __restrict__ rowptr, const int64_t* __restrict__ perm,
                          float* __restrict__ out, const ictc_tp_desc d, int64_t nodes_src, int nblk) {
  using PS = Paths<LIN, LE, LOUT>;
  constexpr DegreeGroup GT = DegreeGroupOf<LIN, LE, LOUT, L1>::tab;
  constexpr int NX = PS::NX, NP = PS::N, NOCF = PS::NOC, NBF = PS::NB;
  constexpr int NPG = GT.np, NOC = GT.noc, NBG = GT.nb, NI = GT.nx;
  constexpr int NV = (NBG + kWave - 1) / kWave;
  constexpr int NT = JVP ? 2 : 1;   // input sets per edge: primal (+ direction)
  constexpr int R = kMsgReduceRows;
  static_assert(NPG > 0, "an input degree without paths has no launch");
  __shared__ float sB[kMsgWaves][NT][NV * kWave];
  __shared__ float sR[kMsgWaves - 1][R][CPL * kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t item = xcd_block(blockIdx.x, gridDim.x);   // receivers contiguous per XCD
  const int64_t node = static_cast<int64_t>(item) / nblk;
  const int chunk0 = static_cast<int>(item - node * nblk) * CPL;
  const int C = d.channels;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;
  bool live[CPL];
  uint32_t vc[CPL];   // lanes past C read channel 0 (discarded) and store nothing
#pragma unroll
  for (int h = 0; h < CPL; ++h) {
    const int c = (chunk0 + h) * kWave + lane;
    live[h] = c < C;
    vc[h] = static_cast<uint32_t>(live[h] ? c : 0) * 4u;
  }
  const uint32_t xbytes = static_cast<uint32_t>(nodes_src * NX * row);
  const rsrc_t rx[2] = {make_rsrc(x, xbytes), make_rsrc(JVP ? t.x : x, xbytes)};   // range-checked gathers
  const float* gs[2] = {g, t.g};
  const float* bsrc[2] = {bonds, t.bonds};
  float acc[CPL][NOC];
#pragma unroll
  for (int h = 0; h < CPL; ++h)
#pragma unroll
    for (int r = 0; r < NOC; ++r) acc[h][r] = 0.f;
  uint32_t boff[NV];   // byte offsets of the lane's bond entries in a bond row
#pragma unroll
  for (int r = 0; r < NV; ++r) {
    const int idx = lane + r * kWave;
    boff[r] = static_cast<uint32_t>(idx < NBG ? kDegreeGroup<LIN, LE, LOUT, L1>.bidx[idx] : 0) * 4u;
  }
  const int64_t s0 = rowptr[node], s1 = rowptr[node + 1];
#pragma clang loop unroll(disable)
  for (int64_t slot = s0 + wave; slot < s1; slot += kMsgWaves) {
    const int64_t e = perm ? perm[slot] : slot;
    float bv[NT][NV], xr[NT][CPL][NI], gv[NT][CPL][NPG];
#pragma unroll
    for (int q = 0; q < NT; ++q) {   // bond entries first (staged into LDS below)
      const rsrc_t rb = make_rsrc(bsrc[q] + e * NBF, NBF * 4u);
#pragma unroll
      for (int r = 0; r < NV; ++r) bv[q][r] = buf_load<1>(rb, boff[r]).v[0];
    }
    const uint32_t xoff = static_cast<uint32_t>(src[e]) * NX * row;
#pragma unroll
    for (int q = 0; q < NT; ++q)
#pragma unroll
      for (int h = 0; h < CPL; ++h)
#pragma unroll
        for (int m = 0; m < NI; ++m) xr[q][h][m] = buf_load_vs(rx[q], xoff + vc[h], (L1 * L1 + m) * row);
#pragma unroll
    for (int q = 0; q < NT; ++q) {
      const rsrc_t rg = make_rsrc(gs[q] + e * NP * C, NP * row);
#pragma unroll
      for (int h = 0; h < CPL; ++h)
#pragma unroll
        for (int k = 0; k < NPG; ++k) gv[q][h][k] = buf_load_vs<kNonTemporal>(rg, vc[h], GT.path[k] * row);
    }
#pragma unroll
    for (int q = 0; q < NT; ++q)
#pragma unroll
      for (int r = 0; r < NV; ++r) sB[wave][q][lane + r * kWave] = bv[q][r];
    wave_lds_sync();
    static_for<0, NPG>([&](auto Q) {
      constexpr int k = Q;
      constexpr int p = GT.path[k];
      constexpr int no = 2 * PS::tab.l3[p] + 1;
      constexpr int ni = NI, bo = GT.bond[k], oo = GT.out[k];
      const float* bp = opaque_lds_row(&sB[wave][0][bo]);
      const float* tp = JVP ? opaque_lds_row(&sB[wave][NT - 1][bo]) : bp;
      __builtin_amdgcn_sched_barrier(0);
      static_for<0, no>([&](auto K) {
        float u[CPL], v[CPL];
#pragma unroll
        for (int h = 0; h < CPL; ++h) u[h] = v[h] = 0.f;
        static_for<0, ni>([&](auto I) {
          const float b = bp[K * ni + I];
          const float tb = JVP ? tp[K * ni + I] : 0.f;
#pragma unroll
          for (int h = 0; h < CPL; ++h) {
            u[h] = fmaf(xr[0][h][I], b, u[h]);
            if constexpr (JVP) {   // TP(tx, M) + TP(x, tM)
              v[h] = fmaf(xr[1][h][I], b, v[h]);
              v[h] = fmaf(xr[0][h][I], tb, v[h]);
            }
          }
        });
#pragma unroll
        for (int h = 0; h < CPL; ++h) {
          if constexpr (JVP)
            acc[h][oo + K] = fmaf(v[h], gv[0][h][k], fmaf(u[h], gv[1][h][k], acc[h][oo + K]));
          else
            acc[h][oo + K] = fmaf(u[h], gv[0][h][k], acc[h][oo + K]);
        }
      });
    });
  }
  const rsrc_t ro = make_rsrc(out + node * NOCF * C, NOCF * row);
  static_for<0, (NOC + R - 1) / R>([&](auto PIECE) {
    constexpr int r0 = PIECE * R;
    constexpr int nr = NOC - r0 < R ? NOC - r0 : R;
    if (wave > 0) {
#pragma unroll
      for (int r = 0; r < nr; ++r)
#pragma unroll
        for (int h = 0; h < CPL; ++h) sR[wave - 1][r][h * kWave + lane] = acc[h][r0 + r];
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int r = 0; r < nr; ++r)
#pragma unroll
        for (int h = 0; h < CPL; ++h) {
          float v = acc[h][r0 + r];
#pragma unroll
          for (int w = 0; w < kMsgWaves - 1; ++w) v += sR[w][r][h * kWave + lane];
          buf_store_lane(ro, live[h], vc[h] + GT.rowmap[r0 + r] * row, v);
        }
    }
    __syncthreads();
  });
}

// One launch per input degree that has paths; two chunks per lane when the channels span two.
template <int LIN, int LE, int LOUT, bool JVP>
int launch_msg_forward_degrees(const ictc_tp_desc& d, const float* x, const float* bonds, const float* g,
                               const MsgTangent& t, const int64_t* src, const int64_t* rowptr,
                               const int64_t* perm, float* out, int64_t nodes_src, int64_t nodes_dst,
                               hipStream_t stream) {
  const int nchunks = (d.channels + kWave - 1) / kWave;
  const bool two = nchunks >= 2;
  const int nblk = two ? (nchunks + 1) / 2 : nchunks;
  const dim3 grid(static_cast<unsigned>(nodes_dst * nblk));
  auto one = [&](auto deg) {
    constexpr int L1 = decltype(deg)::value;
    if constexpr (DegreeGroupOf<LIN, LE, LOUT, L1>::tab.np > 0) {
      if (two)
        hipLaunchKernelGGL((msg_forward_degree_kernel<LIN, LE, LOUT, L1, 2, JVP>), grid, dim3(kMsgBlock), 0, stream,
                           x, bonds, g, t, src, rowptr, perm, out, d, nodes_src, nblk);
      else
        hipLaunchKernelGGL((msg_forward_degree_kernel<LIN, LE, LOUT, L1, 1, JVP>), grid, dim3(kMsgBlock), 0, stream,
                           x, bonds, g, t, src, rowptr, perm, out, d, nodes_src, nblk);
    }
  };
  one(Int<0>{});
  if constexpr (LIN >= 1) one(Int<1>{});
  if constexpr (LIN >= 2) one(Int<2>{});
  if constexpr (LIN >= 3) one(Int<3>{});
  return msg_launch_status();
}

// ----------------------------------------------------------------------------- VJP: per source node
// dx[s] = sum over edges with src(e) = s of dxe[e]  ([NX][C] rows, streamed four edges at a time;
// each row is read once, with the non-temporal cache policy: 7-11 % faster measured).
template <int NX>
__global__ void __launch_bounds__(kMsgBlock)
msg_node_grad_kernel(const float* __restrict__ dxe, const int64_t* __restrict__ rowptr_src,
                     const int64_t* __restrict__ perm_src, float* __restrict__ dx, int C, int64_t nodes_src,
                     int nchunks) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  // source nodes contiguous per XCD
  const int64_t item = static_cast<int64_t>(xcd_block(blockIdx.x, gridDim.x)) * kMsgWaves + wave;
  const int64_t node = item / nchunks;
  if (node >= nodes_src) return;
  const int chunk = static_cast<int>(item - node * nchunks);
  const int c = chunk * kWave + lane;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;
  const bool live = c < C;
  const uint32_t vc = static_cast<uint32_t>(live ? c : 0) * 4u;   // lanes past C re-read channel 0
  float acc[NX];
#pragma unroll
  for (int m = 0; m < NX; ++m) acc[m] = 0.f;
  const int64_t s0 = rowptr_src[node], s1 = rowptr_src[node + 1];
  constexpr int U = 4;
  int64_t slot = s0;
  for (; slot + U <= s1; slot += U) {
    float v[U][NX];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t e = perm_src ? perm_src[slot + u] : slot + u;
      const rsrc_t r = make_rsrc(dxe + e * NX * C, NX * row);
#pragma unroll
      for (int m = 0; m < NX; ++m) v[u][m] = buf_load_vs<kNonTemporal>(r, vc, m * row);
    }
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int m = 0; m < NX; ++m) acc[m] += v[u][m];
  }
  for (; slot < s1; ++slot) {
    const int64_t e = perm_src ? perm_src[slot] : slot;
    const rsrc_t r = make_rsrc(dxe + e * NX * C, NX * row);
#pragma unroll
    for (int m = 0; m < NX; ++m) acc[m] += buf_load_vs<kNonTemporal>(r, vc, m * row);
  }
  const rsrc_t rdx = make_rsrc(dx + node * NX * C, NX * row);
#pragma unroll
  for (int m = 0; m < NX; ++m) buf_store_lane(rdx, live, c * 4u + m * row, acc[m]);
}

// ----------------------------------------------------------------------------- launchers

inline dim3 msg_grid(int64_t nodes, int nchunks) {
  return dim3(static_cast<unsigned>((nodes * nchunks + kMsgWaves - 1) / kMsgWaves));
}

template <int LIN, int LE, int LOUT>
int launch_msg_bonds(const ictc_tp_desc& d, const float* y, float* bonds, int64_t edges, hipStream_t stream) {
  constexpr int NB = Paths<LIN, LE, LOUT>::NB;
  if (NB == 0 || edges == 0 || BondInline<LIN, LE, LOUT>::value) return ICTC_OK;   // rows built in-kernel
  hipLaunchKernelGGL((msg_bond_kernel<LIN, LE, LOUT>),
                     dim3(static_cast<unsigned>((edges + kBondEdges - 1) / kBondEdges)), dim3(256), 0, stream, y,
                     bonds, d, edges);
  return msg_launch_status();
}

template <int LIN, int LE, int LOUT>
int launch_msg_forward(const ictc_tp_desc& d, const float* x, const float* bonds, const float* g,
                       const int64_t* src, const int64_t* rowptr, const int64_t* perm, float* out,
                       int64_t nodes_src, int64_t nodes_dst, hipStream_t stream) {
  if constexpr (!BondInline<LIN, LE, LOUT>::value && Paths<LIN, LE, LOUT>::NB > 0) {
    return launch_msg_forward_degrees<LIN, LE, LOUT, false>(d, x, bonds, g, MsgTangent{}, src, rowptr, perm, out,
                                                           nodes_src, nodes_dst, stream);
  } else {
    const int nchunks = (d.channels + kWave - 1) / kWave;
    const dim3 grid(static_cast<unsigned>(nodes_dst * nchunks));   // one block per (node, chunk)
    hipLaunchKernelGGL((msg_forward_kernel<LIN, LE, LOUT>), grid, dim3(kMsgBlock), 0,
                       stream, x, bonds, g, MsgTangent{}, src, rowptr, perm, out, d, nodes_src, nodes_dst, nchunks);
    return msg_launch_status();
  }
}

template <int LIN, int LE, int LOUT>
int launch_msg_forward_tangent(const ictc_tp_desc& d, const float* x, const float* bonds, const float* g,
                               const MsgTangent& t, const int64_t* src, const int64_t* rowptr,
                               const int64_t* perm, float* out, int64_t nodes_src, int64_t nodes_dst,
                               hipStream_t stream) {
  if constexpr (!BondInline<LIN, LE, LOUT>::value && Paths<LIN, LE, LOUT>::NB > 0) {
    return launch_msg_forward_degrees<LIN, LE, LOUT, true>(d, x, bonds, g, t, src, rowptr, perm, out, nodes_src,
                                                          nodes_dst, stream);
  } else {
    const int nchunks = (d.channels + kWave - 1) / kWave;
    const dim3 grid(static_cast<unsigned>(nodes_dst * nchunks));
    hipLaunchKernelGGL((msg_forward_kernel<LIN, LE, LOUT, true>), grid, dim3(kMsgBlock), 0,
                       stream, x, bonds, g, t, src, rowptr, perm, out, d, nodes_src, nodes_dst, nchunks);
    return msg_launch_status();
  }
}

// ----------------------------------------------------------------------------- VJP by degree
// VJP in one pass per input degree l1 (the groups of msg_forward_degree_kernel: each owns the x rows
// of degree l1, its paths' gates and dout rows, and so its dg columns and dxe rows).  With the bond
// matrices M_p[K][I] = s_p sum_J Y_{l2^2 + J} C_p[I, J, K] the per-edge, per-path adjoints are
//   w_I = sum_K M[K][I] dout_K,  dg_p = sum_I x_I w_I,  dxe_I += g_p w_I,
//   dY_{l2^2 + J} += s_p sum_{I,K} C_p[I, J, K] x_I g_p dout_K   (summed over the channels).
// For receiver n the factor U_p[I][J] = s_p sum_K C_p[I, J, K] dout_n[K] is the same for every edge
// into n: built once per block in LDS, it turns both contractions into ni * nj products per channel,
//   w_I = sum_J Y_{l2^2 + J} U_p[I][J],  v_J = sum_I x_I U_p[I][J],
//   dg_p = sum_J Y_{l2^2 + J} v_J,  dY_{l2^2 + J} += g_p v_J,
// where the bond form costs ni * no for w and ni * no * nj (shared by the lane's channels) for the
// harmonics partials, and each edge needs its harmonics row instead of its bond row (measured at
// C = 128, lmax 3, 105,634 edges: 1.07 -> 1.01 ms for the four launches, the tangent 1.57 -> 1.33 ms;
// C = 64, lmax 2, 855,792 edges: 1.82 -> 1.66 and 2.32 -> 2.11 ms; outputs within 2.5e-7
// relative).  JVP = true gives the directional derivative of all three in direction
// t = (tx, tY, tg) with dout fixed (the mixed second derivatives): tw_I = sum_J tY_{l2^2 + J} U_p[I][J],
//   dg_p = sum_I (tx_I w_I + x_I tw_I),  dxe_I += g_p tw_I + tg_p w_I,
//   dY_{l2^2 + J} += sum_I (tx_I g_p + x_I tg_p) U_p[I][J].
// One block per (receiver, 64-channel chunk); path k's U block is built by wave k mod 4, then every
// wave walks every fourth edge of the receiver.  dY partials [edges, chunks, NY]: group launches run
// in order on one stream; the first writes each (edge, chunk) slot, later groups add to it (a fixed
// order; the caller sums the chunk axis).
struct NodeU {
  int nu = 0;
  int off[ICTC_MAX_PATHS] = {};   // first U entry of each path of the group
};

template <int LIN, int LE, int LOUT, int L1>
constexpr NodeU make_node_u() {
  NodeU u{};
  constexpr DegreeGroup GT = DegreeGroupOf<LIN, LE, LOUT, L1>::tab;
  constexpr PathTable pt = Paths<LIN, LE, LOUT>::tab;
  for (int k = 0; k < GT.np; ++k) {
    u.off[k] = u.nu;
    u.nu += GT.nx * (2 * pt.l2[GT.path[k]] + 1);
  }
  return u;
}

template <int LIN, int LE, int LOUT, int L1>
struct NodeUOf {
  static constexpr NodeU tab = make_node_u<LIN, LE, LOUT, L1>();
};

// Resident waves per SIMD the compiler is held to for an edge-gradient launch of an lmax-3 set
// (register budget 512 / waves), where its LDS allows more waves than its unconstrained register
// allocation: input degree 2 first order at 4 (128 VGPRs; its 39.7 KB table allows 4 blocks per
// CU, 130 VGPRs would allow 3), input degree 3 tangent at 3 (168 VGPRs; 173 allowed 2, its 50 KB
// table 3).
constexpr int msg_edge_grad_waves(int lin, int l1, bool jvp) {
  return lin < 3 ? 1 : l1 == 2 && !jvp ? 4 : l1 == 3 && jvp ? 3 : 1;
}

template <int LIN, int LE, int LOUT, int L1, bool JVP, bool ACC = false>
__global__ void __launch_bounds__(kMsgBlock) __attribute__((amdgpu_waves_per_eu(msg_edge_grad_waves(LIN, L1, JVP))))
msg_edge_grad_degree_kernel(const float* __restrict__ x, const float* __restrict__ y, const float* __restrict__ g,
                          const MsgTangent t, const float* __restrict__ go, const int64_t* __restrict__ src,
                          const int64_t* __restrict__ rowptr, const int64_t* __restrict__ perm,
                          float* __restrict__ dyp, float* __restrict__ dg, float* __restrict__ dxe,
                          const ictc_tp_desc d, int64_t nodes_src, int nchunks, int first) {
  using PS = Paths<LIN, LE, LOUT>;
  constexpr DegreeGroup GT = DegreeGroupOf<LIN, LE, LOUT, L1>::tab;
  constexpr NodeU UT = NodeUOf<LIN, LE, LOUT, L1>::tab;
  constexpr int NX = PS::NX, NY = PS::NY, NP = PS::N, NOCF = PS::NOC;
  constexpr int NPG = GT.np, NI = GT.nx, NU = UT.nu;
  constexpr int NT = JVP ? 2 : 1;   // input sets per edge: primal (+ direction)
  static_assert(NPG > 0, "an input degree without paths has no launch");
  static_assert(NU * kWave * 4 <= 65536, "the node contraction table exceeds 64 KiB of LDS");
  __shared__ float sU[NU * kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t item = xcd_block(blockIdx.x, gridDim.x);   // receivers contiguous per XCD
  const int64_t node = static_cast<int64_t>(item) / nchunks;
  const int chunk = static_cast<int>(item - node * nchunks);
  const int C = d.channels;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;
  const int c = chunk * kWave + lane;
  const bool live = c < C;
  const uint32_t vc = static_cast<uint32_t>(live ? c : 0) * 4u;   // lanes past C read channel 0, zero it
  const uint32_t xdead = live ? 0u : 0xFFFFFFF0u;   // OR-ed into x gather offsets: out of range
  {
    const rsrc_t ron = make_rsrc(go + node * NOCF * C, NOCF * row);
    static_for<0, NPG>([&](auto Q) {
      constexpr int k = Q;
      if (wave == k % kMsgWaves) {   // wave-uniform
        constexpr int p = GT.path[k];
        constexpr int l2 = PS::tab.l2[p], l3 = PS::tab.l3[p];
        constexpr int nj = 2 * l2 + 1, no = 2 * l3 + 1, oo = GT.out[k], uo = UT.off[k];
        using CG = CGTab<L1, l2, l3>;
        float ov[no];
        static_for<0, no>([&](auto K) {
          constexpr uint32_t r = static_cast<uint32_t>(GT.rowmap[oo + K]);
          const float v = buf_load_vs<kNonTemporal>(ron, vc, r * row);
          ov[K] = live ? v : 0.f;
        });
        const float sc = d.scale[p];
        static_for<0, NI>([&](auto I) {
          static_for<0, nj>([&](auto J) {
            float u = 0.f;
            static_for<0, no>([&](auto K) {
              constexpr float cg = CG::v[(I * nj + J) * no + K];
              if constexpr (cg != 0.0f) u = fmaf(cg, ov[K], u);
            });
            sU[(uo + I * nj + J) * kWave + lane] = sc * u;
          });
        });
      }
    });
  }
  __syncthreads();
  const uint32_t xbytes = static_cast<uint32_t>(nodes_src * NX * row);
  const bool xdep = JVP || dg != nullptr || dyp != nullptr;   // the plain dxe needs no x
  const rsrc_t rx[2] = {make_rsrc(xdep ? x : nullptr, xbytes), make_rsrc(JVP ? t.x : nullptr, xbytes)};
  const float* gs[2] = {g, t.g};
  const float* ys[2] = {y, t.y};
  const bool wy = dyp != nullptr;
  using WS = WaveSums<NY>;
  const int wj = WS::index(lane);   // the harmonic whose channel sum this lane ends up holding
  const bool wown = wy && WS::owner(lane) && wj < NY;
  const int wjc = wj < NY ? wj : NY - 1;
  // One edge's inputs: its harmonics rows (wave-uniform loads), the source features of degree l1,
  // the group's gates and the harmonics partial that earlier degree launches left in the slot.
  struct EdgeIn {
    float yv[NT][NY];
    float xr[NT][NI];
    float gv[NT][NPG];
    float dgp[ACC ? NPG : 1];   // ACC: the gate gradients already in dg (this pass adds to them)
    float prev;
  };
  auto fetch = [&](int64_t e, int64_t s, EdgeIn& in) {
#pragma unroll
    for (int q = 0; q < NT; ++q)
#pragma unroll
      for (int j = 0; j < NY; ++j) in.yv[q][j] = ys[q][e * NY + j];
    // Lanes past C get a voffset beyond the descriptor's range (xdead), so the hardware returns
    // 0: a select on the loaded value instead would make the wave wait for this (prefetched)
    // gather before computing the current edge.
    const uint32_t xoff = (static_cast<uint32_t>(s) * NX * row + vc) | xdead;
#pragma unroll
    for (int q = 0; q < NT; ++q)
#pragma unroll
      for (int m = 0; m < NI; ++m) in.xr[q][m] = buf_load_vs(rx[q], xoff, (L1 * L1 + m) * row);
#pragma unroll
    for (int q = 0; q < NT; ++q) {
      const rsrc_t rg = make_rsrc(gs[q] + e * NP * C, NP * row);
#pragma unroll
      for (int k = 0; k < NPG; ++k) in.gv[q][k] = buf_load_vs<kNonTemporal>(rg, vc, GT.path[k] * row);
    }
    if constexpr (ACC) {
      const rsrc_t rdg = make_rsrc(dg + e * NP * C, NP * row);
#pragma unroll
      for (int k = 0; k < NPG; ++k) in.dgp[k] = buf_load_vs(rdg, vc, GT.path[k] * row);
    }
    in.prev = (wy && !first) ? dyp[(e * nchunks + chunk) * NY + wjc] : 0.f;
  };
  auto compute = [&](int64_t e, const EdgeIn& in) {
    const rsrc_t rdg = make_rsrc(dg ? dg + e * NP * C : nullptr, NP * row);
    float dyl[NY], dxl[NI];
#pragma unroll
    for (int j = 0; j < NY; ++j) dyl[j] = 0.f;
#pragma unroll
    for (int m = 0; m < NI; ++m) dxl[m] = 0.f;
    static_for<0, NPG>([&](auto Q) {
      constexpr int k = Q;
      constexpr int p = GT.path[k];
      constexpr int l2 = PS::tab.l2[p];
      constexpr int nj = 2 * l2 + 1, uo = UT.off[k];
      const float* up = opaque_lds_row(sU + uo * kWave);
      __builtin_amdgcn_sched_barrier(0);
      float w[NI], tw[NI];
#pragma unroll
      for (int i = 0; i < NI; ++i) w[i] = tw[i] = 0.f;
      float dgv = 0.f;
      if constexpr (JVP) {
        // harmonics partials from xg_I = tx_I g_p + x_I tg_p
        auto contract = [&](auto WY) {
          float xg[NI], part[nj];
          if constexpr (WY) {
#pragma unroll
            for (int i = 0; i < NI; ++i) xg[i] = fmaf(in.xr[1][i], in.gv[0][k], in.xr[0][i] * in.gv[1][k]);
#pragma unroll
            for (int j = 0; j < nj; ++j) part[j] = 0.f;
          }
          static_for<0, NI>([&](auto I) {
            __builtin_amdgcn_sched_barrier(0);   // one row of U in registers at a time
            static_for<0, nj>([&](auto J) {
              const float u = up[(I * nj + J) * kWave + lane];
              w[I] = fmaf(in.yv[0][l2 * l2 + J], u, w[I]);
              tw[I] = fmaf(in.yv[1][l2 * l2 + J], u, tw[I]);
              if constexpr (WY) part[J] = fmaf(xg[I], u, part[J]);
            });
          });
          if constexpr (WY) {
#pragma unroll
            for (int j = 0; j < nj; ++j) dyl[l2 * l2 + j] += part[j];
          }
        };
        if (wy)
          contract(Int<1>{});
        else
          contract(Int<0>{});
#pragma unroll
        for (int i = 0; i < NI; ++i) {
          dgv = fmaf(in.xr[1][i], w[i], dgv);
          dgv = fmaf(in.xr[0][i], tw[i], dgv);
          dxl[i] = fmaf(in.gv[0][k], tw[i], dxl[i]);
          dxl[i] = fmaf(in.gv[1][k], w[i], dxl[i]);
        }
      } else {
        // with v_J = sum_I x_I U[I][J]: dg_p = sum_J Y_J v_J and the partials are g_p v_J
        auto contract = [&](auto WY) {
          float v[nj];
          if constexpr (WY) {
#pragma unroll
            for (int j = 0; j < nj; ++j) v[j] = 0.f;
          }
          static_for<0, NI>([&](auto I) {
            __builtin_amdgcn_sched_barrier(0);   // one row of U in registers at a time
            static_for<0, nj>([&](auto J) {
              const float u = up[(I * nj + J) * kWave + lane];
              w[I] = fmaf(in.yv[0][l2 * l2 + J], u, w[I]);
              if constexpr (WY) v[J] = fmaf(in.xr[0][I], u, v[J]);
            });
          });
          if constexpr (WY) {
#pragma unroll
            for (int j = 0; j < nj; ++j) {
              dgv = fmaf(in.yv[0][l2 * l2 + j], v[j], dgv);
              dyl[l2 * l2 + j] = fmaf(in.gv[0][k], v[j], dyl[l2 * l2 + j]);
            }
          } else {
#pragma unroll
            for (int i = 0; i < NI; ++i) dgv = fmaf(in.xr[0][i], w[i], dgv);
          }
        };
        if (wy)
          contract(Int<1>{});
        else
          contract(Int<0>{});
#pragma unroll
        for (int i = 0; i < NI; ++i) dxl[i] = fmaf(in.gv[0][k], w[i], dxl[i]);
      }
      if constexpr (ACC) dgv += in.dgp[k];
      buf_store_lane(rdg, live, vc + p * row, dgv);   // null dg: empty descriptor
    });
    if (dxe != nullptr) {
      const rsrc_t rde = make_rsrc(dxe + e * NX * C, NX * row);
#pragma unroll
      for (int m = 0; m < NI; ++m) buf_store_lane(rde, live, vc + (L1 * L1 + m) * row, dxl[m]);
    }
    if (wy) {   // channel sums of the NY partials, one transposing butterfly
      const float tot = WS::reduce(dyl, lane);
      if (wown) dyp[(e * nchunks + chunk) * NY + wj] = in.prev + tot;
    }
  };
  // Software pipeline over the receiver's edges: the next edge's index and source (and, where the
  // registers allow, its loads) are requested before the current edge is computed and stored.
  constexpr bool kPrefetch = !JVP || L1 == 0;
  const int64_t s0 = rowptr[node], s1 = rowptr[node + 1];
  int64_t slot = s0 + wave;
  if (slot < s1) {
    int64_t e = perm ? perm[slot] : slot;
    EdgeIn cur;
    fetch(e, src[e], cur);
#pragma clang loop unroll(disable)
    for (;;) {
      const int64_t nslot = slot + kMsgWaves;
      const bool more = nslot < s1;
      int64_t ne = e, ns = 0;
      EdgeIn nxt;
      if (more) {
        ne = perm ? perm[nslot] : nslot;
        ns = src[ne];
        if constexpr (kPrefetch) fetch(ne, ns, nxt);
      }
      compute(e, cur);
      if (!more) break;
      slot = nslot;
      e = ne;
      if constexpr (kPrefetch)
        cur = nxt;
      else
        fetch(e, ns, cur);
    }
  }
}

// dxe[e, r0 .. r0 + nr) = 0 for every edge e (rows of an input degree without paths); the edge
// count is read from the receiver CSR's last entry.
template <int NX>
__global__ void __launch_bounds__(256)
msg_zero_rows_kernel(const int64_t* __restrict__ rowptr, int64_t nodes_dst, float* __restrict__ dxe, int r0, int nr,
                     int channels) {
  const int64_t edges = rowptr[nodes_dst];
  const int64_t per = static_cast<int64_t>(nr) * channels;
  const int64_t total = edges * per;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t e = i / per, q = i - e * per;
    dxe[e * NX * channels + static_cast<int64_t>(r0) * channels + q] = 0.f;
  }
}

// One launch per input degree that has paths (dY partials accumulated across them in launch order).
// accumulate (first order only, dg non-null): add the gate gradients into dg instead of overwriting
// it (each edge's prior dg values are requested with its other loads).
template <int LIN, int LE, int LOUT, bool JVP>
int launch_msg_edge_grad_degrees(const ictc_tp_desc& d, const float* x, const float* y, const float* g,
                                 const MsgTangent& t, const float* go, const int64_t* src, const int64_t* rowptr,
                                 const int64_t* perm, float* dyp, float* dg, float* dxe, int64_t nodes_src,
                                 int64_t nodes_dst, hipStream_t stream, bool accumulate = false) {
  const int nchunks = (d.channels + kWave - 1) / kWave;
  const dim3 grid(static_cast<unsigned>(nodes_dst * nchunks));   // one block per (receiver, chunk)
  int first = 1;
  auto one = [&](auto deg) {
    constexpr int L1 = decltype(deg)::value;
    if constexpr (DegreeGroupOf<LIN, LE, LOUT, L1>::tab.np > 0) {
      if constexpr (!JVP) {
        if (accumulate) {
          hipLaunchKernelGGL((msg_edge_grad_degree_kernel<LIN, LE, LOUT, L1, false, true>), grid, dim3(kMsgBlock), 0,
                             stream, x, y, g, t, go, src, rowptr, perm, dyp, dg, dxe, d, nodes_src, nchunks, first);
          first = 0;
          return;
        }
      }
      hipLaunchKernelGGL((msg_edge_grad_degree_kernel<LIN, LE, LOUT, L1, JVP>), grid, dim3(kMsgBlock), 0, stream, x,
                         y, g, t, go, src, rowptr, perm, dyp, dg, dxe, d, nodes_src, nchunks, first);
      first = 0;
    }
  };
  one(Int<0>{});
  if constexpr (LIN >= 1) one(Int<1>{});
  if constexpr (LIN >= 2) one(Int<2>{});
  if constexpr (LIN >= 3) one(Int<3>{});
  // input degrees without paths (e.g. l1 > LE + LOUT) own dxe rows no group writes: zero them
  if (dxe != nullptr) {
    auto zero = [&](auto deg) {
      constexpr int L1 = decltype(deg)::value;
      if constexpr (DegreeGroupOf<LIN, LE, LOUT, L1>::tab.np == 0) {
        hipLaunchKernelGGL((msg_zero_rows_kernel<Paths<LIN, LE, LOUT>::NX>), dim3(1024), dim3(256), 0, stream,
                           rowptr, nodes_dst, dxe, L1 * L1, 2 * L1 + 1, d.channels);
      }
    };
    zero(Int<0>{});
    if constexpr (LIN >= 1) zero(Int<1>{});
    if constexpr (LIN >= 2) zero(Int<2>{});
    if constexpr (LIN >= 3) zero(Int<3>{});
  }
  return msg_launch_status();
}

// y: the harmonics [edges, (L_e+1)^2]; t.y the harmonics direction of the tangent pass
template <int LIN, int LE, int LOUT>
int launch_msg_edge_grad(const ictc_tp_desc& d, const float* x, const float* y, const float* g,
                         const float* go, const int64_t* src, const int64_t* rowptr, const int64_t* perm,
                         float* dyp, float* dg, float* dxe, int64_t nodes_src, int64_t nodes_dst,
                         hipStream_t stream, int accumulate_gates) {
  return launch_msg_edge_grad_degrees<LIN, LE, LOUT, false>(d, x, y, g, MsgTangent{}, go, src, rowptr, perm, dyp, dg,
                                                           dxe, nodes_src, nodes_dst, stream,
                                                           accumulate_gates != 0 && dg != nullptr);
}

template <int LIN, int LE, int LOUT>
int launch_msg_edge_grad_tangent(const ictc_tp_desc& d, const float* x, const float* y, const float* g,
                                 const MsgTangent& t, const float* go, const int64_t* src, const int64_t* rowptr,
                                 const int64_t* perm, float* dyp, float* dg, float* dxe, int64_t nodes_src,
                                 int64_t nodes_dst, hipStream_t stream) {
  return launch_msg_edge_grad_degrees<LIN, LE, LOUT, true>(d, x, y, g, t, go, src, rowptr, perm, dyp, dg, dxe,
                                                          nodes_src, nodes_dst, stream);
}

template <int LIN>
int launch_msg_node_grad(int channels, const float* dxe, const int64_t* rowptr_src, const int64_t* perm_src,
                         float* dx, int64_t nodes_src, hipStream_t stream) {
  const int nchunks = (channels + kWave - 1) / kWave;
  hipLaunchKernelGGL((msg_node_grad_kernel<(LIN + 1) * (LIN + 1)>), msg_grid(nodes_src, nchunks),
                     dim3(kMsgBlock), 0, stream, dxe, rowptr_src, perm_src, dx, channels, nodes_src, nchunks);
  return msg_launch_status();
}

}  // namespace ictc
