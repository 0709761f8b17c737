// Degree-generic tensor-product and graph-message kernels (every degree <= 6).
//
// The mathematics of tp_kernels.hpp and message_kernels.hpp (reference ictd_irreps.py:2669-2748,
// backends/ascend/tensor_product.py:30-55 and 159-218, structured_product.py:7-87):
//   M_p[k][i] = s_p * sum_j Y[l2^2 + j] * Chat_p[i][j][k]                 (bond, stored [k][i])
//   out[o_p + k, c] = g[p, c] * sum_i x[l1^2 + i, c] * M_p[k][i]
// with the path set, the output and bond offsets and the CG tensors read at run time instead of
// compiled per degree set, so one kernel serves every (input_lmax, edge_lmax, output_lmax).
//
// Launch shape: one wave per workgroup and one instance (TP row, or receiver-CSR edge of the
// message kernels) at a time, grid-stride over instances.  Per instance the wave builds M_p of
// every path into LDS (lanes over bond entries), then walks the channels in chunks of 64 with
// lane = channel.  Paths are enumerated in ascending l1, so the x rows of one input degree are
// loaded into registers once per chunk and serve every path of that degree; the loops over the
// components of one degree are unrolled to the largest degree (13 components) with the rows past
// a degree's width zeroed or clamped, so their loads issue together.
//
// VJP per path p, with go_k = g_p * dout_k:
//   dg[p]      = sum_k dout_k * sum_i M_p[k][i] x_i
//   dx[l1, i] += sum_k M_p[k][i] go_k                  (registers, one input degree at a time)
//   dY[l2, j] += s_p * sum_{i,k} Chat_p[i][j][k] x_i go_k   (per lane, then summed over lanes)
// For every degree <= 4 the dY term first reduces the products x_i go_k over the chunk's 64
// channels on the matrix cores (T = X^T G, one 16 x 16 tile of v_mfma_f32_16x16x4_f32 per path),
// then each lane contracts its (up to) four T entries with their CG rows Chat_p[i][k][0..n2)
// (stored [i][k][j]) and the path's n2 lane partials are summed over the wave by one transposing
// butterfly (a fixed order).  Above degree 4 (tiles past 16 x 16) it contracts per lane against
// the CG rows read with wave-uniform scalar loads: sum_p n1 n2 n3 FMAs per channel, the ICTC
// coupling tensors being dense (49,684 of the 52,570 entries up to degree 6 are nonzero).
#include "generic.hpp"

#include "ictc_common.hpp"
#include "generated/ictc_cg_generic.hpp"

namespace ictc {
namespace {

constexpr int kLanes = 64;
constexpr int64_t kGridCap = 16384;
constexpr int kMaxN = 2 * kGenericMaxL + 1;   // components of the largest degree
constexpr int kHead = 2 * kLanes;              // LDS head: sY [64] | sDY [64]

static_assert(kGenericMaxL == kCGGenericMaxL, "generic CG table degree");
static_assert(ICTC_MAX_PATHS >= 106, "the (6,6,6) path set has 106 paths");

// Run-time path table of one descriptor (kernel argument, read with scalar loads).
struct GenTable {
  int np, nb, noc, nx, ny, channels, lin, lout;
  int meta[ICTC_MAX_PATHS];    // l1 | l2 << 4 | l3 << 8 | first output row << 12
  int bond[ICTC_MAX_PATHS];    // first bond entry of M_p
  int cg[ICTC_MAX_PATHS];      // first kCGGeneric index of Chat_p ([i][k][j])
  float scale[ICTC_MAX_PATHS];
};

struct PathInfo {
  int l1, l2, l3, n1, n2, n3, out;
};

__device__ __forceinline__ PathInfo path_info(const GenTable& t, int p) {
  const int m = t.meta[p];
  PathInfo r;
  r.l1 = m & 15;
  r.l2 = (m >> 4) & 15;
  r.l3 = (m >> 8) & 15;
  r.n1 = 2 * r.l1 + 1;
  r.n2 = 2 * r.l2 + 1;
  r.n3 = 2 * r.l3 + 1;
  r.out = m >> 12;
  return r;
}

// Calls f(Int<n>{}) for the odd width n = 2 l + 1 <= NM of a degree (a wave-uniform switch), so
// loops over one degree's components run exactly n times.
template <int NM = kMaxN, typename F>
__device__ __forceinline__ void with_width(int n1, F&& f) {
  static_assert(kMaxN == 13 && (NM == 9 || NM == 13), "widths 1..13");
  switch (n1) {
    case 1: f(Int<1>{}); break;
    case 3: f(Int<3>{}); break;
    case 5: f(Int<5>{}); break;
    case 7: f(Int<7>{}); break;
    case 9: f(Int<9>{}); break;
    default:
      if constexpr (NM == 13) {
        if (n1 == 11)
          f(Int<11>{});
        else
          f(Int<13>{});
      }
      break;
  }
}

// M_p of every path into sM from the harmonics in sY (lanes over the bond entries of a path);
// an entry's coefficients Chat_p[i][k][0..n2) are contiguous.
__device__ void build_bonds(const GenTable& t, const float* sY, float* sM, int lane) {
  for (int p = 0; p < t.np; ++p) {
    const PathInfo q = path_info(t, p);
    const float* cg = kCGGeneric + t.cg[p];
    const float s = t.scale[p];
    float* bond = sM + t.bond[p];
    const float* y = sY + q.l2 * q.l2;
    with_width(q.n2, [&](auto N2) {
      for (int e = lane; e < q.n1 * q.n3; e += kLanes) {
        const int k = e / q.n1, i = e - k * q.n1;
        const float* row = cg + (i * q.n3 + k) * N2;
        float c[N2];
#pragma unroll
        for (int j = 0; j < N2; ++j) c[j] = row[j];
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < N2; ++j) acc = fmaf(y[j], c[j], acc);
        bond[e] = acc * s;
      }
    });
  }
}

// LDS -> LDS visibility inside the wave (lanes reading what other lanes wrote).
__device__ __forceinline__ void wave_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// Per-lane byte offset of channel c in a row, or for lanes past C an offset beyond every
// descriptor's range (their loads return 0 and their values are never stored).
__device__ __forceinline__ uint32_t lane_off(int c, bool on) { return on ? static_cast<uint32_t>(c) * 4u : 0xFFFFFFF0u; }

// x rows [l1^2, l1^2 + n1) of the lane's channel into xr[0..n1); the NM - n1 loads past n1
// repeat row n1 - 1 (the wave-uniform row offset is not range checked, so it stays inside the
// degree block).  rx spans the instance's feature row [NX][C]; an empty descriptor (no x, or a
// source index out of range) reads zeros.  No value is inspected here: the loads stay in flight
// until the degree's first path uses them.
template <int NM>
__device__ __forceinline__ void load_x(const GenTable& t, int l1, rsrc_t rx, uint32_t lo, float (&xr)[NM]) {
  const int n1 = 2 * l1 + 1;
  const uint32_t row = static_cast<uint32_t>(t.channels) * 4u;
#pragma unroll
  for (int i = 0; i < NM; ++i) xr[i] = buf_load_vs(rx, lo, static_cast<uint32_t>(l1 * l1 + (i < n1 ? i : n1 - 1)) * row);
}

// A path's gate and its n3 dout rows (rows past n3 repeat row n3 - 1), requested one path ahead.
template <int NM>
struct PathIn {
  float gv;
  float o[NM];
};

template <int NM>
__device__ __forceinline__ void load_path(const GenTable& t, int p, rsrc_t rg, rsrc_t rgo, uint32_t lo,
                                          PathIn<NM>& in) {
  const PathInfo q = path_info(t, p);
  const uint32_t row = static_cast<uint32_t>(t.channels) * 4u;
  in.gv = buf_load_vs(rg, lo, static_cast<uint32_t>(p) * row);
#pragma unroll
  for (int k = 0; k < NM; ++k) in.o[k] = buf_load_vs(rgo, lo, static_cast<uint32_t>(q.out + (k < q.n3 ? k : q.n3 - 1)) * row);
}

// Rows of one instance: x + row * NX * C (or an empty descriptor), and [n][C] blocks.
__device__ __forceinline__ rsrc_t x_row(const float* x, int64_t row, bool valid, const GenTable& t) {
  const uint32_t bytes = static_cast<uint32_t>(t.nx * t.channels) * 4u;
  return make_rsrc(x && valid ? x + row * t.nx * t.channels : nullptr, bytes);
}

__device__ __forceinline__ rsrc_t block_rows(const float* base, int64_t row, int n, int C) {
  return make_rsrc(base ? base + row * n * C : nullptr, static_cast<uint32_t>(n * C) * 4u);
}

// sum_i xr[i] * b[i] over the N1 components of the degree (the bond row k of a path); the row
// is left in bv for the dx update.
template <int N1, int NM>
__device__ __forceinline__ float row_dot(const float* b, const float (&xr)[NM], float (&bv)[NM]) {
#pragma unroll
  for (int i = 0; i < N1; ++i) bv[i] = b[i];
  float acc = 0.f;
#pragma unroll
  for (int i = 0; i < N1; ++i) acc = fmaf(xr[i], bv[i], acc);
  return acc;
}

// Forward of one instance: out rows [NOC][C] written, or added to when accumulate is set.  The
// next path's gate, and the next input degree's x rows, are requested before the current path
// is computed.  `prepare` (the bond build) runs once, after the first chunk's first loads are
// issued.
template <int NM, typename Prepare>
__device__ void forward_instance(const GenTable& t, const float* sM, rsrc_t rx, rsrc_t rg, float* out,
                                 bool accumulate, int lane, Prepare&& prepare) {
  const int C = t.channels;
  const uint32_t row = static_cast<uint32_t>(C) * 4u;
  bool first = true;
  for (int c0 = 0; c0 < C; c0 += kLanes) {
    const int c = c0 + lane;
    const bool on = c < C;
    const uint32_t lo = lane_off(c, on);
    float xr[NM], xn[NM], bv[NM];
    int lcur = path_info(t, 0).l1;
    load_x<NM>(t, lcur, rx, lo, xr);
    float gv = buf_load_vs(rg, lo, 0u);
    if (first) {
      prepare();
      first = false;
    }
    for (int p = 0; p < t.np; ++p) {
      const PathInfo q = path_info(t, p);
      const bool more = p + 1 < t.np;
      const int lnext = more ? path_info(t, p + 1).l1 : q.l1;
      const float gnext = more ? buf_load_vs(rg, lo, static_cast<uint32_t>(p + 1) * row) : 0.f;
      if (lnext != q.l1) load_x<NM>(t, lnext, rx, lo, xn);
      const float* bond = sM + t.bond[p];
      with_width<NM>(q.n1, [&](auto N1) {
        for (int k = 0; k < q.n3; ++k) {
          const float acc = row_dot<N1>(bond + k * N1, xr, bv);
          if (on) {
            float* dst = out + static_cast<int64_t>(q.out + k) * C + c;
            *dst = accumulate ? *dst + acc * gv : acc * gv;
          }
        }
      });
      gv = gnext;
      if (lnext != q.l1) {
#pragma unroll
        for (int i = 0; i < NM; ++i) xr[i] = xn[i];
      }
    }
  }
}

struct BwdLds {
  float* sX;     // [2 lin + 1][64] x rows of the current input degree (lane columns)
  float* sG;     // [2 lout + 1][64] go_k of the current path
  float* sO;     // [2 lout + 1][64] dout_k of the current path
  float* sDY;    // [64] dY of the instance
};

// VJP of one instance (L.sDY zeroed): dg and dx rows written when their pointers are set, the dY
// contributions added to L.sDY when want_dy (x is needed for dg and dY).  Every lane takes part
// in the dY butterflies whatever its channel, so the call is wave-uniform.  The next path's gate
// and dout rows, and the next input degree's x rows, are requested before the current path is
// computed; `prepare` (the bond build) runs once, after the first chunk's first loads are issued.
template <int NM, typename Prepare>
__device__ void backward_instance(const GenTable& t, const float* sM, const BwdLds& L, rsrc_t rx, rsrc_t rg,
                                  rsrc_t rgo, float* dx, float* dg, bool want_dy, int lane, Prepare&& prepare) {
  static_assert(NM <= 16, "dY butterfly width");
  const int C = t.channels;
  bool first = true;
  for (int c0 = 0; c0 < C; c0 += kLanes) {
    const int c = c0 + lane;
    const bool on = c < C;
    const uint32_t lo = lane_off(c, on);
    int staged = -1;
    unsigned seen = 0;   // input degrees with at least one path
    float xr[NM], xn[NM], dxr[NM], bv[NM];
    PathIn<NM> cur, nxt;
    load_x<NM>(t, path_info(t, 0).l1, rx, lo, xr);
    load_path<NM>(t, 0, rg, rgo, lo, cur);
    if (first) {
      prepare();
      first = false;
    }
    auto flush = [&](int l) {
#pragma unroll
      for (int i = 0; i < NM; ++i)
        if (i < 2 * l + 1) dx[static_cast<int64_t>(l * l + i) * C + c] = dxr[i];
    };
    for (int p = 0; p < t.np; ++p) {
      const PathInfo q = path_info(t, p);
      const bool more = p + 1 < t.np;
      const int lnext = more ? path_info(t, p + 1).l1 : q.l1;
      if (more) load_path<NM>(t, p + 1, rg, rgo, lo, nxt);
      if (lnext != q.l1) load_x<NM>(t, lnext, rx, lo, xn);
      if (q.l1 != staged) {
        if (staged >= 0 && dx && on) flush(staged);
        if (want_dy) {   // lanes past C contribute nothing to the dY sums
#pragma unroll
          for (int i = 0; i < NM; ++i)
            if (i < q.n1) L.sX[i * kLanes + lane] = on ? xr[i] : 0.f;
        }
#pragma unroll
        for (int i = 0; i < NM; ++i) dxr[i] = 0.f;
        staged = q.l1;
        seen |= 1u << q.l1;
      }
#pragma unroll
      for (int k = 0; k < NM; ++k)
        if (k < q.n3) {
          L.sO[k * kLanes + lane] = cur.o[k];
          L.sG[k * kLanes + lane] = on ? cur.gv * cur.o[k] : 0.f;
        }
      const float* bond = sM + t.bond[p];
      const float* cg = kCGGeneric + t.cg[p];
      float dgv = 0.f;
      with_width<NM>(q.n1, [&](auto N1) {
        for (int k = 0; k < q.n3; ++k) {
          const float base = row_dot<N1>(bond + k * N1, xr, bv);
          dgv = fmaf(base, L.sO[k * kLanes + lane], dgv);
          const float gk = L.sG[k * kLanes + lane];
#pragma unroll
          for (int i = 0; i < N1; ++i) dxr[i] = fmaf(bv[i], gk, dxr[i]);
        }
      });
      if (want_dy) {
        if constexpr (NM == 9) {
          // T[i][k] = sum over the chunk's 64 channels of x_i go_k on the matrix cores: A = the x
          // rows (lane l gives row l % 16), B = the go rows (column l % 16), four consecutive
          // v_mfma_f32_16x16x4_f32 per 16 channels with channel 16 g + 4 (l / 16) + j in both
          // operands (rows and columns past n1 / n3 repeat the last one and are not used); two
          // accumulators over alternate channel groups.  Lane l then holds T[4 (l / 16) + v][l % 16].
          wave_sync();
          const int fr = lane & 15, fq = (lane >> 4) * 4;
          const float* ar = L.sX + (fr < q.n1 ? fr : q.n1 - 1) * kLanes + fq;
          const float* br = L.sG + (fr < q.n3 ? fr : q.n3 - 1) * kLanes + fq;
          f32x4 t0 = {0.f, 0.f, 0.f, 0.f}, t1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int g4 = 0; g4 < 4; g4 += 2) {
            const f32x4 a0 = *reinterpret_cast<const f32x4*>(ar + 16 * g4);
            const f32x4 b0 = *reinterpret_cast<const f32x4*>(br + 16 * g4);
            const f32x4 a1 = *reinterpret_cast<const f32x4*>(ar + 16 * g4 + 16);
            const f32x4 b1 = *reinterpret_cast<const f32x4*>(br + 16 * g4 + 16);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              t0 = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[j], b0[j], t0, 0, 0, 0);
              t1 = __builtin_amdgcn_mfma_f32_16x16x4f32(a1[j], b1[j], t1, 0, 0, 0);
            }
          }
          // dY_j += s sum_{i,k} Chat[i][k][j] T[i][k]: each lane its (up to) four entries with their
          // CG rows (per-lane loads), then the lane partials summed by one transposing butterfly
          // (a fixed order)
          with_width<NM>(q.n2, [&](auto N2) {
            using WS = WaveSums<N2>;
            float part[N2];
#pragma unroll
            for (int j = 0; j < N2; ++j) part[j] = 0.f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
              const int i = fq + v;
              const bool use = i < q.n1 && fr < q.n3;
              const float tv = use ? t0[v] + t1[v] : 0.f;
              const float* row = cg + (use ? i * q.n3 + fr : 0) * N2;
#pragma unroll
              for (int j = 0; j < N2; ++j) part[j] = fmaf(row[j], tv, part[j]);
            }
            const float tot = WS::reduce(part, lane);
            const int j = WS::index(lane);
            if (WS::owner(lane) && j < N2) L.sDY[q.l2 * q.l2 + j] = fmaf(t.scale[p], tot, L.sDY[q.l2 * q.l2 + j]);
          });
        } else {
          with_width<NM>(q.n2, [&](auto N2) {
            // this lane's sum_{i,k} Chat[i][k][j] x_i go_k against the CG rows (scalar loads), then
            // summed over the lanes (a fixed butterfly) and added by the owner lanes
            using WS = WaveSums<N2>;
            float part[N2];
#pragma unroll
            for (int j = 0; j < N2; ++j) part[j] = 0.f;
            for (int i = 0; i < q.n1; ++i) {
              const float xi = L.sX[i * kLanes + lane];
#pragma unroll 4
              for (int k = 0; k < q.n3; ++k) {
                const float tk = xi * L.sG[k * kLanes + lane];
                const float* row = cg + (i * q.n3 + k) * N2;
#pragma unroll
                for (int j = 0; j < N2; ++j) part[j] = fmaf(row[j], tk, part[j]);
              }
            }
            const float tot = WS::reduce(part, lane);
            const int j = WS::index(lane);
            if (WS::owner(lane) && j < N2) L.sDY[q.l2 * q.l2 + j] = fmaf(t.scale[p], tot, L.sDY[q.l2 * q.l2 + j]);
          });
        }
      }
      if (dg && on) dg[static_cast<int64_t>(p) * C + c] = dgv;
      if (more) {
        cur = nxt;
        if (lnext != q.l1) {
#pragma unroll
          for (int i = 0; i < NM; ++i) xr[i] = xn[i];
        }
      }
    }
    if (dx && on) {
      if (staged >= 0) flush(staged);
      for (int l = 0; l <= t.lin; ++l)        // degrees without a path: zero adjoint
        if (!((seen >> l) & 1u))
          for (int i = 0; i < 2 * l + 1; ++i) dx[static_cast<int64_t>(l * l + i) * C + c] = 0.f;
    }
  }
}

// LDS carve-up, in floats: sY | sDY | sM | (sX | sG | sO)
__host__ __device__ __forceinline__ int bond_floats(const GenTable& t) { return (t.nb + 3) & ~3; }
__host__ __device__ __forceinline__ int fwd_lds_floats(const GenTable& t) { return kHead + bond_floats(t); }
__host__ __device__ __forceinline__ int bwd_lds_floats(const GenTable& t) {
  return fwd_lds_floats(t) + ((2 * t.lin + 1) + 2 * (2 * t.lout + 1)) * kLanes;
}

__device__ __forceinline__ BwdLds carve(float* lds, const GenTable& t) {
  BwdLds L;
  L.sDY = lds + kLanes;
  L.sX = lds + kHead + bond_floats(t);
  L.sG = L.sX + (2 * t.lin + 1) * kLanes;
  L.sO = L.sG + (2 * t.lout + 1) * kLanes;
  return L;
}

// Harmonics of an instance (requested one instance ahead into yv: lanes below NY) into sY, sDY
// zeroed, barrier.  The bonds are built by the instance functions' `prepare` step.
__device__ __forceinline__ void stage_y(float yv, float* lds, int lane) {
  lds[lane] = yv;
  lds[kLanes + lane] = 0.f;
  __syncthreads();
}

__device__ __forceinline__ float load_y(const GenTable& t, const float* y, int64_t r, bool valid, int lane) {
  float v = 0.f;
  if (valid && lane < t.ny) v = y[r * t.ny + lane];
  return v;
}

template <int NM>
__global__ void __launch_bounds__(kLanes)
gen_tp_forward_kernel(const GenTable t, const float* __restrict__ x, const float* __restrict__ y,
                      const float* __restrict__ g, float* __restrict__ out, int64_t rows) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x;
  const int C = t.channels;
  float yv = load_y(t, y, blockIdx.x, blockIdx.x < rows, lane);
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    stage_y(yv, lds, lane);
    yv = load_y(t, y, r + gridDim.x, r + gridDim.x < rows, lane);
    forward_instance<NM>(t, lds + kHead, x_row(x, r, true, t), block_rows(g, r, t.np, C), out + r * t.noc * C,
                         false, lane, [&] {
                           build_bonds(t, lds, lds + kHead, lane);
                           __syncthreads();
                         });
    __syncthreads();
  }
}

template <int NM>
__global__ void __launch_bounds__(kLanes)
gen_tp_backward_kernel(const GenTable t, const float* __restrict__ x, const float* __restrict__ y,
                       const float* __restrict__ g, const float* __restrict__ go, float* __restrict__ dx,
                       float* __restrict__ dy, float* __restrict__ dg, int64_t rows) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x;
  const int C = t.channels;
  const BwdLds L = carve(lds, t);
  float yv = load_y(t, y, blockIdx.x, blockIdx.x < rows, lane);
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    stage_y(yv, lds, lane);
    yv = load_y(t, y, r + gridDim.x, r + gridDim.x < rows, lane);
    backward_instance<NM>(t, lds + kHead, L, x_row(x, r, true, t), block_rows(g, r, t.np, C),
                          block_rows(go, r, t.noc, C), dx ? dx + r * t.nx * C : nullptr,
                          dg ? dg + r * t.np * C : nullptr, dy != nullptr, lane, [&] {
                            build_bonds(t, lds, lds + kHead, lane);
                            __syncthreads();
                          });
    __syncthreads();
    if (dy && lane < t.ny) dy[r * t.ny + lane] = L.sDY[lane];
  }
}

// Receiver-CSR message forward: one node at a time per workgroup, its edges in CSR order.
template <int NM>
__global__ void __launch_bounds__(kLanes)
gen_msg_forward_kernel(const GenTable t, const float* __restrict__ x, const float* __restrict__ y,
                       const float* __restrict__ g, const int64_t* __restrict__ src,
                       const int64_t* __restrict__ rowptr, const int64_t* __restrict__ perm, float* __restrict__ out,
                       int64_t nodes_src, int64_t nodes_dst) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x;
  const int C = t.channels;
  for (int64_t n = blockIdx.x; n < nodes_dst; n += gridDim.x) {
    const int64_t q0 = rowptr[n], q1 = rowptr[n + 1];
    float* orow = out + n * t.noc * C;
    if (q0 == q1) {
      for (int64_t i = lane; i < static_cast<int64_t>(t.noc) * C; i += kLanes) orow[i] = 0.f;
      continue;
    }
    int64_t e = perm ? perm[q0] : q0;
    float yv = load_y(t, y, e, true, lane);
    for (int64_t q = q0; q < q1; ++q) {
      stage_y(yv, lds, lane);
      const int64_t s = src[e];
      const int64_t en = q + 1 < q1 ? (perm ? perm[q + 1] : q + 1) : e;
      yv = load_y(t, y, en, q + 1 < q1, lane);
      forward_instance<NM>(t, lds + kHead, x_row(x, s, s >= 0 && s < nodes_src, t), block_rows(g, e, t.np, C),
                           orow, q != q0, lane, [&] {
                             build_bonds(t, lds, lds + kHead, lane);
                             __syncthreads();
                           });
      __syncthreads();
      e = en;
    }
  }
}

// Receiver-CSR edge adjoint: per edge e of node n, the TP VJP with dout = go[n].
template <int NM>
__global__ void __launch_bounds__(kLanes)
gen_msg_edge_grad_kernel(const GenTable t, const float* __restrict__ x, const float* __restrict__ y,
                         const float* __restrict__ g, const float* __restrict__ go,
                         const int64_t* __restrict__ src, const int64_t* __restrict__ rowptr,
                         const int64_t* __restrict__ perm, float* __restrict__ dyp, float* __restrict__ dg,
                         float* __restrict__ dxe, int64_t nodes_src, int64_t nodes_dst, int chunks) {
  extern __shared__ float lds[];
  const int lane = threadIdx.x;
  const int C = t.channels;
  const BwdLds L = carve(lds, t);
  for (int64_t n = blockIdx.x; n < nodes_dst; n += gridDim.x) {
    const int64_t q0 = rowptr[n], q1 = rowptr[n + 1];
    if (q0 == q1) continue;
    const rsrc_t rgo = block_rows(go, n, t.noc, C);
    int64_t e = perm ? perm[q0] : q0;
    float yv = load_y(t, y, e, true, lane);
    for (int64_t q = q0; q < q1; ++q) {
      stage_y(yv, lds, lane);
      const int64_t s = src[e];
      const int64_t en = q + 1 < q1 ? (perm ? perm[q + 1] : q + 1) : e;
      yv = load_y(t, y, en, q + 1 < q1, lane);
      backward_instance<NM>(t, lds + kHead, L, x_row(x, s, s >= 0 && s < nodes_src, t), block_rows(g, e, t.np, C),
                            rgo, dxe ? dxe + e * t.nx * C : nullptr, dg ? dg + e * t.np * C : nullptr,
                            dyp != nullptr, lane, [&] {
                              build_bonds(t, lds, lds + kHead, lane);
                              __syncthreads();
                            });
      __syncthreads();
      if (dyp) {
        float* d = dyp + e * chunks * t.ny;
        for (int i = lane; i < chunks * t.ny; i += kLanes) d[i] = i < t.ny ? L.sDY[i] : 0.f;
      }
      e = en;
    }
  }
}

int make_table(const ictc_tp_desc& d, GenTable* t) {
  if (d.input_lmax > kGenericMaxL || d.edge_lmax > kGenericMaxL || d.output_lmax > kGenericMaxL)
    return ICTC_ERR_UNSUPPORTED;
  const PathTable pt = make_paths(d.input_lmax, d.edge_lmax, d.output_lmax);
  *t = GenTable{};
  t->np = pt.n;
  t->nb = pt.nbond;
  t->noc = pt.noc;
  t->nx = (d.input_lmax + 1) * (d.input_lmax + 1);
  t->ny = (d.edge_lmax + 1) * (d.edge_lmax + 1);
  t->channels = d.channels;
  t->lin = d.input_lmax;
  t->lout = d.output_lmax;
  constexpr int G = kCGGenericMaxL + 1;
  for (int p = 0; p < pt.n; ++p) {
    const int off = kCGGenericOffset[(pt.l1[p] * G + pt.l2[p]) * G + pt.l3[p]];
    if (off < 0) return ICTC_ERR_INVALID_ARGUMENT;
    t->meta[p] = pt.l1[p] | pt.l2[p] << 4 | pt.l3[p] << 8 | pt.out[p] << 12;
    t->bond[p] = pt.bond[p];
    t->cg[p] = off;
    t->scale[p] = d.scale[p];
  }
  return ICTC_OK;
}

unsigned grid_for(int64_t instances) {
  return static_cast<unsigned>(instances < kGridCap ? instances : kGridCap);
}

int status() { return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH; }

// Every degree <= 4: the kernels keep 9 components per degree in registers instead of 13.
bool narrow(const ictc_tp_desc& d) { return d.input_lmax <= 4 && d.edge_lmax <= 4 && d.output_lmax <= 4; }

}  // namespace

int generic_tp_forward(const ictc_tp_desc& d, const float* x, const float* y, const float* g, float* out,
                       int64_t rows, hipStream_t stream) {
  GenTable t;
  const int st = make_table(d, &t);
  if (st != ICTC_OK) return st;
  const dim3 grid(grid_for(rows)), block(kLanes);
  const size_t lds = fwd_lds_floats(t) * sizeof(float);
  if (narrow(d))
    hipLaunchKernelGGL(gen_tp_forward_kernel<9>, grid, block, lds, stream, t, x, y, g, out, rows);
  else
    hipLaunchKernelGGL(gen_tp_forward_kernel<13>, grid, block, lds, stream, t, x, y, g, out, rows);
  return status();
}

int generic_tp_backward(const ictc_tp_desc& d, const float* x, const float* y, const float* g, const float* go,
                        float* dx, float* dy, float* dg, int64_t rows, hipStream_t stream) {
  GenTable t;
  const int st = make_table(d, &t);
  if (st != ICTC_OK) return st;
  const dim3 grid(grid_for(rows)), block(kLanes);
  const size_t lds = bwd_lds_floats(t) * sizeof(float);
  if (narrow(d))
    hipLaunchKernelGGL(gen_tp_backward_kernel<9>, grid, block, lds, stream, t, x, y, g, go, dx, dy, dg, rows);
  else
    hipLaunchKernelGGL(gen_tp_backward_kernel<13>, grid, block, lds, stream, t, x, y, g, go, dx, dy, dg, rows);
  return status();
}

int generic_msg_forward(const ictc_tp_desc& d, const float* x, const float* y, const float* g, const int64_t* src,
                        const int64_t* rowptr, const int64_t* perm, float* out, int64_t nodes_src,
                        int64_t nodes_dst, hipStream_t stream) {
  GenTable t;
  const int st = make_table(d, &t);
  if (st != ICTC_OK) return st;
  const dim3 grid(grid_for(nodes_dst)), block(kLanes);
  const size_t lds = fwd_lds_floats(t) * sizeof(float);
  if (narrow(d))
    hipLaunchKernelGGL(gen_msg_forward_kernel<9>, grid, block, lds, stream, t, x, y, g, src, rowptr, perm, out,
                       nodes_src, nodes_dst);
  else
    hipLaunchKernelGGL(gen_msg_forward_kernel<13>, grid, block, lds, stream, t, x, y, g, src, rowptr, perm, out,
                       nodes_src, nodes_dst);
  return status();
}

int generic_msg_edge_grad(const ictc_tp_desc& d, const float* x, const float* y, const float* g, const float* go,
                          const int64_t* src, const int64_t* rowptr, const int64_t* perm, float* dyp, float* dg,
                          float* dxe, int64_t nodes_src, int64_t nodes_dst, hipStream_t stream) {
  GenTable t;
  const int st = make_table(d, &t);
  if (st != ICTC_OK) return st;
  const int chunks = (d.channels + kLanes - 1) / kLanes;
  const dim3 grid(grid_for(nodes_dst)), block(kLanes);
  const size_t lds = bwd_lds_floats(t) * sizeof(float);
  if (narrow(d))
    hipLaunchKernelGGL(gen_msg_edge_grad_kernel<9>, grid, block, lds, stream, t, x, y, g, go, src, rowptr, perm, dyp,
                       dg, dxe, nodes_src, nodes_dst, chunks);
  else
    hipLaunchKernelGGL(gen_msg_edge_grad_kernel<13>, grid, block, lds, stream, t, x, y, g, go, src, rowptr, perm,
                       dyp, dg, dxe, nodes_src, nodes_dst, chunks);
  return status();
}

}  // namespace ictc
