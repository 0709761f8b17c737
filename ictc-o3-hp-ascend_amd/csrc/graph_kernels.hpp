// Periodic radius graph over a cell list (gfx950).
//
// Replaces the torch_cluster-based builder of reference
// mace_ictc/utils/graph_utils.py:217-297 (radius_graph_pbc_gpu: one radius query per
// periodic image, then concatenation).  Here atoms are binned once in fractional
// coordinates, every receiver scans the bins within reach of its own (each bin visit
// carries an explicit lattice image, so cells narrower than the cutoff enumerate every
// image exactly once), and the result is exact (no neighbour cap).
//
// Inputs prepared by the host (ictc_o3 graph builder):
//   wpos [N,3] float64: positions wrapped into the cell along periodic axes (cartesian);
//   abin [N,3] int32: each atom's bin coordinates;
//   bin_start [nbins+1] int64, bin_atoms [N] int64: atoms grouped by bin (CSR).
// For a receiver j and every candidate i in a visited bin, with that visit's image u (integer
// lattice coordinates of the bin copy),
//   d = wpos[j] - (wpos[i] + u @ cell),  kept when |d|^2 < cutoff^2 and (i, u) != (j, 0);
// the edge's image in wrapped coordinates is t = -u (vec = wpos[j] - wpos[i] + t @ cell).
// Every kernel below evaluates a candidate through the same bin_visit / scan_visit code, so
// the count and fill passes agree exactly.
//   radius_count_kernel: one wave per receiver, lanes over the (2 reach + 1)^3 bin visits,
//     a wave sum gives the degree;
//   radius_fill_sorted_kernel: one wave per receiver; its hits go to LDS as unique 64-bit keys
//     (src, t) (lexicographic order = the key order) and each is written at its rank in the
//     row, so rows come out ordered by (src, shift) with dst and the final shift written
//     directly (shift = t - n0[dst] + n0[src], n0 = the atoms' wrap images);
//   radius_fill_kernel: one thread per receiver, hits in visiting order (src, t) at the
//     receiver's CSR offset; for rows longer than the LDS key capacity (the host orders them).
#pragma once
#include "ictc_common.hpp"

namespace ictc {

__device__ __forceinline__ void floor_divmod(int b, int n, int& q, int& r) {
  q = b >= 0 ? b / n : -((-b + n - 1) / n);
  r = b - q * n;
}

constexpr int kGraphWaves = 4;        // receivers (waves) per 256-thread workgroup
constexpr int kGraphRowCap = 1024;    // keys per receiver held in LDS by the sorted fill

// Visit v (dz fastest, then dy, then dx) of receiver bin (bx, by, bz): the bin copy and its image.
struct BinVisit {
  int64_t bin;
  int ux, uy, uz;
  bool ok;   // false for an image along a non-periodic axis
};

__device__ __forceinline__ BinVisit bin_visit(const ictc_cell_grid& g, int bx, int by, int bz, int v) {
  const int nz = 2 * g.reach[2] + 1, ny = 2 * g.reach[1] + 1;
  const int dz = v % nz - g.reach[2];
  v /= nz;
  const int dy = v % ny - g.reach[1];
  const int dx = v / ny - g.reach[0];
  BinVisit r;
  int wx, wy, wz;
  floor_divmod(bx + dx, g.bins[0], r.ux, wx);
  floor_divmod(by + dy, g.bins[1], r.uy, wy);
  floor_divmod(bz + dz, g.bins[2], r.uz, wz);
  r.ok = (g.periodic[0] || r.ux == 0) && (g.periodic[1] || r.uy == 0) && (g.periodic[2] || r.uz == 0);
  r.bin = (static_cast<int64_t>(wx) * g.bins[1] + wy) * g.bins[2] + wz;
  return r;
}

__device__ __forceinline__ int visit_count(const ictc_cell_grid& g) {
  return (2 * g.reach[0] + 1) * (2 * g.reach[1] + 1) * (2 * g.reach[2] + 1);
}

// Calls hit(i) for every atom i of the visited bin copy within the cutoff of receiver j.
template <typename F>
__device__ __forceinline__ void scan_visit(const double* __restrict__ wpos, const int64_t* __restrict__ bin_start,
                                           const int64_t* __restrict__ bin_atoms, const ictc_cell_grid& g,
                                           const BinVisit& b, int64_t j, double px, double py, double pz, F&& hit) {
  // cartesian offset of this bin copy: u @ cell (rows of cell are lattice vectors)
  const double fx = b.ux, fy = b.uy, fz = b.uz;
  const double ox = fma(fz, g.cell[6], fma(fy, g.cell[3], fx * g.cell[0]));
  const double oy = fma(fz, g.cell[7], fma(fy, g.cell[4], fx * g.cell[1]));
  const double oz = fma(fz, g.cell[8], fma(fy, g.cell[5], fx * g.cell[2]));
  const bool home = b.ux == 0 && b.uy == 0 && b.uz == 0;
  for (int64_t a = bin_start[b.bin], a1 = bin_start[b.bin + 1]; a < a1; ++a) {
    const int64_t i = bin_atoms[a];
    if (home && i == j) continue;
    const double ex = px - (wpos[3 * i] + ox);
    const double ey = py - (wpos[3 * i + 1] + oy);
    const double ez = pz - (wpos[3 * i + 2] + oz);
    if (fma(ez, ez, fma(ey, ey, ex * ex)) < g.cutoff_sq) hit(i);
  }
}

__global__ void __launch_bounds__(kGraphWaves * kWave)
radius_count_kernel(const double* __restrict__ wpos, const int32_t* __restrict__ abin,
                    const int64_t* __restrict__ bin_start, const int64_t* __restrict__ bin_atoms, int64_t atoms,
                    const ictc_cell_grid g, int64_t* __restrict__ counts) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t j = static_cast<int64_t>(blockIdx.x) * kGraphWaves + threadIdx.x / kWave;
  if (j >= atoms) return;   // whole waves only; no workgroup barrier in this kernel
  const double px = wpos[3 * j], py = wpos[3 * j + 1], pz = wpos[3 * j + 2];
  const int bx = abin[3 * j], by = abin[3 * j + 1], bz = abin[3 * j + 2];
  int k = 0;
  for (int v = lane, nv = visit_count(g); v < nv; v += kWave) {
    const BinVisit b = bin_visit(g, bx, by, bz, v);
    if (b.ok) scan_visit(wpos, bin_start, bin_atoms, g, b, j, px, py, pz, [&](int64_t) { ++k; });
  }
#pragma unroll
  for (int o = kWave / 2; o > 0; o >>= 1) k += __shfl_xor(k, o);
  if (lane == 0) counts[j] = k;
}

// Key of edge (src i, image t): i above three 8-bit image components offset by 128 (|t| <= 65
// with reach <= 64), so integer order = lexicographic (i, tx, ty, tz) order.
__device__ __forceinline__ int64_t edge_key(int64_t i, const BinVisit& b) {
  return (i << 24) | (static_cast<int64_t>(128 - b.ux) << 16) | (static_cast<int64_t>(128 - b.uy) << 8) |
         static_cast<int64_t>(128 - b.uz);
}

// Rows must hold at most kGraphRowCap edges (the host checks the counts; a longer row would be
// cut to its first kGraphRowCap keys, never written out of bounds).
__global__ void __launch_bounds__(kGraphWaves * kWave)
radius_fill_sorted_kernel(const double* __restrict__ wpos, const int32_t* __restrict__ abin,
                          const int64_t* __restrict__ bin_start, const int64_t* __restrict__ bin_atoms,
                          int64_t atoms, const ictc_cell_grid g, const int64_t* __restrict__ rowptr,
                          const int64_t* __restrict__ image_base, int64_t* __restrict__ src_out,
                          int64_t* __restrict__ dst_out, double* __restrict__ shift_out) {
  __shared__ int64_t sKey[kGraphWaves][kGraphRowCap];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int64_t j = static_cast<int64_t>(blockIdx.x) * kGraphWaves + wave;
  const bool valid = j < atoms;   // no early return: the workgroup barrier below needs every wave
  int64_t base = 0, len = 0;
  double px = 0, py = 0, pz = 0;
  int bx = 0, by = 0, bz = 0;
  if (valid) {
    base = rowptr[j];
    len = min(rowptr[j + 1] - base, static_cast<int64_t>(kGraphRowCap));
    px = wpos[3 * j], py = wpos[3 * j + 1], pz = wpos[3 * j + 2];
    bx = abin[3 * j], by = abin[3 * j + 1], bz = abin[3 * j + 2];
  }
  const int nv = valid ? visit_count(g) : 0;
  // pass 1: this lane's hits; exclusive scan over the wave gives its first key slot
  int mine = 0;
  for (int v = lane; v < nv; v += kWave) {
    const BinVisit b = bin_visit(g, bx, by, bz, v);
    if (b.ok) scan_visit(wpos, bin_start, bin_atoms, g, b, j, px, py, pz, [&](int64_t) { ++mine; });
  }
  int incl = mine;
#pragma unroll
  for (int o = 1; o < kWave; o <<= 1) {
    const int t = __shfl_up(incl, o);
    if (lane >= o) incl += t;
  }
  // pass 2: keys into LDS
  int64_t slot = incl - mine;
  for (int v = lane; v < nv; v += kWave) {
    const BinVisit b = bin_visit(g, bx, by, bz, v);
    if (b.ok)
      scan_visit(wpos, bin_start, bin_atoms, g, b, j, px, py, pz, [&](int64_t i) {
        if (slot < len) sKey[wave][slot] = edge_key(i, b);
        ++slot;
      });
  }
  __syncthreads();
  // each key's rank in the row (keys are unique) is its output slot
  const int64_t* __restrict__ keys = sKey[wave];
  for (int64_t e = lane; e < len; e += kWave) {
    const int64_t key = keys[e];
    int64_t r = 0;
    for (int64_t k = 0; k < len; ++k) r += keys[k] < key;
    const int64_t i = key >> 24;
    const int64_t o = base + r;
    src_out[o] = i;
    dst_out[o] = j;
#pragma unroll
    for (int a = 0; a < 3; ++a) {
      const int64_t t = ((key >> (16 - 8 * a)) & 255) - 128;
      shift_out[3 * o + a] = static_cast<double>(t - image_base[3 * j + a] + image_base[3 * i + a]);
    }
  }
}

__global__ void __launch_bounds__(256)
radius_fill_kernel(const double* __restrict__ wpos, const int32_t* __restrict__ abin,
                   const int64_t* __restrict__ bin_start, const int64_t* __restrict__ bin_atoms, int64_t atoms,
                   const ictc_cell_grid g, const int64_t* __restrict__ rowptr, int64_t* __restrict__ src_out,
                   int32_t* __restrict__ image_out) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= atoms) return;
  const double px = wpos[3 * j], py = wpos[3 * j + 1], pz = wpos[3 * j + 2];
  const int bx = abin[3 * j], by = abin[3 * j + 1], bz = abin[3 * j + 2];
  const int64_t base = rowptr[j];
  // at most the row length the count pass found (memory safety even if the passes disagreed)
  const int64_t cap = rowptr[j + 1] - base;
  int64_t k = 0;
  for (int v = 0, nv = visit_count(g); v < nv; ++v) {
    const BinVisit b = bin_visit(g, bx, by, bz, v);
    if (!b.ok) continue;
    scan_visit(wpos, bin_start, bin_atoms, g, b, j, px, py, pz, [&](int64_t i) {
      if (k < cap) {
        src_out[base + k] = i;
        image_out[3 * (base + k)] = -b.ux;
        image_out[3 * (base + k) + 1] = -b.uy;
        image_out[3 * (base + k) + 2] = -b.uz;
      }
      ++k;
    });
  }
}

// ----------------------------------------------------------------------------- edge vectors
// Adjoint of the edge vectors vec[e] = pos[dst(e)] - pos[src(e)] (+ constant shift):
//   grad_pos[n] = sum_{e: dst(e) = n} grad_vec[e] - sum_{e: src(e) = n} grad_vec[e],
// one wave per node over its receiver-CSR and source-CSR rows; lane l takes the slots
// l, l + 64, ... of each row and the lanes' partials meet in a fixed butterfly, so the result
// does not depend on scheduling (no atomics).
template <typename T>
__device__ __forceinline__ T wave_sum_t(T v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

template <typename T>
__global__ void __launch_bounds__(kGraphWaves * kWave)
edge_vector_grad_kernel(const T* __restrict__ grad_vec, const int64_t* __restrict__ rowptr_dst,
                        const int64_t* __restrict__ perm_dst, const int64_t* __restrict__ rowptr_src,
                        const int64_t* __restrict__ perm_src, T* __restrict__ grad_pos, int64_t nodes) {
  const int64_t n = static_cast<int64_t>(blockIdx.x) * kGraphWaves + threadIdx.x / kWave;
  if (n >= nodes) return;
  const int lane = threadIdx.x & (kWave - 1);
  T a0 = 0, a1 = 0, a2 = 0;
  for (int64_t s = rowptr_dst[n] + lane; s < rowptr_dst[n + 1]; s += kWave) {
    const int64_t e = perm_dst ? perm_dst[s] : s;
    a0 += grad_vec[3 * e];
    a1 += grad_vec[3 * e + 1];
    a2 += grad_vec[3 * e + 2];
  }
  for (int64_t s = rowptr_src[n] + lane; s < rowptr_src[n + 1]; s += kWave) {
    const int64_t e = perm_src ? perm_src[s] : s;
    a0 -= grad_vec[3 * e];
    a1 -= grad_vec[3 * e + 1];
    a2 -= grad_vec[3 * e + 2];
  }
  a0 = wave_sum_t(a0);
  a1 = wave_sum_t(a1);
  a2 = wave_sum_t(a2);
  if (lane == 0) {
    grad_pos[3 * n] = a0;
    grad_pos[3 * n + 1] = a1;
    grad_pos[3 * n + 2] = a2;
  }
}

}  // namespace ictc
