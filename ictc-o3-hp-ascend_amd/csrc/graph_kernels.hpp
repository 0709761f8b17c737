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
// One thread per receiver j; for every candidate i in a visited bin, with that visit's
// image u (integer lattice coordinates of the bin copy),
//   d = wpos[j] - (wpos[i] + u @ cell),  kept when |d|^2 < cutoff^2 and (i, u) != (j, 0);
// the edge's image in wrapped coordinates is t = -u (vec = wpos[j] - wpos[i] + t @ cell).
// The count pass writes each receiver's degree; the fill pass writes (src, t) rows at the
// receiver's CSR offset in a fixed visiting order (deterministic).
#pragma once
#include "ictc_common.hpp"

namespace ictc {

__device__ __forceinline__ void floor_divmod(int b, int n, int& q, int& r) {
  q = b >= 0 ? b / n : -((-b + n - 1) / n);
  r = b - q * n;
}

template <bool FILL>
__global__ void __launch_bounds__(256)
radius_graph_kernel(const double* __restrict__ wpos, const int32_t* __restrict__ abin,
                    const int64_t* __restrict__ bin_start, const int64_t* __restrict__ bin_atoms,
                    int64_t atoms, const ictc_cell_grid g, int64_t* __restrict__ counts,
                    const int64_t* __restrict__ rowptr, int64_t* __restrict__ src_out,
                    int32_t* __restrict__ image_out) {
  const int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (j >= atoms) return;
  const double px = wpos[3 * j], py = wpos[3 * j + 1], pz = wpos[3 * j + 2];
  const int bx = abin[3 * j], by = abin[3 * j + 1], bz = abin[3 * j + 2];
  int64_t k = 0;
  const int64_t base = FILL ? rowptr[j] : 0;
  // the fill pass writes at most the row length the count pass found (memory safety even if
  // the two passes ever disagreed; with the explicit fmas below they compute identically)
  const int64_t cap = FILL ? rowptr[j + 1] - base : 0;
  for (int dx = -g.reach[0]; dx <= g.reach[0]; ++dx) {
    int ux, wx;
    floor_divmod(bx + dx, g.bins[0], ux, wx);
    if (!g.periodic[0] && ux != 0) continue;
    for (int dy = -g.reach[1]; dy <= g.reach[1]; ++dy) {
      int uy, wy;
      floor_divmod(by + dy, g.bins[1], uy, wy);
      if (!g.periodic[1] && uy != 0) continue;
      for (int dz = -g.reach[2]; dz <= g.reach[2]; ++dz) {
        int uz, wz;
        floor_divmod(bz + dz, g.bins[2], uz, wz);
        if (!g.periodic[2] && uz != 0) continue;
        // cartesian offset of this bin copy: u @ cell (rows of cell are lattice vectors)
        const double fx = ux, fy = uy, fz = uz;
        const double ox = fma(fz, g.cell[6], fma(fy, g.cell[3], fx * g.cell[0]));
        const double oy = fma(fz, g.cell[7], fma(fy, g.cell[4], fx * g.cell[1]));
        const double oz = fma(fz, g.cell[8], fma(fy, g.cell[5], fx * g.cell[2]));
        const bool home = ux == 0 && uy == 0 && uz == 0;
        const int64_t bin = (static_cast<int64_t>(wx) * g.bins[1] + wy) * g.bins[2] + wz;
        for (int64_t a = bin_start[bin], a1 = bin_start[bin + 1]; a < a1; ++a) {
          const int64_t i = bin_atoms[a];
          if (home && i == j) continue;
          const double ex = px - (wpos[3 * i] + ox);
          const double ey = py - (wpos[3 * i + 1] + oy);
          const double ez = pz - (wpos[3 * i + 2] + oz);
          if (fma(ez, ez, fma(ey, ey, ex * ex)) < g.cutoff_sq) {
            if (FILL && k < cap) {
              src_out[base + k] = i;
              image_out[3 * (base + k)] = -ux;
              image_out[3 * (base + k) + 1] = -uy;
              image_out[3 * (base + k) + 2] = -uz;
            }
            ++k;
          }
        }
      }
    }
  }
  if constexpr (!FILL) counts[j] = k;
}

}  // namespace ictc
