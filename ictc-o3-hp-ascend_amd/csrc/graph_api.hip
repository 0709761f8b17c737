// C ABI of the periodic radius-graph builder (graph_kernels.hpp).
#include "graph_kernels.hpp"

namespace ictc {
namespace {

constexpr int kMaxReach = 64;

int grid_status(const ictc_cell_grid* g, const double* wpos, const int32_t* abin, const int64_t* bin_start,
                const int64_t* bin_atoms, int64_t atoms) {
  if (g == nullptr || atoms < 0) return ICTC_ERR_INVALID_ARGUMENT;
  if (!(g->cutoff_sq > 0.0)) return ICTC_ERR_INVALID_ARGUMENT;
  for (int a = 0; a < 3; ++a) {
    if (g->bins[a] < 1 || g->reach[a] < 0 || g->reach[a] > kMaxReach) return ICTC_ERR_INVALID_ARGUMENT;
    if (g->periodic[a] != 0 && g->periodic[a] != 1) return ICTC_ERR_INVALID_ARGUMENT;
  }
  const int64_t nbins = static_cast<int64_t>(g->bins[0]) * g->bins[1] * g->bins[2];
  if (nbins > (int64_t{1} << 31)) return ICTC_ERR_INVALID_ARGUMENT;
  if (atoms > 0 && (!wpos || !abin || !bin_start || !bin_atoms)) return ICTC_ERR_INVALID_ARGUMENT;
  return ICTC_OK;
}

dim3 grid_blocks(int64_t atoms) { return dim3(static_cast<unsigned>((atoms + 255) / 256)); }
dim3 wave_blocks(int64_t atoms) { return dim3(static_cast<unsigned>((atoms + kGraphWaves - 1) / kGraphWaves)); }

}  // namespace
}  // namespace ictc

extern "C" {

int ictc_hip_radius_graph_count(const ictc_cell_grid* grid, const double* wrapped_positions,
                                const int32_t* atom_bins, const int64_t* bin_start, const int64_t* bin_atoms,
                                int64_t atoms, int64_t* counts, hipStream_t stream) {
  const int st = ictc::grid_status(grid, wrapped_positions, atom_bins, bin_start, bin_atoms, atoms);
  if (st != ICTC_OK) return st;
  if (atoms == 0) return ICTC_OK;
  if (!counts) return ICTC_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(ictc::radius_count_kernel, ictc::wave_blocks(atoms), dim3(ictc::kGraphWaves * ictc::kWave), 0,
                     stream, wrapped_positions, atom_bins, bin_start, bin_atoms, atoms, *grid, counts);
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}

int ictc_hip_radius_graph_fill(const ictc_cell_grid* grid, const double* wrapped_positions,
                               const int32_t* atom_bins, const int64_t* bin_start, const int64_t* bin_atoms,
                               int64_t atoms, const int64_t* rowptr, int64_t* src, int32_t* images,
                               hipStream_t stream) {
  const int st = ictc::grid_status(grid, wrapped_positions, atom_bins, bin_start, bin_atoms, atoms);
  if (st != ICTC_OK) return st;
  if (atoms == 0) return ICTC_OK;
  if (!rowptr || !src || !images) return ICTC_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(ictc::radius_fill_kernel, ictc::grid_blocks(atoms), dim3(256), 0, stream, wrapped_positions,
                     atom_bins, bin_start, bin_atoms, atoms, *grid, rowptr, src, images);
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}

int64_t ictc_hip_radius_graph_row_capacity(void) { return ictc::kGraphRowCap; }

int ictc_hip_radius_graph_fill_sorted(const ictc_cell_grid* grid, const double* wrapped_positions,
                                      const int32_t* atom_bins, const int64_t* bin_start, const int64_t* bin_atoms,
                                      int64_t atoms, const int64_t* rowptr, const int64_t* image_base, int64_t* src,
                                      int64_t* dst, double* shifts, hipStream_t stream) {
  const int st = ictc::grid_status(grid, wrapped_positions, atom_bins, bin_start, bin_atoms, atoms);
  if (st != ICTC_OK) return st;
  if (atoms == 0) return ICTC_OK;
  if (!rowptr || !image_base || !src || !dst || !shifts) return ICTC_ERR_INVALID_ARGUMENT;
  hipLaunchKernelGGL(ictc::radius_fill_sorted_kernel, ictc::wave_blocks(atoms),
                     dim3(ictc::kGraphWaves * ictc::kWave), 0, stream, wrapped_positions, atom_bins, bin_start,
                     bin_atoms, atoms, *grid, rowptr, image_base, src, dst, shifts);
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}

int ictc_hip_edge_vector_grad(int dtype, const void* grad_vec, const int64_t* dst_rowptr, const int64_t* dst_perm,
                              const int64_t* src_rowptr, const int64_t* src_perm, void* grad_pos, int64_t nodes,
                              hipStream_t stream) {
  if (nodes < 0 || (dtype != 0 && dtype != 1)) return ICTC_ERR_INVALID_ARGUMENT;
  if (nodes == 0) return ICTC_OK;
  if (!grad_pos || !dst_rowptr || !src_rowptr || !grad_vec) return ICTC_ERR_INVALID_ARGUMENT;
  if (dtype == 0)
    hipLaunchKernelGGL(ictc::edge_vector_grad_kernel<float>, ictc::wave_blocks(nodes),
                       dim3(ictc::kGraphWaves * ictc::kWave), 0, stream, static_cast<const float*>(grad_vec),
                       dst_rowptr, dst_perm, src_rowptr, src_perm, static_cast<float*>(grad_pos), nodes);
  else
    hipLaunchKernelGGL(ictc::edge_vector_grad_kernel<double>, ictc::wave_blocks(nodes),
                       dim3(ictc::kGraphWaves * ictc::kWave), 0, stream, static_cast<const double*>(grad_vec),
                       dst_rowptr, dst_perm, src_rowptr, src_perm, static_cast<double*>(grad_pos), nodes);
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}

}  // extern "C"
