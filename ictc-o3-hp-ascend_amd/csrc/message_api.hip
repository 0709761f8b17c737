// extern "C" entry points of the graph-message family; per-degree instantiations of the
// bond, forward and edge-adjoint kernels are compiled in generated/msg_inst_*.hip, the
// source-node segmented sum (which depends on the input degree only) here.
#include <mutex>

#include "generic.hpp"
#include "message_kernels.hpp"

namespace ictc {

#define ICTC_DECLARE(A, B, C)                                                                      \
  extern template int launch_msg_bonds<A, B, C>(const ictc_tp_desc&, const float*, float*, int64_t, \
                                                hipStream_t);                                       \
  extern template int launch_msg_forward<A, B, C>(const ictc_tp_desc&, const float*, const float*,  \
                                                  const float*, const int64_t*, const int64_t*,     \
                                                  const int64_t*, float*, int64_t, int64_t,         \
                                                  hipStream_t);                                     \
  extern template int launch_msg_edge_grad<A, B, C>(const ictc_tp_desc&, const float*, const float*, \
                                                    const float*, const float*, const int64_t*,     \
                                                    const int64_t*, const int64_t*, float*, float*,  \
                                                    float*, int64_t, int64_t, hipStream_t, int);     \
  extern template int launch_msg_forward_tangent<A, B, C>(                                          \
      const ictc_tp_desc&, const float*, const float*, const float*, const MsgTangent&,             \
      const int64_t*, const int64_t*, const int64_t*, float*, int64_t, int64_t, hipStream_t);       \
  extern template int launch_msg_edge_grad_tangent<A, B, C>(                                        \
      const ictc_tp_desc&, const float*, const float*, const float*, const MsgTangent&,             \
      const float*, const int64_t*, const int64_t*, const int64_t*, float*, float*, float*,         \
      int64_t, int64_t, hipStream_t);
#include "generated/tp_instances.def"
#undef ICTC_DECLARE

using MsgBonds = int (*)(const ictc_tp_desc&, const float*, float*, int64_t, hipStream_t);
using MsgFwd = int (*)(const ictc_tp_desc&, const float*, const float*, const float*, const int64_t*,
                       const int64_t*, const int64_t*, float*, int64_t, int64_t, hipStream_t);
using MsgEdge = int (*)(const ictc_tp_desc&, const float*, const float*, const float*, const float*,
                        const int64_t*, const int64_t*, const int64_t*, float*, float*, float*, int64_t,
                        int64_t, hipStream_t, int);
using MsgNode = int (*)(int, const float*, const int64_t*, const int64_t*, float*, int64_t, hipStream_t);
using MsgFwdT = int (*)(const ictc_tp_desc&, const float*, const float*, const float*, const MsgTangent&,
                        const int64_t*, const int64_t*, const int64_t*, float*, int64_t, int64_t, hipStream_t);
using MsgEdgeT = int (*)(const ictc_tp_desc&, const float*, const float*, const float*, const MsgTangent&,
                         const float*, const int64_t*, const int64_t*, const int64_t*, float*, float*, float*,
                         int64_t, int64_t, hipStream_t);

#define ICTC_DECLARE(A, B, C) [A * 16 + B * 4 + C] = &launch_msg_bonds<A, B, C>,
const MsgBonds kMsgBonds[64] = {
#include "generated/tp_instances.def"
};
#undef ICTC_DECLARE
#define ICTC_DECLARE(A, B, C) [A * 16 + B * 4 + C] = &launch_msg_forward<A, B, C>,
const MsgFwd kMsgFwd[64] = {
#include "generated/tp_instances.def"
};
#undef ICTC_DECLARE
#define ICTC_DECLARE(A, B, C) [A * 16 + B * 4 + C] = &launch_msg_edge_grad<A, B, C>,
const MsgEdge kMsgEdge[64] = {
#include "generated/tp_instances.def"
};
#undef ICTC_DECLARE
#define ICTC_DECLARE(A, B, C) [A * 16 + B * 4 + C] = &launch_msg_forward_tangent<A, B, C>,
const MsgFwdT kMsgFwdT[64] = {
#include "generated/tp_instances.def"
};
#undef ICTC_DECLARE
#define ICTC_DECLARE(A, B, C) [A * 16 + B * 4 + C] = &launch_msg_edge_grad_tangent<A, B, C>,
const MsgEdgeT kMsgEdgeT[64] = {
#include "generated/tp_instances.def"
};
#undef ICTC_DECLARE
const MsgNode kMsgNode[kGenericMaxL + 1] = {&launch_msg_node_grad<0>, &launch_msg_node_grad<1>,
                                            &launch_msg_node_grad<2>, &launch_msg_node_grad<3>,
                                            &launch_msg_node_grad<4>, &launch_msg_node_grad<5>,
                                            &launch_msg_node_grad<6>};

int tp_check_desc(const ictc_tp_desc* d);  // tp_api.hip

// Node tensors are gathered through 32-bit buffer offsets.
inline bool fits_u32(int64_t rows, int64_t width_floats) {
  return rows >= 0 && rows * width_floats * 4 < (int64_t(1) << 32);
}

inline int msg_index(const ictc_tp_desc* d) { return d->input_lmax * 16 + d->edge_lmax * 4 + d->output_lmax; }

// floats per edge of the bond row: sum over the paths of (2 l1 + 1)(2 l3 + 1)
inline int bond_row_floats(const ictc_tp_desc* d) {
  int nb = 0;
  for (int a = 0; a <= d->input_lmax; ++a)
    for (int b = 0; b <= d->edge_lmax; ++b)
      for (int c = 0; c <= d->output_lmax; ++c) {
        const int lo = a > b ? a - b : b - a;
        if (c < lo || c > a + b || ((a + b + c) & 1)) continue;
        nb += (2 * a + 1) * (2 * c + 1);
      }
  return nb;
}

// width of the caller's bond buffer: 0 when the kernels build the rows from the harmonics
inline int bond_width(const ictc_tp_desc* d) {
  if (generic_degrees(*d)) return 0;
  const int nb = bond_row_floats(d), ny = (d->edge_lmax + 1) * (d->edge_lmax + 1);
  return bond_inline(nb, ny) ? 0 : nb;
}

inline int msg_common(const ictc_tp_desc* d, int64_t nodes_src, int64_t nodes_dst, int64_t edges) {
  const int st = tp_check_desc(d);
  if (st != ICTC_OK) return st;
  if (nodes_src < 0 || nodes_dst < 0 || edges < 0) return ICTC_ERR_INVALID_ARGUMENT;
  const int nx = (d->input_lmax + 1) * (d->input_lmax + 1);
  if (!fits_u32(nodes_src, static_cast<int64_t>(nx) * d->channels) ||
      !fits_u32(nodes_dst, static_cast<int64_t>(d->out_components) * d->channels))
    return ICTC_ERR_UNSUPPORTED;
  return ICTC_OK;
}

}  // namespace ictc

// Staging for ictc_hip_message_edge_grad_static: the per-chunk harmonics partials
// [edges, chunks, NY] of wide channel counts.  One array per device, held until the process
// ends.  Host code never passes this name to a kernel or a copy (on the host it is only a
// stand-in for the device symbol): its device address is fetched once per device with
// hipGetSymbolAddress, with that device current, and only that address is used.
static __device__ __align__(256) float scratch[ICTC_MSG_STATIC_SCRATCH_FLOATS];

namespace ictc {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_lock;
float* g_scratch_address[kMaxDevices] = {};

// Device address of `scratch` on the device that owns `stream` (the current device: a stream
// of another device is rejected).
int static_scratch(hipStream_t stream, float** address) {
  int device = -1;
  if (hipGetDevice(&device) != hipSuccess) return ICTC_ERR_LAUNCH;
  if (device < 0 || device >= kMaxDevices) return ICTC_ERR_UNSUPPORTED;
  if (stream != nullptr) {
    hipDevice_t owner = -1;
    if (hipStreamGetDevice(stream, &owner) != hipSuccess) return ICTC_ERR_LAUNCH;
    if (owner != device) return ICTC_ERR_INVALID_ARGUMENT;
  }
  std::lock_guard<std::mutex> guard(g_scratch_lock);
  if (g_scratch_address[device] == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return ICTC_ERR_LAUNCH;
    g_scratch_address[device] = static_cast<float*>(p);
  }
  *address = g_scratch_address[device];
  return ICTC_OK;
}

// out[e, j] = sum_q partial[e, q, j] (q ascending), one thread per (e, j).
__global__ void __launch_bounds__(256)
chunk_sum_kernel(const float* __restrict__ partial, float* __restrict__ out, int64_t total, int chunks,
                 int width) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const int64_t e = i / width;
  const int64_t j = i - e * width;
  const float* p = partial + e * chunks * width + j;
  float s = p[0];
  for (int q = 1; q < chunks; ++q) s += p[static_cast<int64_t>(q) * width];
  out[i] = s;
}

}  // namespace
}  // namespace ictc

extern "C" {

int ictc_hip_message_chunks(int channels) { return channels < 1 ? -1 : (channels + 63) / 64; }

int ictc_hip_message_bond_width(const ictc_tp_desc* desc) {
  if (ictc::tp_check_desc(desc) != ICTC_OK) return -1;
  return ictc::bond_width(desc);
}

int ictc_hip_message_bonds(const ictc_tp_desc* desc, const float* harmonics, float* bonds, int64_t edges,
                           hipStream_t stream) {
  const int st = ictc::tp_check_desc(desc);
  if (st != ICTC_OK) return st;
  if (edges < 0) return ICTC_ERR_INVALID_ARGUMENT;
  if (edges == 0 || ictc::bond_width(desc) == 0) return ICTC_OK;   // width 0: rows built in-kernel
  if (!harmonics || !bonds) return ICTC_ERR_INVALID_ARGUMENT;
  const ictc::MsgBonds fn = ictc::kMsgBonds[ictc::msg_index(desc)];
  if (fn == nullptr) return ICTC_ERR_UNSUPPORTED;
  return fn(*desc, harmonics, bonds, edges, stream);
}

int ictc_hip_message_forward(const ictc_tp_desc* desc, const float* node_features, const float* bonds,
                             const float* gates, const int64_t* src, const int64_t* dst_rowptr,
                             const int64_t* dst_perm, float* node_out, int64_t nodes_src, int64_t nodes_dst,
                             int64_t edges, hipStream_t stream) {
  const int st = ictc::msg_common(desc, nodes_src, nodes_dst, edges);
  if (st != ICTC_OK) return st;
  if (nodes_dst == 0) return ICTC_OK;
  if (!node_out || !dst_rowptr || (edges > 0 && (!node_features || !bonds || !gates || !src)))
    return ICTC_ERR_INVALID_ARGUMENT;
  if (ictc::generic_degrees(*desc))
    return ictc::generic_msg_forward(*desc, node_features, bonds, gates, src, dst_rowptr, dst_perm, node_out,
                                     nodes_src, nodes_dst, stream);
  const ictc::MsgFwd fn = ictc::kMsgFwd[ictc::msg_index(desc)];
  if (fn == nullptr) return ICTC_ERR_UNSUPPORTED;
  return fn(*desc, node_features, bonds, gates, src, dst_rowptr, dst_perm, node_out, nodes_src, nodes_dst,
            stream);
}

int ictc_hip_message_edge_grad(const ictc_tp_desc* desc, const float* node_features, const float* harmonics,
                               const float* gates, const float* grad_out, const int64_t* src,
                               const int64_t* dst_rowptr, const int64_t* dst_perm,
                               float* grad_harmonics_partial, float* grad_gates, float* edge_grad_features,
                               int64_t nodes_src, int64_t nodes_dst, int64_t edges, int accumulate_gates,
                               hipStream_t stream) {
  const int st = ictc::msg_common(desc, nodes_src, nodes_dst, edges);
  if (st != ICTC_OK) return st;
  if (accumulate_gates != 0 && accumulate_gates != 1) return ICTC_ERR_INVALID_ARGUMENT;
  if (edges == 0 || nodes_dst == 0 || (!grad_harmonics_partial && !grad_gates && !edge_grad_features))
    return ICTC_OK;
  if (!harmonics || !gates || !grad_out || !src || !dst_rowptr) return ICTC_ERR_INVALID_ARGUMENT;
  if ((grad_harmonics_partial || grad_gates) && !node_features) return ICTC_ERR_INVALID_ARGUMENT;
  if (ictc::generic_degrees(*desc)) {
    if (accumulate_gates && grad_gates) return ICTC_ERR_UNSUPPORTED;
    return ictc::generic_msg_edge_grad(*desc, node_features, harmonics, gates, grad_out, src, dst_rowptr, dst_perm,
                                       grad_harmonics_partial, grad_gates, edge_grad_features, nodes_src,
                                       nodes_dst, stream);
  }
  const ictc::MsgEdge fn = ictc::kMsgEdge[ictc::msg_index(desc)];
  if (fn == nullptr) return ICTC_ERR_UNSUPPORTED;
  return fn(*desc, node_features, harmonics, gates, grad_out, src, dst_rowptr, dst_perm, grad_harmonics_partial,
            grad_gates, edge_grad_features, nodes_src, nodes_dst, stream, accumulate_gates);
}

int ictc_hip_message_static_prepare(void) {
  float* address = nullptr;
  return ictc::static_scratch(nullptr, &address);
}

int ictc_hip_message_edge_grad_static(const ictc_tp_desc* desc, const float* node_features, const float* harmonics,
                                      const float* gates, const float* grad_out, const int64_t* src,
                                      const int64_t* dst_rowptr, const int64_t* dst_perm, float* grad_harmonics,
                                      float* grad_gates, float* edge_grad_features, int64_t nodes_src,
                                      int64_t nodes_dst, int64_t edges, hipStream_t stream) {
  const int st = ictc::msg_common(desc, nodes_src, nodes_dst, edges);
  if (st != ICTC_OK) return st;
  if (edges == 0 || nodes_dst == 0 || (!grad_harmonics && !grad_gates && !edge_grad_features)) return ICTC_OK;
  if (!harmonics || !gates || !grad_out || !src || !dst_rowptr) return ICTC_ERR_INVALID_ARGUMENT;
  if ((grad_harmonics || grad_gates) && !node_features) return ICTC_ERR_INVALID_ARGUMENT;
  const bool generic = ictc::generic_degrees(*desc);
  const ictc::MsgEdge fn = generic ? nullptr : ictc::kMsgEdge[ictc::msg_index(desc)];
  if (!generic && fn == nullptr) return ICTC_ERR_UNSUPPORTED;
  const int chunks = ictc_hip_message_chunks(desc->channels);
  const int ny = (desc->edge_lmax + 1) * (desc->edge_lmax + 1);
  float* partial = grad_harmonics;   // one chunk: the kernel writes the sums itself
  if (grad_harmonics != nullptr && chunks > 1) {
    if (edges > ICTC_MSG_STATIC_SCRATCH_FLOATS / (static_cast<int64_t>(chunks) * ny)) return ICTC_ERR_CAPACITY;
    const int sst = ictc::static_scratch(stream, &partial);
    if (sst != ICTC_OK) return sst;
  }
  const int r = generic ? ictc::generic_msg_edge_grad(*desc, node_features, harmonics, gates, grad_out, src, dst_rowptr,
                                                      dst_perm, partial, grad_gates, edge_grad_features, nodes_src,
                                                      nodes_dst, stream)
                        : fn(*desc, node_features, harmonics, gates, grad_out, src, dst_rowptr, dst_perm, partial,
                             grad_gates, edge_grad_features, nodes_src, nodes_dst, stream, 0);
  if (r != ICTC_OK || partial == grad_harmonics) return r;
  const int64_t total = edges * ny;
  hipLaunchKernelGGL(ictc::chunk_sum_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                     stream, partial, grad_harmonics, total, chunks, ny);
  return hipGetLastError() == hipSuccess ? ICTC_OK : ICTC_ERR_LAUNCH;
}

int ictc_hip_message_forward_tangent(const ictc_tp_desc* desc, const float* node_features, const float* bonds,
                                     const float* gates, const float* tangent_features, const float* tangent_bonds,
                                     const float* tangent_gates, const int64_t* src, const int64_t* dst_rowptr,
                                     const int64_t* dst_perm, float* node_out, int64_t nodes_src,
                                     int64_t nodes_dst, int64_t edges, hipStream_t stream) {
  const int st = ictc::msg_common(desc, nodes_src, nodes_dst, edges);
  if (st != ICTC_OK) return st;
  if (nodes_dst == 0) return ICTC_OK;
  if (!node_out || !dst_rowptr ||
      (edges > 0 && (!node_features || !bonds || !gates || !tangent_features || !tangent_bonds ||
                     !tangent_gates || !src)))
    return ICTC_ERR_INVALID_ARGUMENT;
  if (ictc::generic_degrees(*desc)) return ICTC_ERR_UNSUPPORTED;
  const ictc::MsgFwdT fn = ictc::kMsgFwdT[ictc::msg_index(desc)];
  if (fn == nullptr) return ICTC_ERR_UNSUPPORTED;
  const ictc::MsgTangent t{tangent_features, tangent_bonds, tangent_gates};
  return fn(*desc, node_features, bonds, gates, t, src, dst_rowptr, dst_perm, node_out, nodes_src, nodes_dst,
            stream);
}

int ictc_hip_message_edge_grad_tangent(const ictc_tp_desc* desc, const float* node_features, const float* harmonics,
                                       const float* gates, const float* tangent_features,
                                       const float* tangent_harmonics, const float* tangent_gates,
                                       const float* grad_out, const int64_t* src, const int64_t* dst_rowptr,
                                       const int64_t* dst_perm, float* grad_harmonics_partial, float* grad_gates,
                                       float* edge_grad_features, int64_t nodes_src, int64_t nodes_dst,
                                       int64_t edges, hipStream_t stream) {
  const int st = ictc::msg_common(desc, nodes_src, nodes_dst, edges);
  if (st != ICTC_OK) return st;
  if (edges == 0 || nodes_dst == 0 || (!grad_harmonics_partial && !grad_gates && !edge_grad_features))
    return ICTC_OK;
  if (!node_features || !harmonics || !gates || !tangent_features || !tangent_harmonics || !tangent_gates || !grad_out ||
      !src || !dst_rowptr)
    return ICTC_ERR_INVALID_ARGUMENT;
  if (ictc::generic_degrees(*desc)) return ICTC_ERR_UNSUPPORTED;
  const ictc::MsgEdgeT fn = ictc::kMsgEdgeT[ictc::msg_index(desc)];
  if (fn == nullptr) return ICTC_ERR_UNSUPPORTED;
  const ictc::MsgTangent t{tangent_features, nullptr, tangent_gates, tangent_harmonics};
  return fn(*desc, node_features, harmonics, gates, t, grad_out, src, dst_rowptr, dst_perm, grad_harmonics_partial,
            grad_gates, edge_grad_features, nodes_src, nodes_dst, stream);
}

int ictc_hip_message_node_grad(const ictc_tp_desc* desc, const float* edge_grad_features,
                               const int64_t* src_rowptr, const int64_t* src_perm, float* grad_features,
                               int64_t nodes_src, int64_t edges, hipStream_t stream) {
  const int st = ictc::msg_common(desc, nodes_src, 0, edges);
  if (st != ICTC_OK) return st;
  if (nodes_src == 0) return ICTC_OK;
  if (!grad_features || !src_rowptr || (edges > 0 && !edge_grad_features)) return ICTC_ERR_INVALID_ARGUMENT;
  return ictc::kMsgNode[desc->input_lmax](desc->channels, edge_grad_features, src_rowptr, src_perm,
                                          grad_features, nodes_src, stream);
}

}  // extern "C"
