// Degree-generic tensor-product and graph-message kernels (generic_kernels.hip): the path
// table, bond layout and CG tensors are read at run time, so one kernel serves every degree
// set up to kGenericMaxL, including those above the per-degree instantiations (<= 3).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "ictc_hip.h"

namespace ictc {

constexpr int kCompiledMaxL = 3;   // per-degree instantiations: every degree <= 3
constexpr int kGenericMaxL = 6;    // run-time path tables: every degree <= 6

// True when a degree of the descriptor exceeds the per-degree instantiations.
inline bool generic_degrees(const ictc_tp_desc& d) {
  return d.input_lmax > kCompiledMaxL || d.edge_lmax > kCompiledMaxL || d.output_lmax > kCompiledMaxL;
}

// out[r] = TP(x[r], y[r], g[r]) (the tp_forward_kernel contract).
int generic_tp_forward(const ictc_tp_desc& d, const float* x, const float* y, const float* g, float* out,
                       int64_t rows, hipStream_t stream);

// (dx, dy, dg) of the TP for dout go; null outputs are skipped, x may be null when only dx is
// asked for (the tp_backward_kernel contract).
int generic_tp_backward(const ictc_tp_desc& d, const float* x, const float* y, const float* g, const float* go,
                        float* dx, float* dy, float* dg, int64_t rows, hipStream_t stream);

// node_out[n] = sum over the receiver-CSR edges e of n of TP(x[src e], y[e], g[e]), every row of
// node_out written (zero for a node without edges).  y are the harmonics: these kernels build
// the bond rows themselves (bond width 0).  A source index outside [0, nodes_src) reads zeros.
int generic_msg_forward(const ictc_tp_desc& d, const float* x, const float* y, const float* g, const int64_t* src,
                        const int64_t* rowptr, const int64_t* perm, float* out, int64_t nodes_src,
                        int64_t nodes_dst, hipStream_t stream);

// Per edge e (receiver n): dg[e], the feature adjoint dxe[e] and the harmonics gradient of e,
// written as chunk 0 of dyp[e] (dyp [E, chunks, NY]; the other chunks are written zero).
int generic_msg_edge_grad(const ictc_tp_desc& d, const float* x, const float* y, const float* g, const float* go,
                          const int64_t* src, const int64_t* rowptr, const int64_t* perm, float* dyp, float* dg,
                          float* dxe, int64_t nodes_src, int64_t nodes_dst, hipStream_t stream);

}  // namespace ictc
