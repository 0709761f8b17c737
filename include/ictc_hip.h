/*
 * ictc_hip.h -- C ABI of the MI355X (gfx950) ictc_o3 equivariant operator library.
 *
 * libictc_hip.so exports plain extern "C" entry points taking device pointers,
 * sizes and a hipStream_t.  Nothing here allocates device memory (the caller owns
 * every input, output and workspace buffer), with two exceptions: ictc_hip_sgemm's
 * rocBLAS handles (one per host thread and device) allocate their own workspace, and
 * ictc_hip_message_edge_grad_static stages partial sums in a library-owned static
 * device array (16 MiB per GPU, held for the life of the process) that every call on
 * that GPU shares, so overlapping calls on one GPU must be serialised.  Launches are
 * asynchronous on the given stream; every other entry point is reentrant, and the only
 * mutable global state is those rocBLAS handles and the static array's per-device address.
 *
 * Data layout (all float32, row-major, channel-contiguous "ir_mul" packing):
 *   features   [rows, C*(L_in+1)^2]     per degree l: (2l+1) rows of C channels
 *   harmonics  [rows, (L_edge+1)^2]     Y_0 | Y_1 | ... (ICTC basis)
 *   gates      [rows, P*C]              per path p (owner order): C channels
 *   output     [rows, C*NOC]            per output degree l, per path with l3=l
 *                                       (owner order), (2l+1) rows of C channels
 * where P = number of paths and NOC = sum_p (2 l3_p + 1).
 *
 * Return value: ICTC_OK (0) or an ictc_status code; ictc_hip_status_string()
 * names it.  Invalid arguments are rejected before any launch.
 */
#ifndef ICTC_HIP_H
#define ICTC_HIP_H

#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ICTC_MAX_PATHS 128   /* the full (6,6,6) path set has 106 paths */

typedef enum ictc_status {
    ICTC_OK = 0,
    ICTC_ERR_INVALID_ARGUMENT = 1,   /* null pointer, negative size, bad descriptor */
    ICTC_ERR_UNSUPPORTED = 2,        /* degree combination or mode not supported */
    ICTC_ERR_LAUNCH = 3,             /* hipLaunchKernel / hipGetLastError failed */
    ICTC_ERR_INDEX = 4,              /* graph or species index out of range (checked kernels) */
    ICTC_ERR_CAPACITY = 5            /* input exceeds a static scratch array (nothing launched) */
} ictc_status;

/*
 * Path-preserving channelwise tensor-product descriptor.
 *
 * The kernels are compiled for the full triangle/parity path set of
 * (input_lmax, edge_lmax, output_lmax) in ascending (l1,l2,l3) order -- the
 * order of reference ictc_o3/operators.py:54-55 and ictd_irreps.py:2161-2175 --
 * with its canonical layout, and the descriptor must state exactly that:
 *   num_paths      = ictc_hip_tp_slot_count(...), out_components = sum (2 l3 + 1);
 *   gate_index[s]  = s (gates row block of slot s);
 *   out_offset[s]  first output component of slot s: ascending l3, enumeration order
 *                  within one l3 (the owner's path_offset, reference
 *                  ictd_irreps.py:2514-2526 and operators.py:107-115);
 *   scale[s]       per-path normalisation, e.g. 'element' 1/sqrt(#paths with this l3)
 *                  (reference ictd_irreps.py:101-133).  The CG tensors compiled into
 *                  the library carry the 'component' normalisation (ictd_irreps.py:136-142).
 * An owner with a path subset runs the full set with zero gates on the absent paths
 * and keeps its own output rows.
 *
 * Degrees: every degree <= 6.  Degree sets with all degrees <= 3 run kernels compiled per
 * degree set (path loops unrolled, CG constants folded), and so do ictc_hip_tp_forward and
 * ictc_hip_tp_backward for the (4, 4, 4) set; the others run degree-generic
 * kernels that read the path table and the CG tensors at run time (one wave per instance),
 * behind every tensor-product and graph-message entry point except the two message tangent
 * entry points, which return ICTC_ERR_UNSUPPORTED for such degree sets.
 */
typedef struct ictc_tp_desc {
    int32_t channels;          /* C >= 1 */
    int32_t input_lmax;        /* 0..6 */
    int32_t edge_lmax;         /* 0..6 */
    int32_t output_lmax;       /* 0..6 */
    int32_t num_paths;         /* P: number of owner paths (gate blocks) */
    int32_t out_components;    /* NOC */
    int32_t gate_index[ICTC_MAX_PATHS];
    int32_t out_offset[ICTC_MAX_PATHS];
    float scale[ICTC_MAX_PATHS];
} ictc_tp_desc;

/* Human-readable name of a status code (static string). */
const char* ictc_hip_status_string(int status);

/* Library ABI version, bumped on any signature or layout change. */
int ictc_hip_abi_version(void);

/* Number of slots (full path-set size) the kernels enumerate for these degrees. */
int ictc_hip_tp_slot_count(int input_lmax, int edge_lmax, int output_lmax);

/*
 * TP forward:  out[e, path p, k, c] = gates[e,p,c] * sum_i x[e,l1,i,c] * M_p[e,i,k],
 *              M_p[e,i,k] = scale_p * sum_j Y[e,l2,j] * Chat_p[i,j,k].
 * Replaces the packed standalone TP of reference
 * ictc_o3/backends/ascend/packed_tensor_product.py:60-80 (_Product.forward), whose
 * CPU definition is EdgeWeightedPathPreservingTensorProduct._forward_index_add
 * (ictc_o3/basis/ictd_irreps.py:2669-2748).  rows may be 0 (no launch).
 */
int ictc_hip_tp_forward(const ictc_tp_desc* desc,
                        const float* features, const float* harmonics, const float* gates,
                        float* out, int64_t rows, hipStream_t stream);

/*
 * TP vector-Jacobian product.  Given grad_out (same layout as out) writes
 *   grad_features  [rows, C*(L_in+1)^2]   (if non-null)
 *   grad_harmonics [rows, (L_edge+1)^2]   (if non-null)
 *   grad_gates     [rows, P*C]            (if non-null)
 * each fully overwritten (not accumulated).  Replaces
 * packed_tensor_product.py:82-110 (_Product.backward) and the structured adjoints
 * _left_grad/_right_grad/_weight_grad (structured_product.py:49-87), with the
 * bond projection Y -> M folded in (structured_product.py:7-22).  Because the map
 * is trilinear in (features, harmonics, gates), every mixed second derivative is
 * this entry point or ictc_hip_tp_forward with one operand substituted
 * (structured_product.py:146-158).
 */
int ictc_hip_tp_backward(const ictc_tp_desc* desc,
                         const float* features, const float* harmonics, const float* gates,
                         const float* grad_out,
                         float* grad_features, float* grad_harmonics, float* grad_gates,
                         int64_t rows, hipStream_t stream);

/*
 * Graph message:  node_out[n] = sum_{e : dst(e) = n} TP(features[src(e)], harmonics[e], gates[e])
 * with the TP above (same descriptor; node rows use the features / output layouts).
 *
 * The harmonics enter through per-edge bond matrices, computed once per edge by
 * ictc_hip_message_bonds into a caller-owned buffer [edges, ictc_hip_message_bond_width]:
 *   bonds[e][bond_p + k*(2 l1 + 1) + i] = scale_p * sum_j harmonics[e][l2^2 + j] C_p[i, j, k]
 * (the reference's bond projection Y @ P: backends/ascend/tensor_product.py:9-57,
 * structured_product.py:7-22).  The buffer serves the forward and its tangent; the VJP entry
 * points take the harmonics themselves (they contract grad_out with the CG tensors once per
 * receiver instead).  For small degree sets (at most 32 projection coefficients per lane,
 * e.g. lmax 2 or an input lmax of 0) and for every degree set with a degree above 3 the
 * kernels form the bond rows from the harmonics themselves:
 * ictc_hip_message_bond_width then returns 0, ictc_hip_message_bonds does nothing, and the
 * caller passes the harmonics [edges, (L_e+1)^2] as the `bonds` argument.
 *
 * Edges are visited through a CSR over the receivers: dst_rowptr [nodes_dst+1] and
 * dst_perm [edges] (CSR slot -> edge id; null when edges are already sorted by dst).
 * Each destination node is accumulated in registers by one wave per 64-channel chunk,
 * so per-edge messages never reach HBM and the sum order is deterministic (no atomics).
 * node_out [nodes_dst, NOC*C] is fully overwritten (zeros for nodes without edges).
 * Indices must lie in [0, nodes_src) / [0, nodes_dst); gathers are range checked by the
 * hardware (out-of-range reads return zeros).  Node tensors must be < 4 GiB.
 * Replaces graph_message (reference ictc_o3/backends/ascend/tensor_product.py:159-218),
 * channel_message.graph_message (channel_message.py:35-216) and the atomic ictc_epilogue
 * (ascendc/op_kernel/epilogue.cpp:6-212, ascendc/epilogue.py:132-150).
 */
int ictc_hip_message_bond_width(const ictc_tp_desc* desc);

int ictc_hip_message_bonds(const ictc_tp_desc* desc, const float* harmonics, float* bonds,
                           int64_t edges, hipStream_t stream);

int ictc_hip_message_forward(const ictc_tp_desc* desc, const float* node_features,
                             const float* bonds, const float* gates, const int64_t* src,
                             const int64_t* dst_rowptr, const int64_t* dst_perm, float* node_out,
                             int64_t nodes_src, int64_t nodes_dst, int64_t edges,
                             hipStream_t stream);

/* Number of 64-channel chunks a message kernel splits the channels into. */
int ictc_hip_message_chunks(int channels);

/*
 * Message VJP, per-edge part (receiver CSR, grad_out[n] read once per node), from the
 * harmonics [edges, (L_e+1)^2] (not the bond rows): for every edge
 *   grad_gates[e]               = d<grad_out, node_out>/d gates[e]            [edges, P*C]
 *   grad_harmonics_partial[e,q] = partial sums over the channels of the harmonics
 *                                 gradient of edge e              [edges, chunks, NY];
 *                                 their sum over q (which the caller forms) is the
 *                                 gradient.  Which channels a slot holds depends on
 *                                 the kernel schedule (64-channel chunk q for the
 *                                 degrees up to 3); it is fixed per degree set.
 *   edge_grad_features[e]       = sum_p gates[e,p] M_p[e]^T grad_out[dst(e)], the edge's
 *                                 contribution to the source-feature gradient
 *                                 [edges, C*(L_in+1)^2] (features layout)
 * Any output may be null; node_features may be null when only edge_grad_features is
 * requested.  accumulate_gates = 1 adds the gate gradients into grad_gates (which then holds
 * a gradient already, e.g. the other contribution to the same gates in a force-loss double
 * backward) instead of overwriting it; 0 overwrites.  Degree sets with a degree above 3
 * return ICTC_ERR_UNSUPPORTED for accumulate_gates = 1.  Replaces the dr/dg terms of
 * ictc_epilogue_adjoint (ascendc/op_kernel/epilogue_adjoint.cpp:6-208).
 */
int ictc_hip_message_edge_grad(const ictc_tp_desc* desc, const float* node_features,
                               const float* harmonics, const float* gates, const float* grad_out,
                               const int64_t* src, const int64_t* dst_rowptr,
                               const int64_t* dst_perm, float* grad_harmonics_partial,
                               float* grad_gates, float* edge_grad_features, int64_t nodes_src,
                               int64_t nodes_dst, int64_t edges, int accumulate_gates,
                               hipStream_t stream);

/*
 * No counterpart in the reference: for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * ictc_hip_message_edge_grad with the harmonics gradient already summed over the channel
 * chunks: grad_harmonics [edges, (L_e+1)^2] = sum_q grad_harmonics_partial[e, q, :], so no
 * partial buffer is needed; grad_gates and edge_grad_features are as above (bit-identical).
 * With more than one 64-channel chunk the partials are staged in a library-owned device array
 * of ICTC_MSG_STATIC_SCRATCH_FLOATS floats (16 MiB on each GPU the library runs on, held until
 * the process ends); edges * chunks * (L_e+1)^2 above that size returns ICTC_ERR_CAPACITY
 * before any launch.  Every row the call reads from the array it first writes (a receiver CSR
 * that covers every edge once, as for the entry point above).  The stream must belong to the
 * current device.  Allocates nothing.  Calls that overlap on one GPU (concurrent streams or
 * host threads) share the array and race: serialise them.  The array's device address is
 * looked up (hipGetSymbolAddress) on the first call on each device, or earlier by
 * ictc_hip_message_static_prepare: call that once per device, with the device current, before
 * capturing a HIP graph that contains this entry point, so that the capture records launches
 * only.
 */
#define ICTC_MSG_STATIC_SCRATCH_FLOATS 4194304
int ictc_hip_message_static_prepare(void);
int ictc_hip_message_edge_grad_static(const ictc_tp_desc* desc, const float* node_features,
                                      const float* harmonics, const float* gates, const float* grad_out,
                                      const int64_t* src, const int64_t* dst_rowptr,
                                      const int64_t* dst_perm, float* grad_harmonics,
                                      float* grad_gates, float* edge_grad_features,
                                      int64_t nodes_src, int64_t nodes_dst, int64_t edges,
                                      hipStream_t stream);

/*
 * Mixed second derivatives of the message, as directional derivatives (JVPs) in the
 * direction (tangent_features [nodes_src, C*(L_in+1)^2], tangent harmonics, tangent_gates
 * [edges, P*C]).  ictc_hip_message_forward_tangent takes bond rows (bonds, and tangent_bonds
 * from ictc_hip_message_bonds on the tangent harmonics, or the harmonics themselves when the
 * bond width is 0); ictc_hip_message_edge_grad_tangent takes the harmonics and the tangent
 * harmonics [edges, (L_e+1)^2], as ictc_hip_message_edge_grad does.
 *   ictc_hip_message_forward_tangent: node_out = d/de message(x + e tx, Y + e tY, g + e tg)
 *     = sum over each argument replaced by its tangent, the others kept;
 *   ictc_hip_message_edge_grad_tangent: the same derivative of each edge_grad output with
 *     grad_out fixed: grad_gates from (tx, Y) + (x, tY), grad_harmonics_partial from
 *     (tx, g) + (x, tg), edge_grad_features from (tY, g) + (Y, tg).
 * The double backward of the message is these two calls plus one node_grad, instead of one
 * forward and one VJP per tangent argument.  All tangent arguments are required.  Replaces
 * the bilinear substitution of reference backends/ascend/structured_product.py:146-158 and
 * the mixed-second adjoint mode of ascendc/op_kernel/epilogue_adjoint.cpp:6-208.
 */
int ictc_hip_message_forward_tangent(const ictc_tp_desc* desc, const float* node_features,
                                     const float* bonds, const float* gates,
                                     const float* tangent_features, const float* tangent_bonds,
                                     const float* tangent_gates, const int64_t* src,
                                     const int64_t* dst_rowptr, const int64_t* dst_perm,
                                     float* node_out, int64_t nodes_src, int64_t nodes_dst,
                                     int64_t edges, hipStream_t stream);

int ictc_hip_message_edge_grad_tangent(const ictc_tp_desc* desc, const float* node_features,
                                       const float* harmonics, const float* gates,
                                       const float* tangent_features, const float* tangent_harmonics,
                                       const float* tangent_gates, const float* grad_out,
                                       const int64_t* src, const int64_t* dst_rowptr,
                                       const int64_t* dst_perm, float* grad_harmonics_partial,
                                       float* grad_gates, float* edge_grad_features,
                                       int64_t nodes_src, int64_t nodes_dst, int64_t edges,
                                       hipStream_t stream);

/*
 * Message VJP, per-source-node part (source CSR: src_rowptr [nodes_src+1], src_perm
 * [edges] or null): grad_features[s] = sum over edges with src(e) = s of
 * edge_grad_features[e]  [nodes_src, C*(L_in+1)^2], fully overwritten; a deterministic
 * segmented sum.  Replaces the mode-1 scatter of ictc_weighted_map
 * (ascendc/op_kernel/weighted_map.cpp:225-233) without atomics.
 */
int ictc_hip_message_node_grad(const ictc_tp_desc* desc, const float* edge_grad_features,
                               const int64_t* src_rowptr, const int64_t* src_perm,
                               float* grad_features, int64_t nodes_src, int64_t edges,
                               hipStream_t stream);

/*
 * Symmetric contraction (correlation <= 3) with species-selected weights:
 *   out[n, c, l_out, m] = sum_p W[species[n], p, c] * chain_p(x[n, c, :])_m
 * for every target degree l_out <= target_lmax, where the columns p are the coupling
 * chains of the pure-ICTC U tensors (reference ictc_o3/basis/ictd_irreps.py:1387-1517,
 * ICTDPureUSymmetricContractionSO3 at mace_ictc/models/pure_cartesian_ictd_fix.py:1310)
 * and the polynomial is the MACE recursion of _forward_selected_elements
 * (ictc_o3/ops/_mace_symmetric_contraction.py:298-346).  Replaces the factorised NPU
 * schedule (backends/ascend/contraction.py:8-45, ops/factorized_contraction.py:51-149)
 * and the banked ictc_weighted_map (ascendc/op_kernel/weighted_map.cpp:9-276).
 * Layouts: node_features [nodes, C*(lmax+1)^2] with degree blocks [C, 2l+1] (mul_ir);
 * out [nodes, C*(target_lmax+1)^2] likewise; weights [num_elements, KTOT, C] with KTOT =
 * ictc_hip_sc_weight_columns(...), columns per target degree in the order
 * [order correlation, correlation-1, ..., 1] (weights_max, weights[0], ...).
 * species [nodes] int64 in [0, num_elements) (validated by the caller; the kernels
 * clamp out-of-range values to 0 to stay in bounds).  lmax <= 3.
 */
int ictc_hip_sc_weight_columns(int lmax, int target_lmax, int correlation);

int ictc_hip_sc_forward(int lmax, int target_lmax, int correlation, int channels,
                        const float* node_features, const int64_t* species, const float* weights,
                        int num_elements, float* out, int64_t nodes, hipStream_t stream);

/* VJP to the node features: grad_features [nodes, C*(lmax+1)^2] (mul_ir, overwritten). */
int ictc_hip_sc_backward(int lmax, int target_lmax, int correlation, int channels,
                         const float* node_features, const int64_t* species, const float* weights,
                         int num_elements, const float* grad_out, float* grad_features,
                         int64_t nodes, hipStream_t stream);

/*
 * Weight adjoint per node: features_out[n, p, c] = <grad_out[n, c, :], chain_p(x[n, c, :])>
 * [nodes, KTOT, C] (overwritten); the weight gradient is its sum over the nodes of each
 * species (the gradient of the index_select in _forward_selected_elements,
 * _mace_symmetric_contraction.py:316-317).
 */
int ictc_hip_sc_weight_features(int lmax, int target_lmax, int correlation, int channels,
                                const float* node_features, const int64_t* species,
                                int num_elements, const float* grad_out, float* features_out,
                                int64_t nodes, hipStream_t stream);

/*
 * Second-order pieces of the contraction (the double backward used by force
 * training), each a directional derivative along tangent [nodes, C*(lmax+1)^2]
 * (mul_ir, like node_features).  They replace the recursive autograd through the
 * reference's dense restatement for second derivatives (ictc_o3/sparse_product.py:190-204,
 * 232-250; the reference's create_graph path of _forward_selected_elements).
 *   jvp:                  out[n]  = J(x_n) tangent_n                  [nodes, C*(target+1)^2]
 *   hvp:                  grad_features[n] = d/dx <grad_out_n, J(x_n) tangent_n>
 *                                                                      [nodes, C*(lmax+1)^2]
 *   weight_features_jvp:  features_out[n, p, c] = <grad_out[n,c], d chain_p(x[n,c])[tangent[n,c]]>
 *                                                                      [nodes, KTOT, C]
 * (J = d forward / d node_features at the node's species weights.)  All outputs are
 * overwritten.
 */
int ictc_hip_sc_jvp(int lmax, int target_lmax, int correlation, int channels,
                    const float* node_features, const int64_t* species, const float* weights,
                    int num_elements, const float* tangent, float* out, int64_t nodes,
                    hipStream_t stream);

int ictc_hip_sc_hvp(int lmax, int target_lmax, int correlation, int channels,
                    const float* node_features, const int64_t* species, const float* weights,
                    int num_elements, const float* grad_out, const float* tangent,
                    float* grad_features, int64_t nodes, hipStream_t stream);

int ictc_hip_sc_weight_features_jvp(int lmax, int target_lmax, int correlation, int channels,
                                    const float* node_features, const int64_t* species,
                                    int num_elements, const float* grad_out, const float* tangent,
                                    float* features_out, int64_t nodes, hipStream_t stream);

/*
 * Direction harmonics (ICTC basis, component-normalised) and their analytic
 * derivative contractions, one thread per direction.
 *   directions [rows, 3]; Y has (lmax+1)^2 components Y_0 | Y_1 | ...
 *   ICTC_HARM_VALUE : out[rows,(lmax+1)^2] = Y(n)
 *   ICTC_HARM_VJP   : out[rows,3] = d/dn <u, Y(n)>                   (u: [rows,(lmax+1)^2])
 *   ICTC_HARM_JVP   : out[rows,(lmax+1)^2] = dY(n)[t]                (t: [rows,3])
 *   ICTC_HARM_HVP   : out[rows,3] = d2/dn2 <u, Y(n)> [t]
 *   ICTC_HARM_JVP2  : out[rows,(lmax+1)^2] = d2Y(n)[t, s]            (s: [rows,3])
 *   ICTC_HARM_T3    : out[rows,3] = d3/dn3 <u, Y(n)> [t, s]
 * Replaces direction_harmonics_all (reference ictc_o3/basis/ictd_irreps.py:1113-1168)
 * and the generated kernel with analytic first/second adjoints
 * (ictc_o3/ops/generated_direction_harmonics.py:43-194; ascendc/direction.py:11-62).
 * Unused operand pointers may be null.  lmax <= ICTC_HARM_MAX_LMAX.
 */
#define ICTC_HARM_MAX_LMAX 6
typedef enum ictc_harm_mode {
    ICTC_HARM_VALUE = 0,
    ICTC_HARM_VJP = 1,
    ICTC_HARM_JVP = 2,
    ICTC_HARM_HVP = 3,
    ICTC_HARM_JVP2 = 4,
    ICTC_HARM_T3 = 5
} ictc_harm_mode;

int ictc_hip_direction_harmonics(int lmax, int mode, const float* directions, const float* u,
                                 const float* t, const float* s, float* out, int64_t rows,
                                 hipStream_t stream);

/*
 * Periodic radius graph (cell list).  Replaces the neighbour-list builder of reference
 * mace_ictc/utils/graph_utils.py:217-297 (radius_graph_pbc_gpu, one torch_cluster radius
 * query per lattice image) with an exact search over binned atoms.
 *   grid: lattice (rows of cell[9] are the lattice vectors a, b, c), cutoff^2, bins per
 *         axis, bin offsets searched per axis ("reach", <= 64), periodic flags (0/1);
 *   wrapped_positions [atoms,3] float64: positions wrapped into the cell along periodic
 *         axes (cartesian); atom_bins [atoms,3] int32: each atom's bin coordinates;
 *   bin_start [bins+1] int64 and bin_atoms [atoms] int64: atoms grouped by bin
 *         (bin index (bx * bins[1] + by) * bins[2] + bz).
 * count: counts[j] = number of (i, t) with |w_j - w_i + t @ cell| < cutoff, (i,t) != (j,0).
 * fill:  for receiver j, writes its neighbours at rows rowptr[j] .. rowptr[j+1]-1 (rowptr is
 *        the exclusive scan of counts, rowptr[atoms] = edges): src[e] = i and
 *        images[e,0:3] = t (integer lattice image in wrapped coordinates), in a fixed order.
 * The caller converts t to the shift of the unwrapped positions and orders the rows.
 */
typedef struct ictc_cell_grid {
    double cell[9];
    double cutoff_sq;
    int32_t bins[3];
    int32_t reach[3];
    int32_t periodic[3];
} ictc_cell_grid;

int ictc_hip_radius_graph_count(const ictc_cell_grid* grid, const double* wrapped_positions,
                                const int32_t* atom_bins, const int64_t* bin_start,
                                const int64_t* bin_atoms, int64_t atoms, int64_t* counts,
                                hipStream_t stream);

int ictc_hip_radius_graph_fill(const ictc_cell_grid* grid, const double* wrapped_positions,
                               const int32_t* atom_bins, const int64_t* bin_start,
                               const int64_t* bin_atoms, int64_t atoms, const int64_t* rowptr,
                               int64_t* src, int32_t* images, hipStream_t stream);

/*
 * Sorted fill (also replaces graph_utils.py:217-297, including the caller's edge ordering):
 * for every receiver j whose row holds at most ictc_hip_radius_graph_row_capacity() edges
 * (the caller checks the counts; a longer row is cut to that many), writes rows
 * rowptr[j] .. rowptr[j+1]-1 in (src, shift) order:
 *   src[e] = i, dst[e] = j, shifts[e,0:3] = t - image_base[j] + image_base[i] (float64),
 * where image_base [atoms,3] int64 is each atom's wrap image (position = wrapped position +
 * image_base @ cell) and t the lattice image of the fill entry point above.  The rows then
 * form the (dst, src, shift)-ordered edge list of the reference builder's result, with
 * edge vectors pos[dst] - pos[src] + shift @ cell.
 */
int64_t ictc_hip_radius_graph_row_capacity(void);

int ictc_hip_radius_graph_fill_sorted(const ictc_cell_grid* grid, const double* wrapped_positions,
                                      const int32_t* atom_bins, const int64_t* bin_start,
                                      const int64_t* bin_atoms, int64_t atoms, const int64_t* rowptr,
                                      const int64_t* image_base, int64_t* src, int64_t* dst,
                                      double* shifts, hipStream_t stream);

/*
 * Adjoint of the edge vectors vec[e] = pos[dst(e)] - pos[src(e)] + shift[e] (the edge geometry
 * of reference mace_ictc/models/pure_cartesian_ictd_fix.py:2930-2933, whose autograd scatters
 * through index_add):
 *   grad_pos[n] = sum_{e: dst(e)=n} grad_vec[e] - sum_{e: src(e)=n} grad_vec[e]
 * over the receiver CSR (dst_rowptr [nodes+1], dst_perm [edges] or null when sorted) and the
 * source CSR (src_rowptr, src_perm) of one edge list with nodes_src = nodes_dst = nodes.
 * grad_vec [edges,3], grad_pos [nodes,3] (fully overwritten); dtype 0 = float32, 1 = float64.
 * A fixed summation order (one wave per node, fixed lane assignment and butterfly): the
 * result is bit-identical from run to run.
 */
int ictc_hip_edge_vector_grad(int dtype, const void* grad_vec, const int64_t* dst_rowptr,
                              const int64_t* dst_perm, const int64_t* src_rowptr,
                              const int64_t* src_perm, void* grad_pos, int64_t nodes,
                              hipStream_t stream);

/*
 * Edge embedding of the MACE interaction, one elementwise pass per derivative order.  From the
 * edge vectors v [edges, 3] (r = |v|):
 *   directions n = v / max(r, 1e-8)                                           [edges, 3]
 *   embedding  emb_b = sqrt(2 / r_max) sin(b pi r / r_max) / max(r, 1e-12) u(r / r_max)
 *              (b = 1..num_basis; u the polynomial cutoff envelope of power cutoff_p, zero
 *              from r_max on)                                                  [edges, num_basis]
 * Modes (f = (n, emb)):
 *   ICTC_EMBED_VALUE: out_directions = n, out_embedding = emb
 *   ICTC_EMBED_VJP  : out_directions = d<(grad_directions, grad_embedding), f>/dv   (either
 *                     cotangent may be null: zero)
 *   ICTC_EMBED_JVP  : out_directions = dn[tangent], out_embedding = demb[tangent] (either may be
 *                     null)
 *   ICTC_EMBED_HVP  : out_directions = d/dv <(grad_directions, grad_embedding), df[tangent]>
 * Replaces the edge length / direction of reference mace_ictc/models/pure_cartesian_ictd_fix.py:
 * 2935-2936 and mace_polynomial_cutoff / mace_radial_embedding (Bessel, no sqrt(num_basis)
 * factor) of mace_ictc/models/radial_basis.py:11-92, whose library-op compositions take some
 * twenty passes per derivative order.  num_basis <= ICTC_EMBED_MAX_BASIS, 1 <= cutoff_p <=
 * ICTC_EMBED_MAX_POWER, r_max > 0.
 */
enum ictc_embed_mode { ICTC_EMBED_VALUE = 0, ICTC_EMBED_VJP = 1, ICTC_EMBED_JVP = 2, ICTC_EMBED_HVP = 3 };
#define ICTC_EMBED_MAX_BASIS 64
#define ICTC_EMBED_MAX_POWER 16
int ictc_hip_edge_embedding(int mode, const float* vectors, const float* grad_directions,
                            const float* grad_embedding, const float* tangent, float* out_directions,
                            float* out_embedding, int num_basis, int cutoff_p, float r_max, int64_t edges,
                            hipStream_t stream);

/*
 * Element-conditioned linear map on a scalar block (the MACE interaction's self connection):
 *   ICTC_SPECIES_APPLY    : out[n][o] = sum_i weight[species[n]][o][i] x[n][i]
 *   ICTC_SPECIES_TRANSPOSE: out[n][i] = sum_o weight[species[n]][o][i] x[n][o]   (the input
 *                           adjoint of APPLY)
 * weight [num_species, channels, channels] (one torch Linear weight per species, row o), x and out
 * [nodes, channels], species [nodes] int64 in [0, num_species) (validated by the caller; a value
 * outside reads species 0).  Replaces ElementConditionedLinearSO3 on the l = 0 block (reference
 * mace_ictc/models/pure_cartesian_ictd_fix.py:335-390), whose library-op form is one product with
 * every species' weight followed by a gather of each node's block.  1 <= channels <=
 * ICTC_SPECIES_MAX_CHANNELS.
 */
enum ictc_species_mode { ICTC_SPECIES_APPLY = 0, ICTC_SPECIES_TRANSPOSE = 1 };
#define ICTC_SPECIES_MAX_CHANNELS 4096
int ictc_hip_species_linear(int mode, const float* weight, const float* x, const int64_t* species, float* out,
                            int channels, int num_species, int64_t nodes, hipStream_t stream);

/*
 * Atomic-energy readouts of the MACE model, one pass per derivative order.  Per node n, with x the
 * last layer's scalar features [nodes, channels] and y an earlier layer's (or null):
 *   ICTC_READOUT_VALUE: out_atomic[n] = w_lin . y[n] + sum_j w2[j] scale silu(w1[j] . x[n])
 *   ICTC_READOUT_VJP  : for grad_atomic g: grad_y[n] = g[n] w_lin (if non-null) and
 *                       grad_x[n] = sum_j w1[j] scale w2[j] silu'(w1[j] . x[n]) g[n] (if non-null)
 * w_lin [channels], w1 [hidden, channels], w2 [hidden].  Replaces the per-layer readout (bias-free
 * Linear(C, 1), reference EquivariantScalarReadoutSO3, mace_ictc/models/pure_cartesian_ictd_layers.py:
 * 46-70) of one inner layer and the last layer's MLP readout (Linear(C, H), normalised SiLU,
 * Linear(H, 1); mace_ictc/models/pure_cartesian_ictd_fix.py:1434-1449), summed, with their
 * adjoints.  1 <= channels <= ICTC_READOUT_MAX_CHANNELS, 1 <= hidden <= ICTC_READOUT_MAX_HIDDEN.
 */
enum ictc_readout_mode { ICTC_READOUT_VALUE = 0, ICTC_READOUT_VJP = 1 };
#define ICTC_READOUT_MAX_CHANNELS 1024
#define ICTC_READOUT_MAX_HIDDEN 256
int ictc_hip_readout(int mode, const float* y, const float* w_lin, const float* x, const float* w1,
                     const float* w2, float scale, const float* grad_atomic, float* out_atomic, float* grad_y,
                     float* grad_x, int channels, int hidden, int64_t nodes, hipStream_t stream);

/*
 * SiLU derivative forms of force training's double backward through the radial MLP: for the
 * first-order backward y = grad * silu'(x) and a cotangent of y, one elementwise pass over n
 * floats writes
 *   grad_grad[i] = cotangent[i] * silu'(x[i])                 (if non-null)
 *   grad_x[i]    = cotangent[i] * grad[i] * silu''(x[i])      (if non-null; needs grad)
 * with s = sigmoid(x), silu' = s (1 + x (1 - s)), silu'' = s (1 - s) (2 + x (1 - 2 s)).
 * Replaces the silu derivative modes of the fp32 elementwise kernel ictc_binary
 * (ascendc/op_kernel/vector.cpp:6-136, ascendc/elementwise.py:7-97).
 */
int ictc_hip_silu_second(const float* x, const float* grad, const float* cotangent,
                         float* grad_grad, float* grad_x, int64_t n, hipStream_t stream);

/*
 * Radial MLP of the MACE interaction up to its last Linear, on fp32 MFMA (reference
 * mace_ictc/models/pure_cartesian_ictd_fix.py:1545-1553 `fc` without its last layer, applied to
 * the edge features at :1795; _Normalize2MomSiLU :610-619).  Per edge, with f [E, B] row-major
 * (1 <= B <= 16), weights in nn.Linear layout w1 [64, B], w2 [64, 64], w3 [64, 64] and `scale`
 * the normalised-SiLU constant applied to the activations that feed w2 and w3:
 *   h = silu(scale w3 silu(scale w2 silu(w1 f)))                               [E, 64]
 * Modes:
 *   ICTC_RADIAL_VALUE:   out_hidden = h.
 *   ICTC_RADIAL_VJP:     for grad_hidden g [E, 64]: out_grad_feats = J^T g [E, B] and
 *                        grad_w1/2/3 = the gradients of <g, h> in the weights (each optional).
 *   ICTC_RADIAL_VJP_VJP: for g and cotangent u [E, B] of the VJP's feature gradient, the
 *                        derivatives of <u, J^T g>: out_grad_grad_hidden = J u [E, 64] (its
 *                        gradient in g), out_grad_feats = its gradient in f, grad_w1/2/3 = its
 *                        gradients in the weights (each optional).
 * Weight gradients are summed over edges through a workspace of
 * ictc_hip_radial_mlp_workspace(edges) floats (caller-owned; minus the status code for invalid
 * sizes) in a fixed order (bit-identical run to run) and fully overwrite grad_w1/2/3 (zero for
 * edges = 0).  Replaces the Linear/SiLU chain of the reference's radial network and its autograd
 * derivatives (one GEMM per layer and direction, elementwise passes per activation).
 */
enum ictc_radial_mode { ICTC_RADIAL_VALUE = 0, ICTC_RADIAL_VJP = 1, ICTC_RADIAL_VJP_VJP = 2 };
#define ICTC_RADIAL_WIDTH 64
#define ICTC_RADIAL_MAX_BASIS 16
int64_t ictc_hip_radial_mlp_workspace(int64_t edges);

int ictc_hip_radial_mlp(int mode, const float* feats, const float* w1, const float* w2, const float* w3,
                        float scale, const float* grad_hidden, const float* cotangent, float* out_hidden,
                        float* out_grad_feats, float* out_grad_grad_hidden, float* workspace,
                        int64_t workspace_floats, float* grad_w1, float* grad_w2, float* grad_w3,
                        int num_basis, int64_t edges, hipStream_t stream);

/*
 * Per-degree channel linear on fp32 MFMA (v_mfma_f32_16x16x4_f32), for the path-preserving
 * message linear of the MACE interaction (reference
 * mace_ictc/models/pure_cartesian_ictd_fix.py:629-661; native route ictc_o3/ascendc/linear.py:
 * 12-136), reading the message kernels' packed output directly.  For degree l (d = 2l + 1):
 *   x [nodes, sum_l counts[l] d C]: per node and degree, counts[l] path blocks of [d][C]
 *                                    (ir_mul; the ictc_hip_message_forward output layout);
 *   y [nodes, O (lmax+1)^2]:         per node and degree, [O][d] at offset O l^2 (mul_ir);
 *   weights[l] [O, counts[l] C]:     row-major, column k C + c = (path block k, channel c)
 *                                    (weights is a host array of lmax + 1 device pointers).
 *   forward:    y[n, o, m]     = alpha sum_{k,c} weights[l][o, k C + c] x[n, k, m, c]
 *   input_grad: grad_x[n,k,m,c] = alpha sum_o grad_y[n, o, m] weights[l][o, k C + c]
 * (the adjoint of the forward in x; the weight adjoint is ictc_hip_degree_linear_weight_grad
 * below).  y and grad_x are fully overwritten; a degree with counts[l] = 0 gets zero y rows.
 * Fixed summation order (bit-identical run to run).
 */
#define ICTC_LINEAR_MAX_DEGREES 8
typedef struct ictc_degree_linear_desc {
    int32_t lmax;                               /* degrees 0..lmax, lmax < 8 */
    int32_t channels;                           /* C, channels of an input path block */
    int32_t out_channels;                       /* O */
    int32_t counts[ICTC_LINEAR_MAX_DEGREES];    /* path blocks per degree */
} ictc_degree_linear_desc;

int ictc_hip_degree_linear_forward(const ictc_degree_linear_desc* desc, const float* x,
                                   const float* const* weights, float alpha, float* y,
                                   int64_t nodes, hipStream_t stream);

int ictc_hip_degree_linear_input_grad(const ictc_degree_linear_desc* desc, const float* grad_y,
                                      const float* const* weights, float alpha, float* grad_x,
                                      int64_t nodes, hipStream_t stream);

/*
 * The same per-degree channel map on mul_ir rows in and out, with one channel block per degree
 * (counts[l] = 1 for every l, else ICTC_ERR_INVALID_ARGUMENT): for x [nodes, C (lmax+1)^2] and
 * y [nodes, O (lmax+1)^2], both per degree [channels][2l+1] at offsets C l^2 / O l^2,
 *   y[n, o, m] = alpha sum_c weights[l][o, c] x[n, c, m]
 * The e3nn o3.Linear of the MACE product block (reference pure_cartesian_ictd_fix.py:1145-1195,
 * an irreps-preserving C x C map per degree); its input adjoint is this map with the weights
 * transposed (and the roles of C and O swapped).
 */
int ictc_hip_degree_linear_mul_ir(const ictc_degree_linear_desc* desc, const float* x,
                                  const float* const* weights, float alpha, float* y,
                                  int64_t nodes, hipStream_t stream);

/*
 * The same map with the weights given transposed: weights[l] [channels, out_channels] and
 *   y[n, o, m] = alpha sum_c weights[l][c, o] x[n, c, m]
 * i.e. the input adjoint of ictc_hip_degree_linear_mul_ir for the descriptor with channels and
 * out_channels swapped, applied to its own weights without a transposed copy of them (the
 * backward of the product block's o3.Linear, pure_cartesian_ictd_fix.py:1145-1195).
 */
int ictc_hip_degree_linear_mul_ir_transposed(const ictc_degree_linear_desc* desc, const float* x,
                                             const float* const* weights, float alpha, float* y,
                                             int64_t nodes, hipStream_t stream);

/*
 * Weight adjoint of the two maps above, per degree l (rows rho = n d + m, d = 2l + 1):
 *   grad_weights[l][o, j] = alpha sum_{n, m} grad_y[n, o, m] x[rho, j]
 * with x in the forward's layout (x_layout 0: x[n, k, m, c], j = k C + c) or in the mul_ir map's
 * (x_layout 1: x[n, c, m] at offset C l^2, j = c; counts[l] = 1 for every l).  It replaces the
 * weight gradient autograd forms for reference pure_cartesian_ictd_fix.py:629-661 (the
 * path-preserving linear) and :1145-1195 (the product's o3.Linear) from rearranged copies of both
 * operands.  grad_weights is a host array of lmax + 1 device pointers [O, counts[l] C]; a null
 * entry skips that degree.  The rows of a degree are split into ranges whose 128 x 64 partials go
 * to `workspace` (at least ictc_hip_degree_linear_weight_grad_workspace(desc, x_layout, nodes)
 * floats, caller-owned; the query returns minus the status code for an invalid descriptor or
 * layout) and are then summed in range order (bit-identical run to run); every
 * asked-for gradient is fully overwritten (zero for nodes = 0).  x and grad_y must each be below
 * 2 GiB (ICTC_ERR_UNSUPPORTED otherwise).
 */
int64_t ictc_hip_degree_linear_weight_grad_workspace(const ictc_degree_linear_desc* desc, int x_layout,
                                                     int64_t nodes);

int ictc_hip_degree_linear_weight_grad(const ictc_degree_linear_desc* desc, int x_layout,
                                       const float* grad_y, const float* x, float alpha,
                                       float* workspace, int64_t workspace_floats,
                                       float* const* grad_weights, int64_t nodes, hipStream_t stream);

/*
 * Row-major fp32 product C[m,n] = alpha * op(A) op(B) + beta * C on rocBLAS, for the dense
 * channel linears around the operators.  op(A) is [m,k]: A is stored [m,k] (lda >= k) or,
 * with trans_a != 0, [k,m] (lda >= m); likewise B with op(B) [k,n].  Each host thread uses
 * one rocBLAS handle per device; the call is asynchronous on `stream`.  Replaces the fp32
 * Cube GEMM binding of the reference (ictc_o3/ascendc/op_host/matmul_bindings.cpp:24-96,
 * ascendc/linear.py:12-58) behind channel_linear (backends/ascend/linear.py:8-52).
 */
int ictc_hip_sgemm(int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, float alpha,
                   const float* a, int64_t lda, const float* b, int64_t ldb, float beta, float* c,
                   int64_t ldc, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* ICTC_HIP_H */
