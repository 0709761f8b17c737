// extern "C" entry points of the tensor-product family: descriptor validation and
// dispatch to the per-degree instantiations compiled in generated/tp_inst_*.hip.
#include "generic.hpp"
#include "tp_kernels.hpp"

namespace ictc {

// Explicit instantiations live in separate translation units (parallel build).
#define ICTC_DECLARE(A, B, C)                                                                  \
  extern template int launch_forward<A, B, C>(const ictc_tp_desc&, const float*, const float*,   \
                                              const float*, float*, int64_t, hipStream_t);      \
  extern template int launch_backward<A, B, C>(const ictc_tp_desc&, const float*, const float*,  \
                                               const float*, const float*, float*, float*, float*, \
                                               int64_t, hipStream_t);
#include "generated/tp_instances.def"
#undef ICTC_DECLARE

// Compiled wide degree sets (a degree of 4; tp_wide_instances.def), dispatched ahead of the
// degree-generic kernels.
#define ICTC_DECLARE(A, B, C)                                                                  \
  extern template int launch_forward<A, B, C>(const ictc_tp_desc&, const float*, const float*,   \
                                              const float*, float*, int64_t, hipStream_t);      \
  extern template int launch_backward<A, B, C>(const ictc_tp_desc&, const float*, const float*,  \
                                               const float*, const float*, float*, float*, float*, \
                                               int64_t, hipStream_t);
#include "generated/tp_wide_instances.def"
#undef ICTC_DECLARE

inline bool same_degrees(const ictc_tp_desc* d, int a, int b, int c) {
  return d->input_lmax == a && d->edge_lmax == b && d->output_lmax == c;
}

FwdLaunch wide_forward(const ictc_tp_desc* d) {
#define ICTC_DECLARE(A, B, C) \
  if (same_degrees(d, A, B, C)) return &launch_forward<A, B, C>;
#include "generated/tp_wide_instances.def"
#undef ICTC_DECLARE
  return nullptr;
}

BwdLaunch wide_backward(const ictc_tp_desc* d) {
#define ICTC_DECLARE(A, B, C) \
  if (same_degrees(d, A, B, C)) return &launch_backward<A, B, C>;
#include "generated/tp_wide_instances.def"
#undef ICTC_DECLARE
  return nullptr;
}

// Dispatch tables of the per-degree instantiations (every degree <= 3), indexed by
// input_lmax*16 + edge_lmax*4 + output_lmax; entries of combinations left out of a
// (development) build are null and report UNSUPPORTED.
#define ICTC_DECLARE(A, B, C) [A * 16 + B * 4 + C] = &launch_forward<A, B, C>,
const FwdLaunch kFwdTable[64] = {
#include "generated/tp_instances.def"
};
#undef ICTC_DECLARE
#define ICTC_DECLARE(A, B, C) [A * 16 + B * 4 + C] = &launch_backward<A, B, C>,
const BwdLaunch kBwdTable[64] = {
#include "generated/tp_instances.def"
};
#undef ICTC_DECLARE

// Host-side validation of a descriptor against the compiled path enumeration.
int tp_check_desc(const ictc_tp_desc* d) {
  if (d == nullptr) return ICTC_ERR_INVALID_ARGUMENT;
  if (d->channels < 1 || d->num_paths < 0 || d->num_paths > ICTC_MAX_PATHS || d->out_components < 0)
    return ICTC_ERR_INVALID_ARGUMENT;
  if (d->input_lmax < 0 || d->edge_lmax < 0 || d->output_lmax < 0) return ICTC_ERR_INVALID_ARGUMENT;
  if (d->input_lmax > kGenericMaxL || d->edge_lmax > kGenericMaxL || d->output_lmax > kGenericMaxL)
    return ICTC_ERR_UNSUPPORTED;
  // The kernels run the full path set of the degrees with its canonical layout; the
  // descriptor must state exactly that (path subsets are mapped by the caller).
  const PathTable t = make_paths(d->input_lmax, d->edge_lmax, d->output_lmax);
  if (d->num_paths != t.n || d->out_components != t.noc) return ICTC_ERR_INVALID_ARGUMENT;
  for (int s = 0; s < t.n; ++s)
    if (d->gate_index[s] != s || d->out_offset[s] != t.out[s]) return ICTC_ERR_INVALID_ARGUMENT;
  return ICTC_OK;
}

inline int table_index(const ictc_tp_desc* d) {
  return d->input_lmax * 16 + d->edge_lmax * 4 + d->output_lmax;
}

}  // namespace ictc

extern "C" {

const char* ictc_hip_status_string(int status) {
  switch (status) {
    case ICTC_OK: return "ok";
    case ICTC_ERR_INVALID_ARGUMENT: return "invalid argument";
    case ICTC_ERR_UNSUPPORTED: return "unsupported degree combination";
    case ICTC_ERR_LAUNCH: return "kernel launch failed";
    case ICTC_ERR_INDEX: return "index out of range";
    case ICTC_ERR_CAPACITY: return "input exceeds the static scratch capacity";
    default: return "unknown status";
  }
}

int ictc_hip_abi_version(void) { return 21; }

int ictc_hip_tp_slot_count(int input_lmax, int edge_lmax, int output_lmax) {
  constexpr int L = ictc::kGenericMaxL;
  if (input_lmax < 0 || edge_lmax < 0 || output_lmax < 0 || input_lmax > L || edge_lmax > L || output_lmax > L)
    return -1;
  return ictc::make_paths(input_lmax, edge_lmax, output_lmax).n;
}

int ictc_hip_tp_forward(const ictc_tp_desc* desc, const float* features, const float* harmonics,
                        const float* gates, float* out, int64_t rows, hipStream_t stream) {
  const int st = ictc::tp_check_desc(desc);
  if (st != ICTC_OK) return st;
  if (rows < 0) return ICTC_ERR_INVALID_ARGUMENT;
  if (rows == 0) return ICTC_OK;
  if (!features || !harmonics || !gates || !out) return ICTC_ERR_INVALID_ARGUMENT;
  if (const ictc::FwdLaunch wide = ictc::wide_forward(desc))
    return wide(*desc, features, harmonics, gates, out, rows, stream);
  if (ictc::generic_degrees(*desc))
    return ictc::generic_tp_forward(*desc, features, harmonics, gates, out, rows, stream);
  const ictc::FwdLaunch fn = ictc::kFwdTable[ictc::table_index(desc)];
  if (fn == nullptr) return ICTC_ERR_UNSUPPORTED;
  return fn(*desc, features, harmonics, gates, out, rows, stream);
}

int ictc_hip_tp_backward(const ictc_tp_desc* desc, const float* features, const float* harmonics,
                         const float* gates, const float* grad_out, float* grad_features,
                         float* grad_harmonics, float* grad_gates, int64_t rows, hipStream_t stream) {
  const int st = ictc::tp_check_desc(desc);
  if (st != ICTC_OK) return st;
  if (rows < 0) return ICTC_ERR_INVALID_ARGUMENT;
  if (rows == 0) return ICTC_OK;
  if (!harmonics || !gates || !grad_out) return ICTC_ERR_INVALID_ARGUMENT;
  if ((grad_harmonics || grad_gates) && !features) return ICTC_ERR_INVALID_ARGUMENT;
  if (!grad_features && !grad_harmonics && !grad_gates) return ICTC_OK;
  if (const ictc::BwdLaunch wide = ictc::wide_backward(desc))
    return wide(*desc, features, harmonics, gates, grad_out, grad_features, grad_harmonics, grad_gates, rows,
                stream);
  if (ictc::generic_degrees(*desc))
    return ictc::generic_tp_backward(*desc, features, harmonics, gates, grad_out, grad_features, grad_harmonics,
                                     grad_gates, rows, stream);
  const ictc::BwdLaunch fn = ictc::kBwdTable[ictc::table_index(desc)];
  if (fn == nullptr) return ICTC_ERR_UNSUPPORTED;
  return fn(*desc, features, harmonics, gates, grad_out, grad_features, grad_harmonics, grad_gates,
            rows, stream);
}

}  // extern "C"
