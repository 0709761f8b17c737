// extern "C" entry points of the symmetric-contraction family; per-configuration
// instantiations are compiled in generated/sc_inst_*.hip.
#include "sc_kernels.hpp"

namespace ictc {
#define ICTC_SC(L, T, K, KTOT)                                                                     \
  extern template int launch_sc<L, T, K>(int, const float*, const float*, const int64_t*, const float*,   \
                                         const float*, float*, int, int64_t, int, hipStream_t);
#include "generated/sc_instances.def"
#undef ICTC_SC

using ScLaunch = int (*)(int, const float*, const float*, const int64_t*, const float*, const float*, float*,
                         int, int64_t, int, hipStream_t);
struct ScEntry {
  ScLaunch fn;
  int ktot;
};
#define ICTC_SC(L, T, K, KTOT) [L * 16 + T * 4 + K] = {&launch_sc<L, T, K>, KTOT},
const ScEntry kSc[64] = {
#include "generated/sc_instances.def"
};
#undef ICTC_SC

inline const ScEntry* sc_entry(int lmax, int target, int corr) {
  if (lmax < 0 || lmax > 3 || target < 0 || target > lmax || corr < 1 || corr > 3) return nullptr;
  const ScEntry* e = &kSc[lmax * 16 + target * 4 + corr];
  return e->fn ? e : nullptr;
}

// modes: 0 forward, 1 VJP, 2 weight features, 3 JVP, 4 Hessian-vector, 5 weight-feature JVP
inline int sc_call(int mode, int lmax, int target, int corr, int channels, const float* x, const float* t,
                   const int64_t* species, const float* w, int num_species, const float* u, float* out,
                   int64_t nodes, hipStream_t stream) {
  const ScEntry* e = sc_entry(lmax, target, corr);
  if (e == nullptr) return ICTC_ERR_UNSUPPORTED;
  if (channels < 1 || nodes < 0 || num_species < 1) return ICTC_ERR_INVALID_ARGUMENT;
  if (nodes == 0) return ICTC_OK;
  const bool needs_w = mode != 2 && mode != 5, needs_u = mode != 0 && mode != 3, needs_t = mode >= 3;
  if (!x || !species || !out || (needs_w && !w) || (needs_u && !u) || (needs_t && !t))
    return ICTC_ERR_INVALID_ARGUMENT;
  return e->fn(mode, x, t, species, w, u, out, channels, nodes, num_species, stream);
}

}  // namespace ictc

extern "C" {

int ictc_hip_sc_weight_columns(int lmax, int target_lmax, int correlation) {
  const ictc::ScEntry* e = ictc::sc_entry(lmax, target_lmax, correlation);
  return e ? e->ktot : -1;
}

int ictc_hip_sc_forward(int lmax, int target_lmax, int correlation, int channels, const float* node_features,
                        const int64_t* species, const float* weights, int num_elements, float* out,
                        int64_t nodes, hipStream_t stream) {
  return ictc::sc_call(0, lmax, target_lmax, correlation, channels, node_features, nullptr, species, weights,
                       num_elements, nullptr, out, nodes, stream);
}

int ictc_hip_sc_backward(int lmax, int target_lmax, int correlation, int channels, const float* node_features,
                         const int64_t* species, const float* weights, int num_elements, const float* grad_out,
                         float* grad_features, int64_t nodes, hipStream_t stream) {
  return ictc::sc_call(1, lmax, target_lmax, correlation, channels, node_features, nullptr, species, weights,
                       num_elements, grad_out, grad_features, nodes, stream);
}

int ictc_hip_sc_weight_features(int lmax, int target_lmax, int correlation, int channels,
                                const float* node_features, const int64_t* species, int num_elements,
                                const float* grad_out, float* features_out, int64_t nodes,
                                hipStream_t stream) {
  return ictc::sc_call(2, lmax, target_lmax, correlation, channels, node_features, nullptr, species, nullptr,
                       num_elements, grad_out, features_out, nodes, stream);
}

int ictc_hip_sc_jvp(int lmax, int target_lmax, int correlation, int channels, const float* node_features,
                    const int64_t* species, const float* weights, int num_elements, const float* tangent,
                    float* out, int64_t nodes, hipStream_t stream) {
  return ictc::sc_call(3, lmax, target_lmax, correlation, channels, node_features, tangent, species, weights,
                       num_elements, nullptr, out, nodes, stream);
}

int ictc_hip_sc_hvp(int lmax, int target_lmax, int correlation, int channels, const float* node_features,
                    const int64_t* species, const float* weights, int num_elements, const float* grad_out,
                    const float* tangent, float* grad_features, int64_t nodes, hipStream_t stream) {
  return ictc::sc_call(4, lmax, target_lmax, correlation, channels, node_features, tangent, species, weights,
                       num_elements, grad_out, grad_features, nodes, stream);
}

int ictc_hip_sc_weight_features_jvp(int lmax, int target_lmax, int correlation, int channels,
                                    const float* node_features, const int64_t* species, int num_elements,
                                    const float* grad_out, const float* tangent, float* features_out,
                                    int64_t nodes, hipStream_t stream) {
  return ictc::sc_call(5, lmax, target_lmax, correlation, channels, node_features, tangent, species, nullptr,
                       num_elements, grad_out, features_out, nodes, stream);
}

}  // extern "C"
