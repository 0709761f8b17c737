// Dense fp32 products of the operator library's channel linears on rocBLAS, called explicitly
// (no process-wide library preference is changed).
//
// Row-major semantics: C[m, n] = alpha * op(A) op(B) + beta * C with op(A) [m, k] and op(B)
// [k, n]; trans_a != 0 means A is stored as [k, m] (lda >= m), otherwise as [m, k]
// (lda >= k); likewise B.  rocBLAS is column-major, so the row-major product is issued as the
// column-major C^T = op(B)^T op(A)^T.  Each host thread keeps one rocBLAS handle per device
// (a handle must not be used by two threads at once); the stream is set on every call, and
// atomics are disallowed on every handle so repeated products are bit-identical.
#include <hip/hip_runtime.h>
#include <rocblas/rocblas.h>

#include <unordered_map>

#include "ictc_hip.h"

namespace {

rocblas_handle handle_for_current_device() {
  thread_local std::unordered_map<int, rocblas_handle> handles;
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return nullptr;
  auto it = handles.find(device);
  if (it != handles.end()) return it->second;
  rocblas_handle h = nullptr;
  if (rocblas_create_handle(&h) != rocblas_status_success) return nullptr;
  // no kernels that accumulate through atomics: a product's result is the same on every run
  if (rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed) != rocblas_status_success) {
    rocblas_destroy_handle(h);
    return nullptr;
  }
  handles.emplace(device, h);
  return h;
}

}  // namespace

extern "C" int ictc_hip_sgemm(int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, float alpha,
                              const float* a, int64_t lda, const float* b, int64_t ldb, float beta, float* c,
                              int64_t ldc, hipStream_t stream) {
  if (m < 0 || n < 0 || k < 0) return ICTC_ERR_INVALID_ARGUMENT;
  if (m == 0 || n == 0) return ICTC_OK;
  const int64_t int_max = 2147483647;
  if (m > int_max || n > int_max || k > int_max || lda > int_max || ldb > int_max || ldc > int_max)
    return ICTC_ERR_INVALID_ARGUMENT;
  if (c == nullptr || ldc < n || (k > 0 && (a == nullptr || b == nullptr))) return ICTC_ERR_INVALID_ARGUMENT;
  if (k > 0 && (lda < (trans_a ? m : k) || ldb < (trans_b ? k : n))) return ICTC_ERR_INVALID_ARGUMENT;
  rocblas_handle h = handle_for_current_device();
  if (h == nullptr) return ICTC_ERR_LAUNCH;
  if (rocblas_set_stream(h, stream) != rocblas_status_success) return ICTC_ERR_LAUNCH;
  const rocblas_operation op_a = trans_a ? rocblas_operation_transpose : rocblas_operation_none;
  const rocblas_operation op_b = trans_b ? rocblas_operation_transpose : rocblas_operation_none;
  // k == 0 leaves C = beta * C and reads neither operand, but rocBLAS still checks their leading
  // dimensions (at least the stored rows of the column-major views, and 1) and pointers: pass
  // the smallest legal ones and a valid address instead of whatever the caller gave
  const int64_t ldb_rb = k > 0 ? ldb : (trans_b ? 1 : (n > 1 ? n : 1));
  const int64_t lda_rb = k > 0 ? lda : (trans_a ? (m > 1 ? m : 1) : 1);
  const float* a_rb = k > 0 ? a : c;
  const float* b_rb = k > 0 ? b : c;
  // column-major view: C^T [n, m] = op(B)^T [n, k] * op(A)^T [k, m]
  const rocblas_status st = rocblas_sgemm(h, op_b, op_a, static_cast<rocblas_int>(n), static_cast<rocblas_int>(m),
                                          static_cast<rocblas_int>(k), &alpha, b_rb, static_cast<rocblas_int>(ldb_rb),
                                          a_rb, static_cast<rocblas_int>(lda_rb), &beta, c,
                                          static_cast<rocblas_int>(ldc));
  return st == rocblas_status_success ? ICTC_OK : ICTC_ERR_LAUNCH;
}
