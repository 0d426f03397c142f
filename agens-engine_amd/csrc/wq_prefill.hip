// The prefill consumer of the dequantized weights: y[m][ldy] = x[m][k] W^T for bf16 x and W [n][k], fp32 accumulation,
// bf16 output (reference: ak_bf16_linear_f32reduce / _ld, kernels/src/bf16_linear.cu:68-92, a cuBLAS GemmEx with a
// 32F compute type).  Above 128 tokens the model's linear() dequantizes a tile of output rows at a time
// (ak_wq_dequant_kt_rows) and calls these (kernels/m1/m1_model.cu:1876-1897).  Here the GEMM is rocBLAS's gemm_ex
// (a plain library GEMM: bf16 inputs, fp32 compute, bf16 output), one handle per device, created on first use.
#include <rocblas/rocblas.h>

#include <mutex>

#include "agens_kernels.h"
#include "wq_common.h"

namespace agq {
namespace {

rocblas_handle handle_for_device(int* err) {
  static std::mutex mu;
  static rocblas_handle handles[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    *err = AK_INVALID;
    return nullptr;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!handles[dev] && rocblas_create_handle(&handles[dev]) != rocblas_status_success) {
    handles[dev] = nullptr;
    *err = (int)hipErrorUnknown;
    return nullptr;
  }
  *err = 0;
  return handles[dev];
}

int gemm_f32reduce(const void* x, const void* w, void* y, int m, int n, int k, int ldy, hipStream_t s) {
  if (!x || !w || !y || m < 1 || n < 1 || k < 1 || ldy < n) return AK_INVALID;
  int e = 0;
  rocblas_handle h = handle_for_device(&e);
  if (!h) return e;
  if (rocblas_set_stream(h, s) != rocblas_status_success) return (int)hipErrorUnknown;
  const float alpha = 1.f, beta = 0.f;
  // column-major: Y^T [n x m] (ld ldy) = W^T ... as the reference's cublasGemmEx(OP_T, OP_N, n, m, k): A = W stored
  // k x n (lda k, transposed), B = x stored k x m (ldb k), C = D = y (ldc ldy)
  const rocblas_status st = rocblas_gemm_ex(h, rocblas_operation_transpose, rocblas_operation_none, n, m, k, &alpha, w,
                                            rocblas_datatype_bf16_r, k, x, rocblas_datatype_bf16_r, k, &beta, y,
                                            rocblas_datatype_bf16_r, ldy, y, rocblas_datatype_bf16_r, ldy,
                                            rocblas_datatype_f32_r, rocblas_gemm_algo_standard, 0, 0);
  return st == rocblas_status_success ? 0 : (int)hipErrorUnknown;
}

}  // namespace
}  // namespace agq

extern "C" {

int ak_bf16_linear_f32reduce(const void* x, const void* w, void* y, int m, int n, int k, void* stream) {
  return agq::gemm_f32reduce(x, w, y, m, n, k, n, static_cast<hipStream_t>(stream));
}

int ak_bf16_linear_f32reduce_ld(const void* x, const void* w, void* y, int m, int n, int k, int ldy, void* stream) {
  return agq::gemm_f32reduce(x, w, y, m, n, k, ldy, static_cast<hipStream_t>(stream));
}

}  // extern "C"
