// dense.hip — Raster's dense f32 GEMM surface (the float arms of
// raster/linalg/blas.clj:287-337 and nn/linear, raster/dl/nn.clj:161-183) on
// the GPU: a plain library GEMM, so rocBLAS does the product (Raster hands
// the same call to MKL / OpenBLAS cblas_sgemm). Row-major operands map to
// rocBLAS's column-major call with the operands swapped: C^T = op(B)^T op(A)^T.
// rocBLAS allows atomics by default (split-K and Stream-K solutions may then
// sum partial tiles in arrival order); the handle turns them off, so results
// repeat bit for bit.
#include <rocblas/rocblas.h>

#include <algorithm>

#include "rq_internal.h"

namespace rq {

namespace {

// y[r, :] = b for every row r (nn/linear's bias pre-fill, nn.clj:170-171)
__global__ __launch_bounds__(256) void bias_rows_kernel(const float* __restrict__ b, float* __restrict__ y,
                                                        int64_t rows, int64_t cols) {
  const int64_t n = rows * cols;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    y[i] = b[i % cols];
}

}  // namespace

int dense_create(void** handle) {
  rocblas_handle h = nullptr;
  rocblas_status st = rocblas_create_handle(&h);
  if (st != rocblas_status_success) return (int)st;
  st = rocblas_set_atomics_mode(h, rocblas_atomics_not_allowed);
  if (st != rocblas_status_success) {
    (void)rocblas_destroy_handle(h);
    return (int)st;
  }
  *handle = h;
  return 0;
}

void dense_destroy(void* handle) {
  if (handle) (void)rocblas_destroy_handle(static_cast<rocblas_handle>(handle));
}

const char* dense_status_string(int st) { return rocblas_status_to_string((rocblas_status)st); }

int dense_sgemm(void* handle, hipStream_t stream, int trans_a, int trans_b, int64_t m, int64_t n, int64_t k,
                float alpha, const float* a, const float* b, float beta, float* c) {
  rocblas_handle h = static_cast<rocblas_handle>(handle);
  rocblas_status st = rocblas_set_stream(h, stream);
  if (st != rocblas_status_success) return (int)st;
  // row-major op(A) [m x k], op(B) [k x n], C [m x n]: A is stored [m x k]
  // (or [k x m] when transposed), B [k x n] (or [n x k])
  const rocblas_operation opa = trans_a ? rocblas_operation_transpose : rocblas_operation_none;
  const rocblas_operation opb = trans_b ? rocblas_operation_transpose : rocblas_operation_none;
  const rocblas_int lda = (rocblas_int)(trans_a ? m : k), ldb = (rocblas_int)(trans_b ? k : n);
  st = rocblas_sgemm(h, opb, opa, (rocblas_int)n, (rocblas_int)m, (rocblas_int)k, &alpha, b, ldb, a, lda, &beta, c,
                     (rocblas_int)n);
  return (int)st;
}

hipError_t launch_bias_rows(const float* b, float* y, int64_t rows, int64_t cols, hipStream_t stream) {
  const int64_t n = rows * cols;
  const int64_t blocks = std::min<int64_t>((n + 255) / 256, 4096);
  hipLaunchKernelGGL(bias_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, b, y, rows, cols);
  return hipGetLastError();
}

}  // namespace rq
