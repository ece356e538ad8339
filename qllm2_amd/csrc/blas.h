// Library GEMMs (hipBLASLt) used for the plain products of the LM-head backward.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace qpam {
namespace blas {

// Workspace handed to hipBLASLt (carved from the caller's workspace).
constexpr size_t WS_BYTES = size_t(64) << 20;

// false when the environment selects the hand-written GEMM kernels (QPAM_CE_GEMM=hip)
bool enabled();

// Column-major C[m x n] (ldc) = op(A) op(B) + beta C with bf16 A/B, fp32
// accumulation, C in fp32 (c_f32) or bf16; op(A) is m x k, op(B) is k x n.
int gemm_bf16(bool ta, bool tb, int m, int n, int k, const void *A, int64_t lda, const void *B, int64_t ldb,
              float beta, void *C, int64_t ldc, bool c_f32, void *ws, size_t ws_bytes, hipStream_t stream);

}  // namespace blas
}  // namespace qpam
