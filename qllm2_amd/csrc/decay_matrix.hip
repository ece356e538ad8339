// Materialised decay matrix for the fused_decay_matrix API.
//
// Reference: fused_decay_matrix (v11/triton_kernels.py:570-573), forward
// _FusedDecayMatrixFn (420-445) over _decay_matrix_from_cumsum (170-202):
//     c = cumsum(-log(gamma + 1e-6)),  D[t,s] = exp(min(c_s - c_t, 0)) (s <= t), 0 otherwise.
// The scan kernels never build this matrix (they rebuild D from prefix sums in
// registers); this entry point exists for callers of the reference API.
// One workgroup per row: block-wide prefix sum of the log-decay into LDS, then
// coalesced row-major writes of the T x T matrix.
#include "common.h"

namespace qpam {
namespace {

constexpr int THREADS = 256;
constexpr int MAX_T = 4096;

__global__ void __launch_bounds__(THREADS) decay_matrix_kernel(int T, const float *gamma, int64_t ldg, float *out) {
    __shared__ float sC[MAX_T];
    __shared__ float sPart[THREADS];
    const int n = blockIdx.x, tid = threadIdx.x;
    const float *g = gamma + (int64_t)n * ldg;
    const int per = (T + THREADS - 1) / THREADS;
    const int b0 = tid * per;
    float local = 0.f;
    for (int i = 0; i < per; ++i) {
        const int t = b0 + i;
        if (t < T) {
            local += -logf(g[t] + 1e-6f);
            sC[t] = local;  // prefix within this thread's segment
        }
    }
    sPart[tid] = local;
    __syncthreads();
    if (tid == 0) {  // exclusive offsets of the segments (T <= 4096: 256 adds)
        float run = 0.f;
        for (int i = 0; i < THREADS; ++i) {
            const float x = sPart[i];
            sPart[i] = run;
            run += x;
        }
    }
    __syncthreads();
    const float off = sPart[tid];
    for (int i = 0; i < per; ++i) {
        const int t = b0 + i;
        if (t < T) sC[t] += off;
    }
    __syncthreads();
    float *o = out + (int64_t)n * T * T;
    for (int64_t e = tid; e < (int64_t)T * T; e += THREADS) {
        const int t = (int)(e / T), s = (int)(e - (int64_t)t * T);
        o[e] = (s <= t) ? __expf(fminf(sC[s] - sC[t], 0.f)) : 0.f;
    }
}

}  // namespace
}  // namespace qpam

extern "C" int qpam_decay_matrix(int32_t n, int32_t t, const float *gamma, int64_t ldg, float *out, void *stream) {
    using namespace qpam;
    QPAM_REQUIRE(n >= 0 && t >= 1 && t <= MAX_T, "qpam_decay_matrix: bad sizes n=%d t=%d (t <= %d)", n, t, MAX_T);
    QPAM_REQUIRE(gamma && out && ldg >= t, "qpam_decay_matrix: null pointer or ldg < t");
    if (n == 0) return QPAM_OK;
    hipLaunchKernelGGL(decay_matrix_kernel, dim3(n), dim3(THREADS), 0, (hipStream_t)stream, t, gamma, ldg, out);
    return launch_status("decay_matrix_kernel");
}
