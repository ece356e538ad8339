// Shared pieces of the chunked PAM scan kernels (forward and backward).
#pragma once

#include "common.h"

namespace qpam {
namespace scan {

constexpr int D = 64;          // head dim handled by the MFMA scan kernels
constexpr int P = D + 4;       // LDS row pitch (floats) of a 64-wide tile
constexpr int THREADS = 256;   // 4 waves
constexpr int MAX_M = 4;       // states per head
constexpr float LOG_EPS = 1e-6f;  // log(gamma + 1e-6), v11/flash_pam.py:45

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ floatx4 zero4() { return floatx4{0.f, 0.f, 0.f, 0.f}; }

// Load a [rows x 64] planar tile (one plane) of element type T from global
// rows base + t*st (t < valid; rows >= valid are zero) into LDS as fp32,
// multiplied by `scale`.  All 256 threads participate.
template <typename T>
__device__ __forceinline__ void load_tile(float *lds, const T *base, int64_t st, int rows, int valid, float scale);

template <>
__device__ __forceinline__ void load_tile<float>(float *lds, const float *base, int64_t st, int rows, int valid,
                                                 float scale) {
    // 16 float4 per row
    for (int idx = threadIdx.x; idx < rows * 16; idx += THREADS) {
        const int r = idx >> 4, c4 = idx & 15;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < valid) v = *reinterpret_cast<const float4 *>(base + (int64_t)r * st + 4 * c4);
        float *dst = lds + r * P + 4 * c4;
        dst[0] = v.x * scale;
        dst[1] = v.y * scale;
        dst[2] = v.z * scale;
        dst[3] = v.w * scale;
    }
}

template <>
__device__ __forceinline__ void load_tile<unsigned short>(float *lds, const unsigned short *base, int64_t st,
                                                          int rows, int valid, float scale) {
    // 8 x (8 bf16 = 16 bytes) per row
    for (int idx = threadIdx.x; idx < rows * 8; idx += THREADS) {
        const int r = idx >> 3, c8 = idx & 7;
        ushortx8 v = {0, 0, 0, 0, 0, 0, 0, 0};
        if (r < valid) v = *reinterpret_cast<const ushortx8 *>(base + (int64_t)r * st + 8 * c8);
        float *dst = lds + r * P + 8 * c8;
#pragma unroll
        for (int e = 0; e < 8; ++e) dst[e] = bf16_to_f32(v[e]) * scale;
    }
}

// Inclusive prefix sums L[t] = sum_{u<=t} log(gamma[u] + 1e-6) over one chunk of
// `valid` steps (entries >= valid hold L[valid-1]).  Executed by one full wave;
// `g` points at gamma[t0] with stride gs.  Returns L for lane t (t < 64).
__device__ __forceinline__ float chunk_log_prefix(const float *g, int64_t gs, int valid, int lane) {
    float x = (lane < valid) ? logf(g[(int64_t)lane * gs] + LOG_EPS) : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        float y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    return x;
}

}  // namespace scan
}  // namespace qpam
