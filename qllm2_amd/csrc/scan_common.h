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

// ------------------------------------------------------------------------
// bf16 MFMA helpers (v_mfma_f32_16x16x32_bf16).  Operand fragment: lane l
// supplies 8 bf16 for row/col l % 16 and k-group g = l / 16.  Both operands of
// one MFMA use the same (g, element) -> k assignment, so any consistent k
// permutation gives the same product; the register-sourced fragments below
// rely on this.  Accumulator layout: lane holds C[4g + r][l % 16], r = 0..3.
// LDS tiles are 64 rows x 64 bf16 with pitch PB (elements).
constexpr int PB = 72;                  // 144-byte rows
constexpr int PLANE_B = 64 * PB;        // elements per bf16 LDS plane

typedef float floatx8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ floatx4 mfma_bf(bf16x8 a, bf16x8 b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8 neg_bf(bf16x8 x) {
    uint4 u = __builtin_bit_cast(uint4, x);
    u.x ^= 0x80008000u;
    u.y ^= 0x80008000u;
    u.z ^= 0x80008000u;
    u.w ^= 0x80008000u;
    return __builtin_bit_cast(bf16x8, u);
}

__device__ __forceinline__ bf16x8 to_bf(floatx8 x) { return __builtin_convertvector(x, bf16x8); }

__device__ __forceinline__ floatx8 to_f(bf16x8 x) { return __builtin_convertvector(x, floatx8); }

// 8 consecutive bf16 (16-byte LDS read)
__device__ __forceinline__ bf16x8 ld8(const unsigned short *p) { return *reinterpret_cast<const bf16x8 *>(p); }

// two runs of 4 consecutive bf16 (two 8-byte LDS reads): the k order of a
// fragment built from two 16x16 accumulator tiles (rows 4g..4g+3 of each)
__device__ __forceinline__ bf16x8 ld4x2(const unsigned short *p0, const unsigned short *p1) {
    const bf16x4 a = *reinterpret_cast<const bf16x4 *>(p0);
    const bf16x4 b = *reinterpret_cast<const bf16x4 *>(p1);
    return bf16x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
}

// fragment from two accumulator tiles lo/hi (fp32 -> bf16), same k order as ld4x2
__device__ __forceinline__ bf16x8 frag_from_acc(floatx4 lo, floatx4 hi) {
    return to_bf(floatx8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]});
}

// [64 x 64] bf16 rows (row stride st, rows >= valid zero) -> LDS natural [r][c]
__device__ __forceinline__ void lds_nat_bf(unsigned short *lds, const unsigned short *src, int64_t st, int valid) {
    for (int idx = threadIdx.x; idx < 64 * 8; idx += THREADS) {
        const int r = idx >> 3, c8 = idx & 7;
        uint4 v = make_uint4(0, 0, 0, 0);
        if (r < valid) v = *reinterpret_cast<const uint4 *>(src + (int64_t)r * st + 8 * c8);
        *reinterpret_cast<uint4 *>(lds + r * PB + 8 * c8) = v;
    }
}

// [64 x 64] bf16 rows -> LDS transposed [c][r]
__device__ __forceinline__ void lds_tr_bf(unsigned short *lds, const unsigned short *src, int64_t st, int valid) {
    for (int idx = threadIdx.x; idx < 64 * 8; idx += THREADS) {
        const int r = idx & 63, c8 = idx >> 6;
        ushortx8 v = {0, 0, 0, 0, 0, 0, 0, 0};
        if (r < valid) v = *reinterpret_cast<const ushortx8 *>(src + (int64_t)r * st + 8 * c8);
#pragma unroll
        for (int e = 0; e < 8; ++e) lds[(8 * c8 + e) * PB + r] = v[e];
    }
}

// [64 x 64] fp32 rows -> LDS bf16, natural or transposed
template <bool TR>
__device__ __forceinline__ void lds_from_f32(unsigned short *lds, const float *src, int64_t st, int valid) {
    for (int idx = threadIdx.x; idx < 64 * 16; idx += THREADS) {
        const int r = TR ? (idx & 63) : (idx >> 4), c4 = TR ? (idx >> 6) : (idx & 15);
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (r < valid) v = *reinterpret_cast<const float4 *>(src + (int64_t)r * st + 4 * c4);
        const float f[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const unsigned short b = f32_to_bf16(f[e]);
            if (TR) lds[(4 * c4 + e) * PB + r] = b;
            else lds[r * PB + 4 * c4 + e] = b;
        }
    }
}

}  // namespace scan
}  // namespace qpam
