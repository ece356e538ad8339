// Shared helpers of the qpam HIP library (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_bf16.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <string>

#include <mutex>

#include "../../include/qpam.h"

namespace qpam {

// ------------------------------------------------------------- errors ------
std::string &last_error_slot();
int fail(int code, const char *fmt, ...);

#define QPAM_CHECK_HIP(expr)                                                    \
    do {                                                                        \
        hipError_t err__ = (expr);                                              \
        if (err__ != hipSuccess)                                                \
            return ::qpam::fail(QPAM_ERR_HIP, "%s failed: %s", #expr,           \
                                hipGetErrorString(err__));                      \
    } while (0)

#define QPAM_REQUIRE(cond, ...)                                                 \
    do {                                                                        \
        if (!(cond)) return ::qpam::fail(QPAM_ERR_ARG, __VA_ARGS__);            \
    } while (0)

// Fork / join of two independent launch sequences of one call: `side` is an
// extra stream of the current device (non-blocking, default priority) created on
// first use and kept until the process ends, with a pair of events.  The caller
// holds `lock()` from the fork until the join is enqueued, so concurrent callers
// do not interleave their event records.
struct SideStream {
    hipStream_t side;
    hipEvent_t fork, join;
};
int side_stream(SideStream *&out);
std::mutex &side_stream_mutex();

// s_waitcnt immediate (gfx9 encoding) that waits until at most n vector-memory
// operations are outstanding and leaves the other counters unconstrained:
// vmcnt is split over bits [3:0] and [15:14], expcnt is bits [6:4], lgkmcnt [11:8]
constexpr int waitcnt_vm(int n) { return (n & 15) | ((n >> 4) << 14) | 0x70 | 0xF00; }

inline int launch_status(const char *what) {
    hipError_t err = hipGetLastError();
    if (err != hipSuccess) return fail(QPAM_ERR_HIP, "%s launch failed: %s", what, hipGetErrorString(err));
    return QPAM_OK;
}

// Runs on_side(side) and on_main(stream) concurrently, both after the work already
// queued on `stream`; `stream` continues after both (event fork / join, which HIP
// graph capture of `stream` follows).  Each callable enqueues launches and
// returns a status.
template <typename FS, typename FM>
int fork_join(hipStream_t stream, FS &&on_side, FM &&on_main) {
    std::lock_guard<std::mutex> lock(side_stream_mutex());
    SideStream *ss = nullptr;
    int st = side_stream(ss);
    if (st) return st;
    if (hipEventRecord(ss->fork, stream) != hipSuccess || hipStreamWaitEvent(ss->side, ss->fork, 0) != hipSuccess)
        return fail(QPAM_ERR_HIP, "fork_join: fork failed");
    const int st_side = on_side(ss->side);
    const int st_main = on_main(stream);
    // join even after a failed launch, so `stream` never runs ahead of side work
    if (hipEventRecord(ss->join, ss->side) != hipSuccess || hipStreamWaitEvent(stream, ss->join, 0) != hipSuccess)
        return fail(QPAM_ERR_HIP, "fork_join: join failed");
    return st_side ? st_side : st_main;
}


// ------------------------------------------------------------- vectors -----
typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned short ushortx8 __attribute__((ext_vector_type(8)));
typedef unsigned short ushortx4 __attribute__((ext_vector_type(4)));
typedef unsigned uintx4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_to_f32(unsigned short u) {
    return __uint_as_float(((unsigned int)u) << 16);
}

// round-to-nearest-even float -> bf16 bits (finite inputs)
__device__ __forceinline__ unsigned short f32_to_bf16(float f) {
    unsigned int u = __float_as_uint(f);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (unsigned short)(u >> 16);
}

// (lo, hi) -> two bf16 in one dword (hardware round-to-nearest-even conversion)
__device__ __forceinline__ unsigned pack_bf16x2(float lo, float hi) {
    return __builtin_bit_cast(unsigned, __builtin_convertvector(floatx2{lo, hi}, bf16x2));
}

// DPP lane permutations (quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror,
// row_mirror) and reductions over the 16 lanes of a DPP row: every lane of the
// row ends with the result.  Four steps: pairs, quads, halves, rows.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i(int x) {
    return __builtin_amdgcn_update_dpp(0, x, CTRL, 0xF, 0xF, false);
}
__device__ __forceinline__ float row16_max(float x) {
    x = fmaxf(x, dpp_f<0xB1>(x));
    x = fmaxf(x, dpp_f<0x4E>(x));
    x = fmaxf(x, dpp_f<0x141>(x));
    return fmaxf(x, dpp_f<0x140>(x));
}
__device__ __forceinline__ float row16_sum(float x) {
    x += dpp_f<0xB1>(x);
    x += dpp_f<0x4E>(x);
    x += dpp_f<0x141>(x);
    return x + dpp_f<0x140>(x);
}
__device__ __forceinline__ int row16_min(int x) {
    x = min(x, dpp_i<0xB1>(x));
    x = min(x, dpp_i<0x4E>(x));
    x = min(x, dpp_i<0x141>(x));
    return min(x, dpp_i<0x140>(x));
}

template <typename T> struct Elem;
template <> struct Elem<float> {
    __device__ __forceinline__ static float load(const float *p) { return *p; }
};
template <> struct Elem<unsigned short> {
    __device__ __forceinline__ static float load(const unsigned short *p) { return bf16_to_f32(*p); }
};

}  // namespace qpam
