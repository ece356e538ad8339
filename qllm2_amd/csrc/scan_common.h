// Shared pieces of the chunked PAM scan kernels (forward and backward).
#pragma once

#include <type_traits>

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

// Register-staged tile copies: every global load of a tile is issued before any
// LDS store, so a block waits for one memory latency per batch of tiles rather
// than one per load.  fp32 [ROWS x 64] tile: ROWS/16 float4 per thread.
template <int ROWS>
struct F32Tile {
    float4 v[ROWS / 16];
};

template <int ROWS>
__device__ __forceinline__ void tile_load(F32Tile<ROWS> &t, const float *base, int64_t st, int valid) {
#pragma unroll
    for (int i = 0; i < ROWS / 16; ++i) {
        const int idx = threadIdx.x + i * THREADS, r = idx >> 4, c4 = idx & 15;
        t.v[i] = (r < valid) ? *reinterpret_cast<const float4 *>(base + (int64_t)r * st + 4 * c4)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}

template <int ROWS>
__device__ __forceinline__ void tile_store(float *lds, const F32Tile<ROWS> &t, float scale) {
#pragma unroll
    for (int i = 0; i < ROWS / 16; ++i) {
        const int idx = threadIdx.x + i * THREADS, r = idx >> 4, c4 = idx & 15;
        float *dst = lds + r * P + 4 * c4;
        *reinterpret_cast<float4 *>(dst) =
            make_float4(t.v[i].x * scale, t.v[i].y * scale, t.v[i].z * scale, t.v[i].w * scale);
    }
}

// Stage N [C x 64] tiles of element type Tin into fp32 LDS (pitch P), scaled.
// fp32 sources are copied through registers with all loads in flight at once.
template <typename Tin, int C, int N>
__device__ __forceinline__ void stage_tiles(float *const (&dst)[N], const Tin *const (&src)[N],
                                            const int64_t (&st)[N], const float (&scale)[N], int valid) {
    if constexpr (std::is_same<Tin, float>::value) {
        F32Tile<C> t[N];
#pragma unroll
        for (int i = 0; i < N; ++i) tile_load<C>(t[i], src[i], st[i], valid);
#pragma unroll
        for (int i = 0; i < N; ++i) tile_store<C>(dst[i], t[i], scale[i]);
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) load_tile<Tin>(dst[i], src[i], st[i], C, valid, scale[i]);
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

// Sequential state scans: float4 per thread and blocks per (m, b, h) state.
constexpr int SCAN_EPT = 2;
constexpr int SCAN_BLOCKS = (2 * 64 * 64 / 4) / (THREADS * SCAN_EPT);
static_assert(SCAN_BLOCKS * THREADS * SCAN_EPT * 4 == 2 * 64 * 64, "scan tiling");

// Factorised decay.  When every log(gamma + 1e-6) of a chunk is <= 0, the fp32
// prefix sums L are non-increasing (rounding is monotone), so for s <= t
// min(L_t - L_s, 0) = L_t - L_s and no entry is clamped; if also
// L_last >= -FACTOR_RANGE, exp(L_t) and exp(-L_s) are finite and
// D[t,s] = exp(L_t) exp(-L_s) needs no per-element exponential.
constexpr float FACTOR_RANGE = 80.f;

// chunk_log_prefix plus that test for one state (wave-uniform result).
__device__ __forceinline__ float chunk_log_prefix_ok(const float *g, int64_t gs, int valid, int lane, bool &ok) {
    float x = (lane < valid) ? logf(g[(int64_t)lane * gs] + LOG_EPS) : 0.f;
    const bool pos = x > 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        float y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    ok = !__any(pos) && __shfl(x, 63) >= -FACTOR_RANGE;
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

__device__ __forceinline__ ushortx4 to_bf16x4(float4 v) {
    return ushortx4{f32_to_bf16(v.x), f32_to_bf16(v.y), f32_to_bf16(v.z), f32_to_bf16(v.w)};
}

// gfx950 LDS transpose read (ds_read_b64_tr_b16).  Within each group of 16
// lanes, lane 4a+b receives element b of the 8-byte chunks addressed by lanes
// 4e+a (e = 0..3), so 16 lanes addressing a 4 x 16 block of a row-major bf16
// tile receive its columns.
typedef short shortx4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ shortx4 lds_read_tr(const unsigned short *p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) shortx4 *)p);
}

// MFMA operand fragment (8 k values per lane) of a natural row-major [k][n]
// bf16 LDS tile (pitch PB) for a contraction over its rows: lane l16 of each
// 16-lane group receives rows r0..r0+3 then r1..r1+3 of column col0 + l16.  The
// caller folds the lane group into r0/r1; all 64 lanes must execute it.
__device__ __forceinline__ bf16x8 ld_tr(const unsigned short *tile, int r0, int r1, int col0, int pitch = PB) {
    const int l16 = threadIdx.x & 15;
    const unsigned short *p = tile + (l16 >> 2) * pitch + col0 + 4 * (l16 & 3);
    const shortx4 lo = lds_read_tr(p + r0 * pitch), hi = lds_read_tr(p + r1 * pitch);
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// One 16x16 accumulator tile of a complex matrix (element (4g + r, l16) of lane
// 16g + l16) -> rows row0.., columns col0.. of two bf16 planes with row pitch
// PITCH (D in global memory, PB in LDS).  Adjacent lanes swap one row pair
// element (DPP quad_perm [1,0,3,2]) so that each lane writes two consecutive
// columns of one row: a 4-byte store per plane instead of two 2-byte stores.
template <int PITCH = D>
__device__ __forceinline__ void acc_store_bf_pairs(unsigned short *dre, unsigned short *dim, const floatx4 &re,
                                                   const floatx4 &im, int row0, int col0) {
    const int lane = threadIdx.x & 63, l16 = lane & 15, g = lane >> 4;
    const bool odd = l16 & 1;
#pragma unroll
    for (int q = 0; q < 2; ++q) {
        const unsigned p0 = pack_bf16x2(re[2 * q], im[2 * q]), p1 = pack_bf16x2(re[2 * q + 1], im[2 * q + 1]);
        const unsigned keep = odd ? p1 : p0, send = odd ? p0 : p1;
        const unsigned recv = (unsigned)__builtin_amdgcn_update_dpp(0, (int)send, 0xB1, 0xF, 0xF, false);
        const unsigned lo = odd ? recv : keep, hi = odd ? keep : recv;  // columns (l16 & ~1) and +1
        const int row = row0 + 4 * g + 2 * q + (odd ? 1 : 0), col = col0 + (l16 & ~1);
        *reinterpret_cast<unsigned *>(dre + row * PITCH + col) = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
        *reinterpret_cast<unsigned *>(dim + row * PITCH + col) = __builtin_amdgcn_perm(hi, lo, 0x07060302u);
    }
}

// State passes: blocks of PASS_THREADS threads (4 waves) walk the chunks of one
// state; the state's 64 value rows are split over PASS_SPLIT blocks (rows of the
// recurrence are independent, so a chain's halves never exchange data).  Chunk
// tiles travel global -> registers -> LDS in natural layout (thread idx: row
// idx / (CW / 8) and 16-byte column chunk idx % (CW / 8) for bf16, float4 chunks
// for fp32).  Loads clamp rows at and beyond `valid` to
// row valid-1, for consumers that weight those rows by zero: with no conditional
// register initialisation, a load in a software pipeline does not wait for the
// previous load into the same registers.  (Clang vector types: a uint4 / float4
// struct copy from memory would keep the register sets in scratch.)
constexpr int PASS_THREADS = 256;

// The 16-row tile wave w of a 4-wave chunk block works on.  Causal tiles differ
// in cost (the last query tile of a chunk does four times the score work of the
// first, and the reverse for key tiles) and a CU holds two such blocks, typically
// of adjacent dispatch rounds of 256 blocks: alternate rounds take the tiles a
// half-turn apart, so the heavy tiles of the two blocks do not share a SIMD.
// Every tile is computed the same way whichever wave takes it.
__device__ __forceinline__ int causal_tile(int w) {
    const int lin = blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z);
    return (w + 2 * ((lin >> 8) & 1)) & 3;
}
constexpr int PASS_SPLIT = 2;

// bf16 path with 64-step chunks: the chunks of a chain are grouped in segments
// of SEG chunks.  Segment increments are formed chunk-parallel, a short
// elementwise scan links the segments, and the chunk kernels carry the state
// (or its gradient) through the chunks of one segment in registers.
constexpr int SEG = 4;
constexpr int SEG_THREADS = 512;  // 8 waves per segment block

// Forward-workspace offsets (in floats) of the segment data: segment totals
// [chains][n_segs], weights wfwd and wbwd [chains][n * 64].
struct SegLayout {
    int n_segs;
    int64_t segtot, wfwd, wbwd, wgr, wgi;
};
SegLayout seg_layout(const qpam_scan_args &a);
// 64-row tiles of CW columns (64, or a 32-column half at column c0) held in
// registers, NT threads of the block; 16-byte loads along the row.
template <int NT, int CW = 64>
struct BfTileRegs {
    uintx4 v[8 * CW / NT];
};
template <int NT, int CW = 64>
struct F32TileRegs {
    floatx4 v[16 * CW / NT];
};
template <int NT, int CW = 64>
__device__ __forceinline__ void tile_load_bf(BfTileRegs<NT, CW> &t, const unsigned short *src, int64_t st, int valid,
                                             int c0 = 0) {
#pragma unroll
    for (int i = 0; i < 8 * CW / NT; ++i) {
        const int idx = threadIdx.x + i * NT;
        const int r = min(idx / (CW / 8), valid - 1), c8 = idx % (CW / 8);
        t.v[i] = *reinterpret_cast<const uintx4 *>(src + (int64_t)r * st + c0 + 8 * c8);
    }
}
template <int NT, int CW = 64>
__device__ __forceinline__ void tile_store_bf(unsigned short *lds, const BfTileRegs<NT, CW> &t, int c0 = 0) {
#pragma unroll
    for (int i = 0; i < 8 * CW / NT; ++i) {
        const int idx = threadIdx.x + i * NT;
        *reinterpret_cast<uintx4 *>(lds + (idx / (CW / 8)) * PB + c0 + 8 * (idx % (CW / 8))) = t.v[i];
    }
}
// The same store with row r scaled by lane r's `row_scale` (of the calling wave),
// in fp32, rounded once to bf16.
template <int NT, int CW = 64>
__device__ __forceinline__ void tile_store_bf_rowscaled(unsigned short *lds, const BfTileRegs<NT, CW> &t,
                                                        float row_scale, int c0 = 0) {
#pragma unroll
    for (int i = 0; i < 8 * CW / NT; ++i) {
        const int idx = threadIdx.x + i * NT, r = idx / (CW / 8);
        const float f = __shfl(row_scale, r);
        const floatx8 x = to_f(__builtin_bit_cast(bf16x8, t.v[i])) * f;
        *reinterpret_cast<bf16x8 *>(lds + r * PB + c0 + 8 * (idx % (CW / 8))) = to_bf(x);
    }
}
template <int NT, int CW = 64>
__device__ __forceinline__ void tile_load_f32(F32TileRegs<NT, CW> &t, const float *src, int64_t st, int valid,
                                              int c0 = 0) {
#pragma unroll
    for (int i = 0; i < 16 * CW / NT; ++i) {
        const int idx = threadIdx.x + i * NT;
        const int r = min(idx / (CW / 4), valid - 1), c4 = idx % (CW / 4);
        t.v[i] = *reinterpret_cast<const floatx4 *>(src + (int64_t)r * st + c0 + 4 * c4);
    }
}
template <int NT>
__device__ __forceinline__ void tile_store_f32_as_bf(unsigned short *lds, const F32TileRegs<NT> &t) {
#pragma unroll
    for (int i = 0; i < 1024 / NT; ++i) {
        const int idx = threadIdx.x + i * NT;
        const uint2 u = make_uint2(pack_bf16x2(t.v[i][0], t.v[i][1]), pack_bf16x2(t.v[i][2], t.v[i][3]));
        *reinterpret_cast<uint2 *>(lds + (idx >> 4) * PB + 4 * (idx & 15)) = u;
    }
}

// Register-staged bf16 / fp32 -> bf16 tile copies (all loads of a batch are
// issued before the LDS stores).  TR selects the thread -> element mapping that
// suits the transposed store (consecutive lanes on consecutive rows).
struct B16Regs {
    uint4 v[2];
};
template <bool TR>
__device__ __forceinline__ void regs_load_bf(B16Regs &t, const unsigned short *src, int64_t st, int valid) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int idx = threadIdx.x + i * THREADS;
        const int r = TR ? (idx & 63) : (idx >> 3), c8 = TR ? (idx >> 6) : (idx & 7);
        t.v[i] = (r < valid) ? *reinterpret_cast<const uint4 *>(src + (int64_t)r * st + 8 * c8) : make_uint4(0, 0, 0, 0);
    }
}
template <bool TR>
__device__ __forceinline__ void regs_store_bf(unsigned short *lds, const B16Regs &t) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int idx = threadIdx.x + i * THREADS;
        const int r = TR ? (idx & 63) : (idx >> 3), c8 = TR ? (idx >> 6) : (idx & 7);
        if (TR) {
            const ushortx8 u = __builtin_bit_cast(ushortx8, t.v[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) lds[(8 * c8 + e) * PB + r] = u[e];
        } else {
            *reinterpret_cast<uint4 *>(lds + r * PB + 8 * c8) = t.v[i];
        }
    }
}
struct F32Regs {
    float4 v[4];
};
template <bool TR>
__device__ __forceinline__ void regs_load_f32(F32Regs &t, const float *src, int64_t st, int valid) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = threadIdx.x + i * THREADS;
        const int r = TR ? (idx & 63) : (idx >> 4), c4 = TR ? (idx >> 6) : (idx & 15);
        t.v[i] = (r < valid) ? *reinterpret_cast<const float4 *>(src + (int64_t)r * st + 4 * c4)
                             : make_float4(0.f, 0.f, 0.f, 0.f);
    }
}
template <bool TR>
__device__ __forceinline__ void regs_store_f32_as_bf(unsigned short *lds, const F32Regs &t) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int idx = threadIdx.x + i * THREADS;
        const int r = TR ? (idx & 63) : (idx >> 4), c4 = TR ? (idx >> 6) : (idx & 15);
        const float f[4] = {t.v[i].x, t.v[i].y, t.v[i].z, t.v[i].w};
        if (TR) {
#pragma unroll
            for (int e = 0; e < 4; ++e) lds[(4 * c4 + e) * PB + r] = f32_to_bf16(f[e]);
        } else {
            const ushortx4 u = {f32_to_bf16(f[0]), f32_to_bf16(f[1]), f32_to_bf16(f[2]), f32_to_bf16(f[3])};
            *reinterpret_cast<ushortx4 *>(lds + r * PB + 4 * c4) = u;
        }
    }
}

// Batched variants: N tiles, tile i stored transposed when bit i of TRMASK is set.
template <int N, unsigned TRMASK>
__device__ __forceinline__ void stage_bf(unsigned short *const (&dst)[N], const unsigned short *const (&src)[N],
                                         const int64_t (&st)[N], int valid) {
    B16Regs r[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if ((TRMASK >> i) & 1u) regs_load_bf<true>(r[i], src[i], st[i], valid);
        else regs_load_bf<false>(r[i], src[i], st[i], valid);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if ((TRMASK >> i) & 1u) regs_store_bf<true>(dst[i], r[i]);
        else regs_store_bf<false>(dst[i], r[i]);
    }
}
template <int N, unsigned TRMASK>
__device__ __forceinline__ void stage_f32_as_bf(unsigned short *const (&dst)[N], const float *const (&src)[N],
                                                const int64_t (&st)[N], int valid) {
    F32Regs r[N];
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if ((TRMASK >> i) & 1u) regs_load_f32<true>(r[i], src[i], st[i], valid);
        else regs_load_f32<false>(r[i], src[i], st[i], valid);
    }
#pragma unroll
    for (int i = 0; i < N; ++i) {
        if ((TRMASK >> i) & 1u) regs_store_f32_as_bf<true>(dst[i], r[i]);
        else regs_store_f32_as_bf<false>(dst[i], r[i]);
    }
}

// NB bf16 tiles and NF fp32 tiles (stored as bf16) in one batch of loads.
template <int NB, unsigned TRB, int NF, unsigned TRF>
__device__ __forceinline__ void stage_mixed(unsigned short *const (&bdst)[NB], const unsigned short *const (&bsrc)[NB],
                                            const int64_t (&bst)[NB], unsigned short *const (&fdst)[NF],
                                            const float *const (&fsrc)[NF], const int64_t (&fst)[NF], int valid) {
    B16Regs rb[NB];
    F32Regs rf[NF];
#pragma unroll
    for (int i = 0; i < NF; ++i) {
        if ((TRF >> i) & 1u) regs_load_f32<true>(rf[i], fsrc[i], fst[i], valid);
        else regs_load_f32<false>(rf[i], fsrc[i], fst[i], valid);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if ((TRB >> i) & 1u) regs_load_bf<true>(rb[i], bsrc[i], bst[i], valid);
        else regs_load_bf<false>(rb[i], bsrc[i], bst[i], valid);
    }
#pragma unroll
    for (int i = 0; i < NF; ++i) {
        if ((TRF >> i) & 1u) regs_store_f32_as_bf<true>(fdst[i], rf[i]);
        else regs_store_f32_as_bf<false>(fdst[i], rf[i]);
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        if ((TRB >> i) & 1u) regs_store_bf<true>(bdst[i], rb[i]);
        else regs_store_bf<false>(bdst[i], rb[i]);
    }
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
