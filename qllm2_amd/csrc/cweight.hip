// Complex linear weights as one real GEMM operand, and the backward that turns
// that operand's gradient back into the complex weights' gradients.
//
// ComplexLinear (v11/complex_ops.py:146-172) computes re = Wr xr - Wi xi,
// im = Wi xr + Wr xi.  The PAM layer runs its projections as single real GEMMs
// over a packed weight W (qkv_proj and dt_proj in front of the prologue, o_proj
// after the scan, v11/model.py:280, 636, 836).  Packing W took five to seven
// small torch passes per projection (negation, stacks, concatenations) and the
// backward as many again to split W's gradient; here each direction is one
// launch, and the backward also sums the row slices of a sliced weight-gradient
// product in fp32 in a fixed order and rounds once to the weights' dtype.
//
// Layouts (p = output part, q = input part, 0 = re, 1 = im; the value at
// (p, q) is wr, -wi, wi, wr for (0,0), (0,1), (1,0), (1,1)):
//   QPAM_CW_IN:  W[p R + r][2 c + q]   (input interleaved per feature, the
//                outputs as a real then an imaginary block), then `tail_rows`
//                real rows W[2R + h][2 c + q] = tail[h][q C + c] (an nn.Linear
//                over [xr | xi]), then `zero_rows` rows of zeros;
//   QPAM_CW_OUT: W[2 r + p][q C + c]   (input as a real then an imaginary
//                block, outputs interleaved per feature).
// Each thread moves eight consecutive columns of W (16 bytes of bf16).

#include "common.h"

namespace qpam {
namespace {

constexpr int CW_THREADS = 256;

template <typename T> struct V;
template <> struct V<float> {
    template <int N>
    __device__ __forceinline__ static void load(const void *p, int64_t i, float (&x)[N]) {
        const float *f = static_cast<const float *>(p) + i;
#pragma unroll
        for (int k = 0; k < N; k += 4) {
            const float4 v = *reinterpret_cast<const float4 *>(f + k);
            x[k] = v.x, x[k + 1] = v.y, x[k + 2] = v.z, x[k + 3] = v.w;
        }
    }
    template <int N>
    __device__ __forceinline__ static void store(void *p, int64_t i, const float (&x)[N]) {
        float *f = static_cast<float *>(p) + i;
#pragma unroll
        for (int k = 0; k < N; k += 4) *reinterpret_cast<float4 *>(f + k) = make_float4(x[k], x[k + 1], x[k + 2], x[k + 3]);
    }
};
template <> struct V<unsigned short> {
    template <int N>
    __device__ __forceinline__ static void load(const void *p, int64_t i, float (&x)[N]) {
        const unsigned short *h = static_cast<const unsigned short *>(p) + i;
        if constexpr (N == 4) {
            const uint2 v = *reinterpret_cast<const uint2 *>(h);
            x[0] = __uint_as_float(v.x << 16), x[1] = __uint_as_float(v.x & 0xffff0000u);
            x[2] = __uint_as_float(v.y << 16), x[3] = __uint_as_float(v.y & 0xffff0000u);
        } else {
#pragma unroll
            for (int k = 0; k < N; k += 8) {
                const uint4 v = *reinterpret_cast<const uint4 *>(h + k);
                const unsigned u[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    x[k + 2 * j] = __uint_as_float(u[j] << 16), x[k + 2 * j + 1] = __uint_as_float(u[j] & 0xffff0000u);
            }
        }
    }
    template <int N>
    __device__ __forceinline__ static void store(void *p, int64_t i, const float (&x)[N]) {
        unsigned short *h = static_cast<unsigned short *>(p) + i;
        if constexpr (N == 4) {
            *reinterpret_cast<uint2 *>(h) = make_uint2(pack_bf16x2(x[0], x[1]), pack_bf16x2(x[2], x[3]));
        } else {
#pragma unroll
            for (int k = 0; k < N; k += 8)
                *reinterpret_cast<uint4 *>(h + k) = make_uint4(pack_bf16x2(x[k], x[k + 1]), pack_bf16x2(x[k + 2], x[k + 3]),
                                                               pack_bf16x2(x[k + 4], x[k + 5]), pack_bf16x2(x[k + 6], x[k + 7]));
        }
    }
};

struct CwParams {
    int64_t R, C, tail_rows, zero_rows, ldw, slice_stride;
    int slices;
    const void *wr, *wi, *tail, *g;
    void *w, *g_wr, *g_wi, *g_tail;
};

// rows of W the layout has
__host__ __device__ inline int64_t w_rows(const CwParams &p, int layout) {
    return layout == QPAM_CW_IN ? 2 * p.R + p.tail_rows + p.zero_rows : 2 * p.R;
}

template <typename T, int LAYOUT>
__global__ void __launch_bounds__(CW_THREADS) cw_pack_kernel(CwParams p) {
    const int64_t per_row = 2 * p.C / 8;
    const int64_t idx = (int64_t)blockIdx.x * CW_THREADS + threadIdx.x;
    if (idx >= w_rows(p, LAYOUT) * per_row) return;
    const int64_t row = idx / per_row, col0 = 8 * (idx % per_row);
    float o[8];
    if constexpr (LAYOUT == QPAM_CW_IN) {
        const int64_t c0 = col0 / 2;  // four features, (re, im) input columns each
        if (row < 2 * p.R) {
            const int64_t r = row % p.R;
            const bool im_out = row >= p.R;
            float a[4], b[4];
            V<T>::template load<4>(p.wr, r * p.C + c0, a);
            V<T>::template load<4>(p.wi, r * p.C + c0, b);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                o[2 * k] = im_out ? b[k] : a[k];       // q = re: wr (re out), wi (im out)
                o[2 * k + 1] = im_out ? a[k] : -b[k];  // q = im: -wi (re out), wr (im out)
            }
        } else if (row < 2 * p.R + p.tail_rows) {
            const int64_t h = row - 2 * p.R;
            float a[4], b[4];
            V<T>::template load<4>(p.tail, h * 2 * p.C + c0, a);
            V<T>::template load<4>(p.tail, h * 2 * p.C + p.C + c0, b);
#pragma unroll
            for (int k = 0; k < 4; ++k) o[2 * k] = a[k], o[2 * k + 1] = b[k];
        } else {
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = 0.f;
        }
    } else {
        const int64_t r = row >> 1;
        const bool im_out = row & 1, im_in = col0 >= p.C;
        const int64_t c0 = im_in ? col0 - p.C : col0;
        // (re out, re in) wr, (re out, im in) -wi, (im out, re in) wi, (im out, im in) wr
        const bool use_wi = im_out != im_in;
        V<T>::template load<8>(use_wi ? p.wi : p.wr, r * p.C + c0, o);
        if (use_wi && !im_out) {
#pragma unroll
            for (int k = 0; k < 8; ++k) o[k] = -o[k];
        }
    }
    V<T>::template store<8>(p.w, row * p.ldw + col0, o);
}

// N consecutive elements of the gradient of W at (row, col): the sum of the
// slices, in slice order
template <typename G, int N>
__device__ __forceinline__ void g_load(const CwParams &p, int64_t row, int64_t col, float (&x)[N]) {
    V<G>::template load<N>(p.g, row * p.ldw + col, x);
    int s = 1;
    for (; s + 2 <= p.slices; s += 2) {  // two slices' loads in flight, added in slice order
        float y[2][N];
#pragma unroll
        for (int u = 0; u < 2; ++u) V<G>::template load<N>(p.g, (s + u) * p.slice_stride + row * p.ldw + col, y[u]);
#pragma unroll
        for (int u = 0; u < 2; ++u)
#pragma unroll
            for (int k = 0; k < N; ++k) x[k] += y[u][k];
    }
    for (; s < p.slices; ++s) {
        float y[N];
        V<G>::template load<N>(p.g, s * p.slice_stride + row * p.ldw + col, y);
#pragma unroll
        for (int k = 0; k < N; ++k) x[k] += y[k];
    }
}

// one thread per four (IN) or eight (OUT) consecutive features of a weight row,
// or per four features of a tail row
template <typename T, typename G, int LAYOUT>
__global__ void __launch_bounds__(CW_THREADS) cw_unpack_kernel(CwParams p) {
    constexpr int F = LAYOUT == QPAM_CW_IN ? 4 : 8;
    const int64_t per_row = p.C / F;
    const int64_t idx = (int64_t)blockIdx.x * CW_THREADS + threadIdx.x;
    const int64_t rows = p.R + (LAYOUT == QPAM_CW_IN ? p.tail_rows : 0);
    if (idx >= rows * per_row) return;
    const int64_t r = idx / per_row, c0 = F * (idx % per_row);
    if constexpr (LAYOUT == QPAM_CW_IN) {
        float u[8], v[8];
        if (r < p.R) {
            g_load<G, 8>(p, r, 2 * c0, u);        // re out: (wr, -wi) per feature
            g_load<G, 8>(p, p.R + r, 2 * c0, v);  // im out: (wi, wr)
            float gr[4], gi[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                gr[k] = u[2 * k] + v[2 * k + 1];
                gi[k] = v[2 * k] - u[2 * k + 1];
            }
            V<T>::template store<4>(p.g_wr, r * p.C + c0, gr);
            V<T>::template store<4>(p.g_wi, r * p.C + c0, gi);
        } else {
            const int64_t h = r - p.R;
            g_load<G, 8>(p, 2 * p.R + h, 2 * c0, u);
            float a[4], b[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) a[k] = u[2 * k], b[k] = u[2 * k + 1];
            V<T>::template store<4>(p.g_tail, h * 2 * p.C + c0, a);
            V<T>::template store<4>(p.g_tail, h * 2 * p.C + p.C + c0, b);
        }
    } else {
        float a[8], b[8], c[8], d[8];
        g_load<G, 8>(p, 2 * r, c0, a);             // (re out, re in): wr
        g_load<G, 8>(p, 2 * r, p.C + c0, b);       // (re out, im in): -wi
        g_load<G, 8>(p, 2 * r + 1, c0, c);         // (im out, re in): wi
        g_load<G, 8>(p, 2 * r + 1, p.C + c0, d);   // (im out, im in): wr
        float gr[8], gi[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            gr[k] = a[k] + d[k];
            gi[k] = c[k] - b[k];
        }
        V<T>::template store<8>(p.g_wr, r * p.C + c0, gr);
        V<T>::template store<8>(p.g_wi, r * p.C + c0, gi);
    }
}

// out[i] = sum over s of in[s * stride + i] (fp32, slice order), eight
// consecutive elements per thread
template <typename TI, typename TO>
__global__ void __launch_bounds__(CW_THREADS) slice_sum_kernel(int slices, int64_t n8, int64_t stride, const void *in,
                                                               void *out) {
    const int64_t i = (int64_t)blockIdx.x * CW_THREADS + threadIdx.x;
    if (i >= n8) return;
    float x[8];
    V<TI>::template load<8>(in, 8 * i, x);
    int s = 1;
    for (; s + 4 <= slices; s += 4) {  // four slices' loads in flight, added in slice order
        float y[4][8];
#pragma unroll
        for (int u = 0; u < 4; ++u) V<TI>::template load<8>(in, (int64_t)(s + u) * stride + 8 * i, y[u]);
#pragma unroll
        for (int u = 0; u < 4; ++u)
#pragma unroll
            for (int k = 0; k < 8; ++k) x[k] += y[u][k];
    }
    for (; s < slices; ++s) {
        float y[8];
        V<TI>::template load<8>(in, (int64_t)s * stride + 8 * i, y);
#pragma unroll
        for (int k = 0; k < 8; ++k) x[k] += y[k];
    }
    V<TO>::template store<8>(out, 8 * i, x);
}

bool aligned(const void *p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

int check_common(const qpam_cweight_args *a, const char *who) {
    QPAM_REQUIRE(a != nullptr, "%s: null arguments", who);
    QPAM_REQUIRE(a->dtype == QPAM_F32 || a->dtype == QPAM_BF16, "%s: dtype must be QPAM_F32 or QPAM_BF16", who);
    QPAM_REQUIRE(a->layout == QPAM_CW_IN || a->layout == QPAM_CW_OUT, "%s: layout must be QPAM_CW_IN or QPAM_CW_OUT",
                 who);
    QPAM_REQUIRE(a->R > 0 && a->C > 0, "%s: R, C must be positive", who);
    QPAM_REQUIRE(a->C % (a->layout == QPAM_CW_IN ? 4 : 8) == 0, "%s: C = %lld must be a multiple of %d", who,
                 (long long)a->C, a->layout == QPAM_CW_IN ? 4 : 8);
    QPAM_REQUIRE(a->tail_rows >= 0 && a->zero_rows >= 0, "%s: negative tail_rows or zero_rows", who);
    QPAM_REQUIRE(a->layout == QPAM_CW_IN || (a->tail_rows == 0 && a->zero_rows == 0),
                 "%s: tail and zero rows exist only in layout QPAM_CW_IN", who);
    QPAM_REQUIRE(a->ldw >= 2 * a->C && a->ldw % 8 == 0, "%s: ldw %lld must be >= 2 C and a multiple of 8", who,
                 (long long)a->ldw);
    return QPAM_OK;
}

CwParams params(const qpam_cweight_args *a) {
    CwParams p;
    p.R = a->R, p.C = a->C, p.tail_rows = a->tail_rows, p.zero_rows = a->zero_rows, p.ldw = a->ldw;
    p.slices = a->slices > 0 ? a->slices : 1;
    p.slice_stride = a->slice_stride;
    p.wr = a->wr, p.wi = a->wi, p.tail = a->tail, p.g = a->g;
    p.w = a->w, p.g_wr = a->g_wr, p.g_wi = a->g_wi, p.g_tail = a->g_tail;
    return p;
}

dim3 grid_for(int64_t threads) { return dim3((unsigned)((threads + CW_THREADS - 1) / CW_THREADS)); }

}  // namespace
}  // namespace qpam

extern "C" int qpam_cweight_pack(const qpam_cweight_args *a, void *stream) {
    using namespace qpam;
    int st = check_common(a, "qpam_cweight_pack");
    if (st) return st;
    QPAM_REQUIRE(a->wr && a->wi && a->w && aligned(a->wr, 16) && aligned(a->wi, 16) && aligned(a->w, 16),
                 "qpam_cweight_pack: 16-byte aligned wr, wi and w required");
    QPAM_REQUIRE(a->tail_rows == 0 || (a->tail && aligned(a->tail, 16)),
                 "qpam_cweight_pack: 16-byte aligned tail required with tail_rows");
    const CwParams p = params(a);
    const int64_t threads = w_rows(p, a->layout) * (2 * p.C / 8);
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool f = a->dtype == QPAM_F32;
    if (a->layout == QPAM_CW_IN) {
        if (f) hipLaunchKernelGGL((cw_pack_kernel<float, QPAM_CW_IN>), grid_for(threads), dim3(CW_THREADS), 0, s, p);
        else hipLaunchKernelGGL((cw_pack_kernel<unsigned short, QPAM_CW_IN>), grid_for(threads), dim3(CW_THREADS), 0, s, p);
    } else {
        if (f) hipLaunchKernelGGL((cw_pack_kernel<float, QPAM_CW_OUT>), grid_for(threads), dim3(CW_THREADS), 0, s, p);
        else hipLaunchKernelGGL((cw_pack_kernel<unsigned short, QPAM_CW_OUT>), grid_for(threads), dim3(CW_THREADS), 0, s, p);
    }
    return launch_status("cw_pack_kernel");
}

extern "C" int qpam_cweight_unpack(const qpam_cweight_args *a, void *stream) {
    using namespace qpam;
    int st = check_common(a, "qpam_cweight_unpack");
    if (st) return st;
    QPAM_REQUIRE(a->g_dtype == QPAM_F32 || a->g_dtype == QPAM_BF16, "qpam_cweight_unpack: g_dtype must be QPAM_F32 or QPAM_BF16");
    QPAM_REQUIRE(a->slices >= 1, "qpam_cweight_unpack: slices must be >= 1");
    const int64_t wsize = (2 * a->R + a->tail_rows + a->zero_rows) * a->ldw;
    QPAM_REQUIRE(a->slices == 1 || (a->slice_stride >= wsize && a->slice_stride % 8 == 0),
                 "qpam_cweight_unpack: slice_stride %lld must cover one W (%lld) and be a multiple of 8",
                 (long long)a->slice_stride, (long long)wsize);
    QPAM_REQUIRE(a->g && a->g_wr && a->g_wi && aligned(a->g, 16) && aligned(a->g_wr, 16) && aligned(a->g_wi, 16),
                 "qpam_cweight_unpack: 16-byte aligned g, g_wr and g_wi required");
    QPAM_REQUIRE(a->tail_rows == 0 || (a->g_tail && aligned(a->g_tail, 16)),
                 "qpam_cweight_unpack: 16-byte aligned g_tail required with tail_rows");
    const CwParams p = params(a);
    const int64_t threads = (p.R + (a->layout == QPAM_CW_IN ? p.tail_rows : 0)) * (p.C / (a->layout == QPAM_CW_IN ? 4 : 8));
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid = grid_for(threads), block(CW_THREADS);
    const bool ft = a->dtype == QPAM_F32, fg = a->g_dtype == QPAM_F32;
    using U = unsigned short;
    if (a->layout == QPAM_CW_IN) {
        if (ft && fg) hipLaunchKernelGGL((cw_unpack_kernel<float, float, QPAM_CW_IN>), grid, block, 0, s, p);
        else if (ft) hipLaunchKernelGGL((cw_unpack_kernel<float, U, QPAM_CW_IN>), grid, block, 0, s, p);
        else if (fg) hipLaunchKernelGGL((cw_unpack_kernel<U, float, QPAM_CW_IN>), grid, block, 0, s, p);
        else hipLaunchKernelGGL((cw_unpack_kernel<U, U, QPAM_CW_IN>), grid, block, 0, s, p);
    } else {
        if (ft && fg) hipLaunchKernelGGL((cw_unpack_kernel<float, float, QPAM_CW_OUT>), grid, block, 0, s, p);
        else if (ft) hipLaunchKernelGGL((cw_unpack_kernel<float, U, QPAM_CW_OUT>), grid, block, 0, s, p);
        else if (fg) hipLaunchKernelGGL((cw_unpack_kernel<U, float, QPAM_CW_OUT>), grid, block, 0, s, p);
        else hipLaunchKernelGGL((cw_unpack_kernel<U, U, QPAM_CW_OUT>), grid, block, 0, s, p);
    }
    return launch_status("cw_unpack_kernel");
}

extern "C" int qpam_slice_sum(int32_t in_dtype, int32_t out_dtype, int32_t slices, int64_t n, int64_t stride,
                              const void *in, void *out, void *stream) {
    using namespace qpam;
    QPAM_REQUIRE((in_dtype == QPAM_F32 || in_dtype == QPAM_BF16) && (out_dtype == QPAM_F32 || out_dtype == QPAM_BF16),
                 "qpam_slice_sum: dtypes must be QPAM_F32 or QPAM_BF16");
    QPAM_REQUIRE(slices >= 1 && n >= 0 && n % 8 == 0 && (slices == 1 || (stride >= n && stride % 8 == 0)),
                 "qpam_slice_sum: slices >= 1, n a multiple of 8, stride >= n and a multiple of 8");
    QPAM_REQUIRE(n == 0 || (in && out && aligned(in, 16) && aligned(out, 16)),
                 "qpam_slice_sum: 16-byte aligned in and out required");
    if (n == 0) return QPAM_OK;
    const int64_t n8 = n / 8;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid = grid_for(n8), block(CW_THREADS);
    using U = unsigned short;
    const bool fi = in_dtype == QPAM_F32, fo = out_dtype == QPAM_F32;
    if (fi && fo) hipLaunchKernelGGL((slice_sum_kernel<float, float>), grid, block, 0, s, slices, n8, stride, in, out);
    else if (fi) hipLaunchKernelGGL((slice_sum_kernel<float, U>), grid, block, 0, s, slices, n8, stride, in, out);
    else if (fo) hipLaunchKernelGGL((slice_sum_kernel<U, float>), grid, block, 0, s, slices, n8, stride, in, out);
    else hipLaunchKernelGGL((slice_sum_kernel<U, U>), grid, block, 0, s, slices, n8, stride, in, out);
    return launch_status("slice_sum_kernel");
}
