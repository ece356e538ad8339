// Complex elementwise layers on split-real [rows, dim, 2] tensors (interleaved
// re/im), forward and backward.
//
// Reference: the public API of v11/triton_kernels.py — fused_complex_norm
// (forward kernel :48-79, autograd backward :209-260), fused_mod_swish
// (:83-108, :263-304), fused_mod_relu (:112-135, :307-345), fused_cgu_gate
// (:139-166, :348-395); the PyTorch forms they replace are :489-520.  The
// backward formulas here are the closed forms of those autograd Functions.
//
// Layout and parallelism: every op is HBM-bound (a few flops per 8-byte complex
// element).  Forward elementwise ops run a flat grid-stride loop of complex
// elements (8-byte fp32 / 4-byte bf16 accesses, consecutive lanes on consecutive
// columns).  ComplexNorm (a row reduction) and the backward of the ops with
// per-column parameters run one wave per row, lanes over columns: the row sums
// use a wave reduction, and the parameter gradients (column sums over rows)
// accumulate in a per-wave LDS slice that each block folds in fixed order into
// a [block][dim] partial, summed over blocks by a second kernel — deterministic,
// no atomics.
#include <algorithm>
#include <mutex>

#include "common.h"

namespace qpam {
namespace cplx {
namespace {

constexpr int THREADS = 256;  // 4 waves
constexpr int WAVES = THREADS / 64;
constexpr int MAX_BLOCKS = 2048;  // row-kernel blocks (and column partials)
constexpr float MAG_EPS = 1e-8f;  // inside the sqrt and added to the magnitude, as the reference

// V consecutive complex elements starting at complex index e: V = 4 moves 16
// bytes (bf16) or 2 x 16 bytes (fp32) per lane; V = 1 for dims that are not a
// multiple of 4.
template <typename T, int V> struct CVec;
template <int V> struct CVec<float, V> {
    __device__ __forceinline__ static void load(const float *p, int64_t e, float (&re)[V], float (&im)[V]) {
        if constexpr (V == 4) {
            const float4 a = *reinterpret_cast<const float4 *>(p + 2 * e), b = *reinterpret_cast<const float4 *>(p + 2 * e + 4);
            re[0] = a.x, im[0] = a.y, re[1] = a.z, im[1] = a.w, re[2] = b.x, im[2] = b.y, re[3] = b.z, im[3] = b.w;
        } else {
            const float2 a = *reinterpret_cast<const float2 *>(p + 2 * e);
            re[0] = a.x, im[0] = a.y;
        }
    }
    __device__ __forceinline__ static void store(float *p, int64_t e, const float (&re)[V], const float (&im)[V]) {
        if constexpr (V == 4) {
            *reinterpret_cast<float4 *>(p + 2 * e) = make_float4(re[0], im[0], re[1], im[1]);
            *reinterpret_cast<float4 *>(p + 2 * e + 4) = make_float4(re[2], im[2], re[3], im[3]);
        } else {
            *reinterpret_cast<float2 *>(p + 2 * e) = make_float2(re[0], im[0]);
        }
    }
};
template <int V> struct CVec<unsigned short, V> {
    __device__ __forceinline__ static void load(const unsigned short *p, int64_t e, float (&re)[V], float (&im)[V]) {
        if constexpr (V == 4) {
            // rows are streamed once: nontemporal 16-byte loads and stores
            const uintx4 a = __builtin_nontemporal_load(reinterpret_cast<const uintx4 *>(p + 2 * e));
            const unsigned u[4] = {a[0], a[1], a[2], a[3]};
#pragma unroll
            for (int k = 0; k < 4; ++k) re[k] = __uint_as_float(u[k] << 16), im[k] = __uint_as_float(u[k] & 0xFFFF0000u);
        } else {
            const unsigned u = *reinterpret_cast<const unsigned *>(p + 2 * e);
            re[0] = __uint_as_float(u << 16), im[0] = __uint_as_float(u & 0xFFFF0000u);
        }
    }
    __device__ __forceinline__ static void store(unsigned short *p, int64_t e, const float (&re)[V],
                                                 const float (&im)[V]) {
        if constexpr (V == 4) {
            const uintx4 v = {pack_bf16x2(re[0], im[0]), pack_bf16x2(re[1], im[1]), pack_bf16x2(re[2], im[2]),
                              pack_bf16x2(re[3], im[3])};
            __builtin_nontemporal_store(v, reinterpret_cast<uintx4 *>(p + 2 * e));
        } else {
            *reinterpret_cast<unsigned *>(p + 2 * e) = pack_bf16x2(re[0], im[0]);
        }
    }
};

__device__ __forceinline__ float wave_sum(float x) {
    x = row16_sum(x);
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

// hardware square root / reciprocal (1 ulp): the magnitude is >= 1e-4, so no
// denormal operands reach them
__device__ __forceinline__ float magnitude(float re, float im) {
    return __builtin_amdgcn_sqrtf(re * re + im * im + MAG_EPS);
}
__device__ __forceinline__ float rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float sigmoidf(float x) { return rcp(1.f + __expf(-x)); }

struct Params {
    int64_t rows;
    int dim;
    float eps;
    const void *z, *up;
    const float *p0, *p1;
    void *out;
    const void *gout;
    void *gz, *gup;
    float *part;  // backward: [blocks][n_params][dim] column partials
};

// ------------------------------------------------------------------ forward --
template <typename T, int V>
__global__ void __launch_bounds__(THREADS) norm_fwd_kernel(Params p) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const T *z = (const T *)p.z;
    T *out = (T *)p.out;
    const int groups = p.dim / V;
    for (int64_t row = (int64_t)blockIdx.x * WAVES + w; row < p.rows; row += (int64_t)gridDim.x * WAVES) {
        const int64_t e0 = row * p.dim;
        float ss = 0.f;
        for (int j = lane; j < groups; j += 64) {
            float re[V], im[V];
            CVec<T, V>::load(z, e0 + V * j, re, im);
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const float m = magnitude(re[k], im[k]);
                ss += m * m;
            }
        }
        const float rms = sqrtf(wave_sum(ss) / p.dim + p.eps);
        for (int j = lane; j < groups; j += 64) {
            float re[V], im[V];
            CVec<T, V>::load(z, e0 + V * j, re, im);
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const float m = magnitude(re[k], im[k]);
                const float f = (m / rms) * p.p0[V * j + k] / (m + MAG_EPS);
                re[k] *= f;
                im[k] *= f;
            }
            CVec<T, V>::store(out, e0 + V * j, re, im);
        }
    }
}

// OP 1: mod swish, 2: mod relu, 3: CGU gate (elementwise)
template <typename T, int V, int OP>
__global__ void __launch_bounds__(THREADS) pointwise_fwd_kernel(Params p) {
    const T *z = (const T *)p.z;
    T *out = (T *)p.out;
    const int64_t n = p.rows * p.dim / V;  // groups
    for (int64_t j = (int64_t)blockIdx.x * THREADS + threadIdx.x; j < n; j += (int64_t)gridDim.x * THREADS) {
        float re[V], im[V];
        CVec<T, V>::load(z, V * j, re, im);
        if constexpr (OP == 3) {
            float ur[V], ui[V];
            CVec<T, V>::load((const T *)p.up, V * j, ur, ui);
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const float m = magnitude(re[k], im[k]), inv = rcp(m + MAG_EPS), gm = sigmoidf(m);
                const float pr = re[k] * inv, pi = im[k] * inv;
                re[k] = (pr * ur[k] - pi * ui[k]) * gm;
                im[k] = (pr * ui[k] + pi * ur[k]) * gm;
            }
        } else {
            const int c0 = (int)((V * j) % p.dim);
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const float m = magnitude(re[k], im[k]), inv = rcp(m + MAG_EPS);
                const int c = c0 + k;
                const float act = OP == 1 ? m * sigmoidf(p.p1[c] * m + p.p0[c]) : fmaxf(m + p.p0[c], 0.f);
                re[k] *= inv * act;
                im[k] *= inv * act;
            }
        }
        CVec<T, V>::store(out, V * j, re, im);
    }
}

// ----------------------------------------------------------------- backward --
// Rows of this block: [r0, r1); wave w takes r0 + w, r0 + w + WAVES, ...
__device__ __forceinline__ void block_rows(const Params &p, int64_t &r0, int64_t &r1) {
    const int64_t per = (p.rows + gridDim.x - 1) / gridDim.x;
    r0 = (int64_t)blockIdx.x * per;
    r1 = r0 + per < p.rows ? r0 + per : p.rows;
}

// fold the per-wave LDS slices [WAVES][NP][dim] into this block's partial
template <int NP>
__device__ __forceinline__ void write_partials(const Params &p, const float *acc) {
    __syncthreads();
    for (int i = threadIdx.x; i < NP * p.dim; i += THREADS) {
        float s = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) s += acc[w * NP * p.dim + i];
        p.part[(int64_t)blockIdx.x * NP * p.dim + i] = s;
    }
}

template <typename T, int V>
__global__ void __launch_bounds__(THREADS) norm_bwd_kernel(Params p) {
    extern __shared__ float acc[];  // [WAVES][1][dim]
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float *my = acc + w * p.dim;
    for (int c = lane; c < p.dim; c += 64) my[c] = 0.f;
    const T *z = (const T *)p.z, *go = (const T *)p.gout;
    T *gz = (T *)p.gz;
    const int groups = p.dim / V;
    int64_t r0, r1;
    block_rows(p, r0, r1);
    for (int64_t row = r0 + w; row < r1; row += WAVES) {
        const int64_t e0 = row * p.dim;
        // row sums: sum |z|^2 (the rms) and sum (g . unit) scale |z|
        float ss = 0.f, sg = 0.f;
        for (int j = lane; j < groups; j += 64) {
            float zr[V], zi[V], gr[V], gi[V];
            CVec<T, V>::load(z, e0 + V * j, zr, zi);
            CVec<T, V>::load(go, e0 + V * j, gr, gi);
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const float m = magnitude(zr[k], zi[k]), inv = rcp(m + MAG_EPS);
                ss += m * m;
                sg += (gr[k] * zr[k] * inv + gi[k] * zi[k] * inv) * p.p0[V * j + k] * m;
            }
        }
        ss = wave_sum(ss);
        sg = wave_sum(sg);
        const float rms = sqrtf(ss / p.dim + p.eps), inv_rms = 1.f / rms;
        const float grad_rms = -sg * inv_rms * inv_rms;
        for (int j = lane; j < groups; j += 64) {
            float zr[V], zi[V], gr[V], gi[V];
            CVec<T, V>::load(z, e0 + V * j, zr, zi);
            CVec<T, V>::load(go, e0 + V * j, gr, gi);
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const int c = V * j + k;
                const float m = magnitude(zr[k], zi[k]), inv = rcp(m + MAG_EPS);
                const float ur = zr[k] * inv, ui = zi[k] * inv, sc = p.p0[c];
                const float gs = gr[k] * ur + gi[k] * ui;
                my[c] += gs * m * inv_rms;
                const float gmag = gs * sc * inv_rms + grad_rms * m / (p.dim * rms);
                const float smag = m * inv_rms * sc;
                const float pr = gr[k] * smag, pi = gi[k] * smag, dot = pr * ur + pi * ui;
                const float zrk = zr[k], zik = zi[k];
                zr[k] = (pr - ur * dot) * inv + gmag * zrk / m;
                zi[k] = (pi - ui * dot) * inv + gmag * zik / m;
            }
            CVec<T, V>::store(gz, e0 + V * j, zr, zi);
        }
    }
    write_partials<1>(p, acc);
}

// OP 1: mod swish (partials d bias, d beta), 2: mod relu (d bias)
template <typename T, int V, int OP>
__global__ void __launch_bounds__(THREADS) act_bwd_kernel(Params p) {
    constexpr int NP = OP == 1 ? 2 : 1;
    extern __shared__ float acc[];  // [WAVES][NP][dim]
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    float *my = acc + w * NP * p.dim;
    for (int c = lane; c < NP * p.dim; c += 64) my[c] = 0.f;
    const T *z = (const T *)p.z, *go = (const T *)p.gout;
    T *gz = (T *)p.gz;
    const int groups = p.dim / V;
    int64_t r0, r1;
    block_rows(p, r0, r1);
    for (int64_t row = r0 + w; row < r1; row += WAVES) {
        const int64_t e0 = row * p.dim;
        for (int j = lane; j < groups; j += 64) {
            float zr[V], zi[V], gr[V], gi[V];
            CVec<T, V>::load(z, e0 + V * j, zr, zi);
            CVec<T, V>::load(go, e0 + V * j, gr, gi);
#pragma unroll
            for (int k = 0; k < V; ++k) {
                const int c = V * j + k;
                const float m = magnitude(zr[k], zi[k]), inv = rcp(m + MAG_EPS);
                const float ur = zr[k] * inv, ui = zi[k] * inv;
                const float da = gr[k] * ur + gi[k] * ui;  // d activated
                float act, dmag;
                if constexpr (OP == 1) {
                    const float beta = p.p1[c], s = sigmoidf(beta * m + p.p0[c]), sd = s * (1.f - s);
                    act = m * s;
                    dmag = da * (s + m * beta * sd);
                    my[c] += da * m * sd;
                    my[p.dim + c] += da * m * m * sd;
                } else {
                    const float x = m + p.p0[c];
                    act = fmaxf(x, 0.f);
                    dmag = x > 0.f ? da : 0.f;
                    my[c] += dmag;
                }
                const float pr = gr[k] * act, pi = gi[k] * act, dot = pr * ur + pi * ui;
                const float zrk = zr[k], zik = zi[k];
                zr[k] = (pr - ur * dot) * inv + dmag * zrk / m;
                zi[k] = (pi - ui * dot) * inv + dmag * zik / m;
            }
            CVec<T, V>::store(gz, e0 + V * j, zr, zi);
        }
    }
    write_partials<NP>(p, acc);
}

template <typename T, int V>
__global__ void __launch_bounds__(THREADS) cgu_bwd_kernel(Params p) {
    const T *gt = (const T *)p.z, *up = (const T *)p.up, *go = (const T *)p.gout;
    T *dg = (T *)p.gz, *du = (T *)p.gup;
    const int64_t n = p.rows * p.dim / V;
    for (int64_t j = (int64_t)blockIdx.x * THREADS + threadIdx.x; j < n; j += (int64_t)gridDim.x * THREADS) {
        float vr[V], vi[V], ur[V], ui[V], gr[V], gi[V];
        CVec<T, V>::load(gt, V * j, vr, vi);
        CVec<T, V>::load(up, V * j, ur, ui);
        CVec<T, V>::load(go, V * j, gr, gi);
#pragma unroll
        for (int k = 0; k < V; ++k) {
            const float m = magnitude(vr[k], vi[k]), inv = rcp(m + MAG_EPS), gm = sigmoidf(m);
            const float pr = vr[k] * inv, pi = vi[k] * inv;
            const float cr = pr * ur[k] - pi * ui[k], ci = pr * ui[k] + pi * ur[k];
            const float dgm = (gr[k] * cr + gi[k] * ci) * gm * (1.f - gm);
            const float dcr = gr[k] * gm, dci = gi[k] * gm;
            const float dpr = dcr * ur[k] + dci * ui[k], dpi = -dcr * ui[k] + dci * ur[k];
            const float dot = dpr * pr + dpi * pi;
            ur[k] = dcr * pr + dci * pi;  // d up
            ui[k] = -dcr * pi + dci * pr;
            const float vrk = vr[k], vik = vi[k];
            vr[k] = (dpr - pr * dot) * inv + dgm * vrk / m;  // d gate
            vi[k] = (dpi - pi * dot) * inv + dgm * vik / m;
        }
        CVec<T, V>::store(du, V * j, ur, ui);
        CVec<T, V>::store(dg, V * j, vr, vi);
    }
}

// Row kernels with the row in registers: four columns per 16-byte group, up to G
// groups per lane (dim <= 256 G), so the second pass over a row re-reads nothing
// and the parameter-gradient column sums stay in registers across the wave's
// rows (lane l owns columns 4(l + 64 g) .. +3).
template <typename T, int G>
__global__ void __launch_bounds__(THREADS) norm_fwd_reg_kernel(Params p) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const T *z = (const T *)p.z;
    T *out = (T *)p.out;
    const int groups = p.dim / 4;
    float sc[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int j = lane + 64 * g;
        const float4 s4 = j < groups ? *reinterpret_cast<const float4 *>(p.p0 + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
        sc[g][0] = s4.x, sc[g][1] = s4.y, sc[g][2] = s4.z, sc[g][3] = s4.w;
    }
    for (int64_t row = (int64_t)blockIdx.x * WAVES + w; row < p.rows; row += (int64_t)gridDim.x * WAVES) {
        const int64_t e0 = row * p.dim;
        float re[G][4], im[G][4], m[G][4];
        float ss = 0.f;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int j = lane + 64 * g;
            if (j < groups) CVec<T, 4>::load(z, e0 + 4 * j, re[g], im[g]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                m[g][k] = magnitude(re[g][k], im[g][k]);
                if (j < groups) ss += m[g][k] * m[g][k];
            }
        }
        const float inv_rms = rcp(sqrtf(wave_sum(ss) / p.dim + p.eps));
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int j = lane + 64 * g;
            if (j >= groups) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float f = m[g][k] * inv_rms * sc[g][k] * rcp(m[g][k] + MAG_EPS);
                re[g][k] *= f;
                im[g][k] *= f;
            }
            CVec<T, 4>::store(out, e0 + 4 * j, re[g], im[g]);
        }
    }
}

// mod swish (OP 1) / mod relu (OP 2) forward over register-resident parameters
template <typename T, int G, int OP>
__global__ void __launch_bounds__(THREADS) act_fwd_reg_kernel(Params p) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const T *z = (const T *)p.z;
    T *out = (T *)p.out;
    const int groups = p.dim / 4;
    float b0[G][4], b1[G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int j = lane + 64 * g;
        const float4 x0 = j < groups ? *reinterpret_cast<const float4 *>(p.p0 + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 x1 = (OP == 1 && j < groups) ? *reinterpret_cast<const float4 *>(p.p1 + 4 * j)
                                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        b0[g][0] = x0.x, b0[g][1] = x0.y, b0[g][2] = x0.z, b0[g][3] = x0.w;
        b1[g][0] = x1.x, b1[g][1] = x1.y, b1[g][2] = x1.z, b1[g][3] = x1.w;
    }
    for (int64_t row = (int64_t)blockIdx.x * WAVES + w; row < p.rows; row += (int64_t)gridDim.x * WAVES) {
        const int64_t e0 = row * p.dim;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int j = lane + 64 * g;
            if (j >= groups) continue;
            float re[4], im[4];
            CVec<T, 4>::load(z, e0 + 4 * j, re, im);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float m = magnitude(re[k], im[k]), inv = rcp(m + MAG_EPS);
                const float act = OP == 1 ? m * sigmoidf(b1[g][k] * m + b0[g][k]) : fmaxf(m + b0[g][k], 0.f);
                re[k] *= inv * act;
                im[k] *= inv * act;
            }
            CVec<T, 4>::store(out, e0 + 4 * j, re, im);
        }
    }
}

// fold per-lane register column sums (NP parameters x G groups x 4 columns)
// across the block's waves in fixed order into this block's partial
template <int NP, int G>
__device__ __forceinline__ void write_partials_reg(const Params &p, const float (&acc)[NP][G][4], float *lds) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, groups = p.dim / 4;
#pragma unroll
    for (int q = 0; q < NP; ++q)
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int j = lane + 64 * g;
            if (j < groups)
                *reinterpret_cast<float4 *>(lds + (w * NP + q) * p.dim + 4 * j) =
                    make_float4(acc[q][g][0], acc[q][g][1], acc[q][g][2], acc[q][g][3]);
        }
    write_partials<NP>(p, lds);
}

template <typename T, int G>
__global__ void __launch_bounds__(THREADS) norm_bwd_reg_kernel(Params p) {
    extern __shared__ float lds[];  // [WAVES][1][dim], used once at the end
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const T *z = (const T *)p.z, *go = (const T *)p.gout;
    T *gz = (T *)p.gz;
    const int groups = p.dim / 4;
    float sc[G][4], acc[1][G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int j = lane + 64 * g;
        const float4 s4 = j < groups ? *reinterpret_cast<const float4 *>(p.p0 + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
        sc[g][0] = s4.x, sc[g][1] = s4.y, sc[g][2] = s4.z, sc[g][3] = s4.w;
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[0][g][k] = 0.f;
    }
    int64_t r0, r1;
    block_rows(p, r0, r1);
    for (int64_t row = r0 + w; row < r1; row += WAVES) {
        const int64_t e0 = row * p.dim;
        float zr[G][4], zi[G][4], gr[G][4], gi[G][4];
        float ss = 0.f, sg = 0.f;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int j = lane + 64 * g;
            if (j >= groups) continue;
            CVec<T, 4>::load(z, e0 + 4 * j, zr[g], zi[g]);
            CVec<T, 4>::load(go, e0 + 4 * j, gr[g], gi[g]);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float m = magnitude(zr[g][k], zi[g][k]), inv = rcp(m + MAG_EPS);
                ss += m * m;
                sg += (gr[g][k] * zr[g][k] + gi[g][k] * zi[g][k]) * inv * sc[g][k] * m;
            }
        }
        ss = wave_sum(ss);
        sg = wave_sum(sg);
        const float rms = sqrtf(ss / p.dim + p.eps), inv_rms = rcp(rms);
        const float grad_rms = -sg * inv_rms * inv_rms, rms_term = grad_rms * rcp(p.dim * rms);
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int j = lane + 64 * g;
            if (j >= groups) continue;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float m = magnitude(zr[g][k], zi[g][k]), inv = rcp(m + MAG_EPS), rm = rcp(m);
                const float ur = zr[g][k] * inv, ui = zi[g][k] * inv;
                const float gs = gr[g][k] * ur + gi[g][k] * ui;
                acc[0][g][k] += gs * m * inv_rms;
                const float gmag = gs * sc[g][k] * inv_rms + rms_term * m;
                const float smag = m * inv_rms * sc[g][k];
                const float pr = gr[g][k] * smag, pi = gi[g][k] * smag, dot = pr * ur + pi * ui;
                const float a = zr[g][k], b = zi[g][k];
                zr[g][k] = (pr - ur * dot) * inv + gmag * a * rm;
                zi[g][k] = (pi - ui * dot) * inv + gmag * b * rm;
            }
            CVec<T, 4>::store(gz, e0 + 4 * j, zr[g], zi[g]);
        }
    }
    write_partials_reg<1, G>(p, acc, lds);
}

template <typename T, int G, int OP>
__global__ void __launch_bounds__(THREADS) act_bwd_reg_kernel(Params p) {
    constexpr int NP = OP == 1 ? 2 : 1;
    extern __shared__ float lds[];  // [WAVES][NP][dim], used once at the end
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const T *z = (const T *)p.z, *go = (const T *)p.gout;
    T *gz = (T *)p.gz;
    const int groups = p.dim / 4;
    float b0[G][4], b1[G][4], acc[NP][G][4];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const int j = lane + 64 * g;
        const float4 x0 = j < groups ? *reinterpret_cast<const float4 *>(p.p0 + 4 * j) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 x1 = (OP == 1 && j < groups) ? *reinterpret_cast<const float4 *>(p.p1 + 4 * j)
                                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        b0[g][0] = x0.x, b0[g][1] = x0.y, b0[g][2] = x0.z, b0[g][3] = x0.w;
        b1[g][0] = x1.x, b1[g][1] = x1.y, b1[g][2] = x1.z, b1[g][3] = x1.w;
#pragma unroll
        for (int q = 0; q < NP; ++q)
#pragma unroll
            for (int k = 0; k < 4; ++k) acc[q][g][k] = 0.f;
    }
    int64_t r0, r1;
    block_rows(p, r0, r1);
    for (int64_t row = r0 + w; row < r1; row += WAVES) {
        const int64_t e0 = row * p.dim;
#pragma unroll
        for (int g = 0; g < G; ++g) {
            const int j = lane + 64 * g;
            if (j >= groups) continue;
            float zr[4], zi[4], gr[4], gi[4];
            CVec<T, 4>::load(z, e0 + 4 * j, zr, zi);
            CVec<T, 4>::load(go, e0 + 4 * j, gr, gi);
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float m = magnitude(zr[k], zi[k]), inv = rcp(m + MAG_EPS), rm = rcp(m);
                const float ur = zr[k] * inv, ui = zi[k] * inv;
                const float da = gr[k] * ur + gi[k] * ui;
                float act, dmag;
                if constexpr (OP == 1) {
                    const float beta = b1[g][k], sg = sigmoidf(beta * m + b0[g][k]), sd = sg * (1.f - sg);
                    act = m * sg;
                    dmag = da * (sg + m * beta * sd);
                    acc[0][g][k] += da * m * sd;
                    acc[NP - 1][g][k] += OP == 1 ? da * m * m * sd : 0.f;
                } else {
                    const float x = m + b0[g][k];
                    act = fmaxf(x, 0.f);
                    dmag = x > 0.f ? da : 0.f;
                    acc[0][g][k] += dmag;
                }
                const float pr = gr[k] * act, pi = gi[k] * act, dot = pr * ur + pi * ui;
                const float a = zr[k], b = zi[k];
                zr[k] = (pr - ur * dot) * inv + dmag * a * rm;
                zi[k] = (pi - ui * dot) * inv + dmag * b * rm;
            }
            CVec<T, 4>::store(gz, e0 + 4 * j, zr, zi);
        }
    }
    write_partials_reg<NP, G>(p, acc, lds);
}

// Row-team kernels (16-byte groups, dim / 4 a multiple of 64 up to TEAM_MAX): a
// block of dim / 4 threads is one row wide, thread i owning columns 4 i .. 4 i + 3
// of every row, so the parameters and the parameter-gradient column sums stay in
// registers for the block's whole life and no wave re-reads a row; R rows are
// loaded per iteration before any is reduced, and the ComplexNorm row sums cross
// the block's waves through LDS (one barrier pair per R rows).  The backward
// writes the input gradient in the form A g + B z (A, B real per element):
//   ComplexNorm:  A = |z| sc / (rms (|z| + eps)),   B = gmag / |z| - A (g.u) / (|z| + eps)
//   mod swish / relu: A = act / (|z| + eps),        B = dmag / |z| - A (g.u) / (|z| + eps)
// with u = z / (|z| + eps) and gmag, dmag the gradients of the output magnitude
// (the closed forms of the reference's autograd backward, v11/triton_kernels.py:209-345).
constexpr int TEAM_MAX = 512;  // threads per row team (dim <= 2048)
// The grid of a row-team kernel is the blocks that are resident at once (its
// occupancy times the device's CUs: a grid beyond that runs a partly empty last
// round), at most TEAM_RESIDENT_MAX threads, which the parameter-gradient
// workspace is sized for.
constexpr int64_t TEAM_RESIDENT_MAX = 256 * 2048;

template <int R>
__device__ __forceinline__ void team_row_sums(float (&a)[R], float (&b)[R], float *red) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        a[r] = wave_sum(a[r]);
        b[r] = wave_sum(b[r]);
    }
    if (lane == 0) {
#pragma unroll
        for (int r = 0; r < R; ++r) red[(2 * r) * (TEAM_MAX / 64) + w] = a[r], red[(2 * r + 1) * (TEAM_MAX / 64) + w] = b[r];
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < R; ++r) {
        a[r] = b[r] = 0.f;
        for (int k = 0; k < nw; ++k) a[r] += red[(2 * r) * (TEAM_MAX / 64) + k], b[r] += red[(2 * r + 1) * (TEAM_MAX / 64) + k];
    }
    __syncthreads();  // red is rewritten by the next iteration
}

// rows row0 .. row0 + R - 1 of the block's iteration (rows past the end re-read the last row)
template <typename T, int R>
__device__ __forceinline__ void team_load(const T *base, const Params &p, int64_t row0, float (&re)[R][4],
                                          float (&im)[R][4]) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = row0 + r < p.rows ? row0 + r : p.rows - 1;
        CVec<T, 4>::load(base, row * p.dim + 4 * threadIdx.x, re[r], im[r]);
    }
}

template <typename T, int R>
__global__ void __launch_bounds__(TEAM_MAX) norm_fwd_team_kernel(Params p) {
    __shared__ float red[2 * R * (TEAM_MAX / 64)];
    const T *z = (const T *)p.z;
    T *out = (T *)p.out;
    const float4 s4 = *reinterpret_cast<const float4 *>(p.p0 + 4 * threadIdx.x);
    const float sc[4] = {s4.x, s4.y, s4.z, s4.w};
    for (int64_t row0 = (int64_t)blockIdx.x * R; row0 < p.rows; row0 += (int64_t)gridDim.x * R) {
        float re[R][4], im[R][4], ss[R], unused[R];
        team_load<T, R>(z, p, row0, re, im);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            ss[r] = unused[r] = 0.f;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float m = magnitude(re[r][k], im[r][k]);
                ss[r] += m * m;
            }
        }
        team_row_sums<R>(ss, unused, red);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (row0 + r >= p.rows) break;
            const float inv_rms = rcp(sqrtf(ss[r] / p.dim + p.eps));
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float m = magnitude(re[r][k], im[r][k]);
                const float f = m * inv_rms * sc[k] * rcp(m + MAG_EPS);
                re[r][k] *= f;
                im[r][k] *= f;
            }
            CVec<T, 4>::store(out, (row0 + r) * p.dim + 4 * threadIdx.x, re[r], im[r]);
        }
    }
}

// OP 0: ComplexNorm (partial d scale), 1: mod swish (d bias, d beta), 2: mod relu (d bias)
template <typename T, int R, int OP>
__global__ void __launch_bounds__(TEAM_MAX) bwd_team_kernel(Params p) {
    constexpr int NP = OP == 1 ? 2 : 1;
    __shared__ float red[2 * R * (TEAM_MAX / 64)];
    const T *z = (const T *)p.z, *go = (const T *)p.gout;
    T *gz = (T *)p.gz;
    const int c0 = 4 * threadIdx.x;
    const float4 x0 = *reinterpret_cast<const float4 *>(p.p0 + c0);
    const float4 x1 = OP == 1 ? *reinterpret_cast<const float4 *>(p.p1 + c0) : make_float4(0.f, 0.f, 0.f, 0.f);
    const float q0[4] = {x0.x, x0.y, x0.z, x0.w}, q1[4] = {x1.x, x1.y, x1.z, x1.w};
    float acc[NP][4];
#pragma unroll
    for (int q = 0; q < NP; ++q)
#pragma unroll
        for (int k = 0; k < 4; ++k) acc[q][k] = 0.f;
    for (int64_t row0 = (int64_t)blockIdx.x * R; row0 < p.rows; row0 += (int64_t)gridDim.x * R) {
        float zr[R][4], zi[R][4], gr[R][4], gi[R][4];
        team_load<T, R>(z, p, row0, zr, zi);
        team_load<T, R>(go, p, row0, gr, gi);
        float ss[R], sg[R];
        if constexpr (OP == 0) {
            // row sums: sum |z|^2 (the rms) and sum (g.u) sc |z|
#pragma unroll
            for (int r = 0; r < R; ++r) {
                ss[r] = sg[r] = 0.f;
#pragma unroll
                for (int k = 0; k < 4; ++k) {
                    const float m = magnitude(zr[r][k], zi[r][k]);
                    ss[r] += m * m;
                    sg[r] += (gr[r][k] * zr[r][k] + gi[r][k] * zi[r][k]) * rcp(m + MAG_EPS) * q0[k] * m;
                }
            }
            team_row_sums<R>(ss, sg, red);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (row0 + r >= p.rows) break;
            float inv_rms = 0.f, rms_term = 0.f;
            if constexpr (OP == 0) {
                const float rms = sqrtf(ss[r] / p.dim + p.eps);
                inv_rms = rcp(rms);
                rms_term = -sg[r] * inv_rms * inv_rms * rcp(p.dim * rms);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const float m = magnitude(zr[r][k], zi[r][k]), inv = rcp(m + MAG_EPS), rm = rcp(m);
                const float gu = (gr[r][k] * zr[r][k] + gi[r][k] * zi[r][k]) * inv;  // g.u
                float A, dmag;
                if constexpr (OP == 0) {
                    acc[0][k] += gu * m * inv_rms;
                    dmag = gu * q0[k] * inv_rms + rms_term * m;
                    A = m * inv_rms * q0[k] * inv;
                } else if constexpr (OP == 1) {
                    const float beta = q1[k], sgm = sigmoidf(beta * m + q0[k]), sd = sgm * (1.f - sgm);
                    dmag = gu * (sgm + m * beta * sd);
                    acc[0][k] += gu * m * sd;
                    acc[NP - 1][k] += gu * m * m * sd;
                    A = m * sgm * inv;
                } else {
                    const float x = m + q0[k];
                    dmag = x > 0.f ? gu : 0.f;
                    acc[0][k] += dmag;
                    A = fmaxf(x, 0.f) * inv;
                }
                const float Bc = dmag * rm - A * gu * inv;
                const float a = zr[r][k], b = zi[r][k];
                zr[r][k] = A * gr[r][k] + Bc * a;
                zi[r][k] = A * gi[r][k] + Bc * b;
            }
            CVec<T, 4>::store(gz, (row0 + r) * p.dim + c0, zr[r], zi[r]);
        }
    }
#pragma unroll
    for (int q = 0; q < NP; ++q)
        *reinterpret_cast<float4 *>(p.part + ((int64_t)blockIdx.x * NP + q) * p.dim + c0) =
            make_float4(acc[q][0], acc[q][1], acc[q][2], acc[q][3]);
}

// out[i] = sum over blocks of part[b][i], in a fixed order: 16 waves each sum
// the blocks b = w, w + 16, ... (eight loads in flight), then wave 0 adds the 16
constexpr int SUM_THREADS = 1024;
__global__ void __launch_bounds__(SUM_THREADS) partial_sum_kernel(const float *part, int blocks, int n, float *o0,
                                                                  float *o1, int dim) {
    __shared__ float red[SUM_THREADS / 64][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int i = blockIdx.x * 64 + lane;
    float s = 0.f;
    if (i < n) {
        float acc8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        int b = w;
        for (; b + 7 * (SUM_THREADS / 64) < blocks; b += 8 * (SUM_THREADS / 64)) {
#pragma unroll
            for (int k = 0; k < 8; ++k) acc8[k] += part[(int64_t)(b + k * (SUM_THREADS / 64)) * n + i];
        }
        for (; b < blocks; b += SUM_THREADS / 64) acc8[0] += part[(int64_t)b * n + i];
#pragma unroll
        for (int k = 0; k < 8; ++k) s += acc8[k];
    }
    red[w][lane] = s;
    __syncthreads();
    if (w == 0 && i < n) {
        float t = 0.f;
#pragma unroll
        for (int k = 0; k < SUM_THREADS / 64; ++k) t += red[k][lane];
        if (i < dim) o0[i] = t;
        else o1[i - dim] = t;
    }
}

int n_params(int op) { return op == QPAM_CPLX_NORM || op == QPAM_CPLX_MOD_RELU ? 1 : op == QPAM_CPLX_MOD_SWISH ? 2 : 0; }

int row_blocks(int64_t rows) { return (int)std::min<int64_t>((rows + WAVES - 1) / WAVES, MAX_BLOCKS); }
// flat elementwise grid: one 16-byte group per thread up to 65536 blocks (a grid-stride loop past that);
// measured at 65536 x 1024 complex bf16: CGU gate fwd+bwd 0.386 ms with an 8192-block cap, 0.356 ms here
int flat_blocks(int64_t n) { return (int)std::min<int64_t>((n + THREADS - 1) / THREADS, 65536); }

int validate(const qpam_cplx_args *a, const char *who, bool bwd) {
    QPAM_REQUIRE(a != nullptr, "%s: null args", who);
    QPAM_REQUIRE(a->op >= QPAM_CPLX_NORM && a->op <= QPAM_CPLX_CGU_GATE, "%s: unknown op %d", who, a->op);
    QPAM_REQUIRE(a->dtype == QPAM_F32 || a->dtype == QPAM_BF16, "%s: dtype %d", who, a->dtype);
    QPAM_REQUIRE(a->rows >= 0 && a->dim >= 1, "%s: bad sizes rows=%lld dim=%d", who, (long long)a->rows, a->dim);
    const int np = n_params(a->op);
    QPAM_REQUIRE(a->dim * np <= 8192, "%s: dim %d too large for the parameter-gradient slices (max %d)", who, a->dim,
                 np ? 8192 / np : 0);
    if (a->rows == 0) {  // nothing to read or write but the (zero) parameter gradients
        QPAM_REQUIRE(!bwd || np < 1 || a->gp0 != nullptr, "%s: missing parameter gradient", who);
        QPAM_REQUIRE(!bwd || np < 2 || a->gp1 != nullptr, "%s: missing beta gradient", who);
        return QPAM_OK;
    }
    QPAM_REQUIRE(a->z != nullptr, "%s: null z", who);
    QPAM_REQUIRE(a->op != QPAM_CPLX_CGU_GATE || a->up != nullptr, "%s: CGU gate needs up", who);
    QPAM_REQUIRE(np < 1 || a->p0 != nullptr, "%s: missing parameter", who);
    QPAM_REQUIRE(np < 2 || a->p1 != nullptr, "%s: missing beta", who);
    if (!bwd) {
        QPAM_REQUIRE(a->out != nullptr, "%s: null out", who);
    } else {
        QPAM_REQUIRE(a->gout && a->gz, "%s: null gradient pointers", who);
        QPAM_REQUIRE(a->op != QPAM_CPLX_CGU_GATE || a->gup != nullptr, "%s: CGU gate needs gup", who);
        QPAM_REQUIRE(np < 1 || a->gp0 != nullptr, "%s: missing parameter gradient", who);
        QPAM_REQUIRE(np < 2 || a->gp1 != nullptr, "%s: missing beta gradient", who);
        QPAM_REQUIRE(np == 0 || (a->workspace != nullptr && a->workspace_bytes >= qpam_cplx_workspace_size(a)),
                     "%s: workspace needs %zu bytes (got %zu)", who, qpam_cplx_workspace_size(a), a->workspace_bytes);
    }
    return QPAM_OK;
}

Params params(const qpam_cplx_args *a) {
    Params p;
    p.rows = a->rows;
    p.dim = a->dim;
    p.eps = a->eps;
    p.z = a->z;
    p.up = a->up;
    p.p0 = a->p0;
    p.p1 = a->p1;
    p.out = a->out;
    p.gout = a->gout;
    p.gz = a->gz;
    p.gup = a->gup;
    p.part = (float *)a->workspace;
    return p;
}

// groups of 4 columns per lane for the register-row kernels: 1, 2, 4 or 8 (dim <= 2048); 0 = use the
// LDS-accumulating kernels
int reg_groups(int dim) {
    const int g = (dim / 4 + 63) / 64;
    return g <= 1 ? 1 : g <= 2 ? 2 : g <= 4 ? 4 : g <= 8 ? 8 : 0;
}

// threads of the row team (dim / 4 when it is a multiple of 64 up to TEAM_MAX), 0 = no team path
int team_threads(int dim) {
    const int t = dim / 4;
    return (t % 64 == 0 && t <= TEAM_MAX) ? t : 0;
}
constexpr int TEAM_ROWS_FWD = 4, TEAM_ROWS_NORM_BWD = 4, TEAM_ROWS_ACT_BWD = 2;
// blocks of R rows per iteration, at most TEAM_RESIDENT_MAX / threads (no kernel: the bound)
int team_blocks(int64_t rows, int threads, int r, const void *kernel = nullptr) {
    int64_t resident = TEAM_RESIDENT_MAX / threads;
    if (kernel) {
        // resident blocks per CU of (kernel, threads) on each device, looked up once
        struct Entry {
            const void *k;
            int dev, threads, blocks;
        };
        static std::mutex mu;
        static Entry cache[64];
        static int n_cache = 0;
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess) return 0;
        int per_cu = -1;
        {
            std::lock_guard<std::mutex> lock(mu);
            for (int i = 0; i < n_cache; ++i)
                if (cache[i].k == kernel && cache[i].dev == dev && cache[i].threads == threads) per_cu = cache[i].blocks;
        }
        if (per_cu < 0) {
            int cus = 0, occ = 0;
            if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
                hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, kernel, threads, 0) != hipSuccess)
                return 0;
            per_cu = std::max(1, occ) * cus;
            std::lock_guard<std::mutex> lock(mu);
            if (n_cache < 64) cache[n_cache++] = Entry{kernel, dev, threads, per_cu};
        }
        resident = std::min<int64_t>(resident, per_cu);
    }
    return (int)std::max<int64_t>(1, std::min<int64_t>((rows + r - 1) / r, resident));
}

template <typename T, int OP>
int launch_act_fwd_reg(int g, int64_t rows, hipStream_t stream, const Params &p) {
    const dim3 grid(row_blocks(rows));
    switch (g) {
        case 1: hipLaunchKernelGGL((act_fwd_reg_kernel<T, 1, OP>), grid, dim3(THREADS), 0, stream, p); break;
        case 2: hipLaunchKernelGGL((act_fwd_reg_kernel<T, 2, OP>), grid, dim3(THREADS), 0, stream, p); break;
        case 4: hipLaunchKernelGGL((act_fwd_reg_kernel<T, 4, OP>), grid, dim3(THREADS), 0, stream, p); break;
        default: hipLaunchKernelGGL((act_fwd_reg_kernel<T, 8, OP>), grid, dim3(THREADS), 0, stream, p);
    }
    return launch_status("qpam_cplx_fwd");
}

template <typename T, int G>
int launch_bwd_reg_g(int op, int blocks, size_t smem, hipStream_t stream, const Params &p) {
    const void *k = op == QPAM_CPLX_NORM ? (const void *)norm_bwd_reg_kernel<T, G>
                    : op == QPAM_CPLX_MOD_SWISH ? (const void *)act_bwd_reg_kernel<T, G, 1>
                                                : (const void *)act_bwd_reg_kernel<T, G, 2>;
    QPAM_CHECK_HIP(hipFuncSetAttribute(k, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    if (op == QPAM_CPLX_NORM)
        hipLaunchKernelGGL((norm_bwd_reg_kernel<T, G>), dim3(blocks), dim3(THREADS), smem, stream, p);
    else if (op == QPAM_CPLX_MOD_SWISH)
        hipLaunchKernelGGL((act_bwd_reg_kernel<T, G, 1>), dim3(blocks), dim3(THREADS), smem, stream, p);
    else
        hipLaunchKernelGGL((act_bwd_reg_kernel<T, G, 2>), dim3(blocks), dim3(THREADS), smem, stream, p);
    return launch_status("qpam_cplx_bwd");
}

template <typename T>
int launch_bwd_reg(int op, int g, int blocks, size_t smem, hipStream_t stream, const Params &p) {
    switch (g) {
        case 1: return launch_bwd_reg_g<T, 1>(op, blocks, smem, stream, p);
        case 2: return launch_bwd_reg_g<T, 2>(op, blocks, smem, stream, p);
        case 4: return launch_bwd_reg_g<T, 4>(op, blocks, smem, stream, p);
        default: return launch_bwd_reg_g<T, 8>(op, blocks, smem, stream, p);
    }
}

template <typename T, int V>
int fwd(const qpam_cplx_args *a, hipStream_t stream) {
    const Params p = params(a);
    const int64_t n = a->rows * (int64_t)a->dim / V;
    switch (a->op) {
        case QPAM_CPLX_NORM:
            if (V == 4 && team_threads(a->dim)) {
                const int tt = team_threads(a->dim);
                const void *k = (const void *)norm_fwd_team_kernel<T, TEAM_ROWS_FWD>;
                const int tb = team_blocks(a->rows, tt, TEAM_ROWS_FWD, k);
                if (tb == 0) return fail(QPAM_ERR_HIP, "qpam_cplx_fwd: occupancy query failed");
                hipLaunchKernelGGL((norm_fwd_team_kernel<T, TEAM_ROWS_FWD>), dim3(tb), dim3(tt), 0, stream, p);
                break;
            }
            if (V == 4 && reg_groups(a->dim)) {
                const dim3 grid(row_blocks(a->rows));
                switch (reg_groups(a->dim)) {
                    case 1: hipLaunchKernelGGL((norm_fwd_reg_kernel<T, 1>), grid, dim3(THREADS), 0, stream, p); break;
                    case 2: hipLaunchKernelGGL((norm_fwd_reg_kernel<T, 2>), grid, dim3(THREADS), 0, stream, p); break;
                    case 4: hipLaunchKernelGGL((norm_fwd_reg_kernel<T, 4>), grid, dim3(THREADS), 0, stream, p); break;
                    default: hipLaunchKernelGGL((norm_fwd_reg_kernel<T, 8>), grid, dim3(THREADS), 0, stream, p);
                }
                break;
            }
            hipLaunchKernelGGL((norm_fwd_kernel<T, V>), dim3(row_blocks(a->rows)), dim3(THREADS), 0, stream, p);
            break;
        case QPAM_CPLX_MOD_SWISH:
            if (V == 4 && reg_groups(a->dim)) return launch_act_fwd_reg<T, 1>(reg_groups(a->dim), a->rows, stream, p);
            hipLaunchKernelGGL((pointwise_fwd_kernel<T, V, 1>), dim3(flat_blocks(n)), dim3(THREADS), 0, stream, p);
            break;
        case QPAM_CPLX_MOD_RELU:
            if (V == 4 && reg_groups(a->dim)) return launch_act_fwd_reg<T, 2>(reg_groups(a->dim), a->rows, stream, p);
            hipLaunchKernelGGL((pointwise_fwd_kernel<T, V, 2>), dim3(flat_blocks(n)), dim3(THREADS), 0, stream, p);
            break;
        default:
            hipLaunchKernelGGL((pointwise_fwd_kernel<T, V, 3>), dim3(flat_blocks(n)), dim3(THREADS), 0, stream, p);
    }
    return launch_status("qpam_cplx_fwd");
}

template <typename T, int V>
int bwd(const qpam_cplx_args *a, hipStream_t stream) {
    const Params p = params(a);
    const int np = n_params(a->op);
    const int blocks = row_blocks(a->rows);
    const size_t smem = (size_t)WAVES * np * a->dim * sizeof(float);
    if (V == 4 && team_threads(a->dim) && a->op != QPAM_CPLX_CGU_GATE) {
        const int tt = team_threads(a->dim);
        const int rr = a->op == QPAM_CPLX_NORM ? TEAM_ROWS_NORM_BWD : TEAM_ROWS_ACT_BWD;
        const void *k = a->op == QPAM_CPLX_NORM ? (const void *)bwd_team_kernel<T, TEAM_ROWS_NORM_BWD, 0>
                        : a->op == QPAM_CPLX_MOD_SWISH ? (const void *)bwd_team_kernel<T, TEAM_ROWS_ACT_BWD, 1>
                                                       : (const void *)bwd_team_kernel<T, TEAM_ROWS_ACT_BWD, 2>;
        const int tb = team_blocks(a->rows, tt, rr, k);
        if (tb == 0) return fail(QPAM_ERR_HIP, "qpam_cplx_bwd: occupancy query failed");
        if (a->op == QPAM_CPLX_NORM)
            hipLaunchKernelGGL((bwd_team_kernel<T, TEAM_ROWS_NORM_BWD, 0>), dim3(tb), dim3(tt), 0, stream, p);
        else if (a->op == QPAM_CPLX_MOD_SWISH)
            hipLaunchKernelGGL((bwd_team_kernel<T, TEAM_ROWS_ACT_BWD, 1>), dim3(tb), dim3(tt), 0, stream, p);
        else
            hipLaunchKernelGGL((bwd_team_kernel<T, TEAM_ROWS_ACT_BWD, 2>), dim3(tb), dim3(tt), 0, stream, p);
        int st = launch_status("qpam_cplx_bwd");
        if (st) return st;
        const int n = np * a->dim;
        hipLaunchKernelGGL(partial_sum_kernel, dim3((n + 63) / 64), dim3(SUM_THREADS), 0, stream,
                           (const float *)a->workspace, tb, n, a->gp0, a->gp1, a->dim);
        return launch_status("qpam_cplx_bwd (parameter gradients)");
    }
    if (V == 4 && reg_groups(a->dim) && a->op != QPAM_CPLX_CGU_GATE) {
        int st = launch_bwd_reg<T>(a->op, reg_groups(a->dim), blocks, smem, stream, p);
        if (st) return st;
        const int n = np * a->dim;
        hipLaunchKernelGGL(partial_sum_kernel, dim3((n + 63) / 64), dim3(SUM_THREADS), 0, stream,
                           (const float *)a->workspace, blocks, n, a->gp0, a->gp1, a->dim);
        return launch_status("qpam_cplx_bwd (parameter gradients)");
    }
    switch (a->op) {
        case QPAM_CPLX_NORM:
            QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)norm_bwd_kernel<T, V>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
            hipLaunchKernelGGL((norm_bwd_kernel<T, V>), dim3(blocks), dim3(THREADS), smem, stream, p);
            break;
        case QPAM_CPLX_MOD_SWISH:
            QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)act_bwd_kernel<T, V, 1>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
            hipLaunchKernelGGL((act_bwd_kernel<T, V, 1>), dim3(blocks), dim3(THREADS), smem, stream, p);
            break;
        case QPAM_CPLX_MOD_RELU:
            QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)act_bwd_kernel<T, V, 2>,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
            hipLaunchKernelGGL((act_bwd_kernel<T, V, 2>), dim3(blocks), dim3(THREADS), smem, stream, p);
            break;
        default:
            hipLaunchKernelGGL((cgu_bwd_kernel<T, V>), dim3(flat_blocks(a->rows * (int64_t)a->dim / V)),
                               dim3(THREADS), 0, stream, p);
            return launch_status("qpam_cplx_bwd (CGU gate)");
    }
    int st = launch_status("qpam_cplx_bwd");
    if (st) return st;
    const int n = np * a->dim;
    hipLaunchKernelGGL(partial_sum_kernel, dim3((n + 63) / 64), dim3(SUM_THREADS), 0, stream,
                       (const float *)a->workspace, blocks, n, a->gp0, a->gp1, a->dim);
    return launch_status("qpam_cplx_bwd (parameter gradients)");
}

// 16-byte vectors of four complex elements when every row starts 16-byte aligned
bool vec4(const qpam_cplx_args *a) {
    const uintptr_t m = (uintptr_t)a->z | (uintptr_t)a->up | (uintptr_t)a->out | (uintptr_t)a->gout |
                        (uintptr_t)a->gz | (uintptr_t)a->gup | (uintptr_t)a->p0 | (uintptr_t)a->p1;
    return a->dim % 4 == 0 && (m & 15) == 0;
}

template <typename T>
int fwd_t(const qpam_cplx_args *a, hipStream_t stream) { return vec4(a) ? fwd<T, 4>(a, stream) : fwd<T, 1>(a, stream); }
template <typename T>
int bwd_t(const qpam_cplx_args *a, hipStream_t stream) { return vec4(a) ? bwd<T, 4>(a, stream) : bwd<T, 1>(a, stream); }

// ------------------------------------------------ decode block glue --
// Inference: the work between the GEMMs of a V11 block in the model-level
// decode (a few hundred rows), one launch each instead of the casts, splits,
// scaled adds and norms torch runs there one at a time.

// four consecutive complex values, plain (cached) 16- / 32-byte accesses: the
// outputs are read back at once by the next GEMM
template <typename T> struct Row4;
template <> struct Row4<float> {
    __device__ __forceinline__ static void load(const float *p, float (&re)[4], float (&im)[4]) {
        const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
        re[0] = a.x, im[0] = a.y, re[1] = a.z, im[1] = a.w, re[2] = b.x, im[2] = b.y, re[3] = b.z, im[3] = b.w;
    }
    __device__ __forceinline__ static void store(float *p, const float (&re)[4], const float (&im)[4]) {
        *reinterpret_cast<float4 *>(p) = make_float4(re[0], im[0], re[1], im[1]);
        *reinterpret_cast<float4 *>(p + 4) = make_float4(re[2], im[2], re[3], im[3]);
    }
};
template <> struct Row4<unsigned short> {
    __device__ __forceinline__ static void load(const unsigned short *p, float (&re)[4], float (&im)[4]) {
        const uint4 a = *reinterpret_cast<const uint4 *>(p);
        const unsigned u[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) re[k] = __uint_as_float(u[k] << 16), im[k] = __uint_as_float(u[k] & 0xFFFF0000u);
    }
    __device__ __forceinline__ static void store(unsigned short *p, const float (&re)[4], const float (&im)[4]) {
        *reinterpret_cast<uint4 *>(p) = make_uint4(pack_bf16x2(re[0], im[0]), pack_bf16x2(re[1], im[1]),
                                                   pack_bf16x2(re[2], im[2]), pack_bf16x2(re[3], im[3]));
    }
};

struct ResidNormParams {
    int64_t rows;
    int dim;
    float eps;
    float *x;
    int64_t ldx;
    const void *y;
    int64_t ldy;
    const float *y_scale;
    const float *scale;
    void *out;
    int64_t ldo;
};

// One block per row, a thread per four complex columns (threads past dim / 4
// add zero to the row sum).  x + y * s is rounded as a product and then a sum
// (the reference's two tensor ops); the norm follows norm_fwd_team_kernel's
// operation order (per-thread sum over its four columns, wave sums, then the
// waves in order), so a row without y matches qpam_cplx_fwd's ComplexNorm.
template <typename TY, typename TO>
__global__ void __launch_bounds__(TEAM_MAX) resid_norm_kernel(ResidNormParams q) {
    __shared__ float red[TEAM_MAX / 64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, nw = blockDim.x >> 6;
    const int64_t row = blockIdx.x;
    const int c = 4 * threadIdx.x;
    const bool on = c < q.dim;
    float re[4] = {0.f, 0.f, 0.f, 0.f}, im[4] = {0.f, 0.f, 0.f, 0.f};
    float ss = 0.f;
    if (on) {
        float *xr = q.x + row * q.ldx + 2 * c;
        Row4<float>::load(xr, re, im);
        if (q.y) {
            float yr[4], yi[4];
            Row4<TY>::load(static_cast<const TY *>(q.y) + row * q.ldy + 2 * c, yr, yi);
            const float s = *q.y_scale;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                // two roundings, as the reference's product and sum (no fused multiply-add)
#pragma clang fp contract(off)
                re[k] = re[k] + yr[k] * s;
                im[k] = im[k] + yi[k] * s;
            }
            Row4<float>::store(xr, re, im);
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float m = magnitude(re[k], im[k]);
            ss += m * m;
        }
    }
    ss = wave_sum(ss);
    if (lane == 0) red[w] = ss;
    __syncthreads();
    float tot = 0.f;
    for (int k = 0; k < nw; ++k) tot += red[k];
    if (!on) return;
    const float inv_rms = rcp(sqrtf(tot / q.dim + q.eps));
    const float4 s4 = *reinterpret_cast<const float4 *>(q.scale + c);
    const float sc[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float m = magnitude(re[k], im[k]);
        const float f = m * inv_rms * sc[k] * rcp(m + MAG_EPS);
        re[k] *= f;
        im[k] *= f;
    }
    Row4<TO>::store(static_cast<TO *>(q.out) + row * q.ldo + 2 * c, re, im);
}

struct CguMixParams {
    int64_t rows;
    int hid;
    const void *gu;
    int64_t ldg;
    const float *bias, *beta, *pa, *pb;
    void *out;
    int64_t ldo;
};

// ACT 1: mod swish, 2: mod relu, 3: phase-modulated; a thread per four complex
// columns of a row (grid-stride), the activation of up and then the gate, each
// with pointwise_fwd_kernel's formulas
template <typename TG, typename TO, int ACT>
__global__ void __launch_bounds__(THREADS) cgu_mix_kernel(CguMixParams q) {
    const int groups = q.hid / 4;
    const int64_t n = q.rows * groups;
    for (int64_t j = (int64_t)blockIdx.x * THREADS + threadIdx.x; j < n; j += (int64_t)gridDim.x * THREADS) {
        const int64_t row = j / groups;
        const int c = 4 * (int)(j - row * groups);
        const TG *g = static_cast<const TG *>(q.gu) + row * q.ldg;
        float gr[4], gi[4], ur[4], ui[4];
        Row4<TG>::load(g + 2 * c, gr, gi);
        Row4<TG>::load(g + 2 * q.hid + 2 * c, ur, ui);
        const float4 b4 = *reinterpret_cast<const float4 *>(q.bias + c);
        const float bs[4] = {b4.x, b4.y, b4.z, b4.w};
        float bt[4] = {0.f, 0.f, 0.f, 0.f}, pa[4] = {0.f, 0.f, 0.f, 0.f}, pb[4] = {0.f, 0.f, 0.f, 0.f};
        if constexpr (ACT != 2) {
            const float4 t4 = *reinterpret_cast<const float4 *>(q.beta + c);
            bt[0] = t4.x, bt[1] = t4.y, bt[2] = t4.z, bt[3] = t4.w;
        }
        if constexpr (ACT == 3) {
            const float4 a4 = *reinterpret_cast<const float4 *>(q.pa + c), c4 = *reinterpret_cast<const float4 *>(q.pb + c);
            pa[0] = a4.x, pa[1] = a4.y, pa[2] = a4.z, pa[3] = a4.w;
            pb[0] = c4.x, pb[1] = c4.y, pb[2] = c4.z, pb[3] = c4.w;
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float m = magnitude(ur[k], ui[k]), inv = rcp(m + MAG_EPS);
            const float act = ACT == 2 ? fmaxf(m + bs[k], 0.f) : m * sigmoidf(bt[k] * m + bs[k]);
            if constexpr (ACT == 3) {
                // unit phase turned by phase_alpha |u| + phase_beta, then scaled
                float sn, cs;
                sincosf(pa[k] * m + pb[k], &sn, &cs);
                const float pr = ur[k] * inv, pi = ui[k] * inv;
                ur[k] = (pr * cs - pi * sn) * act;
                ui[k] = (pr * sn + pi * cs) * act;
            } else {
                ur[k] *= inv * act;
                ui[k] *= inv * act;
            }
            const float mg = magnitude(gr[k], gi[k]), ig = rcp(mg + MAG_EPS), gm = sigmoidf(mg);
            const float pr = gr[k] * ig, pi = gi[k] * ig;
            gr[k] = (pr * ur[k] - pi * ui[k]) * gm;
            gi[k] = (pr * ui[k] + pi * ur[k]) * gm;
        }
        Row4<TO>::store(static_cast<TO *>(q.out) + row * q.ldo + 2 * c, gr, gi);
    }
}

bool al16(const void *p) { return ((uintptr_t)p & 15) == 0; }
int elems16(int dtype) { return dtype == QPAM_BF16 ? 8 : 4; }  // elements per 16 bytes

template <typename TY, typename TO>
void launch_resid_norm(const ResidNormParams &q, hipStream_t s) {
    const int threads = (q.dim / 4 + 63) / 64 * 64;
    hipLaunchKernelGGL((resid_norm_kernel<TY, TO>), dim3((unsigned)q.rows), dim3(threads), 0, s, q);
}

template <typename TG, typename TO>
void launch_cgu_mix(const CguMixParams &q, int act, hipStream_t s) {
    const dim3 grid(flat_blocks(q.rows * (q.hid / 4)));
    if (act == 1) hipLaunchKernelGGL((cgu_mix_kernel<TG, TO, 1>), grid, dim3(THREADS), 0, s, q);
    else if (act == 2) hipLaunchKernelGGL((cgu_mix_kernel<TG, TO, 2>), grid, dim3(THREADS), 0, s, q);
    else hipLaunchKernelGGL((cgu_mix_kernel<TG, TO, 3>), grid, dim3(THREADS), 0, s, q);
}

}  // namespace
}  // namespace cplx
}  // namespace qpam

extern "C" size_t qpam_cplx_workspace_size(const qpam_cplx_args *a) {
    using namespace qpam::cplx;
    if (!a || a->rows <= 0 || a->dim <= 0) return 0;
    // partials of the kernel the call runs: the row-team grid (16-byte aligned
    // operands) or one block per four rows; sized for the larger, so the size
    // does not depend on the pointers
    int blocks = row_blocks(a->rows);
    if (const int tt = team_threads(a->dim))
        blocks = std::max(blocks, team_blocks(a->rows, tt, std::min(TEAM_ROWS_NORM_BWD, TEAM_ROWS_ACT_BWD)));
    return (size_t)blocks * n_params(a->op) * a->dim * sizeof(float);
}

extern "C" int qpam_cplx_fwd(const qpam_cplx_args *a, void *stream) {
    using namespace qpam::cplx;
    int st = validate(a, "qpam_cplx_fwd", false);
    if (st) return st;
    if (a->rows == 0) return QPAM_OK;
    return a->dtype == QPAM_BF16 ? fwd_t<unsigned short>(a, (hipStream_t)stream) : fwd_t<float>(a, (hipStream_t)stream);
}

extern "C" int qpam_cplx_bwd(const qpam_cplx_args *a, void *stream) {
    using namespace qpam::cplx;
    int st = validate(a, "qpam_cplx_bwd", true);
    if (st) return st;
    if (a->rows == 0) {
        // no rows: parameter gradients are zero (a sum over zero blocks; a kernel,
        // not a memset, so that the call can be captured in a HIP graph)
        const int n = n_params(a->op) * a->dim;
        if (n > 0)
            hipLaunchKernelGGL(partial_sum_kernel, dim3((n + 63) / 64), dim3(SUM_THREADS), 0, (hipStream_t)stream,
                               (const float *)nullptr, 0, n, a->gp0, a->gp1, a->dim);
        return n > 0 ? qpam::launch_status("qpam_cplx_bwd (zero parameter gradients)") : QPAM_OK;
    }
    return a->dtype == QPAM_BF16 ? bwd_t<unsigned short>(a, (hipStream_t)stream) : bwd_t<float>(a, (hipStream_t)stream);
}

extern "C" int qpam_resid_norm(const qpam_resid_norm_args *a, void *stream) {
    using namespace qpam::cplx;
    QPAM_REQUIRE(a != nullptr, "qpam_resid_norm: null arguments");
    QPAM_REQUIRE(a->rows >= 0 && a->rows <= INT32_MAX, "qpam_resid_norm: rows = %lld", (long long)a->rows);
    QPAM_REQUIRE(a->dim >= 4 && a->dim % 4 == 0 && a->dim <= 4 * TEAM_MAX,
                 "qpam_resid_norm: dim %d must be a multiple of 4 and at most %d", a->dim, 4 * TEAM_MAX);
    QPAM_REQUIRE(a->out_dtype == QPAM_F32 || a->out_dtype == QPAM_BF16, "qpam_resid_norm: out_dtype %d", a->out_dtype);
    QPAM_REQUIRE(a->y == nullptr || a->y_dtype == QPAM_F32 || a->y_dtype == QPAM_BF16,
                 "qpam_resid_norm: y_dtype %d", a->y_dtype);
    if (a->rows == 0) return QPAM_OK;
    QPAM_REQUIRE(a->x && a->out && a->norm_scale && al16(a->x) && al16(a->out) && al16(a->norm_scale),
                 "qpam_resid_norm: x, out and norm_scale must be set and 16-byte aligned");
    QPAM_REQUIRE(a->ldx >= 2 * a->dim && a->ldx % 4 == 0 && a->ldo >= 2 * a->dim && a->ldo % elems16(a->out_dtype) == 0,
                 "qpam_resid_norm: row strides must cover a row and keep 16-byte row starts");
    QPAM_REQUIRE(a->y == nullptr || (a->y_scale && al16(a->y) && a->ldy >= 2 * a->dim && a->ldy % elems16(a->y_dtype) == 0),
                 "qpam_resid_norm: y needs y_scale, 16-byte row starts and a row stride covering a row");
    QPAM_REQUIRE(a->out != (void *)a->x && a->out != a->y, "qpam_resid_norm: out may not alias x or y");
    ResidNormParams q{a->rows, a->dim, a->eps, a->x, a->ldx, a->y, a->ldy, a->y_scale, a->norm_scale, a->out, a->ldo};
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool ybf = a->y && a->y_dtype == QPAM_BF16, obf = a->out_dtype == QPAM_BF16;
    if (ybf && obf) launch_resid_norm<unsigned short, unsigned short>(q, s);
    else if (ybf) launch_resid_norm<unsigned short, float>(q, s);
    else if (obf) launch_resid_norm<float, unsigned short>(q, s);
    else launch_resid_norm<float, float>(q, s);
    return qpam::launch_status("qpam_resid_norm");
}

extern "C" int qpam_cgu_mix(const qpam_cgu_mix_args *a, void *stream) {
    using namespace qpam::cplx;
    QPAM_REQUIRE(a != nullptr, "qpam_cgu_mix: null arguments");
    QPAM_REQUIRE(a->rows >= 0 && a->hid >= 4 && a->hid % 4 == 0, "qpam_cgu_mix: rows %lld, hid %d (a multiple of 4)",
                 (long long)a->rows, a->hid);
    QPAM_REQUIRE((a->gu_dtype == QPAM_F32 || a->gu_dtype == QPAM_BF16) && (a->out_dtype == QPAM_F32 || a->out_dtype == QPAM_BF16),
                 "qpam_cgu_mix: gu_dtype %d / out_dtype %d", a->gu_dtype, a->out_dtype);
    QPAM_REQUIRE((a->phase_alpha == nullptr) == (a->phase_beta == nullptr),
                 "qpam_cgu_mix: phase_alpha and phase_beta are given together");
    QPAM_REQUIRE(a->phase_alpha == nullptr || a->beta != nullptr, "qpam_cgu_mix: the phase-modulated activation needs beta");
    if (a->rows == 0) return QPAM_OK;
    QPAM_REQUIRE(a->gu && a->out && a->bias && al16(a->gu) && al16(a->out) && al16(a->bias) &&
                     (a->beta == nullptr || al16(a->beta)) && (a->phase_alpha == nullptr || (al16(a->phase_alpha) && al16(a->phase_beta))),
                 "qpam_cgu_mix: gu, out and the parameters must be set and 16-byte aligned");
    QPAM_REQUIRE(a->ldg >= 4 * (int64_t)a->hid && a->ldg % elems16(a->gu_dtype) == 0 && a->ldo >= 2 * (int64_t)a->hid &&
                     a->ldo % elems16(a->out_dtype) == 0,
                 "qpam_cgu_mix: row strides must cover a row and keep 16-byte row starts");
    const int act = a->beta == nullptr ? 2 : a->phase_alpha == nullptr ? 1 : 3;
    CguMixParams q{a->rows, a->hid, a->gu, a->ldg, a->bias, a->beta, a->phase_alpha, a->phase_beta, a->out, a->ldo};
    hipStream_t s = static_cast<hipStream_t>(stream);
    const bool gbf = a->gu_dtype == QPAM_BF16, obf = a->out_dtype == QPAM_BF16;
    if (gbf && obf) launch_cgu_mix<unsigned short, unsigned short>(q, act, s);
    else if (gbf) launch_cgu_mix<unsigned short, float>(q, act, s);
    else if (obf) launch_cgu_mix<float, unsigned short>(q, act, s);
    else launch_cgu_mix<float, float>(q, act, s);
    return qpam::launch_status("qpam_cgu_mix");
}
