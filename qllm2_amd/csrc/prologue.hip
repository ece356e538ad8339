// PAM layer prologue: projections -> scan inputs in one HBM pass, and its
// backward.
//
// Reference semantics (v11/model.py): _project's RoPE product and optional
// qk-norm (:290-305), the decay / GSP blend of _gamma_all_and_vprime and
// _gamma_and_vprime (:630-655, :309-347, gamma floor :193-201), and the state
// rotations routing * e^{i phase} of _phase_and_alpha (:230-257) that
// _forward_multistate_fused hands to the chunk loop (:741-746).  The reference
// runs these as separate elementwise passes plus the [B,T,H] -> [B,H,T]
// transposes; here one kernel reads each projection element once and writes
// the scan's planar [B,H,T,d] operands, the decays and the rotations.
//
// Layout: one block of 4 waves per (b, h, 64 consecutive tokens); the
// operand planes are written with ordinary stores (see Element I/O below for
// why not non-temporal ones).  The per-token
// scalars (decays of the M states, protect gate, rotations) take one thread per
// (state, token), so their [M,B,H,T] rows are written as 256-byte runs.  For
// the vectors a token row of d complex elements takes d / 4 lanes (4 elements
// each: one 16-byte fp32 or 8-byte bf16 access per plane; d = 64: a DPP row of
// 16 lanes, 4 tokens per wave step), and a wave covers 16 tokens of the block.
// Head dims 16, 32, 64 and 128.
#include "common.h"

namespace qpam {
namespace {

constexpr int PT = 64;        // tokens per block
constexpr int PTHREADS = 256;

struct Bf16 {};

// Element I/O.  Stores are ordinary (cached) stores: the scan kernels and the
// projection GEMM that read these outputs next find them in the last-level
// cache.  Nontemporal stores make the prologue kernels themselves faster (50 vs
// 72 us forward at the config-3 shape) and the layer step slower (2.31 vs
// 2.25 ms), as do nontemporal loads of the projection just written by the GEMM.
template <typename T> struct Io;
typedef unsigned uintx2 __attribute__((ext_vector_type(2)));

template <> struct Io<float> {
    typedef floatx4 Raw;    // four elements as loaded
    __device__ __forceinline__ static Raw load_raw(const void *base, int64_t off) {
        return *reinterpret_cast<const floatx4 *>(static_cast<const float *>(base) + off);
    }
    __device__ __forceinline__ static void unpack(const Raw &v, float (&o)[4]) {
        o[0] = v.x, o[1] = v.y, o[2] = v.z, o[3] = v.w;
    }
    __device__ __forceinline__ static float load1(const void *base, int64_t off) {
        return static_cast<const float *>(base)[off];
    }
    __device__ __forceinline__ static void store1(void *base, int64_t off, float v) {
        static_cast<float *>(base)[off] = v;
    }
    __device__ __forceinline__ static void load4(const void *base, int64_t off, float (&o)[4]) {
        const floatx4 v = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(base) + off);
        o[0] = v.x, o[1] = v.y, o[2] = v.z, o[3] = v.w;
    }
    __device__ __forceinline__ static void store4(void *base, int64_t off, const float (&v)[4]) {
        *reinterpret_cast<floatx4 *>(static_cast<float *>(base) + off) = floatx4{v[0], v[1], v[2], v[3]};
    }
};
template <> struct Io<Bf16> {
    typedef uintx2 Raw;
    __device__ __forceinline__ static Raw load_raw(const void *base, int64_t off) {
        return *reinterpret_cast<const uintx2 *>(static_cast<const unsigned short *>(base) + off);
    }
    __device__ __forceinline__ static void unpack(const Raw &v, float (&o)[4]) {
        o[0] = __uint_as_float(v.x << 16), o[1] = __uint_as_float(v.x & 0xffff0000u);
        o[2] = __uint_as_float(v.y << 16), o[3] = __uint_as_float(v.y & 0xffff0000u);
    }
    __device__ __forceinline__ static float load1(const void *base, int64_t off) {
        return bf16_to_f32(static_cast<const unsigned short *>(base)[off]);
    }
    __device__ __forceinline__ static void store1(void *base, int64_t off, float v) {
        static_cast<unsigned short *>(base)[off] = f32_to_bf16(v);
    }
    __device__ __forceinline__ static void load4(const void *base, int64_t off, float (&o)[4]) {
        const uint2 v = *reinterpret_cast<const uint2 *>(static_cast<const unsigned short *>(base) + off);
        o[0] = __uint_as_float(v.x << 16), o[1] = __uint_as_float(v.x & 0xffff0000u);
        o[2] = __uint_as_float(v.y << 16), o[3] = __uint_as_float(v.y & 0xffff0000u);
    }
    __device__ __forceinline__ static void store4(void *base, int64_t off, const float (&v)[4]) {
        const uintx2 w = {pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        *reinterpret_cast<uintx2 *>(static_cast<unsigned short *>(base) + off) = w;
    }
};

__device__ __forceinline__ float softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float sigmoid(float x) { return 1.f / (1.f + expf(-x)); }

// element i of a parameter vector in param_dtype
__device__ __forceinline__ float param_at(const void *p, int32_t dtype, int i) {
    return dtype == QPAM_BF16 ? bf16_to_f32(static_cast<const unsigned short *>(p)[i]) : static_cast<const float *>(p)[i];
}

// decay logit of state m: dt + dt_bias (+ dt_bias2) + state_offset
template <typename TI>
__device__ __forceinline__ float pre_sum(const qpam_prologue_args &a, int b, int t, int h, int m) {
    float bias = param_at(a.dt_bias, a.param_dtype, h);
    if (a.dt_bias2) bias += param_at(a.dt_bias2, a.param_dtype, h);
    return Io<TI>::load1(a.dt, b * a.sd_b + (int64_t)t * a.sd_t + h * a.sd_h) + bias +
           (a.state_offset ? param_at(a.state_offset, a.param_dtype, m) : 0.f);
}

// a logit gradient in dlogit_dtype
__device__ __forceinline__ void store_logit(void *p, int32_t dtype, int64_t o, float v) {
    if (dtype == QPAM_BF16) static_cast<unsigned short *>(p)[o] = f32_to_bf16(v);
    else static_cast<float *>(p)[o] = v;
}

// exp(-softplus(pre)) lifted onto [floor, 1) when floor > 0
__device__ __forceinline__ float lifted_decay(const qpam_prologue_args &a, float pre) {
    const float base = expf(-softplus(pre));
    return a.gamma_floor > 0.f ? a.gamma_floor + (1.f - a.gamma_floor) * base : base;
}

template <typename TI>
__device__ __forceinline__ float protect_prob(const qpam_prologue_args &a, int b, int t, int h) {
    return a.protect ? sigmoid(Io<TI>::load1(a.protect, b * a.sp_b + (int64_t)t * a.sp_t + h * a.sp_h)) : 0.f;
}

// routing weight and e^{i phase} of state m at (b, t, h)
template <typename TI>
__device__ __forceinline__ void rotation(const qpam_prologue_args &a, int b, int t, int h, int m, float &r, float &cs,
                                         float &sn) {
    const int64_t po = b * a.sr_b + (int64_t)t * a.sr_t + h * a.sr_h + m * a.sr_m;
    r = a.routing ? Io<TI>::load1(a.routing, po) : 1.f;
    sincosf(Io<TI>::load1(a.phase, po), &sn, &cs);
}

// sum over the d / 4 lanes of a token row (lanes of a row are consecutive and
// aligned): quad, half-row and row DPP steps, and a cross-row step for 32 lanes
template <int LR> __device__ __forceinline__ float row_sum(float x) {
    static_assert(LR == 4 || LR == 8 || LR == 16 || LR == 32, "row of 4 to 32 lanes");
    x += dpp_f<0xB1>(x);
    x += dpp_f<0x4E>(x);
    if constexpr (LR >= 8) x += dpp_f<0x141>(x);
    if constexpr (LR >= 16) x += dpp_f<0x140>(x);
    if constexpr (LR == 32) x += __shfl_xor(x, 16);
    return x;
}

// this lane's 4 rope factors (c, s) for the token at position rope_offset + t
template <int D>
__device__ __forceinline__ void rope4(const qpam_prologue_args &a, int t, int c4, float (&c)[4], float (&s)[4]) {
    const int p = min(max(a.rope_offset + t, 0), a.rope_len - 1);
    const floatx4 *rp = reinterpret_cast<const floatx4 *>(a.rope + ((int64_t)p * D + c4) * 2);
    const floatx4 r0 = rp[0], r1 = rp[1];
    c[0] = r0.x, s[0] = r0.y, c[1] = r0.z, s[1] = r0.w, c[2] = r1.x, s[2] = r1.y, c[3] = r1.z, s[3] = r1.w;
}

__device__ __forceinline__ int64_t tile_count(const qpam_prologue_args &a) { return (a.T + PT - 1) / PT; }

template <int D, typename TI, typename TO>
__global__ void __launch_bounds__(PTHREADS) prologue_fwd_kernel(qpam_prologue_args a) {
    constexpr int LR = D / 4, RW = 64 / LR, ITS = 16 / RW;  // lanes per token row, rows per wave step, steps
    __shared__ float s_keep[PT];
    const int nt = (int)tile_count(a);
    const int bh = blockIdx.x / nt, tile = blockIdx.x - bh * nt;
    const int b = bh / a.H, h = bh - b * a.H;
    const int t0 = tile * PT, tid = threadIdx.x;
    const int w = tid >> 6, lane = tid & 63, c4 = (lane & (LR - 1)) * 4;

    // this lane's projection elements of its ITS tokens, loaded before the
    // scalar work so the loads overlap it (rows past T re-read row T - 1 and
    // are not stored)
    typename Io<TI>::Raw raw[ITS][6];
    const void *planes[6] = {a.q_re, a.q_im, a.k_re, a.k_im, a.v_re, a.v_im};
#pragma unroll
    for (int it = 0; it < ITS; ++it) {
        const int t = min(t0 + w * 16 + it * RW + lane / LR, a.T - 1);
        const int64_t xo = b * a.sx_b + (int64_t)t * a.sx_t + h * a.sx_h + c4;
#pragma unroll
        for (int pl = 0; pl < 6; ++pl) raw[it][pl] = Io<TI>::load_raw(planes[pl], xo);
    }

    {   // scalars: thread = (state m, token)
        const int tt = tid & (PT - 1), m = tid / PT, t = t0 + tt;
        if (t < a.T) {
            const float p = protect_prob<TI>(a, b, t, h);
            if (m == 0) s_keep[tt] = 1.f - p;
            if (m < a.M) {
                const float base = lifted_decay(a, pre_sum<TI>(a, b, t, h, m));
                const int64_t o = (((int64_t)m * a.B + b) * a.H + h) * a.T + t;
                a.gamma[o] = base * (1.f - p) + p;
                if (a.phase) {
                    float r, cs, sn;
                    rotation<TI>(a, b, t, h, m, r, cs, sn);
                    a.rot_re[o] = r * cs;
                    a.rot_im[o] = r * sn;
                }
            }
        }
    }
    __syncthreads();

#pragma unroll
    for (int it = 0; it < ITS; ++it) {
        const int tt = w * 16 + it * RW + lane / LR, t = t0 + tt;
        if (t >= a.T) continue;
        float qr[4], qi[4], kr[4], ki[4], vr[4], vi[4];
        Io<TI>::unpack(raw[it][0], qr), Io<TI>::unpack(raw[it][1], qi);
        Io<TI>::unpack(raw[it][2], kr), Io<TI>::unpack(raw[it][3], ki);
        Io<TI>::unpack(raw[it][4], vr), Io<TI>::unpack(raw[it][5], vi);
        if (a.rope) {
            float c[4], s[4];
            rope4<D>(a, t, c4, c, s);
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float q0 = qr[j], k0 = kr[j];
                qr[j] = q0 * c[j] - qi[j] * s[j], qi[j] = q0 * s[j] + qi[j] * c[j];
                kr[j] = k0 * c[j] - ki[j] * s[j], ki[j] = k0 * s[j] + ki[j] * c[j];
            }
        }
        if (a.qk_norm) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float iq = 1.f / sqrtf(qr[j] * qr[j] + qi[j] * qi[j] + 1e-8f);
                const float ik = 1.f / sqrtf(kr[j] * kr[j] + ki[j] * ki[j] + 1e-8f);
                qr[j] *= iq, qi[j] *= iq, kr[j] *= ik, ki[j] *= ik;
            }
        }
        const float keep = s_keep[tt];
#pragma unroll
        for (int j = 0; j < 4; ++j) vr[j] *= keep, vi[j] *= keep;
        const int64_t oo = (((int64_t)b * a.H + h) * a.T + t) * D + c4;
        Io<TO>::store4(a.oq_re, oo, qr), Io<TO>::store4(a.oq_im, oo, qi);
        Io<TO>::store4(a.ok_re, oo, kr), Io<TO>::store4(a.ok_im, oo, ki);
        Io<TO>::store4(a.ov_re, oo, vr), Io<TO>::store4(a.ov_im, oo, vi);
    }
}

// Backward of z -> nrm(z * r) for one element: g is dL/d(output); returns
// dL/dz.  With u = z r (|r| = 1), nrm(u) = u / m, m = sqrt(|u|^2 + 1e-8):
// du = g / m - u (g.u) / m^3, then dz = du * conj(r).
__device__ __forceinline__ void rope_norm_bwd(float zr, float zi, float c, float s, bool rope, bool norm, float &gr,
                                              float &gi) {
    if (norm) {
        const float ur = rope ? zr * c - zi * s : zr, ui = rope ? zr * s + zi * c : zi;
        const float im = 1.f / sqrtf(ur * ur + ui * ui + 1e-8f);
        const float dot = (gr * ur + gi * ui) * im * im;
        gr = (gr - ur * dot) * im;
        gi = (gi - ui * dot) * im;
    }
    if (rope) {
        const float r0 = gr;
        gr = r0 * c + gi * s;
        gi = gi * c - r0 * s;
    }
}

// Backward layout: one block of 4 waves per (b, 16 consecutive tokens) and all
// heads, so the projection gradients are written as whole rows of the
// projection matrix (writes of 128-byte pieces spread over the rows, as a
// per-head block would make them, measured twice as slow).  A (token, head)
// row of d complex elements takes d / 4 lanes (d = 64: one DPP row of 16
// lanes, 16 rows per pass), BWD_PASSES passes' loads issued before their
// arithmetic.  The per-(token, head,
// state) scalars are computed in token order (coalesced reads of the [M,B,H,T]
// gradients), kept in LDS, and written state-fastest to the [B,T,H,M] outputs.
constexpr int BT = 16;
// passes of 16 rows whose loads are issued before their arithmetic: two keep the
// kernel at four waves per SIMD (110 registers), so the 1024 blocks of a
// B = 8, T = 2048 backward are resident at once; four (147 registers, three
// waves per SIMD) left a third-full second round: 105 -> 96 us at that shape
constexpr int BWD_PASSES = 2;

template <int D, typename TI, typename TO>
__global__ void __launch_bounds__(PTHREADS, 4) prologue_bwd_kernel(qpam_prologue_bwd_args g, qpam_prologue_args a) {
    constexpr int LR = D / 4, RPP = PTHREADS / LR;  // lanes per row, rows per pass
    extern __shared__ float lds[];
    const int rows = BT * a.H, M = a.M;
    float *s_keep = lds, *s_gvv = lds + rows;
    float *s_dpre = lds + 2 * rows, *s_dpm = s_dpre + M * rows, *s_dph = s_dpm + M * rows, *s_dro = s_dph + M * rows;
    const int ntile = (a.T + BT - 1) / BT;
    const int b = blockIdx.x / ntile, t0 = (blockIdx.x - b * ntile) * BT;
    const int tid = threadIdx.x, lane = tid & 63, c4 = (lane & (LR - 1)) * 4, slot = tid / LR;

    for (int r = tid; r < rows; r += PTHREADS) {  // row r = token-in-tile * H + head
        const int tt = r / a.H, h = r - tt * a.H, t = t0 + tt;
        s_keep[r] = t < a.T ? 1.f - protect_prob<TI>(a, b, t, h) : 1.f;
    }
    __syncthreads();

    const bool rope = a.rope != nullptr, norm = a.qk_norm != 0;
    const void *gplanes[6] = {g.gq_re, g.gq_im, g.gk_re, g.gk_im, g.gv_re, g.gv_im};
    for (int r0 = 0; r0 < rows; r0 += RPP * BWD_PASSES) {
        typename Io<TO>::Raw graw[BWD_PASSES][6];
        typename Io<TI>::Raw vraw[BWD_PASSES][2];
#pragma unroll
        for (int k = 0; k < BWD_PASSES; ++k) {   // rows past the tile re-read a valid row and are not stored
            const int r = min(r0 + RPP * k + slot, rows - 1);
            const int tt = r / a.H, h = r - tt * a.H, t = min(t0 + tt, a.T - 1);
            const int64_t oo = (((int64_t)b * a.H + h) * a.T + t) * D + c4;
            const int64_t xo = b * a.sx_b + (int64_t)t * a.sx_t + h * a.sx_h + c4;
#pragma unroll
            for (int pl = 0; pl < 6; ++pl) graw[k][pl] = Io<TO>::load_raw(gplanes[pl], oo);
            vraw[k][0] = Io<TI>::load_raw(a.v_re, xo);
            vraw[k][1] = Io<TI>::load_raw(a.v_im, xo);
        }
#pragma unroll
        for (int k = 0; k < BWD_PASSES; ++k) {
            const int r = r0 + RPP * k + slot;
            const int tt = r / a.H, h = r - tt * a.H, t = t0 + tt;
            // the lanes of a row share r, so they are either all in or all out
            if (r >= rows || t >= a.T) continue;
            const int64_t xo = b * a.sx_b + (int64_t)t * a.sx_t + h * a.sx_h + c4;
            const int64_t go = b * g.sg_b + (int64_t)t * g.sg_t + h * g.sg_h + c4;
            float gqr[4], gqi[4], gkr[4], gki[4], gvr[4], gvi[4], vr[4], vi[4];
            Io<TO>::unpack(graw[k][0], gqr), Io<TO>::unpack(graw[k][1], gqi);
            Io<TO>::unpack(graw[k][2], gkr), Io<TO>::unpack(graw[k][3], gki);
            Io<TO>::unpack(graw[k][4], gvr), Io<TO>::unpack(graw[k][5], gvi);
            Io<TI>::unpack(vraw[k][0], vr), Io<TI>::unpack(vraw[k][1], vi);
            if (rope || norm) {
                float c[4] = {1.f, 1.f, 1.f, 1.f}, sn[4] = {0.f, 0.f, 0.f, 0.f};
                if (rope) rope4<D>(a, t, c4, c, sn);
                float qr[4], qi[4], kr[4], ki[4];
                if (norm) {
                    Io<TI>::load4(a.q_re, xo, qr), Io<TI>::load4(a.q_im, xo, qi);
                    Io<TI>::load4(a.k_re, xo, kr), Io<TI>::load4(a.k_im, xo, ki);
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    rope_norm_bwd(norm ? qr[j] : 0.f, norm ? qi[j] : 0.f, c[j], sn[j], rope, norm, gqr[j], gqi[j]);
                    rope_norm_bwd(norm ? kr[j] : 0.f, norm ? ki[j] : 0.f, c[j], sn[j], rope, norm, gkr[j], gki[j]);
                }
            }
            const float keep = s_keep[r];
            float dot = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                dot += gvr[j] * vr[j] + gvi[j] * vi[j];
                gvr[j] *= keep, gvi[j] *= keep;
            }
            dot = row_sum<LR>(dot);
            if ((lane & (LR - 1)) == 0) s_gvv[r] = dot;
            Io<TI>::store4(g.dq_re, go, gqr), Io<TI>::store4(g.dq_im, go, gqi);
            Io<TI>::store4(g.dk_re, go, gkr), Io<TI>::store4(g.dk_im, go, gki);
            Io<TI>::store4(g.dv_re, go, gvr), Io<TI>::store4(g.dv_im, go, gvi);
        }
    }

    // scalars, token-fastest over (state, head, token)
    const int items = M * rows;
    const float lift = a.gamma_floor > 0.f ? 1.f - a.gamma_floor : 1.f;
    for (int i = tid; i < items; i += PTHREADS) {
        const int tt = i % BT, mh = i / BT, h = mh % a.H, m = mh / a.H, t = t0 + tt;
        const int r = tt * a.H + h;
        float dpre = 0.f, dpm = 0.f, dph = 0.f, dro = 0.f;
        if (t < a.T) {
            const int64_t o = (((int64_t)m * a.B + b) * a.H + h) * a.T + t;
            const float p = 1.f - s_keep[r];
            // d gamma / d pre = (1 - p) (1 - floor) (-exp(-softplus(pre))) softplus'(pre)
            const float pre = pre_sum<TI>(a, b, t, h, m);
            const float raw = expf(-softplus(pre));
            const float dsp = pre > 20.f ? 1.f : sigmoid(pre);
            const float gg = g.ggamma[o];
            dpre = -gg * (1.f - p) * lift * raw * dsp;
            dpm = gg * (1.f - lifted_decay(a, pre));  // d gamma_m / d p = 1 - base_m
            if (a.phase) {
                float rr, cs, sn;
                rotation<TI>(a, b, t, h, m, rr, cs, sn);
                const float gr = g.grot_re[o], gi = g.grot_im[o];
                dph = rr * (gi * cs - gr * sn);
                dro = gr * cs + gi * sn;
            }
        }
        s_dpre[m * rows + r] = dpre, s_dpm[m * rows + r] = dpm, s_dph[m * rows + r] = dph, s_dro[m * rows + r] = dro;
    }
    __syncthreads();
    const bool sums = g.dbias || g.doffset;
    // logit-gradient strides (all zero: the contiguous layouts)
    const bool qdef = (g.sdq_b | g.sdq_t | g.sdq_h | g.sdq_m) == 0, pdef = (g.sdp_b | g.sdp_t | g.sdp_h) == 0;
    const int64_t qb = qdef ? (int64_t)a.T * a.H * M : g.sdq_b, qt = qdef ? (int64_t)a.H * M : g.sdq_t,
                  qh = qdef ? M : g.sdq_h, qm = qdef ? 1 : g.sdq_m;
    const int64_t pb = pdef ? (int64_t)a.T * a.H : g.sdp_b, pt = pdef ? a.H : g.sdp_t, ph = pdef ? 1 : g.sdp_h;
    for (int i = tid; i < items; i += PTHREADS) {   // state-fastest: contiguous [B,T,H,M] rows
        const int m = i % M, r = i / M, tt = r / a.H, h = r - tt * a.H, t = t0 + tt;
        if (t >= a.T) continue;
        if (!sums) g.dpre[(((int64_t)b * a.T + t) * a.H + h) * M + m] = s_dpre[m * rows + r];
        if (a.phase) {
            const int64_t o = b * qb + (int64_t)t * qt + h * qh + m * qm;
            store_logit(g.dphase, g.dlogit_dtype, o, s_dph[m * rows + r]);
            if (g.drouting) store_logit(g.drouting, g.dlogit_dtype, o, s_dro[m * rows + r]);
        }
    }
    if (sums) {  // this block's sums of dpre over its tokens, per (h, m), in token order
        const int hm = a.H * M, valid = min(BT, a.T - t0);
        for (int j = tid; j < hm; j += PTHREADS) {
            const int h = j / M, m = j - h * M;
            float x = 0.f;
            for (int tt = 0; tt < valid; ++tt) x += s_dpre[m * rows + tt * a.H + h];
            g.dpre[(int64_t)blockIdx.x * hm + j] = x;
        }
    }
    for (int r = tid; r < rows; r += PTHREADS) {
        const int tt = r / a.H, h = r - tt * a.H, t = t0 + tt;
        if (t >= a.T) continue;
        float ddt = 0.f, dp = -s_gvv[r];             // d v' / d p = -v
        for (int m = 0; m < M; ++m) ddt += s_dpre[m * rows + r], dp += s_dpm[m * rows + r];
        if (g.ddt) {
            const int64_t o = b * g.sdd_b + (int64_t)t * g.sdd_t + h * g.sdd_h;
            Io<TI>::store1(g.ddt, o, ddt);
            if (h == a.H - 1)  // the padding columns after dt's
                for (int k = 1; k <= g.ddt_pad; ++k) Io<TI>::store1(g.ddt, o + k * g.sdd_h, 0.f);
        }
        if (a.protect) {
            const float p = 1.f - s_keep[r];
            store_logit(g.dprotect, g.dlogit_dtype, b * pb + (int64_t)t * pt + h * ph, dp * p * (1.f - p));
        }
    }
}

// d dt_bias [H] and d state_offset [M] from the per-block partial sums
// part[blocks][H M] of the backward, in one block: thread (group g, column j)
// sums the rows of its group's contiguous range in row order (its loads all in
// flight), the groups' sums are added in group order per column, then over m
// (dbias) and over h (doffset) in index order -- a fixed order throughout
constexpr int BIAS_THREADS = 1024;
__global__ void __launch_bounds__(BIAS_THREADS) prologue_bias_grad_kernel(const float *part, int blocks, int H, int M,
                                                                          int32_t dtype, void *dbias, void *doffset) {
    extern __shared__ float red[];  // [groups][H M], then the column sums
    const int hm = H * M, groups = max(1, BIAS_THREADS / hm), per = (blocks + groups - 1) / groups;
    float *col = red + groups * hm;
    for (int i = threadIdx.x; i < groups * hm; i += BIAS_THREADS) {
        const int gr = i / hm, j = i - gr * hm, k1 = min(blocks, (gr + 1) * per);
        float x = 0.f;
#pragma unroll 8
        for (int k = gr * per; k < k1; ++k) x += part[(int64_t)k * hm + j];
        red[i] = x;
    }
    __syncthreads();
    for (int j = threadIdx.x; j < hm; j += BIAS_THREADS) {
        float x = 0.f;
        for (int gr = 0; gr < groups; ++gr) x += red[gr * hm + j];
        col[j] = x;
    }
    __syncthreads();
    for (int h = threadIdx.x; dbias && h < H; h += BIAS_THREADS) {
        float x = 0.f;
        for (int m = 0; m < M; ++m) x += col[h * M + m];
        store_logit(dbias, dtype, h, x);
    }
    for (int m = threadIdx.x; doffset && m < M; m += BIAS_THREADS) {
        float x = 0.f;
        for (int h = 0; h < H; ++h) x += col[h * M + m];
        store_logit(doffset, dtype, m, x);
    }
}
size_t bias_grad_lds(int H, int M) {
    const int hm = H * M, groups = std::max(1, BIAS_THREADS / hm);
    return (size_t)(groups + 1) * hm * sizeof(float);
}

size_t bwd_lds_bytes(const qpam_prologue_args &a) { return (size_t)(2 + 4 * a.M) * BT * a.H * sizeof(float); }

// |z| = sqrt(re^2 + im^2 + 1e-8) of interleaved complex elements, four per
// thread, and its backward dz = g z / |z|
template <typename T>
__global__ void __launch_bounds__(256) cabs_fwd_kernel(int64_t n4, const void *z, void *mag) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    float a[4], b[4], m[4];
    Io<T>::load4(z, 8 * i, a), Io<T>::load4(z, 8 * i + 4, b);
    m[0] = sqrtf(a[0] * a[0] + a[1] * a[1] + 1e-8f), m[1] = sqrtf(a[2] * a[2] + a[3] * a[3] + 1e-8f);
    m[2] = sqrtf(b[0] * b[0] + b[1] * b[1] + 1e-8f), m[3] = sqrtf(b[2] * b[2] + b[3] * b[3] + 1e-8f);
    Io<T>::store4(mag, 4 * i, m);
}

// ACC: gz += (the gradient), the input's other gradient already in gz
template <typename T, bool ACC>
__global__ void __launch_bounds__(256) cabs_bwd_kernel(int64_t n4, const void *z, const void *mag, const void *gmag,
                                                       void *gz) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    float a[4], b[4], m[4], g[4];
    Io<T>::load4(z, 8 * i, a), Io<T>::load4(z, 8 * i + 4, b);
    Io<T>::load4(mag, 4 * i, m), Io<T>::load4(gmag, 4 * i, g);
    float s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = g[j] / m[j];
    a[0] *= s[0], a[1] *= s[0], a[2] *= s[1], a[3] *= s[1];
    b[0] *= s[2], b[1] *= s[2], b[2] *= s[3], b[3] *= s[3];
    if constexpr (ACC) {
        float c[4], e[4];
        Io<T>::load4(gz, 8 * i, c), Io<T>::load4(gz, 8 * i + 4, e);
#pragma unroll
        for (int j = 0; j < 4; ++j) a[j] += c[j], b[j] += e[j];
    }
    Io<T>::store4(gz, 8 * i, a), Io<T>::store4(gz, 8 * i + 4, b);
}

bool aligned(const void *p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

// everything the backward reads of the forward description (not its outputs)
int validate_inputs(const qpam_prologue_args *a) {
    QPAM_REQUIRE(a != nullptr, "qpam_prologue: null arguments");
    QPAM_REQUIRE(a->B >= 0 && a->T >= 0 && a->H >= 1 && a->M >= 1 && a->M <= 4,
                 "qpam_prologue: invalid sizes B=%d T=%d H=%d M=%d (1 <= M <= 4)", a->B, a->T, a->H, a->M);
    QPAM_REQUIRE(a->d == 16 || a->d == 32 || a->d == 64 || a->d == 128,
                 "qpam_prologue: head_dim %d unsupported (16, 32, 64 or 128)", a->d);
    QPAM_REQUIRE((a->in_dtype == QPAM_F32 || a->in_dtype == QPAM_BF16) &&
                     (a->out_dtype == QPAM_F32 || a->out_dtype == QPAM_BF16),
                 "qpam_prologue: dtypes must be QPAM_F32 or QPAM_BF16");
    const int vin = a->in_dtype == QPAM_F32 ? 16 : 8;
    QPAM_REQUIRE(a->q_re && a->q_im && a->k_re && a->k_im && a->v_re && a->v_im && a->dt && a->dt_bias,
                 "qpam_prologue: q, k, v, dt and dt_bias are required");
    QPAM_REQUIRE(aligned(a->q_re, vin) && aligned(a->q_im, vin) && aligned(a->k_re, vin) && aligned(a->k_im, vin) &&
                     aligned(a->v_re, vin) && aligned(a->v_im, vin) && a->sx_b % 4 == 0 && a->sx_t % 4 == 0 &&
                     a->sx_h % 4 == 0,
                 "qpam_prologue: projection planes need %d-byte aligned rows (strides multiple of 4)", vin);
    QPAM_REQUIRE(a->rope == nullptr || (a->rope_len >= 1 && aligned(a->rope, 16)),
                 "qpam_prologue: rope needs rope_len >= 1 and a 16-byte aligned table");
    QPAM_REQUIRE(a->routing == nullptr || a->phase, "qpam_prologue: routing needs phase");
    QPAM_REQUIRE(a->param_dtype == QPAM_F32 || a->param_dtype == QPAM_BF16,
                 "qpam_prologue: param_dtype must be QPAM_F32 or QPAM_BF16");
    return QPAM_OK;
}

int validate_outputs(const qpam_prologue_args *a) {
    const int vout = a->out_dtype == QPAM_F32 ? 16 : 8;
    QPAM_REQUIRE(a->oq_re && a->oq_im && a->ok_re && a->ok_im && a->ov_re && a->ov_im && a->gamma &&
                     aligned(a->oq_re, vout) && aligned(a->oq_im, vout) && aligned(a->ok_re, vout) &&
                     aligned(a->ok_im, vout) && aligned(a->ov_re, vout) && aligned(a->ov_im, vout),
                 "qpam_prologue: outputs q', k', v' (%d-byte aligned) and gamma required", vout);
    QPAM_REQUIRE(a->phase == nullptr || (a->rot_re && a->rot_im), "qpam_prologue: phase given without rot outputs");
    return QPAM_OK;
}


// Gate logits from the magnitudes of the layer input, one row per block:
//   out[r][g] = bias[g] + sum_j w[g][j] |z[r][j]|,  |z| = sqrt(re^2 + im^2 + 1e-8)
// (the protect gate and the phase projection both read cabs(x)).  The rows'
// magnitudes go to LDS once; wave w takes output groups of MAG_G rows of w
// (groups w, w + 4, ...: the protect gate and an E3 phase projection, 12 + 36
// outputs, are one group per wave), its lanes striding over j: per pass over
// 12 x 64 columns (all of a 768-wide row) the 12 MAG_G coalesced loads of w
// are all in flight before any is used; then a butterfly sum per output.
// Decode-time shapes (a few hundred rows, G of tens, dim of hundreds) make
// this a latency problem: a library GEMM of that shape has only a few output
// tiles, and a loop that uses each load as it arrives waits one L2 round trip
// per element step.  Measured at 192 rows x 48 outputs x 768: 45 us with one
// load in flight per lane, 9.4 us with 48, 20.7 us with four rows per block
// (a quarter of the blocks, each four times longer).
constexpr int MAG_THREADS = 256, MAG_MAX_DIM = 4096, MAG_G = 12, MAG_U = 12, MAG_R = 1;
template <typename T, typename To>
__global__ void __launch_bounds__(MAG_THREADS) mag_linear_kernel(int64_t rows, int dim, int G, const void *z,
                                                                 const float *w, const float *bias, void *out,
                                                                 int64_t ld_out) {
    __shared__ float mag[MAG_R][MAG_MAX_DIM];
    const int64_t r0 = (int64_t)blockIdx.x * MAG_R;
    const int nr = (int)min((int64_t)MAG_R, rows - r0);
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63;
    for (int rr = 0; rr < nr; ++rr)
        for (int j = tid; j < dim; j += MAG_THREADS) {
            const int64_t e = ((r0 + rr) * dim + j) * 2;
            const float a = Io<T>::load1(z, e), b = Io<T>::load1(z, e + 1);
            mag[rr][j] = sqrtf(a * a + b * b + 1e-8f);
        }
    __syncthreads();
    for (int g0 = wv * MAG_G; g0 < G; g0 += (MAG_THREADS / 64) * MAG_G) {
        float acc[MAG_R][MAG_G];
#pragma unroll
        for (int rr = 0; rr < MAG_R; ++rr)
#pragma unroll
            for (int k = 0; k < MAG_G; ++k) acc[rr][k] = 0.f;
        for (int j0 = lane; j0 < dim; j0 += 64 * MAG_U) {
            float wk[MAG_U][MAG_G];
#pragma unroll
            for (int u = 0; u < MAG_U; ++u)
#pragma unroll
                for (int k = 0; k < MAG_G; ++k) {
                    const int j = j0 + 64 * u;
                    wk[u][k] = (g0 + k < G && j < dim) ? w[(int64_t)(g0 + k) * dim + j] : 0.f;
                }
#pragma unroll
            for (int u = 0; u < MAG_U; ++u) {
                const int j = j0 + 64 * u;
#pragma unroll
                for (int rr = 0; rr < MAG_R; ++rr) {
                    const float m = (j < dim && rr < nr) ? mag[rr][j] : 0.f;
#pragma unroll
                    for (int k = 0; k < MAG_G; ++k) acc[rr][k] += wk[u][k] * m;
                }
            }
        }
#pragma unroll
        for (int rr = 0; rr < MAG_R; ++rr)
#pragma unroll
            for (int k = 0; k < MAG_G; ++k) {
                float x = acc[rr][k];
#pragma unroll
                for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
                if (lane == 0 && g0 + k < G && rr < nr)
                    Io<To>::store1(out, (r0 + rr) * ld_out + g0 + k, x + (bias ? bias[g0 + k] : 0.f));
            }
    }
}
template <int D>
void launch_fwd(const qpam_prologue_args &a, hipStream_t s) {
    const dim3 grid((unsigned)((long long)a.B * a.H * ((a.T + PT - 1) / PT))), block(PTHREADS);
    const bool fi = a.in_dtype == QPAM_F32, fo = a.out_dtype == QPAM_F32;
    if (fi && fo) hipLaunchKernelGGL((prologue_fwd_kernel<D, float, float>), grid, block, 0, s, a);
    else if (fi) hipLaunchKernelGGL((prologue_fwd_kernel<D, float, Bf16>), grid, block, 0, s, a);
    else if (fo) hipLaunchKernelGGL((prologue_fwd_kernel<D, Bf16, float>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((prologue_fwd_kernel<D, Bf16, Bf16>), grid, block, 0, s, a);
}

template <int D>
void launch_bwd(const qpam_prologue_bwd_args &g, const qpam_prologue_args &a, long long blocks, size_t lds,
                hipStream_t s) {
    const dim3 grid((unsigned)blocks), block(PTHREADS);
    const bool fi = a.in_dtype == QPAM_F32, fo = a.out_dtype == QPAM_F32;
    if (fi && fo) hipLaunchKernelGGL((prologue_bwd_kernel<D, float, float>), grid, block, lds, s, g, a);
    else if (fi) hipLaunchKernelGGL((prologue_bwd_kernel<D, float, Bf16>), grid, block, lds, s, g, a);
    else if (fo) hipLaunchKernelGGL((prologue_bwd_kernel<D, Bf16, float>), grid, block, lds, s, g, a);
    else hipLaunchKernelGGL((prologue_bwd_kernel<D, Bf16, Bf16>), grid, block, lds, s, g, a);
}
}  // namespace
}  // namespace qpam

using namespace qpam;

extern "C" int qpam_prologue_fwd(const qpam_prologue_args *a, void *stream) {
    int st = validate_inputs(a);
    if (!st) st = validate_outputs(a);
    if (st) return st;
    const long long blocks = (long long)a->B * a->H * ((a->T + PT - 1) / PT);
    if (blocks == 0) return QPAM_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (a->d) {
        case 16: launch_fwd<16>(*a, s); break;
        case 32: launch_fwd<32>(*a, s); break;
        case 64: launch_fwd<64>(*a, s); break;
        default: launch_fwd<128>(*a, s);
    }
    return launch_status("prologue_fwd_kernel");
}

extern "C" int qpam_prologue_bwd(const qpam_prologue_bwd_args *g, void *stream) {
    QPAM_REQUIRE(g != nullptr && g->fwd != nullptr, "qpam_prologue_bwd: null arguments");
    const qpam_prologue_args &a = *g->fwd;
    int st = validate_inputs(&a);
    if (st) return st;
    const int vin = a.in_dtype == QPAM_F32 ? 16 : 8, vout = a.out_dtype == QPAM_F32 ? 16 : 8;
    QPAM_REQUIRE(g->gq_re && g->gq_im && g->gk_re && g->gk_im && g->gv_re && g->gv_im && g->ggamma &&
                     aligned(g->gq_re, vout) && aligned(g->gq_im, vout) && aligned(g->gk_re, vout) &&
                     aligned(g->gk_im, vout) && aligned(g->gv_re, vout) && aligned(g->gv_im, vout),
                 "qpam_prologue_bwd: gradients of q', k', v' and gamma required, %d-byte aligned", vout);
    QPAM_REQUIRE(g->dq_re && g->dq_im && g->dk_re && g->dk_im && g->dv_re && g->dv_im && aligned(g->dq_re, vin) &&
                     aligned(g->dq_im, vin) && aligned(g->dk_re, vin) && aligned(g->dk_im, vin) &&
                     aligned(g->dv_re, vin) && aligned(g->dv_im, vin) && g->sg_b % 4 == 0 && g->sg_t % 4 == 0 &&
                     g->sg_h % 4 == 0,
                 "qpam_prologue_bwd: projection gradients required, %d-byte aligned rows", vin);
    QPAM_REQUIRE(g->dpre != nullptr, "qpam_prologue_bwd: dpre required");
    QPAM_REQUIRE(a.protect == nullptr || g->dprotect != nullptr, "qpam_prologue_bwd: dprotect required with protect");
    QPAM_REQUIRE(a.phase == nullptr || (g->grot_re && g->grot_im && g->dphase),
                 "qpam_prologue_bwd: rot gradients and dphase required with phase");
    QPAM_REQUIRE(g->dlogit_dtype == QPAM_F32 || g->dlogit_dtype == QPAM_BF16,
                 "qpam_prologue_bwd: dlogit_dtype must be QPAM_F32 or QPAM_BF16");
    QPAM_REQUIRE(g->ddt_pad >= 0 && (g->ddt_pad == 0 || g->ddt), "qpam_prologue_bwd: ddt_pad needs ddt");
    const size_t lds = bwd_lds_bytes(a);
    QPAM_REQUIRE(lds <= 64 * 1024, "qpam_prologue_bwd: H=%d, M=%d need %zu bytes of LDS (64 KiB max)", a.H, a.M, lds);
    const long long blocks = (long long)a.B * ((a.T + BT - 1) / BT);
    const bool sums = g->dbias || g->doffset;
    QPAM_REQUIRE(!sums || bias_grad_lds(a.H, a.M) <= 64 * 1024,
                 "qpam_prologue_bwd: H * M = %d too large for the bias gradients", a.H * a.M);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (blocks == 0) {
        if (!sums) return QPAM_OK;
        // no tokens: zero gradients (a fill by the same reduction over no blocks)
        hipLaunchKernelGGL(prologue_bias_grad_kernel, dim3(1), dim3(BIAS_THREADS), bias_grad_lds(a.H, a.M), s, g->dpre,
                           0, a.H, a.M, a.param_dtype, g->dbias, g->doffset);
        return launch_status("prologue_bias_grad_kernel");
    }
    switch (a.d) {
        case 16: launch_bwd<16>(*g, a, blocks, lds, s); break;
        case 32: launch_bwd<32>(*g, a, blocks, lds, s); break;
        case 64: launch_bwd<64>(*g, a, blocks, lds, s); break;
        default: launch_bwd<128>(*g, a, blocks, lds, s);
    }
    int st2 = launch_status("prologue_bwd_kernel");
    if (st2 || !sums) return st2;
    hipLaunchKernelGGL(prologue_bias_grad_kernel, dim3(1), dim3(BIAS_THREADS), bias_grad_lds(a.H, a.M), s, g->dpre,
                       (int)blocks, a.H, a.M, a.param_dtype, g->dbias, g->doffset);
    return launch_status("prologue_bias_grad_kernel");
}

extern "C" int qpam_cabs_fwd(int32_t dtype, int64_t n, const void *z, void *mag, void *stream) {
    QPAM_REQUIRE(dtype == QPAM_F32 || dtype == QPAM_BF16, "qpam_cabs_fwd: dtype must be QPAM_F32 or QPAM_BF16");
    QPAM_REQUIRE(n >= 0 && n % 4 == 0, "qpam_cabs_fwd: element count %lld must be a multiple of 4", (long long)n);
    const int va = dtype == QPAM_F32 ? 16 : 8;
    QPAM_REQUIRE(n == 0 || (z && mag && aligned(z, va) && aligned(mag, va)), "qpam_cabs_fwd: %d-byte aligned z, mag required", va);
    if (n == 0) return QPAM_OK;
    const int64_t n4 = n / 4;
    const dim3 grid((unsigned)((n4 + 255) / 256)), block(256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == QPAM_F32) hipLaunchKernelGGL(cabs_fwd_kernel<float>, grid, block, 0, s, n4, z, mag);
    else hipLaunchKernelGGL(cabs_fwd_kernel<Bf16>, grid, block, 0, s, n4, z, mag);
    return launch_status("cabs_fwd_kernel");
}

extern "C" int qpam_cabs_bwd(int32_t dtype, int64_t n, const void *z, const void *mag, const void *gmag, void *gz,
                             void *stream) {
    QPAM_REQUIRE(dtype == QPAM_F32 || dtype == QPAM_BF16, "qpam_cabs_bwd: dtype must be QPAM_F32 or QPAM_BF16");
    QPAM_REQUIRE(n >= 0 && n % 4 == 0, "qpam_cabs_bwd: element count %lld must be a multiple of 4", (long long)n);
    const int va = dtype == QPAM_F32 ? 16 : 8;
    QPAM_REQUIRE(n == 0 || (z && mag && gmag && gz && aligned(z, va) && aligned(mag, va) && aligned(gmag, va) &&
                            aligned(gz, va)),
                 "qpam_cabs_bwd: %d-byte aligned buffers required", va);
    if (n == 0) return QPAM_OK;
    const int64_t n4 = n / 4;
    const dim3 grid((unsigned)((n4 + 255) / 256)), block(256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == QPAM_F32) hipLaunchKernelGGL((cabs_bwd_kernel<float, false>), grid, block, 0, s, n4, z, mag, gmag, gz);
    else hipLaunchKernelGGL((cabs_bwd_kernel<Bf16, false>), grid, block, 0, s, n4, z, mag, gmag, gz);
    return launch_status("cabs_bwd_kernel");
}

extern "C" int qpam_cabs_bwd_acc(int32_t dtype, int64_t n, const void *z, const void *mag, const void *gmag, void *gz,
                                 void *stream) {
    QPAM_REQUIRE(dtype == QPAM_F32 || dtype == QPAM_BF16, "qpam_cabs_bwd_acc: dtype must be QPAM_F32 or QPAM_BF16");
    QPAM_REQUIRE(n >= 0 && n % 4 == 0, "qpam_cabs_bwd_acc: element count %lld must be a multiple of 4", (long long)n);
    const int va = dtype == QPAM_F32 ? 16 : 8;
    QPAM_REQUIRE(n == 0 || (z && mag && gmag && gz && aligned(z, va) && aligned(mag, va) && aligned(gmag, va) &&
                            aligned(gz, va)),
                 "qpam_cabs_bwd_acc: %d-byte aligned buffers required", va);
    if (n == 0) return QPAM_OK;
    const int64_t n4 = n / 4;
    const dim3 grid((unsigned)((n4 + 255) / 256)), block(256);
    hipStream_t s = static_cast<hipStream_t>(stream);
    if (dtype == QPAM_F32) hipLaunchKernelGGL((cabs_bwd_kernel<float, true>), grid, block, 0, s, n4, z, mag, gmag, gz);
    else hipLaunchKernelGGL((cabs_bwd_kernel<Bf16, true>), grid, block, 0, s, n4, z, mag, gmag, gz);
    return launch_status("cabs_bwd_kernel");
}

extern "C" int qpam_mag_linear(int32_t dtype, int32_t out_dtype, int64_t rows, int32_t dim, int32_t G, const void *z,
                               const float *w, const float *bias, void *out, int64_t ld_out, void *stream) {
    QPAM_REQUIRE((dtype == QPAM_F32 || dtype == QPAM_BF16) && (out_dtype == QPAM_F32 || out_dtype == QPAM_BF16),
                 "qpam_mag_linear: dtypes must be QPAM_F32 or QPAM_BF16");
    QPAM_REQUIRE(rows >= 0 && rows < (1ll << 31) && dim >= 1 && dim <= MAG_MAX_DIM && G >= 1 && ld_out >= G,
                 "qpam_mag_linear: bad sizes rows=%lld dim=%d G=%d ld_out=%lld (dim <= %d)", (long long)rows, dim, G,
                 (long long)ld_out, MAG_MAX_DIM);
    if (rows == 0) return QPAM_OK;
    QPAM_REQUIRE(z && w && out, "qpam_mag_linear: null z, w or out");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid((unsigned)((rows + MAG_R - 1) / MAG_R)), block(MAG_THREADS);
    if (dtype == QPAM_F32) {
        if (out_dtype == QPAM_F32)
            hipLaunchKernelGGL((mag_linear_kernel<float, float>), grid, block, 0, s, rows, dim, G, z, w, bias, out, ld_out);
        else hipLaunchKernelGGL((mag_linear_kernel<float, Bf16>), grid, block, 0, s, rows, dim, G, z, w, bias, out, ld_out);
    } else {
        if (out_dtype == QPAM_F32)
            hipLaunchKernelGGL((mag_linear_kernel<Bf16, float>), grid, block, 0, s, rows, dim, G, z, w, bias, out, ld_out);
        else hipLaunchKernelGGL((mag_linear_kernel<Bf16, Bf16>), grid, block, 0, s, rows, dim, G, z, w, bias, out, ld_out);
    }
    return launch_status("mag_linear_kernel");
}
