// E2 delta-rule write of the PAM layer, forward and backward (fp32).
//
// Reference semantics: V11PAMLayer._forward_delta (v11/model.py:491-576), the
// chunked UT-transform form, whose result is the token recurrence
//     S <- g~_t S;  p = S k_t;  u = beta_t (v_t - p);  S <- S + u (x) k_t*;
//     y_t = S q~_t                       (g~ = gamma + 1e-6, q~ = q_scale q)
// (its per-chunk solve (I + M) U = W with M[t,s] = beta_t D[t,s] k_t.k_s* is
// exactly this recurrence unrolled over the chunk; _recur_step_delta,
// v11/model.py:967-1002, is the same step with g~ = gamma).
//
// Design: the rows of S are independent under the recurrence (row i reads
// only k, q, v_i, gamma, beta), so one block of 8 waves owns one (b, h) chain
// and each lane owns 2 rows x 4 columns of the 64 x 64 complex state in
// registers; the per-row dot products S k and S q~ are DPP reductions over the
// 16 lanes of a row group, and no other communication happens in the forward.
// A token costs ~100 dependent VALU/DPP operations and no solve; the chunked
// form's O(C^2 d + C^3) per-chunk work (the Gram matrix, the 2C x 2C real
// solve, the dual-form products) is not needed on a GPU whose state fits in
// the registers of one block.  The forward stores the state before every
// 16th token (the backward's checkpoints).
//
// Backward: blocks walk the chains' 16-token groups in reverse; each group is
// recomputed from its checkpoint with the state before every 4th token kept in
// a per-block scratch, then each 4-token sub-group is recomputed into
// registers and differentiated in reverse.  Gradients of k, q, gamma and beta
// are sums over the 64 rows: lanes -> row groups by shuffles, waves through
// LDS once per sub-group, in a fixed order (deterministic).
#include "common.h"

namespace qpam {
namespace {

constexpr int D = 64;
constexpr int DTHREADS = 512;   // 8 waves x 8 rows
constexpr int GROUP = 16;       // tokens per forward checkpoint
constexpr int SUB = 4;          // tokens per backward sub-group
constexpr int SUBS = GROUP / SUB;

struct Lane {
    int w, rg, cg, r0;   // wave, row group (0..3), column group (0..15), first row
    __device__ Lane(int tid) {
        w = tid >> 6;
        const int lane = tid & 63;
        rg = lane >> 4, cg = lane & 15;
        r0 = 8 * w + 2 * rg;
    }
};

// one token's inputs as this lane sees them
struct Tok {
    float kr[4], ki[4], qr[4], qi[4];  // the lane's 4 columns (q already scaled)
    float vr[2], vi[2];                // the lane's 2 rows
    float g, b;                        // gamma + eps, beta
};

struct State {
    float r[2][4], i[2][4];
};

__device__ __forceinline__ Tok load_tok(const qpam_delta_args &a, int b, int h, int t, const Lane &L) {
    Tok x;
    const int64_t kq = b * a.k.s0 + h * a.k.s1 + (int64_t)t * a.k.s2 + 4 * L.cg;
    const int64_t qq = b * a.q.s0 + h * a.q.s1 + (int64_t)t * a.q.s2 + 4 * L.cg;
    const int64_t vv = b * a.v.s0 + h * a.v.s1 + (int64_t)t * a.v.s2 + L.r0;
    const floatx4 kr = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(a.k.re) + kq);
    const floatx4 ki = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(a.k.im) + kq);
    const floatx4 qr = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(a.q.re) + qq);
    const floatx4 qi = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(a.q.im) + qq);
    const floatx2 vr = *reinterpret_cast<const floatx2 *>(static_cast<const float *>(a.v.re) + vv);
    const floatx2 vi = *reinterpret_cast<const floatx2 *>(static_cast<const float *>(a.v.im) + vv);
    x.kr[0] = kr.x, x.kr[1] = kr.y, x.kr[2] = kr.z, x.kr[3] = kr.w;
    x.ki[0] = ki.x, x.ki[1] = ki.y, x.ki[2] = ki.z, x.ki[3] = ki.w;
    x.qr[0] = qr.x * a.q_scale, x.qr[1] = qr.y * a.q_scale, x.qr[2] = qr.z * a.q_scale, x.qr[3] = qr.w * a.q_scale;
    x.qi[0] = qi.x * a.q_scale, x.qi[1] = qi.y * a.q_scale, x.qi[2] = qi.z * a.q_scale, x.qi[3] = qi.w * a.q_scale;
    x.vr[0] = vr.x, x.vr[1] = vr.y, x.vi[0] = vi.x, x.vi[1] = vi.y;
    const int64_t go = b * a.sg_b + h * a.sg_h + (int64_t)t * a.sg_t;
    x.g = a.gamma[go] + a.gamma_eps;
    x.b = a.beta[go];
    return x;
}

// One token: S <- g S + u (x) k*, u = b (v - g S k); returns y = S q~ for the
// lane's 2 rows (complete in every lane of the row group).
__device__ __forceinline__ void fwd_step(State &s, const Tok &x, float (&yr)[2], float (&yi)[2]) {
    float pkr[2], pki[2], pqr[2], pqi[2];
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
        float a0 = 0.f, a1 = 0.f, b0 = 0.f, b1 = 0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const float sr = s.r[rr][c], si = s.i[rr][c];
            a0 += sr * x.kr[c] - si * x.ki[c];
            a1 += sr * x.ki[c] + si * x.kr[c];
            b0 += sr * x.qr[c] - si * x.qi[c];
            b1 += sr * x.qi[c] + si * x.qr[c];
        }
        pkr[rr] = row16_sum(a0), pki[rr] = row16_sum(a1), pqr[rr] = row16_sum(b0), pqi[rr] = row16_sum(b1);
    }
    // k^H q~ over all columns
    float cr = 0.f, ci = 0.f;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        cr += x.kr[c] * x.qr[c] + x.ki[c] * x.qi[c];
        ci += x.kr[c] * x.qi[c] - x.ki[c] * x.qr[c];
    }
    cr = row16_sum(cr), ci = row16_sum(ci);
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
        const float ur = x.b * (x.vr[rr] - x.g * pkr[rr]), ui = x.b * (x.vi[rr] - x.g * pki[rr]);
        yr[rr] = x.g * pqr[rr] + ur * cr - ui * ci;
        yi[rr] = x.g * pqi[rr] + ur * ci + ui * cr;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            // u conj(k_c)
            const float or_ = ur * x.kr[c] + ui * x.ki[c], oi = ui * x.kr[c] - ur * x.ki[c];
            s.r[rr][c] = x.g * s.r[rr][c] + or_;
            s.i[rr][c] = x.g * s.i[rr][c] + oi;
        }
    }
}

__device__ __forceinline__ int chain_groups(int T) { return (T + GROUP - 1) / GROUP; }

// per-thread 16 floats of state at [chain][slot][tid], float4-coalesced
__device__ __forceinline__ void store_state(float *base, const State &s, int tid) {
    floatx4 *p = reinterpret_cast<floatx4 *>(base) + 4 * tid;
    p[0] = floatx4{s.r[0][0], s.r[0][1], s.r[0][2], s.r[0][3]};
    p[1] = floatx4{s.i[0][0], s.i[0][1], s.i[0][2], s.i[0][3]};
    p[2] = floatx4{s.r[1][0], s.r[1][1], s.r[1][2], s.r[1][3]};
    p[3] = floatx4{s.i[1][0], s.i[1][1], s.i[1][2], s.i[1][3]};
}
__device__ __forceinline__ void load_state(const float *base, State &s, int tid) {
    const floatx4 *p = reinterpret_cast<const floatx4 *>(base) + 4 * tid;
    const floatx4 a = p[0], b = p[1], c = p[2], d = p[3];
    s.r[0][0] = a.x, s.r[0][1] = a.y, s.r[0][2] = a.z, s.r[0][3] = a.w;
    s.i[0][0] = b.x, s.i[0][1] = b.y, s.i[0][2] = b.z, s.i[0][3] = b.w;
    s.r[1][0] = c.x, s.r[1][1] = c.y, s.r[1][2] = c.z, s.r[1][3] = c.w;
    s.i[1][0] = d.x, s.i[1][1] = d.y, s.i[1][2] = d.z, s.i[1][3] = d.w;
}
constexpr int STATE_FLOATS = 2 * D * D;   // one chain's state, thread-private layout

__global__ void __launch_bounds__(DTHREADS) delta_fwd_kernel(qpam_delta_args a) {
    const int chain = blockIdx.x, b = chain / a.H, h = chain - b * a.H, tid = threadIdx.x;
    const Lane L(tid);
    State s;
#pragma unroll
    for (int rr = 0; rr < 2; ++rr)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (a.s0_re) {
                const int64_t o = (int64_t)chain * D * D + (L.r0 + rr) * D + 4 * L.cg + c;
                s.r[rr][c] = a.s0_re[o], s.i[rr][c] = a.s0_im[o];
            } else {
                s.r[rr][c] = 0.f, s.i[rr][c] = 0.f;
            }
        }
    float *ckpt = static_cast<float *>(a.workspace) + (int64_t)chain * chain_groups(a.T) * STATE_FLOATS;
    Tok cur = load_tok(a, b, h, 0, L);
    for (int t = 0; t < a.T; ++t) {
        const Tok nxt = load_tok(a, b, h, min(t + 1, a.T - 1), L);
        if (t % GROUP == 0 && ckpt) store_state(ckpt + (int64_t)(t / GROUP) * STATE_FLOATS, s, tid);
        float yr[2], yi[2];
        fwd_step(s, cur, yr, yi);
        if (L.cg == 0) {
            const int64_t yo = b * a.y.s0 + h * a.y.s1 + (int64_t)t * a.y.s2 + L.r0;
            *reinterpret_cast<floatx2 *>(a.y.re + yo) = floatx2{yr[0], yr[1]};
            *reinterpret_cast<floatx2 *>(a.y.im + yo) = floatx2{yi[0], yi[1]};
        }
        cur = nxt;
    }
#pragma unroll
    for (int rr = 0; rr < 2; ++rr) {
        const int64_t o = (int64_t)chain * D * D + (L.r0 + rr) * D + 4 * L.cg;
        *reinterpret_cast<floatx4 *>(a.s_re + o) = floatx4{s.r[rr][0], s.r[rr][1], s.r[rr][2], s.r[rr][3]};
        *reinterpret_cast<floatx4 *>(a.s_im + o) = floatx4{s.i[rr][0], s.i[rr][1], s.i[rr][2], s.i[rr][3]};
    }
}

// sum over the 4 row groups of a wave (lanes cg, cg+16, cg+32, cg+48)
__device__ __forceinline__ float rows4_sum(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

__global__ void __launch_bounds__(DTHREADS) delta_bwd_kernel(qpam_delta_bwd_args g, qpam_delta_args a) {
    // per sub-group: [token][wave][column][dq re, dq im, dk re, dk im] and
    // [token][wave * 4 + row group][dgamma, dbeta]
    __shared__ floatx4 red[SUB][8][D];
    __shared__ floatx2 sred[SUB][32];
    const int chain = blockIdx.x, b = chain / a.H, h = chain - b * a.H, tid = threadIdx.x;
    const Lane L(tid);
    const int ng = chain_groups(a.T);
    const float *ckpt = static_cast<const float *>(a.workspace) + (int64_t)chain * ng * STATE_FLOATS;
    float *sub = static_cast<float *>(g.workspace) + (int64_t)chain * SUBS * STATE_FLOATS;

    State gs;   // adjoint of the state after the current token
#pragma unroll
    for (int rr = 0; rr < 2; ++rr)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            if (g.ds_re) {
                const int64_t o = (int64_t)chain * D * D + (L.r0 + rr) * D + 4 * L.cg + c;
                gs.r[rr][c] = g.ds_re[o], gs.i[rr][c] = g.ds_im[o];
            } else {
                gs.r[rr][c] = 0.f, gs.i[rr][c] = 0.f;
            }
        }

    for (int grp = ng - 1; grp >= 0; --grp) {
        const int t0 = grp * GROUP, tn = min(t0 + GROUP, a.T);
        // recompute the group, keeping the state before every SUB-th token
        State s;
        load_state(ckpt + (int64_t)grp * STATE_FLOATS, s, tid);
        for (int t = t0; t < tn; ++t) {
            if ((t - t0) % SUB == 0) store_state(sub + (int64_t)((t - t0) / SUB) * STATE_FLOATS, s, tid);
            const Tok x = load_tok(a, b, h, t, L);
            float yr[2], yi[2];
            fwd_step(s, x, yr, yi);
        }
        for (int sg = (tn - t0 - 1) / SUB; sg >= 0; --sg) {
            const int s0 = t0 + sg * SUB, n = min(SUB, tn - s0);
            // states before each token of the sub-group
            State prev[SUB];
            load_state(sub + (int64_t)sg * STATE_FLOATS, prev[0], tid);
#pragma unroll
            for (int j = 1; j < SUB; ++j) {
                prev[j] = prev[j - 1];
                if (j < n) {
                    const Tok x = load_tok(a, b, h, s0 + j - 1, L);
                    float yr[2], yi[2];
                    fwd_step(prev[j], x, yr, yi);
                }
            }
#pragma unroll
            for (int j = SUB - 1; j >= 0; --j) {
                if (j >= n) continue;
                const int t = s0 + j;
                const Tok x = load_tok(a, b, h, t, L);
                const int64_t dyo = b * g.dy.s0 + h * g.dy.s1 + (int64_t)t * g.dy.s2 + L.r0;
                const floatx2 dyr = *reinterpret_cast<const floatx2 *>(static_cast<const float *>(g.dy.re) + dyo);
                const floatx2 dyi = *reinterpret_cast<const floatx2 *>(static_cast<const float *>(g.dy.im) + dyo);
                const float gyr[2] = {dyr.x, dyr.y}, gyi[2] = {dyi.x, dyi.y};
                const State &sp = prev[j];
                // forward quantities of this token
                float ar[2][4], ai[2][4], pr[2], pi[2], ur[2], ui[2];
#pragma unroll
                for (int rr = 0; rr < 2; ++rr) {
                    float p0 = 0.f, p1 = 0.f;
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        ar[rr][c] = x.g * sp.r[rr][c], ai[rr][c] = x.g * sp.i[rr][c];
                        p0 += ar[rr][c] * x.kr[c] - ai[rr][c] * x.ki[c];
                        p1 += ar[rr][c] * x.ki[c] + ai[rr][c] * x.kr[c];
                    }
                    pr[rr] = row16_sum(p0), pi[rr] = row16_sum(p1);
                    ur[rr] = x.b * (x.vr[rr] - pr[rr]), ui[rr] = x.b * (x.vi[rr] - pi[rr]);
                }
                float gq[4][2] = {}, gk[4][2] = {};
                float ggam = 0.f, gbet = 0.f;
                float gur[2], gui[2];
#pragma unroll
                for (int rr = 0; rr < 2; ++rr) {
                    float u0 = 0.f, u1 = 0.f;
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        // s = a + u conj(k) (the state after the token)
                        const float sr = ar[rr][c] + ur[rr] * x.kr[c] + ui[rr] * x.ki[c];
                        const float si = ai[rr][c] + ui[rr] * x.kr[c] - ur[rr] * x.ki[c];
                        // y = s . q~:  g_s += conj(q~) g_y;  g_q~ += conj(s) g_y
                        gs.r[rr][c] += x.qr[c] * gyr[rr] + x.qi[c] * gyi[rr];
                        gs.i[rr][c] += x.qr[c] * gyi[rr] - x.qi[c] * gyr[rr];
                        gq[c][0] += sr * gyr[rr] + si * gyi[rr];
                        gq[c][1] += sr * gyi[rr] - si * gyr[rr];
                        // g_u = sum_c k_c g_s_c
                        u0 += x.kr[c] * gs.r[rr][c] - x.ki[c] * gs.i[rr][c];
                        u1 += x.kr[c] * gs.i[rr][c] + x.ki[c] * gs.r[rr][c];
                        // g_k_c += u conj(g_s_c)
                        gk[c][0] += ur[rr] * gs.r[rr][c] + ui[rr] * gs.i[rr][c];
                        gk[c][1] += ui[rr] * gs.r[rr][c] - ur[rr] * gs.i[rr][c];
                    }
                    gur[rr] = row16_sum(u0), gui[rr] = row16_sum(u1);
                }
#pragma unroll
                for (int rr = 0; rr < 2; ++rr) {
                    // u = beta (v - p)
                    gbet += (x.vr[rr] - pr[rr]) * gur[rr] + (x.vi[rr] - pi[rr]) * gui[rr];
                    const float gpr = -x.b * gur[rr], gpi = -x.b * gui[rr];
                    float gg = 0.f;
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        // p = sum_c a_c k_c:  g_a += conj(k) g_p;  g_k += conj(a) g_p
                        const float gar = gs.r[rr][c] + x.kr[c] * gpr + x.ki[c] * gpi;
                        const float gai = gs.i[rr][c] + x.kr[c] * gpi - x.ki[c] * gpr;
                        gk[c][0] += ar[rr][c] * gpr + ai[rr][c] * gpi;
                        gk[c][1] += ar[rr][c] * gpi - ai[rr][c] * gpr;
                        // a = g~ s_prev:  g_g~ += Re(conj(s_prev) g_a);  g_s_prev = g~ g_a
                        gg += sp.r[rr][c] * gar + sp.i[rr][c] * gai;
                        gs.r[rr][c] = x.g * gar;
                        gs.i[rr][c] = x.g * gai;
                    }
                    ggam += gg;
                }
                if (L.cg == 0) {
                    const int64_t vo = b * g.dv.s0 + h * g.dv.s1 + (int64_t)t * g.dv.s2 + L.r0;
                    *reinterpret_cast<floatx2 *>(g.dv.re + vo) = floatx2{x.b * gur[0], x.b * gur[1]};
                    *reinterpret_cast<floatx2 *>(g.dv.im + vo) = floatx2{x.b * gui[0], x.b * gui[1]};
                }
                // column sums over the wave's 8 rows, then one slot per wave
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    gq[c][0] = rows4_sum(gq[c][0]), gq[c][1] = rows4_sum(gq[c][1]);
                    gk[c][0] = rows4_sum(gk[c][0]), gk[c][1] = rows4_sum(gk[c][1]);
                }
                if (L.rg == 0) {
#pragma unroll
                    for (int c = 0; c < 4; ++c)
                        red[j][L.w][4 * L.cg + c] = floatx4{gq[c][0], gq[c][1], gk[c][0], gk[c][1]};
                }
                // ggam holds this lane's columns; gbet is already the row group's value
                ggam = row16_sum(ggam);
                if (L.cg == 0) sred[j][4 * L.w + L.rg] = floatx2{ggam, gbet};
            }
            __syncthreads();
            // reduce the 8 wave slots of each (token, column) in a fixed order
            for (int i = tid; i < n * D; i += DTHREADS) {
                const int j = i / D, c = i - j * D, t = s0 + j;
                floatx4 acc = red[j][0][c];
#pragma unroll
                for (int w = 1; w < 8; ++w) acc += red[j][w][c];
                const int64_t qo = b * g.dq.s0 + h * g.dq.s1 + (int64_t)t * g.dq.s2 + c;
                const int64_t ko = b * g.dk.s0 + h * g.dk.s1 + (int64_t)t * g.dk.s2 + c;
                g.dq.re[qo] = acc.x * a.q_scale, g.dq.im[qo] = acc.y * a.q_scale;
                g.dk.re[ko] = acc.z, g.dk.im[ko] = acc.w;
            }
            if (tid < n) {
                floatx2 acc = sred[tid][0];
                for (int k = 1; k < 32; ++k) acc += sred[tid][k];
                const int64_t go = b * a.sg_b + h * a.sg_h + (int64_t)(s0 + tid) * a.sg_t;
                g.dgamma[go] = acc.x;
                g.dbeta[go] = acc.y;
            }
            __syncthreads();
        }
    }
    if (g.ds0_re) {
#pragma unroll
        for (int rr = 0; rr < 2; ++rr) {
            const int64_t o = (int64_t)chain * D * D + (L.r0 + rr) * D + 4 * L.cg;
            *reinterpret_cast<floatx4 *>(g.ds0_re + o) = floatx4{gs.r[rr][0], gs.r[rr][1], gs.r[rr][2], gs.r[rr][3]};
            *reinterpret_cast<floatx4 *>(g.ds0_im + o) = floatx4{gs.i[rr][0], gs.i[rr][1], gs.i[rr][2], gs.i[rr][3]};
        }
    }
}

bool aligned(const void *p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

bool cview_ok(const qpam_cview &v) {
    return v.re && v.im && aligned(v.re, 16) && aligned(v.im, 16) && v.s0 % 4 == 0 && v.s1 % 4 == 0 && v.s2 % 4 == 0;
}
bool mview_ok(const qpam_mview &v) {
    return v.re && v.im && aligned(v.re, 16) && aligned(v.im, 16) && v.s0 % 4 == 0 && v.s1 % 4 == 0 && v.s2 % 4 == 0;
}

size_t fwd_ws(const qpam_delta_args &a) {
    return (size_t)a.B * a.H * ((a.T + GROUP - 1) / GROUP) * STATE_FLOATS * sizeof(float);
}
size_t bwd_ws(const qpam_delta_args &a) { return (size_t)a.B * a.H * SUBS * STATE_FLOATS * sizeof(float); }

int validate(const qpam_delta_args *a) {
    QPAM_REQUIRE(a != nullptr, "qpam_delta: null arguments");
    QPAM_REQUIRE(a->B >= 0 && a->H >= 1 && a->T >= 0, "qpam_delta: invalid sizes B=%d H=%d T=%d", a->B, a->H, a->T);
    QPAM_REQUIRE(a->d == D, "qpam_delta: head_dim %d unsupported (64 only)", a->d);
    QPAM_REQUIRE(cview_ok(a->q) && cview_ok(a->k) && cview_ok(a->v),
                 "qpam_delta: q, k, v must be 16-byte aligned fp32 planes with strides multiple of 4");
    QPAM_REQUIRE(a->gamma && a->beta, "qpam_delta: gamma and beta required");
    QPAM_REQUIRE((a->s0_re == nullptr) == (a->s0_im == nullptr), "qpam_delta: s0 needs both planes");
    QPAM_REQUIRE(a->s0_re == nullptr || (aligned(a->s0_re, 16) && aligned(a->s0_im, 16)),
                 "qpam_delta: s0 planes must be 16-byte aligned");
    return QPAM_OK;
}

}  // namespace
}  // namespace qpam

using namespace qpam;

extern "C" size_t qpam_delta_workspace_size(const qpam_delta_args *a) { return a ? fwd_ws(*a) : 0; }

extern "C" int qpam_delta_fwd(const qpam_delta_args *a, void *stream) {
    int st = validate(a);
    if (st) return st;
    QPAM_REQUIRE(mview_ok(a->y) && a->s_re && a->s_im && aligned(a->s_re, 16) && aligned(a->s_im, 16),
                 "qpam_delta_fwd: y (16-byte aligned planes) and the final state are required");
    QPAM_REQUIRE(a->workspace == nullptr || (aligned(a->workspace, 16) && a->workspace_bytes >= fwd_ws(*a)),
                 "qpam_delta_fwd: workspace of %zu bytes needed (or NULL without a backward)", fwd_ws(*a));
    if (a->B == 0) return QPAM_OK;
    QPAM_REQUIRE(a->T >= 1, "qpam_delta_fwd: T must be >= 1");
    hipLaunchKernelGGL(delta_fwd_kernel, dim3(a->B * a->H), dim3(DTHREADS), 0, static_cast<hipStream_t>(stream), *a);
    return launch_status("delta_fwd_kernel");
}

extern "C" size_t qpam_delta_bwd_workspace_size(const qpam_delta_bwd_args *g) {
    return (g && g->fwd) ? bwd_ws(*g->fwd) : 0;
}

extern "C" int qpam_delta_bwd(const qpam_delta_bwd_args *g, void *stream) {
    QPAM_REQUIRE(g != nullptr && g->fwd != nullptr, "qpam_delta_bwd: null arguments");
    const qpam_delta_args &a = *g->fwd;
    int st = validate(&a);
    if (st) return st;
    QPAM_REQUIRE(a.workspace && aligned(a.workspace, 16) && a.workspace_bytes >= fwd_ws(a),
                 "qpam_delta_bwd: the forward's workspace (checkpoints) is required");
    QPAM_REQUIRE(g->workspace && aligned(g->workspace, 16) && g->workspace_bytes >= bwd_ws(a),
                 "qpam_delta_bwd: workspace of %zu bytes needed", bwd_ws(a));
    QPAM_REQUIRE(cview_ok(g->dy) && mview_ok(g->dq) && mview_ok(g->dk) && mview_ok(g->dv),
                 "qpam_delta_bwd: dy, dq, dk, dv must be 16-byte aligned fp32 planes with strides multiple of 4");
    QPAM_REQUIRE(g->dgamma && g->dbeta, "qpam_delta_bwd: dgamma and dbeta required");
    QPAM_REQUIRE((g->ds_re == nullptr) == (g->ds_im == nullptr) && (g->ds0_re == nullptr) == (g->ds0_im == nullptr),
                 "qpam_delta_bwd: ds / ds0 need both planes");
    if (a.B == 0 || a.T == 0) return QPAM_OK;
    hipLaunchKernelGGL(delta_bwd_kernel, dim3(a.B * a.H), dim3(DTHREADS), 0, static_cast<hipStream_t>(stream), *g, a);
    return launch_status("delta_bwd_kernel");
}
