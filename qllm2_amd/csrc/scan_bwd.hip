// Chunked dual-form PAM scan, backward (fp32 MFMA, d = 64).
//
// The reference obtains these gradients with torch autograd through
// _forward_chunked_head / _fused_chunk_step (v11/model.py:378-417, 657-737)
// and the closed-form decay-matrix backward (v11/triton_kernels.py:447-480).
// Per chunk, with G_Y = dL/dY, G'_m = dL/dS_m after the chunk, S_m the state
// entering it, A = W . D~, rho_m = r_m cum_m:
//   dA   = G_Y V^H                    gW = dA . conj(D~)   gD~ = dA . conj(W)
//   dQ~ += gW K + sum_m conj(rho_m) (G_Y conj(S_m))
//   dK  += gW^H Q~ + sum_m dl_m . (V conj(G'_m))
//   dV  += A^H G_Y + sum_m dl_m . (K G'_m^T)
//   dS_m = total_m G'_m + sum_t conj(rho_m[t]) G_Y[t] (x) conj(Q~[t])
// and the log-decay gradient collects D (rows +, columns -), cum, total and
// decay_last contributions before a reverse cumsum and 1/(gamma + 1e-6).
//
// Launches (mirroring the forward):
//   1. grad_chunk_state (chunk-parallel): the per-chunk dS increment;
//   2. grad_state_scan  (reverse, elementwise): dS after every chunk, dS0;
//   3. query_side (chunk-parallel, wave = query tile): dQ, d rot, the decay
//      gradient of D and cum -> partial dL/dL_t in the workspace;
//   4. key_side (chunk-parallel, wave = key tile): dK, dV, the decay_last and
//      total gradients, and the final d gamma of the chunk.
// bf16 inputs with 64-step chunks: grad_pass_bf16 (the sequential dS chain,
// writing a bf16 snapshot of dS after every chunk), then chunk_grad_bf16 (the
// query and key sides of a chunk in one block).
#include <type_traits>

#include "scan_common.h"

namespace qpam {
namespace scan {

int validate_scan(const qpam_scan_args *a, const char *who, bool fwd_outputs);
size_t fwd_workspace_bytes(const qpam_scan_args &a);
bool uses_snapshots(const qpam_scan_args &a);
size_t fwd_snapshot_offset(const qpam_scan_args &a);
int64_t fwd_totals_offset(const qpam_scan_args &a);

namespace {

struct BwdParams {
    qpam_scan_args a;
    qpam_cview dy;           // fp32
    const float *ds_re, *ds_im;
    qpam_mview dq, dk, dv;   // element type = input dtype
    float *dgamma;
    float *drot_re, *drot_im;
    float *ds0_re, *ds0_im;
    int n_chunks;
    const float *states;     // forward: state entering each chunk
    const float *totals;     // forward: chunk decay totals
    float *gstates;          // dS increment per chunk -> dS after each chunk
    float *gl;               // [M][B][H][n*C] partial dL/dL_t (query side)
    // bf16 path: entering states (forward snapshots) and dS after each chunk, bf16
    const unsigned short *snap;
    unsigned short *gsnap;
    const float *wgr, *wgi;  // bf16 path: the forward's per-step weights conj(rho_m[t]) q_scale
    int dy_bf16;             // dy planes are bf16 (bf16 path only)
};

__device__ __forceinline__ int64_t chain_idx(const BwdParams &p, int m, int b, int h) {
    return ((int64_t)m * p.a.B + b) * p.a.H + h;
}
__device__ __forceinline__ const float *fstate(const BwdParams &p, int m, int b, int h, int c) {
    return p.states + (chain_idx(p, m, b, h) * p.n_chunks + c) * (2 * D * D);
}
__device__ __forceinline__ float *gstate(const BwdParams &p, int m, int b, int h, int c) {
    return p.gstates + (chain_idx(p, m, b, h) * p.n_chunks + c) * (2 * D * D);
}
__device__ __forceinline__ const unsigned short *fsnap(const BwdParams &p, int m, int b, int h, int c) {
    return p.snap + (chain_idx(p, m, b, h) * p.n_chunks + c) * (2 * D * D);
}
__device__ __forceinline__ unsigned short *gsnap(const BwdParams &p, int m, int b, int h, int c) {
    return p.gsnap + (chain_idx(p, m, b, h) * p.n_chunks + c) * (2 * D * D);
}
__device__ __forceinline__ float ftotal(const BwdParams &p, int m, int b, int h, int c) {
    return p.totals[chain_idx(p, m, b, h) * p.n_chunks + c];
}

template <typename T>
__device__ __forceinline__ void store_elem(float *base, int64_t idx, float v);
template <>
__device__ __forceinline__ void store_elem<float>(float *base, int64_t idx, float v) {
    base[idx] = v;
}
template <>
__device__ __forceinline__ void store_elem<unsigned short>(float *base, int64_t idx, float v) {
    reinterpret_cast<unsigned short *>(base)[idx] = f32_to_bf16(v);
}

// contiguous 64x64 fp32 planes (re, im) -> LDS (pitch P); both loads in flight together
__device__ __forceinline__ void load_state_planes(float *lds_re, float *lds_im, const float *src) {
    F32Tile<D> tr, ti;
    tile_load<D>(tr, src, D, D);
    tile_load<D>(ti, src + D * D, D, D);
    tile_store<D>(lds_re, tr, 1.f);
    tile_store<D>(lds_im, ti, 1.f);
}

// Stage the fp32 upstream-gradient tiles (NG of them) and the input tiles (NI)
// of one chunk; with fp32 inputs all loads form one batch.
template <typename Tin, int C, int NG, int NI>
__device__ __forceinline__ void stage_grad_and_inputs(float *const (&gdst)[NG], const float *const (&gsrc)[NG],
                                                      int64_t gst, float *const (&idst)[NI],
                                                      const Tin *const (&isrc)[NI], const int64_t (&ist)[NI],
                                                      const float (&isc)[NI], int valid) {
    if constexpr (std::is_same<Tin, float>::value) {
        float *dst[NG + NI];
        const float *src[NG + NI];
        int64_t st[NG + NI];
        float sc[NG + NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) dst[i] = idst[i], src[i] = isrc[i], st[i] = ist[i], sc[i] = isc[i];
#pragma unroll
        for (int i = 0; i < NG; ++i) dst[NI + i] = gdst[i], src[NI + i] = gsrc[i], st[NI + i] = gst, sc[NI + i] = 1.f;
        F32Tile<C> t[NG + NI];
#pragma unroll
        for (int i = 0; i < NG + NI; ++i) tile_load<C>(t[i], src[i], st[i], valid);
#pragma unroll
        for (int i = 0; i < NG + NI; ++i) tile_store<C>(dst[i], t[i], sc[i]);
    } else {
        float gsc[NG];
        int64_t gsts[NG];
#pragma unroll
        for (int i = 0; i < NG; ++i) gsc[i] = 1.f, gsts[i] = gst;
        stage_tiles<float, C, NG>(gdst, gsrc, gsts, gsc, valid);
        stage_tiles<Tin, C, NI>(idst, isrc, ist, isc, valid);
    }
}

// Per-chunk prologue shared by the chunk-parallel backward kernels: log-decay
// prefix sums and rotations of every state (wave 0).
__device__ __forceinline__ void chunk_decay_prologue(const qpam_scan_args &a, int b, int h, int c0, int valid,
                                                     float *sL, float *sRr, float *sRi) {
    const int lane = threadIdx.x & 63;
    for (int m = 0; m < a.M; ++m) {
        const float *gp = a.gamma + m * a.sg_m + b * a.sg_b + h * a.sg_h + (int64_t)c0 * a.sg_t;
        sL[m * 64 + lane] = chunk_log_prefix(gp, a.sg_t, valid, lane);
        float rr = 1.f, ri = 0.f;
        if (a.rot_re && lane < valid) {
            const int64_t ro = m * a.sr_m + b * a.sr_b + h * a.sr_h + (int64_t)(c0 + lane) * a.sr_t;
            rr = a.rot_re[ro];
            ri = a.rot_im[ro];
        }
        sRr[m * 64 + lane] = rr;
        sRi[m * 64 + lane] = ri;
    }
}

// chunk_decay_prologue plus the factorised-decay tables of the bf16 kernels:
// sF[m][t] = exp(-L_m[t]) and, when sPr is given, sPr/sPi[m][t] = r_m[t] exp(L_m[t]);
// *sFast = 1 when every state of the chunk passes the factorisation test.
template <int M>
__device__ __forceinline__ void chunk_decay_prologue_f(const qpam_scan_args &a, int b, int h, int c0, int valid,
                                                       float *sL, float *sRr, float *sRi, float *sF, float *sPr,
                                                       float *sPi, int *sFast) {
    const int lane = threadIdx.x & 63;
    bool fast = true;
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float *gp = a.gamma + m * a.sg_m + b * a.sg_b + h * a.sg_h + (int64_t)c0 * a.sg_t;
        bool ok;
        const float L = chunk_log_prefix_ok(gp, a.sg_t, valid, lane, ok);
        fast = fast && ok;
        float rr = 1.f, ri = 0.f;
        if (a.rot_re && lane < valid) {
            const int64_t ro = m * a.sr_m + b * a.sr_b + h * a.sr_h + (int64_t)(c0 + lane) * a.sr_t;
            rr = a.rot_re[ro];
            ri = a.rot_im[ro];
        }
        sL[m * 64 + lane] = L;
        sRr[m * 64 + lane] = rr;
        sRi[m * 64 + lane] = ri;
        sF[m * 64 + lane] = __expf(-L);  // unused (possibly inf) when the test fails
        if (sPr) {
            const float e = __expf(L);
            sPr[m * 64 + lane] = rr * e;
            sPi[m * 64 + lane] = ri * e;
        }
    }
    if (lane == 0) *sFast = fast ? 1 : 0;
}

// ---------------------------------------------------------------- kernel 1 --
// dS increment of chunk c: dG_m[i][j] = sum_t conj(rho_m[t]) G_Y[t][i] conj(Q~[t][j])
template <typename Tin, int C>
__global__ void __launch_bounds__(THREADS) grad_chunk_state_kernel(BwdParams p) {
    extern __shared__ float smem[];
    float *sGr = smem, *sGi = sGr + C * P, *sQr = sGi + C * P, *sQi = sQr + C * P;
    float *sL = sQi + C * P, *sRr = sL + MAX_M * 64, *sRi = sRr + MAX_M * 64;

    const qpam_scan_args &a = p.a;
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int c0 = c * C, valid = min(C, a.T - c0);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;

    if (c == 0 && a.s0_re == nullptr) {  // no initial state: chunk 0 carries nothing
        for (int m = 0; m < a.M; ++m) {
            float *dst = gstate(p, m, b, h, 0);
            for (int e = tid; e < 2 * D * D / 4; e += THREADS)
                reinterpret_cast<float4 *>(dst)[e] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
        return;
    }
    const int64_t go = b * p.dy.s0 + h * p.dy.s1 + (int64_t)c0 * p.dy.s2;
    const int64_t qo = b * a.q.s0 + h * a.q.s1 + (int64_t)c0 * a.q.s2;
    {
        float *const gd[2] = {sGr, sGi};
        const float *const gs[2] = {(const float *)p.dy.re + go, (const float *)p.dy.im + go};
        float *const id[2] = {sQr, sQi};
        const Tin *const is[2] = {(const Tin *)a.q.re + qo, (const Tin *)a.q.im + qo};
        const int64_t ist[2] = {a.q.s2, a.q.s2};
        const float isc[2] = {a.q_scale, a.q_scale};
        stage_grad_and_inputs<Tin, C, 2, 2>(gd, gs, p.dy.s2, id, is, ist, isc, valid);
    }
    if (w == 0) chunk_decay_prologue(a, b, h, c0, valid, sL, sRr, sRi);
    __syncthreads();

    for (int m = 0; m < a.M; ++m) {
        floatx4 accR[4], accI[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) accR[jt] = accI[jt] = zero4();
#pragma unroll 4
        for (int ks = 0; ks < C / 4; ++ks) {
            const int t = 4 * ks + g;
            const float cum = (t < valid) ? __expf(sL[m * 64 + t]) : 0.f;
            const float wr = sRr[m * 64 + t] * cum, wi = -sRi[m * 64 + t] * cum;  // conj(rho)
            const float gr = sGr[t * P + 16 * w + l16], gi = sGi[t * P + 16 * w + l16];
            const float vr = wr * gr - wi * gi, vi = wr * gi + wi * gr;
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                const float qr = sQr[t * P + 16 * jt + l16];
                const float qi = sQi[t * P + 16 * jt + l16];
                accR[jt] = mfma4(vr, qr, accR[jt]);
                accR[jt] = mfma4(vi, qi, accR[jt]);
                accI[jt] = mfma4(vi, qr, accI[jt]);
                accI[jt] = mfma4(vr, -qi, accI[jt]);
            }
        }
        float *dst = gstate(p, m, b, h, c);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * w + 4 * g + r, j = 16 * jt + l16;
                dst[i * D + j] = accR[jt][r];
                dst[D * D + i * D + j] = accI[jt][r];
            }
    }
}

// ---------------------------------------------------------------- kernel 2 --
// Reverse scan: G = dS_final; for c = n-1..0: slot[c] <- G (dS after chunk c),
// G = total_c G + increment_c.  At the end G = dS0.  Thread layout and the
// two-chunk prefetch as in the forward state scan.
__global__ void __launch_bounds__(THREADS) grad_state_scan_kernel(BwdParams p) {
    const qpam_scan_args &a = p.a;
    const int chain = blockIdx.x / SCAN_BLOCKS;
    const int bh = chain % (a.B * a.H), m = chain / (a.B * a.H);
    const int b = bh / a.H, h = bh % a.H;
    const int64_t cs = 2 * D * D;  // floats per chunk state
    float *base = gstate(p, m, b, h, 0);
    unsigned short *sbase = p.gsnap ? gsnap(p, m, b, h, 0) : nullptr;
    const int n = p.n_chunks;

    int off[SCAN_EPT];
    float4 G[SCAN_EPT], b0[SCAN_EPT], b1[SCAN_EPT];
#pragma unroll
    for (int e = 0; e < SCAN_EPT; ++e) {
        off[e] = 4 * ((blockIdx.x % SCAN_BLOCKS) * THREADS * SCAN_EPT + e * THREADS + threadIdx.x);
        const int plane = off[e] >= D * D;
        G[e] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (p.ds_re)
            G[e] = *reinterpret_cast<const float4 *>((plane ? p.ds_im : p.ds_re) + (int64_t)chain * D * D +
                                                     off[e] - plane * D * D);
        b0[e] = *reinterpret_cast<const float4 *>(base + (n - 1) * cs + off[e]);
        if (n > 1) b1[e] = *reinterpret_cast<const float4 *>(base + (n - 2) * cs + off[e]);
    }
    for (int c = n - 1; c >= 0; --c) {
        const float t = ftotal(p, m, b, h, c);
#pragma unroll
        for (int e = 0; e < SCAN_EPT; ++e) {
            const float4 inc = b0[e];
            b0[e] = b1[e];
            if (c >= 2) b1[e] = *reinterpret_cast<const float4 *>(base + (c - 2) * cs + off[e]);
            if (sbase) *reinterpret_cast<ushortx4 *>(sbase + c * cs + off[e]) = to_bf16x4(G[e]);
            else *reinterpret_cast<float4 *>(base + c * cs + off[e]) = G[e];
            G[e].x = t * G[e].x + inc.x;
            G[e].y = t * G[e].y + inc.y;
            G[e].z = t * G[e].z + inc.z;
            G[e].w = t * G[e].w + inc.w;
        }
    }
    if (p.ds0_re) {
#pragma unroll
        for (int e = 0; e < SCAN_EPT; ++e) {
            const int plane = off[e] >= D * D;
            *reinterpret_cast<float4 *>((plane ? p.ds0_im : p.ds0_re) + (int64_t)chain * D * D + off[e] -
                                        plane * D * D) = G[e];
        }
    }
}

// ---------------------------------------------------------------- kernel 3 --
template <typename Tin, int C>
__global__ void __launch_bounds__(THREADS) query_side_kernel(BwdParams p) {
    extern __shared__ float smem[];
    float *sQr = smem, *sQi = sQr + C * P;
    float *sKr = sQi + C * P, *sKi = sKr + C * P;
    float *sVr = sKi + C * P, *sVi = sVr + D * P;  // V tile, later the state S_m
    float *sGr = sVi + D * P, *sGi = sGr + C * P;
    float *sL = sGi + C * P, *sRr = sL + MAX_M * 64, *sRi = sRr + MAX_M * 64;
    float *sGL = sRi + MAX_M * 64, *sDRr = sGL + MAX_M * 64, *sDRi = sDRr + MAX_M * 64;
    // per-wave partial log-decay gradients of the score phase [wave][m][64]: every
    // wave adds only into its own slice, the slices are summed in wave order after
    // it (a fixed summation order: the result does not depend on wave timing)
    float *sGLw = sDRi + MAX_M * 64;

    const qpam_scan_args &a = p.a;
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int c0 = c * C, valid = min(C, a.T - c0);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const bool carry = (c > 0) || (a.s0_re != nullptr);
    const int M = a.M;

    {
        const int64_t qo = b * a.q.s0 + h * a.q.s1 + (int64_t)c0 * a.q.s2;
        const int64_t ko = b * a.k.s0 + h * a.k.s1 + (int64_t)c0 * a.k.s2;
        const int64_t vo = b * a.v.s0 + h * a.v.s1 + (int64_t)c0 * a.v.s2;
        const int64_t go = b * p.dy.s0 + h * p.dy.s1 + (int64_t)c0 * p.dy.s2;
        float *const gd[2] = {sGr, sGi};
        const float *const gs[2] = {(const float *)p.dy.re + go, (const float *)p.dy.im + go};
        float *const id[6] = {sQr, sQi, sKr, sKi, sVr, sVi};
        const Tin *const is[6] = {(const Tin *)a.q.re + qo, (const Tin *)a.q.im + qo, (const Tin *)a.k.re + ko,
                                  (const Tin *)a.k.im + ko, (const Tin *)a.v.re + vo, (const Tin *)a.v.im + vo};
        const int64_t ist[6] = {a.q.s2, a.q.s2, a.k.s2, a.k.s2, a.v.s2, a.v.s2};
        const float isc[6] = {a.q_scale, a.q_scale, 1.f, 1.f, 1.f, 1.f};
        stage_grad_and_inputs<Tin, C, 2, 6>(gd, gs, p.dy.s2, id, is, ist, isc, valid);
    }
    if (w == 0) chunk_decay_prologue(a, b, h, c0, valid, sL, sRr, sRi);
    for (int e = tid; e < 7 * MAX_M * 64; e += THREADS) sGL[e] = 0.f;  // sGL, sDRr, sDRi, sGLw
    __syncthreads();

    const int tt = causal_tile(w);
    const bool active = tt < C / 16;
    float *gl_w = sGLw + w * MAX_M * 64;  // this wave's partials
    floatx4 gqR[4], gqI[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) gqR[jt] = gqI[jt] = zero4();

    if (active) {
        const int t = 16 * tt + l16;  // this lane's query row in the transposed tiles
        floatx4 wr[4], wi[4], dr[4], di[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) wr[st] = wi[st] = dr[st] = di[st] = zero4();
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const float4 bq_r = *reinterpret_cast<const float4 *>(sQr + t * P + 16 * q4 + 4 * g);
            const float4 bq_i = *reinterpret_cast<const float4 *>(sQi + t * P + 16 * q4 + 4 * g);
            const float4 bg_r = *reinterpret_cast<const float4 *>(sGr + t * P + 16 * q4 + 4 * g);
            const float4 bg_i = *reinterpret_cast<const float4 *>(sGi + t * P + 16 * q4 + 4 * g);
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                if (st > tt || 16 * st >= C) continue;
                const int s = 16 * st + l16;
                const float4 ak_r = *reinterpret_cast<const float4 *>(sKr + s * P + 16 * q4 + 4 * g);
                const float4 ak_i = *reinterpret_cast<const float4 *>(sKi + s * P + 16 * q4 + 4 * g);
                const float4 av_r = *reinterpret_cast<const float4 *>(sVr + s * P + 16 * q4 + 4 * g);
                const float4 av_i = *reinterpret_cast<const float4 *>(sVi + s * P + 16 * q4 + 4 * g);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    // W^T[s][t] = sum_j q~[t,j] conj(k[s,j])
                    wr[st] = mfma4(ak_r[kk], bq_r[kk], wr[st]);
                    wr[st] = mfma4(ak_i[kk], bq_i[kk], wr[st]);
                    wi[st] = mfma4(ak_r[kk], bq_i[kk], wi[st]);
                    wi[st] = mfma4(-ak_i[kk], bq_r[kk], wi[st]);
                    // dA^T[s][t] = sum_i G[t,i] conj(v[s,i])
                    dr[st] = mfma4(av_r[kk], bg_r[kk], dr[st]);
                    dr[st] = mfma4(av_i[kk], bg_i[kk], dr[st]);
                    di[st] = mfma4(av_r[kk], bg_i[kk], di[st]);
                    di[st] = mfma4(-av_i[kk], bg_r[kk], di[st]);
                }
            }
        }
        // elementwise decay algebra; lane holds s = 16st + 4g + r, t = 16tt + l16
        float rowp[MAX_M], grr[MAX_M], gri[MAX_M];
#pragma unroll
        for (int m = 0; m < MAX_M; ++m) rowp[m] = grr[m] = gri[m] = 0.f;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            if (st > tt || 16 * st >= C) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int s = 16 * st + 4 * g + r;
                float gwr = 0.f, gwi = 0.f;
                float colp[MAX_M];
#pragma unroll
                for (int m = 0; m < MAX_M; ++m) colp[m] = 0.f;
                if (s <= t) {
                    float Dm[MAX_M], nc[MAX_M];
                    float dtr = 0.f, dti = 0.f;
#pragma unroll
                    for (int m = 0; m < MAX_M; ++m) {
                        Dm[m] = nc[m] = 0.f;
                        if (m < M) {
                            const float x = sL[m * 64 + t] - sL[m * 64 + s];
                            Dm[m] = __expf(fminf(x, 0.f));
                            nc[m] = (x <= 0.f && s != t) ? 1.f : 0.f;  // diagonal: +g and -g cancel
                            dtr += sRr[m * 64 + t] * Dm[m];
                            dti += sRi[m * 64 + t] * Dm[m];
                        }
                    }
                    const float Ar = dr[st][r], Ai = di[st][r];   // dA
                    const float Wr = wr[st][r], Wi = wi[st][r];   // W
                    gwr = Ar * dtr + Ai * dti;                    // dA conj(D~)
                    gwi = Ai * dtr - Ar * dti;
                    const float gdr = Ar * Wr + Ai * Wi;          // dA conj(W)
                    const float gdi = Ai * Wr - Ar * Wi;
#pragma unroll
                    for (int m = 0; m < MAX_M; ++m) {
                        if (m < M) {
                            const float gdm = gdr * sRr[m * 64 + t] + gdi * sRi[m * 64 + t];
                            const float gp = gdm * Dm[m] * nc[m];
                            rowp[m] += gp;
                            colp[m] = -gp;
                            grr[m] += gdr * Dm[m];
                            gri[m] += gdi * Dm[m];
                        }
                    }
                }
                // column sums over the 16 query rows of this tile (lanes sharing g)
#pragma unroll
                for (int m = 0; m < MAX_M; ++m) {
                    if (m < M) {
                        float x = colp[m];
#pragma unroll
                        for (int off = 1; off < 16; off <<= 1) x += __shfl_xor(x, off);
                        if (l16 == 0) gl_w[m * 64 + s] += x;
                    }
                }
                wr[st][r] = gwr;
                wi[st][r] = gwi;
            }
        }
#pragma unroll
        for (int m = 0; m < MAX_M; ++m) {
            if (m < M) {
                float x = rowp[m], yr = grr[m], yi = gri[m];
                x += __shfl_xor(x, 16);
                x += __shfl_xor(x, 32);
                yr += __shfl_xor(yr, 16);
                yr += __shfl_xor(yr, 32);
                yi += __shfl_xor(yi, 16);
                yi += __shfl_xor(yi, 32);
                if (g == 0) {  // rows t are this wave's own
                    gl_w[m * 64 + t] += x;
                    sDRr[m * 64 + t] += yr;
                    sDRi[m * 64 + t] += yi;
                }
            }
        }
        // intra dQ~[t][j] += sum_s gW[t,s] K[s,j]
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            if (st > tt || 16 * st >= C) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int s = 16 * st + 4 * g + r;
                const float ar = wr[st][r], ai = wi[st][r];
#pragma unroll
                for (int jt = 0; jt < 4; ++jt) {
                    const float kr = sKr[s * P + 16 * jt + l16];
                    const float ki = sKi[s * P + 16 * jt + l16];
                    gqR[jt] = mfma4(ar, kr, gqR[jt]);
                    gqR[jt] = mfma4(-ai, ki, gqR[jt]);
                    gqI[jt] = mfma4(ar, ki, gqI[jt]);
                    gqI[jt] = mfma4(ai, kr, gqI[jt]);
                }
            }
        }
    }

    __syncthreads();
    for (int e = tid; e < M * 64; e += THREADS)  // the waves' partials, in wave order
        sGL[e] += ((sGLw[e] + sGLw[MAX_M * 64 + e]) + sGLw[2 * MAX_M * 64 + e]) + sGLw[3 * MAX_M * 64 + e];
    // carried read: X_m = G_Y conj(S_m); dQ~ += conj(rho_m) X_m; g_rho_m[t] = sum_j conj(q~[t,j]) X_m[t,j]
    // (rows tr are this wave's own: plain updates)
    if (carry) {
        for (int m = 0; m < M; ++m) {
            __syncthreads();
            const float *src = fstate(p, m, b, h, c);
            load_state_planes(sVr, sVi, src);
            __syncthreads();
            if (!active) continue;
            const int t = 16 * tt + l16;
            floatx4 xr[4], xi[4];
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) xr[jt] = xi[jt] = zero4();
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 ag_r = *reinterpret_cast<const float4 *>(sGr + t * P + 16 * q4 + 4 * g);
                const float4 ag_i = *reinterpret_cast<const float4 *>(sGi + t * P + 16 * q4 + 4 * g);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const int i = 16 * q4 + 4 * g + kk;
#pragma unroll
                    for (int jt = 0; jt < 4; ++jt) {
                        const float sr = sVr[i * P + 16 * jt + l16], si = sVi[i * P + 16 * jt + l16];
                        xr[jt] = mfma4(ag_r[kk], sr, xr[jt]);
                        xr[jt] = mfma4(ag_i[kk], si, xr[jt]);
                        xi[jt] = mfma4(ag_i[kk], sr, xi[jt]);
                        xi[jt] = mfma4(-ag_r[kk], si, xi[jt]);
                    }
                }
            }
            // lane holds X[t' = 16tt + 4g + r][j = 16jt + l16]
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tr = 16 * tt + 4 * g + r;
                const float cum = __expf(sL[m * 64 + tr]);
                const float rr = sRr[m * 64 + tr], ri = sRi[m * 64 + tr];
                const float rhr = rr * cum, rhi = ri * cum;
                float pr = 0.f, pi = 0.f;
#pragma unroll
                for (int jt = 0; jt < 4; ++jt) {
                    const float x_r = xr[jt][r], x_i = xi[jt][r];
                    gqR[jt][r] += rhr * x_r + rhi * x_i;  // conj(rho) X
                    gqI[jt][r] += rhr * x_i - rhi * x_r;
                    const float qr = sQr[tr * P + 16 * jt + l16], qi = sQi[tr * P + 16 * jt + l16];
                    pr += qr * x_r + qi * x_i;  // conj(q~) X
                    pi += qr * x_i - qi * x_r;
                }
#pragma unroll
                for (int off = 1; off < 16; off <<= 1) {
                    pr += __shfl_xor(pr, off);
                    pi += __shfl_xor(pi, off);
                }
                if (l16 == 0) {
                    sDRr[m * 64 + tr] += pr * cum;
                    sDRi[m * 64 + tr] += pi * cum;
                    sGL[m * 64 + tr] += (pr * rr + pi * ri) * cum;  // Re(g_rho conj(r)) cum
                }
            }
        }
    }
    __syncthreads();

    if (active) {
        const int64_t qo = b * p.dq.s0 + h * p.dq.s1 + (int64_t)c0 * p.dq.s2;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * tt + 4 * g + r;
                if (t < valid) {
                    const int64_t o = qo + (int64_t)t * p.dq.s2 + 16 * jt + l16;
                    store_elem<Tin>(p.dq.re, o, gqR[jt][r] * a.q_scale);
                    store_elem<Tin>(p.dq.im, o, gqI[jt][r] * a.q_scale);
                }
            }
    }
    if (tid < 64 && tid < valid) {
        for (int m = 0; m < M; ++m) {
            p.gl[chain_idx(p, m, b, h) * (int64_t)p.n_chunks * C + c0 + tid] = sGL[m * 64 + tid];
            if (p.drot_re) {
                const int64_t ro = m * a.sr_m + b * a.sr_b + h * a.sr_h + (int64_t)(c0 + tid) * a.sr_t;
                p.drot_re[ro] = sDRr[m * 64 + tid];
                p.drot_im[ro] = sDRi[m * 64 + tid];
            }
        }
    }
}

// ---------------------------------------------------------------- kernel 4 --
template <typename Tin, int C>
__global__ void __launch_bounds__(THREADS) key_side_kernel(BwdParams p) {
    extern __shared__ float smem[];
    float *sQr = smem, *sQi = sQr + D * P;           // Q~ tile, later G'_m
    float *sKr = sQi + D * P, *sKi = sKr + C * P;
    float *sVr = sKi + C * P, *sVi = sVr + C * P;
    float *sGr = sVi + C * P, *sGi = sGr + D * P;    // G_Y tile, later S_m
    float *sL = sGi + D * P, *sRr = sL + MAX_M * 64, *sRi = sRr + MAX_M * 64;
    float *sGL = sRi + MAX_M * 64, *sDl = sGL + MAX_M * 64;
    float *sRed = sDl + MAX_M * 64;                  // [4] wave partials
    float *sGp = sRed + 4;                           // [64] per-key decay_last terms of one state

    const qpam_scan_args &a = p.a;
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int c0 = c * C, valid = min(C, a.T - c0);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const bool carry = (c > 0) || (a.s0_re != nullptr);
    const int M = a.M;

    {
        const int64_t qo = b * a.q.s0 + h * a.q.s1 + (int64_t)c0 * a.q.s2;
        const int64_t ko = b * a.k.s0 + h * a.k.s1 + (int64_t)c0 * a.k.s2;
        const int64_t vo = b * a.v.s0 + h * a.v.s1 + (int64_t)c0 * a.v.s2;
        const int64_t go = b * p.dy.s0 + h * p.dy.s1 + (int64_t)c0 * p.dy.s2;
        float *const gd[2] = {sGr, sGi};
        const float *const gs[2] = {(const float *)p.dy.re + go, (const float *)p.dy.im + go};
        float *const id[6] = {sQr, sQi, sKr, sKi, sVr, sVi};
        const Tin *const is[6] = {(const Tin *)a.q.re + qo, (const Tin *)a.q.im + qo, (const Tin *)a.k.re + ko,
                                  (const Tin *)a.k.im + ko, (const Tin *)a.v.re + vo, (const Tin *)a.v.im + vo};
        const int64_t ist[6] = {a.q.s2, a.q.s2, a.k.s2, a.k.s2, a.v.s2, a.v.s2};
        const float isc[6] = {a.q_scale, a.q_scale, 1.f, 1.f, 1.f, 1.f};
        stage_grad_and_inputs<Tin, C, 2, 6>(gd, gs, p.dy.s2, id, is, ist, isc, valid);
    }
    if (w == 0) {
        chunk_decay_prologue(a, b, h, c0, valid, sL, sRr, sRi);
        for (int m = 0; m < M; ++m) {
            const float L = sL[m * 64 + lane];
            const float Llast = sL[m * 64 + valid - 1];
            sDl[m * 64 + lane] = (lane < valid) ? __expf(fminf(Llast - L, 0.f)) : 0.f;
            sGL[m * 64 + lane] =
                (lane < valid) ? p.gl[chain_idx(p, m, b, h) * (int64_t)p.n_chunks * C + c0 + lane] : 0.f;
        }
    }
    __syncthreads();

    const int st = causal_tile(w);  // key rows s in [16st, 16st+16)
    const bool active = st < C / 16;
    floatx4 gvR[4], gvI[4], gkR[4], gkI[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) gvR[it] = gvI[it] = gkR[it] = gkI[it] = zero4();

    if (active) {
        const int s = 16 * st + l16;  // this lane's key row as MFMA B operand
        floatx4 wr[4], wi[4], dr[4], di[4];  // W[t][s], dA[t][s] for t-tiles tt >= st
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) wr[tt] = wi[tt] = dr[tt] = di[tt] = zero4();
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const float4 bk_r = *reinterpret_cast<const float4 *>(sKr + s * P + 16 * q4 + 4 * g);
            const float4 bk_i = *reinterpret_cast<const float4 *>(sKi + s * P + 16 * q4 + 4 * g);
            const float4 bv_r = *reinterpret_cast<const float4 *>(sVr + s * P + 16 * q4 + 4 * g);
            const float4 bv_i = *reinterpret_cast<const float4 *>(sVi + s * P + 16 * q4 + 4 * g);
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                if (tt < st || 16 * tt >= C) continue;
                const int t = 16 * tt + l16;
                const float4 aq_r = *reinterpret_cast<const float4 *>(sQr + t * P + 16 * q4 + 4 * g);
                const float4 aq_i = *reinterpret_cast<const float4 *>(sQi + t * P + 16 * q4 + 4 * g);
                const float4 ag_r = *reinterpret_cast<const float4 *>(sGr + t * P + 16 * q4 + 4 * g);
                const float4 ag_i = *reinterpret_cast<const float4 *>(sGi + t * P + 16 * q4 + 4 * g);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    wr[tt] = mfma4(aq_r[kk], bk_r[kk], wr[tt]);
                    wr[tt] = mfma4(aq_i[kk], bk_i[kk], wr[tt]);
                    wi[tt] = mfma4(aq_i[kk], bk_r[kk], wi[tt]);
                    wi[tt] = mfma4(-aq_r[kk], bk_i[kk], wi[tt]);
                    dr[tt] = mfma4(ag_r[kk], bv_r[kk], dr[tt]);
                    dr[tt] = mfma4(ag_i[kk], bv_i[kk], dr[tt]);
                    di[tt] = mfma4(ag_i[kk], bv_r[kk], di[tt]);
                    di[tt] = mfma4(-ag_r[kk], bv_i[kk], di[tt]);
                }
            }
        }
        // lane holds t = 16tt + 4g + r, s = 16st + l16: A = W D~ -> (wr, wi); gW = dA conj(D~) -> (dr, di)
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            if (tt < st || 16 * tt >= C) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * tt + 4 * g + r;
                float dtr = 0.f, dti = 0.f;
                if (s <= t) {
#pragma unroll
                    for (int m = 0; m < MAX_M; ++m) {
                        if (m < M) {
                            const float Dm = __expf(fminf(sL[m * 64 + t] - sL[m * 64 + s], 0.f));
                            dtr += sRr[m * 64 + t] * Dm;
                            dti += sRi[m * 64 + t] * Dm;
                        }
                    }
                }
                const float Wr = wr[tt][r], Wi = wi[tt][r], Ar = dr[tt][r], Ai = di[tt][r];
                wr[tt][r] = Wr * dtr - Wi * dti;
                wi[tt][r] = Wr * dti + Wi * dtr;
                dr[tt][r] = Ar * dtr + Ai * dti;
                di[tt][r] = Ai * dtr - Ar * dti;
            }
        }
        // dV[s][i] += sum_t conj(A[t,s]) G[t,i];  dK[s][j] += sum_t conj(gW[t,s]) Q~[t,j]
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            if (tt < st || 16 * tt >= C) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * tt + 4 * g + r;
                const float ar = wr[tt][r], ai = wi[tt][r], gr_ = dr[tt][r], gi_ = di[tt][r];
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    const float yr = sGr[t * P + 16 * it + l16], yi = sGi[t * P + 16 * it + l16];
                    gvR[it] = mfma4(ar, yr, gvR[it]);
                    gvR[it] = mfma4(ai, yi, gvR[it]);
                    gvI[it] = mfma4(ar, yi, gvI[it]);
                    gvI[it] = mfma4(-ai, yr, gvI[it]);
                    const float qr = sQr[t * P + 16 * it + l16], qi = sQi[t * P + 16 * it + l16];
                    gkR[it] = mfma4(gr_, qr, gkR[it]);
                    gkR[it] = mfma4(gi_, qi, gkR[it]);
                    gkI[it] = mfma4(gr_, qi, gkI[it]);
                    gkI[it] = mfma4(-gi_, qr, gkI[it]);
                }
            }
        }
    }

    // state-write gradients: G'_m = dS after this chunk
    for (int m = 0; m < M; ++m) {
        __syncthreads();
        const float *gsrc = gstate(p, m, b, h, c);
        if (carry) {
            const float *ssrc = fstate(p, m, b, h, c);
            F32Tile<D> t[4];
            tile_load<D>(t[0], gsrc, D, D);
            tile_load<D>(t[1], gsrc + D * D, D, D);
            tile_load<D>(t[2], ssrc, D, D);
            tile_load<D>(t[3], ssrc + D * D, D, D);
            tile_store<D>(sQr, t[0], 1.f);
            tile_store<D>(sQi, t[1], 1.f);
            tile_store<D>(sGr, t[2], 1.f);
            tile_store<D>(sGi, t[3], 1.f);
        } else {
            load_state_planes(sQr, sQi, gsrc);
        }
        __syncthreads();
        // g_total = sum Re(conj(G') S)
        if (carry) {
            float part = 0.f;
            for (int e = tid; e < D * D; e += THREADS) {
                const int i = e >> 6, j = e & 63;
                part += sQr[i * P + j] * sGr[i * P + j] + sQi[i * P + j] * sGi[i * P + j];
            }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off);
            if (lane == 0) sRed[w] = part;
        }
        if (active) {
            const int s = 16 * st + l16;
            const float dls = sDl[m * 64 + s];
            // Z[s][i] = sum_j K[s,j] G'[i,j]
            floatx4 zr[4], zi[4];
#pragma unroll
            for (int it = 0; it < 4; ++it) zr[it] = zi[it] = zero4();
#pragma unroll
            for (int q4 = 0; q4 < 4; ++q4) {
                const float4 ak_r = *reinterpret_cast<const float4 *>(sKr + s * P + 16 * q4 + 4 * g);
                const float4 ak_i = *reinterpret_cast<const float4 *>(sKi + s * P + 16 * q4 + 4 * g);
                const float4 av_r = *reinterpret_cast<const float4 *>(sVr + s * P + 16 * q4 + 4 * g);
                const float4 av_i = *reinterpret_cast<const float4 *>(sVi + s * P + 16 * q4 + 4 * g);
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    const int i = 16 * it + l16;
                    const float4 bg_r = *reinterpret_cast<const float4 *>(sQr + i * P + 16 * q4 + 4 * g);
                    const float4 bg_i = *reinterpret_cast<const float4 *>(sQi + i * P + 16 * q4 + 4 * g);
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        zr[it] = mfma4(ak_r[kk], bg_r[kk], zr[it]);
                        zr[it] = mfma4(-ak_i[kk], bg_i[kk], zr[it]);
                        zi[it] = mfma4(ak_r[kk], bg_i[kk], zi[it]);
                        zi[it] = mfma4(ak_i[kk], bg_r[kk], zi[it]);
                    }
                }
                // dK[s][j] += dl[s] sum_i V[s,i] conj(G'[i,j])  (i = 16 q4 + 4 g + kk)
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    const int i = 16 * q4 + 4 * g + kk;
                    const float vr = av_r[kk] * dls, vi = av_i[kk] * dls;
#pragma unroll
                    for (int jt = 0; jt < 4; ++jt) {
                        const float gr_ = sQr[i * P + 16 * jt + l16], gi_ = sQi[i * P + 16 * jt + l16];
                        gkR[jt] = mfma4(vr, gr_, gkR[jt]);
                        gkR[jt] = mfma4(vi, gi_, gkR[jt]);
                        gkI[jt] = mfma4(vi, gr_, gkI[jt]);
                        gkI[jt] = mfma4(-vr, gi_, gkI[jt]);
                    }
                }
            }
            // lane holds Z[s' = 16st + 4g + r][i = 16it + l16]
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int sr_ = 16 * st + 4 * g + r;
                const float dl = sDl[m * 64 + sr_];
                float gdl = 0.f;
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    const float z_r = zr[it][r], z_i = zi[it][r];
                    const float vr = sVr[sr_ * P + 16 * it + l16], vi = sVi[sr_ * P + 16 * it + l16];
                    gdl += vr * z_r + vi * z_i;
                    gvR[it][r] += dl * z_r;
                    gvI[it][r] += dl * z_i;
                }
#pragma unroll
                for (int off = 1; off < 16; off <<= 1) gdl += __shfl_xor(gdl, off);
                if (l16 == 0 && sr_ < C) {  // key sr_ is this lane's own: plain updates
                    const float x = sL[m * 64 + valid - 1] - sL[m * 64 + sr_];
                    const float gp = (sr_ < valid && sr_ != valid - 1 && x <= 0.f) ? gdl * dl : 0.f;
                    sGL[m * 64 + sr_] -= gp;
                    sGp[sr_] = gp;  // summed into the last step below, in a fixed order
                }
            }
        }
        __syncthreads();
        if (w == 0) {
            float x = lane < C ? sGp[lane] : 0.f;
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
            if (lane == 0) {
                if (carry) x += (sRed[0] + sRed[1] + sRed[2] + sRed[3]) * __expf(sL[m * 64 + valid - 1]);
                sGL[m * 64 + valid - 1] += x;
            }
        }
    }
    __syncthreads();

    if (active) {
        const int64_t ko = b * p.dk.s0 + h * p.dk.s1 + (int64_t)c0 * p.dk.s2;
        const int64_t vo = b * p.dv.s0 + h * p.dv.s1 + (int64_t)c0 * p.dv.s2;
#pragma unroll
        for (int it = 0; it < 4; ++it)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int s = 16 * st + 4 * g + r;
                if (s < valid) {
                    const int64_t o1 = ko + (int64_t)s * p.dk.s2 + 16 * it + l16;
                    store_elem<Tin>(p.dk.re, o1, gkR[it][r]);
                    store_elem<Tin>(p.dk.im, o1, gkI[it][r]);
                    const int64_t o2 = vo + (int64_t)s * p.dv.s2 + 16 * it + l16;
                    store_elem<Tin>(p.dv.re, o2, gvR[it][r]);
                    store_elem<Tin>(p.dv.im, o2, gvI[it][r]);
                }
            }
    }
    // d gamma: reverse cumsum of dL/dL_t inside the chunk, then / (gamma + 1e-6)
    if (w == 0) {
        for (int m = 0; m < M; ++m) {
            float x = (lane < valid) ? sGL[m * 64 + lane] : 0.f;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const float y = __shfl_down(x, off);
                if (lane + off < 64) x += y;
            }
            if (lane < valid) {
                const int64_t go = m * a.sg_m + b * a.sg_b + h * a.sg_h + (int64_t)(c0 + lane) * a.sg_t;
                p.dgamma[go] = x / (a.gamma[go] + LOG_EPS);
            }
        }
    }
}

// ------------------------------------------------------ bf16 MFMA path ----
// bf16 q/k/v with C = 64: the three chunk-parallel backward kernels on
// v_mfma_f32_16x16x32_bf16 with bf16 LDS tiles (dY and the fp32 states are
// rounded to bf16 when staged; accumulation stays fp32).  q is staged
// unscaled; q_scale is applied where q~ enters an fp32 result.
using U16 = unsigned short;

// Gradient-state pass (reverse): PASS_SPLIT blocks of GPASS_THREADS (8 waves) per
// (b, h) walk the chunks from last to first with the running dS of every state m
// in registers (fp32, accumulator layout; block `half` owns value rows 32 half..
// (dY columns 32 half..), its wave w the 16 x 16 tile (rows 16 it.., it = 2 half
// + (w & 1); key columns 16 (w >> 1)..) of each state).  The chunk's Q and dY
// tiles are loaded once for all states: per chunk, every state's bf16 snapshot
// of dS after the chunk, then dS_m <- total_m dS_m + sum_t conj(rho_m[t]) q_scale
// dY_t (x) conj(q_t) on MFMA.  dS0 is written when requested.  Chunk c-2's dY, Q,
// per-step weights and totals are loaded while chunk c is processed (two register
// sets).  The weights conj(rho_m[t]) q_scale come from the forward's per-step
// table (seg_decay forms them beside its decay prefixes: formed here, the
// chunk's log-prefix scan and the cross-lane moves of its weights were 40 % of
// every step of this sequential pass), and dY is staged once per state already
// weighted (fp32 product rounded once to bf16), so the MFMA operands come
// straight from LDS.  Rows past the end of the sequence carry zero weights.
constexpr int GSNAP_ROWS = 64 / PASS_SPLIT;  // dS rows of one block
constexpr int GPASS_THREADS = 512;
template <int M>
constexpr size_t gpass_bf16_smem() {
    return (size_t)2 * PLANE_B * 2                 // Q [plane][64][PB]
           + (size_t)2 * M * PLANE_B * 2           // weighted dY (bf16) [state][plane][64][PB] (this block's columns)
           + (size_t)2 * M * GSNAP_ROWS * PB * 2;  // bf16 snapshots of the block's dS rows [state][plane][32][PB]
}

template <int M, bool DYBF>
__global__ void __launch_bounds__(GPASS_THREADS) grad_pass_bf16_kernel(BwdParams p) {
    constexpr int NT = GPASS_THREADS;
    extern __shared__ float smem[];
    U16 *sQ = reinterpret_cast<U16 *>(smem);  // + plane * PLANE_B
    U16 *sG = sQ + 2 * PLANE_B;               // + (2 m + plane) * PLANE_B
    U16 *sS = sG + 2 * M * PLANE_B;           // + (2 m + plane) * GSNAP_ROWS * PB

    const qpam_scan_args &a = p.a;
    // the halves of a (b, h) are B H blocks apart (same XCD when 8 | B H)
    const int n_bh = a.B * a.H;
    const int bh = blockIdx.x % n_bh, half = blockIdx.x / n_bh;
    const int b = bh / a.H, h = bh % a.H;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int it = 2 * half + (w & 1), jt = w >> 1;
    const int yc0 = 32 * half;  // dY columns of this block's value rows
    const int n = p.n_chunks;
    const U16 *qre = (const U16 *)a.q.re + b * a.q.s0 + h * a.q.s1, *qim = (const U16 *)a.q.im + b * a.q.s0 + h * a.q.s1;
    // dY planes: fp32, or bf16 when DYBF (the same element offsets)
    using YT = typename std::conditional<DYBF, U16, float>::type;
    const YT *yre = (const YT *)p.dy.re + b * p.dy.s0 + h * p.dy.s1;
    const YT *yim = (const YT *)p.dy.im + b * p.dy.s0 + h * p.dy.s1;
    const bool need_ds0 = p.ds0_re != nullptr;

    floatx4 gR[M], gI[M];  // dS_m[i][j], rows 16it + 4g + r, cols 16jt + l16
#pragma unroll
    for (int m = 0; m < M; ++m) {
        gR[m] = gI[m] = zero4();
        if (p.ds_re) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t o = chain_idx(p, m, b, h) * D * D + (int64_t)(16 * it + 4 * g + r) * D + 16 * jt + l16;
                gR[m][r] = p.ds_re[o];
                gI[m][r] = p.ds_im[o];
            }
        }
    }

    // this block's dY columns of a chunk: one 16-byte piece per thread and plane
    // (bf16: 256 pieces, held by threads t and t + 256 alike; the two halves of the
    // block then stage alternate states)
    constexpr int YNT = DYBF ? 256 : NT;
    const int ytid = tid & (YNT - 1);
    using YRegs = typename std::conditional<DYBF, BfTileRegs<YNT, 32>, F32TileRegs<YNT, 32>>::type;
    // the dY row this thread stages (one 16-byte piece per plane; the weights
    // of that row, conj(rho_m[t]) q_scale, come from the forward's per-step table)
    const int wrow = DYBF ? (ytid >> 2) : (ytid / 8);
    struct ChunkRegs {
        YRegs yr, yi;
        BfTileRegs<NT> qr, qi;
        float wr[M], wi[M], tot[M];
    };
    ChunkRegs cr0, cr1;
    float tot_cur[M];  // total decays of the chunk staged last (the one the next step processes)
#pragma unroll
    for (int m = 0; m < M; ++m) tot_cur[m] = 1.f;
    auto load_chunk = [&](int c, ChunkRegs &x) {
        const int c0 = c * 64, valid = min(64, a.T - c0);
        const int64_t yo = (int64_t)c0 * p.dy.s2;
        if constexpr (DYBF) {
            const int r = min(ytid >> 2, valid - 1), c8 = ytid & 3;
            x.yr.v[0] = *reinterpret_cast<const uintx4 *>(yre + yo + (int64_t)r * p.dy.s2 + yc0 + 8 * c8);
            x.yi.v[0] = *reinterpret_cast<const uintx4 *>(yim + yo + (int64_t)r * p.dy.s2 + yc0 + 8 * c8);
        } else {
            tile_load_f32<YNT, 32>(x.yr, yre + yo, p.dy.s2, valid, yc0);
            tile_load_f32<YNT, 32>(x.yi, yim + yo, p.dy.s2, valid, yc0);
        }
        const int64_t qo = (int64_t)c0 * a.q.s2;
        tile_load_bf<NT>(x.qr, qre + qo, a.q.s2, valid);
        tile_load_bf<NT>(x.qi, qim + qo, a.q.s2, valid);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            // rows past the end of the sequence carry the forward's zero weights
            const int64_t wo = chain_idx(p, m, b, h) * p.n_chunks * 64 + c0 + wrow;
            x.wr[m] = p.wgr[wo];
            x.wi[m] = p.wgi[wo];
            // a vector load (lane-dependent address; lane 0's value is taken when the
            // chunk is staged): a scalar load would share the LDS counter, and the next
            // LDS wait would wait for it too
            x.tot[m] = p.totals[chain_idx(p, m, b, h) * p.n_chunks + max(c - (lane & 1), 0)];
        }
    };
    auto stage_chunk = [&](int c, const ChunkRegs &x) {
        // nothing of the staging moves above this point: its first use of the staged
        // register set is where the compiler waits for that set's loads, and the
        // memory counter completes in order, so a use hoisted to the top of the step
        // would also wait for everything loaded one step earlier
        __builtin_amdgcn_sched_barrier(0);
        const int valid = min(64, a.T - c * 64);
        tile_store_bf<NT>(sQ, x.qr);
        tile_store_bf<NT>(sQ + PLANE_B, x.qi);
#pragma unroll
        for (int m = 0; m < M; ++m) tot_cur[m] = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(x.tot[m])));
#pragma unroll
        for (int m = 0; m < M; ++m) {
            if (DYBF && (tid >> 8) != (m & 1)) continue;  // (bf16: the other half stages state m)
            // row wrow of dY times conj(rho_m[t]) q_scale, rounded once to bf16
            const float wr = x.wr[m], wi = x.wi[m];
            U16 *gr = sG + 2 * m * PLANE_B, *gi = gr + PLANE_B;
            if constexpr (DYBF) {
                const int o = wrow * PB + yc0 + 8 * (ytid & 3);
                const floatx8 ya = to_f(__builtin_bit_cast(bf16x8, x.yr.v[0]));
                const floatx8 yb = to_f(__builtin_bit_cast(bf16x8, x.yi.v[0]));
                *reinterpret_cast<bf16x8 *>(gr + o) = to_bf(wr * ya - wi * yb);
                *reinterpret_cast<bf16x8 *>(gi + o) = to_bf(wr * yb + wi * ya);
            } else {
                const int o = wrow * PB + yc0 + 4 * (ytid % 8);
                const floatx4 ya = x.yr.v[0], yb = x.yi.v[0];
                const floatx4 pr = wr * ya - wi * yb, pi = wr * yb + wi * ya;
                *reinterpret_cast<uint2 *>(gr + o) = make_uint2(pack_bf16x2(pr[0], pr[1]), pack_bf16x2(pr[2], pr[3]));
                *reinterpret_cast<uint2 *>(gi + o) = make_uint2(pack_bf16x2(pi[0], pi[1]), pack_bf16x2(pi[2], pi[3]));
            }
        }
    };

    // reverse order: step k handles chunk c = n-1-k; chunk c - 2 (dY, Q, gammas,
    // rotations, totals) is loaded into register set k & 1 and staged at the end of
    // step k + 1 (one LDS buffer, staged between two barriers)
    auto step = [&](int k, ChunkRegs &mine, ChunkRegs &next) {
        const int c = n - 1 - k;
        // unconditional (chunk 0 is re-read near the end): the same memory operation
        // count on every path keeps the compiler's waits for the staged set exact
        load_chunk(max(c - 2, 0), mine);
        // bf16 snapshots of dS after chunk c: into LDS now, to global memory as
        // 16-byte row pieces after the next barrier
#pragma unroll
        for (int m = 0; m < M; ++m)
            acc_store_bf_pairs<PB>(sS + 2 * m * GSNAP_ROWS * PB, sS + (2 * m + 1) * GSNAP_ROWS * PB, gR[m], gI[m],
                                   16 * (w & 1), 16 * jt);
        if (c > 0 || need_ds0) {
            // dG rows (value i) x cols (key j): A = (conj(rho) q_scale dY)^T, B = Q (k = t)
            const U16 *Qr = sQ, *Qi = sQ + PLANE_B;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const U16 *Gr = sG + 2 * m * PLANE_B, *Gi = Gr + PLANE_B;
                floatx4 accR = zero4(), accI = zero4();
#pragma unroll
                for (int kp = 0; kp < 2; ++kp) {
                    const int t0 = 32 * kp + 8 * g;
                    const bf16x8 ar = ld_tr(Gr, t0, t0 + 4, 16 * it), ai = ld_tr(Gi, t0, t0 + 4, 16 * it),
                                 nar = neg_bf(ar);
                    const bf16x8 qr = ld_tr(Qr, t0, t0 + 4, 16 * jt), qi = ld_tr(Qi, t0, t0 + 4, 16 * jt);
                    accR = mfma_bf(ar, qr, accR);
                    accR = mfma_bf(ai, qi, accR);
                    accI = mfma_bf(ai, qr, accI);
                    accI = mfma_bf(nar, qi, accI);
                }
                const float tot = tot_cur[m];  // chunk c's total, loaded two steps ahead
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    gR[m][r] = tot * gR[m][r] + accR[r];
                    gI[m][r] = tot * gI[m][r] + accI[r];
                }
            }
        }
        // also unconditional: past the end, chunk 0 (which `next` then holds) is
        // staged again
        __syncthreads();
        {  // the snapshot rows: 16 bytes per thread and state
            const int pl = tid >> 8, row = (tid & 255) >> 3, q = tid & 7;
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const uint4 v = *reinterpret_cast<const uint4 *>(sS + (2 * m + pl) * GSNAP_ROWS * PB + row * PB + 8 * q);
                *reinterpret_cast<uint4 *>(gsnap(p, m, b, h, c) + pl * D * D + (GSNAP_ROWS * half + row) * D + 8 * q) = v;
            }
        }
        stage_chunk(max(c - 1, 0), next);
        __syncthreads();
    };
    load_chunk(n - 1, cr0);
    load_chunk(max(n - 2, 0), cr1);
    stage_chunk(n - 1, cr0);
    __syncthreads();
    // pairs of steps without conditions inside the loop, odd tail after it
    int k = 0;
    for (; k + 1 < n; k += 2) {
        step(k, cr0, cr1);
        step(k + 1, cr1, cr0);
    }
    if (k < n) step(k, cr0, cr1);
    if (need_ds0) {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t o = chain_idx(p, m, b, h) * D * D + (int64_t)(16 * it + 4 * g + r) * D + 16 * jt + l16;
                p.ds0_re[o] = gR[m][r];
                p.ds0_im[o] = gI[m][r];
            }
    }
}

// Decay inputs of state m of a chunk for one wave (lane = step): gamma and the
// rotation, loaded at kernel entry so that their latency overlaps the tile loads.
struct DecayIn {
    float gam, rr, ri;
};
__device__ __forceinline__ DecayIn decay_load(const qpam_scan_args &a, int m, int b, int h, int c0, int valid) {
    const int lane = threadIdx.x & 63;
    DecayIn d{1.f, 1.f, 0.f};
    if (lane < valid) {
        d.gam = a.gamma[m * a.sg_m + b * a.sg_b + h * a.sg_h + (int64_t)(c0 + lane) * a.sg_t];
        if (a.rot_re) {
            const int64_t ro = m * a.sr_m + b * a.sr_b + h * a.sr_h + (int64_t)(c0 + lane) * a.sr_t;
            d.rr = a.rot_re[ro];
            d.ri = a.rot_im[ro];
        }
    }
    return d;
}
// The chunk tables of state m (one wave): L = the log-decay prefix sums (as
// chunk_log_prefix_ok forms them), the rotations, F = exp(-L) and P = r exp(L);
// returns the factorisation test of the state.
__device__ __forceinline__ bool decay_tables(const DecayIn &d, int m, int valid, float *sL, float *sRr, float *sRi,
                                             float *sF, float *sPr, float *sPi) {
    const int lane = threadIdx.x & 63;
    float x = (lane < valid) ? logf(d.gam + LOG_EPS) : 0.f;
    const bool pos = x > 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float y = __shfl_up(x, off);
        if (lane >= off) x += y;
    }
    const bool ok = !__any(pos) && __shfl(x, 63) >= -FACTOR_RANGE;
    sL[m * 64 + lane] = x;
    sRr[m * 64 + lane] = d.rr;
    sRi[m * 64 + lane] = d.ri;
    sF[m * 64 + lane] = __expf(-x);  // unused (possibly inf) when the test fails
    const float e = __expf(x);
    sPr[m * 64 + lane] = d.rr * e;
    sPi[m * 64 + lane] = d.ri * e;
    return ok;
}

// Own-row operands of the chunk kernels: lane (g, l16) of a wave that owns 16
// rows of the chunk reads row l16 of them straight from global memory, either
// columns 32 kp + 8 g .. +7 (an MFMA operand fragment) or the four columns
// 16 jt + 4 g .. +3 that the transposed accumulators of the wave hold; rows at
// or past `valid` read as zero.
__device__ __forceinline__ bf16x8 own_frag(const U16 *row, int kp, bool ok) {
    const int g = (threadIdx.x & 63) >> 4;
    return ok ? *reinterpret_cast<const bf16x8 *>(row + 32 * kp + 8 * g) : __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
}
__device__ __forceinline__ bf16x8 own_frag_f32(const float *row, int kp, bool ok) {
    const int g = (threadIdx.x & 63) >> 4;
    if (!ok) return __builtin_bit_cast(bf16x8, make_uint4(0, 0, 0, 0));
    const floatx4 x0 = *reinterpret_cast<const floatx4 *>(row + 32 * kp + 8 * g);
    const floatx4 x1 = *reinterpret_cast<const floatx4 *>(row + 32 * kp + 8 * g + 4);
    return to_bf(floatx8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]});
}
__device__ __forceinline__ uint2 own_quad(const U16 *row, int jt, bool ok) {
    const int g = (threadIdx.x & 63) >> 4;
    return ok ? *reinterpret_cast<const uint2 *>(row + 16 * jt + 4 * g) : make_uint2(0u, 0u);
}
// element r of four bf16 held in two dwords
__device__ __forceinline__ float quad_elem(uint2 u, int r) {
    const unsigned x = (r < 2) ? u.x : u.y;
    return __uint_as_float((r & 1) ? (x & 0xffff0000u) : (x << 16));
}
// scale * v -> bf16, columns 16 jt + 4 g .. +3 of `row` (one 8-byte store)
__device__ __forceinline__ void store_quad(U16 *row, int jt, const floatx4 &v, float scale) {
    const int g = (threadIdx.x & 63) >> 4;
    *reinterpret_cast<uint2 *>(row + 16 * jt + 4 * g) =
        make_uint2(pack_bf16x2(v[0] * scale, v[1] * scale), pack_bf16x2(v[2] * scale, v[3] * scale));
}

// Query and key sides of a chunk in one pass (bf16 operands, chunk 64): the
// chunk's q, k, v and dY tiles are staged once and each state's snapshots are
// read once.  Wave w takes the query tile and the key tile of the same index i
// (causal work (i + 1) + (4 - i) = 5 tile pairs on every wave).  Phases: the
// query side's score tiles (dQ~ intra, decay-gradient row sums), the key side's
// (dV and dK intra, column sums), then per state the carried read (S_m staged in
// the q tile) and the state write (G'_m, dS after the chunk, in the same tile).
// The score phases are the query- and key-side kernels' own: transposed score
// tiles with the factorised decay D~ and its row / column sums on fp32 MFMA,
// dQ~, dK, dV accumulated transposed and stored as 8-byte runs.
template <int M, bool DYBF>
__global__ void __launch_bounds__(THREADS, 2) chunk_grad_bf16_kernel(BwdParams p) {
    extern __shared__ float smem[];
    U16 *sQr = reinterpret_cast<U16 *>(smem), *sQi = sQr + PLANE_B;  // q, then S_m and G'_m
    U16 *sKr = sQi + PLANE_B, *sKi = sKr + PLANE_B;
    U16 *sVr = sKi + PLANE_B, *sVi = sVr + PLANE_B;
    U16 *sGr = sVi + PLANE_B, *sGi = sGr + PLANE_B;  // dY
    // per-step vectors [M][64]: decay tables; the query rows' results (each wave
    // its own rows); the key side's decay-gradient terms
    float *sL = reinterpret_cast<float *>(sGi + PLANE_B), *sRr = sL + M * 64, *sRi = sRr + M * 64;
    float *sF = sRi + M * 64, *sPr = sF + M * 64, *sPi = sPr + M * 64;
    float *sGq = sPi + M * 64, *sDqr = sGq + M * 64, *sDqi = sDqr + M * 64;
    float *sGL = sDqi + M * 64;
    float *sRed = sGL + M * 64;
    int *sFast = reinterpret_cast<int *>(sRed + 4);  // [M] factorisation tests
    float *sGpw = sRed + 8;                          // [4] wave sums of the decay_last terms of one state

    const qpam_scan_args &a = p.a;
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int c0 = c * 64, valid = min(64, a.T - c0);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const bool carry = (c > 0) || (a.s0_re != nullptr);
    const float qs = a.q_scale;
    // global loads first: decay inputs of state m = w and the Q, K, V, dY tiles
    DecayIn din;
    if (w < M) din = decay_load(a, w, b, h, c0, valid);
    const int tt = causal_tile(w), st = tt;  // query tile and key tile of this wave
    const int t = 16 * tt + l16, s = 16 * st + l16;
    const bool tv = t < valid, sv = s < valid;
    // snapshots of state m (dS after the chunk, and the entering state): state 0
    // is in flight during the score phases, state m+1 while m is processed
    B16Regs gr[2], sr[2];
    auto load_state = [&](int m) {
        const U16 *gsrc = gsnap(p, m, b, h, c);
        regs_load_bf<false>(gr[0], gsrc, D, D);
        regs_load_bf<false>(gr[1], gsrc + D * D, D, D);
        if (carry) {
            const U16 *ssrc = fsnap(p, m, b, h, c);
            regs_load_bf<false>(sr[0], ssrc, D, D);
            regs_load_bf<false>(sr[1], ssrc + D * D, D, D);
        }
    };
    {
        const int64_t qo = b * a.q.s0 + h * a.q.s1 + (int64_t)c0 * a.q.s2;
        const int64_t ko = b * a.k.s0 + h * a.k.s1 + (int64_t)c0 * a.k.s2;
        const int64_t vo = b * a.v.s0 + h * a.v.s1 + (int64_t)c0 * a.v.s2;
        const int64_t go = b * p.dy.s0 + h * p.dy.s1 + (int64_t)c0 * p.dy.s2;
        U16 *const bd[6] = {sQr, sQi, sKr, sKi, sVr, sVi};
        const U16 *const bs[6] = {(const U16 *)a.q.re + qo, (const U16 *)a.q.im + qo, (const U16 *)a.k.re + ko,
                                  (const U16 *)a.k.im + ko, (const U16 *)a.v.re + vo, (const U16 *)a.v.im + vo};
        const int64_t bst[6] = {a.q.s2, a.q.s2, a.k.s2, a.k.s2, a.v.s2, a.v.s2};
        B16Regs rb[8];
        F32Regs rf[2];
#pragma unroll
        for (int i = 0; i < 6; ++i) regs_load_bf<false>(rb[i], bs[i], bst[i], valid);
        if constexpr (DYBF) {
            regs_load_bf<false>(rb[6], (const U16 *)p.dy.re + go, p.dy.s2, valid);
            regs_load_bf<false>(rb[7], (const U16 *)p.dy.im + go, p.dy.s2, valid);
        } else {
            regs_load_f32<false>(rf[0], (const float *)p.dy.re + go, p.dy.s2, valid);
            regs_load_f32<false>(rf[1], (const float *)p.dy.im + go, p.dy.s2, valid);
        }
        if (w < M) {
            const bool ok = decay_tables(din, w, valid, sL, sRr, sRi, sF, sPr, sPi);
            if (lane == 0) sFast[w] = ok ? 1 : 0;
            sGL[w * 64 + lane] = 0.f;
        }
#pragma unroll
        for (int i = 0; i < 6; ++i) regs_store_bf<false>(bd[i], rb[i]);
        if constexpr (DYBF) {
            regs_store_bf<false>(sGr, rb[6]);
            regs_store_bf<false>(sGi, rb[7]);
        } else {
            regs_store_f32_as_bf<false>(sGr, rf[0]);
            regs_store_f32_as_bf<false>(sGi, rf[1]);
        }
    }
    __syncthreads();
    // state 0's snapshots are first read after the score phases: issued here,
    // they do not add to the staging wait (every block of a round loads its
    // tiles at once, so the entry is bandwidth-bound)
    load_state(0);

    bool fast = true;
#pragma unroll
    for (int m = 0; m < M; ++m) fast = fast && sFast[m] != 0;
    // q and dY rows t as MFMA operand fragments
    bf16x8 bq[2][2], bg[2][2];  // [kp][re, im]
#pragma unroll
    for (int kp = 0; kp < 2; ++kp) {
        const int k0 = 32 * kp + 8 * g;
        bq[kp][0] = ld8(sQr + t * PB + k0);
        bq[kp][1] = ld8(sQi + t * PB + k0);
        bg[kp][0] = ld8(sGr + t * PB + k0);
        bg[kp][1] = ld8(sGi + t * PB + k0);
    }
    floatx4 gqR[4], gqI[4];
#pragma unroll
    for (int jt = 0; jt < 4; ++jt) gqR[jt] = gqI[jt] = zero4();
    {
        // fast path: Z_m[t] in element m of lanes g == 0 (fp32 MFMA, rows m); gD~[t][t]
        floatx4 zR = zero4(), zI = zero4();
        float dgr = 0.f, dgi = 0.f;
        // general path: per-lane partial row sums
        float rowp[MAX_M], grr[MAX_M], gri[MAX_M];
#pragma unroll
        for (int m = 0; m < MAX_M; ++m) rowp[m] = grr[m] = gri[m] = 0.f;
        // B operand of the decay-factor product: lane (g = m, l16) holds P_m[t]
        const float pbr = (g < M) ? sPr[g * 64 + t] : 0.f, pbi = (g < M) ? sPi[g * 64 + t] : 0.f;
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            if (2 * kp > tt) continue;
            floatx4 gwr[2], gwi[2];  // gW^T tiles st = 2 kp, 2 kp + 1
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int st = 2 * kp + h2;
                gwr[h2] = gwi[h2] = zero4();
                if (st > tt) continue;
                const int s = 16 * st + l16;
                // W^T[s][t] = sum_j conj(k[s,j]) q[t,j],  dA^T[s][t] = sum_i conj(v[s,i]) dY[t,i]
                floatx4 wr = zero4(), wi = zero4(), dr = zero4(), di = zero4();
#pragma unroll
                for (int kq = 0; kq < 2; ++kq) {
                    const int k0 = 32 * kq + 8 * g;
                    const bf16x8 akr = ld8(sKr + s * PB + k0), aki = ld8(sKi + s * PB + k0);
                    const bf16x8 avr = ld8(sVr + s * PB + k0), avi = ld8(sVi + s * PB + k0);
                    wr = mfma_bf(akr, bq[kq][0], wr);
                    wr = mfma_bf(aki, bq[kq][1], wr);
                    wi = mfma_bf(akr, bq[kq][1], wi);
                    wi = mfma_bf(neg_bf(aki), bq[kq][0], wi);
                    dr = mfma_bf(avr, bg[kq][0], dr);
                    dr = mfma_bf(avi, bg[kq][1], dr);
                    di = mfma_bf(avr, bg[kq][1], di);
                    di = mfma_bf(neg_bf(avi), bg[kq][0], di);
                }
                if (fast) {
                    // D~^T[s][t] = sum_m F_m[s] P_m[t]: A lane (g = m, l16) holds F_m[16 st + l16]
                    const float fa = (g < M) ? sF[g * 64 + s] : 0.f;
                    const floatx4 Dr = mfma4(fa, pbr, zero4()), Di = mfma4(fa, pbi, zero4());
                    floatx4 gdr, gdi;  // gD~ = dA conj(W), q_scale applied to the row sums
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        gwr[h2][r] = dr[r] * Dr[r] + di[r] * Di[r];
                        gwi[h2][r] = di[r] * Dr[r] - dr[r] * Di[r];
                        gdr[r] = dr[r] * wr[r] + di[r] * wi[r];
                        gdi[r] = di[r] * wr[r] - dr[r] * wi[r];
                    }
                    if (st == tt) {  // diagonal tile: gW on s <= t, row sums over s < t, gD~[t][t] apart
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int si = 4 * g + r;
                            if (si == l16) dgr = gdr[r], dgi = gdi[r];
                            gwr[h2][r] = (si <= l16) ? gwr[h2][r] : 0.f;
                            gwi[h2][r] = (si <= l16) ? gwi[h2][r] : 0.f;
                            gdr[r] = (si < l16) ? gdr[r] : 0.f;
                            gdi[r] = (si < l16) ? gdi[r] : 0.f;
                        }
                    }
                    // Z_m[t] += sum_s F_m[s] gD~[t][s]: A lane (g, l16 = m) holds F_m[16 st + 4 g + r]
                    floatx4 fz = zero4();
                    if (l16 < M) fz = *reinterpret_cast<const floatx4 *>(sF + l16 * 64 + 16 * st + 4 * g);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        zR = mfma4(fz[r], gdr[r], zR);
                        zI = mfma4(fz[r], gdi[r], zI);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int sr = 16 * st + 4 * g + r;
                        if (sr > t) continue;
                        float Dm[MAX_M], nc[MAX_M];
                        float dtr = 0.f, dti = 0.f;
#pragma unroll
                        for (int m = 0; m < MAX_M; ++m) {
                            Dm[m] = nc[m] = 0.f;
                            if (m < M) {
                                const float x = sL[m * 64 + t] - sL[m * 64 + sr];
                                Dm[m] = __expf(fminf(x, 0.f));
                                nc[m] = (x <= 0.f && sr != t) ? 1.f : 0.f;
                                dtr += sRr[m * 64 + t] * Dm[m];
                                dti += sRi[m * 64 + t] * Dm[m];
                            }
                        }
                        const float Ar = dr[r], Ai = di[r];
                        const float Wr = wr[r] * qs, Wi = wi[r] * qs;
                        gwr[h2][r] = Ar * dtr + Ai * dti;
                        gwi[h2][r] = Ai * dtr - Ar * dti;
                        const float gdr = Ar * Wr + Ai * Wi, gdi = Ai * Wr - Ar * Wi;
#pragma unroll
                        for (int m = 0; m < MAX_M; ++m) {
                            if (m < M) {
                                const float gdm = gdr * sRr[m * 64 + t] + gdi * sRi[m * 64 + t];
                                rowp[m] += gdm * Dm[m] * nc[m];  // the column part is summed by the key side
                                grr[m] += gdr * Dm[m];
                                gri[m] += gdi * Dm[m];
                            }
                        }
                    }
                }
            }
            // dQ~^T[j][t] += sum_s K[s][j] gW[t][s]  (transposed reads of K x register gW)
            const bf16x8 ar = frag_from_acc(gwr[0], gwr[1]), ai = frag_from_acc(gwi[0], gwi[1]);
            const bf16x8 nai = neg_bf(ai);
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                const int r0 = 32 * kp + 4 * g;
                const bf16x8 kr = ld_tr(sKr, r0, r0 + 16, 16 * jt), ki = ld_tr(sKi, r0, r0 + 16, 16 * jt);
                gqR[jt] = mfma_bf(kr, ar, gqR[jt]);
                gqR[jt] = mfma_bf(ki, nai, gqR[jt]);
                gqI[jt] = mfma_bf(ki, ar, gqI[jt]);
                gqI[jt] = mfma_bf(kr, ai, gqI[jt]);
            }
        }
        // row results of the intra-chunk part -> sGq / sDq* (lanes g == 0; each wave its own rows)
        if (fast) {
            dgr += __shfl_xor(dgr, 16);  // one lane of the column holds gD~[t][t], the others 0
            dgr += __shfl_xor(dgr, 32);
            dgi += __shfl_xor(dgi, 16);
            dgi += __shfl_xor(dgi, 32);
            if (g == 0) {
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float e = __expf(sL[m * 64 + t]) * qs;
                    const float er = zR[m] * e, ei = zI[m] * e;
                    sGq[m * 64 + t] = sRr[m * 64 + t] * er + sRi[m * 64 + t] * ei;
                    sDqr[m * 64 + t] = er + qs * dgr;
                    sDqi[m * 64 + t] = ei + qs * dgi;
                }
            }
        } else {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float x = rowp[m], yr = grr[m], yi = gri[m];
                x += __shfl_xor(x, 16);
                x += __shfl_xor(x, 32);
                yr += __shfl_xor(yr, 16);
                yr += __shfl_xor(yr, 32);
                yi += __shfl_xor(yi, 16);
                yi += __shfl_xor(yi, 32);
                if (g == 0) {
                    sGq[m * 64 + t] = x;
                    sDqr[m * 64 + t] = yr;
                    sDqi[m * 64 + t] = yi;
                }
            }
        }
    }

    floatx4 gvR[4], gvI[4], gkR[4], gkI[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) gvR[it] = gvI[it] = gkR[it] = gkI[it] = zero4();
    {
        // fast path: the column sums C[m][s] in element m of lanes g == 0 (fp32 MFMA)
        floatx4 cR = zero4();
        float colp[MAX_M];  // general path, per-lane partials
#pragma unroll
        for (int m = 0; m < MAX_M; ++m) colp[m] = 0.f;
        // B operand of the decay-factor product: lane (g = m, l16) holds q_scale F_m[s]
        const float fb = (g < M) ? sF[g * 64 + s] * qs : 0.f;
        bf16x8 bk[2][2], bv[2][2];  // [k half][re, im] of k and v, rows s
#pragma unroll
        for (int kq = 0; kq < 2; ++kq) {
            const int k0 = 32 * kq + 8 * g;
            bk[kq][0] = ld8(sKr + s * PB + k0);
            bk[kq][1] = ld8(sKi + s * PB + k0);
            bv[kq][0] = ld8(sVr + s * PB + k0);
            bv[kq][1] = ld8(sVi + s * PB + k0);
        }
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            if (2 * kp + 1 < st) continue;
            floatx4 aR[2], aI[2], gR[2], gI[2];  // A' = q_scale W D~ and gA = q_scale dA conj(D~), t tiles 2kp + h2
#pragma unroll
            for (int h2 = 0; h2 < 2; ++h2) {
                const int tt = 2 * kp + h2;
                aR[h2] = aI[h2] = gR[h2] = gI[h2] = zero4();
                if (tt < st) continue;
                const int t = 16 * tt + l16;
                // W[t][s] = sum_j q[t,j] conj(k[s,j]),  dA[t][s] = sum_i dY[t,i] conj(v[s,i])
                floatx4 wr = zero4(), wi = zero4(), dr = zero4(), di = zero4();
#pragma unroll
                for (int kq = 0; kq < 2; ++kq) {
                    const int k0 = 32 * kq + 8 * g;
                    const bf16x8 aqr = ld8(sQr + t * PB + k0), aqi = ld8(sQi + t * PB + k0);
                    const bf16x8 agr = ld8(sGr + t * PB + k0), agi = ld8(sGi + t * PB + k0);
                    wr = mfma_bf(aqr, bk[kq][0], wr);
                    wr = mfma_bf(aqi, bk[kq][1], wr);
                    wi = mfma_bf(aqi, bk[kq][0], wi);
                    wi = mfma_bf(neg_bf(aqr), bk[kq][1], wi);
                    dr = mfma_bf(agr, bv[kq][0], dr);
                    dr = mfma_bf(agi, bv[kq][1], dr);
                    di = mfma_bf(agi, bv[kq][0], di);
                    di = mfma_bf(neg_bf(agr), bv[kq][1], di);
                }
                if (fast) {
                    // q_scale D~[t][s] = sum_m P_m[t] q_scale F_m[s]: A lane (g = m, l16) holds P_m[16 tt + l16]
                    const float par = (g < M) ? sPr[g * 64 + t] : 0.f, pai = (g < M) ? sPi[g * 64 + t] : 0.f;
                    floatx4 Dr = mfma4(par, fb, zero4()), Di = mfma4(pai, fb, zero4());
                    if (tt == st) {  // diagonal tile: A' and gA on t >= s
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            Dr[r] = (4 * g + r >= l16) ? Dr[r] : 0.f;
                            Di[r] = (4 * g + r >= l16) ? Di[r] : 0.f;
                        }
                    }
                    floatx4 gdr, gdi;  // gD~ = dA conj(W), q_scale applied to the column sums
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        aR[h2][r] = wr[r] * Dr[r] - wi[r] * Di[r];
                        aI[h2][r] = wr[r] * Di[r] + wi[r] * Dr[r];
                        gR[h2][r] = dr[r] * Dr[r] + di[r] * Di[r];
                        gI[h2][r] = di[r] * Dr[r] - dr[r] * Di[r];
                        gdr[r] = dr[r] * wr[r] + di[r] * wi[r];
                        gdi[r] = di[r] * wr[r] - dr[r] * wi[r];
                    }
                    if (tt == st) {  // column sums over t > s
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            gdr[r] = (4 * g + r > l16) ? gdr[r] : 0.f;
                            gdi[r] = (4 * g + r > l16) ? gdi[r] : 0.f;
                        }
                    }
                    // C[m][s] += sum_t Re(gD~[t][s] conj(P_m[t])): A lane (g, l16 = m) holds P_m[16 tt + 4 g + r]
                    floatx4 p4r = zero4(), p4i = zero4();
                    if (l16 < M) {
                        p4r = *reinterpret_cast<const floatx4 *>(sPr + l16 * 64 + 16 * tt + 4 * g);
                        p4i = *reinterpret_cast<const floatx4 *>(sPi + l16 * 64 + 16 * tt + 4 * g);
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        cR = mfma4(p4r[r], gdr[r], cR);
                        cR = mfma4(p4i[r], gdi[r], cR);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int tr = 16 * tt + 4 * g + r;
                        const float Wr = wr[r] * qs, Wi = wi[r] * qs, Ar = dr[r], Ai = di[r];
                        const float gdr = Ar * Wr + Ai * Wi, gdi = Ai * Wr - Ar * Wi;
                        float dtr = 0.f, dti = 0.f;
                        if (s <= tr) {
#pragma unroll
                            for (int m = 0; m < MAX_M; ++m) {
                                if (m < M) {
                                    const float x = sL[m * 64 + tr] - sL[m * 64 + s];
                                    const float Dm = __expf(fminf(x, 0.f));
                                    const float rr = sRr[m * 64 + tr], ri = sRi[m * 64 + tr];
                                    dtr += rr * Dm;
                                    dti += ri * Dm;
                                    if (x <= 0.f && s != tr) colp[m] += (gdr * rr + gdi * ri) * Dm;
                                }
                            }
                        }
                        aR[h2][r] = Wr * dtr - Wi * dti;
                        aI[h2][r] = Wr * dti + Wi * dtr;
                        gR[h2][r] = (Ar * dtr + Ai * dti) * qs;
                        gI[h2][r] = (Ai * dtr - Ar * dti) * qs;
                    }
                }
            }
            // dV^T[i][s] += sum_t dY[t][i] conj(A'[t][s]);  dK^T[j][s] += sum_t q[t][j] conj(gA[t][s])
            const bf16x8 ar = frag_from_acc(aR[0], aR[1]), ai = frag_from_acc(aI[0], aI[1]);
            const bf16x8 gr_ = frag_from_acc(gR[0], gR[1]), gi_ = frag_from_acc(gI[0], gI[1]);
            const bf16x8 nai = neg_bf(ai), ngi = neg_bf(gi_);
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                const int r0 = 32 * kp + 4 * g;
                const bf16x8 yr = ld_tr(sGr, r0, r0 + 16, 16 * it), yi = ld_tr(sGi, r0, r0 + 16, 16 * it);
                gvR[it] = mfma_bf(yr, ar, gvR[it]);
                gvR[it] = mfma_bf(yi, ai, gvR[it]);
                gvI[it] = mfma_bf(yi, ar, gvI[it]);
                gvI[it] = mfma_bf(yr, nai, gvI[it]);
                const bf16x8 qr = ld_tr(sQr, r0, r0 + 16, 16 * it), qi = ld_tr(sQi, r0, r0 + 16, 16 * it);
                gkR[it] = mfma_bf(qr, gr_, gkR[it]);
                gkR[it] = mfma_bf(qi, gi_, gkR[it]);
                gkI[it] = mfma_bf(qi, gr_, gkI[it]);
                gkI[it] = mfma_bf(qr, ngi, gkI[it]);
            }
        }
        // column part of the decay-matrix gradient: dL_m[s] -= F_m[s] C[m][s] (this wave's keys)
        if (fast) {
            if (g == 0) {
#pragma unroll
                for (int m = 0; m < M; ++m) sGL[m * 64 + s] -= cR[m] * sF[m * 64 + s] * qs;
            }
        } else {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float x = colp[m];
                x += __shfl_xor(x, 16);
                x += __shfl_xor(x, 32);
                if (g == 0) sGL[m * 64 + s] -= x;
            }
        }
    }

    // q of row t (the q tile is overwritten by the states): re-read from global
    // memory where the carried read needs it, in the transposed accumulator
    // layout (held in registers through the state loop, it made the kernel spill)
    const int64_t qrow = b * a.q.s0 + h * a.q.s1 + (int64_t)(c0 + t) * a.q.s2;
    const U16 *qrow_r = (const U16 *)a.q.re + qrow, *qrow_i = (const U16 *)a.q.im + qrow;
    for (int m = 0; m < M; ++m) {
        __syncthreads();  // nothing reads the q tile (m = 0) or G'_{m-1} any more
        if (carry) {  // S_m natural into the q tile; this thread's share of Re<G'_m, S_m>
            regs_store_bf<false>(sQr, sr[0]);
            regs_store_bf<false>(sQi, sr[1]);
            float part = 0.f;
#pragma unroll
            for (int pl = 0; pl < 2; ++pl)
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const uint4 x = gr[pl].v[i], y = sr[pl].v[i];
                    part = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.x),
                                                           __builtin_bit_cast(bf16x2, y.x), part, false);
                    part = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.y),
                                                           __builtin_bit_cast(bf16x2, y.y), part, false);
                    part = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.z),
                                                           __builtin_bit_cast(bf16x2, y.z), part, false);
                    part = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, x.w),
                                                           __builtin_bit_cast(bf16x2, y.w), part, false);
                }
#pragma unroll
            for (int off = 32; off >= 1; off >>= 1) part += __shfl_xor(part, off);
            if (lane == 0) sRed[w] = part;
        }
        __syncthreads();
        if (carry) {
#pragma unroll
            for (int kp = 0; kp < 2; ++kp) {
                const int k0 = 32 * kp + 8 * g;
                bg[kp][0] = ld8(sGr + t * PB + k0);
                bg[kp][1] = ld8(sGi + t * PB + k0);
            }
                // X^T[j][t] = sum_k conj(S_m[k][j]) dY[t][k], two column tiles jt at a time;
                // dQ~ += conj(rho_m[t]) X (rho_m = P_m); d rho_m[t] = sum_j q~[t][j] conj(X[t][j])
                const float rhr = sPr[m * 64 + t], rhi = sPi[m * 64 + t];
                float pr = 0.f, pi = 0.f;
    #pragma unroll
                for (int jh = 0; jh < 2; ++jh) {
                    floatx4 xr[2], xi[2];
    #pragma unroll
                    for (int jj = 0; jj < 2; ++jj) xr[jj] = xi[jj] = zero4();
    #pragma unroll
                    for (int kp = 0; kp < 2; ++kp) {
                        const int k0 = 32 * kp + 8 * g;
                        const bf16x8 ngr = neg_bf(bg[kp][0]);
    #pragma unroll
                        for (int jj = 0; jj < 2; ++jj) {
                            const int jt = 2 * jh + jj;
                            const bf16x8 sr = ld_tr(sQr, k0, k0 + 4, 16 * jt), si = ld_tr(sQi, k0, k0 + 4, 16 * jt);
                            xr[jj] = mfma_bf(sr, bg[kp][0], xr[jj]);
                            xr[jj] = mfma_bf(si, bg[kp][1], xr[jj]);
                            xi[jj] = mfma_bf(sr, bg[kp][1], xi[jj]);
                            xi[jj] = mfma_bf(si, ngr, xi[jj]);
                        }
                    }
    #pragma unroll
                    for (int jj = 0; jj < 2; ++jj) {
                        const int jt = 2 * jh + jj;
                        const uint2 q4r = own_quad(qrow_r, jt, tv), q4i = own_quad(qrow_i, jt, tv);
    #pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const float x_r = xr[jj][r], x_i = xi[jj][r];
                            gqR[jt][r] += rhr * x_r + rhi * x_i;
                            gqI[jt][r] += rhr * x_i - rhi * x_r;
                            const float qr = quad_elem(q4r, r), qi = quad_elem(q4i, r);
                            pr += qr * x_r + qi * x_i;
                            pi += qr * x_i - qi * x_r;
                        }
                    }
                }
                pr += __shfl_xor(pr, 16);
                pr += __shfl_xor(pr, 32);
                pi += __shfl_xor(pi, 16);
                pi += __shfl_xor(pi, 32);
                if (g == 0) {
                    const float cum = __expf(sL[m * 64 + t]) * qs;
                    sDqr[m * 64 + t] += pr * cum;
                    sDqi[m * 64 + t] += pi * cum;
                    sGq[m * 64 + t] += (pr * sRr[m * 64 + t] + pi * sRi[m * 64 + t]) * cum;
                }

        }
        __syncthreads();  // S_m is no longer read: G'_m natural into the q tile
        regs_store_bf<false>(sQr, gr[0]);
        regs_store_bf<false>(sQi, gr[1]);
        if (m + 1 < M) load_state(m + 1);
        __syncthreads();
        const float dls = sv ? __expf(fminf(sL[m * 64 + valid - 1] - sL[m * 64 + s], 0.f)) : 0.f;
        floatx4 zr[4], zi[4];
#pragma unroll
        for (int it = 0; it < 4; ++it) zr[it] = zi[it] = zero4();
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            const int k0 = 32 * kp + 8 * g;
            const bf16x8 akr = ld8(sKr + s * PB + k0), aki = ld8(sKi + s * PB + k0), nki = neg_bf(aki);
            const bf16x8 avr = to_bf(to_f(ld8(sVr + s * PB + k0)) * dls), avi = to_bf(to_f(ld8(sVi + s * PB + k0)) * dls);
            const bf16x8 navr = neg_bf(avr);
#pragma unroll
            for (int it = 0; it < 4; ++it) {
                // Z^T[i][s] = sum_j G'[i][j] k[s][j]
                const int row = (16 * it + l16) * PB + k0;
                const bf16x8 gpr = ld8(sQr + row), gpi = ld8(sQi + row);
                zr[it] = mfma_bf(gpr, akr, zr[it]);
                zr[it] = mfma_bf(gpi, nki, zr[it]);
                zi[it] = mfma_bf(gpi, akr, zi[it]);
                zi[it] = mfma_bf(gpr, aki, zi[it]);
                // dK^T[j][s] += dl[s] sum_i conj(G'[i][j]) v[s][i]   (transposed reads of G')
                const bf16x8 gtr = ld_tr(sQr, k0, k0 + 4, 16 * it), gti = ld_tr(sQi, k0, k0 + 4, 16 * it);
                gkR[it] = mfma_bf(gtr, avr, gkR[it]);
                gkR[it] = mfma_bf(gti, avi, gkR[it]);
                gkI[it] = mfma_bf(gtr, avi, gkI[it]);
                gkI[it] = mfma_bf(gti, navr, gkI[it]);
            }
        }
        // dV += dl Z; the dl gradient sum_i Re(v[s][i] conj(Z[s][i]))
        float gdl = 0.f;
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            const uint2 vr4 = *reinterpret_cast<const uint2 *>(sVr + s * PB + 16 * it + 4 * g);
            const uint2 vi4 = *reinterpret_cast<const uint2 *>(sVi + s * PB + 16 * it + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float z_r = zr[it][r], z_i = zi[it][r];
                gvR[it][r] += dls * z_r;
                gvI[it][r] += dls * z_i;
                gdl += quad_elem(vr4, r) * z_r + quad_elem(vi4, r) * z_i;
            }
        }
        gdl += __shfl_xor(gdl, 16);
        gdl += __shfl_xor(gdl, 32);
        {
            const float x = sL[m * 64 + valid - 1] - sL[m * 64 + s];
            float gp = (g == 0 && sv && s != valid - 1 && x <= 0.f) ? gdl * dls : 0.f;
            if (g == 0) sGL[m * 64 + s] -= gp;  // this lane's own key
            gp = row16_sum(gp);                 // the wave's keys (lanes 0-15), a fixed order
            if (lane == 0) sGpw[w] = gp;
        }
        __syncthreads();
        if (tid == 0) {  // the decay_last terms of every key, in wave order, on the last step
            float x = ((sGpw[0] + sGpw[1]) + sGpw[2]) + sGpw[3];
            if (carry) x += (sRed[0] + sRed[1] + sRed[2] + sRed[3]) * __expf(sL[m * 64 + valid - 1]);
            sGL[m * 64 + valid - 1] += x;
        }
    }
    __syncthreads();

    if (tv) {
        const int64_t o = b * p.dq.s0 + h * p.dq.s1 + (int64_t)(c0 + t) * p.dq.s2;
        U16 *dre = (U16 *)p.dq.re + o, *dim = (U16 *)p.dq.im + o;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            store_quad(dre, jt, gqR[jt], qs);
            store_quad(dim, jt, gqI[jt], qs);
        }
        if (g == 0 && p.drot_re) {
            for (int m = 0; m < M; ++m) {
                const int64_t ro = m * a.sr_m + b * a.sr_b + h * a.sr_h + (int64_t)(c0 + t) * a.sr_t;
                p.drot_re[ro] = sDqr[m * 64 + t];
                p.drot_im[ro] = sDqi[m * 64 + t];
            }
        }
    }
    if (sv) {
        const int64_t ok_ = b * p.dk.s0 + h * p.dk.s1 + (int64_t)(c0 + s) * p.dk.s2;
        const int64_t ov_ = b * p.dv.s0 + h * p.dv.s1 + (int64_t)(c0 + s) * p.dv.s2;
        U16 *kre = (U16 *)p.dk.re + ok_, *kim = (U16 *)p.dk.im + ok_;
        U16 *vre = (U16 *)p.dv.re + ov_, *vim = (U16 *)p.dv.im + ov_;
#pragma unroll
        for (int it = 0; it < 4; ++it) {
            store_quad(kre, it, gkR[it], 1.f);
            store_quad(kim, it, gkI[it], 1.f);
            store_quad(vre, it, gvR[it], 1.f);
            store_quad(vim, it, gvI[it], 1.f);
        }
    }
    if (w < M) {  // state w: row part + column part + state terms -> reverse cumsum -> d gamma
        const int m = w;
        float x = (lane < valid) ? sGL[m * 64 + lane] + sGq[m * 64 + lane] : 0.f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float y = __shfl_down(x, off);
            if (lane + off < 64) x += y;
        }
        if (lane < valid) {
            const int64_t go = m * a.sg_m + b * a.sg_b + h * a.sg_h + (int64_t)(c0 + lane) * a.sg_t;
            p.dgamma[go] = x / (din.gam + LOG_EPS);  // din: gamma of state w, loaded at entry
        }
    }
}

// 8 bf16 planes + 10 per-step vectors: two blocks share a CU's 160 KiB LDS up to M = 3
template <int M>
constexpr size_t chunk_grad_bf16_smem() { return (size_t)8 * PLANE_B * 2 + (10 * M * 64 + 8 + 4) * sizeof(float); }
static_assert(2 * chunk_grad_bf16_smem<3>() <= 160 * 1024, "LDS budget");

template <int M>
int launch_bwd_bf16_m(const BwdParams &p, hipStream_t stream) {
    const qpam_scan_args &a = p.a;
    dim3 grid(p.n_chunks, a.H, a.B);
    const size_t s1 = gpass_bf16_smem<M>(), s3 = chunk_grad_bf16_smem<M>();
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)grad_pass_bf16_kernel<M, false>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)s1));
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)grad_pass_bf16_kernel<M, true>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)s1));
    const void *ck = p.dy_bf16 ? (const void *)chunk_grad_bf16_kernel<M, true>
                               : (const void *)chunk_grad_bf16_kernel<M, false>;
    QPAM_CHECK_HIP(hipFuncSetAttribute(ck, hipFuncAttributeMaxDynamicSharedMemorySize, (int)s3));
    // the gradient-state pass (sequential chains) writes dS after every chunk;
    // the chunk pass then forms every gradient of the chunk
    const dim3 pg(PASS_SPLIT * a.B * a.H);
    if (p.dy_bf16) hipLaunchKernelGGL((grad_pass_bf16_kernel<M, true>), pg, dim3(GPASS_THREADS), s1, stream, p);
    else hipLaunchKernelGGL((grad_pass_bf16_kernel<M, false>), pg, dim3(GPASS_THREADS), s1, stream, p);
    int st = launch_status("grad_pass_bf16_kernel");
    if (st) return st;
    if (p.dy_bf16) hipLaunchKernelGGL((chunk_grad_bf16_kernel<M, true>), grid, dim3(THREADS), s3, stream, p);
    else hipLaunchKernelGGL((chunk_grad_bf16_kernel<M, false>), grid, dim3(THREADS), s3, stream, p);
    return launch_status("chunk_grad_bf16_kernel");
}

// The state count is a compile-time constant of the chunk-gradient kernel.
int launch_bwd_bf16(const BwdParams &p, hipStream_t stream) {
    switch (p.a.M) {
        case 1: return launch_bwd_bf16_m<1>(p, stream);
        case 2: return launch_bwd_bf16_m<2>(p, stream);
        case 3: return launch_bwd_bf16_m<3>(p, stream);
        default: return launch_bwd_bf16_m<4>(p, stream);
    }
}

template <int C>
size_t gcs_smem() { return (size_t)(4 * C * P + 3 * MAX_M * 64) * sizeof(float); }
template <int C>
size_t qside_smem() { return (size_t)(6 * C * P + 2 * D * P + 10 * MAX_M * 64) * sizeof(float); }
template <int C>
size_t kside_smem() { return (size_t)(4 * C * P + 4 * D * P + 5 * MAX_M * 64 + 4 + 64) * sizeof(float); }

template <typename Tin, int C>
int launch_bwd(const BwdParams &p, hipStream_t stream) {
    const qpam_scan_args &a = p.a;
    dim3 grid(p.n_chunks, a.H, a.B);
    const size_t s1 = gcs_smem<C>(), s3 = qside_smem<C>(), s4 = kside_smem<C>();
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)grad_chunk_state_kernel<Tin, C>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)s1));
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)query_side_kernel<Tin, C>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)s3));
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)key_side_kernel<Tin, C>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)s4));
    // gradient-state chain and query side concurrently (independent); key side after both
    int st = fork_join(
        stream,
        [&](hipStream_t s) {
            hipLaunchKernelGGL((grad_chunk_state_kernel<Tin, C>), grid, dim3(THREADS), s1, s, p);
            int r = launch_status("grad_chunk_state_kernel");
            if (r) return r;
            hipLaunchKernelGGL(grad_state_scan_kernel, dim3(a.M * a.B * a.H * SCAN_BLOCKS), dim3(THREADS), 0, s, p);
            return launch_status("grad_state_scan_kernel");
        },
        [&](hipStream_t s) {
            hipLaunchKernelGGL((query_side_kernel<Tin, C>), grid, dim3(THREADS), s3, s, p);
            return launch_status("query_side_kernel");
        });
    if (st) return st;
    hipLaunchKernelGGL((key_side_kernel<Tin, C>), grid, dim3(THREADS), s4, stream, p);
    return launch_status("key_side_kernel");
}

// fp32 increments/gradient states, the partial log-decay gradient, then (bf16
// path) the bf16 gradient-state snapshots at a 256-byte aligned offset.
// Workspace: fp32 per-chunk gradient states (fp32 path only), the fp32 per-token
// log-decay gradients, then at a 256-byte aligned offset the bf16 gradient-state
// snapshots (snapshot path only).
int64_t bwd_gl_offset(const qpam_scan_args &a) {  // in floats
    const int64_t n = (a.T + a.C - 1) / a.C;
    return uses_snapshots(a) ? 0 : (int64_t)a.M * a.B * a.H * n * 2 * D * D;
}

size_t bwd_snapshot_offset(const qpam_scan_args &a) {
    const int64_t n = (a.T + a.C - 1) / a.C;
    const int64_t chains = (int64_t)a.M * a.B * a.H;
    return ((size_t)(bwd_gl_offset(a) + chains * n * a.C) * sizeof(float) + 255) & ~(size_t)255;
}

size_t bwd_workspace_bytes(const qpam_scan_args &a) {
    const int64_t n = (a.T + a.C - 1) / a.C;
    const int64_t chains = (int64_t)a.M * a.B * a.H;
    size_t bytes = bwd_snapshot_offset(a);
    if (uses_snapshots(a)) bytes += (size_t)chains * n * 2 * D * D * sizeof(unsigned short);
    return bytes;
}

}  // namespace

int scan_bwd(const qpam_scan_bwd_args *bw, hipStream_t stream) {
    QPAM_REQUIRE(bw != nullptr && bw->fwd != nullptr, "qpam_scan_bwd: null args");
    const qpam_scan_args *a = bw->fwd;
    int st = validate_scan(a, "qpam_scan_bwd", false);
    if (st) return st;
    QPAM_REQUIRE(bw->dy.re && bw->dy.im && ((uintptr_t)bw->dy.re % 16) == 0 && ((uintptr_t)bw->dy.im % 16) == 0 &&
                     bw->dy.s0 % 4 == 0 && bw->dy.s1 % 4 == 0 && bw->dy.s2 % 4 == 0,
                 "qpam_scan_bwd: dy must be 16-byte aligned fp32 planes with strides multiple of 4");
    QPAM_REQUIRE(bw->dy_dtype == QPAM_F32 ||
                     (bw->dy_dtype == QPAM_BF16 && a->dtype == QPAM_BF16 && a->C == 64 && bw->dy.s0 % 8 == 0 &&
                      bw->dy.s1 % 8 == 0 && bw->dy.s2 % 8 == 0),
                 "qpam_scan_bwd: dy_dtype %d (bf16 dy needs bf16 inputs, chunk 64 and strides multiple of 8)",
                 bw->dy_dtype);
    QPAM_REQUIRE(bw->dq.re && bw->dq.im && bw->dk.re && bw->dk.im && bw->dv.re && bw->dv.im && bw->dgamma,
                 "qpam_scan_bwd: null output");
    QPAM_REQUIRE((bw->ds_re == nullptr) == (bw->ds_im == nullptr), "qpam_scan_bwd: ds needs both planes");
    QPAM_REQUIRE((bw->drot_re == nullptr) == (bw->drot_im == nullptr), "qpam_scan_bwd: drot needs both planes");
    QPAM_REQUIRE(bw->drot_re == nullptr || a->rot_re != nullptr, "qpam_scan_bwd: drot without rot");
    QPAM_REQUIRE((bw->ds0_re == nullptr) == (bw->ds0_im == nullptr), "qpam_scan_bwd: ds0 needs both planes");
    const uintptr_t al = (uintptr_t)bw->ds_re | (uintptr_t)bw->ds_im | (uintptr_t)bw->ds0_re | (uintptr_t)bw->ds0_im;
    QPAM_REQUIRE(al % 16 == 0, "qpam_scan_bwd: state gradients must be 16-byte aligned");
    if (uses_snapshots(*a)) {  // the bf16 chunk-64 kernels store dq/dk/dv rows in 8-byte runs
        const qpam_mview *os[3] = {&bw->dq, &bw->dk, &bw->dv};
        for (const qpam_mview *o : os)
            QPAM_REQUIRE(((uintptr_t)o->re % 8) == 0 && ((uintptr_t)o->im % 8) == 0 && o->s0 % 4 == 0 &&
                             o->s1 % 4 == 0 && o->s2 % 4 == 0,
                         "qpam_scan_bwd: bf16 dq/dk/dv planes must be 8-byte aligned with strides multiple of 4");
    }
    QPAM_REQUIRE(bw->workspace && bw->workspace_bytes >= bwd_workspace_bytes(*a) &&
                     ((uintptr_t)bw->workspace % 16) == 0,
                 "qpam_scan_bwd: workspace needs %zu bytes (got %zu)", bwd_workspace_bytes(*a),
                 bw->workspace_bytes);
    BwdParams p;
    p.a = *a;
    p.dy = bw->dy;
    p.ds_re = bw->ds_re;
    p.ds_im = bw->ds_im;
    p.dq = bw->dq;
    p.dk = bw->dk;
    p.dv = bw->dv;
    p.dgamma = bw->dgamma;
    p.drot_re = bw->drot_re;
    p.drot_im = bw->drot_im;
    p.ds0_re = bw->ds0_re;
    p.ds0_im = bw->ds0_im;
    p.n_chunks = (a->T + a->C - 1) / a->C;
    p.states = uses_snapshots(*a) ? nullptr : (const float *)a->workspace;
    p.totals = (const float *)a->workspace + fwd_totals_offset(*a);
    p.gstates = uses_snapshots(*a) ? nullptr : (float *)bw->workspace;
    p.gl = (float *)bw->workspace + bwd_gl_offset(*a);
    p.snap = nullptr;
    p.gsnap = nullptr;
    p.dy_bf16 = bw->dy_dtype == QPAM_BF16 ? 1 : 0;
    const bool bf = a->dtype == QPAM_BF16;
    if (uses_snapshots(*a)) {
        p.snap = reinterpret_cast<const unsigned short *>((const char *)a->workspace + fwd_snapshot_offset(*a));
        p.gsnap = reinterpret_cast<unsigned short *>((char *)bw->workspace + bwd_snapshot_offset(*a));
        const SegLayout l = seg_layout(*a);
        p.wgr = (const float *)a->workspace + l.wgr;
        p.wgi = (const float *)a->workspace + l.wgi;
        return launch_bwd_bf16(p, stream);
    }
    switch (a->C) {
        case 16: return bf ? launch_bwd<unsigned short, 16>(p, stream) : launch_bwd<float, 16>(p, stream);
        case 32: return bf ? launch_bwd<unsigned short, 32>(p, stream) : launch_bwd<float, 32>(p, stream);
        default: return bf ? launch_bwd<unsigned short, 64>(p, stream) : launch_bwd<float, 64>(p, stream);
    }
}

size_t scan_bwd_workspace(const qpam_scan_bwd_args *bw) {
    return (bw && bw->fwd) ? bwd_workspace_bytes(*bw->fwd) : 0;
}

}  // namespace scan
}  // namespace qpam

extern "C" size_t qpam_scan_bwd_workspace_size(const qpam_scan_bwd_args *a) {
    return qpam::scan::scan_bwd_workspace(a);
}

extern "C" int qpam_scan_bwd(const qpam_scan_bwd_args *a, void *stream) {
    return qpam::scan::scan_bwd(a, (hipStream_t)stream);
}
