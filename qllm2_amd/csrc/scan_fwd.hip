// Chunked dual-form PAM scan, forward (fp32 MFMA, d = 64).
//
// Reference semantics: V11PAMLayer._forward_chunked_head (v11/model.py:378-417)
// for M = 1 and _fused_chunk_step/_forward_multistate_fused
// (v11/model.py:657-781) for M states with rotations r_m = alpha e^{i phi}.
//
// The only sequential dependency of the scan is the d x d state carry, and the
// state rows are independent, so the forward is split into a state pass and a
// chunk-parallel output pass:
//   fp32 inputs: state_pass_f32 (sequential over chunks, MFMA, the state in
//      registers): per chain (m, b, h) the state entering every chunk -> workspace,
//      S_m <- total_m,c S_m + dS_m,c with dS_m,c = sum_s D_m[C-1,s] v_s (x) conj(k_s),
//      chunk totals, the final state;
//   bf16 inputs with 16- or 32-step chunks: chunk_state (chunk-parallel increments
//      dS_m,c -> workspace) then state_scan (the prefix over chunks, in place);
//   bf16 inputs with 64-step chunks: state_pass_bf16 (bf16 snapshots);
//   then chunk_output (chunk-parallel, MFMA): Y_c = (W . D~) V + sum_m rho_m
//      (Q~ S_in,m^T) with W = Q~ K^H, D~ = sum_m r_m D_m, rho_m = r_m cum_m.
// Decay matrices are never materialised: each lane rebuilds D[t,s] from the
// chunk's log-decay prefix sums held in LDS.  The score tile is computed
// transposed (rows s, cols t) so the MFMA accumulator layout is directly the
// A operand of the (W . D~) V product.
#include <map>
#include <mutex>

#include "scan_common.h"

namespace qpam {
namespace scan {
namespace {

struct FwdParams {
    qpam_scan_args a;
    int n_chunks;
    float *states;         // [M][B][H][n][2][64][64]
    float *totals;         // [M][B][H][n]
    unsigned short *snap;  // bf16 path: [M][B][H][n][2][64][64] bf16 entering states (else null)
    float *dlast;          // fp32 64-step path: [M][B][H][n][64] D[C-1, s] of every chunk (else null)
    // bf16 64-step path (segments of SEG chunks, else null):
    int n_segs;
    float *segs;    // [M][B][H][n_segs][2][64][64]: segment increments, then the state entering each segment
    float *segtot;  // [M][B][H][n_segs] decay total of each segment
    float *wfwd;    // [M][B][H][n*64] weight of step t in its segment's end state
    float *wbwd;    // [M][B][H][n*64] decay from its segment's start through step t
    float *wgr, *wgi;  // [M][B][H][n*64] the backward's per-step weights conj(rho_m[t]) q_scale
};

__device__ __forceinline__ float *chunk_state_ptr(const FwdParams &p, int m, int b, int h, int c) {
    const int64_t idx = (((int64_t)m * p.a.B + b) * p.a.H + h) * p.n_chunks + c;
    return p.states + idx * (2 * D * D);
}

__device__ __forceinline__ unsigned short *chunk_snap_ptr(const FwdParams &p, int m, int b, int h, int c) {
    const int64_t idx = (((int64_t)m * p.a.B + b) * p.a.H + h) * p.n_chunks + c;
    return p.snap + idx * (2 * D * D);
}

__device__ __forceinline__ float *chunk_total_ptr(const FwdParams &p, int m, int b, int h, int c) {
    return p.totals + (((int64_t)m * p.a.B + b) * p.a.H + h) * p.n_chunks + c;
}

// ---------------------------------------------------------------- kernel 1 --
template <typename Tin, int C>
__global__ void __launch_bounds__(THREADS) chunk_state_kernel(FwdParams p) {
    extern __shared__ float smem[];
    float *sKr = smem, *sKi = sKr + C * P, *sVr = sKi + C * P, *sVi = sVr + C * P;
    float *sDl = sVi + C * P;  // [MAX_M][64]

    const qpam_scan_args &a = p.a;
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int c0 = c * C;
    const int valid = min(C, a.T - c0);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;

    const int64_t ko = b * a.k.s0 + h * a.k.s1 + (int64_t)c0 * a.k.s2;
    const int64_t vo = b * a.v.s0 + h * a.v.s1 + (int64_t)c0 * a.v.s2;
    {
        float *const dst[4] = {sKr, sKi, sVr, sVi};
        const Tin *const src[4] = {(const Tin *)a.k.re + ko, (const Tin *)a.k.im + ko, (const Tin *)a.v.re + vo,
                                   (const Tin *)a.v.im + vo};
        const int64_t st[4] = {a.k.s2, a.k.s2, a.v.s2, a.v.s2};
        const float sc[4] = {1.f, 1.f, 1.f, 1.f};
        stage_tiles<Tin, C, 4>(dst, src, st, sc, valid);
    }
    if (w == 0) {
        for (int m = 0; m < a.M; ++m) {
            const float *gp = a.gamma + m * a.sg_m + b * a.sg_b + h * a.sg_h + (int64_t)c0 * a.sg_t;
            const float L = chunk_log_prefix(gp, a.sg_t, valid, lane);
            const float Llast = __shfl(L, valid - 1);
            sDl[m * 64 + lane] = (lane < valid) ? __expf(fminf(Llast - L, 0.f)) : 0.f;
            if (lane == 0) *chunk_total_ptr(p, m, b, h, c) = __expf(Llast);
        }
    }
    __syncthreads();

    // wave w owns value rows i in [16w, 16w+16); all 64 key columns j.
    // dS = sum_s dl_s v_s conj(k_s) with three MFMAs per complex product:
    // re = T1 + T2, im = T3 - T1 + T2, T1 = vr kr, T2 = vi ki, T3 = (vr + vi)(kr - ki)
    for (int m = 0; m < a.M; ++m) {
        floatx4 t1[4], t2[4], t3[4];
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) t1[jt] = t2[jt] = t3[jt] = zero4();
#pragma unroll 4
        for (int ks = 0; ks < C / 4; ++ks) {
            const int s = 4 * ks + g;
            const float dl = sDl[m * 64 + s];
            const float vr = sVr[s * P + 16 * w + l16] * dl;
            const float vi = sVi[s * P + 16 * w + l16] * dl;
            const float vs = vr + vi;
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                const float kr = sKr[s * P + 16 * jt + l16];
                const float ki = sKi[s * P + 16 * jt + l16];
                t1[jt] = mfma4(vr, kr, t1[jt]);
                t2[jt] = mfma4(vi, ki, t2[jt]);
                t3[jt] = mfma4(vs, kr - ki, t3[jt]);
            }
        }
        float *dst = chunk_state_ptr(p, m, b, h, c);
#pragma unroll
        for (int jt = 0; jt < 4; ++jt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = 16 * w + 4 * g + r, j = 16 * jt + l16;
                dst[i * D + j] = t1[jt][r] + t2[jt][r];
                dst[D * D + i * D + j] = t3[jt][r] - t1[jt][r] + t2[jt][r];
            }
    }
}

// ---------------------------------------------------------------- kernel 2 --
// Each thread owns SCAN_EPT float4 of one (m, b, h) state (2048 float4: re
// plane then im plane), SCAN_BLOCKS blocks per state, and keeps the increments
// of the next two chunks in flight.  The running state stays fp32; the entering
// state of every chunk goes either back over the increment (fp32 path) or,
// rounded once, into the bf16 snapshot (bf16 path).
__global__ void __launch_bounds__(THREADS) state_scan_kernel(FwdParams p) {
    const qpam_scan_args &a = p.a;
    const int chain = blockIdx.x / SCAN_BLOCKS;
    const int bh = chain % (a.B * a.H), m = chain / (a.B * a.H);
    const int b = bh / a.H, h = bh % a.H;
    const int64_t cs = 2 * D * D;  // floats per chunk state
    float *base = chunk_state_ptr(p, m, b, h, 0);
    unsigned short *sbase = p.snap ? chunk_snap_ptr(p, m, b, h, 0) : nullptr;
    const float *tot = chunk_total_ptr(p, m, b, h, 0);
    const int n = p.n_chunks;

    int off[SCAN_EPT];  // float offset inside the [2][64][64] state
    float4 S[SCAN_EPT], b0[SCAN_EPT], b1[SCAN_EPT];
#pragma unroll
    for (int e = 0; e < SCAN_EPT; ++e) {
        off[e] = 4 * ((blockIdx.x % SCAN_BLOCKS) * THREADS * SCAN_EPT + e * THREADS + threadIdx.x);
        const int plane = off[e] >= D * D;
        S[e] = make_float4(0.f, 0.f, 0.f, 0.f);
        if (a.s0_re)
            S[e] = *reinterpret_cast<const float4 *>((plane ? a.s0_im : a.s0_re) + (int64_t)chain * D * D +
                                                     off[e] - plane * D * D);
        b0[e] = *reinterpret_cast<const float4 *>(base + off[e]);
        if (n > 1) b1[e] = *reinterpret_cast<const float4 *>(base + cs + off[e]);
    }
    for (int c = 0; c < n; ++c) {
        const float t = tot[c];
#pragma unroll
        for (int e = 0; e < SCAN_EPT; ++e) {
            const float4 ds = b0[e];
            b0[e] = b1[e];
            if (c + 2 < n) b1[e] = *reinterpret_cast<const float4 *>(base + (c + 2) * cs + off[e]);
            if (sbase) *reinterpret_cast<ushortx4 *>(sbase + c * cs + off[e]) = to_bf16x4(S[e]);
            else *reinterpret_cast<float4 *>(base + c * cs + off[e]) = S[e];
            S[e].x = t * S[e].x + ds.x;
            S[e].y = t * S[e].y + ds.y;
            S[e].z = t * S[e].z + ds.z;
            S[e].w = t * S[e].w + ds.w;
        }
    }
    if (a.s_re) {
#pragma unroll
        for (int e = 0; e < SCAN_EPT; ++e) {
            const int plane = off[e] >= D * D;
            *reinterpret_cast<float4 *>((plane ? a.s_im : a.s_re) + (int64_t)chain * D * D + off[e] - plane * D * D) =
                S[e];
        }
    }
}

// ---------------------------------------------------------------- kernel 3 --
// fp32 inputs.  Complex products take three real MFMAs (Gauss):
//   a b       = (T1 - T2) + i (T3 - T1 - T2),  T1 = ar br, T2 = ai bi, T3 = (ar + ai)(br + bi)
//   conj(a) b = (T1 + T2) + i (T3 - T1 + T2),  T3 = (ar - ai)(br + bi)
// LDS holds Q and one 64-row tile that is K, then V, then each carried state
// (about 72 KiB, two blocks per CU); V and the next state wait in registers.
template <int C>
__global__ void __launch_bounds__(THREADS) chunk_output_f32_kernel(FwdParams p) {
    extern __shared__ float smem[];
    float *sQr = smem, *sQi = sQr + C * P;
    float *sXr = sQi + C * P, *sXi = sXr + D * P;  // K tile, then V, then S_m
    float *sL = sXi + D * P;                        // [MAX_M][64] log-decay prefix
    float *sRr = sL + MAX_M * 64, *sRi = sRr + MAX_M * 64;

    const qpam_scan_args &a = p.a;
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int c0 = c * C;
    const int valid = min(C, a.T - c0);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const bool general = (a.M > 1) || (a.rot_re != nullptr);
    const bool carry = (c > 0) || (a.s0_re != nullptr);

    const int64_t qo = b * a.q.s0 + h * a.q.s1 + (int64_t)c0 * a.q.s2;
    const int64_t ko = b * a.k.s0 + h * a.k.s1 + (int64_t)c0 * a.k.s2;
    const int64_t vo = b * a.v.s0 + h * a.v.s1 + (int64_t)c0 * a.v.s2;
    F32Tile<C> vrt, vit;
    {
        F32Tile<C> t4[4];
        tile_load<C>(t4[0], (const float *)a.q.re + qo, a.q.s2, valid);
        tile_load<C>(t4[1], (const float *)a.q.im + qo, a.q.s2, valid);
        tile_load<C>(t4[2], (const float *)a.k.re + ko, a.k.s2, valid);
        tile_load<C>(t4[3], (const float *)a.k.im + ko, a.k.s2, valid);
        tile_load<C>(vrt, (const float *)a.v.re + vo, a.v.s2, valid);
        tile_load<C>(vit, (const float *)a.v.im + vo, a.v.s2, valid);
        tile_store<C>(sQr, t4[0], a.q_scale);
        tile_store<C>(sQi, t4[1], a.q_scale);
        tile_store<C>(sXr, t4[2], 1.f);
        tile_store<C>(sXi, t4[3], 1.f);
    }
    if (w == 0) {
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
    __syncthreads();

    const int tt = causal_tile(w);  // query rows t in [16tt, 16tt+16)
    const bool active = tt < C / 16;
    const int t = 16 * tt + l16;
    floatx4 wr[4], wi[4];  // A = W . D~ per s-tile; lane holds s = 16st+4g+r, t
    if (active) {
        // ---- transposed score tiles W^T[s][t] = sum_j conj(K[s,j]) Q~[t,j], s-tiles st <= tt
        floatx4 s1[4], s2[4], s3[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) s1[st] = s2[st] = s3[st] = zero4();
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            const float4 qr = *reinterpret_cast<const float4 *>(sQr + t * P + 16 * q4 + 4 * g);
            const float4 qi = *reinterpret_cast<const float4 *>(sQi + t * P + 16 * q4 + 4 * g);
            const float4 qs4 = make_float4(qr.x + qi.x, qr.y + qi.y, qr.z + qi.z, qr.w + qi.w);
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                if (st > tt || 16 * st >= C) continue;
                const float4 kr = *reinterpret_cast<const float4 *>(sXr + (16 * st + l16) * P + 16 * q4 + 4 * g);
                const float4 ki = *reinterpret_cast<const float4 *>(sXi + (16 * st + l16) * P + 16 * q4 + 4 * g);
                const float kd[4] = {kr.x - ki.x, kr.y - ki.y, kr.z - ki.z, kr.w - ki.w};
                const float krr[4] = {kr.x, kr.y, kr.z, kr.w}, kii[4] = {ki.x, ki.y, ki.z, ki.w};
                const float qrr[4] = {qr.x, qr.y, qr.z, qr.w}, qii[4] = {qi.x, qi.y, qi.z, qi.w};
                const float qss[4] = {qs4.x, qs4.y, qs4.z, qs4.w};
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    s1[st] = mfma4(krr[kk], qrr[kk], s1[st]);
                    s2[st] = mfma4(kii[kk], qii[kk], s2[st]);
                    s3[st] = mfma4(kd[kk], qss[kk], s3[st]);
                }
            }
        }
        // ---- W = conj(K) Q~, then the (complex) decay D~[t,s]
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            if (st > tt || 16 * st >= C) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int s = 16 * st + 4 * g + r;
                const float xr = s1[st][r] + s2[st][r], xi = s3[st][r] - s1[st][r] + s2[st][r];
                float dre = 0.f, dim = 0.f;
                if (s <= t) {
                    if (!general) {
                        dre = __expf(fminf(sL[t] - sL[s], 0.f));
                    } else {
                        for (int m = 0; m < a.M; ++m) {
                            const float dm = __expf(fminf(sL[m * 64 + t] - sL[m * 64 + s], 0.f));
                            dre += sRr[m * 64 + t] * dm;
                            dim += sRi[m * 64 + t] * dm;
                        }
                    }
                }
                wr[st][r] = xr * dre - xi * dim;
                wi[st][r] = xr * dim + xi * dre;
            }
        }
    }
    // K is consumed: V takes its LDS tile; the first carried state waits in registers
    F32Tile<D> nr, ni;
    if (carry) {
        const float *src = chunk_state_ptr(p, 0, b, h, c);
        tile_load<D>(nr, src, D, D);
        tile_load<D>(ni, src + D * D, D, D);
    }
    __syncthreads();
    tile_store<C>(sXr, vrt, 1.f);
    tile_store<C>(sXi, vit, 1.f);
    __syncthreads();

    floatx4 y1[4], y2[4], y3[4];  // Y = (y1 - y2) + i (y3 - y1 - y2)
#pragma unroll
    for (int it = 0; it < 4; ++it) y1[it] = y2[it] = y3[it] = zero4();
    if (active) {
        // ---- intra-chunk read  Y += A V   (k = s, 4 k-steps per s-tile)
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            if (st > tt || 16 * st >= C) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int s = 16 * st + 4 * g + r;
                const float ar = wr[st][r], ai = wi[st][r], as = ar + ai;
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    const float vr = sXr[s * P + 16 * it + l16];
                    const float vi = sXi[s * P + 16 * it + l16];
                    y1[it] = mfma4(ar, vr, y1[it]);
                    y2[it] = mfma4(ai, vi, y2[it]);
                    y3[it] = mfma4(as, vr + vi, y3[it]);
                }
            }
        }
    }

    // ---- carried read  Y += sum_m (rho_m . Q~) S_in,m^T
    if (carry) {
        for (int m = 0; m < a.M; ++m) {
            __syncthreads();  // previous readers of sX are done
            tile_store<D>(sXr, nr, 1.f);
            tile_store<D>(sXi, ni, 1.f);
            if (m + 1 < a.M) {
                const float *src = chunk_state_ptr(p, m + 1, b, h, c);
                tile_load<D>(nr, src, D, D);
                tile_load<D>(ni, src + D * D, D, D);
            }
            __syncthreads();
            if (active) {
                const float cum = __expf(sL[m * 64 + t]);
                const float rho_r = sRr[m * 64 + t] * cum, rho_i = sRi[m * 64 + t] * cum;
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const float4 qr = *reinterpret_cast<const float4 *>(sQr + t * P + 16 * q4 + 4 * g);
                    const float4 qi = *reinterpret_cast<const float4 *>(sQi + t * P + 16 * q4 + 4 * g);
                    const float qrr[4] = {qr.x, qr.y, qr.z, qr.w}, qii[4] = {qi.x, qi.y, qi.z, qi.w};
                    float pr[4], pi[4], ps[4];
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) {
                        pr[kk] = rho_r * qrr[kk] - rho_i * qii[kk];
                        pi[kk] = rho_r * qii[kk] + rho_i * qrr[kk];
                        ps[kk] = pr[kk] + pi[kk];
                    }
#pragma unroll
                    for (int it = 0; it < 4; ++it) {
                        const float4 sr = *reinterpret_cast<const float4 *>(sXr + (16 * it + l16) * P + 16 * q4 + 4 * g);
                        const float4 si = *reinterpret_cast<const float4 *>(sXi + (16 * it + l16) * P + 16 * q4 + 4 * g);
                        const float srr[4] = {sr.x, sr.y, sr.z, sr.w}, sii[4] = {si.x, si.y, si.z, si.w};
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) {
                            y1[it] = mfma4(pr[kk], srr[kk], y1[it]);
                            y2[it] = mfma4(pi[kk], sii[kk], y2[it]);
                            y3[it] = mfma4(ps[kk], srr[kk] + sii[kk], y3[it]);
                        }
                    }
                }
            }
        }
    }

    if (active) {
        const int64_t yo = b * a.y.s0 + h * a.y.s1 + (int64_t)c0 * a.y.s2;
#pragma unroll
        for (int it = 0; it < 4; ++it)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tr = 16 * tt + 4 * g + r;
                if (tr < valid) {
                    a.y.re[yo + (int64_t)tr * a.y.s2 + 16 * it + l16] = y1[it][r] - y2[it][r];
                    a.y.im[yo + (int64_t)tr * a.y.s2 + 16 * it + l16] = y3[it][r] - y1[it][r] - y2[it][r];
                }
            }
    }
}

// ---------------------------------------------------- fp32 state pass --
// fp32 inputs: the carried state of every chain (m, b, h) walks its chunks in
// registers, one launch for what chunk_state + state_scan do in two with the
// per-chunk increments written to HBM and read back.  Block rb of a chain owns
// value rows [16 rb, 16 rb + 16) (rows of the recurrence are independent); of
// its 8 waves, wave (half, w) owns key columns [16 w, 16 w + 16) and half of
// the chunk's tokens, so the first-half wave keeps a 4 x 1 piece of S per
// plane.  Per chunk: store the entering state (accumulated transposed, a lane
// holds one row and four consecutive columns, so it leaves in 16-byte stores;
// the output kernel and the backward read it), form both halves' products for dS = sum_s D[C-1,s] v_s
// conj(k_s) on MFMA (operands straight from global memory in MFMA layout, the
// next two chunks' loads in flight), add the second half's through LDS,
// S <- total S + dS.  The pass is a dependency chain over the chunks, so its
// speed is the latency of one step: eight waves per block halve each wave's
// MFMA chain and give the SIMDs twice the waves to switch between.
// Measured alternative not kept: one launch in which each chunk's block hands
// the state to the next one through device memory (release / acquire flags)
// costs 7-9 us per hand-off alone and 16-21 us with 96 chains in flight on
// MI355X, so a 32-chunk chain took 0.89 ms against 0.31 ms for three launches.
constexpr int PASS32_SPLIT = 2;      // row blocks per chain (32 value rows each)
constexpr int PASS32_THREADS = 512;  // 8 waves: 2 row tiles x 4 column tiles of 16 x 16

// One LDS stage of the pass, one flat array (the compiler's tracking of
// direct-to-LDS loads tells whole arrays apart, so each stage is one object):
// the chunk's K tile [64 tokens][64 columns] per plane at P32_KR / P32_KI, the
// block's V slice [64 tokens][32 value rows] per plane at P32_VR / P32_VI,
// fp32, and the chunk's 64 gammas at P32_G + 64 wv (each wave loads its own copy,
// so every wave issues the same memory operations).  Rows are stored as 16-byte chunks
// XOR-swizzled so that the MFMA-layout reads (16 lanes along a row, four rows
// s = 4 ks + g) hit 64 distinct banks: K chunk c of row r at c ^ ((r & 3) << 2),
// V chunk c of row r at c ^ (((r >> 1) & 1) << 2).
constexpr int P32_KR = 0, P32_KI = 64 * 64, P32_VR = 2 * 64 * 64, P32_VI = P32_VR + 64 * 32,
              P32_DL = P32_VI + 64 * 32, P32_TOT = P32_DL + 8 * 64, P32_STAGE = P32_TOT + 8 * 64;

__device__ __forceinline__ float pass32_k(const float *plane, int s, int col) {
    return plane[s * 64 + 4 * ((col >> 2) ^ ((s & 3) << 2)) + (col & 3)];
}

__device__ __forceinline__ float pass32_v(const float *plane, int s, int col) {
    return plane[s * 32 + 4 * ((col >> 2) ^ (((s >> 1) & 1) << 2)) + (col & 3)];
}

// Direct global -> LDS loads of chunk c (tokens from c0 = 64 c) into stage `st`:
// six 1 KiB loads per wave (K: 16 rows of 64 floats per load, V: 32 rows of 32
// floats per two loads) and the wave's copies of the chunk's decay weights and
// total (`drow`, `tot`: this chain's entries of the pre-pass outputs); rows
// beyond the sequence re-read row T-1 (their decay weight is zero).
__device__ __forceinline__ void pass32_dma(float *st, const qpam_scan_args &a, const float *kre, const float *kim,
                                           const float *vre, const float *vim, const float *drow, const float *tot,
                                           int c, int i0, int wv, int lane) {
    const int last = a.T - 1, c0 = 64 * c;
    __builtin_amdgcn_global_load_lds(drow + 64 * (int64_t)c + lane, st + P32_DL + 64 * wv, 4, 0, 0);
    __builtin_amdgcn_global_load_lds(tot + c, st + P32_TOT + 64 * wv, 4, 0, 0);
#pragma unroll
    for (int q2 = 0; q2 < 2; ++q2) {
        const int q = 2 * wv + q2;                  // K load q: rows 4q .. 4q+3
        const int r = 4 * q + (lane >> 4), slot = lane & 15;
        const int c = slot ^ ((r & 3) << 2);
        const int64_t o = (int64_t)min(c0 + r, last) * a.k.s2 + 4 * c;
        __builtin_amdgcn_global_load_lds(kre + o, st + P32_KR + q * 256, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(kim + o, st + P32_KI + q * 256, 16, 0, 0);
    }
    {
        const int r = 8 * wv + (lane >> 3), slot = lane & 7;  // V load wv: rows 8wv .. 8wv+7
        const int c = slot ^ (((r >> 1) & 1) << 2);
        const int64_t o = (int64_t)min(c0 + r, last) * a.v.s2 + i0 + 4 * c;
        __builtin_amdgcn_global_load_lds(vre + o, st + P32_VR + wv * 256, 16, 0, 0);
        __builtin_amdgcn_global_load_lds(vim + o, st + P32_VI + wv * 256, 16, 0, 0);
    }
}

// The wait at the end of a step.  Every wave issues per step first the
// two 16-byte stores of the entering state (re, im), then the
// PASS32_LOADS direct loads of chunk c + 2 (pass32_dma: the decay row, the
// total, four K and two V pieces).  Waiting until at most PASS32_LOADS
// operations are outstanding retires everything issued before this step's
// loads -- in particular chunk c + 1's loads, which the next step reads --
// whether or not loads and stores complete in order relative to each other:
// loads complete in order among themselves, so an older load still in flight
// would keep all of this step's loads in flight too.
constexpr int PASS32_LOADS = 8;
constexpr int PASS32_WAIT = waitcnt_vm(PASS32_LOADS);

// Decay weights of every (chain, chunk) for the state pass, all chunks at once
// (a wave per chunk): D[C-1, s] = exp(min(L_last - L_s, 0)) (0 beyond the
// chunk) and the chunk's total decay exp(L_last), L the inclusive prefix of
// log(gamma + 1e-6).  The sequential pass then does no scan of its own.
__global__ void __launch_bounds__(THREADS) chunk_decay_f32_kernel(FwdParams p) {
    const qpam_scan_args &a = p.a;
    const int lane = threadIdx.x & 63;
    const int64_t item = (int64_t)blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6);
    const int n = p.n_chunks;
    if (item >= (int64_t)a.M * a.B * a.H * n) return;  // whole waves exit together
    const int c = (int)(item % n);
    const int64_t chain = item / n;
    const int bh = (int)(chain % (a.B * a.H)), m = (int)(chain / (a.B * a.H));
    const int b = bh / a.H, h = bh % a.H;
    const int c0 = c * 64, valid = min(64, a.T - c0);
    const float L = chunk_log_prefix(a.gamma + m * a.sg_m + b * a.sg_b + h * a.sg_h + (int64_t)c0 * a.sg_t, a.sg_t,
                                     valid, lane);
    const float Llast = __shfl(L, valid - 1);
    p.dlast[item * 64 + lane] = (lane < valid) ? __expf(fminf(Llast - L, 0.f)) : 0.f;
    if (lane == 0) p.totals[item] = __expf(Llast);
}

__device__ __forceinline__ void state_pass_f32_body(const FwdParams &p) {
    __shared__ __align__(16) float st0[P32_STAGE], st1[P32_STAGE], st2[P32_STAGE];
    const qpam_scan_args &a = p.a;
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int rt = wv >> 2, w = wv & 3;  // row tile, column tile
    const int rb = blockIdx.x % PASS32_SPLIT, chain = blockIdx.x / PASS32_SPLIT;
    const int bh = chain % (a.B * a.H), m = chain / (a.B * a.H);
    const int b = bh / a.H, h = bh % a.H;
    const int n = p.n_chunks;
    const int i0 = 32 * rb;                                  // the block's value rows
    // S accumulates transposed: this lane holds row ri, columns j0 .. j0 + 3; its MFMA
    // operands are K column j and V column 16 rt + l16
    const int ri = i0 + 16 * rt + l16, j0 = 16 * w + 4 * g, j = 16 * w + l16;
    const float *kre = (const float *)a.k.re + b * a.k.s0 + h * a.k.s1;
    const float *kim = (const float *)a.k.im + b * a.k.s0 + h * a.k.s1;
    const float *vre = (const float *)a.v.re + b * a.v.s0 + h * a.v.s1;
    const float *vim = (const float *)a.v.im + b * a.v.s0 + h * a.v.s1;
    const float *drow = p.dlast + (int64_t)chain * n * 64;   // this chain's decay weights
    const float *tot = p.totals + (int64_t)chain * n;

    floatx4 sr = zero4(), si = zero4();
    if (a.s0_re) {
        const int64_t o = (int64_t)chain * D * D + ri * D + j0;
        sr = *reinterpret_cast<const floatx4 *>(a.s0_re + o);
        si = *reinterpret_cast<const floatx4 *>(a.s0_im + o);
    }
    pass32_dma(st0, a, kre, kim, vre, vim, drow, tot, 0, i0, wv, lane);
    pass32_dma(st1, a, kre, kim, vre, vim, drow, tot, min(1, n - 1), i0, wv, lane);
    // chunk 0's loads are the oldest: wait for them (chunk 1's eight may still run)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(8));
    __builtin_amdgcn_s_barrier();

    // one chunk: store S_in(c), stream chunk c+2 into NXT, dS from CUR, S <- total S + dS
    // (the stages rotate through three unrolled steps)
#define QPAM_PASS32_STEP(CUR, NXT)                                                                     \
    {                                                                                                  \
        float *dst = chunk_state_ptr(p, m, b, h, c);                                                   \
        *reinterpret_cast<floatx4 *>(dst + ri * D + j0) = sr;                                          \
        *reinterpret_cast<floatx4 *>(dst + D * D + ri * D + j0) = si;                                  \
        __builtin_amdgcn_sched_barrier(0);                                                             \
        pass32_dma(NXT, a, kre, kim, vre, vim, drow, tot, min(c + 2, n - 1), i0, wv, lane);            \
        __builtin_amdgcn_sched_barrier(0);                                                             \
        float d_[16], vr_[16], vi_[16], kr_[16], ki_[16];                                              \
        _Pragma("unroll") for (int ks = 0; ks < 16; ++ks) {                                            \
            const int s_ = 4 * ks + g;                                                                 \
            d_[ks] = CUR[P32_DL + 64 * wv + s_];                                                       \
            vr_[ks] = pass32_v(CUR + P32_VR, s_, 16 * rt + l16);                                       \
            vi_[ks] = pass32_v(CUR + P32_VI, s_, 16 * rt + l16);                                       \
            kr_[ks] = pass32_k(CUR + P32_KR, s_, j);                                                   \
            ki_[ks] = pass32_k(CUR + P32_KI, s_, j);                                                   \
        }                                                                                              \
        const float tc = CUR[P32_TOT + 64 * wv + lane];                                                \
        floatx4 u1 = zero4(), u2 = zero4(), u3 = zero4();                                              \
        _Pragma("unroll") for (int ks = 0; ks < 16; ++ks) {                                            \
            const float vr = vr_[ks] * d_[ks], vi = vi_[ks] * d_[ks];                                  \
            u1 = mfma4(kr_[ks], vr, u1);                                                               \
            u2 = mfma4(ki_[ks], vi, u2);                                                               \
            u3 = mfma4(kr_[ks] - ki_[ks], vr + vi, u3);                                                \
        }                                                                                              \
        sr = tc * sr + (u1 + u2);                                                                      \
        si = tc * si + (u3 - u1 + u2);                                                                 \
        __builtin_amdgcn_s_waitcnt(PASS32_WAIT);                                                       \
        __builtin_amdgcn_s_barrier();                                                                  \
        ++c;                                                                                           \
    }
    int c = 0;
    while (c + 3 <= n) {
        QPAM_PASS32_STEP(st0, st2)
        QPAM_PASS32_STEP(st1, st0)
        QPAM_PASS32_STEP(st2, st1)
    }
    if (c < n) QPAM_PASS32_STEP(st0, st2)
    if (c < n) QPAM_PASS32_STEP(st1, st0)
#undef QPAM_PASS32_STEP
    // drain the direct loads still in flight before the wave ends
    __builtin_amdgcn_s_waitcnt(waitcnt_vm(0));
    if (a.s_re) {
        const int64_t o = (int64_t)chain * D * D + ri * D + j0;
        *reinterpret_cast<floatx4 *>(a.s_re + o) = sr;
        *reinterpret_cast<floatx4 *>(a.s_im + o) = si;
    }
}

__global__ void __launch_bounds__(PASS32_THREADS) state_pass_f32_kernel(FwdParams p) { state_pass_f32_body(p); }

// Generic form (fp32 LDS tiles; used for bf16 inputs with 16- or 32-step chunks).
template <typename Tin, int C>
__global__ void __launch_bounds__(THREADS) chunk_output_kernel(FwdParams p) {
    extern __shared__ float smem[];
    float *sQr = smem, *sQi = sQr + C * P;
    float *sKr = sQi + C * P, *sKi = sKr + D * P;  // K tile, later the carried state S_m
    float *sVr = sKi + D * P, *sVi = sVr + C * P;
    float *sL = sVi + C * P;         // [MAX_M][64] log-decay prefix
    float *sRr = sL + MAX_M * 64;    // [MAX_M][64] rotation
    float *sRi = sRr + MAX_M * 64;

    const qpam_scan_args &a = p.a;
    const int c = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int c0 = c * C;
    const int valid = min(C, a.T - c0);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const bool general = (a.M > 1) || (a.rot_re != nullptr);
    const bool carry = (c > 0) || (a.s0_re != nullptr);

    const int64_t qo = b * a.q.s0 + h * a.q.s1 + (int64_t)c0 * a.q.s2;
    const int64_t ko = b * a.k.s0 + h * a.k.s1 + (int64_t)c0 * a.k.s2;
    const int64_t vo = b * a.v.s0 + h * a.v.s1 + (int64_t)c0 * a.v.s2;
    {
        float *const dst[6] = {sQr, sQi, sKr, sKi, sVr, sVi};
        const Tin *const src[6] = {(const Tin *)a.q.re + qo, (const Tin *)a.q.im + qo, (const Tin *)a.k.re + ko,
                                   (const Tin *)a.k.im + ko, (const Tin *)a.v.re + vo, (const Tin *)a.v.im + vo};
        const int64_t st[6] = {a.q.s2, a.q.s2, a.k.s2, a.k.s2, a.v.s2, a.v.s2};
        const float sc[6] = {a.q_scale, a.q_scale, 1.f, 1.f, 1.f, 1.f};
        stage_tiles<Tin, C, 6>(dst, src, st, sc, valid);
    }
    if (w == 0) {
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
    __syncthreads();

    const int tt = causal_tile(w);  // query rows t in [16tt, 16tt+16)
    const bool active = tt < C / 16;
    floatx4 yR[4], yI[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) yR[it] = yI[it] = zero4();

    if (active) {
        // ---- transposed score tiles W^T[s][t] for s-tiles st <= tt (causal)
        floatx4 wr[4], wi[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) wr[st] = wi[st] = zero4();
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
            // k-steps 4q4..4q4+3 use key/query columns j = 16 q4 + 4 g + kk
            const float4 bq_r = *reinterpret_cast<const float4 *>(sQr + (16 * tt + l16) * P + 16 * q4 + 4 * g);
            const float4 bq_i = *reinterpret_cast<const float4 *>(sQi + (16 * tt + l16) * P + 16 * q4 + 4 * g);
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                if (st > tt || 16 * st >= C) continue;
                const float4 ak_r = *reinterpret_cast<const float4 *>(sKr + (16 * st + l16) * P + 16 * q4 + 4 * g);
                const float4 ak_i = *reinterpret_cast<const float4 *>(sKi + (16 * st + l16) * P + 16 * q4 + 4 * g);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) {
                    wr[st] = mfma4(ak_r[kk], bq_r[kk], wr[st]);
                    wr[st] = mfma4(ak_i[kk], bq_i[kk], wr[st]);
                    wi[st] = mfma4(ak_r[kk], bq_i[kk], wi[st]);
                    wi[st] = mfma4(-ak_i[kk], bq_r[kk], wi[st]);
                }
            }
        }
        // ---- apply the (complex) decay D~[t,s]; lane holds s = 16st+4g+r, t = 16tt+l16
        const int t = 16 * tt + l16;
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            if (st > tt || 16 * st >= C) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int s = 16 * st + 4 * g + r;
                float dre = 0.f, dim = 0.f;
                if (s <= t) {
                    if (!general) {
                        dre = __expf(fminf(sL[t] - sL[s], 0.f));
                    } else {
                        for (int m = 0; m < a.M; ++m) {
                            const float dm = __expf(fminf(sL[m * 64 + t] - sL[m * 64 + s], 0.f));
                            dre += sRr[m * 64 + t] * dm;
                            dim += sRi[m * 64 + t] * dm;
                        }
                    }
                }
                const float xr = wr[st][r], xi = wi[st][r];
                wr[st][r] = xr * dre - xi * dim;
                wi[st][r] = xr * dim + xi * dre;
            }
        }
        // ---- intra-chunk read  Y += (W . D~) V   (k = s, 4 k-steps per s-tile)
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            if (st > tt || 16 * st >= C) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int s = 16 * st + 4 * g + r;
                const float ar = wr[st][r], ai = wi[st][r];
#pragma unroll
                for (int it = 0; it < 4; ++it) {
                    const float vr = sVr[s * P + 16 * it + l16];
                    const float vi = sVi[s * P + 16 * it + l16];
                    yR[it] = mfma4(ar, vr, yR[it]);
                    yR[it] = mfma4(-ai, vi, yR[it]);
                    yI[it] = mfma4(ar, vi, yI[it]);
                    yI[it] = mfma4(ai, vr, yI[it]);
                }
            }
        }
    }

    // ---- carried read  Y += sum_m (rho_m . Q~) S_in,m^T
    if (carry) {
        for (int m = 0; m < a.M; ++m) {
            __syncthreads();  // previous users of sK* are done
            const float *src = chunk_state_ptr(p, m, b, h, c);
            {
                F32Tile<D> sr, si;
                tile_load<D>(sr, src, D, D);
                tile_load<D>(si, src + D * D, D, D);
                tile_store<D>(sKr, sr, 1.f);
                tile_store<D>(sKi, si, 1.f);
            }
            __syncthreads();
            if (active) {
                const int t = 16 * tt + l16;
                const float cum = __expf(sL[m * 64 + t]);
                const float rho_r = sRr[m * 64 + t] * cum, rho_i = sRi[m * 64 + t] * cum;
#pragma unroll
                for (int q4 = 0; q4 < 4; ++q4) {
                    const float4 qr = *reinterpret_cast<const float4 *>(sQr + t * P + 16 * q4 + 4 * g);
                    const float4 qi = *reinterpret_cast<const float4 *>(sQi + t * P + 16 * q4 + 4 * g);
#pragma unroll
                    for (int it = 0; it < 4; ++it) {
                        const float4 sr = *reinterpret_cast<const float4 *>(sKr + (16 * it + l16) * P + 16 * q4 + 4 * g);
                        const float4 si = *reinterpret_cast<const float4 *>(sKi + (16 * it + l16) * P + 16 * q4 + 4 * g);
#pragma unroll
                        for (int kk = 0; kk < 4; ++kk) {
                            const float pr = rho_r * qr[kk] - rho_i * qi[kk];
                            const float pi = rho_r * qi[kk] + rho_i * qr[kk];
                            yR[it] = mfma4(pr, sr[kk], yR[it]);
                            yR[it] = mfma4(-pi, si[kk], yR[it]);
                            yI[it] = mfma4(pr, si[kk], yI[it]);
                            yI[it] = mfma4(pi, sr[kk], yI[it]);
                        }
                    }
                }
            }
        }
    }

    if (active) {
        const int64_t yo = b * a.y.s0 + h * a.y.s1 + (int64_t)c0 * a.y.s2;
#pragma unroll
        for (int it = 0; it < 4; ++it)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * tt + 4 * g + r;
                if (t < valid) {
                    a.y.re[yo + (int64_t)t * a.y.s2 + 16 * it + l16] = yR[it][r];
                    a.y.im[yo + (int64_t)t * a.y.s2 + 16 * it + l16] = yI[it][r];
                }
            }
    }
}

// ------------------------------------------------------ bf16 MFMA path ----
// bf16 q/k/v with C = 64 on v_mfma_f32_16x16x32_bf16 with bf16 LDS tiles and
// fp32 accumulation; q is staged unscaled and q_scale is applied to the fp32
// results it enters.
//
// The chunks of a chain are grouped in segments of SEG chunks, so the only
// sequential work is an elementwise scan over the segments:
//   seg_decay (a wave per chunk): log-decay prefix of the chunk, chunk totals,
//      segment totals and two per-step weights: wfwd[t], the weight of step t's
//      write in its segment's end state (D[C-1, t] of its chunk times the totals
//      of the segment's later chunks), and wbwd[t], the decay from the segment's
//      start through t (used by the backward);
//   seg_state (a block per (b, h, segment), all M states): the segment's
//      increment dS_m = sum_t wfwd_m[t] v_t (x) conj(k_t) on MFMA;
//   seg_scan (elementwise): S entering segment g+1 = total_g S_g + dS_g, in place
//      over the increments, and the final state;
//   seg_output (a block per (b, h, segment)): walks the segment's chunks with
//      the carried states S_m in registers (fp32): Y_c = (W . D~) V + sum_m rho_m
//      (Q~ S_m^T) with the bf16 copy of S_m in LDS, the bf16 snapshot of S_m for
//      the backward, and S_m <- total_m S_m + sum_s D_m[C-1,s] v_s (x) conj(k_s)
//      before the next chunk.
// A chain's chunk totals multiply in the same order as a chunk-by-chunk pass
// only up to fp32 rounding: the segment weights are exponentials of sums of
// log-decays rather than products of per-chunk exponentials.

// One wave per chunk: wave q of block (chain, g) takes chunk SEG g + q.
__global__ void __launch_bounds__(THREADS) seg_decay_kernel(FwdParams p) {
    static_assert(SEG * 64 == THREADS, "a wave per chunk of the segment");
    __shared__ float s_last[SEG];
    const qpam_scan_args &a = p.a;
    const int64_t chain = blockIdx.x / p.n_segs;
    const int sg = blockIdx.x % p.n_segs;
    const int bh = (int)(chain % (a.B * a.H)), m = (int)(chain / (a.B * a.H));
    const int b = bh / a.H, h = bh % a.H;
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = sg * SEG + w;
    const bool live = c < p.n_chunks;
    float L = 0.f, Llast = 0.f;
    int valid = 0;
    if (live) {
        valid = min(64, a.T - c * 64);
        const float *gp = a.gamma + m * a.sg_m + b * a.sg_b + h * a.sg_h + (int64_t)c * 64 * a.sg_t;
        L = chunk_log_prefix(gp, a.sg_t, valid, lane);
        Llast = __shfl(L, valid - 1);
    }
    if (lane == 0) s_last[w] = Llast;  // 0 past the end of the sequence
    __syncthreads();
    float before = 0.f, after = 0.f, total = 0.f;
#pragma unroll
    for (int q = 0; q < SEG; ++q) {
        const float x = s_last[q];
        total += x;
        before += q < w ? x : 0.f;
        after += q > w ? x : 0.f;
    }
    if (live) {
        const int64_t o = chain * p.n_chunks * 64 + (int64_t)c * 64 + lane;
        p.wfwd[o] = lane < valid ? __expf(fminf(Llast - L, 0.f) + after) : 0.f;
        p.wbwd[o] = lane < valid ? __expf(L + before) : 0.f;
        // the backward's weight of step t: conj(r_m[t]) e^{L_t} q_scale (L within the chunk)
        const float cum = lane < valid ? __expf(L) * a.q_scale : 0.f;
        float rr = 1.f, ri = 0.f;
        if (a.rot_re && lane < valid) {
            const int64_t ro = m * a.sr_m + b * a.sr_b + h * a.sr_h + (int64_t)(c * 64 + lane) * a.sr_t;
            rr = a.rot_re[ro];
            ri = a.rot_im[ro];
        }
        p.wgr[o] = rr * cum;
        p.wgi[o] = -ri * cum;
        if (lane == 0) *chunk_total_ptr(p, m, b, h, c) = __expf(Llast);
    }
    if (threadIdx.x == 0) p.segtot[chain * p.n_segs + sg] = __expf(total);
}

__device__ __forceinline__ int64_t seg_chain(const qpam_scan_args &a, int m, int b, int h) {
    return ((int64_t)m * a.B + b) * a.H + h;
}

// Segment increments.  Wave w owns value-row tile it = w & 3 and key-column tiles
// 2 jh, 2 jh + 1 (jh = w >> 2) of every state's increment.  Per chunk: K in LDS
// as loaded, V once per state with row t scaled by wfwd_m[t] (fp32 product,
// rounded once); the next chunk's tiles and weights are in flight meanwhile.
template <int M>
constexpr size_t seg_state_smem() { return (size_t)(2 + 2 * M) * PLANE_B * 2; }

template <int M>
__global__ void __launch_bounds__(SEG_THREADS) seg_state_kernel(FwdParams p) {
    constexpr int NT = SEG_THREADS;
    extern __shared__ float smem[];
    using U = unsigned short;
    U *sK = reinterpret_cast<U *>(smem);  // [plane][64][PB]
    U *sV = sK + 2 * PLANE_B;             // [m][plane][64][PB]
    const qpam_scan_args &a = p.a;
    const int sg = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int it = w & 3, jh = w >> 2;
    const int c_begin = sg * SEG, c_end = min(c_begin + SEG, p.n_chunks);
    const U *kre = (const U *)a.k.re + b * a.k.s0 + h * a.k.s1, *kim = (const U *)a.k.im + b * a.k.s0 + h * a.k.s1;
    const U *vre = (const U *)a.v.re + b * a.v.s0 + h * a.v.s1, *vim = (const U *)a.v.im + b * a.v.s0 + h * a.v.s1;

    struct ChunkRegs {
        BfTileRegs<NT> kr, ki, vr, vi;
        float wm[M];
    };
    auto load_chunk = [&](int c, ChunkRegs &x) {
        const int c0 = c * 64, valid = min(64, a.T - c0);
        tile_load_bf<NT>(x.kr, kre + (int64_t)c0 * a.k.s2, a.k.s2, valid);
        tile_load_bf<NT>(x.ki, kim + (int64_t)c0 * a.k.s2, a.k.s2, valid);
        tile_load_bf<NT>(x.vr, vre + (int64_t)c0 * a.v.s2, a.v.s2, valid);
        tile_load_bf<NT>(x.vi, vim + (int64_t)c0 * a.v.s2, a.v.s2, valid);
#pragma unroll
        for (int m = 0; m < M; ++m) x.wm[m] = p.wfwd[seg_chain(a, m, b, h) * p.n_chunks * 64 + c0 + lane];
    };
    auto stage_chunk = [&](const ChunkRegs &x) {
        tile_store_bf<NT>(sK, x.kr);
        tile_store_bf<NT>(sK + PLANE_B, x.ki);
#pragma unroll
        for (int m = 0; m < M; ++m) {
            tile_store_bf_rowscaled<NT>(sV + 2 * m * PLANE_B, x.vr, x.wm[m]);
            tile_store_bf_rowscaled<NT>(sV + (2 * m + 1) * PLANE_B, x.vi, x.wm[m]);
        }
    };

    floatx4 accR[M][2], accI[M][2];
#pragma unroll
    for (int m = 0; m < M; ++m)
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) accR[m][jj] = accI[m][jj] = zero4();
    ChunkRegs cr;
    load_chunk(c_begin, cr);
    for (int c = c_begin; c < c_end; ++c) {
        __syncthreads();
        stage_chunk(cr);
        __syncthreads();
        if (c + 1 < c_end) load_chunk(c + 1, cr);
        // dS_m[i][j] += sum_s (w_m V)[s,i] conj(K[s,j]), accumulated transposed (A = K, B = weighted V; k = s)
#pragma unroll
        for (int kp = 0; kp < 2; ++kp) {
            const int s0 = 32 * kp + 8 * g;
            bf16x8 kr[2], ki[2];
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                kr[jj] = ld_tr(sK, s0, s0 + 4, 16 * (2 * jh + jj));
                ki[jj] = ld_tr(sK + PLANE_B, s0, s0 + 4, 16 * (2 * jh + jj));
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const bf16x8 ar = ld_tr(sV + 2 * m * PLANE_B, s0, s0 + 4, 16 * it);
                const bf16x8 ai = ld_tr(sV + (2 * m + 1) * PLANE_B, s0, s0 + 4, 16 * it);
                const bf16x8 nar = neg_bf(ar);
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {  // transposed: lane holds row i = 16 it + l16, columns 4g + r
                    accR[m][jj] = mfma_bf(kr[jj], ar, accR[m][jj]);
                    accR[m][jj] = mfma_bf(ki[jj], ai, accR[m][jj]);
                    accI[m][jj] = mfma_bf(kr[jj], ai, accI[m][jj]);
                    accI[m][jj] = mfma_bf(ki[jj], nar, accI[m][jj]);
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < M; ++m) {
        float *dst = p.segs + (seg_chain(a, m, b, h) * p.n_segs + sg) * (2 * D * D);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int o = (16 * it + l16) * D + 16 * (2 * jh + jj) + 4 * g;
            *reinterpret_cast<floatx4 *>(dst + o) = accR[m][jj];
            *reinterpret_cast<floatx4 *>(dst + D * D + o) = accI[m][jj];
        }
    }
}

// Elementwise scan over the segments of every chain, in place: the increment of
// segment g is replaced by the state entering it (s0, or zero, for g = 0); the
// state after the last segment is the final state.  A thread per float4 of a
// chain's two 64 x 64 planes; a batch of segments' loads in flight at once.
constexpr int SEG_SCAN_BATCH = 8;
__global__ void __launch_bounds__(THREADS) seg_scan_fwd_kernel(FwdParams p) {
    const qpam_scan_args &a = p.a;
    const int64_t chain = blockIdx.x >> 3;
    const int e = ((blockIdx.x & 7) << 8) + threadIdx.x;  // float4 index in [2][64][64]
    const int plane = e >> 10, off = (e & 1023) * 4;
    float4 *buf = reinterpret_cast<float4 *>(p.segs + chain * p.n_segs * (2 * D * D)) + e;
    const float *tot = p.segtot + chain * p.n_segs;
    float4 S = make_float4(0.f, 0.f, 0.f, 0.f);
    if (a.s0_re) S = *reinterpret_cast<const float4 *>((plane ? a.s0_im : a.s0_re) + chain * D * D + off);
    for (int g0 = 0; g0 < p.n_segs; g0 += SEG_SCAN_BATCH) {
        const int nb = min(SEG_SCAN_BATCH, p.n_segs - g0);
        float4 d[SEG_SCAN_BATCH];
#pragma unroll
        for (int i = 0; i < SEG_SCAN_BATCH; ++i)
            if (i < nb) d[i] = buf[(int64_t)(g0 + i) * (2 * D * D / 4)];
#pragma unroll
        for (int i = 0; i < SEG_SCAN_BATCH; ++i) {
            if (i < nb) {
                buf[(int64_t)(g0 + i) * (2 * D * D / 4)] = S;
                const float t = tot[g0 + i];
                S = make_float4(t * S.x + d[i].x, t * S.y + d[i].y, t * S.z + d[i].z, t * S.w + d[i].w);
            }
        }
    }
    if (a.s_re) *reinterpret_cast<float4 *>((plane ? a.s_im : a.s_re) + chain * D * D + off) = S;
}

// Output pass over one segment.  Wave roles (w = 0..7; waves w and w + 4 share a
// SIMD):
//   output: query tile tt = w (w < 4) or 7 - w, value tiles 2 ih, 2 ih + 1
//     (ih = w >> 2): the causal score tiles of tt (both waves of a tt form them),
//     so each SIMD holds one light and one heavy query tile;
//   state: value-row tile iu = w & 3 and key-column tiles 2 jh, 2 jh + 1 of every
//     carried state S_m.
// LDS: Q, K, V tiles of the chunk, the bf16 copy of each S_m, the per-step decay
// vectors of each state.  The next chunk's tiles, gamma and rotation are loaded
// into registers while the chunk is processed.
template <int M>
constexpr size_t seg_output_smem() {
    return (size_t)(6 + 2 * M) * PLANE_B * 2 + (7 * M * 64 + 2 * MAX_M) * sizeof(float);
}

template <int M>
__global__ void __launch_bounds__(SEG_THREADS) seg_output_kernel(FwdParams p) {
    constexpr int NT = SEG_THREADS;
    extern __shared__ float smem[];
    using U = unsigned short;
    U *sQr = reinterpret_cast<U *>(smem), *sQi = sQr + PLANE_B;
    U *sKr = sQi + PLANE_B, *sKi = sKr + PLANE_B;
    U *sVr = sKi + PLANE_B, *sVi = sVr + PLANE_B;
    U *sS = sVi + PLANE_B;  // [m][plane][64][PB] bf16 state entering the chunk
    float *sL = reinterpret_cast<float *>(sS + 2 * M * PLANE_B);  // per-step vectors [M][64]
    float *sRr = sL + M * 64, *sRi = sRr + M * 64, *sF = sRi + M * 64, *sDl = sF + M * 64;
    float *sPr = sDl + M * 64, *sPi = sPr + M * 64;           // rho_m q_scale
    float *sTot = sPi + M * 64;                               // [MAX_M]
    int *sFast = reinterpret_cast<int *>(sTot + MAX_M);       // [MAX_M]

    const qpam_scan_args &a = p.a;
    const int sg = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int c_begin = sg * SEG, c_end = min(c_begin + SEG, p.n_chunks);
    const bool general = (M > 1) || (a.rot_re != nullptr);
    const float qs = a.q_scale;
    const int tt = w < 4 ? w : 7 - w, ih = w >> 2;
    const int iu = w & 3, jh = w >> 2;
    const int64_t qb = b * a.q.s0 + h * a.q.s1, kb = b * a.k.s0 + h * a.k.s1, vb = b * a.v.s0 + h * a.v.s1;

    struct ChunkRegs {
        BfTileRegs<NT> qr, qi, kr, ki, vr, vi;
        float gam, rr, ri;
    };
    auto load_chunk = [&](int c, ChunkRegs &x) {
        const int c0 = c * 64, valid = min(64, a.T - c0);
        tile_load_bf<NT>(x.qr, (const U *)a.q.re + qb + (int64_t)c0 * a.q.s2, a.q.s2, valid);
        tile_load_bf<NT>(x.qi, (const U *)a.q.im + qb + (int64_t)c0 * a.q.s2, a.q.s2, valid);
        tile_load_bf<NT>(x.kr, (const U *)a.k.re + kb + (int64_t)c0 * a.k.s2, a.k.s2, valid);
        tile_load_bf<NT>(x.ki, (const U *)a.k.im + kb + (int64_t)c0 * a.k.s2, a.k.s2, valid);
        tile_load_bf<NT>(x.vr, (const U *)a.v.re + vb + (int64_t)c0 * a.v.s2, a.v.s2, valid);
        tile_load_bf<NT>(x.vi, (const U *)a.v.im + vb + (int64_t)c0 * a.v.s2, a.v.s2, valid);
        x.gam = 1.f;
        x.rr = 1.f;
        x.ri = 0.f;
        if (w < M) {  // wave m forms state m's decay vectors
            const int64_t t = c0 + min(lane, valid - 1);
            x.gam = a.gamma[w * a.sg_m + b * a.sg_b + h * a.sg_h + t * a.sg_t];
            if (a.rot_re) {
                const int64_t ro = w * a.sr_m + b * a.sr_b + h * a.sr_h + t * a.sr_t;
                x.rr = a.rot_re[ro];
                x.ri = a.rot_im[ro];
            }
        }
    };
    auto stage_chunk = [&](int c, const ChunkRegs &x) {
        tile_store_bf<NT>(sQr, x.qr);
        tile_store_bf<NT>(sQi, x.qi);
        tile_store_bf<NT>(sKr, x.kr);
        tile_store_bf<NT>(sKi, x.ki);
        tile_store_bf<NT>(sVr, x.vr);
        tile_store_bf<NT>(sVi, x.vi);
        if (w < M) {
            const int valid = min(64, a.T - c * 64);
            float L = (lane < valid) ? logf(x.gam + LOG_EPS) : 0.f;
            const bool pos = L > 0.f;
#pragma unroll
            for (int off = 1; off < 64; off <<= 1) {
                const float y = __shfl_up(L, off);
                if (lane >= off) L += y;
            }
            const bool ok = !__any(pos) && __shfl(L, 63) >= -FACTOR_RANGE;
            const float Llast = __shfl(L, valid - 1);
            const float rr = lane < valid ? x.rr : 1.f, ri = lane < valid ? x.ri : 0.f;
            const float cum = __expf(L) * a.q_scale;
            sL[w * 64 + lane] = L;
            sRr[w * 64 + lane] = rr;
            sRi[w * 64 + lane] = ri;
            sPr[w * 64 + lane] = rr * cum;
            sPi[w * 64 + lane] = ri * cum;
            sF[w * 64 + lane] = __expf(-L);  // unused (possibly inf) when the test fails
            sDl[w * 64 + lane] = lane < valid ? __expf(fminf(Llast - L, 0.f)) : 0.f;
            if (lane == 0) {
                sTot[w] = __expf(Llast);
                sFast[w] = ok ? 1 : 0;
            }
        }
    };
    // carried state S_m of this wave's tiles (fp32, accumulated transposed: lane holds
    // row i = 16 iu + l16, columns 16 (2 jh + jj) + 4 g .. +3) -> bf16 LDS copy
    floatx4 sR[M][2], sI[M][2];
    auto publish_state = [&](int c) {
#pragma unroll
        for (int m = 0; m < M; ++m)
#pragma unroll
            for (int jj = 0; jj < 2; ++jj) {
                const int o = (16 * iu + l16) * PB + 16 * (2 * jh + jj) + 4 * g;
                *reinterpret_cast<uint2 *>(sS + 2 * m * PLANE_B + o) =
                    make_uint2(pack_bf16x2(sR[m][jj][0], sR[m][jj][1]), pack_bf16x2(sR[m][jj][2], sR[m][jj][3]));
                *reinterpret_cast<uint2 *>(sS + (2 * m + 1) * PLANE_B + o) =
                    make_uint2(pack_bf16x2(sI[m][jj][0], sI[m][jj][1]), pack_bf16x2(sI[m][jj][2], sI[m][jj][3]));
            }
    };
    // the published copy -> the backward's snapshot of chunk c, as 16-byte row
    // pieces (32 bytes per thread and state), after the barrier that follows it
    auto copy_snapshot = [&](int c) {
        const int pl = tid >> 8, row = (tid & 255) >> 2, q = tid & 3;
#pragma unroll
        for (int m = 0; m < M; ++m) {
            const uint4 *src = reinterpret_cast<const uint4 *>(sS + (2 * m + pl) * PLANE_B + row * PB + 16 * q);
            const uint4 v0 = src[0], v1 = src[1];
            uint4 *dst = reinterpret_cast<uint4 *>(chunk_snap_ptr(p, m, b, h, c) + pl * D * D + row * D + 16 * q);
            dst[0] = v0;
            dst[1] = v1;
        }
    };

    ChunkRegs cr;
    load_chunk(c_begin, cr);
#pragma unroll
    for (int m = 0; m < M; ++m) {
        const float *src = p.segs + (seg_chain(a, m, b, h) * p.n_segs + sg) * (2 * D * D);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {
            const int o = (16 * iu + l16) * D + 16 * (2 * jh + jj) + 4 * g;
            sR[m][jj] = *reinterpret_cast<const floatx4 *>(src + o);
            sI[m][jj] = *reinterpret_cast<const floatx4 *>(src + D * D + o);
        }
    }
    publish_state(c_begin);
    stage_chunk(c_begin, cr);
    __syncthreads();
    copy_snapshot(c_begin);

    for (int c = c_begin; c < c_end; ++c) {
        const int c0 = c * 64, valid = min(64, a.T - c0);
        const bool more = c + 1 < c_end;
        const bool carry = (c > 0) || (a.s0_re != nullptr);
        bool fast = true;
#pragma unroll
        for (int m = 0; m < M; ++m) fast = fast && sFast[m];
        const int t = 16 * tt + l16;  // this lane's query row in the transposed score tiles
        floatx4 yR[2], yI[2];
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) yR[ii] = yI[ii] = zero4();
        {
            floatx4 wr[4], wi[4];
#pragma unroll
            for (int st = 0; st < 4; ++st) wr[st] = wi[st] = zero4();
#pragma unroll
            for (int kp = 0; kp < 2; ++kp) {
                const bf16x8 bqr = ld8(sQr + t * PB + 32 * kp + 8 * g), bqi = ld8(sQi + t * PB + 32 * kp + 8 * g);
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    if (st > tt) continue;
                    const int s = 16 * st + l16;
                    const bf16x8 akr = ld8(sKr + s * PB + 32 * kp + 8 * g), aki = ld8(sKi + s * PB + 32 * kp + 8 * g);
                    wr[st] = mfma_bf(akr, bqr, wr[st]);
                    wr[st] = mfma_bf(aki, bqi, wr[st]);
                    wi[st] = mfma_bf(akr, bqi, wi[st]);
                    wi[st] = mfma_bf(neg_bf(aki), bqr, wi[st]);
                }
            }
            // A = (q_scale W) . D~ ; lane holds s = 16st + 4g + r, t = 16tt + l16
            if (fast) {
                // D_m[t,s] = E_m[t] F_m[s]: D~ = sum_m (r_m E_m)[t] F_m[s]
                float pr_t[MAX_M], pi_t[MAX_M];
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    pr_t[m] = sPr[m * 64 + t];
                    pi_t[m] = sPi[m * 64 + t];
                }
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    if (st > tt) continue;
                    float4 F4[MAX_M];
#pragma unroll
                    for (int m = 0; m < M; ++m) F4[m] = *reinterpret_cast<const float4 *>(sF + m * 64 + 16 * st + 4 * g);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int s = 16 * st + 4 * g + r;
                        float dre = 0.f, dim = 0.f;
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            const float f = r == 0 ? F4[m].x : r == 1 ? F4[m].y : r == 2 ? F4[m].z : F4[m].w;
                            dre += pr_t[m] * f;
                            dim += pi_t[m] * f;
                        }
                        const bool keep = st < tt || s <= t;
                        dre = keep ? dre : 0.f;
                        dim = keep ? dim : 0.f;
                        const float xr = wr[st][r], xi = wi[st][r];
                        wr[st][r] = xr * dre - xi * dim;
                        wi[st][r] = xr * dim + xi * dre;
                    }
                }
            } else {
#pragma unroll
                for (int st = 0; st < 4; ++st) {
                    if (st > tt) continue;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int s = 16 * st + 4 * g + r;
                        float dre = 0.f, dim = 0.f;
                        if (s <= t) {
                            if (!general) {
                                dre = __expf(fminf(sL[t] - sL[s], 0.f));
                            } else {
#pragma unroll
                                for (int m = 0; m < M; ++m) {
                                    const float dm = __expf(fminf(sL[m * 64 + t] - sL[m * 64 + s], 0.f));
                                    dre += sRr[m * 64 + t] * dm;
                                    dim += sRi[m * 64 + t] * dm;
                                }
                            }
                        }
                        const float xr = wr[st][r] * qs, xi = wi[st][r] * qs;
                        wr[st][r] = xr * dre - xi * dim;
                        wi[st][r] = xr * dim + xi * dre;
                    }
                }
            }
            // Y += A V: k-step kp covers s-tiles 2kp, 2kp+1 (registers); transposed reads of V
#pragma unroll
            for (int kp = 0; kp < 2; ++kp) {
                if (2 * kp > tt) continue;
                const bf16x8 ar = frag_from_acc(wr[2 * kp], wr[2 * kp + 1]);
                const bf16x8 ai = frag_from_acc(wi[2 * kp], wi[2 * kp + 1]);
                const bf16x8 nai = neg_bf(ai);
#pragma unroll
                for (int ii = 0; ii < 2; ++ii) {  // Y accumulates transposed: lane holds row t, columns 4g + r
                    const int it = 2 * ih + ii, r0 = 32 * kp + 4 * g;
                    const bf16x8 vr = ld_tr(sVr, r0, r0 + 16, 16 * it), vi = ld_tr(sVi, r0, r0 + 16, 16 * it);
                    yR[ii] = mfma_bf(vr, ar, yR[ii]);
                    yR[ii] = mfma_bf(vi, nai, yR[ii]);
                    yI[ii] = mfma_bf(vi, ar, yI[ii]);
                    yI[ii] = mfma_bf(vr, ai, yI[ii]);
                }
            }
        }
        // carried read  Y[t,i] += rho_m[t] q_scale U_m[t,i],  U_m = Q S_m^T on MFMA (operands straight
        // from LDS, shared Q fragments); rho is applied to the fp32 product
        if (carry) {
            bf16x8 aqr[2], aqi[2], naqi[2];
#pragma unroll
            for (int kp = 0; kp < 2; ++kp) {
                aqr[kp] = ld8(sQr + t * PB + 32 * kp + 8 * g);
                aqi[kp] = ld8(sQi + t * PB + 32 * kp + 8 * g);
                naqi[kp] = neg_bf(aqi[kp]);
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const U *Sr = sS + 2 * m * PLANE_B, *Si = Sr + PLANE_B;
                floatx4 uR[2], uI[2];
#pragma unroll
                for (int ii = 0; ii < 2; ++ii) uR[ii] = uI[ii] = zero4();
#pragma unroll
                for (int kp = 0; kp < 2; ++kp) {
#pragma unroll
                    for (int ii = 0; ii < 2; ++ii) {
                        const int row = (16 * (2 * ih + ii) + l16) * PB + 32 * kp + 8 * g;
                        const bf16x8 sr = ld8(Sr + row), si = ld8(Si + row);
                        uR[ii] = mfma_bf(sr, aqr[kp], uR[ii]);
                        uR[ii] = mfma_bf(si, naqi[kp], uR[ii]);
                        uI[ii] = mfma_bf(si, aqr[kp], uI[ii]);
                        uI[ii] = mfma_bf(sr, aqi[kp], uI[ii]);
                    }
                }
                const float prv = sPr[m * 64 + t], piv = sPi[m * 64 + t];  // rho_m q_scale of row t
#pragma unroll
                for (int ii = 0; ii < 2; ++ii) {
                    yR[ii] += prv * uR[ii] - piv * uI[ii];
                    yI[ii] += prv * uI[ii] + piv * uR[ii];
                }
            }
        }
        if (t < valid) {  // row t, columns 16 (2 ih + ii) + 4 g .. +3: 16-byte (fp32) or 8-byte (bf16) runs
            const int64_t yo = b * a.y.s0 + h * a.y.s1 + (int64_t)(c0 + t) * a.y.s2;
#pragma unroll
            for (int ii = 0; ii < 2; ++ii) {
                const int64_t o = yo + 16 * (2 * ih + ii) + 4 * g;
                if (a.y_dtype == QPAM_BF16) {
                    *reinterpret_cast<uint2 *>(reinterpret_cast<U *>(a.y.re) + o) =
                        make_uint2(pack_bf16x2(yR[ii][0], yR[ii][1]), pack_bf16x2(yR[ii][2], yR[ii][3]));
                    *reinterpret_cast<uint2 *>(reinterpret_cast<U *>(a.y.im) + o) =
                        make_uint2(pack_bf16x2(yI[ii][0], yI[ii][1]), pack_bf16x2(yI[ii][2], yI[ii][3]));
                } else {
                    *reinterpret_cast<floatx4 *>(a.y.re + o) = yR[ii];
                    *reinterpret_cast<floatx4 *>(a.y.im + o) = yI[ii];
                }
            }
        }
        if (!more) break;
        load_chunk(c + 1, cr);
        // S_m <- total_m S_m + sum_s D_m[C-1,s] v_s (x) conj(k_s): the scaled state is the MFMA
        // accumulator; A = dl-weighted V^T, B = K (k = s)
        {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float tot = sTot[m];
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    sR[m][jj] *= tot;
                    sI[m][jj] *= tot;
                }
            }
#pragma unroll
            for (int kp = 0; kp < 2; ++kp) {
                const int s0 = 32 * kp + 8 * g;
                bf16x8 kr[2], ki[2];
#pragma unroll
                for (int jj = 0; jj < 2; ++jj) {
                    kr[jj] = ld_tr(sKr, s0, s0 + 4, 16 * (2 * jh + jj));
                    ki[jj] = ld_tr(sKi, s0, s0 + 4, 16 * (2 * jh + jj));
                }
                const floatx8 vr = to_f(ld_tr(sVr, s0, s0 + 4, 16 * iu)), vi = to_f(ld_tr(sVi, s0, s0 + 4, 16 * iu));
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float4 d0 = *reinterpret_cast<const float4 *>(sDl + m * 64 + s0);
                    const float4 d1 = *reinterpret_cast<const float4 *>(sDl + m * 64 + s0 + 4);
                    const floatx8 dl = {d0.x, d0.y, d0.z, d0.w, d1.x, d1.y, d1.z, d1.w};
                    const bf16x8 ar = to_bf(vr * dl), ai = to_bf(vi * dl), nar = neg_bf(ar);
#pragma unroll
                    for (int jj = 0; jj < 2; ++jj) {  // transposed (A = K, B = weighted V)
                        sR[m][jj] = mfma_bf(kr[jj], ar, sR[m][jj]);
                        sR[m][jj] = mfma_bf(ki[jj], ai, sR[m][jj]);
                        sI[m][jj] = mfma_bf(kr[jj], ai, sI[m][jj]);
                        sI[m][jj] = mfma_bf(ki[jj], nar, sI[m][jj]);
                    }
                }
            }
        }
        __syncthreads();  // every read of this chunk's LDS tiles and states is done
        publish_state(c + 1);
        stage_chunk(c + 1, cr);
        __syncthreads();
        copy_snapshot(c + 1);
    }
}

template <int M>
int launch_fwd_bf16_m(const FwdParams &p, hipStream_t stream) {
    const qpam_scan_args &a = p.a;
    const int64_t chains = (int64_t)a.M * a.B * a.H;
    QPAM_REQUIRE(chains * p.n_segs < (1ll << 31) && chains * 8 < (1ll << 31), "qpam_scan_fwd: grid too large");
    const dim3 grid(p.n_segs, a.H, a.B);
    const size_t s_state = seg_state_smem<M>(), s_out = seg_output_smem<M>();
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)seg_state_kernel<M>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)s_state));
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)seg_output_kernel<M>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)s_out));
    hipLaunchKernelGGL(seg_decay_kernel, dim3((unsigned)(chains * p.n_segs)), dim3(THREADS), 0, stream, p);
    int st = launch_status("seg_decay_kernel");
    if (st) return st;
    hipLaunchKernelGGL(seg_state_kernel<M>, grid, dim3(SEG_THREADS), s_state, stream, p);
    st = launch_status("seg_state_kernel");
    if (st) return st;
    hipLaunchKernelGGL(seg_scan_fwd_kernel, dim3((unsigned)(chains * 8)), dim3(THREADS), 0, stream, p);
    st = launch_status("seg_scan_fwd_kernel");
    if (st) return st;
    if (a.prof_ev[0]) QPAM_CHECK_HIP(hipEventRecord((hipEvent_t)a.prof_ev[0], stream));
    hipLaunchKernelGGL(seg_output_kernel<M>, grid, dim3(SEG_THREADS), s_out, stream, p);
    st = launch_status("seg_output_kernel");
    if (st) return st;
    if (a.prof_ev[1]) QPAM_CHECK_HIP(hipEventRecord((hipEvent_t)a.prof_ev[1], stream));
    return QPAM_OK;
}

// The state count is a compile-time constant of the segment kernels.
int launch_fwd_bf16(const FwdParams &p, hipStream_t stream) {
    switch (p.a.M) {
        case 1: return launch_fwd_bf16_m<1>(p, stream);
        case 2: return launch_fwd_bf16_m<2>(p, stream);
        case 3: return launch_fwd_bf16_m<3>(p, stream);
        default: return launch_fwd_bf16_m<4>(p, stream);
    }
}

template <int C>
size_t state_smem() { return (size_t)(4 * C * P + MAX_M * 64) * sizeof(float); }
template <int C>
size_t output_smem() { return (size_t)(4 * C * P + 2 * D * P + 3 * MAX_M * 64) * sizeof(float); }
template <int C>
size_t output_f32_smem() { return (size_t)(2 * C * P + 2 * D * P + 3 * MAX_M * 64) * sizeof(float); }

template <typename Tin, int C>
int launch_fwd(const FwdParams &p, hipStream_t stream) {
    const qpam_scan_args &a = p.a;
    dim3 grid(p.n_chunks, a.H, a.B);
    constexpr bool f32 = std::is_same<Tin, float>::value;
    const void *out_kernel = f32 ? (const void *)chunk_output_f32_kernel<C> : (const void *)chunk_output_kernel<Tin, C>;
    const size_t s1 = state_smem<C>(), s3 = f32 ? output_f32_smem<C>() : output_smem<C>();
    QPAM_CHECK_HIP(hipFuncSetAttribute(out_kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)s3));
    int st;
    if constexpr (f32 && C == 64) {
        const long long blocks = (long long)a.M * a.B * a.H * PASS32_SPLIT;
        QPAM_REQUIRE(blocks < (1ll << 31), "qpam_scan_fwd: grid too large");
        const long long items = (long long)a.M * a.B * a.H * p.n_chunks;
        hipLaunchKernelGGL(chunk_decay_f32_kernel, dim3((unsigned)((items + 3) / 4)), dim3(THREADS), 0, stream, p);
        st = launch_status("chunk_decay_f32_kernel");
        if (st) return st;
        hipLaunchKernelGGL(state_pass_f32_kernel, dim3((unsigned)blocks), dim3(PASS32_THREADS), 0, stream, p);
        st = launch_status("state_pass_f32_kernel");
        if (st) return st;
    } else {
        QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)chunk_state_kernel<Tin, C>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)s1));
        hipLaunchKernelGGL((chunk_state_kernel<Tin, C>), grid, dim3(THREADS), s1, stream, p);
        st = launch_status("chunk_state_kernel");
        if (st) return st;
        hipLaunchKernelGGL(state_scan_kernel, dim3(a.M * a.B * a.H * SCAN_BLOCKS), dim3(THREADS), 0, stream, p);
        st = launch_status("state_scan_kernel");
        if (st) return st;
    }
    if (a.prof_ev[0]) QPAM_CHECK_HIP(hipEventRecord((hipEvent_t)a.prof_ev[0], stream));
    if constexpr (f32) hipLaunchKernelGGL((chunk_output_f32_kernel<C>), grid, dim3(THREADS), s3, stream, p);
    else hipLaunchKernelGGL((chunk_output_kernel<Tin, C>), grid, dim3(THREADS), s3, stream, p);
    st = launch_status("chunk_output_kernel");
    if (st) return st;
    if (a.prof_ev[1]) QPAM_CHECK_HIP(hipEventRecord((hipEvent_t)a.prof_ev[1], stream));
    return QPAM_OK;
}

}  // namespace

bool uses_snapshots(const qpam_scan_args &a) { return a.dtype == QPAM_BF16 && a.C == 64; }

// Workspace: fp32 per-chunk states (fp32 inputs), fp32 chunk totals, then (bf16 path with 64-step chunks) the segment totals and the
// two per-step segment weights; at a 256-byte aligned offset either the bf16
// entering-state snapshots followed by the fp32 segment states (bf16, 64-step
// chunks) or the fp32 state pass's decay weights (fp32, 64-step chunks).
int64_t fwd_totals_offset(const qpam_scan_args &a) {  // in floats
    const int64_t n = (a.T + a.C - 1) / a.C;
    return uses_snapshots(a) ? 0 : (int64_t)a.M * a.B * a.H * n * 2 * D * D;
}

SegLayout seg_layout(const qpam_scan_args &a) {
    const int64_t n = (a.T + a.C - 1) / a.C, n_segs = (n + SEG - 1) / SEG;
    const int64_t chains = (int64_t)a.M * a.B * a.H;
    SegLayout l;
    l.n_segs = (int)n_segs;
    l.segtot = fwd_totals_offset(a) + chains * n;
    l.wfwd = l.segtot + chains * n_segs;
    l.wbwd = l.wfwd + chains * n * 64;
    l.wgr = l.wbwd + chains * n * 64;
    l.wgi = l.wgr + chains * n * 64;
    return l;
}

size_t fwd_snapshot_offset(const qpam_scan_args &a) {
    const int64_t n = (a.T + a.C - 1) / a.C;
    const int64_t chains = (int64_t)a.M * a.B * a.H;
    const int64_t floats = uses_snapshots(a) ? seg_layout(a).wgi + chains * n * 64 : fwd_totals_offset(a) + chains * n;
    return ((size_t)floats * sizeof(float) + 255) & ~(size_t)255;
}

size_t fwd_segs_offset(const qpam_scan_args &a) {
    const int64_t n = (a.T + a.C - 1) / a.C;
    const int64_t chains = (int64_t)a.M * a.B * a.H;
    return fwd_snapshot_offset(a) + (size_t)chains * n * 2 * D * D * sizeof(unsigned short);
}

// fp32 path with 64-step chunks: the state pass's decay weights sit where the
// snapshot path keeps its snapshots
bool uses_dlast(const qpam_scan_args &a) { return a.dtype == QPAM_F32 && a.C == 64; }

size_t fwd_workspace_bytes(const qpam_scan_args &a) {
    const int64_t n = (a.T + a.C - 1) / a.C;
    const int64_t chains = (int64_t)a.M * a.B * a.H;
    if (uses_snapshots(a)) return fwd_segs_offset(a) + (size_t)chains * seg_layout(a).n_segs * 2 * D * D * sizeof(float);
    size_t bytes = fwd_snapshot_offset(a);
    if (uses_dlast(a)) bytes += (size_t)chains * n * 64 * sizeof(float);
    return bytes;
}

int validate_scan(const qpam_scan_args *a, const char *who, bool fwd_outputs) {
    QPAM_REQUIRE(a != nullptr, "%s: null args", who);
    QPAM_REQUIRE(a->B >= 1 && a->H >= 1 && a->T >= 1 && a->M >= 1, "%s: bad sizes B=%d H=%d T=%d M=%d", who, a->B,
                 a->H, a->T, a->M);
    if (a->d != D) return fail(QPAM_ERR_UNSUPPORTED, "%s: head dim %d (this build supports 64)", who, a->d);
    if (a->C != 16 && a->C != 32 && a->C != 64)
        return fail(QPAM_ERR_UNSUPPORTED, "%s: chunk %d (supported 16, 32, 64)", who, a->C);
    if (a->M > MAX_M) return fail(QPAM_ERR_UNSUPPORTED, "%s: %d states (max %d)", who, a->M, MAX_M);
    QPAM_REQUIRE(a->dtype == QPAM_F32 || a->dtype == QPAM_BF16, "%s: dtype %d", who, a->dtype);
    const qpam_cview *vs[3] = {&a->q, &a->k, &a->v};
    const int vec = a->dtype == QPAM_F32 ? 4 : 8;  // elements per 16-byte load
    for (const qpam_cview *v : vs) {
        QPAM_REQUIRE(v->re && v->im, "%s: null q/k/v plane", who);
        QPAM_REQUIRE(((uintptr_t)v->re % 16) == 0 && ((uintptr_t)v->im % 16) == 0,
                     "%s: q/k/v planes must be 16-byte aligned", who);
        QPAM_REQUIRE(v->s0 % vec == 0 && v->s1 % vec == 0 && v->s2 % vec == 0,
                     "%s: q/k/v strides must be multiples of %d elements", who, vec);
    }
    QPAM_REQUIRE(a->gamma != nullptr, "%s: null gamma", who);
    QPAM_REQUIRE((a->rot_re == nullptr) == (a->rot_im == nullptr), "%s: rot needs both planes", who);
    QPAM_REQUIRE((a->s0_re == nullptr) == (a->s0_im == nullptr), "%s: s0 needs both planes", who);
    QPAM_REQUIRE((a->s_re == nullptr) == (a->s_im == nullptr), "%s: s_out needs both planes", who);
    QPAM_REQUIRE(!fwd_outputs || (a->y.re && a->y.im), "%s: null y", who);
    QPAM_REQUIRE(a->y_dtype == QPAM_F32 || (a->y_dtype == QPAM_BF16 && a->dtype == QPAM_BF16 && a->C == 64),
                 "%s: y_dtype %d (bf16 y needs bf16 inputs and chunk 64)", who, a->y_dtype);
    const uintptr_t al = (uintptr_t)a->s0_re | (uintptr_t)a->s0_im | (uintptr_t)a->s_re | (uintptr_t)a->s_im;
    QPAM_REQUIRE(al % 16 == 0, "%s: state buffers must be 16-byte aligned", who);
    if (fwd_outputs && uses_snapshots(*a)) {  // Y rows leave in 16-byte (fp32) / 8-byte (bf16) runs
        const uintptr_t ya = (uintptr_t)a->y.re | (uintptr_t)a->y.im;
        QPAM_REQUIRE(ya % (a->y_dtype == QPAM_BF16 ? 8 : 16) == 0 && a->y.s0 % 4 == 0 && a->y.s1 % 4 == 0 &&
                         a->y.s2 % 4 == 0,
                     "%s: y planes must be %d-byte aligned with strides multiple of 4", who,
                     a->y_dtype == QPAM_BF16 ? 8 : 16);
    }
    QPAM_REQUIRE(a->workspace != nullptr && a->workspace_bytes >= fwd_workspace_bytes(*a) &&
                     ((uintptr_t)a->workspace % 16) == 0,
                 "%s: workspace needs %zu bytes (got %zu)", who, fwd_workspace_bytes(*a), a->workspace_bytes);
    return QPAM_OK;
}

int scan_fwd(const qpam_scan_args *a, hipStream_t stream) {
    int st = validate_scan(a, "qpam_scan_fwd", true);
    if (st) return st;
    FwdParams p;
    p.a = *a;
    p.n_chunks = (a->T + a->C - 1) / a->C;
    p.states = uses_snapshots(*a) ? nullptr : (float *)a->workspace;
    p.totals = (float *)a->workspace + fwd_totals_offset(*a);
    p.snap = uses_snapshots(*a)
                 ? reinterpret_cast<unsigned short *>((char *)a->workspace + fwd_snapshot_offset(*a))
                 : nullptr;
    p.dlast = uses_dlast(*a) ? reinterpret_cast<float *>((char *)a->workspace + fwd_snapshot_offset(*a)) : nullptr;
    p.n_segs = 0;
    p.segs = p.segtot = p.wfwd = p.wbwd = p.wgr = p.wgi = nullptr;
    if (uses_snapshots(*a)) {
        const SegLayout l = seg_layout(*a);
        p.n_segs = l.n_segs;
        p.segtot = (float *)a->workspace + l.segtot;
        p.wfwd = (float *)a->workspace + l.wfwd;
        p.wbwd = (float *)a->workspace + l.wbwd;
        p.wgr = (float *)a->workspace + l.wgr;
        p.wgi = (float *)a->workspace + l.wgi;
        p.segs = reinterpret_cast<float *>((char *)a->workspace + fwd_segs_offset(*a));
    }
    QPAM_REQUIRE(p.n_chunks <= 65535 && a->H <= 65535 && a->B <= 65535, "qpam_scan_fwd: grid too large");
    const bool bf = a->dtype == QPAM_BF16;
    if (uses_snapshots(*a)) return launch_fwd_bf16(p, stream);
    switch (a->C) {
        case 16: return bf ? launch_fwd<unsigned short, 16>(p, stream) : launch_fwd<float, 16>(p, stream);
        case 32: return bf ? launch_fwd<unsigned short, 32>(p, stream) : launch_fwd<float, 32>(p, stream);
        default: return bf ? launch_fwd<unsigned short, 64>(p, stream) : launch_fwd<float, 64>(p, stream);
    }
}

}  // namespace scan
}  // namespace qpam

extern "C" size_t qpam_scan_workspace_size(const qpam_scan_args *a) {
    return a ? qpam::scan::fwd_workspace_bytes(*a) : 0;
}

extern "C" int qpam_scan_fwd(const qpam_scan_args *a, void *stream) {
    return qpam::scan::scan_fwd(a, (hipStream_t)stream);
}

// ------------------------------------------------ allocation-free entry --
// qpam_scan_fwd with the per-chunk states in `scratch`, a device array of the
// library (one copy per GPU, alive until the process ends), instead of a
// caller workspace.  Host code never passes the array's name to a kernel (on
// the host it is only a stand-in for the symbol): the device address comes
// from hipGetSymbolAddress, once per device, kept in that device's entry.
// The forward kernels overwrite every workspace word they later read, so no
// part of the array has to start at zero.
//
// Misuse check: each call records an event on its stream after its launches;
// a call on another stream while the previous call's event is still pending
// (hipEventQuery, no host wait) would share the array with work in flight, and
// is refused.  Calls on one stream are ordered by the stream and always pass.
namespace {

static __device__ __align__(256) unsigned char scratch[QPAM_SCAN_FWD_NOALLOC_MAX_BYTES];

struct NoallocDevice {
    void *ptr = nullptr;            // device address of `scratch` on this device
    hipEvent_t done = nullptr;      // recorded after the last call's launches
    hipStream_t last = nullptr;     // the stream of the last call
    bool recorded = false;
};

std::mutex &noalloc_mutex() {
    static std::mutex mu;
    return mu;
}

// The device's entry, set up on its first call (symbol address and event).
int noalloc_device(NoallocDevice *&out) {
    static std::map<int, NoallocDevice> devs;  // guarded by noalloc_mutex()
    int dev = 0;
    QPAM_CHECK_HIP(hipGetDevice(&dev));
    auto it = devs.find(dev);
    if (it == devs.end()) {
        NoallocDevice d;
        QPAM_CHECK_HIP(hipGetSymbolAddress(&d.ptr, HIP_SYMBOL(scratch)));
        QPAM_REQUIRE(d.ptr != nullptr && ((uintptr_t)d.ptr % 256) == 0, "qpam_scan_fwd_noalloc: bad scratch address");
        QPAM_CHECK_HIP(hipEventCreateWithFlags(&d.done, hipEventDisableTiming));
        it = devs.emplace(dev, d).first;
    }
    out = &it->second;
    return QPAM_OK;
}

}  // namespace

extern "C" int qpam_scan_fwd_noalloc(const qpam_scan_args *a, void *stream) {
    QPAM_REQUIRE(a != nullptr, "qpam_scan_fwd_noalloc: null args");
    QPAM_REQUIRE(a->B >= 1 && a->H >= 1 && a->T >= 1 && a->M >= 1 && a->C >= 1,
                 "qpam_scan_fwd_noalloc: bad sizes B=%d H=%d T=%d M=%d C=%d", a->B, a->H, a->T, a->M, a->C);
    const size_t need = qpam::scan::fwd_workspace_bytes(*a);
    if (need > (size_t)QPAM_SCAN_FWD_NOALLOC_MAX_BYTES)
        return qpam::fail(QPAM_ERR_WORKSPACE,
                          "qpam_scan_fwd_noalloc: this call needs %zu bytes of scan state, the library's scratch "
                          "holds %zu (use qpam_scan_fwd with a caller workspace)",
                          need, (size_t)QPAM_SCAN_FWD_NOALLOC_MAX_BYTES);
    const hipStream_t s = (hipStream_t)stream;
    std::lock_guard<std::mutex> lock(noalloc_mutex());
    NoallocDevice *d = nullptr;
    int st = noalloc_device(d);
    if (st) return st;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    QPAM_CHECK_HIP(hipStreamIsCapturing(s, &cap));
    const bool capturing = cap != hipStreamCaptureStatusNone;
    if (!capturing && d->recorded && d->last != s) {
        const hipError_t q = hipEventQuery(d->done);
        if (q == hipErrorNotReady)
            return qpam::fail(QPAM_ERR_ARG,
                              "qpam_scan_fwd_noalloc: the previous call on another stream is still running; calls "
                              "that overlap on one GPU would share the library's scratch (use one stream, or "
                              "qpam_scan_fwd with a workspace per call)");
        if (q != hipSuccess) return qpam::fail(QPAM_ERR_HIP, "hipEventQuery failed: %s", hipGetErrorString(q));
    }
    qpam_scan_args b = *a;
    b.workspace = d->ptr;
    b.workspace_bytes = (size_t)QPAM_SCAN_FWD_NOALLOC_MAX_BYTES;
    st = qpam::scan::scan_fwd(&b, s);
    if (st) return st;
    if (!capturing) {  // under graph capture the graph's own replays are the caller's to order
        QPAM_CHECK_HIP(hipEventRecord(d->done, s));
        d->last = s;
        d->recorded = true;
    }
    return QPAM_OK;
}
