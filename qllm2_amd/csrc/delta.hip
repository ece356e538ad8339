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
// Forward: the chunked form on fp32 MFMA (delta_prep_kernel, chunk-parallel,
// then delta_chunk_kernel along the chunks; described at the kernels).
// The rows of S are independent under the recurrence (row i reads only k, q,
// v_i, gamma, beta), so the chunk pass splits a chain's 64 value rows over four
// blocks.
//
// Backward: the same chunked form differentiated, on fp32 MFMA in three
// launches (described at the kernels): a reverse pass along the chunks for the
// gradient of the state (rows of it are independent again: four blocks per
// chain), then two chunk-parallel kernels for the score-matrix gradients and
// for dq, dk, dgamma, dbeta.  The forward leaves what they need in its
// workspace: the state entering every chunk, U, and the chunk's products in the
// orders the backward reads them.
#include "common.h"

namespace qpam {
namespace {

constexpr int D = 64;

// ---------------------------------------------------------------------------
// Forward over 64-step chunks on fp32 MFMA (v_mfma_f32_16x16x4f32).  Unrolled
// over a chunk, the recurrence is the reference's UT form: with L_t the
// inclusive prefix of log(gamma + eps) from the chunk's start, alpha_t = e^{L_t},
// D[t,s] = e^{min(L_t - L_s, 0)} (the reference's decay matrix) and S_0 the state
// entering the chunk,
//     (I + M) U = W,   M[t,s] = beta_t D[t,s] (k_t . conj(k_s))  (s < t),
//     W_t = beta_t (v_t - alpha_t S_0 k_t),
//     y_t = alpha_t S_0 q~_t + sum_{s<=t} D[t,s] (q~_t . conj(k_s)) u_s,
//     S_end = alpha_last S_0 + sum_s tail_s u_s (x) conj(k_s),
// tail_s = alpha_last / (alpha_s + 1e-12) as the reference writes the state
// (v11/model.py:565-566; the exact ratio e^{L_last - L_s} except where alpha_s
// nears 1e-12, and D = e^{L_t - L_s} except for gamma + eps > 1).
// delta_prep_kernel (chunk-parallel, a block per (b, h, chunk)) forms everything
// that does not depend on S: the Gram and query-key products, T = (I + M)^{-1}
// (diagonal 16 x 16 blocks by forward substitution, the blocks below them as
// T_bc = -T_bb sum_k M_bk T_kc) and Ahat[t,s] = D[t,s] (q~_t . conj(k_s)), stored
// per chunk in the MFMA A-operand order.  delta_chunk_kernel then walks the
// chunks of one (b, h) for 16 value rows (rows of the recurrence are
// independent: four blocks per chain) with S^T in LDS: W = beta (V - alpha K S^T),
// U = T W, the state update, then Y = Ahat U + alpha Q~ S^T with the chunk's
// entering state.
constexpr int CH = 64;                 // kernel rows per chunk
constexpr int ROW_BLOCKS = 4;          // blocks per chain in the chunk pass (16 value rows each)
// Steps per chunk of a call: the reference's chunk length (its delta_chunk,
// 1..CH; 0 selects CH).  Each chunk of the call runs as one kernel chunk of CH
// rows whose rows past the chunk's steps are zero (beta 0), exactly as a ragged
// last chunk, so the chunk-dependent parts of the chunked form (the clamped decay
// matrix, the state-write weight alpha_last / (alpha_s + 1e-12)) follow the
// reference's chunk boundaries.
__host__ __device__ __forceinline__ int chunk_len(const qpam_delta_args &a) { return a.chunk > 0 ? a.chunk : CH; }
// log of a step's decay factor (gamma + gamma_eps, kept at or above the smallest
// normal float so that gamma = 0 stays finite)
__device__ __forceinline__ float decay_log(float gamma, float eps) { return logf(fmaxf(gamma + eps, 1.17549435e-38f)); }
// The state-write weight of step s in its chunk: the reference's chunked form
// alpha_last / (alpha_s + 1e-12), or exp(L_last - L_s) (the token recurrence's
// weight, 1 for the last step) when the call asks for the exact write.
__device__ __forceinline__ float write_weight(const qpam_delta_args &a, float Ls, float Llast) {
    return a.exact_write ? __expf(Llast - Ls) : __expf(Llast) / (__expf(Ls) + 1e-12f);
}
// d weight / d L_s divided by -weight: alpha_s / (alpha_s + 1e-12), or 1 (exact write)
__device__ __forceinline__ float write_weight_dl(const qpam_delta_args &a, float Ls) {
    if (a.exact_write) return 1.f;
    const float al = __expf(Ls);
    return al / (al + 1e-12f);
}
constexpr int KP = CH + 4;             // LDS pitch of [64][64] fp32 tiles read element-wise
constexpr int SP = 16;                 // LDS pitch of [64][16] fp32 tiles
constexpr int NBLK = 10;               // 16 x 16 blocks on and below the diagonal of a 64 x 64 matrix
constexpr int BLK = 2 * 256;           // floats of one complex 16 x 16 block (re plane, then im)
constexpr int PREP_T = 0, PREP_A = NBLK * BLK, PREP_L = 2 * NBLK * BLK;
constexpr int PREP_FLOATS = PREP_L + CH;  // per chunk: T blocks, Ahat blocks, L

// The forward's workspace (kept for the backward), one record per (b, h, chunk):
// the entering state S [plane][i][j] and U [plane][t][i] (row-major), then the
// chunk's products in the orders the backward reads them: T^H and Ahat^H in
// A-operand order (T^H block (rows a, cols b >= a) at index blk(b, a), likewise
// Ahat^H), and Ahat and D.Gk (D[t,s] k_t.conj(k_s) for s < t) in accumulator
// order (block (bt, bs), lane (l16, g), element r <-> t = 16 bt + 4 g + r,
// s = 16 bs + l16, float4 per lane and plane), and L.
constexpr int WS_S = 0, WS_U = 2 * D * D, WS_TH = 4 * D * D, WS_AH = WS_TH + NBLK * BLK,
              WS_AA = WS_AH + NBLK * BLK, WS_GA = WS_AA + NBLK * BLK, WS_L = WS_GA + NBLK * BLK,
              WS_REC = WS_L + CH;
// The backward's workspace, one record per (b, h, chunk): G (the gradient of the
// state after the chunk) [plane][i][j], dW [plane][t][i], dP = D.dAhat and
// dGk = beta D.dM in two layouts each (x_Q: transposed accumulator order, lane
// (l16, g), r <-> t = 16 bt + l16, s = 16 bs + 4 g + r; x_K: accumulator order),
// and two per-step vectors: the score part of the log-decay gradient and the
// beta gradient through M.
constexpr int BW_G = 0, BW_W = 2 * D * D, BW_PQ = 4 * D * D, BW_PK = BW_PQ + NBLK * BLK,
              BW_GQ = BW_PK + NBLK * BLK, BW_GK = BW_GQ + NBLK * BLK, BW_V = BW_GK + NBLK * BLK,
              BW_REC = BW_V + 2 * CH;

__device__ __forceinline__ int blk(int b, int c) { return b * (b + 1) / 2 + c; }  // c <= b

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Complex 16 x 16 blocks in the prep kernel's LDS: rows of LP floats (one pad
// float: the MFMA A-operand reads step the 16 lanes of a group over rows, which a
// pitch of 16 would put on one bank in four), re plane then im plane (LPL apart).
constexpr int LP = 17, LPL = 16 * LP, LBLK = 2 * LPL;

__device__ __forceinline__ void blk_store(float *dst, const floatx4 &cr, const floatx4 &ci, int l16, int g) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        dst[(4 * g + r) * LP + l16] = cr[r];
        dst[LPL + (4 * g + r) * LP + l16] = ci[r];
    }
}

__device__ __forceinline__ int64_t chunk_prep(int64_t chain, int n_chunks, int c) {
    return (chain * n_chunks + c) * PREP_FLOATS;
}

// LDS block [16][16] (re, im) -> global in A-operand order: lane (l16 = row, g)
// reads float4 {A[row][4 ks + g], ks = 0..3} at (g * 16 + row) * 4 (per plane)
__device__ __forceinline__ void blk_export(float *dst, const float *src, int tid, int nthreads) {
    for (int e = tid; e < 512; e += nthreads) {
        const int pl = e >> 8, idx = e & 255, ln = idx >> 2, ks = idx & 3;
        const int row = ln & 15, gg = ln >> 4;
        dst[e] = src[pl * LPL + row * LP + 4 * ks + gg];
    }
}

// Gauss accumulation of a complex product over k: t1 += ar br, t2 += ai bi,
// t3 += (ar + ai)(br + bi); then re = t1 - t2, im = t3 - t1 - t2.  Three real
// MFMAs per complex product instead of four.
struct Gauss {
    floatx4 t1, t2, t3;
};
__device__ __forceinline__ void gz(Gauss &x) {
    x.t1 = x.t2 = x.t3 = floatx4{0.f, 0.f, 0.f, 0.f};
}
__device__ __forceinline__ void gstep(Gauss &x, float ar, float ai, float br, float bi) {
    x.t1 = mfma4(ar, br, x.t1);
    x.t2 = mfma4(ai, bi, x.t2);
    x.t3 = mfma4(ar + ai, br + bi, x.t3);
}
__device__ __forceinline__ floatx4 gre(const Gauss &x) { return x.t1 - x.t2; }
__device__ __forceinline__ floatx4 gim(const Gauss &x) { return x.t3 - x.t1 - x.t2; }

// C = A B for complex 16 x 16 LDS blocks (Gauss)
__device__ __forceinline__ void blk_mul_g(Gauss &x, const float *A, const float *B, int l16, int g) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int k = 4 * ks + g;
        gstep(x, A[l16 * LP + k], A[LPL + l16 * LP + k], B[k * LP + l16], B[LPL + k * LP + l16]);
    }
}
// element (4g + r, l16) of an LDS block, re and im
__device__ __forceinline__ float blk_re(const float *A, int g, int r, int l16) { return A[(4 * g + r) * LP + l16]; }
__device__ __forceinline__ float blk_im(const float *A, int g, int r, int l16) {
    return A[LPL + (4 * g + r) * LP + l16];
}

// The prep block's LDS: K and q_scale Q of the chunk while the Gram and
// query-key products run; the same bytes then hold M, T and each wave's four
// scratch blocks of the diagonal inversion, whose first three blocks later hold
// the partial sums of the blocks below the diagonal (two blocks per CU).
constexpr int PREP_KQ = 4 * CH * KP;
constexpr int PREP_INV = NBLK * LBLK * 2 + 16 * LBLK;
constexpr size_t PREP_SMEM = (size_t)((PREP_KQ > PREP_INV ? PREP_KQ : PREP_INV) + 2 * CH) * sizeof(float);

__global__ void __launch_bounds__(256, 2) delta_prep_kernel(qpam_delta_args a, float *prep, int n_chunks) {
    extern __shared__ float sm[];
    float *sKr = sm, *sKi = sKr + CH * KP, *sQr = sKi + CH * KP, *sQi = sQr + CH * KP;
    float *sM = sm;                // after the products: M blocks [blk][re | im][16][16] (diagonal included)
    float *sT = sM + NBLK * LBLK;  // T blocks
    float *sX = sT + NBLK * LBLK;  // four scratch blocks per wave
    float *sR = sX;                // after the inversion: three partial sums
    const int big = PREP_KQ > PREP_INV ? PREP_KQ : PREP_INV;
    float *sL = sm + big, *sB = sL + CH;
    const int chain = blockIdx.x / n_chunks, c = blockIdx.x % n_chunks;
    const int b = chain / a.H, h = chain % a.H;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int t0 = c * chunk_len(a), valid = min(chunk_len(a), a.T - t0);
    // the backward's record of this chunk (when a backward follows)
    float *wrec = a.workspace ? static_cast<float *>(a.workspace) + ((int64_t)chain * n_chunks + c) * WS_REC : nullptr;
    {  // K and q_scale Q, rows past the end zero
        const float *kre = static_cast<const float *>(a.k.re) + b * a.k.s0 + h * a.k.s1;
        const float *kim = static_cast<const float *>(a.k.im) + b * a.k.s0 + h * a.k.s1;
        const float *qre = static_cast<const float *>(a.q.re) + b * a.q.s0 + h * a.q.s1;
        const float *qim = static_cast<const float *>(a.q.im) + b * a.q.s0 + h * a.q.s1;
        for (int idx = tid; idx < CH * 16; idx += 256) {
            const int r = idx >> 4, c4 = 4 * (idx & 15);
            floatx4 kr = {0.f, 0.f, 0.f, 0.f}, ki = kr, qr = kr, qi = kr;
            if (r < valid) {
                const int64_t tk = (int64_t)(t0 + r) * a.k.s2 + c4, tq = (int64_t)(t0 + r) * a.q.s2 + c4;
                kr = *reinterpret_cast<const floatx4 *>(kre + tk);
                ki = *reinterpret_cast<const floatx4 *>(kim + tk);
                qr = *reinterpret_cast<const floatx4 *>(qre + tq) * a.q_scale;
                qi = *reinterpret_cast<const floatx4 *>(qim + tq) * a.q_scale;
            }
            *reinterpret_cast<floatx4 *>(sKr + r * KP + c4) = kr;
            *reinterpret_cast<floatx4 *>(sKi + r * KP + c4) = ki;
            *reinterpret_cast<floatx4 *>(sQr + r * KP + c4) = qr;
            *reinterpret_cast<floatx4 *>(sQi + r * KP + c4) = qi;
        }
    }
    if (w == 0) {  // inclusive prefix of log(gamma + eps); held past the end
        const int64_t go = b * a.sg_b + h * a.sg_h + (int64_t)(t0 + min(lane, valid - 1)) * a.sg_t;
        float x = lane < valid ? decay_log(a.gamma[go], a.gamma_eps) : 0.f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float y = __shfl_up(x, off);
            if (lane >= off) x += y;
        }
        sL[lane] = x;
        sB[lane] = lane < valid ? a.beta[go] : 0.f;
        prep[chunk_prep(chain, n_chunks, c) + PREP_L + lane] = x;
        if (wrec) wrec[WS_L + lane] = x;
    }
    __syncthreads();
    // 20 products (10 blocks on and below the diagonal, Gram G[t,s] = k_t . conj(k_s) and
    // query-key P[t,s] = q~_t . conj(k_s)), five per wave: items w, w + 4, ..., w + 16
    // (item i: kind i & 1, block i >> 1)
    Gauss acc[5];
#pragma unroll
    for (int it = 0; it < 5; ++it) {
        const int item = w + 4 * it, kind = item & 1, bk = item >> 1;
        const int bb = (bk >= 1) + (bk >= 3) + (bk >= 6), cc = bk - bb * (bb + 1) / 2;
        const float *Ar = kind ? sQr : sKr, *Ai = kind ? sQi : sKi;
        const int ra = (16 * bb + l16) * KP, rb = (16 * cc + l16) * KP;
        gz(acc[it]);
#pragma unroll 4
        for (int ks = 0; ks < 16; ++ks) {
            const int j = 4 * ks + g;
            gstep(acc[it], Ar[ra + j], Ai[ra + j], sKr[rb + j], -sKi[rb + j]);  // times conj(k_s)
        }
    }
    __syncthreads();  // K and Q no longer read: their bytes become M, T and scratch
#pragma unroll
    for (int it = 0; it < 5; ++it) {
        const int item = w + 4 * it, kind = item & 1, bk = item >> 1;
        const int bb = (bk >= 1) + (bk >= 3) + (bk >= 6), cc = bk - bb * (bb + 1) / 2;
        const floatx4 xr = gre(acc[it]), xi = gim(acc[it]);
        if (kind == 0) {
            float *Mb = sM + bk * LBLK;
            floatx4 gr, gi;  // D.Gk for the backward
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * bb + 4 * g + r, s = 16 * cc + l16;
                const float dts = s < t ? __expf(fminf(sL[t] - sL[s], 0.f)) : 0.f;
                const float m = sB[t] * dts;
                Mb[(4 * g + r) * LP + l16] = m * xr[r];
                Mb[LPL + (4 * g + r) * LP + l16] = m * xi[r];
                gr[r] = dts * xr[r];
                gi[r] = dts * xi[r];
            }
            if (wrec) {
                float *dst = wrec + WS_GA + bk * BLK + (g * 16 + l16) * 4;
                *reinterpret_cast<floatx4 *>(dst) = gr;
                *reinterpret_cast<floatx4 *>(dst + 256) = gi;
            }
        } else {
            // Ahat in A-operand order: element (row 4g + r, col l16) -> lane (col % 4) * 16 + row, slot col / 4
            float *dst = prep + chunk_prep(chain, n_chunks, c) + PREP_A + bk * BLK;
            floatx4 ar, ai;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * bb + 4 * g + r, s = 16 * cc + l16;
                const float dts = s <= t ? __expf(fminf(sL[t] - sL[s], 0.f)) : 0.f;
                const int ln = (l16 & 3) * 16 + 4 * g + r, ks = l16 >> 2;
                ar[r] = dts * xr[r];
                ai[r] = dts * xi[r];
                dst[ln * 4 + ks] = ar[r];
                dst[256 + ln * 4 + ks] = ai[r];
            }
            if (wrec) {
                // Ahat in accumulator order; Ahat^H in A-operand order (rows s: lane (l16, r), slot g)
                float *da = wrec + WS_AA + bk * BLK + (g * 16 + l16) * 4;
                *reinterpret_cast<floatx4 *>(da) = ar;
                *reinterpret_cast<floatx4 *>(da + 256) = ai;
                float *dh = wrec + WS_AH + bk * BLK;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    dh[(r * 16 + l16) * 4 + g] = ar[r];
                    dh[256 + (r * 16 + l16) * 4 + g] = -ai[r];
                }
            }
        }
    }
    __syncthreads();
    {  // T_bb = (I + N)^{-1} = (I - N)(I + N^2)(I + N^4)(I + N^8), N = M_bb nilpotent (N^16 = 0); wave b
        const float *N = sM + blk(w, w) * LBLK;
        float *X = sX + w * 4 * LBLK;  // N^2, N^4, N^8, P1 (then P2 over N^2)
        Gauss x;
        gz(x);
        blk_mul_g(x, N, N, l16, g);
        blk_store(X, gre(x), gim(x), l16, g);
        gz(x);
        blk_mul_g(x, X, X, l16, g);
        blk_store(X + LBLK, gre(x), gim(x), l16, g);
        gz(x);
        blk_mul_g(x, X + LBLK, X + LBLK, l16, g);
        blk_store(X + 2 * LBLK, gre(x), gim(x), l16, g);
        // P1 = I - N + N^2 - N N^2
        gz(x);
        blk_mul_g(x, N, X, l16, g);
        {
            floatx4 pr = -gre(x), pi = -gim(x);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pr[r] += (4 * g + r == l16 ? 1.f : 0.f) - blk_re(N, g, r, l16) + blk_re(X, g, r, l16);
                pi[r] += -blk_im(N, g, r, l16) + blk_im(X, g, r, l16);
            }
            blk_store(X + 3 * LBLK, pr, pi, l16, g);
        }
        // P2 = P1 + P1 N^4 (over N^2)
        gz(x);
        blk_mul_g(x, X + 3 * LBLK, X + LBLK, l16, g);
        {
            floatx4 pr = gre(x), pi = gim(x);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pr[r] += blk_re(X + 3 * LBLK, g, r, l16);
                pi[r] += blk_im(X + 3 * LBLK, g, r, l16);
            }
            blk_store(X, pr, pi, l16, g);
        }
        // T = P2 + P2 N^8
        gz(x);
        blk_mul_g(x, X, X + 2 * LBLK, l16, g);
        {
            floatx4 pr = gre(x), pi = gim(x);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pr[r] += blk_re(X, g, r, l16);
                pi[r] += blk_im(X, g, r, l16);
            }
            blk_store(sT + blk(w, w) * LBLK, pr, pi, l16, g);
        }
    }
    __syncthreads();
    // blocks below the diagonal by distance: T_bc = -T_bb sum_{k=c}^{b-1} M_bk T_kc
    for (int dist = 1; dist < 4; ++dist) {
        const bool mine = w + dist < 4;
        const int bb = w + dist, cc = w;
        if (mine) {
            Gauss x;
            gz(x);
            for (int k = cc; k < bb; ++k) blk_mul_g(x, sM + blk(bb, k) * LBLK, sT + blk(k, cc) * LBLK, l16, g);
            blk_store(sR + w * LBLK, gre(x), gim(x), l16, g);
        }
        __syncthreads();
        if (mine) {
            Gauss x;
            gz(x);
            blk_mul_g(x, sT + blk(bb, bb) * LBLK, sR + w * LBLK, l16, g);
            blk_store(sT + blk(bb, cc) * LBLK, -gre(x), -gim(x), l16, g);
        }
        __syncthreads();
    }
    for (int k = 0; k < NBLK; ++k)
        blk_export(prep + chunk_prep(chain, n_chunks, c) + PREP_T + k * BLK, sT + k * LBLK, tid, 256);
    if (wrec) {
        // T^H in A-operand order: block (rows cc, cols bb) of T^H, element (x, 4 ks + g) =
        // conj(T_(bb, cc)[4 ks + g][x]), stored at T's block index
        for (int e = tid; e < NBLK * BLK; e += 256) {
            const int k = e >> 9, pl = (e >> 8) & 1, idx = e & 255, ln = idx >> 2, ks = idx & 3;
            const int row = ln & 15, gg = ln >> 4;
            const float v = sT[k * LBLK + pl * LPL + (4 * ks + gg) * LP + row];
            wrec[WS_TH + e] = pl ? -v : v;
        }
    }
}

// a [64][64] fp32 complex tile of the chunk (rows past the end zero) in registers:
// thread tid owns row tid / 4, columns 16 (tid % 4) .. + 15
struct TileRegs {
    floatx4 re[4], im[4];
};
__device__ __forceinline__ void tile_fetch(TileRegs &x, const qpam_cview &v, int b, int h, int t0, int valid, int tid,
                                           float scale) {
    const int r = tid >> 2, c0 = 16 * (tid & 3);
    const float *re = static_cast<const float *>(v.re) + b * v.s0 + h * v.s1 + (int64_t)(t0 + min(r, valid - 1)) * v.s2 + c0;
    const float *im = static_cast<const float *>(v.im) + b * v.s0 + h * v.s1 + (int64_t)(t0 + min(r, valid - 1)) * v.s2 + c0;
    const float f = r < valid ? scale : 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        x.re[e] = *reinterpret_cast<const floatx4 *>(re + 4 * e) * f;
        x.im[e] = *reinterpret_cast<const floatx4 *>(im + 4 * e) * f;
    }
}
__device__ __forceinline__ void tile_put(float *sr, float *si, const TileRegs &x, int tid) {
    const int r = tid >> 2, c0 = 16 * (tid & 3);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        *reinterpret_cast<floatx4 *>(sr + r * KP + c0 + 4 * e) = x.re[e];
        *reinterpret_cast<floatx4 *>(si + r * KP + c0 + 4 * e) = x.im[e];
    }
}
// the A-operand blocks (w, 0..w) of one prepared matrix: 4 k-elements per lane and plane
struct OpRegs {
    floatx4 re[4], im[4];
};
__device__ __forceinline__ void ops_fetch(OpRegs &x, const float *base, int w, int lane) {
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
        if (cc <= w) {
            const float *p = base + blk(w, cc) * BLK;
            x.re[cc] = *reinterpret_cast<const floatx4 *>(p + lane * 4);
            x.im[cc] = *reinterpret_cast<const floatx4 *>(p + 256 + lane * 4);
        }
    }
}

__global__ void __launch_bounds__(256, 2) delta_chunk_kernel(qpam_delta_args a, const float *prep, int n_chunks) {
    __shared__ __align__(16) float sKQr[CH * KP], sKQi[CH * KP];   // K, then q_scale Q, of the chunk
    __shared__ __align__(16) float sUr[CH * SP], sUi[CH * SP];     // W, then U  [t][i]
    __shared__ __align__(16) float sSr[2][CH * SP], sSi[2][CH * SP];  // S^T [j][i], entering / next
    __shared__ float sL[CH], sBt[CH];
    const int n_chains = a.B * a.H;
    const int chain = blockIdx.x % n_chains, rblk = blockIdx.x / n_chains;  // a chain's blocks share an XCD
    const int b = chain / a.H, h = chain % a.H;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int i0 = 16 * rblk;  // the block's value rows
    // the backward's records of this chain: entering states and U
    float *wrec = a.workspace ? static_cast<float *>(a.workspace) + (int64_t)chain * n_chunks * WS_REC : nullptr;

    for (int idx = tid; idx < CH * 16; idx += 256) {  // S0^T
        const int i = idx & 15, j = idx >> 4;
        const int64_t o = (int64_t)chain * D * D + (i0 + i) * D + j;
        sSr[0][j * SP + i] = a.s0_re ? a.s0_re[o] : 0.f;
        sSi[0][j * SP + i] = a.s0_re ? a.s0_im[o] : 0.f;
    }
    TileRegs xr;
    tile_fetch(xr, a.k, b, h, 0, min(chunk_len(a), a.T), tid, 1.f);
    // V of this lane's W elements and the T blocks of the chunk: loaded one chunk ahead
    float vr4[4], vi4[4];
    OpRegs opT;
    auto fetch_vt = [&](int c) {
        const int t0 = c * chunk_len(a), valid = min(chunk_len(a), a.T - t0);
        const float *vre = static_cast<const float *>(a.v.re) + b * a.v.s0 + h * a.v.s1 + i0 + l16;
        const float *vim = static_cast<const float *>(a.v.im) + b * a.v.s0 + h * a.v.s1 + i0 + l16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t o = (int64_t)(t0 + min(16 * w + 4 * g + r, valid - 1)) * a.v.s2;
            vr4[r] = vre[o];
            vi4[r] = vim[o];
        }
        ops_fetch(opT, prep + chunk_prep(chain, n_chunks, c) + PREP_T, w, lane);
    };
    fetch_vt(0);
    float lnext = prep[chunk_prep(chain, n_chunks, 0) + PREP_L + lane];
    float bnext = a.beta[b * a.sg_b + h * a.sg_h + (int64_t)min(lane, a.T - 1) * a.sg_t];
    int cur = 0;
    __syncthreads();
    for (int c = 0; c < n_chunks; ++c) {
        const int t0 = c * chunk_len(a), valid = min(chunk_len(a), a.T - t0);
        const int64_t pc = chunk_prep(chain, n_chunks, c);
        tile_put(sKQr, sKQi, xr, tid);
        if (w == 0) {
            sL[lane] = lnext;
            sBt[lane] = lane < valid ? bnext : 0.f;
        }
        __syncthreads();
        tile_fetch(xr, a.q, b, h, t0, valid, tid, a.q_scale);  // in flight through the state work
        OpRegs ops;
        const int t = 16 * w + l16;  // this lane's row in A-operand reads
        // W[t][i] = beta_t (v_t[i] - alpha_t (K S^T)[t][i]), row tile w
        floatx4 ar, ai;
        {
            Gauss x;
            gz(x);
#pragma unroll 4
            for (int ks = 0; ks < 16; ++ks) {
                const int j = 4 * ks + g;
                gstep(x, sKQr[t * KP + j], sKQi[t * KP + j], sSr[cur][j * SP + l16], sSi[cur][j * SP + l16]);
            }
            ar = gre(x);
            ai = gim(x);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int tr = 16 * w + 4 * g + r;
            const float al = __expf(sL[tr]), bt = sBt[tr];
            sUr[tr * SP + l16] = bt * (vr4[r] - al * ar[r]);
            sUi[tr * SP + l16] = bt * (vi4[r] - al * ai[r]);
        }
        __syncthreads();
        // U = T W, row tile w: sum over column tiles cc <= w
        floatx4 ur, ui;
        {
            Gauss x;
            gz(x);
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                if (cc > w) continue;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int s = 16 * cc + 4 * ks + g;
                    gstep(x, opT.re[cc][ks], opT.im[cc][ks], sUr[s * SP + l16], sUi[s * SP + l16]);
                }
            }
            ur = gre(x);
            ui = gim(x);
        }
        __syncthreads();
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sUr[(16 * w + 4 * g + r) * SP + l16] = ur[r];
            sUi[(16 * w + 4 * g + r) * SP + l16] = ui[r];
        }
        if (wrec) {  // U [t][i] of the block's rows
            float *du = wrec + (int64_t)c * WS_REC + WS_U + i0 + l16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                du[(16 * w + 4 * g + r) * D] = ur[r];
                du[D * D + (16 * w + 4 * g + r) * D] = ui[r];
            }
        }
        __syncthreads();
        const int wy = 3 - w;  // Y row tile: the wave with the most T blocks gets the fewest Ahat blocks
        ops_fetch(ops, prep + pc + PREP_A, wy, lane);  // Ahat, in flight through the state update
        // state update, row tile w of S^T (j = 16 w + 4 g + r, i = l16):
        // S <- alpha_last S + sum_s tail_s u_s (x) conj(k_s), tail_s = alpha_last / (alpha_s + 1e-12)
        {
            floatx4 sr, si;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sr[r] = sSr[cur][(16 * w + 4 * g + r) * SP + l16];
                si[r] = sSi[cur][(16 * w + 4 * g + r) * SP + l16];
            }
            if (wrec) {  // entering state: S[i0 + l16][16 w + 4 g + r], 16-byte pieces
                float *ds = wrec + (int64_t)c * WS_REC + WS_S + (i0 + l16) * D + 16 * w + 4 * g;
                *reinterpret_cast<floatx4 *>(ds) = sr;
                *reinterpret_cast<floatx4 *>(ds + D * D) = si;
            }
            const float atot = __expf(sL[CH - 1]);
            Gauss x;
            gz(x);
#pragma unroll 4
            for (int ks = 0; ks < 16; ++ks) {
                const int s = 4 * ks + g;
                const float wq = write_weight(a, sL[s], sL[CH - 1]);
                // conj(K)^T [j][s] (A) times (tail U)[s][i] (B)
                gstep(x, sKQr[s * KP + 16 * w + l16], -sKQi[s * KP + 16 * w + l16], sUr[s * SP + l16] * wq,
                      sUi[s * SP + l16] * wq);
            }
            sr = atot * sr + gre(x);
            si = atot * si + gim(x);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sSr[cur ^ 1][(16 * w + 4 * g + r) * SP + l16] = sr[r];
                sSi[cur ^ 1][(16 * w + 4 * g + r) * SP + l16] = si[r];
            }
        }
        __syncthreads();  // K no longer read
        tile_put(sKQr, sKQi, xr, tid);
        if (c + 1 < n_chunks) {
            const int cs = chunk_len(a), v1 = min(cs, a.T - t0 - cs);
            tile_fetch(xr, a.k, b, h, t0 + cs, v1, tid, 1.f);
            fetch_vt(c + 1);
            lnext = prep[chunk_prep(chain, n_chunks, c + 1) + PREP_L + lane];
            bnext = a.beta[b * a.sg_b + h * a.sg_h + (int64_t)(t0 + cs + min(lane, v1 - 1)) * a.sg_t];
        }
        __syncthreads();
        // Y = Ahat U + alpha Q~ S^T (entering state), row tile w
        {
            Gauss x;
            gz(x);
#pragma unroll
            for (int cc = 0; cc < 4; ++cc) {
                if (cc > wy) continue;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int s = 16 * cc + 4 * ks + g;
                    gstep(x, ops.re[cc][ks], ops.im[cc][ks], sUr[s * SP + l16], sUi[s * SP + l16]);
                }
            }
            const int ty = 16 * wy + l16;
            const float al = __expf(sL[ty]);
#pragma unroll 4
            for (int ks = 0; ks < 16; ++ks) {
                const int j = 4 * ks + g;
                gstep(x, al * sKQr[ty * KP + j], al * sKQi[ty * KP + j], sSr[cur][j * SP + l16], sSi[cur][j * SP + l16]);
            }
            const floatx4 yr = gre(x), yi = gim(x);
            float *yre = a.y.re + b * a.y.s0 + h * a.y.s1 + i0 + l16;
            float *yim = a.y.im + b * a.y.s0 + h * a.y.s1 + i0 + l16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int tr = 16 * wy + 4 * g + r;
                if (tr < valid) {
                    yre[(int64_t)(t0 + tr) * a.y.s2] = yr[r];
                    yim[(int64_t)(t0 + tr) * a.y.s2] = yi[r];
                }
            }
        }
        __syncthreads();  // before the next chunk's tiles replace Q and U
        cur ^= 1;
    }
    for (int idx = tid; idx < CH * 16; idx += 256) {  // final state from S^T
        const int j = idx & 63, i = idx >> 6;
        const int64_t o = (int64_t)chain * D * D + (i0 + i) * D + j;
        a.s_re[o] = sSr[cur][j * SP + i];
        a.s_im[o] = sSi[cur][j * SP + i];
    }
}

// ---------------------------------------------------------------------------
// Backward over the same 64-step chunks.  With G the gradient of the state after
// a chunk and S the state entering it, the chunk's forward above differentiates to
//     dU = Ahat^H dY + diag(dl) K G^T,   dW = T^H dU,   dv = diag(beta) dW,
//     G_before = A_C G + (diag(alpha) dY)^T conj(Q~) - (diag(alpha beta) dW)^T conj(K)
// (dl_s = tail_s = A_C / (alpha_s + 1e-12), A_C = alpha_last) and
//     dAhat = dY U^H on s <= t,   dM = -dW U^H on s < t,   dP = D.dAhat,   dGk = beta_t D.dM,
//     dq~ = dP K + diag(alpha) dY conj(S),
//     dk  = dP^H Q~ + dGk K + dGk^H K - diag(alpha beta) dW conj(S) + diag(dl) U conj(G),
//     dbeta_t  = Re sum_i conj(v_ti) dW_ti - alpha_t Re sum_j conj(k_tj) (dW conj S)_tj
//                + Re sum_s conj(D.Gk)_ts dM_ts,
//     dalpha_t = Re sum_j conj(q~_tj) (dY conj S)_tj - beta_t Re sum_j conj(k_tj) (dW conj S)_tj,
//     ddl_s = Re sum_j k_sj conj(U conj G)_sj,   dA_C = Re <S, G>,
// and the log-decay gradient dL_t = sum_s E_ts - sum_s E_st + dalpha_t alpha_t
// - ddl_t dl_t alpha_t / (alpha_t + 1e-12), E = (Re(conj(Ahat) dAhat) + beta_t
// Re(conj(D.Gk) dM)) where L_t - L_s <= 0 (D's clamp passes no gradient elsewhere),
// the chunk's last step also taking sum_s ddl_s dl_s + dA_C A_C;
// dgamma_t = sum_{t' >= t} dL_t' / (gamma_t + eps).

// the A-operand blocks (w, bb >= w) of an upper-triangular product (T^H, Ahat^H:
// block (rows w, cols bb) stored at index blk(bb, w))
__device__ __forceinline__ void ops_fetch_up(OpRegs &x, const float *base, int w, int lane) {
#pragma unroll
    for (int bb = 0; bb < 4; ++bb) {
        if (bb >= w) {
            const float *p = base + blk(bb, w) * BLK;
            x.re[bb] = *reinterpret_cast<const floatx4 *>(p + lane * 4);
            x.im[bb] = *reinterpret_cast<const floatx4 *>(p + 256 + lane * 4);
        }
    }
}

__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt / expcnt unconstrained
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) x += __shfl_xor(x, off);
    return x;
}

// delta_bwd_chain_kernel: the first two lines above along the chunks in reverse,
// a block per (b, h) and 16 value rows (rows of G are independent as those of S
// are; a chain's four blocks share an XCD), G^T [j][i] in LDS and each wave's
// column tile of it in registers.  Per chunk: G leaves as the chunk's record,
// X^T = conj(Q~)^T (alpha dY) is formed while K arrives, dU (row tile w) = dl K G^T
// + Ahat^H dY, dW (row tile w) = T^H dU -> the record and dv, then
// G^T <- A_C G^T + X^T - conj(K)^T (alpha beta dW).  The previous chunk's q~, dY,
// L and beta are in flight from the middle of the step.
__global__ void __launch_bounds__(256, 2) delta_bwd_chain_kernel(qpam_delta_bwd_args bw, qpam_delta_args a,
                                                                 int n_chunks) {
    __shared__ __align__(16) float sKQr[CH * KP], sKQi[CH * KP];  // q~, then K, of the chunk
    __shared__ __align__(16) float sYr[CH * SP], sYi[CH * SP];    // dY [t][i] (the block's rows)
    __shared__ __align__(16) float sUr[CH * SP], sUi[CH * SP];    // dU, then alpha beta dW  [t][i]
    __shared__ __align__(16) float sGr[CH * SP], sGi[CH * SP];    // G^T [j][i]
    __shared__ float sL[CH], sA[CH], sBt[CH];
    const int n_chains = a.B * a.H;
    const int chain = blockIdx.x % n_chains, rblk = blockIdx.x / n_chains;
    const int b = chain / a.H, h = chain % a.H;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int i0 = 16 * rblk;
    const float *wsf = static_cast<const float *>(a.workspace) + (int64_t)chain * n_chunks * WS_REC;
    float *bws = static_cast<float *>(bw.workspace) + (int64_t)chain * n_chunks * BW_REC;
    const int n = n_chunks;

    // G^T column tile w: lane holds G[i0 + l16][16 w + 4 g + r]
    floatx4 gR = {0.f, 0.f, 0.f, 0.f}, gI = gR;
    if (bw.ds_re) {
        const int64_t o = (int64_t)chain * D * D + (i0 + l16) * D + 16 * w + 4 * g;
        gR = *reinterpret_cast<const floatx4 *>(bw.ds_re + o);
        gI = *reinterpret_cast<const floatx4 *>(bw.ds_im + o);
    }
    // dY of a chunk for the block's rows: thread -> step tid / 4, columns i0 + 4 (tid % 4) ..
    const int yt = tid >> 2, yc = 4 * (tid & 3);
    floatx4 dyr, dyi;
    auto fetch_dy = [&](int c) {
        const int t0 = c * chunk_len(a), valid = min(chunk_len(a), a.T - t0);
        const int64_t o = b * bw.dy.s0 + h * bw.dy.s1 + (int64_t)(t0 + min(yt, valid - 1)) * bw.dy.s2 + i0 + yc;
        const float f = yt < valid ? 1.f : 0.f;
        dyr = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(bw.dy.re) + o) * f;
        dyi = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(bw.dy.im) + o) * f;
    };
    float lnext = 0.f, bnext = 0.f;
    auto fetch_lb = [&](int c) {  // wave 0: L and beta of chunk c (beta 0 past the end)
        const int t0 = c * chunk_len(a), valid = min(chunk_len(a), a.T - t0);
        lnext = wsf[(int64_t)c * WS_REC + WS_L + lane];
        const float bt = a.beta[b * a.sg_b + h * a.sg_h + (int64_t)(t0 + min(lane, valid - 1)) * a.sg_t];
        bnext = lane < valid ? bt : 0.f;
    };
    TileRegs xr;
    auto stage = [&]() {
        tile_put(sKQr, sKQi, xr, tid);
        *reinterpret_cast<floatx4 *>(sYr + yt * SP + yc) = dyr;
        *reinterpret_cast<floatx4 *>(sYi + yt * SP + yc) = dyi;
        if (w == 0) {
            sL[lane] = lnext;
            sA[lane] = __expf(lnext);
            sBt[lane] = bnext;
        }
    };
    {
        const int t0 = (n - 1) * chunk_len(a);
        tile_fetch(xr, a.q, b, h, t0, min(chunk_len(a), a.T - t0), tid, a.q_scale);
        fetch_dy(n - 1);
        if (w == 0) fetch_lb(n - 1);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        sGr[(16 * w + 4 * g + r) * SP + l16] = gR[r];
        sGi[(16 * w + 4 * g + r) * SP + l16] = gI[r];
    }
    stage();
    __syncthreads();

    for (int c = n - 1; c >= 0; --c) {
        const int t0 = c * chunk_len(a), valid = min(chunk_len(a), a.T - t0);
        const float *rec = wsf + (int64_t)c * WS_REC;
        float *brec = bws + (int64_t)c * BW_REC;
        {  // G after this chunk -> the record (16-byte pieces of rows i0 + l16)
            float *dg = brec + BW_G + (i0 + l16) * D + 16 * w + 4 * g;
            *reinterpret_cast<floatx4 *>(dg) = gR;
            *reinterpret_cast<floatx4 *>(dg + D * D) = gI;
        }
        tile_fetch(xr, a.k, b, h, t0, valid, tid, 1.f);  // K, in flight through X
        OpRegs ah, th;
        ops_fetch_up(ah, rec + WS_AH, w, lane);
        ops_fetch_up(th, rec + WS_TH, w, lane);
        // X^T[j][i] = sum_t conj(q~_t[j]) alpha_t dY[t][i], column tile w
        Gauss xq;
        gz(xq);
#pragma unroll 4
        for (int ks = 0; ks < 16; ++ks) {
            const int t = 4 * ks + g;
            const float al = sA[t];
            gstep(xq, sKQr[t * KP + 16 * w + l16], -sKQi[t * KP + 16 * w + l16], al * sYr[t * SP + l16],
                  al * sYi[t * SP + l16]);
        }
        __syncthreads();  // q~ no longer read
        tile_put(sKQr, sKQi, xr, tid);
        if (c > 0) {  // the previous (full) chunk's q~, dY, L and beta, in flight through the rest
            tile_fetch(xr, a.q, b, h, t0 - chunk_len(a), chunk_len(a), tid, a.q_scale);
            fetch_dy(c - 1);
            if (w == 0) fetch_lb(c - 1);
        }
        __syncthreads();
        const float Llast = sL[CH - 1];
        // dU[s][i] = dl_s sum_j K[s][j] G^T[j][i] + sum_{t >= s} conj(Ahat[t][s]) dY[t][i], row tile w
        {
            Gauss x;
            gz(x);
#pragma unroll 4
            for (int ks = 0; ks < 16; ++ks) {
                const int j = 4 * ks + g;
                gstep(x, sKQr[(16 * w + l16) * KP + j], sKQi[(16 * w + l16) * KP + j], sGr[j * SP + l16],
                      sGi[j * SP + l16]);
            }
            floatx4 ur = gre(x), ui = gim(x);
            const float atot = __expf(Llast);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float tl = write_weight(a, sL[16 * w + 4 * g + r], Llast);  // the state-write weight
                ur[r] *= tl;
                ui[r] *= tl;
            }
            Gauss y;
            gz(y);
#pragma unroll
            for (int bt = 0; bt < 4; ++bt) {
                if (bt < w) continue;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int t = 16 * bt + 4 * ks + g;
                    gstep(y, ah.re[bt][ks], ah.im[bt][ks], sYr[t * SP + l16], sYi[t * SP + l16]);
                }
            }
            ur += gre(y);
            ui += gim(y);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sUr[(16 * w + 4 * g + r) * SP + l16] = ur[r];
                sUi[(16 * w + 4 * g + r) * SP + l16] = ui[r];
            }
        }
        __syncthreads();
        // dW[t][i] = sum_{s >= t} conj(T[s][t]) dU[s][i], row tile w
        floatx4 wr, wi;
        {
            Gauss x;
            gz(x);
#pragma unroll
            for (int bs = 0; bs < 4; ++bs) {
                if (bs < w) continue;
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int s = 16 * bs + 4 * ks + g;
                    gstep(x, th.re[bs][ks], th.im[bs][ks], sUr[s * SP + l16], sUi[s * SP + l16]);
                }
            }
            wr = gre(x);
            wi = gim(x);
        }
        {  // dW -> the record; dv = beta dW
            float *dw = brec + BW_W + i0 + l16;
            float *dvr = bw.dv.re + b * bw.dv.s0 + h * bw.dv.s1 + i0 + l16;
            float *dvi = bw.dv.im + b * bw.dv.s0 + h * bw.dv.s1 + i0 + l16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * w + 4 * g + r;
                dw[t * D] = wr[r];
                dw[D * D + t * D] = wi[r];
                if (t < valid) {
                    const float bt = sBt[t];
                    dvr[(int64_t)(t0 + t) * bw.dv.s2] = bt * wr[r];
                    dvi[(int64_t)(t0 + t) * bw.dv.s2] = bt * wi[r];
                }
            }
        }
        __syncthreads();  // dU no longer read
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int t = 16 * w + 4 * g + r;
            const float ab = sA[t] * sBt[t];
            sUr[t * SP + l16] = ab * wr[r];
            sUi[t * SP + l16] = ab * wi[r];
        }
        __syncthreads();
        // G^T <- A_C G^T + X^T - sum_t conj(k_t[j]) alpha_t beta_t dW[t][i], column tile w
        {
            Gauss x;
            gz(x);
#pragma unroll 4
            for (int ks = 0; ks < 16; ++ks) {
                const int t = 4 * ks + g;
                gstep(x, sKQr[t * KP + 16 * w + l16], -sKQi[t * KP + 16 * w + l16], sUr[t * SP + l16],
                      sUi[t * SP + l16]);
            }
            const float ac = __expf(Llast);
            gR = ac * gR + gre(xq) - gre(x);
            gI = ac * gI + gim(xq) - gim(x);
        }
        __syncthreads();  // K, dY, alpha beta dW and the old G^T no longer read
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            sGr[(16 * w + 4 * g + r) * SP + l16] = gR[r];
            sGi[(16 * w + 4 * g + r) * SP + l16] = gI[r];
        }
        if (c > 0) stage();
        __syncthreads();
    }
    if (bw.ds0_re) {
        const int64_t o = (int64_t)chain * D * D + (i0 + l16) * D + 16 * w + 4 * g;
        *reinterpret_cast<floatx4 *>(bw.ds0_re + o) = gR;
        *reinterpret_cast<floatx4 *>(bw.ds0_im + o) = gI;
    }
}

// delta_bwd_score_kernel: the score-matrix gradients of one chunk (a block per
// (b, h, chunk), 4 waves).  U is staged in LDS; wave w forms dAhat on query tile
// w and dM on query tile 3 - w (five 16 x 16 blocks either way), its dY and dW
// rows straight from global memory as MFMA operands (k = i in the order
// 16 q + 4 g + r: 16-byte loads), U rows as 16-byte LDS reads.  dP and dGk leave
// in both layouts (a 16 x 16 LDS transpose per block and wave); E's row sums and
// the beta part complete in the wave, its column sums per block through LDS,
// added in a fixed order.
__global__ void __launch_bounds__(256) delta_bwd_score_kernel(qpam_delta_bwd_args bw, qpam_delta_args a,
                                                              int n_chunks) {
    __shared__ __align__(16) float sUr[CH * KP], sUi[CH * KP];  // U [s][i]
    __shared__ float sX[4][2][16 * 17];                         // each wave's transpose of one block
    __shared__ float sRow[2][CH], sCol[2][4][CH], sDb[CH], sL[CH], sBt[CH];
    const int chain = blockIdx.x / n_chunks, c = blockIdx.x % n_chunks;
    const int b = chain / a.H, h = chain % a.H;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int t0 = c * chunk_len(a), valid = min(chunk_len(a), a.T - t0);
    const float *rec = static_cast<const float *>(a.workspace) + ((int64_t)chain * n_chunks + c) * WS_REC;
    float *brec = static_cast<float *>(bw.workspace) + ((int64_t)chain * n_chunks + c) * BW_REC;
    // this lane's MFMA A rows: dY of step 16 w + l16, dW of step 16 (3 - w) + l16;
    // element (q, r) is column 16 q + 4 g + r
    floatx4 opr[2][4], opi[2][4];
    {
        const int t = 16 * w + l16;
        const float f = t < valid ? 1.f : 0.f;
        const int64_t o = b * bw.dy.s0 + h * bw.dy.s1 + (int64_t)(t0 + min(t, valid - 1)) * bw.dy.s2 + 4 * g;
        const float *dw = brec + BW_W + (16 * (3 - w) + l16) * D + 4 * g;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            opr[0][q] = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(bw.dy.re) + o + 16 * q) * f;
            opi[0][q] = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(bw.dy.im) + o + 16 * q) * f;
            opr[1][q] = *reinterpret_cast<const floatx4 *>(dw + 16 * q);
            opi[1][q] = *reinterpret_cast<const floatx4 *>(dw + D * D + 16 * q);
        }
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {  // U -> LDS, 16-byte pieces
        const int e = tid + 256 * k, pl = e >> 10, row = (e >> 4) & 63, c4 = 4 * (e & 15);
        const floatx4 v = *reinterpret_cast<const floatx4 *>(rec + WS_U + pl * D * D + row * D + c4);
        *reinterpret_cast<floatx4 *>((pl ? sUi : sUr) + row * KP + c4) = v;
    }
    if (w == 0) {
        sL[lane] = rec[WS_L + lane];
        const float bt = a.beta[b * a.sg_b + h * a.sg_h + (int64_t)(t0 + min(lane, valid - 1)) * a.sg_t];
        sBt[lane] = lane < valid ? bt : 0.f;
    }
    __syncthreads();

    float rowacc[2][4], db2[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) rowacc[0][r] = rowacc[1][r] = db2[r] = 0.f;
    float *X = sX[w][0], *Xi = sX[w][1];
#pragma unroll
    for (int kind = 0; kind < 2; ++kind) {
        const int tt = kind ? 3 - w : w;  // query tile of this product
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            if (st > tt) continue;
            const int s = 16 * st + l16;
            // acc[t = 16 tt + 4 g + r][s] = sum_i A[t][i] conj(U[s][i])
            Gauss x;
            gz(x);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const floatx4 ur4 = *reinterpret_cast<const floatx4 *>(sUr + s * KP + 16 * q + 4 * g);
                const floatx4 ui4 = *reinterpret_cast<const floatx4 *>(sUi + s * KP + 16 * q + 4 * g);
#pragma unroll
                for (int r = 0; r < 4; ++r) gstep(x, opr[kind][q][r], opi[kind][q][r], ur4[r], -ui4[r]);
            }
            const floatx4 dr = gre(x), di = gim(x);
            const float *src = rec + (kind ? WS_GA : WS_AA) + blk(tt, st) * BLK + lane * 4;
            const floatx4 xr4 = *reinterpret_cast<const floatx4 *>(src);       // Ahat or D.Gk
            const floatx4 xi4 = *reinterpret_cast<const floatx4 *>(src + 256);
            const float Ls = sL[s];
            floatx4 pr, pi;
            float cs = 0.f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * tt + 4 * g + r;
                const bool keep = kind ? (s < t) : (s <= t);
                const float lx = sL[t] - Ls;
                const float Dv = keep ? __expf(fminf(lx, 0.f)) : 0.f;
                const float through = lx <= 0.f ? 1.f : 0.f;  // D's clamp: no gradient to L past it
                float e;
                if (kind == 0) {  // dP = D dAhat; E = Re(conj(Ahat) dAhat)
                    pr[r] = Dv * dr[r];
                    pi[r] = Dv * di[r];
                    e = through * (xr4[r] * dr[r] + xi4[r] * di[r]);
                } else {  // dM = -acc; dGk = beta D dM; E = beta Re(conj(D.Gk) dM)
                    const float bt = sBt[t];
                    const float e2 = -(xr4[r] * dr[r] + xi4[r] * di[r]);
                    pr[r] = -bt * Dv * dr[r];
                    pi[r] = -bt * Dv * di[r];
                    e = through * bt * e2;
                    db2[r] += e2;
                }
                rowacc[kind][r] += e;
                cs += e;
            }
            cs += __shfl_xor(cs, 16);
            cs += __shfl_xor(cs, 32);
            if (g == 0) sCol[kind][tt][s] = cs;
            // x_K layout: the accumulator order
            float *dk_ = brec + (kind ? BW_GK : BW_PK) + blk(tt, st) * BLK + lane * 4;
            *reinterpret_cast<floatx4 *>(dk_) = pr;
            *reinterpret_cast<floatx4 *>(dk_ + 256) = pi;
            // x_Q layout: lane (l16 = t, g), r <-> s = 4 g + r, through the wave's LDS block
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                X[(4 * g + r) * 17 + l16] = pr[r];
                Xi[(4 * g + r) * 17 + l16] = pi[r];
            }
            wave_lds_sync();
            floatx4 qr4, qi4;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                qr4[r] = X[l16 * 17 + 4 * g + r];
                qi4[r] = Xi[l16 * 17 + 4 * g + r];
            }
            float *dq_ = brec + (kind ? BW_GQ : BW_PQ) + blk(tt, st) * BLK + lane * 4;
            *reinterpret_cast<floatx4 *>(dq_) = qr4;
            *reinterpret_cast<floatx4 *>(dq_ + 256) = qi4;
            wave_lds_sync();
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const float v0 = row16_sum(rowacc[0][r]), v1 = row16_sum(rowacc[1][r]), vb = row16_sum(db2[r]);
        if (l16 == 0) {
            sRow[0][16 * w + 4 * g + r] = v0;
            sRow[1][16 * (3 - w) + 4 * g + r] = v1;
            sDb[16 * (3 - w) + 4 * g + r] = vb;
        }
    }
    __syncthreads();
    if (tid < CH) {
        const int t = tid;
        float col = 0.f;
#pragma unroll
        for (int kind = 0; kind < 2; ++kind)
            for (int tt = t >> 4; tt < 4; ++tt) col += sCol[kind][tt][t];
        brec[BW_V + t] = sRow[0][t] + sRow[1][t] - col;
        brec[BW_V + CH + t] = sDb[t];
    }
}

// delta_bwd_grad_kernel: dq, dk, dgamma and dbeta of one chunk (a block per
// (b, h, chunk), 8 waves).  K, q~, S and G are staged in LDS (pitch KP: the
// MFMA reads of rows 4 g + r, 16 consecutive columns, hit distinct banks); waves
// 0-3 take query tile w: dq~ = dP K + alpha dY conj(S) and the t-side part of dk,
// dGk K - alpha beta dW conj(S); waves 4-7 key tile w: dP^H q~ + dGk^H K +
// dl U conj(G).  Outputs accumulate transposed (a lane holds one step and four
// consecutive columns, so rows leave as 16-byte pieces), with the lane's own
// operands (dP, dGk blocks in the matching layout, dY, dW, U rows) straight from
// global memory.  The key side stores its part of dk and the query side adds
// its own after a barrier; the per-step sums (dalpha, dbeta, ddl) and Re<S, G>
// meet in LDS, and wave 4 forms dL, its reverse cumsum and dgamma.
constexpr int G2_TILE = 2 * CH * KP;
constexpr size_t G2_SMEM = (size_t)(4 * G2_TILE + 7 * CH + 8) * sizeof(float);

__global__ void __launch_bounds__(512) delta_bwd_grad_kernel(qpam_delta_bwd_args bw, qpam_delta_args a,
                                                             int n_chunks) {
    extern __shared__ __align__(16) float sm[];
    float *sK = sm, *sQ = sK + G2_TILE, *sS = sQ + G2_TILE, *sG = sS + G2_TILE;  // [plane][row][KP]
    float *sL = sG + G2_TILE, *sBt = sL + CH, *sLp = sBt + CH, *sDb2 = sLp + CH;
    float *sDa = sDb2 + CH, *sDb = sDa + CH, *sDdl = sDb + CH, *sRed = sDdl + CH;
    const int chain = blockIdx.x / n_chunks, c = blockIdx.x % n_chunks;
    const int b = chain / a.H, h = chain % a.H;
    const int tid = threadIdx.x, wv = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int w = wv & 3;
    const bool qside = wv < 4;
    const int t0 = c * chunk_len(a), valid = min(chunk_len(a), a.T - t0);
    const float *rec = static_cast<const float *>(a.workspace) + ((int64_t)chain * n_chunks + c) * WS_REC;
    const float *brec = static_cast<const float *>(bw.workspace) + ((int64_t)chain * n_chunks + c) * BW_REC;
    constexpr int PL = CH * KP;  // offset of the im plane in a staged tile
    // stage K, q~ (rows past the end zero), S and G: 16 16-byte pieces per thread
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        const int e = tid + 512 * k, m = e >> 11, pl = (e >> 10) & 1, row = (e >> 4) & 63, c4 = 4 * (e & 15);
        floatx4 v;
        if (m < 2) {
            const qpam_cview &x = m ? a.q : a.k;
            const float *base = static_cast<const float *>(pl ? x.im : x.re);
            const float f = row < valid ? (m ? a.q_scale : 1.f) : 0.f;
            v = *reinterpret_cast<const floatx4 *>(base + b * x.s0 + h * x.s1 +
                                                   (int64_t)(t0 + min(row, valid - 1)) * x.s2 + c4) * f;
        } else {
            const float *src = (m == 2 ? rec + WS_S : brec + BW_G) + pl * D * D;
            v = *reinterpret_cast<const floatx4 *>(src + row * D + c4);
        }
        *reinterpret_cast<floatx4 *>(sm + m * G2_TILE + pl * PL + row * KP + c4) = v;
    }
    if (wv == 0) {
        sL[lane] = rec[WS_L + lane];
        const float bt = a.beta[b * a.sg_b + h * a.sg_h + (int64_t)(t0 + min(lane, valid - 1)) * a.sg_t];
        sBt[lane] = lane < valid ? bt : 0.f;
        sLp[lane] = brec[BW_V + lane];
        sDb2[lane] = brec[BW_V + CH + lane];
    }
    __syncthreads();
    {  // Re<S, G>: this thread's 8 elements, summed per wave
        float part = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int e = tid + 512 * k, row = e >> 6, col = e & 63;
            part += sS[row * KP + col] * sG[row * KP + col] + sS[PL + row * KP + col] * sG[PL + row * KP + col];
        }
        part = wave_sum(part);
        if (lane == 0) sRed[wv] = part;
    }

    floatx4 xkr[4], xki[4];  // the query side's part of dk, [column tile]
    if (qside) {
        const int t = 16 * w + l16;  // this lane's step
        const float al = __expf(sL[t]), bt = sBt[t];
        const float *opbase;
        floatx4 orr[4], oi[4], pr[4], pi[4];
        {  // dY rows (zero past the end) and the dP blocks (w, st <= w) in x_Q layout
            const float f = t < valid ? 1.f : 0.f;
            const int64_t o = b * bw.dy.s0 + h * bw.dy.s1 + (int64_t)(t0 + min(t, valid - 1)) * bw.dy.s2 + 4 * g;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                orr[q] = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(bw.dy.re) + o + 16 * q) * f;
                oi[q] = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(bw.dy.im) + o + 16 * q) * f;
            }
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                if (st > w) continue;
                opbase = brec + BW_PQ + blk(w, st) * BLK + lane * 4;
                pr[st] = *reinterpret_cast<const floatx4 *>(opbase);
                pi[st] = *reinterpret_cast<const floatx4 *>(opbase + 256);
            }
        }
        float dal = 0.f;
        float *dqr = bw.dq.re + b * bw.dq.s0 + h * bw.dq.s1 + (int64_t)(t0 + t) * bw.dq.s2;
        float *dqi = bw.dq.im + b * bw.dq.s0 + h * bw.dq.s1 + (int64_t)(t0 + t) * bw.dq.s2;
#pragma unroll 1  // (unrolled, the compiler keeps every column tile's operands live and spills)
        for (int jt = 0; jt < 4; ++jt) {
            const int j = 16 * jt + l16;
            // sum_s K[s][j] dP[t][s]  (k = s = 16 st + 4 g + r)
            Gauss x;
            gz(x);
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                if (st > w) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int s = 16 * st + 4 * g + r;
                    gstep(x, sK[s * KP + j], sK[PL + s * KP + j], pr[st][r], pi[st][r]);
                }
            }
            // YS^T[j][t] = sum_i conj(S[i][j]) dY[t][i]  (k = i = 16 q + 4 g + r)
            Gauss y;
            gz(y);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int i = 16 * q + 4 * g + r;
                    gstep(y, sS[i * KP + j], -sS[PL + i * KP + j], orr[q][r], oi[q][r]);
                }
            const floatx4 ysr = gre(y), ysi = gim(y);
            const floatx4 qr4 = *reinterpret_cast<const floatx4 *>(sQ + t * KP + 16 * jt + 4 * g);
            const floatx4 qi4 = *reinterpret_cast<const floatx4 *>(sQ + PL + t * KP + 16 * jt + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; ++r) dal += qr4[r] * ysr[r] + qi4[r] * ysi[r];
            if (t < valid) {
                *reinterpret_cast<floatx4 *>(dqr + 16 * jt + 4 * g) = (gre(x) + al * ysr) * a.q_scale;
                *reinterpret_cast<floatx4 *>(dqi + 16 * jt + 4 * g) = (gim(x) + al * ysi) * a.q_scale;
            }
        }
        {  // dW rows and the dGk blocks (w, st <= w) in x_Q layout
            const float *dw = brec + BW_W + t * D + 4 * g;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                orr[q] = *reinterpret_cast<const floatx4 *>(dw + 16 * q);
                oi[q] = *reinterpret_cast<const floatx4 *>(dw + D * D + 16 * q);
            }
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                if (st > w) continue;
                opbase = brec + BW_GQ + blk(w, st) * BLK + lane * 4;
                pr[st] = *reinterpret_cast<const floatx4 *>(opbase);
                pi[st] = *reinterpret_cast<const floatx4 *>(opbase + 256);
            }
        }
        float dk2 = 0.f;
#pragma unroll
        for (int jt = 0; jt < 4; ++jt) {
            const int j = 16 * jt + l16;
            Gauss x;  // sum_s K[s][j] dGk[t][s]
            gz(x);
#pragma unroll
            for (int st = 0; st < 4; ++st) {
                if (st > w) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int s = 16 * st + 4 * g + r;
                    gstep(x, sK[s * KP + j], sK[PL + s * KP + j], pr[st][r], pi[st][r]);
                }
            }
            Gauss y;  // WS^T[j][t] = sum_i conj(S[i][j]) dW[t][i]
            gz(y);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int i = 16 * q + 4 * g + r;
                    gstep(y, sS[i * KP + j], -sS[PL + i * KP + j], orr[q][r], oi[q][r]);
                }
            const floatx4 wsr = gre(y), wsi = gim(y);
            const floatx4 kr4 = *reinterpret_cast<const floatx4 *>(sK + t * KP + 16 * jt + 4 * g);
            const floatx4 ki4 = *reinterpret_cast<const floatx4 *>(sK + PL + t * KP + 16 * jt + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; ++r) dk2 += kr4[r] * wsr[r] + ki4[r] * wsi[r];
            xkr[jt] = gre(x) - (al * bt) * wsr;
            xki[jt] = gim(x) - (al * bt) * wsi;
        }
        float dba = 0.f;  // Re sum_i conj(v[t][i]) dW[t][i]
        {
            const int64_t o = b * a.v.s0 + h * a.v.s1 + (int64_t)(t0 + min(t, valid - 1)) * a.v.s2 + 4 * g;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const floatx4 vr4 = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(a.v.re) + o + 16 * q);
                const floatx4 vi4 = *reinterpret_cast<const floatx4 *>(static_cast<const float *>(a.v.im) + o + 16 * q);
#pragma unroll
                for (int r = 0; r < 4; ++r) dba += vr4[r] * orr[q][r] + vi4[r] * oi[q][r];
            }
        }
        dal += __shfl_xor(dal, 16);
        dal += __shfl_xor(dal, 32);
        dk2 += __shfl_xor(dk2, 16);
        dk2 += __shfl_xor(dk2, 32);
        dba += __shfl_xor(dba, 16);
        dba += __shfl_xor(dba, 32);
        if (g == 0) {
            sDa[t] = dal - bt * dk2;
            sDb[t] = dba - al * dk2;
        }
    } else {
        const int s = 16 * w + l16;  // this lane's step (key side)
        const float dl = write_weight(a, sL[s], sL[CH - 1]);  // the state-write weight
        float *dkr = bw.dk.re + b * bw.dk.s0 + h * bw.dk.s1 + (int64_t)(t0 + s) * bw.dk.s2;
        float *dki = bw.dk.im + b * bw.dk.s0 + h * bw.dk.s1 + (int64_t)(t0 + s) * bw.dk.s2;
        floatx4 urr[4], ui[4], pr[4], pi[4], hr[4], hi[4];
        {  // U rows; dP, dGk blocks (tt >= w, w) in x_K layout
            const float *du = rec + WS_U + s * D + 4 * g;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                urr[q] = *reinterpret_cast<const floatx4 *>(du + 16 * q);
                ui[q] = *reinterpret_cast<const floatx4 *>(du + D * D + 16 * q);
            }
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                if (tt < w) continue;
                const float *p = brec + BW_PK + blk(tt, w) * BLK + lane * 4;
                const float *q = brec + BW_GK + blk(tt, w) * BLK + lane * 4;
                pr[tt] = *reinterpret_cast<const floatx4 *>(p);
                pi[tt] = *reinterpret_cast<const floatx4 *>(p + 256);
                hr[tt] = *reinterpret_cast<const floatx4 *>(q);
                hi[tt] = *reinterpret_cast<const floatx4 *>(q + 256);
            }
        }
        float ddl = 0.f;
#pragma unroll 1  // (unrolled, the compiler keeps every column tile's operands live and spills)
        for (int jt = 0; jt < 4; ++jt) {
            const int j = 16 * jt + l16;
            // sum_t q~[t][j] conj(dP[t][s]) + K[t][j] conj(dGk[t][s])  (k = t = 16 tt + 4 g + r)
            Gauss x;
            gz(x);
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                if (tt < w) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int t = 16 * tt + 4 * g + r;
                    gstep(x, sQ[t * KP + j], sQ[PL + t * KP + j], pr[tt][r], -pi[tt][r]);
                    gstep(x, sK[t * KP + j], sK[PL + t * KP + j], hr[tt][r], -hi[tt][r]);
                }
            }
            // UG^T[j][s] = sum_i conj(G[i][j]) U[s][i]
            Gauss y;
            gz(y);
#pragma unroll
            for (int q = 0; q < 4; ++q)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int i = 16 * q + 4 * g + r;
                    gstep(y, sG[i * KP + j], -sG[PL + i * KP + j], urr[q][r], ui[q][r]);
                }
            const floatx4 ugr = gre(y), ugi = gim(y);
            const floatx4 kr4 = *reinterpret_cast<const floatx4 *>(sK + s * KP + 16 * jt + 4 * g);
            const floatx4 ki4 = *reinterpret_cast<const floatx4 *>(sK + PL + s * KP + 16 * jt + 4 * g);
#pragma unroll
            for (int r = 0; r < 4; ++r) ddl += kr4[r] * ugr[r] + ki4[r] * ugi[r];
            if (s < valid) {  // the key side's part of dk; the query side adds its part below
                *reinterpret_cast<floatx4 *>(dkr + 16 * jt + 4 * g) = gre(x) + dl * ugr;
                *reinterpret_cast<floatx4 *>(dki + 16 * jt + 4 * g) = gim(x) + dl * ugi;
            }
        }
        ddl += __shfl_xor(ddl, 16);
        ddl += __shfl_xor(ddl, 32);
        if (g == 0) sDdl[s] = ddl;
    }
    __syncthreads();  // the key side's dk rows are written (and visible to the block)
    if (qside) {
        const int t = 16 * w + l16;
        if (t < valid) {
            float *dkr = bw.dk.re + b * bw.dk.s0 + h * bw.dk.s1 + (int64_t)(t0 + t) * bw.dk.s2 + 4 * g;
            float *dki = bw.dk.im + b * bw.dk.s0 + h * bw.dk.s1 + (int64_t)(t0 + t) * bw.dk.s2 + 4 * g;
#pragma unroll
            for (int jt = 0; jt < 4; ++jt) {
                *reinterpret_cast<floatx4 *>(dkr + 16 * jt) += xkr[jt];
                *reinterpret_cast<floatx4 *>(dki + 16 * jt) += xki[jt];
            }
        }
    }
    if (wv == 4) {  // lane = step: dL, its reverse cumsum, dgamma and dbeta
        const int t = lane;
        const float Lt = sL[t], Llast = sL[CH - 1];
        const float al = __expf(Lt), atot = __expf(Llast), dl = write_weight(a, Lt, Llast);
        const bool tv = t < valid;
        float x = tv ? sLp[t] + sDa[t] * al - sDdl[t] * dl * write_weight_dl(a, Lt) : 0.f;
        const float tot = wave_sum(tv ? sDdl[t] * dl : 0.f);
        float dac = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) dac += sRed[k];
        if (t == valid - 1) x += tot + dac * atot;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float y = __shfl_down(x, off);
            if (lane + off < 64) x += y;
        }
        if (tv) {
            const int64_t go = b * a.sg_b + h * a.sg_h + (int64_t)(t0 + t) * a.sg_t;
            bw.dgamma[go] = x / fmaxf(a.gamma[go] + a.gamma_eps, 1.17549435e-38f);  // as decay_log
            bw.dbeta[go] = sDb[t] + sDb2[t];
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

size_t n_chunks_of(const qpam_delta_args &a) { return (size_t)((a.T + chunk_len(a) - 1) / chunk_len(a)); }
size_t fwd_ws(const qpam_delta_args &a) { return (size_t)a.B * a.H * n_chunks_of(a) * WS_REC * sizeof(float); }
size_t prep_bytes(const qpam_delta_args &a) { return (size_t)a.B * a.H * n_chunks_of(a) * PREP_FLOATS * sizeof(float); }
size_t bwd_ws(const qpam_delta_args &a) { return (size_t)a.B * a.H * n_chunks_of(a) * BW_REC * sizeof(float); }

int validate(const qpam_delta_args *a) {
    QPAM_REQUIRE(a != nullptr, "qpam_delta: null arguments");
    QPAM_REQUIRE(a->B >= 0 && a->H >= 1 && a->T >= 0, "qpam_delta: invalid sizes B=%d H=%d T=%d", a->B, a->H, a->T);
    QPAM_REQUIRE(a->d == D, "qpam_delta: head_dim %d unsupported (64 only)", a->d);
    QPAM_REQUIRE(a->chunk >= 0 && a->chunk <= CH, "qpam_delta: chunk %d outside 1..%d (0 = %d)", a->chunk, CH, CH);
    QPAM_REQUIRE(a->exact_write == 0 || a->exact_write == 1, "qpam_delta: exact_write must be 0 or 1");
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

extern "C" size_t qpam_delta_scratch_size(const qpam_delta_args *a) { return a ? prep_bytes(*a) : 0; }

extern "C" int qpam_delta_fwd(const qpam_delta_args *a, void *stream) {
    int st = validate(a);
    if (st) return st;
    QPAM_REQUIRE(mview_ok(a->y) && a->s_re && a->s_im && aligned(a->s_re, 16) && aligned(a->s_im, 16),
                 "qpam_delta_fwd: y (16-byte aligned planes) and the final state are required");
    QPAM_REQUIRE(a->workspace == nullptr || (aligned(a->workspace, 16) && a->workspace_bytes >= fwd_ws(*a)),
                 "qpam_delta_fwd: workspace of %zu bytes needed (or NULL without a backward)", fwd_ws(*a));
    if (a->B == 0) return QPAM_OK;
    QPAM_REQUIRE(a->T >= 1, "qpam_delta_fwd: T must be >= 1");
    QPAM_REQUIRE(a->scratch && aligned(a->scratch, 16) && a->scratch_bytes >= prep_bytes(*a),
                 "qpam_delta_fwd: scratch of %zu bytes needed", prep_bytes(*a));
    const int n_chunks = (int)n_chunks_of(*a);
    const int64_t items = (int64_t)a->B * a->H * n_chunks;
    QPAM_REQUIRE(items < (1ll << 31) && (int64_t)a->B * a->H * ROW_BLOCKS < (1ll << 31), "qpam_delta_fwd: grid too large");
    hipStream_t s = static_cast<hipStream_t>(stream);
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)delta_prep_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)PREP_SMEM));
    float *prep = static_cast<float *>(a->scratch);
    hipLaunchKernelGGL(delta_prep_kernel, dim3((unsigned)items), dim3(256), PREP_SMEM, s, *a, prep, n_chunks);
    st = launch_status("delta_prep_kernel");
    if (st) return st;
    hipLaunchKernelGGL(delta_chunk_kernel, dim3((unsigned)(a->B * a->H * ROW_BLOCKS)), dim3(256), 0, s, *a,
                       (const float *)prep, n_chunks);
    return launch_status("delta_chunk_kernel");
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
                 "qpam_delta_bwd: the forward's workspace (its per-chunk records) is required");
    QPAM_REQUIRE(g->workspace && aligned(g->workspace, 16) && g->workspace_bytes >= bwd_ws(a),
                 "qpam_delta_bwd: workspace of %zu bytes needed", bwd_ws(a));
    QPAM_REQUIRE(cview_ok(g->dy) && mview_ok(g->dq) && mview_ok(g->dk) && mview_ok(g->dv),
                 "qpam_delta_bwd: dy, dq, dk, dv must be 16-byte aligned fp32 planes with strides multiple of 4");
    QPAM_REQUIRE(g->dgamma && g->dbeta, "qpam_delta_bwd: dgamma and dbeta required");
    QPAM_REQUIRE((g->ds_re == nullptr) == (g->ds_im == nullptr) && (g->ds0_re == nullptr) == (g->ds0_im == nullptr),
                 "qpam_delta_bwd: ds / ds0 need both planes");
    if (a.B == 0 || a.T == 0) return QPAM_OK;
    const int n_chunks = (int)n_chunks_of(a);
    const int64_t items = (int64_t)a.B * a.H * n_chunks;
    QPAM_REQUIRE(items < (1ll << 31), "qpam_delta_bwd: grid too large");
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(delta_bwd_chain_kernel, dim3((unsigned)(a.B * a.H * ROW_BLOCKS)), dim3(256), 0, s, *g, a,
                       n_chunks);
    st = launch_status("delta_bwd_chain_kernel");
    if (st) return st;
    hipLaunchKernelGGL(delta_bwd_score_kernel, dim3((unsigned)items), dim3(256), 0, s, *g, a, n_chunks);
    st = launch_status("delta_bwd_score_kernel");
    if (st) return st;
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)delta_bwd_grad_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)G2_SMEM));
    hipLaunchKernelGGL(delta_bwd_grad_kernel, dim3((unsigned)items), dim3(512), G2_SMEM, s, *g, a, n_chunks);
    return launch_status("delta_bwd_grad_kernel");
}
