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
// then delta_chunk_kernel along the chunks; described at the kernels), with
// the state before every 16th token stored as the backward's checkpoints.
// The rows of S are independent under the recurrence (row i reads only k, q,
// v_i, gamma, beta), so the chunk pass splits a chain's 64 value rows over four
// blocks.
//
// Backward (token recurrence in registers): a lane owns 1 row x 4 columns of
// S, and the per-row dot products S k and S q~ are DPP reductions over the 16
// lanes of a row group.
// Backward: four workgroups of 4 waves (16 rows each) per chain walk its
// 16-token groups in reverse; each group is recomputed from its checkpoint
// with the state before every 4th token kept in a scratch, then each 4-token
// sub-group is recomputed into registers and differentiated in reverse.
// Gradients of k, q, gamma and beta are sums over the 64 rows: lanes -> row
// groups by shuffles, waves through LDS every 2 tokens, workgroups through
// per-part partial sums that a second kernel adds in a fixed order
// (deterministic).
#include "common.h"

namespace qpam {
namespace {

constexpr int D = 64;
constexpr int RPL = 1;               // rows per lane
constexpr int NW = D / (4 * RPL);    // waves per chain (16)
constexpr int GROUP = 16;            // tokens per forward checkpoint
constexpr int SUB = 4;               // tokens per backward sub-group
constexpr int SUBS = GROUP / SUB;
constexpr int FL = 2;                // tokens per backward cross-wave reduction
constexpr int PARTS = 4;             // backward workgroups per chain
constexpr int PW = NW / PARTS;       // waves per backward workgroup
constexpr int PROWS = 4 * RPL * PW;  // rows per backward workgroup
constexpr int BWD_THREADS = 64 * PW;

struct Lane {
    int w, lane, rg, cg, r0;   // wave of the chain, lane, row group (0..3), column group (0..15), first row
    __device__ Lane(int wave, int ln) {
        w = wave, lane = ln;
        rg = ln >> 4, cg = ln & 15;
        r0 = (4 * w + rg) * RPL;
    }
    __device__ int slot() const { return w * 64 + lane; }   // thread-private state slot of the chain
};

// one token's inputs as this lane sees them
struct Tok {
    float kr[4], ki[4], qr[4], qi[4];  // the lane's 4 columns (q already scaled)
    float vr[RPL], vi[RPL];            // the lane's rows
    float g, b;                        // gamma + eps, beta
};

struct State {
    float r[RPL][4], i[RPL][4];
};

// The inputs of NT consecutive tokens staged in LDS: the k and q planes of
// every column (q scaled), v of the ROWS rows the workgroup owns, gamma + eps
// and beta.  Global loads go to registers first (fetch) and to LDS later
// (commit), so a span's loads overlap the previous span's arithmetic.
template <int NT, int ROWS>
struct Span {
    floatx4 kq[NT][4][16];   // [token][k re, k im, q re, q im][column / 4]
    float v[NT][2][ROWS];
    float gb[NT][2];
};

template <int NT, int ROWS, int NTHR>
struct SpanRegs {
    static constexpr int KQ = NT * 64 / NTHR;                 // float4 per thread
    static constexpr int VV = (NT * 2 * ROWS + NTHR - 1) / NTHR;
    static_assert(KQ >= 1 && KQ * NTHR == NT * 64, "span shape");
    floatx4 kq[KQ];
    float v[VV];
    float gb;

    // rows past T re-read row T - 1 (their results are not stored)
    __device__ __forceinline__ void fetch(const qpam_delta_args &a, int b, int h, int t0, int row0, int tid) {
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
            const int i = tid + k * NTHR, tok = i >> 6, pl = (i >> 4) & 3, c4 = i & 15;
            const int t = min(t0 + tok, a.T - 1);
            const qpam_cview &v = pl < 2 ? a.k : a.q;
            const float *base = static_cast<const float *>((pl & 1) ? v.im : v.re);
            kq[k] = *reinterpret_cast<const floatx4 *>(base + b * v.s0 + h * v.s1 + (int64_t)t * v.s2 + 4 * c4);
            if (pl >= 2) kq[k] *= a.q_scale;
        }
#pragma unroll
        for (int k = 0; k < VV; ++k) {
            const int i = min(tid + k * NTHR, NT * 2 * ROWS - 1);
            const int tok = i / (2 * ROWS), rem = i - tok * 2 * ROWS, ri = rem / ROWS, r = rem - ri * ROWS;
            const int t = min(t0 + tok, a.T - 1);
            const float *base = static_cast<const float *>(ri ? a.v.im : a.v.re);
            v[k] = base[b * a.v.s0 + h * a.v.s1 + (int64_t)t * a.v.s2 + row0 + r];
        }
        const int i = min(tid, 2 * NT - 1), t = min(t0 + (i >> 1), a.T - 1);
        const int64_t go = b * a.sg_b + h * a.sg_h + (int64_t)t * a.sg_t;
        gb = (i & 1) ? a.beta[go] : a.gamma[go] + a.gamma_eps;
    }

    __device__ __forceinline__ void commit(Span<NT, ROWS> &sp, int tid) const {
#pragma unroll
        for (int k = 0; k < KQ; ++k) {
            const int i = tid + k * NTHR;
            sp.kq[i >> 6][(i >> 4) & 3][i & 15] = kq[k];
        }
#pragma unroll
        for (int k = 0; k < VV; ++k) {
            const int i = tid + k * NTHR;
            if (i < NT * 2 * ROWS) {
                const int tok = i / (2 * ROWS), rem = i - tok * 2 * ROWS, ri = rem / ROWS, r = rem - ri * ROWS;
                sp.v[tok][ri][r] = v[k];
            }
        }
        if (tid < 2 * NT) sp.gb[tid >> 1][tid & 1] = gb;
    }
};

// token j of a span as this lane sees it; `row` = the lane's first row in the span's rows
template <int NT, int ROWS>
__device__ __forceinline__ Tok span_tok(const Span<NT, ROWS> &sp, int j, int cg, int row) {
    Tok x;
    const floatx4 kr = sp.kq[j][0][cg], ki = sp.kq[j][1][cg], qr = sp.kq[j][2][cg], qi = sp.kq[j][3][cg];
    x.kr[0] = kr.x, x.kr[1] = kr.y, x.kr[2] = kr.z, x.kr[3] = kr.w;
    x.ki[0] = ki.x, x.ki[1] = ki.y, x.ki[2] = ki.z, x.ki[3] = ki.w;
    x.qr[0] = qr.x, x.qr[1] = qr.y, x.qr[2] = qr.z, x.qr[3] = qr.w;
    x.qi[0] = qi.x, x.qi[1] = qi.y, x.qi[2] = qi.z, x.qi[3] = qi.w;
#pragma unroll
    for (int rr = 0; rr < RPL; ++rr) x.vr[rr] = sp.v[j][0][row + rr], x.vi[rr] = sp.v[j][1][row + rr];
    x.g = sp.gb[j][0], x.b = sp.gb[j][1];
    return x;
}

// One token: S <- g S + u (x) k*, u = b (v - g S k); returns y = S q~ for the
// lane's 2 rows (complete in every lane of the row group).
__device__ __forceinline__ void fwd_step(State &s, const Tok &x, float (&yr)[RPL], float (&yi)[RPL]) {
    float pkr[RPL], pki[RPL], pqr[RPL], pqi[RPL];
#pragma unroll
    for (int rr = 0; rr < RPL; ++rr) {
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
    for (int rr = 0; rr < RPL; ++rr) {
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

// a thread's 8 RPL floats of state at [chain][checkpoint][slot], float4-coalesced
__device__ __forceinline__ void store_state(float *base, const State &s, int slot) {
    floatx4 *p = reinterpret_cast<floatx4 *>(base) + 2 * RPL * slot;
#pragma unroll
    for (int rr = 0; rr < RPL; ++rr) {
        p[2 * rr] = floatx4{s.r[rr][0], s.r[rr][1], s.r[rr][2], s.r[rr][3]};
        p[2 * rr + 1] = floatx4{s.i[rr][0], s.i[rr][1], s.i[rr][2], s.i[rr][3]};
    }
}
__device__ __forceinline__ void load_state(const float *base, State &s, int slot) {
    const floatx4 *p = reinterpret_cast<const floatx4 *>(base) + 2 * RPL * slot;
#pragma unroll
    for (int rr = 0; rr < RPL; ++rr) {
        const floatx4 a = p[2 * rr], b = p[2 * rr + 1];
        s.r[rr][0] = a.x, s.r[rr][1] = a.y, s.r[rr][2] = a.z, s.r[rr][3] = a.w;
        s.i[rr][0] = b.x, s.i[rr][1] = b.y, s.i[rr][2] = b.z, s.i[rr][3] = b.w;
    }
}

__device__ __forceinline__ void init_state(State &s, const float *re, const float *im, int64_t chain, const Lane &L) {
#pragma unroll
    for (int rr = 0; rr < RPL; ++rr) {
        if (re) {
            const int64_t o = chain * D * D + (L.r0 + rr) * D + 4 * L.cg;
            const floatx4 a = *reinterpret_cast<const floatx4 *>(re + o), b = *reinterpret_cast<const floatx4 *>(im + o);
            s.r[rr][0] = a.x, s.r[rr][1] = a.y, s.r[rr][2] = a.z, s.r[rr][3] = a.w;
            s.i[rr][0] = b.x, s.i[rr][1] = b.y, s.i[rr][2] = b.z, s.i[rr][3] = b.w;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) s.r[rr][c] = 0.f, s.i[rr][c] = 0.f;
        }
    }
}

__device__ __forceinline__ void write_state(float *re, float *im, const State &s, int64_t chain, const Lane &L) {
#pragma unroll
    for (int rr = 0; rr < RPL; ++rr) {
        const int64_t o = chain * D * D + (L.r0 + rr) * D + 4 * L.cg;
        *reinterpret_cast<floatx4 *>(re + o) = floatx4{s.r[rr][0], s.r[rr][1], s.r[rr][2], s.r[rr][3]};
        *reinterpret_cast<floatx4 *>(im + o) = floatx4{s.i[rr][0], s.i[rr][1], s.i[rr][2], s.i[rr][3]};
    }
}
constexpr int STATE_FLOATS = 2 * D * D;   // one chain's state, thread-private layout

// backward workspace: sub-group states [chain][SUBS][state], then the parts' partial sums
__host__ __device__ __forceinline__ size_t bwd_sub_bytes(const qpam_delta_args &a) {
    return (size_t)a.B * a.H * SUBS * STATE_FLOATS * sizeof(float);
}

// ---------------------------------------------------------------------------
// Forward over 64-step chunks on fp32 MFMA (v_mfma_f32_16x16x4f32).  Unrolled
// over a chunk, the recurrence is the reference's UT form: with L_t the
// inclusive prefix of log(gamma + eps) from the chunk's start, alpha_t = e^{L_t},
// D[t,s] = e^{L_t - L_s} and S_0 the state entering the chunk,
//     (I + M) U = W,   M[t,s] = beta_t D[t,s] (k_t . conj(k_s))  (s < t),
//     W_t = beta_t (v_t - alpha_t S_0 k_t),
//     y_t = alpha_t S_0 q~_t + sum_{s<=t} D[t,s] (q~_t . conj(k_s)) u_s,
//     S_end = alpha_last S_0 + sum_s D[last,s] u_s (x) conj(k_s).
// delta_prep_kernel (chunk-parallel, a block per (b, h, chunk)) forms everything
// that does not depend on S: the Gram and query-key products, T = (I + M)^{-1}
// (diagonal 16 x 16 blocks by forward substitution, the blocks below them as
// T_bc = -T_bb sum_k M_bk T_kc) and Ahat[t,s] = D[t,s] (q~_t . conj(k_s)), stored
// per chunk in the MFMA A-operand order.  delta_chunk_kernel then walks the
// chunks of one (b, h) for 16 value rows (rows of the recurrence are
// independent: four blocks per chain) with S^T in LDS: W = beta (V - alpha K S^T),
// U = T W, the state update in four 16-step quarters (each quarter's end state is
// the backward's checkpoint before the next 16 steps), then Y = Ahat U + alpha
// Q~ S^T with the chunk's entering state.
constexpr int CH = 64;                 // steps per chunk
constexpr int ROW_BLOCKS = 4;          // blocks per chain in the chunk pass (16 value rows each)
constexpr int KP = CH + 4;             // LDS pitch of [64][64] fp32 tiles read element-wise
constexpr int SP = 16;                 // LDS pitch of [64][16] fp32 tiles
constexpr int NBLK = 10;               // 16 x 16 blocks on and below the diagonal of a 64 x 64 matrix
constexpr int BLK = 2 * 256;           // floats of one complex 16 x 16 block (re plane, then im)
constexpr int PREP_T = 0, PREP_A = NBLK * BLK, PREP_L = 2 * NBLK * BLK;
constexpr int PREP_FLOATS = PREP_L + CH;  // per chunk: T blocks, Ahat blocks, L

__device__ __forceinline__ int blk(int b, int c) { return b * (b + 1) / 2 + c; }  // c <= b

__device__ __forceinline__ floatx4 mfma4(float a, float b, floatx4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void blk_store(float *dst, const floatx4 &cr, const floatx4 &ci, int l16, int g) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        dst[(4 * g + r) * 16 + l16] = cr[r];
        dst[256 + (4 * g + r) * 16 + l16] = ci[r];
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
        dst[e] = src[pl * 256 + row * 16 + 4 * ks + gg];
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
        gstep(x, A[l16 * 16 + k], A[256 + l16 * 16 + k], B[k * 16 + l16], B[256 + k * 16 + l16]);
    }
}
// element (4g + r, l16) of an LDS block, re and im
__device__ __forceinline__ float blk_re(const float *A, int g, int r, int l16) { return A[(4 * g + r) * 16 + l16]; }
__device__ __forceinline__ float blk_im(const float *A, int g, int r, int l16) {
    return A[256 + (4 * g + r) * 16 + l16];
}

// The prep block's LDS: K and q_scale Q of the chunk while the Gram and
// query-key products run; the same bytes then hold M, T and each wave's four
// scratch blocks of the diagonal inversion, whose first three blocks later hold
// the partial sums of the blocks below the diagonal (two blocks per CU).
constexpr int PREP_KQ = 4 * CH * KP;
constexpr int PREP_INV = NBLK * BLK * 2 + 16 * BLK;
constexpr size_t PREP_SMEM = (size_t)((PREP_KQ > PREP_INV ? PREP_KQ : PREP_INV) + 2 * CH) * sizeof(float);

__global__ void __launch_bounds__(256, 2) delta_prep_kernel(qpam_delta_args a, float *prep, int n_chunks) {
    extern __shared__ float sm[];
    float *sKr = sm, *sKi = sKr + CH * KP, *sQr = sKi + CH * KP, *sQi = sQr + CH * KP;
    float *sM = sm;                // after the products: M blocks [blk][re | im][16][16] (diagonal included)
    float *sT = sM + NBLK * BLK;   // T blocks
    float *sX = sT + NBLK * BLK;   // four scratch blocks per wave
    float *sR = sX;                // after the inversion: three partial sums
    const int big = PREP_KQ > PREP_INV ? PREP_KQ : PREP_INV;
    float *sL = sm + big, *sB = sL + CH;
    const int chain = blockIdx.x / n_chunks, c = blockIdx.x % n_chunks;
    const int b = chain / a.H, h = chain % a.H;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int t0 = c * CH, valid = min(CH, a.T - t0);
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
        float x = lane < valid ? logf(a.gamma[go] + a.gamma_eps) : 0.f;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
            const float y = __shfl_up(x, off);
            if (lane >= off) x += y;
        }
        sL[lane] = x;
        sB[lane] = lane < valid ? a.beta[go] : 0.f;
        prep[chunk_prep(chain, n_chunks, c) + PREP_L + lane] = x;
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
            float *Mb = sM + bk * BLK;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * bb + 4 * g + r, s = 16 * cc + l16;
                const float m = s < t ? sB[t] * __expf(sL[t] - sL[s]) : 0.f;
                Mb[(4 * g + r) * 16 + l16] = m * xr[r];
                Mb[256 + (4 * g + r) * 16 + l16] = m * xi[r];
            }
        } else {
            // Ahat in A-operand order: element (row 4g + r, col l16) -> lane (col % 4) * 16 + row, slot col / 4
            float *dst = prep + chunk_prep(chain, n_chunks, c) + PREP_A + bk * BLK;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = 16 * bb + 4 * g + r, s = 16 * cc + l16;
                const float dts = s <= t ? __expf(sL[t] - sL[s]) : 0.f;
                const int ln = (l16 & 3) * 16 + 4 * g + r, ks = l16 >> 2;
                dst[ln * 4 + ks] = dts * xr[r];
                dst[256 + ln * 4 + ks] = dts * xi[r];
            }
        }
    }
    __syncthreads();
    {  // T_bb = (I + N)^{-1} = (I - N)(I + N^2)(I + N^4)(I + N^8), N = M_bb nilpotent (N^16 = 0); wave b
        const float *N = sM + blk(w, w) * BLK;
        float *X = sX + w * 4 * BLK;  // N^2, N^4, N^8, P1 (then P2 over N^2)
        Gauss x;
        gz(x);
        blk_mul_g(x, N, N, l16, g);
        blk_store(X, gre(x), gim(x), l16, g);
        gz(x);
        blk_mul_g(x, X, X, l16, g);
        blk_store(X + BLK, gre(x), gim(x), l16, g);
        gz(x);
        blk_mul_g(x, X + BLK, X + BLK, l16, g);
        blk_store(X + 2 * BLK, gre(x), gim(x), l16, g);
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
            blk_store(X + 3 * BLK, pr, pi, l16, g);
        }
        // P2 = P1 + P1 N^4 (over N^2)
        gz(x);
        blk_mul_g(x, X + 3 * BLK, X + BLK, l16, g);
        {
            floatx4 pr = gre(x), pi = gim(x);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pr[r] += blk_re(X + 3 * BLK, g, r, l16);
                pi[r] += blk_im(X + 3 * BLK, g, r, l16);
            }
            blk_store(X, pr, pi, l16, g);
        }
        // T = P2 + P2 N^8
        gz(x);
        blk_mul_g(x, X, X + 2 * BLK, l16, g);
        {
            floatx4 pr = gre(x), pi = gim(x);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                pr[r] += blk_re(X, g, r, l16);
                pi[r] += blk_im(X, g, r, l16);
            }
            blk_store(sT + blk(w, w) * BLK, pr, pi, l16, g);
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
            for (int k = cc; k < bb; ++k) blk_mul_g(x, sM + blk(bb, k) * BLK, sT + blk(k, cc) * BLK, l16, g);
            blk_store(sR + w * BLK, gre(x), gim(x), l16, g);
        }
        __syncthreads();
        if (mine) {
            Gauss x;
            gz(x);
            blk_mul_g(x, sT + blk(bb, bb) * BLK, sR + w * BLK, l16, g);
            blk_store(sT + blk(bb, cc) * BLK, -gre(x), -gim(x), l16, g);
        }
        __syncthreads();
    }
    for (int k = 0; k < NBLK; ++k)
        blk_export(prep + chunk_prep(chain, n_chunks, c) + PREP_T + k * BLK, sT + k * BLK, tid, 256);
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

// the chain's checkpoint layout (the backward's): float (slot * 8 + plane * 4 + j % 4) of
// group state, slot = (i / 4) * 64 + (i % 4) * 16 + j / 4
__device__ __forceinline__ void ckpt_store(float *dst, int i, int j4, const floatx4 &re, const floatx4 &im) {
    const int slot = (i >> 2) * 64 + (i & 3) * 16 + j4;
    *reinterpret_cast<floatx4 *>(dst + slot * 8) = re;
    *reinterpret_cast<floatx4 *>(dst + slot * 8 + 4) = im;
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
    const int n_groups = (a.T + 15) / 16;
    float *ckpt = a.workspace ? static_cast<float *>(a.workspace) + (int64_t)chain * n_groups * (2 * D * D) : nullptr;

    for (int idx = tid; idx < CH * 16; idx += 256) {  // S0^T
        const int i = idx & 15, j = idx >> 4;
        const int64_t o = (int64_t)chain * D * D + (i0 + i) * D + j;
        sSr[0][j * SP + i] = a.s0_re ? a.s0_re[o] : 0.f;
        sSi[0][j * SP + i] = a.s0_re ? a.s0_im[o] : 0.f;
    }
    TileRegs xr;
    tile_fetch(xr, a.k, b, h, 0, min(CH, a.T), tid, 1.f);
    float lnext = prep[chunk_prep(chain, n_chunks, 0) + PREP_L + lane];
    float bnext = a.beta[b * a.sg_b + h * a.sg_h + (int64_t)min(lane, a.T - 1) * a.sg_t];
    int cur = 0;
    __syncthreads();
    if (ckpt) {  // group 0: the entering state
        floatx4 er, ei;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            er[r] = sSr[0][(16 * w + 4 * g + r) * SP + l16];
            ei[r] = sSi[0][(16 * w + 4 * g + r) * SP + l16];
        }
        ckpt_store(ckpt, i0 + l16, 4 * w + g, er, ei);
    }
    for (int c = 0; c < n_chunks; ++c) {
        const int t0 = c * CH, valid = min(CH, a.T - t0);
        const int64_t pc = chunk_prep(chain, n_chunks, c);
        tile_put(sKQr, sKQi, xr, tid);
        if (w == 0) {
            sL[lane] = lnext;
            sBt[lane] = lane < valid ? bnext : 0.f;
        }
        __syncthreads();
        tile_fetch(xr, a.q, b, h, t0, valid, tid, a.q_scale);  // in flight through the state work
        OpRegs ops;
        ops_fetch(ops, prep + pc + PREP_T, w, lane);
        float vr4[4], vi4[4];  // V of this lane's W elements
        {
            const float *vre = static_cast<const float *>(a.v.re) + b * a.v.s0 + h * a.v.s1 + i0 + l16;
            const float *vim = static_cast<const float *>(a.v.im) + b * a.v.s0 + h * a.v.s1 + i0 + l16;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int64_t o = (int64_t)(t0 + min(16 * w + 4 * g + r, valid - 1)) * a.v.s2;
                vr4[r] = vre[o];
                vi4[r] = vim[o];
            }
        }
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
                    gstep(x, ops.re[cc][ks], ops.im[cc][ks], sUr[s * SP + l16], sUi[s * SP + l16]);
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
        __syncthreads();
        const int wy = 3 - w;  // Y row tile: the wave with the most T blocks gets the fewest Ahat blocks
        ops_fetch(ops, prep + pc + PREP_A, wy, lane);  // Ahat, in flight through the state update
        // state update, row tile w of S^T (j = 16 w + 4 g + r, i = l16), in four 16-step quarters
        {
            floatx4 sr, si;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sr[r] = sSr[cur][(16 * w + 4 * g + r) * SP + l16];
                si[r] = sSi[cur][(16 * w + 4 * g + r) * SP + l16];
            }
            float Lprev = 0.f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float Lq = sL[16 * q + 15];
                const float f = __expf(Lq - Lprev);
                sr *= f;
                si *= f;
                Gauss x;
                gz(x);
#pragma unroll
                for (int ks = 0; ks < 4; ++ks) {
                    const int s = 16 * q + 4 * ks + g;
                    const float wq = __expf(Lq - sL[s]);
                    // conj(K)^T [j][s] (A) times (D U)[s][i] (B)
                    gstep(x, sKQr[s * KP + 16 * w + l16], -sKQi[s * KP + 16 * w + l16], sUr[s * SP + l16] * wq,
                          sUi[s * SP + l16] * wq);
                }
                sr += gre(x);
                si += gim(x);
                Lprev = Lq;
                const int grp = 4 * c + q + 1;  // the state before step 16 grp
                if (ckpt && 16 * grp < a.T) ckpt_store(ckpt + (int64_t)grp * (2 * D * D), i0 + l16, 4 * w + g, sr, si);
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                sSr[cur ^ 1][(16 * w + 4 * g + r) * SP + l16] = sr[r];
                sSi[cur ^ 1][(16 * w + 4 * g + r) * SP + l16] = si[r];
            }
        }
        __syncthreads();  // K no longer read
        tile_put(sKQr, sKQi, xr, tid);
        if (c + 1 < n_chunks) {
            const int v1 = min(CH, a.T - t0 - CH);
            tile_fetch(xr, a.k, b, h, t0 + CH, v1, tid, 1.f);
            lnext = prep[chunk_prep(chain, n_chunks, c + 1) + PREP_L + lane];
            bnext = a.beta[b * a.sg_b + h * a.sg_h + (int64_t)(t0 + CH + min(lane, v1 - 1)) * a.sg_t];
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

// sum over the 4 row groups of a wave (lanes cg, cg+16, cg+32, cg+48)
__device__ __forceinline__ float rows4_sum(float x) {
    x += __shfl_xor(x, 16);
    return x + __shfl_xor(x, 32);
}

// Per-workgroup partial sums over its rows, [part][chain][t]: (dq~ re, dq~ im,
// dk re, dk im) per column and (dgamma, dbeta); summed over the parts in a
// fixed order by delta_reduce_kernel.
__global__ void __launch_bounds__(BWD_THREADS) delta_bwd_kernel(qpam_delta_bwd_args g, qpam_delta_args a) {
    // per flush: [token][wave][column] = (dq~ re, dq~ im, dk re, dk im) and
    // [token][wave * 4 + row group] = (dgamma, dbeta)
    __shared__ floatx4 red[FL][PW][D];
    __shared__ floatx2 sred[FL][4 * PW];
    __shared__ Span<GROUP, PROWS> sp;          // the group's token inputs for this workgroup's rows
    __shared__ float sdy[GROUP][2][PROWS];     // and output gradients
    const int chain = blockIdx.x / PARTS, part = blockIdx.x - chain * PARTS;
    const int b = chain / a.H, h = chain - b * a.H, tid = threadIdx.x;
    const Lane L(part * PW + (tid >> 6), tid & 63);
    const int row0 = part * PROWS;
    const int64_t nbht = (int64_t)a.B * a.H * a.T;
    floatx4 *pcol = reinterpret_cast<floatx4 *>(static_cast<char *>(g.workspace) + bwd_sub_bytes(a)) +
                    ((int64_t)part * a.B * a.H + chain) * a.T * D;
    floatx2 *pscal = reinterpret_cast<floatx2 *>(reinterpret_cast<floatx4 *>(static_cast<char *>(g.workspace) +
                                                                             bwd_sub_bytes(a)) + PARTS * nbht * D) +
                     ((int64_t)part * a.B * a.H + chain) * a.T;
    const int ng = chain_groups(a.T);
    const float *ckpt = static_cast<const float *>(a.workspace) + (int64_t)chain * ng * STATE_FLOATS;
    float *sub = static_cast<float *>(g.workspace) + (int64_t)chain * SUBS * STATE_FLOATS;

    State gs;   // adjoint of the state after the current token
    init_state(gs, g.ds_re, g.ds_im, chain, L);

    for (int grp = ng - 1; grp >= 0; --grp) {
        const int t0 = grp * GROUP, tn = min(t0 + GROUP, a.T);
        {   // stage the group's inputs and output gradients
            SpanRegs<GROUP, PROWS, BWD_THREADS> regs;
            regs.fetch(a, b, h, t0, row0, tid);
            constexpr int NDY = GROUP * 2 * PROWS / BWD_THREADS;
            float dyv[NDY];
#pragma unroll
            for (int k = 0; k < NDY; ++k) {
                const int i = tid + k * BWD_THREADS, tok = i / (2 * PROWS), rem = i - tok * 2 * PROWS;
                const int ri = rem / PROWS, r = rem - ri * PROWS;
                const int t = min(t0 + tok, a.T - 1);
                dyv[k] = static_cast<const float *>(ri ? g.dy.im : g.dy.re)[b * g.dy.s0 + h * g.dy.s1 +
                                                                            (int64_t)t * g.dy.s2 + row0 + r];
            }
            __syncthreads();   // the previous group's readers are done
            regs.commit(sp, tid);
#pragma unroll
            for (int k = 0; k < NDY; ++k) {
                const int i = tid + k * BWD_THREADS, tok = i / (2 * PROWS), rem = i - tok * 2 * PROWS;
                const int ri = rem / PROWS, r = rem - ri * PROWS;
                sdy[tok][ri][r] = dyv[k];
            }
            __syncthreads();
        }
        // recompute the group, keeping the state before every SUB-th token
        State s;
        load_state(ckpt + (int64_t)grp * STATE_FLOATS, s, L.slot());
        for (int t = t0; t < tn; ++t) {
            if ((t - t0) % SUB == 0) store_state(sub + (int64_t)((t - t0) / SUB) * STATE_FLOATS, s, L.slot());
            const Tok x = span_tok(sp, t - t0, L.cg, L.r0 - row0);
            float yr[RPL], yi[RPL];
            fwd_step(s, x, yr, yi);
        }
        for (int sg = (tn - t0 - 1) / SUB; sg >= 0; --sg) {
            const int s0 = t0 + sg * SUB, n = min(SUB, tn - s0);
            // states before each token of the sub-group
            State prev[SUB];
            load_state(sub + (int64_t)sg * STATE_FLOATS, prev[0], L.slot());
#pragma unroll
            for (int j = 1; j < SUB; ++j) {
                prev[j] = prev[j - 1];
                if (j < n) {
                    const Tok x = span_tok(sp, s0 + j - 1 - t0, L.cg, L.r0 - row0);
                    float yr[RPL], yi[RPL];
                    fwd_step(prev[j], x, yr, yi);
                }
            }
#pragma unroll
            for (int j = SUB - 1; j >= 0; --j) {
                if (j < n) {
                    const int t = s0 + j;
                    const Tok x = span_tok(sp, t - t0, L.cg, L.r0 - row0);
                    float gyr[RPL], gyi[RPL];
#pragma unroll
                    for (int rr = 0; rr < RPL; ++rr)
                        gyr[rr] = sdy[t - t0][0][L.r0 - row0 + rr], gyi[rr] = sdy[t - t0][1][L.r0 - row0 + rr];
                    const State &sp = prev[j];
                    // forward quantities of this token
                    float ar[RPL][4], ai[RPL][4], pr[RPL], pi[RPL], ur[RPL], ui[RPL];
#pragma unroll
                    for (int rr = 0; rr < RPL; ++rr) {
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
                    float gur[RPL], gui[RPL];
#pragma unroll
                    for (int rr = 0; rr < RPL; ++rr) {
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
                    for (int rr = 0; rr < RPL; ++rr) {
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
#pragma unroll
                        for (int rr = 0; rr < RPL; ++rr) g.dv.re[vo + rr] = x.b * gur[rr], g.dv.im[vo + rr] = x.b * gui[rr];
                    }
                    // column sums over the wave's rows, then one slot per wave
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        gq[c][0] = rows4_sum(gq[c][0]), gq[c][1] = rows4_sum(gq[c][1]);
                        gk[c][0] = rows4_sum(gk[c][0]), gk[c][1] = rows4_sum(gk[c][1]);
                    }
                    if (L.rg == 0) {
#pragma unroll
                        for (int c = 0; c < 4; ++c)
                            red[j % FL][L.w - part * PW][4 * L.cg + c] = floatx4{gq[c][0], gq[c][1], gk[c][0], gk[c][1]};
                    }
                    // ggam holds this lane's columns; gbet is already the row group's value
                    ggam = row16_sum(ggam);
                    if (L.cg == 0) sred[j % FL][4 * (L.w - part * PW) + L.rg] = floatx2{ggam, gbet};
                }
                if (j % FL == 0) {
                    __syncthreads();
                    // tokens j .. j + FL - 1 of the sub-group: reduce the wave slots in a fixed order
                    const int m = min(FL, n - j);
                    for (int i = tid; i < m * D; i += BWD_THREADS) {
                        const int jj = i / D, c = i - jj * D, t = s0 + j + jj;
                        floatx4 acc = red[jj][0][c];
#pragma unroll
                        for (int w = 1; w < PW; ++w) acc += red[jj][w][c];
                        pcol[(int64_t)t * D + c] = acc;
                    }
                    if (tid < m) {
                        floatx2 acc = sred[tid][0];
                        for (int k = 1; k < 4 * PW; ++k) acc += sred[tid][k];
                        pscal[s0 + j + tid] = acc;
                    }
                    __syncthreads();
                }
            }
        }
    }
    if (g.ds0_re) write_state(g.ds0_re, g.ds0_im, gs, chain, L);
}

// dq = q_scale * sum of the parts' dq~, dk, dgamma, dbeta: one thread per (chain, t, column)
__global__ void __launch_bounds__(256) delta_reduce_kernel(qpam_delta_bwd_args g, qpam_delta_args a) {
    const int64_t nbht = (int64_t)a.B * a.H * a.T;
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= nbht * D) return;
    const int64_t ct = i / D;
    const int c = (int)(i - ct * D);
    const int chain = (int)(ct / a.T), t = (int)(ct - (int64_t)chain * a.T);
    const int b = chain / a.H, h = chain - b * a.H;
    const floatx4 *pcol = reinterpret_cast<const floatx4 *>(static_cast<const char *>(g.workspace) + bwd_sub_bytes(a));
    floatx4 acc = pcol[i];
#pragma unroll
    for (int p = 1; p < PARTS; ++p) acc += pcol[p * nbht * D + i];
    const int64_t qo = b * g.dq.s0 + h * g.dq.s1 + (int64_t)t * g.dq.s2 + c;
    const int64_t ko = b * g.dk.s0 + h * g.dk.s1 + (int64_t)t * g.dk.s2 + c;
    g.dq.re[qo] = acc.x * a.q_scale, g.dq.im[qo] = acc.y * a.q_scale;
    g.dk.re[ko] = acc.z, g.dk.im[ko] = acc.w;
    if (c == 0) {
        const floatx2 *pscal = reinterpret_cast<const floatx2 *>(pcol + PARTS * nbht * D);
        floatx2 sacc = pscal[ct];
#pragma unroll
        for (int p = 1; p < PARTS; ++p) sacc += pscal[p * nbht + ct];
        const int64_t go = b * a.sg_b + h * a.sg_h + (int64_t)t * a.sg_t;
        g.dgamma[go] = sacc.x;
        g.dbeta[go] = sacc.y;
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
size_t prep_bytes(const qpam_delta_args &a) {
    return (size_t)a.B * a.H * ((a.T + CH - 1) / CH) * PREP_FLOATS * sizeof(float);
}
size_t bwd_ws(const qpam_delta_args &a) {
    const size_t nbht = (size_t)a.B * a.H * a.T;
    return bwd_sub_bytes(a) + PARTS * nbht * (D * sizeof(floatx4) + sizeof(floatx2));
}

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
    const int n_chunks = (a->T + CH - 1) / CH;
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
                 "qpam_delta_bwd: the forward's workspace (checkpoints) is required");
    QPAM_REQUIRE(g->workspace && aligned(g->workspace, 16) && g->workspace_bytes >= bwd_ws(a),
                 "qpam_delta_bwd: workspace of %zu bytes needed", bwd_ws(a));
    QPAM_REQUIRE(cview_ok(g->dy) && mview_ok(g->dq) && mview_ok(g->dk) && mview_ok(g->dv),
                 "qpam_delta_bwd: dy, dq, dk, dv must be 16-byte aligned fp32 planes with strides multiple of 4");
    QPAM_REQUIRE(g->dgamma && g->dbeta, "qpam_delta_bwd: dgamma and dbeta required");
    QPAM_REQUIRE((g->ds_re == nullptr) == (g->ds_im == nullptr) && (g->ds0_re == nullptr) == (g->ds0_im == nullptr),
                 "qpam_delta_bwd: ds / ds0 need both planes");
    if (a.B == 0 || a.T == 0) return QPAM_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipLaunchKernelGGL(delta_bwd_kernel, dim3(a.B * a.H * PARTS), dim3(BWD_THREADS), 0, s, *g, a);
    st = launch_status("delta_bwd_kernel");
    if (st) return st;
    const int64_t n = (int64_t)a.B * a.H * a.T * D;
    hipLaunchKernelGGL(delta_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, *g, a);
    return launch_status("delta_reduce_kernel");
}
