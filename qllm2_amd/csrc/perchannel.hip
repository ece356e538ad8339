// E1 per-channel decay: the chunk-local decay fold of queries and keys (and
// its backward) and the per-column decayed state scan, the two steps of
// V11PAMLayer._forward_chunked_perchannel (v11/model.py:421-489) that are not
// plain complex GEMMs.  Both are streaming kernels: a block per (chain, chunk)
// for the fold, and one lane per state element walking the chunks for the
// scan.
#include "common.h"

namespace qpam {
namespace {

constexpr int PC_THREADS = 256;
constexpr int PC_MAX_CHUNK = 64;
constexpr float PC_GAMMA_FLOOR = 1e-6f;  // gamma.clamp_min(1e-6), v11/model.py:436
constexpr float PC_CUM_FLOOR = -30.f;    // cumsum.clamp(min=-30), v11/model.py:438

__device__ __forceinline__ float ld(const void *p, int64_t off, int dt) {
    return dt == QPAM_BF16 ? bf16_to_f32(static_cast<const unsigned short *>(p)[off]) : static_cast<const float *>(p)[off];
}
__device__ __forceinline__ void st(void *p, int64_t off, float v, int dt) {
    if (dt == QPAM_BF16) static_cast<unsigned short *>(p)[off] = f32_to_bf16(v);
    else static_cast<float *>(p)[off] = v;
}
__device__ __forceinline__ float2 ld2(const float *p, int64_t off) {
    return p ? *reinterpret_cast<const float2 *>(p + off) : make_float2(0.f, 0.f);
}

// Fold layout: a block per (chain, chunk, 64 key channels); thread (j, grp) owns
// key channel j and the chunk's steps 16 grp .. 16 grp + 15.  The log-decay
// prefix runs within the thread's 16 steps, the group totals meet in LDS (in
// group order), and every global access of a step is a coalesced row of 64
// channels; a thread's 16 steps are independent loads.
constexpr int PC_ROWS = 16;                  // steps per thread
constexpr int PC_GROUPS = PC_MAX_CHUNK / PC_ROWS;
static_assert(PC_GROUPS * 64 == PC_THREADS, "fold block shape");

struct Lane {
    int64_t cc;  // chain * n + c
    int j, jl, grp, c, b, h, t0, valid;
    bool jv;
};
__device__ __forceinline__ Lane lane_of(const qpam_pc_fold_args &a, int n) {
    Lane l;
    l.cc = blockIdx.x;
    l.jl = threadIdx.x & 63;
    l.grp = threadIdx.x >> 6;
    l.j = blockIdx.y * 64 + l.jl;
    l.jv = l.j < a.d;
    l.c = (int)(l.cc % n);
    const int64_t chain = l.cc / n;
    l.b = (int)(chain / a.H);
    l.h = (int)(chain % a.H);
    l.t0 = l.c * a.chunk;
    l.valid = (int)min((int64_t)a.chunk, a.T - l.t0);
    return l;
}

// The thread's inclusive log-decay prefixes (unclamped) of its 16 steps, the
// exclusive offset of the earlier groups added; L_last of the chunk (clamped)
// from the group holding step valid - 1.
__device__ __forceinline__ void fold_prefix(const qpam_pc_fold_args &a, const Lane &l, int64_t go, float (&cs)[PC_ROWS],
                                            float *sTot, float *sLast, float &Llast) {
    float run = 0.f;
#pragma unroll
    for (int r = 0; r < PC_ROWS; ++r) {
        const int t = PC_ROWS * l.grp + r;
        const float x = (l.jv && t < l.valid) ? logf(fmaxf(ld(a.gamma, go + t * a.g_st, a.g_dtype), PC_GAMMA_FLOOR)) : 0.f;
        run += x;
        cs[r] = run;
    }
    sTot[l.grp * 64 + l.jl] = run;
    __syncthreads();
    float off = 0.f;
    for (int g = 0; g < l.grp; ++g) off += sTot[g * 64 + l.jl];
#pragma unroll
    for (int r = 0; r < PC_ROWS; ++r) cs[r] += off;
    const int last = l.valid - 1;
    if (l.grp == last / PC_ROWS) {
        float v = 0.f;
#pragma unroll
        for (int r = 0; r < PC_ROWS; ++r) v = (r == last % PC_ROWS) ? cs[r] : v;
        sLast[l.jl] = fmaxf(v, PC_CUM_FLOOR);
    }
    __syncthreads();
    Llast = sLast[l.jl];
}

__global__ void __launch_bounds__(PC_THREADS) pc_fold_fwd_kernel(qpam_pc_fold_args a, int n) {
    __shared__ float sTot[PC_GROUPS * 64], sLast[64];
    const Lane l = lane_of(a, n);
    const int64_t go = l.b * a.g_sb + l.h * a.g_sh + (int64_t)l.t0 * a.g_st + l.j;
    const int64_t qo = l.b * a.q_sb + l.h * a.q_sh + (int64_t)l.t0 * a.q_st + 2 * l.j;
    const int64_t ko = l.b * a.k_sb + l.h * a.k_sh + (int64_t)l.t0 * a.k_st + 2 * l.j;
    float cs[PC_ROWS], Llast;
    fold_prefix(a, l, go, cs, sTot, sLast, Llast);
    if (!l.jv) return;
    const int64_t oo = (l.cc * a.chunk) * a.d + l.j;  // element (t, j) at oo + t d
#pragma unroll
    for (int r = 0; r < PC_ROWS; ++r) {
        const int t = PC_ROWS * l.grp + r;
        if (t >= a.chunk) continue;
        float2 qf = make_float2(0.f, 0.f), kf = qf, wf = qf;
        if (t < l.valid) {
            const float L = fmaxf(cs[r], PC_CUM_FLOOR);
            const float al = __expf(L) * a.q_scale, be = __expf(-L), ta = __expf(Llast - L);
            const float qr = ld(a.q, qo + t * a.q_st, a.dtype), qi = ld(a.q, qo + t * a.q_st + 1, a.dtype);
            const float kr = ld(a.k, ko + t * a.k_st, a.dtype), ki = ld(a.k, ko + t * a.k_st + 1, a.dtype);
            qf = make_float2(qr * al, qi * al);
            kf = make_float2(kr * be, ki * be);
            wf = make_float2(kr * ta, ki * ta);
        }
        const int64_t o = 2 * (oo + (int64_t)t * a.d);
        *reinterpret_cast<float2 *>(a.qf + o) = qf;
        *reinterpret_cast<float2 *>(a.kf + o) = kf;
        *reinterpret_cast<float2 *>(a.wf + o) = wf;
    }
    if (l.grp == 0) a.atot[l.cc * a.d + l.j] = __expf(Llast);
}

// Backward: dq = dqf e^{L} q_scale, dk = dkf e^{-L} + dwf e^{L_last - L}, and
// the log-decay gradient
//   dL_t = Re(conj(qf) dqf) - Re(conj(kf) dkf) - Re(conj(wf) dwf)
//          (+ at the last step: sum_s Re(conj(wf_s) dwf_s) + atot datot),
// masked where the prefix sat below -30, summed from the end of the chunk
// (the cumsum's gradient: each thread's suffix sums plus the later groups'
// totals) and divided by gamma where gamma >= 1e-6.
__global__ void __launch_bounds__(PC_THREADS) pc_fold_bwd_kernel(qpam_pc_fold_args a, int n) {
    __shared__ float sTot[PC_GROUPS * 64], sLast[64], sW[PC_GROUPS * 64], sD[PC_GROUPS * 64];
    const Lane l = lane_of(a, n);
    const int64_t go = l.b * a.g_sb + l.h * a.g_sh + (int64_t)l.t0 * a.g_st + l.j;
    const int64_t qo = l.b * a.q_sb + l.h * a.q_sh + (int64_t)l.t0 * a.q_st + 2 * l.j;
    const int64_t ko = l.b * a.k_sb + l.h * a.k_sh + (int64_t)l.t0 * a.k_st + 2 * l.j;
    const int64_t oo = (l.cc * a.chunk) * a.d + l.j;
    const int64_t out_o = ((int64_t)(l.b * a.H + l.h) * a.T + l.t0) * a.d + l.j;  // contiguous outputs
    float cs[PC_ROWS], Llast;
    fold_prefix(a, l, go, cs, sTot, sLast, Llast);
    // sum_s e^{-L_s} Re(conj(k_s) dwf_s) over the chunk: thread partials, then the groups in order
    float wpart = 0.f;
    float2 dq[PC_ROWS], dk[PC_ROWS], dw[PC_ROWS];
    float kr[PC_ROWS], ki[PC_ROWS];
#pragma unroll
    for (int r = 0; r < PC_ROWS; ++r) {
        const int t = PC_ROWS * l.grp + r;
        const bool ok = l.jv && t < l.valid;
        const int64_t o = 2 * (oo + (int64_t)t * a.d);
        dq[r] = ok ? ld2(a.dqf, o) : make_float2(0.f, 0.f);
        dk[r] = ok ? ld2(a.dkf, o) : make_float2(0.f, 0.f);
        dw[r] = ok ? ld2(a.dwf, o) : make_float2(0.f, 0.f);
        kr[r] = ok ? ld(a.k, ko + t * a.k_st, a.dtype) : 0.f;
        ki[r] = ok ? ld(a.k, ko + t * a.k_st + 1, a.dtype) : 0.f;
        wpart += ok ? __expf(-fmaxf(cs[r], PC_CUM_FLOOR)) * (kr[r] * dw[r].x + ki[r] * dw[r].y) : 0.f;
    }
    sW[l.grp * 64 + l.jl] = wpart;
    __syncthreads();
    float wsum = 0.f;
    for (int g = 0; g < PC_GROUPS; ++g) wsum += sW[g * 64 + l.jl];
    const float Elast = __expf(Llast);
    const float dLlast = Elast * (wsum + ((a.datot && l.jv) ? a.datot[l.cc * a.d + l.j] : 0.f));
    // the thread's steps from its last to its first: the masked dL and their suffix sums
    float suf[PC_ROWS], run = 0.f;
#pragma unroll
    for (int r = PC_ROWS - 1; r >= 0; --r) {
        const int t = PC_ROWS * l.grp + r;
        float dcs = 0.f;
        if (l.jv && t < l.valid) {
            const float L = fmaxf(cs[r], PC_CUM_FLOOR);
            const float al = __expf(L) * a.q_scale, be = __expf(-L), ta = __expf(Llast - L);
            const float qr = ld(a.q, qo + t * a.q_st, a.dtype), qi = ld(a.q, qo + t * a.q_st + 1, a.dtype);
            // conj(x f) dx = f conj(x) dx for a real factor f
            float dL = al * (qr * dq[r].x + qi * dq[r].y) - be * (kr[r] * dk[r].x + ki[r] * dk[r].y) -
                       ta * (kr[r] * dw[r].x + ki[r] * dw[r].y);
            if (t == l.valid - 1) dL += dLlast;
            dcs = (cs[r] >= PC_CUM_FLOOR) ? dL : 0.f;
            const int64_t so = out_o + (int64_t)t * a.d;
            st(a.dq, 2 * so, dq[r].x * al, a.dtype);
            st(a.dq, 2 * so + 1, dq[r].y * al, a.dtype);
            st(a.dk, 2 * so, dk[r].x * be + dw[r].x * ta, a.dtype);
            st(a.dk, 2 * so + 1, dk[r].y * be + dw[r].y * ta, a.dtype);
        }
        run += dcs;
        suf[r] = run;
    }
    sD[l.grp * 64 + l.jl] = run;
    __syncthreads();
    float later = 0.f;
    for (int g = PC_GROUPS - 1; g > l.grp; --g) later += sD[g * 64 + l.jl];
#pragma unroll
    for (int r = 0; r < PC_ROWS; ++r) {
        const int t = PC_ROWS * l.grp + r;
        if (l.jv && t < l.valid) {
            const float gam = ld(a.gamma, go + t * a.g_st, a.g_dtype);
            st(a.dgamma, out_o + (int64_t)t * a.d, gam >= PC_GAMMA_FLOOR ? (suf[r] + later) / gam : 0.f, a.g_dtype);
        }
    }
}

// One lane per complex state element (chain, i, j); the next two chunks' inputs
// are loaded ahead of the running update.
__global__ void __launch_bounds__(PC_THREADS) pc_scan_kernel(qpam_pc_scan_args a) {
    const int64_t e = (int64_t)blockIdx.x * PC_THREADS + threadIdx.x;
    const int64_t dd = a.d * a.d;
    if (e >= a.N * dd) return;
    const int64_t chain = e / dd, ij = e % dd;
    const int j = (int)(ij % a.d);
    float2 S = a.init ? *reinterpret_cast<const float2 *>(a.init + 2 * e) : make_float2(0.f, 0.f);
    auto chunk_of = [&](int64_t k) { return a.reverse ? a.n - 1 - k : k; };
    auto xo = [&](int64_t c) { return 2 * ((chain * a.n + c) * dd + ij); };
    auto ao = [&](int64_t c) { return (chain * a.n + c) * a.d + j; };
    float2 x0 = make_float2(0.f, 0.f), x1 = x0;
    float a0 = 0.f, a1 = 0.f;
    if (a.n > 0) x0 = *reinterpret_cast<const float2 *>(a.x + xo(chunk_of(0))), a0 = a.a[ao(chunk_of(0))];
    if (a.n > 1) x1 = *reinterpret_cast<const float2 *>(a.x + xo(chunk_of(1))), a1 = a.a[ao(chunk_of(1))];
    for (int64_t k = 0; k < a.n; ++k) {
        const int64_t c = chunk_of(k);
        const float2 x = x0;
        const float av = a0;
        x0 = x1;
        a0 = a1;
        if (k + 2 < a.n) {
            x1 = *reinterpret_cast<const float2 *>(a.x + xo(chunk_of(k + 2)));
            a1 = a.a[ao(chunk_of(k + 2))];
        }
        *reinterpret_cast<float2 *>(a.out + xo(c)) = S;
        S = make_float2(av * S.x + x.x, av * S.y + x.y);
    }
    if (a.fin) *reinterpret_cast<float2 *>(a.fin + 2 * e) = S;
}

int validate_fold(const qpam_pc_fold_args *a, const char *who) {
    QPAM_REQUIRE(a != nullptr, "%s: null args", who);
    QPAM_REQUIRE(a->B > 0 && a->H > 0 && a->T > 0 && a->d > 0, "%s: B, H, T, d must be positive", who);
    QPAM_REQUIRE(a->chunk >= 1 && a->chunk <= PC_MAX_CHUNK, "%s: chunk must be in 1..%d", who, PC_MAX_CHUNK);
    QPAM_REQUIRE((a->dtype == QPAM_F32 || a->dtype == QPAM_BF16) && (a->g_dtype == QPAM_F32 || a->g_dtype == QPAM_BF16),
                 "%s: dtype and g_dtype must be QPAM_F32 or QPAM_BF16", who);
    QPAM_REQUIRE(a->q && a->k && a->gamma, "%s: q, k and gamma are required", who);
    QPAM_REQUIRE(a->B * a->H * ((a->T + a->chunk - 1) / a->chunk) < (1ll << 31), "%s: grid too large", who);
    return QPAM_OK;
}

}  // namespace
}  // namespace qpam

using namespace qpam;

extern "C" int qpam_pc_fold_fwd(const qpam_pc_fold_args *a, void *stream) {
    int st_ = validate_fold(a, "qpam_pc_fold_fwd");
    if (st_) return st_;
    QPAM_REQUIRE(a->qf && a->kf && a->wf && a->atot, "qpam_pc_fold_fwd: qf, kf, wf and atot are required");
    const int n = (int)((a->T + a->chunk - 1) / a->chunk);
    hipLaunchKernelGGL(pc_fold_fwd_kernel, dim3((unsigned)(a->B * a->H * n), (unsigned)((a->d + 63) / 64)),
                       dim3(PC_THREADS), 0, (hipStream_t)stream, *a, n);
    return launch_status("pc_fold_fwd_kernel");
}

extern "C" int qpam_pc_fold_bwd(const qpam_pc_fold_args *a, void *stream) {
    int st_ = validate_fold(a, "qpam_pc_fold_bwd");
    if (st_) return st_;
    QPAM_REQUIRE(a->dq && a->dk && a->dgamma, "qpam_pc_fold_bwd: dq, dk and dgamma are required");
    const int n = (int)((a->T + a->chunk - 1) / a->chunk);
    hipLaunchKernelGGL(pc_fold_bwd_kernel, dim3((unsigned)(a->B * a->H * n), (unsigned)((a->d + 63) / 64)),
                       dim3(PC_THREADS), 0, (hipStream_t)stream, *a, n);
    return launch_status("pc_fold_bwd_kernel");
}

extern "C" int qpam_pc_scan(const qpam_pc_scan_args *a, void *stream) {
    QPAM_REQUIRE(a != nullptr, "qpam_pc_scan: null args");
    QPAM_REQUIRE(a->N > 0 && a->n > 0 && a->d > 0, "qpam_pc_scan: N, n, d must be positive");
    QPAM_REQUIRE(a->x && a->a && a->out, "qpam_pc_scan: x, a and out are required");
    QPAM_REQUIRE(a->reverse == 0 || a->reverse == 1, "qpam_pc_scan: reverse must be 0 or 1");
    const int64_t lanes = a->N * a->d * a->d;
    hipLaunchKernelGGL(pc_scan_kernel, dim3((unsigned)((lanes + PC_THREADS - 1) / PC_THREADS)), dim3(PC_THREADS), 0,
                       (hipStream_t)stream, *a);
    return launch_status("pc_scan_kernel");
}
