// Ragged continuous-batching PAM decode step (HBM-bound streaming kernel).
//
// Reference semantics: V11PAMLayer._recur_step_additive (v11/model.py:927-965)
// applied per state and phase-routed/summed as in _recurrent
// (v11/model.py:874-906):
//     S <- gamma S + v (x) conj(k);   y = sum_m r_m (S_m @ q~)
// with a head decay, or (gamma_per_channel) one decay per key column j, the
// per-channel branch (v11/model.py:952-954).
//
// Design: one workgroup per (listed slot, group).  The d x d interleaved
// complex state of each of the M states is streamed once with non-temporal
// 16-byte loads and stores (consecutive lanes on consecutive 16 bytes, so a
// wave instruction covers a contiguous 1 KiB; the state is touched once per
// step, so it bypasses the caches).  Each lane owns a fixed pair of key
// columns, so q~ and k are loaded once per lane; the row sums of S q~ are
// reduced across the lanes of a row with a halving butterfly (each step
// halves the number of live partial sums).  Slots that are not listed cost
// nothing: the grid is n_active * n_groups.
//
// Optional per-slot rotary positions rotate q and k as they are loaded.  With
// vec_by_rank the per-token operands (q, k, v, gamma, rot, y) are the compact
// rows of the listed slots (row i for active[i]): a continuous-batching engine
// projects only its live sequences and needs no scatter into slot-sized
// buffers; states and positions stay indexed by slot.
//
// Kernels: the single-state, unrotated step (the continuous-batching common
// case) keeps every register for loads in flight, 512 threads per 64 x 64
// state and no LDS or barriers; up to 4 states (E3 models use 3), with or
// without read rotations, take the multi-state kernel, which loads every state
// up front and folds the rotations into the lane partials (d = 128: one
// state); more states take the general kernel, which loops over them
// through LDS.
#include "common.h"

namespace qpam {
namespace {

template <int D, int T>
struct DecodeShape {
    static constexpr int PAIRS = D / 2;                       // float4 per state row
    static constexpr int THREADS = (D * D / 2) < T ? (D * D / 2) : T;
    static constexpr int ROWS_PER_IT = THREADS / PAIRS;       // rows covered per iteration
    static constexpr int ITERS = D / ROWS_PER_IT;             // float4 per lane per state
    static constexpr int NV = 2 * ITERS;                      // partial sums per lane (re, im per row)
    // lane-offset bits of the reduction steps that are plain butterflies (all
    // lanes of the pair end with the same sum): a lane owns its sums when
    // these bits of its lane id are zero
    static constexpr int bfly_mask() {
        int nv = NV, m = 0;
        for (int off = PAIRS / 2; off >= 1; off >>= 1) {
            if (nv > 1) nv /= 2;
            else m |= off;
        }
        return m;
    }
};

// Two consecutive complex features (re, im, re, im) of a q or k row: one 16-byte
// load of the interleaved row, or two 8-byte loads of the planar row (im != null).
template <bool PL>
__device__ __forceinline__ float4 load_pair(const float *re, const float *im, int64_t row, int cp) {
    if constexpr (!PL) return *reinterpret_cast<const float4 *>(re + row + 4 * cp);
    const float2 r = *reinterpret_cast<const float2 *>(re + row + 2 * cp);
    const float2 i = *reinterpret_cast<const float2 *>(im + row + 2 * cp);
    return make_float4(r.x, i.x, r.y, i.y);
}
// complex feature `e` of a v row, interleaved or planar
template <bool PL>
__device__ __forceinline__ float2 load_one(const float *re, const float *im, int e) {
    if constexpr (!PL) return *reinterpret_cast<const float2 *>(re + 2 * e);
    return make_float2(re[e], im[e]);
}

// decay of this lane's key columns 2 cp, 2 cp + 1 for the state whose decay
// entry starts at `off`: the head decay of (slot, group, state), or its two
// per-channel decays (gamma_per_channel)
__device__ __forceinline__ float2 lane_decay(const qpam_decode_args &a, int64_t off, int cp) {
    if (!a.gamma_per_channel) {
        const float g = a.gamma[off];
        return make_float2(g, g);
    }
    return make_float2(a.gamma[off + 2 * cp], a.gamma[off + 2 * cp + 1]);
}

// element `e` of the y row at `row` (element offset), fp32 or bf16
__device__ __forceinline__ void store_y(const qpam_decode_args &a, int64_t row, int e, float v) {
    if (a.y_dtype == QPAM_BF16) reinterpret_cast<unsigned short *>(a.y)[row + e] = f32_to_bf16(v);
    else a.y[row + e] = v;
}

// q and k of the slot times rope[pos[slot]] (two complex features per float4)
template <int D>
__device__ __forceinline__ void apply_rope(const qpam_decode_args &a, int slot, int cp, float4 &qv, float4 &kv) {
    if (!a.rope) return;
    const int p = min(max(a.pos[slot], 0), a.rope_len - 1);
    const float4 r = *reinterpret_cast<const float4 *>(a.rope + (int64_t)p * 2 * D + 4 * cp);
    const float4 q = qv, k = kv;
    qv = make_float4(q.x * r.x - q.y * r.y, q.x * r.y + q.y * r.x, q.z * r.z - q.w * r.w, q.z * r.w + q.w * r.z);
    kv = make_float4(k.x * r.x - k.y * r.y, k.x * r.y + k.y * r.x, k.z * r.z - k.w * r.w, k.z * r.w + k.w * r.z);
}

// Reduce NV values across P aligned lanes by halving; on return the lane holds
// `nv` complete sums for value indices [idx_base, idx_base + nv).
template <int NV, int P>
__device__ __forceinline__ void halving_reduce(float (&v)[NV], int lane, int &idx_base, int &nv_out) {
    int nv = NV;
    idx_base = 0;
#pragma unroll
    for (int off = P / 2; off >= 1; off >>= 1) {
        if (nv > 1) {
            const int half = nv / 2;
            const bool up = (lane & off) != 0;
#pragma unroll
            for (int j = 0; j < NV / 2; ++j) {
                if (j < half) {
                    float send = up ? v[j] : v[j + half];
                    float keep = up ? v[j + half] : v[j];
                    v[j] = keep + __shfl_xor(send, off);
                }
            }
            if (up) idx_base += half;
            nv = half;
        } else {
            v[0] += __shfl_xor(v[0], off);
        }
    }
    nv_out = nv;
}

// S <- gam S + v (x) conj(k) on this lane's ITERS float4 (two complex entries
// each), streamed in place; returns the lane's partial sums of S q~ per row.
template <typename S, bool PL>
__device__ __forceinline__ void update_state(float *st, int tid, int r0, float2 gam, const float *vrow,
                                             const float *vrow_im, float4 kv,
                                             float q0r, float q0i, float q1r, float q1i, float (&part)[S::NV]) {
    floatx4 s[S::ITERS];
#pragma unroll
    for (int it = 0; it < S::ITERS; ++it)
        s[it] = __builtin_nontemporal_load(reinterpret_cast<const floatx4 *>(st + 4 * (it * S::THREADS + tid)));
#pragma unroll
    for (int it = 0; it < S::ITERS; ++it) {
        const int row = it * S::ROWS_PER_IT + r0;
        const float2 vv = load_one<PL>(vrow, vrow_im, row);
        // v_i conj(k_j) for the two columns
        const float o0r = vv.x * kv.x + vv.y * kv.y, o0i = vv.y * kv.x - vv.x * kv.y;
        const float o1r = vv.x * kv.z + vv.y * kv.w, o1i = vv.y * kv.z - vv.x * kv.w;
        floatx4 n;
        n.x = gam.x * s[it].x + o0r;
        n.y = gam.x * s[it].y + o0i;
        n.z = gam.y * s[it].z + o1r;
        n.w = gam.y * s[it].w + o1i;
        __builtin_nontemporal_store(n, reinterpret_cast<floatx4 *>(st + 4 * (it * S::THREADS + tid)));
        part[2 * it] = n.x * q0r - n.y * q0i + n.z * q1r - n.w * q1i;
        part[2 * it + 1] = n.x * q0i + n.y * q0r + n.z * q1i + n.w * q1r;
    }
}

// ------------------------------------------------ one state, no rotation --
template <int D, bool PL>
__global__ void __launch_bounds__((DecodeShape<D, 512>::THREADS)) decode_single_kernel(qpam_decode_args a) {
    using S = DecodeShape<D, 512>;
    const int tid = threadIdx.x;
    const int ai = blockIdx.x / a.n_groups;
    const int g = blockIdx.x - ai * a.n_groups;
    const int slot = a.active ? a.active[ai] : ai;
    if (slot < 0 || slot >= a.n_slots) return;
    const int vr = a.vec_by_rank ? ai : slot;   // row of q, k, v, gamma, rot, y
    const int cp = tid % S::PAIRS, r0 = tid / S::PAIRS, lane = tid & 63;
    float4 qv = load_pair<PL>(a.q, a.q_im, vr * a.sq_slot + g * a.sq_group, cp);
    float4 kv = load_pair<PL>(a.k, a.k_im, vr * a.sk_slot + g * a.sk_group, cp);
    apply_rope<D>(a, slot, cp, qv, kv);
    const float2 gam = lane_decay(a, vr * a.sg_slot + g * a.sg_group, cp);
    float part[S::NV];
    const int64_t vo = vr * a.sv_slot + g * a.sv_group;
    update_state<S, PL>(a.state + slot * a.st_slot + g * a.st_group, tid, r0, gam, a.v + vo, PL ? a.v_im + vo : nullptr,
                    kv, qv.x * a.q_scale, qv.y * a.q_scale, qv.z * a.q_scale, qv.w * a.q_scale, part);
    int base, nv;
    halving_reduce<S::NV, S::PAIRS>(part, lane, base, nv);
    if ((lane & S::bfly_mask()) == 0) {
        const int64_t yrow = vr * a.sy_slot + g * a.sy_group;
#pragma unroll
        for (int j = 0; j < S::NV; ++j) {
            if (j < nv) {
                const int vi = base + j;
                store_y(a, yrow, 2 * ((vi >> 1) * S::ROWS_PER_IT + r0) + (vi & 1), part[j]);
            }
        }
    }
}

// ------------------------------- 1..4 states, rotations, all loads in flight --
// Every state of the (slot, group) is loaded before any is updated, so the M
// state streams overlap; each state's lane partials of S_m q~ are rotated by
// r_m and summed in registers, and one halving reduction produces y (no LDS).
template <int D>
constexpr int multi_threads() { return 1024; }  // at d = 64, M = 3: 72 % of HBM against 70 % with 512

template <int D, int MS, bool PL>
__global__ void __launch_bounds__((DecodeShape<D, multi_threads<D>()>::THREADS)) decode_multi_kernel(qpam_decode_args a) {
    using S = DecodeShape<D, multi_threads<D>()>;
    const int tid = threadIdx.x;
    const int ai = blockIdx.x / a.n_groups;
    const int g = blockIdx.x - ai * a.n_groups;
    const int slot = a.active ? a.active[ai] : ai;
    if (slot < 0 || slot >= a.n_slots) return;
    const int vr = a.vec_by_rank ? ai : slot;   // row of q, k, v, gamma, rot, y
    const int cp = tid % S::PAIRS, r0 = tid / S::PAIRS, lane = tid & 63;
    float *st0 = a.state + slot * a.st_slot + g * a.st_group;
    floatx4 s[MS][S::ITERS];
#pragma unroll
    for (int m = 0; m < MS; ++m)
#pragma unroll
        for (int it = 0; it < S::ITERS; ++it)
            s[m][it] = __builtin_nontemporal_load(
                reinterpret_cast<const floatx4 *>(st0 + m * a.st_state + 4 * (it * S::THREADS + tid)));
    float4 qv = load_pair<PL>(a.q, a.q_im, vr * a.sq_slot + g * a.sq_group, cp);
    float4 kv = load_pair<PL>(a.k, a.k_im, vr * a.sk_slot + g * a.sk_group, cp);
    apply_rope<D>(a, slot, cp, qv, kv);
    const float q0r = qv.x * a.q_scale, q0i = qv.y * a.q_scale, q1r = qv.z * a.q_scale, q1i = qv.w * a.q_scale;
    const int64_t vo = vr * a.sv_slot + g * a.sv_group;
    const float *vrow = a.v + vo, *vrow_im = PL ? a.v_im + vo : nullptr;
    float2 vv[S::ITERS];
#pragma unroll
    for (int it = 0; it < S::ITERS; ++it) vv[it] = load_one<PL>(vrow, vrow_im, it * S::ROWS_PER_IT + r0);
    float tot[S::NV];
#pragma unroll
    for (int j = 0; j < S::NV; ++j) tot[j] = 0.f;
#pragma unroll
    for (int m = 0; m < MS; ++m) {
        const float2 gam = lane_decay(a, vr * a.sg_slot + g * a.sg_group + m * a.sg_state, cp);
        float rr = 1.f, ri = 0.f;
        if (a.rot) {
            const int64_t ro = vr * a.sr_slot + g * a.sr_group + m * a.sr_state;
            rr = a.rot[ro];
            ri = a.rot_im ? a.rot_im[ro] : a.rot[ro + 1];
        }
#pragma unroll
        for (int it = 0; it < S::ITERS; ++it) {
            const float o0r = vv[it].x * kv.x + vv[it].y * kv.y, o0i = vv[it].y * kv.x - vv[it].x * kv.y;
            const float o1r = vv[it].x * kv.z + vv[it].y * kv.w, o1i = vv[it].y * kv.z - vv[it].x * kv.w;
            floatx4 n;
            n.x = gam.x * s[m][it].x + o0r;
            n.y = gam.x * s[m][it].y + o0i;
            n.z = gam.y * s[m][it].z + o1r;
            n.w = gam.y * s[m][it].w + o1i;
            __builtin_nontemporal_store(n, reinterpret_cast<floatx4 *>(st0 + m * a.st_state + 4 * (it * S::THREADS + tid)));
            const float pr = n.x * q0r - n.y * q0i + n.z * q1r - n.w * q1i;
            const float pi = n.x * q0i + n.y * q0r + n.z * q1i + n.w * q1r;
            tot[2 * it] += rr * pr - ri * pi;
            tot[2 * it + 1] += rr * pi + ri * pr;
        }
    }
    int base, nv;
    halving_reduce<S::NV, S::PAIRS>(tot, lane, base, nv);
    if ((lane & S::bfly_mask()) == 0) {
        const int64_t yrow = vr * a.sy_slot + g * a.sy_group;
#pragma unroll
        for (int j = 0; j < S::NV; ++j) {
            if (j < nv) {
                const int vi = base + j;
                store_y(a, yrow, 2 * ((vi >> 1) * S::ROWS_PER_IT + r0) + (vi & 1), tot[j]);
            }
        }
    }
}

// ------------------------------------ the decode prologue fused (d = 64) --
// One block per (row, group g) as the multi-state kernel, with q, k, v, the
// decays and the rotations formed from the layer's projection row and gate
// logits instead of read: qpam_prologue_fwd's formulas in its order (q and k
// normalised per element before the RoPE this kernel applies, as the unfused
// engine does: |rope| = 1), so the prologue's launch and its fp32 planes go.
template <typename TP> __device__ __forceinline__ float pld(const void *p, int64_t i);
template <> __device__ __forceinline__ float pld<float>(const void *p, int64_t i) { return static_cast<const float *>(p)[i]; }
template <> __device__ __forceinline__ float pld<unsigned short>(const void *p, int64_t i) {
    return bf16_to_f32(static_cast<const unsigned short *>(p)[i]);
}
// elements i, i + 1 (i even)
template <typename TP> __device__ __forceinline__ float2 pld2(const void *p, int64_t i);
template <> __device__ __forceinline__ float2 pld2<float>(const void *p, int64_t i) {
    return *reinterpret_cast<const float2 *>(static_cast<const float *>(p) + i);
}
template <> __device__ __forceinline__ float2 pld2<unsigned short>(const void *p, int64_t i) {
    const unsigned u = *reinterpret_cast<const unsigned *>(static_cast<const unsigned short *>(p) + i);
    return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xffff0000u));
}
__device__ __forceinline__ float p_softplus(float x) { return x > 20.f ? x : log1pf(expf(x)); }
__device__ __forceinline__ float p_sigmoid(float x) { return 1.f / (1.f + expf(-x)); }
__device__ __forceinline__ void p_nrm(float &re, float &im) {
    const float inv = 1.f / sqrtf(re * re + im * im + 1e-8f);
    re *= inv, im *= inv;
}

template <int MS, typename TP>
__global__ void __launch_bounds__((DecodeShape<64, multi_threads<64>()>::THREADS)) decode_proj_kernel(qpam_decode_args a) {
    constexpr int D = 64;
    using S = DecodeShape<D, multi_threads<D>()>;
    const int tid = threadIdx.x;
    const int ai = blockIdx.x / a.n_groups;
    const int g = blockIdx.x - ai * a.n_groups;
    const int slot = a.active ? a.active[ai] : ai;
    if (slot < 0 || slot >= a.n_slots) return;
    const int vr = a.vec_by_rank ? ai : slot;   // row of proj, gate, y
    const int cp = tid % S::PAIRS, r0 = tid / S::PAIRS, lane = tid & 63;
    float *st0 = a.state + slot * a.st_slot + g * a.st_group;
    floatx4 s[MS][S::ITERS];
#pragma unroll
    for (int m = 0; m < MS; ++m)
#pragma unroll
        for (int it = 0; it < S::ITERS; ++it)
            s[m][it] = __builtin_nontemporal_load(
                reinterpret_cast<const floatx4 *>(st0 + m * a.st_state + 4 * (it * S::THREADS + tid)));
    const int64_t GD = (int64_t)a.n_groups * D, prow = (int64_t)vr * a.proj_ld, col = (int64_t)g * D;
    const float2 qre = pld2<TP>(a.proj, prow + col + 2 * cp), qim = pld2<TP>(a.proj, prow + 3 * GD + col + 2 * cp);
    const float2 kre = pld2<TP>(a.proj, prow + GD + col + 2 * cp), kim = pld2<TP>(a.proj, prow + 4 * GD + col + 2 * cp);
    float4 qv = make_float4(qre.x, qim.x, qre.y, qim.y), kv = make_float4(kre.x, kim.x, kre.y, kim.y);
    if (a.qk_norm) {
        p_nrm(qv.x, qv.y), p_nrm(qv.z, qv.w);
        p_nrm(kv.x, kv.y), p_nrm(kv.z, kv.w);
    }
    apply_rope<D>(a, slot, cp, qv, kv);
    const float q0r = qv.x * a.q_scale, q0i = qv.y * a.q_scale, q1r = qv.z * a.q_scale, q1i = qv.w * a.q_scale;
    // the gates of (row, group), formed once per block (lane m of wave 0: state m's
    // decay and rotation) while the state loads are in flight, shared through LDS
    __shared__ float sc[4][3], skeep;
    const int64_t grow = (int64_t)vr * a.gate_ld;
    if (tid < MS) {
        const float p = (a.gate && a.protect_col >= 0) ? p_sigmoid(pld<TP>(a.gate, grow + a.protect_col + g)) : 0.f;
        const float dt = pld<TP>(a.proj, prow + 6 * GD + g) + a.dt_bias[g];
        float base = expf(-p_softplus(dt + (a.state_offset ? a.state_offset[tid] : 0.f)));
        if (a.gamma_floor > 0.f) base = a.gamma_floor + (1.f - a.gamma_floor) * base;
        sc[tid][0] = base * (1.f - p) + p;
        float rr = 1.f, ri = 0.f;
        if (a.gate && a.phase_col >= 0) sincosf(pld<TP>(a.gate, grow + a.phase_col + g * MS + tid), &ri, &rr);
        sc[tid][1] = rr, sc[tid][2] = ri;
        if (tid == 0) skeep = 1.f - p;
    }
    __syncthreads();
    const float keep = skeep;
    float2 vv[S::ITERS];
#pragma unroll
    for (int it = 0; it < S::ITERS; ++it) {
        const int row = it * S::ROWS_PER_IT + r0;
        vv[it] = make_float2(pld<TP>(a.proj, prow + 2 * GD + col + row) * keep,
                             pld<TP>(a.proj, prow + 5 * GD + col + row) * keep);
    }
    float tot[S::NV];
#pragma unroll
    for (int j = 0; j < S::NV; ++j) tot[j] = 0.f;
#pragma unroll
    for (int m = 0; m < MS; ++m) {
        const float gam = sc[m][0], rr = sc[m][1], ri = sc[m][2];
#pragma unroll
        for (int it = 0; it < S::ITERS; ++it) {
            const float o0r = vv[it].x * kv.x + vv[it].y * kv.y, o0i = vv[it].y * kv.x - vv[it].x * kv.y;
            const float o1r = vv[it].x * kv.z + vv[it].y * kv.w, o1i = vv[it].y * kv.z - vv[it].x * kv.w;
            floatx4 n;
            n.x = gam * s[m][it].x + o0r;
            n.y = gam * s[m][it].y + o0i;
            n.z = gam * s[m][it].z + o1r;
            n.w = gam * s[m][it].w + o1i;
            __builtin_nontemporal_store(n, reinterpret_cast<floatx4 *>(st0 + m * a.st_state + 4 * (it * S::THREADS + tid)));
            const float pr = n.x * q0r - n.y * q0i + n.z * q1r - n.w * q1i;
            const float pi = n.x * q0i + n.y * q0r + n.z * q1i + n.w * q1r;
            tot[2 * it] += rr * pr - ri * pi;
            tot[2 * it + 1] += rr * pi + ri * pr;
        }
    }
    int base, nv;
    halving_reduce<S::NV, S::PAIRS>(tot, lane, base, nv);
    if ((lane & S::bfly_mask()) == 0) {
        const int64_t yrow = vr * a.sy_slot + g * a.sy_group;
#pragma unroll
        for (int j = 0; j < S::NV; ++j) {
            if (j < nv) {
                const int vi = base + j;
                store_y(a, yrow, 2 * ((vi >> 1) * S::ROWS_PER_IT + r0) + (vi & 1), tot[j]);
            }
        }
    }
}

template <typename TP>
int launch_decode_proj(const qpam_decode_args &a, hipStream_t stream) {
    const long long blocks = (long long)a.n_active * a.n_groups;
    if (blocks == 0) return QPAM_OK;
    constexpr int MT = DecodeShape<64, multi_threads<64>()>::THREADS;
    switch (a.n_states) {
        case 1: hipLaunchKernelGGL((decode_proj_kernel<1, TP>), dim3((unsigned)blocks), dim3(MT), 0, stream, a); break;
        case 2: hipLaunchKernelGGL((decode_proj_kernel<2, TP>), dim3((unsigned)blocks), dim3(MT), 0, stream, a); break;
        case 3: hipLaunchKernelGGL((decode_proj_kernel<3, TP>), dim3((unsigned)blocks), dim3(MT), 0, stream, a); break;
        default: hipLaunchKernelGGL((decode_proj_kernel<4, TP>), dim3((unsigned)blocks), dim3(MT), 0, stream, a);
    }
    return launch_status("decode_proj_kernel");
}

// ------------------------------------------------ M states, rotations -----
template <int D>
constexpr int general_threads() { return D >= 128 ? 1024 : 256; }  // 8 float4 of state per lane at d = 64, 128

template <int D, bool PL>
__global__ void __launch_bounds__((DecodeShape<D, general_threads<D>()>::THREADS)) decode_general_kernel(qpam_decode_args a) {
    using S = DecodeShape<D, general_threads<D>()>;
    __shared__ float ys[D][2];

    const int tid = threadIdx.x;
    const int ai = blockIdx.x / a.n_groups;
    const int g = blockIdx.x - ai * a.n_groups;
    const int slot = a.active ? a.active[ai] : ai;
    if (slot < 0 || slot >= a.n_slots) return;  // whole block exits together
    const int vr = a.vec_by_rank ? ai : slot;   // row of q, k, v, gamma, rot, y

    const int cp = tid % S::PAIRS;      // this lane's key-column pair: j = 2cp, 2cp+1
    const int r0 = tid / S::PAIRS;      // first row of this lane
    const int lane = tid & 63;

    float4 qv = load_pair<PL>(a.q, a.q_im, vr * a.sq_slot + g * a.sq_group, cp);
    float4 kv = load_pair<PL>(a.k, a.k_im, vr * a.sk_slot + g * a.sk_group, cp);
    apply_rope<D>(a, slot, cp, qv, kv);
    const int64_t vo = vr * a.sv_slot + g * a.sv_group;
    const float *vrow = a.v + vo, *vrow_im = PL ? a.v_im + vo : nullptr;

    float yacc_r = 0.f, yacc_i = 0.f;  // lanes tid < D accumulate row tid
    for (int m = 0; m < a.n_states; ++m) {
        const float2 gam = lane_decay(a, vr * a.sg_slot + g * a.sg_group + m * a.sg_state, cp);
        float part[S::NV];
        update_state<S, PL>(a.state + slot * a.st_slot + g * a.st_group + m * a.st_state, tid, r0, gam, vrow, vrow_im, kv,
                        qv.x * a.q_scale, qv.y * a.q_scale, qv.z * a.q_scale, qv.w * a.q_scale, part);
        int base, nv;
        halving_reduce<S::NV, S::PAIRS>(part, lane, base, nv);
#pragma unroll
        for (int j = 0; j < S::NV; ++j) {
            if (j < nv) {
                const int vi = base + j;
                ys[(vi >> 1) * S::ROWS_PER_IT + r0][vi & 1] = part[j];
            }
        }
        __syncthreads();
        if (tid < D) {
            const float yr = ys[tid][0], yi = ys[tid][1];
            if (a.rot) {
                const int64_t ro = vr * a.sr_slot + g * a.sr_group + m * a.sr_state;
                const float rr = a.rot[ro], ri = a.rot_im ? a.rot_im[ro] : a.rot[ro + 1];
                yacc_r += rr * yr - ri * yi;
                yacc_i += rr * yi + ri * yr;
            } else {
                yacc_r += yr;
                yacc_i += yi;
            }
        }
        __syncthreads();
    }
    if (tid < D) {
        const int64_t yrow = vr * a.sy_slot + g * a.sy_group;
        if (a.y_dtype == QPAM_BF16) {
            *reinterpret_cast<unsigned *>(reinterpret_cast<unsigned short *>(a.y) + yrow + 2 * tid) =
                pack_bf16x2(yacc_r, yacc_i);
        } else {
            *reinterpret_cast<float2 *>(a.y + yrow + 2 * tid) = make_float2(yacc_r, yacc_i);
        }
    }
}

template <int D, bool PL>
int launch_decode_pl(const qpam_decode_args &a, hipStream_t stream) {
    const long long blocks = (long long)a.n_active * a.n_groups;
    if (blocks == 0) return QPAM_OK;
    if (a.n_states == 1 && a.rot == nullptr) {
        hipLaunchKernelGGL((decode_single_kernel<D, PL>), dim3((unsigned)blocks), dim3(DecodeShape<D, 512>::THREADS), 0,
                           stream, a);
        return launch_status("decode_single_kernel");
    }
    constexpr int MT = DecodeShape<D, multi_threads<D>()>::THREADS;
    // the multi-state kernel holds M x ITERS float4 of state per lane: up to 4
    // states of a 64 x 64 state, one of a 128 x 128 state (more would spill)
    constexpr int MAX_MS = D >= 128 ? 1 : 4;
    switch (a.n_states) {
        case 1:
            hipLaunchKernelGGL((decode_multi_kernel<D, 1, PL>), dim3((unsigned)blocks), dim3(MT), 0, stream, a);
            return launch_status("decode_multi_kernel<1>");
        case 2:
            if constexpr (MAX_MS >= 2) {
                hipLaunchKernelGGL((decode_multi_kernel<D, 2, PL>), dim3((unsigned)blocks), dim3(MT), 0, stream, a);
                return launch_status("decode_multi_kernel<2>");
            }
            break;
        case 3:
            if constexpr (MAX_MS >= 3) {
                hipLaunchKernelGGL((decode_multi_kernel<D, 3, PL>), dim3((unsigned)blocks), dim3(MT), 0, stream, a);
                return launch_status("decode_multi_kernel<3>");
            }
            break;
        case 4:
            if constexpr (MAX_MS >= 4) {
                hipLaunchKernelGGL((decode_multi_kernel<D, 4, PL>), dim3((unsigned)blocks), dim3(MT), 0, stream, a);
                return launch_status("decode_multi_kernel<4>");
            }
            break;
        default:
            break;
    }
    hipLaunchKernelGGL((decode_general_kernel<D, PL>), dim3((unsigned)blocks), dim3(DecodeShape<D, general_threads<D>()>::THREADS), 0, stream,
                       a);
    return launch_status("decode_general_kernel");
}

// planar q, k, v (q_im set) or interleaved rows
template <int D>
int launch_decode(const qpam_decode_args &a, hipStream_t stream) {
    return a.q_im ? launch_decode_pl<D, true>(a, stream) : launch_decode_pl<D, false>(a, stream);
}

// ------------------------------------------------ backward of one step --
// One block per state.  Lane (r0, cp) owns key columns 2 cp, 2 cp + 1 and rows
// r0, r0 + ROWS_PER_IT, ...: it recomputes S' from S, forms
// G = dS' + dy conj(q) (the gradient of S'), writes dS = gamma G, and keeps its
// partial column sums of dq = S'^H dy, dk_j = sum_i v_i conj(G_ij) and
// dgamma_j = sum_i Re(conj(S_ij) G_ij) and its row sums of dv = G k; both are
// summed through LDS in a fixed order.
template <int D>
constexpr int bwd_threads() { return (D * D / 2) < 256 ? (D * D / 2) : 256; }

template <int D>
__global__ void __launch_bounds__(bwd_threads<D>()) decode_bwd_kernel(qpam_decode_bwd_args a) {
    using S = DecodeShape<D, bwd_threads<D>()>;
    constexpr int NC = 10;                           // column partials: dq, dk (re, im x 2), dgamma x 2
    __shared__ float cols[S::THREADS * NC];          // [r0][cp][NC]
    __shared__ float rows[D * S::PAIRS * 2];         // [i][cp][re, im]
    __shared__ float gsum[S::PAIRS];
    const int64_t e = blockIdx.x;
    const int tid = threadIdx.x, cp = tid % S::PAIRS, r0 = tid / S::PAIRS;
    const float *st = a.state + e * D * D * 2;
    const float *gst = a.dstate_new ? a.dstate_new + e * D * D * 2 : nullptr;
    float *dst = a.dstate + e * D * D * 2;
    const float4 q = *reinterpret_cast<const float4 *>(a.q + e * D * 2 + 4 * cp);
    const float4 k = *reinterpret_cast<const float4 *>(a.k + e * D * 2 + 4 * cp);
    float g0, g1;
    if (a.gamma_per_channel) {
        g0 = a.gamma[e * D + 2 * cp];
        g1 = a.gamma[e * D + 2 * cp + 1];
    } else {
        g0 = g1 = a.gamma[e];
    }
    float c[NC];
#pragma unroll
    for (int x = 0; x < NC; ++x) c[x] = 0.f;
#pragma unroll
    for (int it = 0; it < S::ITERS; ++it) {
        const int i = it * S::ROWS_PER_IT + r0;
        const int64_t o = (int64_t)i * D * 2 + 4 * cp;
        const float4 s = *reinterpret_cast<const float4 *>(st + o);
        const float4 gs = gst ? *reinterpret_cast<const float4 *>(gst + o) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float2 v = *reinterpret_cast<const float2 *>(a.v + e * D * 2 + 2 * i);
        const float2 dy = *reinterpret_cast<const float2 *>(a.dy + e * D * 2 + 2 * i);
        // S' = gamma S + v conj(k)
        const float p0r = g0 * s.x + v.x * k.x + v.y * k.y, p0i = g0 * s.y + v.y * k.x - v.x * k.y;
        const float p1r = g1 * s.z + v.x * k.z + v.y * k.w, p1i = g1 * s.w + v.y * k.z - v.x * k.w;
        // G = dS' + dy conj(q)
        const float G0r = gs.x + dy.x * q.x + dy.y * q.y, G0i = gs.y + dy.y * q.x - dy.x * q.y;
        const float G1r = gs.z + dy.x * q.z + dy.y * q.w, G1i = gs.w + dy.y * q.z - dy.x * q.w;
        *reinterpret_cast<float4 *>(dst + o) = make_float4(g0 * G0r, g0 * G0i, g1 * G1r, g1 * G1i);
        // dq_j += conj(S'_ij) dy_i
        c[0] += p0r * dy.x + p0i * dy.y;
        c[1] += p0r * dy.y - p0i * dy.x;
        c[2] += p1r * dy.x + p1i * dy.y;
        c[3] += p1r * dy.y - p1i * dy.x;
        // dk_j += v_i conj(G_ij)
        c[4] += v.x * G0r + v.y * G0i;
        c[5] += v.y * G0r - v.x * G0i;
        c[6] += v.x * G1r + v.y * G1i;
        c[7] += v.y * G1r - v.x * G1i;
        // dgamma_j += Re(conj(S_ij) G_ij)
        c[8] += s.x * G0r + s.y * G0i;
        c[9] += s.z * G1r + s.w * G1i;
        // dv_i partial: G_i,2cp k_2cp + G_i,2cp+1 k_2cp+1
        rows[(i * S::PAIRS + cp) * 2] = G0r * k.x - G0i * k.y + G1r * k.z - G1i * k.w;
        rows[(i * S::PAIRS + cp) * 2 + 1] = G0r * k.y + G0i * k.x + G1r * k.w + G1i * k.z;
    }
#pragma unroll
    for (int x = 0; x < NC; ++x) cols[(r0 * S::PAIRS + cp) * NC + x] = c[x];
    __syncthreads();
    if (tid < S::PAIRS) {  // column pair cp = tid: sum over the row groups in order
        float t[NC];
#pragma unroll
        for (int x = 0; x < NC; ++x) t[x] = 0.f;
        for (int r = 0; r < S::ROWS_PER_IT; ++r)
#pragma unroll
            for (int x = 0; x < NC; ++x) t[x] += cols[(r * S::PAIRS + tid) * NC + x];
        *reinterpret_cast<float4 *>(a.dq + e * D * 2 + 4 * tid) = make_float4(t[0], t[1], t[2], t[3]);
        *reinterpret_cast<float4 *>(a.dk + e * D * 2 + 4 * tid) = make_float4(t[4], t[5], t[6], t[7]);
        if (a.gamma_per_channel) {
            a.dgamma[e * D + 2 * tid] = t[8];
            a.dgamma[e * D + 2 * tid + 1] = t[9];
        } else {
            gsum[tid] = t[8] + t[9];
        }
    }
    if (tid < D) {  // row i = tid: sum over the column pairs in order
        float vr = 0.f, vi = 0.f;
        for (int p = 0; p < S::PAIRS; ++p) {
            vr += rows[(tid * S::PAIRS + p) * 2];
            vi += rows[(tid * S::PAIRS + p) * 2 + 1];
        }
        *reinterpret_cast<float2 *>(a.dv + e * D * 2 + 2 * tid) = make_float2(vr, vi);
    }
    if (!a.gamma_per_channel) {
        __syncthreads();
        if (tid == 0) {
            float x = 0.f;
            for (int p = 0; p < S::PAIRS; ++p) x += gsum[p];
            a.dgamma[e] = x;
        }
    }
}

bool aligned(const void *p, int bytes) { return ((uintptr_t)p % bytes) == 0; }

}  // namespace
}  // namespace qpam

extern "C" int qpam_decode_step(const qpam_decode_args *a, void *stream) {
    using namespace qpam;
    QPAM_REQUIRE(a != nullptr, "qpam_decode_step: null args");
    QPAM_REQUIRE(a->n_slots >= 0 && a->n_active >= 0 && a->n_groups >= 1 && a->n_states >= 1,
                 "qpam_decode_step: bad sizes (slots %d active %d groups %d states %d)", a->n_slots,
                 a->n_active, a->n_groups, a->n_states);
    QPAM_REQUIRE(a->active != nullptr || a->n_active <= a->n_slots,
                 "qpam_decode_step: n_active > n_slots without an active list");
    if (a->proj) {  // the decode prologue fused (ABI 12)
        QPAM_REQUIRE(a->state && a->y && a->dt_bias, "qpam_decode_step: state, y and dt_bias required with proj");
        QPAM_REQUIRE(a->d == 64 && a->n_states <= 4, "qpam_decode_step: proj needs d = 64 and at most 4 states");
        QPAM_REQUIRE(a->proj_dtype == QPAM_F32 || a->proj_dtype == QPAM_BF16,
                     "qpam_decode_step: proj_dtype must be F32 or BF16");
        QPAM_REQUIRE(a->y_dtype == QPAM_F32 || a->y_dtype == QPAM_BF16, "qpam_decode_step: y_dtype must be F32 or BF16");
        QPAM_REQUIRE(a->active != nullptr || a->n_active <= a->n_slots,
                     "qpam_decode_step: n_active > n_slots without an active list");
        QPAM_REQUIRE(a->rope == nullptr || (a->pos != nullptr && a->rope_len >= 1 && aligned(a->rope, 16)),
                     "qpam_decode_step: rope needs positions, rope_len >= 1 and a 16-byte aligned table");
        QPAM_REQUIRE((long long)a->n_active * a->n_groups < (1ll << 31), "qpam_decode_step: grid too large");
        QPAM_REQUIRE(a->gamma_per_channel == 0, "qpam_decode_step: proj takes head decays only");
        QPAM_REQUIRE(a->proj_ld >= 6ll * a->n_groups * 64 + a->n_groups && a->proj_ld % 2 == 0 && aligned(a->proj, 8),
                     "qpam_decode_step: proj rows of >= 6 G d + G elements, an even stride, 8-byte aligned");
        QPAM_REQUIRE(a->gate || (a->protect_col < 0 && a->phase_col < 0),
                     "qpam_decode_step: protect_col / phase_col need gate");
        QPAM_REQUIRE(aligned(a->state, 16) && aligned(a->y, 8) && a->st_slot % 4 == 0 && a->st_group % 4 == 0 &&
                         a->st_state % 4 == 0 && a->sy_slot % 2 == 0 && a->sy_group % 2 == 0,
                     "qpam_decode_step: misaligned state or y");
        hipStream_t s = (hipStream_t)stream;
        return a->proj_dtype == QPAM_BF16 ? launch_decode_proj<unsigned short>(*a, s) : launch_decode_proj<float>(*a, s);
    }
    QPAM_REQUIRE(a->state && a->q && a->k && a->v && a->gamma && a->y, "qpam_decode_step: null pointer");
    QPAM_REQUIRE(a->rope == nullptr || (a->pos != nullptr && a->rope_len >= 1 && aligned(a->rope, 16)),
                 "qpam_decode_step: rope needs positions, rope_len >= 1 and a 16-byte aligned table");
    QPAM_REQUIRE((long long)a->n_active * a->n_groups < (1ll << 31), "qpam_decode_step: grid too large");
    QPAM_REQUIRE(a->rot_im == nullptr || a->rot != nullptr, "qpam_decode_step: rot_im without rot");
    QPAM_REQUIRE(a->gamma_per_channel == 0 || a->gamma_per_channel == 1,
                 "qpam_decode_step: gamma_per_channel must be 0 or 1");
    QPAM_REQUIRE(a->y_dtype == QPAM_F32 || a->y_dtype == QPAM_BF16, "qpam_decode_step: y_dtype must be F32 or BF16");
    const bool planar = a->q_im != nullptr;
    QPAM_REQUIRE((a->k_im != nullptr) == planar && (a->v_im != nullptr) == planar,
                 "qpam_decode_step: q_im, k_im and v_im are all set (planar q, k, v) or all NULL");
    // 16-byte vector access of S and interleaved q, k (8-byte planar), 8-byte access of v (4-byte planar), y
    const int qa = planar ? 8 : 16, va = planar ? 4 : 8, qs = planar ? 2 : 4, vs = planar ? 1 : 2;
    QPAM_REQUIRE(aligned(a->state, 16) && aligned(a->q, qa) && aligned(a->k, qa) && aligned(a->v, va) &&
                     (!planar || (aligned(a->q_im, qa) && aligned(a->k_im, qa) && aligned(a->v_im, va))) &&
                     aligned(a->y, 8),
                 "qpam_decode_step: misaligned operand");
    QPAM_REQUIRE(a->st_slot % 4 == 0 && a->st_group % 4 == 0 && a->st_state % 4 == 0 && a->sq_slot % qs == 0 &&
                     a->sq_group % qs == 0 && a->sk_slot % qs == 0 && a->sk_group % qs == 0 &&
                     a->sv_slot % vs == 0 && a->sv_group % vs == 0 && a->sy_slot % 2 == 0 && a->sy_group % 2 == 0,
                 "qpam_decode_step: strides must keep the vector accesses of S, q, k, v and y aligned");
    hipStream_t s = (hipStream_t)stream;
    switch (a->d) {
        case 16: return launch_decode<16>(*a, s);
        case 32: return launch_decode<32>(*a, s);
        case 64: return launch_decode<64>(*a, s);
        case 128: return launch_decode<128>(*a, s);
        default: return fail(QPAM_ERR_UNSUPPORTED, "qpam_decode_step: d=%d (supported 16, 32, 64, 128)", a->d);
    }
}

extern "C" int qpam_decode_step_bwd(const qpam_decode_bwd_args *a, void *stream) {
    using namespace qpam;
    QPAM_REQUIRE(a != nullptr, "qpam_decode_step_bwd: null args");
    QPAM_REQUIRE(a->n >= 0 && a->n < (1ll << 31), "qpam_decode_step_bwd: bad n %lld", (long long)a->n);
    QPAM_REQUIRE(a->gamma_per_channel == 0 || a->gamma_per_channel == 1,
                 "qpam_decode_step_bwd: gamma_per_channel must be 0 or 1");
    QPAM_REQUIRE(a->state && a->gamma && a->q && a->k && a->v && a->dy && a->dstate && a->dgamma && a->dq && a->dk &&
                     a->dv,
                 "qpam_decode_step_bwd: null pointer");
    QPAM_REQUIRE(aligned(a->state, 16) && aligned(a->q, 16) && aligned(a->k, 16) && aligned(a->v, 8) &&
                     aligned(a->dy, 8) && aligned(a->dstate, 16) && aligned(a->dq, 16) && aligned(a->dk, 16) &&
                     aligned(a->dv, 8) && (a->dstate_new == nullptr || aligned(a->dstate_new, 16)),
                 "qpam_decode_step_bwd: misaligned operand");
    if (a->n == 0) return QPAM_OK;
    hipStream_t s = (hipStream_t)stream;
    const dim3 grid((unsigned)a->n);
    switch (a->d) {
        case 16: hipLaunchKernelGGL(decode_bwd_kernel<16>, grid, dim3(bwd_threads<16>()), 0, s, *a); break;
        case 32: hipLaunchKernelGGL(decode_bwd_kernel<32>, grid, dim3(bwd_threads<32>()), 0, s, *a); break;
        case 64: hipLaunchKernelGGL(decode_bwd_kernel<64>, grid, dim3(bwd_threads<64>()), 0, s, *a); break;
        case 128: hipLaunchKernelGGL(decode_bwd_kernel<128>, grid, dim3(bwd_threads<128>()), 0, s, *a); break;
        default: return fail(QPAM_ERR_UNSUPPORTED, "qpam_decode_step_bwd: d=%d (supported 16, 32, 64, 128)", a->d);
    }
    return launch_status("decode_bwd_kernel");
}
