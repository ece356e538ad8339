// Tied complex LM-head cross-entropy (fused GEMM + softmax statistics).
//
// Reference: _FusedLinearCE (v11/fused_ce.py:26-82), linear_ce_per_token and
// linear_ce_stats (v11/fused_ce.py:98-141), called from V11LM.ce_from_lm
// (v11/model.py:1175-1190) with H = [lm_r | lm_i], W = [E_r | E_i] so that
// H W^T = Re(h conj(E)^T).
//
// Forward: one MFMA GEMM tile per (rows, vocab) block (256 x 128 for bf16,
// 128 x 128 for fp32) whose epilogue reduces the tile to per-row (max, sum exp,
// argmax); logits never leave registers.  A per-row finalize merges the vocab
// tiles into lse, adds the target logit (a direct dot product) and writes the
// per-row loss; a single-block reduction produces the loss sum and the
// denominator.
// Backward, per `chunk` rows: the same GEMM recomputes the logits tile and its
// epilogue writes G = (softmax - onehot) * scale in the input dtype as
// G^T [vocab][rows] (and G [rows][vocab] where a hand-written GEMM reads it);
// then the two plain GEMMs dW += G^T H and dH = G W run through hipBLASLt
// (bf16, blas.hip) or through the hand-written K-contiguous GEMM kernels (W^T
// and H^T transposed once into the workspace).  The G buffers hold `chunk`
// rows, the reference's own memory bound (it keeps chunk x V fp32 logits and
// softmax alive).
#include <algorithm>

#include "blas.h"
#include "common.h"

namespace qpam {
namespace ce {
namespace {

constexpr int THREADS = 256;
constexpr int BM = 128, BN = 128, BK = 32;
constexpr int VT = 128;  // vocab tile

template <typename T> struct Mma;

// bf16 inputs: v_mfma_f32_16x16x32_bf16, lane supplies 8 consecutive k
template <> struct Mma<unsigned short> {
    static constexpr int PITCH = BK + 8;  // elements per LDS row (80 bytes)
    static constexpr int ROW16 = BK * 2 / 16;  // 16-byte chunks per tile row
    __device__ __forceinline__ static void step(const unsigned short *sA, const unsigned short *sB, int arow0,
                                                int brow0, floatx4 (&acc)[4][4], int l16, int g) {
        bf16x8 af[4], bfr[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            af[i] = *reinterpret_cast<const bf16x8 *>(sA + (arow0 + 16 * i + l16) * PITCH + 8 * g);
            bfr[i] = *reinterpret_cast<const bf16x8 *>(sB + (brow0 + 16 * i + l16) * PITCH + 8 * g);
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
                acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], bfr[ni], acc[mi][ni], 0, 0, 0);
    }
};

// fp32 inputs: v_mfma_f32_16x16x4_f32, k-steps use k = 16q + 4g + kk
template <> struct Mma<float> {
    static constexpr int PITCH = BK + 4;
    static constexpr int ROW16 = BK * 4 / 16;
    __device__ __forceinline__ static void step(const float *sA, const float *sB, int arow0, int brow0,
                                                floatx4 (&acc)[4][4], int l16, int g) {
#pragma unroll
        for (int q = 0; q < BK / 16; ++q) {
            float4 af[4], bfr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                af[i] = *reinterpret_cast<const float4 *>(sA + (arow0 + 16 * i + l16) * PITCH + 16 * q + 4 * g);
                bfr[i] = *reinterpret_cast<const float4 *>(sB + (brow0 + 16 * i + l16) * PITCH + 16 * q + 4 * g);
            }
#pragma unroll
            for (int kk = 0; kk < 4; ++kk)
#pragma unroll
                for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                    for (int ni = 0; ni < 4; ++ni)
                        acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x4f32(af[mi][kk], bfr[ni][kk], acc[mi][ni], 0,
                                                                           0, 0);
        }
    }
};

template <typename T>
constexpr size_t gemm_smem() { return (size_t)2 * (BM + BN) * Mma<T>::PITCH * sizeof(T); }

// C[m][n] = sum_k A[m][k] B[n][k] for one BM x BN tile; A and B point at the
// tile's first row; rows beyond a_rows / b_rows read as zero; K % BK == 0.
// Wave w owns rows 64*(w>>1).., cols 64*(w&1)..; acc[mi][ni] lane holds
// C[64*(w>>1) + 16mi + 4g + r][64*(w&1) + 16ni + l16].
template <typename T>
__device__ __forceinline__ void gemm_tile(const T *A, int64_t lda, int a_rows, const T *B, int64_t ldb, int b_rows,
                                          int K, floatx4 (&acc)[4][4], T *smem) {
    using MM = Mma<T>;
    constexpr int PITCH = MM::PITCH, R16 = MM::ROW16, EPC = 16 / sizeof(T);
    constexpr int LOADS = BM * R16 / THREADS;  // 16-byte loads per thread per operand
    T *sA[2] = {smem, smem + (BM + BN) * PITCH};
    T *sB[2] = {smem + BM * PITCH, smem + (BM + BN) * PITCH + BM * PITCH};
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int arow0 = 64 * (w >> 1), brow0 = 64 * (w & 1);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};

    uint4 ra[LOADS], rb[LOADS];
    auto gload = [&](int k0) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int ci = tid + i * THREADS, row = ci / R16, c = ci % R16;
            ra[i] = (row < a_rows) ? *reinterpret_cast<const uint4 *>(A + row * lda + k0 + c * EPC)
                                   : make_uint4(0, 0, 0, 0);
            rb[i] = (row < b_rows) ? *reinterpret_cast<const uint4 *>(B + row * ldb + k0 + c * EPC)
                                   : make_uint4(0, 0, 0, 0);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int i = 0; i < LOADS; ++i) {
            const int ci = tid + i * THREADS, row = ci / R16, c = ci % R16;
            *reinterpret_cast<uint4 *>(sA[buf] + row * PITCH + c * EPC) = ra[i];
            *reinterpret_cast<uint4 *>(sB[buf] + row * PITCH + c * EPC) = rb[i];
        }
    };
    const int KT = K / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < KT; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < KT) gload((kt + 1) * BK);
        MM::step(sA[buf], sB[buf], arow0, brow0, acc, l16, g);
        if (kt + 1 < KT) lstore(buf ^ 1);
        __syncthreads();
    }
}

// ------------------------------------------------------------ forward -----
struct FwdParams {
    qpam_ce_fwd_args a;
    int n_vt;
    float *part_m, *part_s;  // [N][n_vt]
    int *part_i;             // [N][n_vt] argmax
    float *red;              // [2] loss sum, denominator
};

template <typename T>
__global__ void __launch_bounds__(THREADS) ce_fwd_tile_kernel(FwdParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    T *smem = reinterpret_cast<T *>(smem_raw);
    __shared__ float sM[2][BM], sS[2][BM];
    __shared__ int sI[2][BM];
    const qpam_ce_fwd_args &a = p.a;
    const int vt = blockIdx.x, rt = blockIdx.y;
    const int r0 = rt * BM, v0 = vt * VT;
    floatx4 acc[4][4];
    gemm_tile<T>((const T *)a.h + (int64_t)r0 * a.ldh, a.ldh, min(BM, a.N - r0), (const T *)a.w + (int64_t)v0 * a.ldw,
                 a.ldw, min(BN, a.V - v0), a.D, acc, smem);

    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float mx = -INFINITY;
            int ix = 0x7fffffff;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const int v = v0 + 64 * wn + 16 * ni + l16;
                const float x = (v < a.V) ? acc[mi][ni][r] : -INFINITY;
                if (x > mx) { mx = x; ix = v; }
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) {
                const float om = __shfl_xor(mx, off);
                const int oi = __shfl_xor(ix, off);
                if (om > mx || (om == mx && oi < ix)) { mx = om; ix = oi; }
            }
            float s = 0.f;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const int v = v0 + 64 * wn + 16 * ni + l16;
                if (v < a.V) s += __expf(acc[mi][ni][r] - mx);
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off);
            if (l16 == 0) {
                const int row = 64 * wm + 16 * mi + 4 * g + r;
                sM[wn][row] = mx;
                sS[wn][row] = s;
                sI[wn][row] = ix;
            }
        }
    }
    __syncthreads();
    if (tid < BM && r0 + tid < a.N) {
        const float m0 = sM[0][tid], m1 = sM[1][tid];
        const float m = fmaxf(m0, m1);
        float s = 0.f;
        if (m0 > -INFINITY) s += sS[0][tid] * __expf(m0 - m);
        if (m1 > -INFINITY) s += sS[1][tid] * __expf(m1 - m);
        const int i = (m1 > m0 || (m1 == m0 && sI[1][tid] < sI[0][tid])) ? sI[1][tid] : sI[0][tid];
        const int64_t o = (int64_t)(r0 + tid) * p.n_vt + vt;
        p.part_m[o] = m;
        p.part_s[o] = s;
        p.part_i[o] = i;
    }
}

// one wave per row: merge the vocab tiles, add the target logit
template <typename T>
__global__ void __launch_bounds__(THREADS) ce_fwd_finalize_kernel(FwdParams p) {
    const qpam_ce_fwd_args &a = p.a;
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (THREADS / 64) + (threadIdx.x >> 6);
    if (row >= a.N) return;
    float m = -INFINITY, s = 0.f;
    int ix = 0x7fffffff;
    for (int vt = lane; vt < p.n_vt; vt += 64) {
        const int64_t o = (int64_t)row * p.n_vt + vt;
        const float pm = p.part_m[o], ps = p.part_s[o];
        const int pi = a.correct ? p.part_i[o] : 0;  // tile argmax, written only when requested
        if (pm > m || (pm == m && pi < ix)) ix = pi;
        const float nm = fmaxf(m, pm);
        s = (m > -INFINITY ? s * __expf(m - nm) : 0.f) + (pm > -INFINITY ? ps * __expf(pm - nm) : 0.f);
        m = nm;
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const float om = __shfl_xor(m, off), os = __shfl_xor(s, off);
        const int oi = __shfl_xor(ix, off);
        const float nm = fmaxf(m, om);
        const float ns = (m > -INFINITY ? s * __expf(m - nm) : 0.f) + (om > -INFINITY ? os * __expf(om - nm) : 0.f);
        if (om > m || (om == m && oi < ix)) ix = oi;
        m = nm;
        s = ns;
    }
    const float lse = m + __logf(s);
    const int64_t t = a.targets[row];
    const bool valid = (t != a.ignore_index) && t >= 0 && t < a.V;
    float dot = 0.f;
    if (valid) {
        const T *hr = (const T *)a.h + (int64_t)row * a.ldh;
        const T *wr = (const T *)a.w + t * a.ldw;
        for (int k = lane; k < a.D; k += 64) dot += Elem<T>::load(hr + k) * Elem<T>::load(wr + k);
    }
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) dot += __shfl_xor(dot, off);
    if (lane == 0) {
        float loss = valid ? (lse - dot) : 0.f;
        if (a.mask) loss *= a.mask[row];
        a.lse[row] = lse;
        a.loss[row] = loss;
        if (a.correct) a.correct[row] = (valid && ix == t) ? 1.f : 0.f;
    }
}

// deterministic single-block sum: red[0] = sum loss, red[1] = denominator
__global__ void __launch_bounds__(1024) ce_reduce_kernel(FwdParams p) {
    const qpam_ce_fwd_args &a = p.a;
    __shared__ float s1[32], s2[32];
    float x = 0.f, y = 0.f;
    for (int r = threadIdx.x; r < a.N; r += 1024) {
        x += a.loss[r];
        if (a.mask) {
            y += a.mask[r];
        } else {
            const int64_t t = a.targets[r];
            y += (t != a.ignore_index) ? 1.f : 0.f;
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        x += __shfl_xor(x, off);
        y += __shfl_xor(y, off);
    }
    if ((threadIdx.x & 63) == 0) {
        s1[threadIdx.x >> 6] = x;
        s2[threadIdx.x >> 6] = y;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float tx = 0.f, ty = 0.f;
        for (int i = 0; i < 16; ++i) {
            tx += s1[i];
            ty += s2[i];
        }
        a.loss_sum[0] = tx;
        a.loss_sum[1] = ty;
    }
}

// ----------------------------------------------------------- backward -----
struct BwdParams {
    qpam_ce_bwd_args a;
    int Vp;          // vocab padded to VT
    int Rp;          // chunk rows padded to BK
    int row0;        // first row of the chunk
    int rows;        // rows in the chunk
    void *wt;        // [D][Vp]
    void *gbuf;      // [rows][Vp]
    void *gtbuf;     // [Vp][Rp]
    void *ht;        // [D][Rp]
    int write_g;     // bf16 path: also write G (only the hand-written dH GEMM reads it)
};

// out[c][r] = in[r][c] for an R x Cc tile grid (64 x 64 LDS tiles); rows >= R
// and cols >= Cc of the (padded) output are written as zero.
template <typename T>
__global__ void __launch_bounds__(THREADS) transpose_kernel(const T *in, int64_t ldi, int R, int Cc, T *out,
                                                           int64_t ldo, int out_rows, int out_cols) {
    __shared__ T tile[64][65];
    const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
    for (int e = threadIdx.x; e < 64 * 64; e += THREADS) {
        const int rr = e >> 6, cc = e & 63;
        const int r = r0 + rr, c = c0 + cc;
        tile[rr][cc] = (r < R && c < Cc) ? in[(int64_t)r * ldi + c] : T(0);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < 64 * 64; e += THREADS) {
        const int cc = e >> 6, rr = e & 63;
        const int orow = c0 + cc, ocol = r0 + rr;
        if (orow < out_rows && ocol < out_cols) out[(int64_t)orow * ldo + ocol] = tile[rr][cc];
    }
}

template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ unsigned short from_f32<unsigned short>(float x) { return f32_to_bf16(x); }

// G tile: recompute logits, G = (exp(x - lse) - [v == t]) * scale; write G and G^T
template <typename T>
__global__ void __launch_bounds__(THREADS) ce_grad_tile_kernel(BwdParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    T *smem = reinterpret_cast<T *>(smem_raw);
    __shared__ float sLse[BM], sScale[BM];
    __shared__ int sTgt[BM];
    const qpam_ce_bwd_args &a = p.a;
    const int vt = blockIdx.x, rt = blockIdx.y;
    const int lr0 = rt * BM, v0 = vt * VT;          // chunk-local row
    const int tid = threadIdx.x;
    if (tid < BM) {
        const int lr = lr0 + tid, row = p.row0 + lr;
        float lse = 0.f, sc = 0.f;
        int tg = -1;
        if (lr < p.rows) {
            const int64_t t = a.targets[row];
            const bool valid = (t != a.ignore_index) && t >= 0 && t < a.V;
            lse = a.lse[row];
            sc = valid ? a.grad_scale[0] * (a.mask ? a.mask[row] : 1.f) : 0.f;
            tg = valid ? (int)t : -1;
        }
        sLse[tid] = lse;
        sScale[tid] = sc;
        sTgt[tid] = tg;
    }
    floatx4 acc[4][4];
    gemm_tile<T>((const T *)a.h + (int64_t)(p.row0 + lr0) * a.ldh, a.ldh, min(BM, p.rows - lr0),
                 (const T *)a.w + (int64_t)v0 * a.ldw, a.ldw, min(BN, a.V - v0), a.D, acc, smem);
    const int w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
    T *G = (T *)p.gbuf;
    T *GT = (T *)p.gtbuf;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const int vloc = 64 * wn + 16 * ni + l16, v = v0 + vloc;
            T gv[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int rl = 64 * wm + 16 * mi + 4 * g + r;
                float x = 0.f;
                if (v < a.V && sScale[rl] != 0.f) {
                    x = __expf(acc[mi][ni][r] - sLse[rl]);
                    if (v == sTgt[rl]) x -= 1.f;
                    x *= sScale[rl];
                }
                gv[r] = from_f32<T>(x);
                const int lr = lr0 + rl;
                if (lr < p.rows) G[(int64_t)lr * p.Vp + v] = gv[r];
            }
            // G^T[v][lr0 + 64wm + 16mi + 4g .. +3]: 4 consecutive rows
            T *dst = GT + (int64_t)v * p.Rp + lr0 + 64 * wm + 16 * mi + 4 * g;
            if (lr0 + 64 * wm + 16 * mi + 4 * g + 3 < p.Rp) {
#pragma unroll
                for (int r = 0; r < 4; ++r) dst[r] = gv[r];
            }
        }
    }
}

// C = A B^T with the epilogue writing dtype T (dH) or accumulating fp32 (dW)
template <typename T, bool ACCUM>
__global__ void __launch_bounds__(THREADS) ce_gemm_kernel(const T *A, int64_t lda, int M, const T *B, int64_t ldb,
                                                         int N, int K, void *C, int64_t ldc) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    T *smem = reinterpret_cast<T *>(smem_raw);
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    floatx4 acc[4][4];
    gemm_tile<T>(A + (int64_t)m0 * lda, lda, min(BM, M - m0), B + (int64_t)n0 * ldb, ldb, min(BN, N - n0), K, acc,
                 smem);
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 64 * wm + 16 * mi + 4 * g + r, n = n0 + 64 * wn + 16 * ni + l16;
                if (m < M && n < N) {
                    if (ACCUM) {
                        float *c = (float *)C + (int64_t)m * ldc + n;
                        *c += acc[mi][ni][r];
                    } else {
                        ((T *)C)[(int64_t)m * ldc + n] = from_f32<T>(acc[mi][ni][r]);
                    }
                }
            }
}

// ------------------------------------------------------ bf16 big tiles ----
// bf16 operands use 256 x 256 block tiles: 4 waves of 128 x 128, 8 x 8
// accumulator tiles (256 fp32 per lane, AGPR resident), 64 MFMA per 32-wide
// k-step against 16 fragment reads (64 flops per LDS byte), global loads
// prefetched two k-steps ahead through registers into a double-buffered LDS.
namespace big {
constexpr int BTM = 256;                // block tile rows (A operand)
constexpr int BTN = 128;                // block tile cols (B operand)
constexpr int PITCH = BK + 8;           // bf16 elements per LDS row
constexpr int LOADS_A = BTM * 4 / THREADS;  // 16-byte loads per thread per k-step
constexpr int LOADS_B = BTN * 4 / THREADS;
constexpr size_t SMEM = (size_t)2 * (BTM + BTN) * PITCH * sizeof(unsigned short);  // 60 KiB
using U16 = unsigned short;

struct Frag {
    uint4 a[LOADS_A], b[LOADS_B];
};

// Workgroups are dispatched round-robin over the 8 XCDs, each with its own L2.
// Give every XCD a contiguous range of work items (grid = 8 * per; items >=
// total are idle) so that concurrently running tiles of one XCD share rows.
constexpr int XCDS = 8;
__device__ __forceinline__ int xcd_item(int bid, int total) {
    const int per = (total + XCDS - 1) / XCDS;
    return (bid % XCDS) * per + bid / XCDS;
}
inline int xcd_grid(int total) { return XCDS * ((total + XCDS - 1) / XCDS); }

// Item -> (row tile, col tile), grouping GM row tiles: consecutive items walk
// the GM row tiles of one column tile, then the next column tile, so a window
// of ~32 items touches GM row tiles and ~32/GM column tiles.
constexpr int GM = 4;
__device__ __forceinline__ void grouped_tile(int item, int n_rt, int n_ct, int &rt, int &ct) {
    const int group = item / (GM * n_ct);
    const int in_group = item - group * GM * n_ct;
    const int rows = min(GM, n_rt - group * GM);
    rt = group * GM + in_group % rows;
    ct = in_group / rows;
}

__device__ __forceinline__ void gload(Frag &f, const U16 *A, int64_t lda, int a_rows, const U16 *B, int64_t ldb,
                                      int b_rows, int k0) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < LOADS_A; ++i) {
        const int ci = tid + i * THREADS, row = ci >> 2, c = ci & 3;
        f.a[i] = (row < a_rows) ? *reinterpret_cast<const uint4 *>(A + row * lda + k0 + 8 * c) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < LOADS_B; ++i) {
        const int ci = tid + i * THREADS, row = ci >> 2, c = ci & 3;
        f.b[i] = (row < b_rows) ? *reinterpret_cast<const uint4 *>(B + row * ldb + k0 + 8 * c) : make_uint4(0, 0, 0, 0);
    }
}

__device__ __forceinline__ void lstore(const Frag &f, U16 *sA, U16 *sB) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int i = 0; i < LOADS_A; ++i) {
        const int ci = tid + i * THREADS, row = ci >> 2, c = ci & 3;
        *reinterpret_cast<uint4 *>(sA + row * PITCH + 8 * c) = f.a[i];
    }
#pragma unroll
    for (int i = 0; i < LOADS_B; ++i) {
        const int ci = tid + i * THREADS, row = ci >> 2, c = ci & 3;
        *reinterpret_cast<uint4 *>(sB + row * PITCH + 8 * c) = f.b[i];
    }
}

__device__ __forceinline__ void mma_step(const U16 *sA, const U16 *sB, floatx4 (&acc)[8][4], int arow0, int brow0,
                                         int l16, int g) {
    // B fragments stay in registers for the step; A fragments are read per row tile
    bf16x8 bfr[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) bfr[i] = *reinterpret_cast<const bf16x8 *>(sB + (brow0 + 16 * i + l16) * PITCH + 8 * g);
#pragma unroll
    for (int mi = 0; mi < 8; ++mi) {
        const bf16x8 af = *reinterpret_cast<const bf16x8 *>(sA + (arow0 + 16 * mi + l16) * PITCH + 8 * g);
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af, bfr[ni], acc[mi][ni], 0, 0, 0);
    }
}

// C[m][n] = sum_{k in [k_begin, k_end)} A[m][k] B[n][k] for one 256 x 128 tile.
// acc[mi][ni] lane holds C[128*(w>>1) + 16mi + 4g + r][64*(w&1) + 16ni + l16].
// DEEP prefetches two k-steps ahead (two register stages); otherwise one.
template <bool DEEP>
__device__ __forceinline__ void gemm_tile(const U16 *A, int64_t lda, int a_rows, const U16 *B, int64_t ldb,
                                          int b_rows, int k_begin, int k_end, floatx4 (&acc)[8][4], U16 *smem) {
    U16 *sA[2] = {smem, smem + (BTM + BTN) * PITCH};
    U16 *sB[2] = {smem + BTM * PITCH, smem + (BTM + BTN) * PITCH + BTM * PITCH};
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int arow0 = 128 * (w >> 1), brow0 = 64 * (w & 1);
#pragma unroll
    for (int mi = 0; mi < 8; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int KT = (k_end - k_begin) / BK;
    if (KT <= 0) return;
    if (!DEEP) {
        Frag f;
        gload(f, A, lda, a_rows, B, ldb, b_rows, k_begin);
        lstore(f, sA[0], sB[0]);
        __syncthreads();
        for (int kt = 0; kt < KT; ++kt) {
            const int buf = kt & 1;
            if (kt + 1 < KT) gload(f, A, lda, a_rows, B, ldb, b_rows, k_begin + (kt + 1) * BK);
            mma_step(sA[buf], sB[buf], acc, arow0, brow0, l16, g);
            if (kt + 1 < KT) lstore(f, sA[buf ^ 1], sB[buf ^ 1]);
            __syncthreads();
        }
        return;
    }
    Frag f0, f1;
    gload(f0, A, lda, a_rows, B, ldb, b_rows, k_begin);
    if (KT > 1) gload(f1, A, lda, a_rows, B, ldb, b_rows, k_begin + BK);
    lstore(f0, sA[0], sB[0]);
    __syncthreads();
    for (int kt = 0; kt < KT; kt += 2) {
        // even step: tile kt in buffer 0, tile kt+1 waiting in f1
        if (kt + 2 < KT) gload(f0, A, lda, a_rows, B, ldb, b_rows, k_begin + (kt + 2) * BK);
        mma_step(sA[0], sB[0], acc, arow0, brow0, l16, g);
        if (kt + 1 < KT) lstore(f1, sA[1], sB[1]);
        __syncthreads();
        if (kt + 1 >= KT) break;
        // odd step: tile kt+1 in buffer 1, tile kt+2 waiting in f0
        if (kt + 3 < KT) gload(f1, A, lda, a_rows, B, ldb, b_rows, k_begin + (kt + 3) * BK);
        mma_step(sA[1], sB[1], acc, arow0, brow0, l16, g);
        if (kt + 2 < KT) lstore(f0, sA[0], sB[0]);
        __syncthreads();
    }
}

// forward: per (256 rows, 128 vocab) tile -> per-row (max, sum exp, argmax)
__global__ void __launch_bounds__(THREADS, 2) fwd_tile_kernel(FwdParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ float sM[2][BTM], sS[2][BTM];
    __shared__ int sI[2][BTM];
    const qpam_ce_fwd_args &a = p.a;
    const int n_rt = (a.N + BTM - 1) / BTM;
    const int item = xcd_item(blockIdx.x, n_rt * p.n_vt);
    if (item >= n_rt * p.n_vt) return;
    int rt, vt;
    grouped_tile(item, n_rt, p.n_vt, rt, vt);
    const int r0 = rt * BTM, v0 = vt * BTN;
    floatx4 acc[8][4];
    gemm_tile<true>((const U16 *)a.h + (int64_t)r0 * a.ldh, a.ldh, min(BTM, a.N - r0), (const U16 *)a.w + (int64_t)v0 * a.ldw,
              a.ldw, min(BTN, a.V - v0), 0, a.D, acc, reinterpret_cast<U16 *>(smem_raw));
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
#pragma unroll
    for (int mi = 0; mi < 8; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float mx = -INFINITY;
            int ix = 0x7fffffff;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const int v = v0 + 64 * wn + 16 * ni + l16;
                const float x = (v < a.V) ? acc[mi][ni][r] : -INFINITY;
                if (x > mx) { mx = x; ix = v; }
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) {
                const float om = __shfl_xor(mx, off);
                const int oi = __shfl_xor(ix, off);
                if (om > mx || (om == mx && oi < ix)) { mx = om; ix = oi; }
            }
            float s = 0.f;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const int v = v0 + 64 * wn + 16 * ni + l16;
                if (v < a.V) s += __expf(acc[mi][ni][r] - mx);
            }
#pragma unroll
            for (int off = 1; off < 16; off <<= 1) s += __shfl_xor(s, off);
            if (l16 == 0) {
                const int row = 128 * wm + 16 * mi + 4 * g + r;
                sM[wn][row] = mx;
                sS[wn][row] = s;
                sI[wn][row] = ix;
            }
        }
    }
    __syncthreads();
    if (r0 + tid < a.N) {
        const float m0 = sM[0][tid], m1 = sM[1][tid];
        const float m = fmaxf(m0, m1);
        float s = 0.f;
        if (m0 > -INFINITY) s += sS[0][tid] * __expf(m0 - m);
        if (m1 > -INFINITY) s += sS[1][tid] * __expf(m1 - m);
        const int i = (m1 > m0 || (m1 == m0 && sI[1][tid] < sI[0][tid])) ? sI[1][tid] : sI[0][tid];
        const int64_t o = (int64_t)(r0 + tid) * p.n_vt + vt;
        p.part_m[o] = m;
        p.part_s[o] = s;
        p.part_i[o] = i;
    }
}

// backward G tile (256 rows x 128 vocab): recompute logits, write G and G^T
__global__ void __launch_bounds__(THREADS, 2) grad_tile_kernel(BwdParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ float sLse[BTM], sScale[BTM];
    __shared__ int sTgt[BTM];
    const qpam_ce_bwd_args &a = p.a;
    const int n_rt = p.Rp / BTM, n_vt = p.Vp / BTN;
    const int item = xcd_item(blockIdx.x, n_rt * n_vt);
    if (item >= n_rt * n_vt) return;
    int rt, vt;
    grouped_tile(item, n_rt, n_vt, rt, vt);
    const int lr0 = rt * BTM, v0 = vt * BTN;
    const int tid = threadIdx.x;
    {
        const int lr = lr0 + tid, row = p.row0 + lr;
        float lse = 0.f, sc = 0.f;
        int tg = -1;
        if (lr < p.rows) {
            const int64_t t = a.targets[row];
            const bool valid = (t != a.ignore_index) && t >= 0 && t < a.V;
            lse = a.lse[row];
            sc = valid ? a.grad_scale[0] * (a.mask ? a.mask[row] : 1.f) : 0.f;
            tg = valid ? (int)t : -1;
        }
        sLse[tid] = lse;
        sScale[tid] = sc;
        sTgt[tid] = tg;
    }
    floatx4 acc[8][4];
    gemm_tile<false>((const U16 *)a.h + (int64_t)(p.row0 + lr0) * a.ldh, a.ldh, min(BTM, p.rows - lr0),
              (const U16 *)a.w + (int64_t)v0 * a.ldw, a.ldw, min(BTN, a.V - v0), 0, a.D, acc,
              reinterpret_cast<U16 *>(smem_raw));
    const int w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
    U16 *G = (U16 *)p.gbuf;
    U16 *GT = (U16 *)p.gtbuf;
#pragma unroll
    for (int mi = 0; mi < 8; ++mi) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const int v = v0 + 64 * wn + 16 * ni + l16;
            const int rl0 = 128 * wm + 16 * mi + 4 * g;
            ushortx4 gv;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int rl = rl0 + r;
                float x = 0.f;
                if (v < a.V && sScale[rl] != 0.f) {
                    x = __expf(acc[mi][ni][r] - sLse[rl]);
                    if (v == sTgt[rl]) x -= 1.f;
                    x *= sScale[rl];
                }
                gv[r] = f32_to_bf16(x);
                if (p.write_g && lr0 + rl < p.rows) G[(int64_t)(lr0 + rl) * p.Vp + v] = gv[r];
            }
            *reinterpret_cast<ushortx4 *>(GT + (int64_t)v * p.Rp + lr0 + rl0) = gv;
        }
    }
}

// backward GEMMs: dW tiles (dW[v][d] += sum_r G^T[v][r] H^T[d][r]) and
// split-K partials of dH (dH_s[r][d] = sum_{v in split s} G[r][v] W^T[d][v])
// into fp32, as two kernels so each keeps two waves per SIMD.
struct GroupParams {
    BwdParams p;
    int n_dw, dw_ntiles_n;     // dW tiles, tiles along D
    int dh_ntiles_m, dh_ntiles_n, splits, ksplit;
    float *dh_part;            // [splits][rows][D]
};

__global__ void __launch_bounds__(THREADS, 2) dw_gemm_kernel(GroupParams q) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const BwdParams &p = q.p;
    const qpam_ce_bwd_args &a = p.a;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
    floatx4 acc[8][4];
    const int bid = xcd_item(blockIdx.x, q.n_dw);
    if (bid >= q.n_dw) return;
    const int mt = bid / q.dw_ntiles_n, nt = bid % q.dw_ntiles_n;
    const int m0 = mt * BTM, n0 = nt * BTN;
    gemm_tile<false>((const U16 *)p.gtbuf + (int64_t)m0 * p.Rp, p.Rp, min(BTM, a.V - m0),
              (const U16 *)p.ht + (int64_t)n0 * p.Rp, p.Rp, min(BTN, a.D - n0), 0, p.Rp, acc,
              reinterpret_cast<U16 *>(smem_raw));
#pragma unroll
    for (int mi = 0; mi < 8; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 128 * wm + 16 * mi + 4 * g + r, n = n0 + 64 * wn + 16 * ni + l16;
                if (m < a.V && n < a.D) static_cast<float *>(a.dw)[(int64_t)m * a.lddw + n] += acc[mi][ni][r];
            }
}

__global__ void __launch_bounds__(THREADS, 2) dh_gemm_kernel(GroupParams q) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    const BwdParams &p = q.p;
    const qpam_ce_bwd_args &a = p.a;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
    floatx4 acc[8][4];
    const int total = q.splits * q.dh_ntiles_m * q.dh_ntiles_n;
    const int bid = xcd_item(blockIdx.x, total);
    if (bid >= total) return;
    const int s = bid / (q.dh_ntiles_m * q.dh_ntiles_n);
    const int t = bid % (q.dh_ntiles_m * q.dh_ntiles_n);
    const int mt = t / q.dh_ntiles_n, nt = t % q.dh_ntiles_n;
    const int m0 = mt * BTM, n0 = nt * BTN;
    const int kb = s * q.ksplit, ke = min(p.Vp, kb + q.ksplit);
    gemm_tile<false>((const U16 *)p.gbuf + (int64_t)m0 * p.Vp, p.Vp, min(BTM, p.rows - m0),
              (const U16 *)p.wt + (int64_t)n0 * p.Vp, p.Vp, min(BTN, a.D - n0), kb, ke, acc,
              reinterpret_cast<U16 *>(smem_raw));
    float *dst = q.dh_part + (int64_t)s * p.rows * a.D;
#pragma unroll
    for (int mi = 0; mi < 8; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = m0 + 128 * wm + 16 * mi + 4 * g + r, n = n0 + 64 * wn + 16 * ni + l16;
                if (m < p.rows && n < a.D) dst[(int64_t)m * a.D + n] = acc[mi][ni][r];
            }
}

// dH rows of the chunk = sum of the split partials, written as bf16
__global__ void __launch_bounds__(THREADS) dh_reduce_kernel(GroupParams q) {
    const BwdParams &p = q.p;
    const qpam_ce_bwd_args &a = p.a;
    const int64_t n = (int64_t)p.rows * a.D;
    for (int64_t e = blockIdx.x * (int64_t)THREADS + threadIdx.x; e < n; e += (int64_t)gridDim.x * THREADS) {
        float x = 0.f;
        for (int s = 0; s < q.splits; ++s) x += q.dh_part[s * n + e];
        const int64_t r = e / a.D, c = e - r * a.D;
        reinterpret_cast<U16 *>(a.dh)[(int64_t)(p.row0 + r) * a.lddh + c] = f32_to_bf16(x);
    }
}

constexpr int DH_SPLITS = 8;
}  // namespace big

// 256 x 256 tiles for the bf16 logits GEMMs (hidden size a multiple of 64): one
// block of 4 waves per tile, each wave a 128 x 128 quadrant (64 accumulator
// tiles, one wave per SIMD), k-steps of 64 through double-buffered LDS (72 KiB
// per stage) with the next stage's global loads in flight in registers.  Rows
// past the end of an operand re-read its last row (the epilogues mask them), so
// the pipelined loads carry no conditional register initialisation.
namespace wide {
constexpr int TM = 256, TN = 256, WK = 64;
constexpr float LOG2E = 1.4426950408889634f;
constexpr int WTHREADS = 512;   // 8 waves: 4 row groups x 2 column groups, 64 x 128 each
constexpr int WPITCH = WK + 8;  // bf16 elements per LDS row (144 bytes: conflict-free 16-byte reads)
constexpr int WLOADS = TM * WK / 8 / WTHREADS;  // 16-byte loads per thread per operand per k-step (4)
constexpr size_t WSMEM = (size_t)2 * (TM + TN) * WPITCH * sizeof(unsigned short);  // 144 KiB
using U16 = unsigned short;

struct WFrag {
    uintx4 a[WLOADS], b[WLOADS];
};

// Rows past the end of an operand re-read its last row (the epilogues mask them).
// Addresses are a wave-uniform base plus a 32-bit byte offset per load.
__device__ __forceinline__ void wgload(WFrag &f, const U16 *A, int64_t lda, int a_rows, const U16 *B, int64_t ldb,
                                       int b_rows, int k0) {
    const int tid = threadIdx.x, c8 = 8 * (tid & 7);
    const char *ab = reinterpret_cast<const char *>(A + k0), *bb = reinterpret_cast<const char *>(B + k0);
#pragma unroll
    for (int i = 0; i < WLOADS; ++i) {
        const int row = (tid >> 3) + 64 * i;
        const unsigned ao = 2u * (unsigned)(min(row, a_rows - 1) * (int)lda + c8);
        const unsigned bo = 2u * (unsigned)(min(row, b_rows - 1) * (int)ldb + c8);
        f.a[i] = *reinterpret_cast<const uintx4 *>(ab + ao);
        f.b[i] = *reinterpret_cast<const uintx4 *>(bb + bo);
    }
}

__device__ __forceinline__ void wlstore(const WFrag &f, U16 *sA, U16 *sB) {
    const int tid = threadIdx.x, c8 = 8 * (tid & 7);
#pragma unroll
    for (int i = 0; i < WLOADS; ++i) {
        const int row = (tid >> 3) + 64 * i;
        *reinterpret_cast<uintx4 *>(sA + row * WPITCH + c8) = f.a[i];
        *reinterpret_cast<uintx4 *>(sB + row * WPITCH + c8) = f.b[i];
    }
}

// One k-step (64) of the wave's 64 x 128 block: per 32-wide half, the four A
// fragments stay in registers while the eight B fragments stream through (each
// feeds four MFMAs).
__device__ __forceinline__ void wmma_stage(const U16 *sA, const U16 *sB, floatx4 (&acc)[4][8], int arow0, int brow0,
                                           int l16, int g) {
#pragma unroll
    for (int ks = 0; ks < WK / 32; ++ks) {
        bf16x8 af[4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
            af[mi] = *reinterpret_cast<const bf16x8 *>(sA + (arow0 + 16 * mi + l16) * WPITCH + 32 * ks + 8 * g);
#pragma unroll
        for (int ni = 0; ni < 8; ++ni) {
            const bf16x8 bfr = *reinterpret_cast<const bf16x8 *>(sB + (brow0 + 16 * ni + l16) * WPITCH + 32 * ks + 8 * g);
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
                acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], bfr, acc[mi][ni], 0, 0, 0);
        }
    }
}

// C[m][n] = sum_k A[m][k] B[n][k] (k in [0, K), K a multiple of 64) for one 256 x 256
// tile; acc[mi][ni] lane holds C[64*(w>>1) + 16mi + 4g + r][128*(w&1) + 16ni + l16].
// The global loads of k-step kt + 1 are issued (and pinned) before the MFMAs of
// k-step kt and reach the other LDS buffer after them; the second wave on each
// SIMD covers the rest of their latency.
__device__ __forceinline__ void wgemm_tile(const U16 *A, int64_t lda, int a_rows, const U16 *B, int64_t ldb,
                                           int b_rows, int K, floatx4 (&acc)[4][8], U16 *smem) {
    U16 *sA0 = smem, *sB0 = smem + TM * WPITCH;
    U16 *sA1 = smem + (TM + TN) * WPITCH, *sB1 = sA1 + TM * WPITCH;
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int arow0 = 64 * (w >> 1), brow0 = 128 * (w & 1);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 8; ++ni) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int KT = K / WK;
    WFrag f;
    wgload(f, A, lda, a_rows, B, ldb, b_rows, 0);
    wlstore(f, sA0, sB0);
    __syncthreads();
    // two k-steps per iteration (buffers by compile-time index); the loads are
    // unconditional (past the end they re-read the last k-step) so that every path
    // has the same memory operations
    int kt = 0;
    for (; kt + 1 < KT; kt += 2) {
        wgload(f, A, lda, a_rows, B, ldb, b_rows, (kt + 1) * WK);
        __builtin_amdgcn_sched_barrier(0);
        wmma_stage(sA0, sB0, acc, arow0, brow0, l16, g);
        __builtin_amdgcn_sched_barrier(0);
        wlstore(f, sA1, sB1);
        __syncthreads();
        wgload(f, A, lda, a_rows, B, ldb, b_rows, min(kt + 2, KT - 1) * WK);
        __builtin_amdgcn_sched_barrier(0);
        wmma_stage(sA1, sB1, acc, arow0, brow0, l16, g);
        __builtin_amdgcn_sched_barrier(0);
        wlstore(f, sA0, sB0);
        __syncthreads();
    }
    if (kt < KT) wmma_stage(sA0, sB0, acc, arow0, brow0, l16, g);
}

// The same tile product with the operands streamed global -> LDS by direct
// (no register) loads: four LDS stages of k = 32 (128 KiB), the loads of k-step
// kt + 3 issued when k-step kt starts, so each load has three k-steps to land.
// Each direct load writes 64 lanes x 16 bytes = 16 rows x 64 bytes contiguously;
// the 16-byte chunks of a row are XOR-swizzled (chunk c of row r at c ^ ((r >> 1) & 3))
// so that the fragment reads (16 rows, one chunk) hit distinct banks.  Separate
// arrays per stage let the compiler's memory-counter tracking tell the stages apart;
// the wait before each barrier is explicit: every k-step issues exactly four
// direct loads per wave (past the end they re-read the last k-step into a free
// stage), so "own loads of the next k-step done" is vmcnt <= 8.
constexpr int DK = 32, DSTAGES = 4;
constexpr bool USE_DMA = true;                  // direct-load mainloop (else register-staged)
constexpr size_t KSMEM = USE_DMA ? 0 : WSMEM;   // dynamic LDS of the tile kernels
__device__ __forceinline__ int swz(int row, int c) { return c ^ ((row >> 1) & 3); }

template <int S>
__device__ __forceinline__ void dma_stage(U16 (&sA)[TM * DK], U16 (&sB)[TN * DK], const U16 *A, int64_t lda,
                                          int a_rows, const U16 *B, int64_t ldb, int b_rows, int k0) {
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int r0 = 32 * w + 16 * j, row = r0 + (lane >> 2), c = swz(row, lane & 3);
        __builtin_amdgcn_global_load_lds(A + (int64_t)min(row, a_rows - 1) * lda + k0 + 8 * c, &sA[r0 * DK], 16, 0, 0);
        __builtin_amdgcn_global_load_lds(B + (int64_t)min(row, b_rows - 1) * ldb + k0 + 8 * c, &sB[r0 * DK], 16, 0, 0);
    }
}

__device__ __forceinline__ void dma_mma(const U16 *sA, const U16 *sB, floatx4 (&acc)[4][8], int arow0, int brow0,
                                        int l16, int g) {
    bf16x8 af[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
        const int row = arow0 + 16 * mi + l16;
        af[mi] = *reinterpret_cast<const bf16x8 *>(sA + row * DK + 8 * swz(row, g));
    }
#pragma unroll
    for (int ni = 0; ni < 8; ++ni) {
        const int row = brow0 + 16 * ni + l16;
        const bf16x8 bfr = *reinterpret_cast<const bf16x8 *>(sB + row * DK + 8 * swz(row, g));
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
            acc[mi][ni] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[mi], bfr, acc[mi][ni], 0, 0, 0);
    }
}

// s_waitcnt with vmcnt <= 8 and the other counters unconstrained
constexpr int WAIT_VM8 = 8 | 0x70 | 0xF00;

__device__ __forceinline__ void wgemm_tile_dma(const U16 *A, int64_t lda, int a_rows, const U16 *B, int64_t ldb,
                                               int b_rows, int K, floatx4 (&acc)[4][8]) {
    __shared__ __align__(16) U16 sA0[TM * DK], sA1[TM * DK], sA2[TM * DK], sA3[TM * DK];
    __shared__ __align__(16) U16 sB0[TN * DK], sB1[TN * DK], sB2[TN * DK], sB3[TN * DK];
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int arow0 = 64 * (w >> 1), brow0 = 128 * (w & 1);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 8; ++ni) acc[mi][ni] = floatx4{0.f, 0.f, 0.f, 0.f};
    const int KT = K / DK;
    dma_stage<0>(sA0, sB0, A, lda, a_rows, B, ldb, b_rows, 0);
    dma_stage<1>(sA1, sB1, A, lda, a_rows, B, ldb, b_rows, min(1, KT - 1) * DK);
    dma_stage<2>(sA2, sB2, A, lda, a_rows, B, ldb, b_rows, min(2, KT - 1) * DK);
    __builtin_amdgcn_s_waitcnt(WAIT_VM8);
    __builtin_amdgcn_s_barrier();
#define QPAM_DMA_STEP(KT_, CUR_A, CUR_B, NXT_A, NXT_B, NS)                                                    \
    dma_stage<NS>(NXT_A, NXT_B, A, lda, a_rows, B, ldb, b_rows, min((KT_) + 3, KT - 1) * DK);                 \
    __builtin_amdgcn_sched_barrier(0);                                                                         \
    dma_mma(CUR_A, CUR_B, acc, arow0, brow0, l16, g);                                                          \
    __builtin_amdgcn_s_waitcnt(WAIT_VM8);                                                                      \
    __builtin_amdgcn_s_barrier();
    int kt = 0;
    for (; kt + 3 < KT; kt += 4) {
        QPAM_DMA_STEP(kt, sA0, sB0, sA3, sB3, 3)
        QPAM_DMA_STEP(kt + 1, sA1, sB1, sA0, sB0, 0)
        QPAM_DMA_STEP(kt + 2, sA2, sB2, sA1, sB1, 1)
        QPAM_DMA_STEP(kt + 3, sA3, sB3, sA2, sB2, 2)
    }
    if (kt < KT) { QPAM_DMA_STEP(kt, sA0, sB0, sA3, sB3, 3) }
    if (kt + 1 < KT) { QPAM_DMA_STEP(kt + 1, sA1, sB1, sA0, sB0, 0) }
    if (kt + 2 < KT) { QPAM_DMA_STEP(kt + 2, sA2, sB2, sA1, sB1, 1) }
#undef QPAM_DMA_STEP
    // drain the direct loads still in flight before the LDS is reused or the wave ends
    __builtin_amdgcn_s_waitcnt(0 | 0x70 | 0xF00);
}

__device__ __forceinline__ int xcd_item(int bid, int total) { return big::xcd_item(bid, total); }

// Order a wave's LDS accesses around a point: its earlier LDS operations are
// complete (lgkmcnt 0) and no LDS access moves across it.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), vmcnt / expcnt unconstrained
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// forward: per (256 rows, 256 vocab) tile -> per-row (max, sum exp[, argmax]).
// Row statistics over a wave's 128 columns: per lane over its 8 columns, then
// across the 16 lanes that hold the row (DPP); the argmax (first column at the
// maximum) only when accuracy counts are requested.
template <bool ARGMAX>
__global__ void __launch_bounds__(WTHREADS) fwd_tile_kernel(FwdParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ float sM[2][TM], sS[2][TM];
    __shared__ int sI[2][TM];
    const qpam_ce_fwd_args &a = p.a;
    const int n_rt = (a.N + TM - 1) / TM;
    const int item = xcd_item(blockIdx.x, n_rt * p.n_vt);
    if (item >= n_rt * p.n_vt) return;
    int rt, vt;
    big::grouped_tile(item, n_rt, p.n_vt, rt, vt);
    const int r0 = rt * TM, v0 = vt * TN;
    floatx4 acc[4][8];
    if constexpr (USE_DMA)
        wgemm_tile_dma((const U16 *)a.h + (int64_t)r0 * a.ldh, a.ldh, min(TM, a.N - r0),
                       (const U16 *)a.w + (int64_t)v0 * a.ldw, a.ldw, min(TN, a.V - v0), a.D, acc);
    else
        wgemm_tile((const U16 *)a.h + (int64_t)r0 * a.ldh, a.ldh, min(TM, a.N - r0),
                   (const U16 *)a.w + (int64_t)v0 * a.ldw, a.ldw, min(TN, a.V - v0), a.D, acc,
                   reinterpret_cast<U16 *>(smem_raw));
    const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
    const int vl = v0 + 128 * wn + l16;  // this lane's column in tile ni: vl + 16 ni
    const bool full = v0 + TN <= a.V;    // no column past the vocabulary: no per-element checks
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            float lm = -INFINITY;
#pragma unroll
            for (int ni = 0; ni < 8; ++ni)
                if (full || vl + 16 * ni < a.V) lm = fmaxf(lm, acc[mi][ni][r]);
            const float mx = row16_max(lm);
            float s = 0.f;
            int ix = 0x7fffffff;
            if (mx > -INFINITY) {
                const float mx2 = mx * LOG2E;  // exp(x - mx) = exp2(x log2e - mx log2e)
#pragma unroll
                for (int ni = 0; ni < 8; ++ni)
                    if (full || vl + 16 * ni < a.V) {
                        const float x = acc[mi][ni][r];
                        s += __builtin_amdgcn_exp2f(__builtin_fmaf(x, LOG2E, -mx2));
                        if (ARGMAX && x == mx) ix = min(ix, vl + 16 * ni);
                    }
            }
            s = row16_sum(s);
            if (ARGMAX) ix = row16_min(ix);
            if (l16 == 0) {
                const int row = 64 * wm + 16 * mi + 4 * g + r;
                sM[wn][row] = mx;
                sS[wn][row] = s;
                if (ARGMAX) sI[wn][row] = ix;
            }
        }
    }
    __syncthreads();
    if (tid < TM && r0 + tid < a.N) {
        const float m0 = sM[0][tid], m1 = sM[1][tid];
        const float m = fmaxf(m0, m1);
        float s = 0.f;
        if (m0 > -INFINITY) s += sS[0][tid] * __expf(m0 - m);
        if (m1 > -INFINITY) s += sS[1][tid] * __expf(m1 - m);
        const int64_t o = (int64_t)(r0 + tid) * p.n_vt + vt;
        p.part_m[o] = m;
        p.part_s[o] = s;
        if (ARGMAX) p.part_i[o] = (m1 > m0 || (m1 == m0 && sI[1][tid] < sI[0][tid])) ? sI[1][tid] : sI[0][tid];
    }
}

// backward G tile (256 rows x 256 vocab): recompute logits, write G^T [Vp][Rp]
// (and G [rows][Vp] when write_g)
__global__ void __launch_bounds__(WTHREADS) grad_tile_kernel(BwdParams p) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    __shared__ float sLse[TM], sScale[TM];
    __shared__ int sTgt[TM];
    const qpam_ce_bwd_args &a = p.a;
    const int n_rt = p.Rp / TM, n_vt = p.Vp / TN;
    const int item = xcd_item(blockIdx.x, n_rt * n_vt);
    if (item >= n_rt * n_vt) return;
    int rt, vt;
    big::grouped_tile(item, n_rt, n_vt, rt, vt);
    const int lr0 = rt * TM, v0 = vt * TN;
    const int tid = threadIdx.x;
    if (tid < TM) {
        const int lr = lr0 + tid, row = p.row0 + lr;
        float lse = 0.f, sc = 0.f;
        int tg = -1;
        if (lr < p.rows) {
            const int64_t t = a.targets[row];
            const bool valid = (t != a.ignore_index) && t >= 0 && t < a.V;
            lse = a.lse[row];
            sc = valid ? a.grad_scale[0] * (a.mask ? a.mask[row] : 1.f) : 0.f;
            tg = valid ? (int)t : -1;
        }
        sLse[tid] = lse;
        sScale[tid] = sc;
        sTgt[tid] = tg;
    }
    floatx4 acc[4][8];
    if constexpr (USE_DMA)
        wgemm_tile_dma((const U16 *)a.h + (int64_t)(p.row0 + lr0) * a.ldh, a.ldh, min(TM, p.rows - lr0),
                       (const U16 *)a.w + (int64_t)v0 * a.ldw, a.ldw, min(TN, a.V - v0), a.D, acc);
    else
        wgemm_tile((const U16 *)a.h + (int64_t)(p.row0 + lr0) * a.ldh, a.ldh, min(TM, p.rows - lr0),
                   (const U16 *)a.w + (int64_t)v0 * a.ldw, a.ldw, min(TN, a.V - v0), a.D, acc,
                   reinterpret_cast<U16 *>(smem_raw));
    const int w = tid >> 6, lane = tid & 63, l16 = lane & 15, g = lane >> 4;
    const int wm = w >> 1, wn = w & 1;
    U16 *G = (U16 *)p.gbuf;
    U16 *GT = (U16 *)p.gtbuf;
    // G^T rows (one per vocab entry) hold the tile's rows contiguously: each
    // 16-wide vocab slab of a wave's 64 x 128 tile goes through LDS so that it
    // leaves as 128-byte runs (the accumulator layout alone would write 32-byte
    // pieces).
    constexpr int GT_LD = 72;   // bf16 per staged vocab row: 64 tile rows + padding against bank conflicts
    __shared__ __align__(16) U16 sEpi[8 * 16 * GT_LD];
    U16 *tw = sEpi + w * 16 * GT_LD;
    // the 16 rows of this lane (rows 64 wm + 16 mi + 4 g + r) in registers: lse in
    // log2 units (exp(x - lse) = exp2(x log2e - lse log2e), one fma and one exp2),
    // +inf for rows without a gradient (their G is exp2(-inf) = 0), the scale and
    // the target column
    float hl[4][4], hs[4][4];
    int ht[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int rl = 64 * wm + 16 * mi + 4 * g + r;
            hs[mi][r] = sScale[rl];
            hl[mi][r] = hs[mi][r] != 0.f ? sLse[rl] * LOG2E : INFINITY;
            ht[mi][r] = sTgt[rl];
        }
    const bool full = v0 + TN <= a.V;  // every column of the tile is a vocabulary entry
#pragma unroll
    for (int ni = 0; ni < 8; ++ni) {
        const int vb = v0 + 128 * wn + 16 * ni, v = vb + l16;
        const bool vok = full || v < a.V;
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            const int rl0 = 64 * wm + 16 * mi + 4 * g;
            float x[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(acc[mi][ni][r], LOG2E, -hl[mi][r]));
                x[r] = vok ? (e - (v == ht[mi][r] ? 1.f : 0.f)) * hs[mi][r] : 0.f;
            }
            const unsigned lo = pack_bf16x2(x[0], x[1]), hi = pack_bf16x2(x[2], x[3]);
            if (p.write_g) {
                const unsigned short gb[4] = {(unsigned short)(lo & 0xFFFFu), (unsigned short)(lo >> 16),
                                              (unsigned short)(hi & 0xFFFFu), (unsigned short)(hi >> 16)};
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (lr0 + rl0 + r < p.rows) G[(int64_t)(lr0 + rl0 + r) * p.Vp + v] = gb[r];
            }
            *reinterpret_cast<uint2 *>(tw + l16 * GT_LD + 16 * mi + 4 * g) = make_uint2(lo, hi);
        }
        // the slab is this wave's own: its LDS writes complete before its reads
        // (and the reads before the next slab's writes) without a block barrier
        wave_lds_sync();
        {   // lane -> (vocab row lane / 4, 16 tile rows (lane % 4) * 16 ..): 32 bytes each
            const int vl = lane >> 2, part = lane & 3;
            const uint4 *src = reinterpret_cast<const uint4 *>(tw + vl * GT_LD + 16 * part);
            const uint4 d0 = src[0], d1 = src[1];
            uint4 *dst = reinterpret_cast<uint4 *>(GT + (int64_t)(vb + vl) * p.Rp + lr0 + 64 * wm + 16 * part);
            dst[0] = d0;
            dst[1] = d1;
        }
        wave_lds_sync();
    }
}
}  // namespace wide

int round_up(int x, int m) { return (x + m - 1) / m * m; }

template <typename T> constexpr bool is_bf() { return sizeof(T) == 2; }

// bf16 with a hidden size that is a multiple of 64 takes the 256 x 256 tiles
bool use_wide(int D) { return D % wide::WK == 0; }

// vocab tile of the forward logits kernel (128 on the fp32 and narrow bf16 paths:
// the larger partial count, used to size the workspace)
template <typename T> constexpr int vocab_tile() { return is_bf<T>() ? big::BTN : VT; }
// vocab / row padding of the backward G buffers (one value per dtype, whichever
// bf16 tile runs: 256 is a multiple of both bf16 tile widths)
template <typename T> constexpr int vocab_pad() { return is_bf<T>() ? wide::TN : VT; }
template <typename T> constexpr int row_tile() { return is_bf<T>() ? big::BTM : BM; }

template <typename T>
size_t fwd_ws(const qpam_ce_fwd_args &a) {
    const int64_t n_vt = (a.V + vocab_tile<T>() - 1) / vocab_tile<T>();
    return (size_t)a.N * n_vt * 12 + 256;
}

// Rows of one backward pass.  The reference keeps the fp32 logits and softmax of
// `chunk` rows alive (8 bytes per row and vocabulary entry); a pass here covers
// as many rows as fit those bytes: bf16 G^T alone (library GEMMs) takes 2 bytes,
// bf16 G and G^T (hand-written GEMMs) 4 bytes, fp32 G and G^T 8 bytes.
int pass_rows(const qpam_ce_bwd_args &a) {
    const int64_t factor = a.dtype == QPAM_BF16 ? (blas::enabled() ? 4 : 2) : 1;
    return (int)std::min<int64_t>((int64_t)a.chunk * factor, a.N);
}

template <typename T>
size_t bwd_ws_base(const qpam_ce_bwd_args &a) {
    const int64_t Vp = round_up(a.V, vocab_pad<T>()), chunk = pass_rows(a);
    const int64_t Rp = round_up((int)chunk, row_tile<T>());
    if (is_bf<T>() && blas::enabled())  // G^T and the library GEMMs' workspace
        return (size_t)(Vp * Rp * sizeof(T)) + 4 * 256 +
               std::max((size_t)big::DH_SPLITS * chunk * a.D * sizeof(float), blas::WS_BYTES) + 256;
    const int64_t elems = (int64_t)a.D * Vp + chunk * Vp + Vp * Rp + (int64_t)a.D * Rp;
    size_t bytes = (size_t)(elems * sizeof(T)) + 4 * 256;
    // bf16: split-K partials of the hand-written dH GEMM
    if (is_bf<T>()) bytes += std::max((size_t)big::DH_SPLITS * chunk * a.D * sizeof(float), blas::WS_BYTES) + 256;
    return bytes;
}

// dw_out 1 or 2 with bf16 inputs, the library GEMMs and one pass over the rows:
// the dW GEMM writes the gradient itself (beta 0) from its fp32 sums, in bf16
// or fp32
bool dw_direct(const qpam_ce_bwd_args &a) {
    return a.dw_out != 0 && a.dtype == QPAM_BF16 && blas::enabled() && pass_rows(a) >= a.N;
}

// dw_out 1 otherwise: bf16 inputs accumulate dW in fp32 after the passes' own
// workspace (V x D, 256-byte aligned) and convert it once at the end
template <typename T>
size_t bwd_ws(const qpam_ce_bwd_args &a) {
    const size_t base = bwd_ws_base<T>(a);
    if (a.dw_out != 1 || !is_bf<T>() || dw_direct(a)) return base;
    return base + 256 + (size_t)a.V * a.D * sizeof(float);
}

__global__ void __launch_bounds__(THREADS) dw_fill_kernel(float *p, int64_t rows, int cols, int64_t ld) {
    const int64_t n = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * THREADS) {
        const int64_t r = i / cols;
        p[r * ld + (i - r * cols)] = 0.f;
    }
}

__global__ void __launch_bounds__(THREADS) dw_cast_kernel(const float *src, int64_t lds, unsigned short *dst,
                                                          int64_t ldd, int64_t rows, int cols) {
    const int64_t n = rows * cols;
    for (int64_t i = (int64_t)blockIdx.x * THREADS + threadIdx.x; i < n; i += (int64_t)gridDim.x * THREADS) {
        const int64_t r = i / cols, c = i - r * cols;
        dst[r * ldd + c] = f32_to_bf16(src[r * lds + c]);
    }
}

template <typename T>
int run_fwd(const qpam_ce_fwd_args &a, hipStream_t stream) {
    FwdParams p;
    p.a = a;
    const bool wide_tiles = is_bf<T>() && use_wide(a.D);
    p.n_vt = wide_tiles ? (a.V + wide::TN - 1) / wide::TN : (a.V + vocab_tile<T>() - 1) / vocab_tile<T>();
    char *ws = (char *)a.workspace;
    const int64_t cnt = (int64_t)a.N * p.n_vt;
    p.part_m = (float *)ws;
    p.part_s = p.part_m + cnt;
    p.part_i = (int *)(p.part_s + cnt);
    p.red = nullptr;
    int st;
    if (wide_tiles) {
        // the argmax (accuracy counts) only when requested
        const void *kern = a.correct ? (const void *)wide::fwd_tile_kernel<true> : (const void *)wide::fwd_tile_kernel<false>;
        QPAM_CHECK_HIP(hipFuncSetAttribute(kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)wide::KSMEM));
        dim3 grid(big::xcd_grid(p.n_vt * ((a.N + wide::TM - 1) / wide::TM)));
        if (a.correct)
            hipLaunchKernelGGL(wide::fwd_tile_kernel<true>, grid, dim3(wide::WTHREADS), wide::KSMEM, stream, p);
        else
            hipLaunchKernelGGL(wide::fwd_tile_kernel<false>, grid, dim3(wide::WTHREADS), wide::KSMEM, stream, p);
        st = launch_status("ce fwd_tile_kernel (bf16, 256 x 256)");
    } else if (is_bf<T>()) {
        QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)big::fwd_tile_kernel,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)big::SMEM));
        dim3 grid(big::xcd_grid(p.n_vt * ((a.N + big::BTM - 1) / big::BTM)));
        hipLaunchKernelGGL(big::fwd_tile_kernel, grid, dim3(THREADS), big::SMEM, stream, p);
        st = launch_status("ce fwd_tile_kernel (bf16)");
    } else {
        const size_t smem = gemm_smem<T>();
        QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)ce_fwd_tile_kernel<T>,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
        dim3 grid(p.n_vt, (a.N + BM - 1) / BM);
        hipLaunchKernelGGL(ce_fwd_tile_kernel<T>, grid, dim3(THREADS), smem, stream, p);
        st = launch_status("ce_fwd_tile_kernel");
    }
    if (st) return st;
    hipLaunchKernelGGL(ce_fwd_finalize_kernel<T>, dim3((a.N + 3) / 4), dim3(THREADS), 0, stream, p);
    st = launch_status("ce_fwd_finalize_kernel");
    if (st) return st;
    if (a.loss_sum) {
        hipLaunchKernelGGL(ce_reduce_kernel, dim3(1), dim3(1024), 0, stream, p);
        st = launch_status("ce_reduce_kernel");
    }
    return st;
}

// dw_write: dW written (beta 0; one pass over the rows) by the library GEMM, in
// bf16 (dw_out 1) or fp32 (dw_out 2); otherwise added into the fp32 dW
int run_bwd_bf16(const qpam_ce_bwd_args &a, hipStream_t stream, bool dw_write = false) {
    using U = unsigned short;
    big::GroupParams q;
    BwdParams &p = q.p;
    p.a = a;
    p.Vp = round_up(a.V, vocab_pad<U>());
    const int chunk = pass_rows(a);
    const int Rmax = round_up(chunk, big::BTM);
    const bool wide_tiles = use_wide(a.D);
    // the G-tile kernel: 256 x 256 tiles, or 256 x 128 for hidden sizes that are not
    // a multiple of 64 (Vp and Rp are multiples of both)
    const void *gkern = wide_tiles ? (const void *)wide::grad_tile_kernel : (const void *)big::grad_tile_kernel;
    const size_t gsmem = wide_tiles ? wide::KSMEM : big::SMEM;
    auto launch_grad = [&]() {
        const int tiles = (p.Vp / (wide_tiles ? wide::TN : big::BTN)) * (p.Rp / big::BTM);
        if (wide_tiles)
            hipLaunchKernelGGL(wide::grad_tile_kernel, dim3(big::xcd_grid(tiles)), dim3(wide::WTHREADS), gsmem, stream, p);
        else
            hipLaunchKernelGGL(big::grad_tile_kernel, dim3(big::xcd_grid(tiles)), dim3(THREADS), gsmem, stream, p);
        return launch_status(wide_tiles ? "ce grad_tile_kernel (bf16, 256 x 256)" : "ce grad_tile_kernel (bf16)");
    };
    U *ws = (U *)a.workspace;
    const size_t smem = big::SMEM;
    if (blas::enabled()) {
        p.wt = p.gbuf = p.ht = nullptr;
        p.gtbuf = ws;
        q.dh_part = (float *)(((uintptr_t)(ws + (int64_t)p.Vp * Rmax) + 255) & ~(uintptr_t)255);
        // G^T [Vp][Rp] from the fused grad tiles, then two library GEMMs (column-major views):
        //   dW^T[D][V] += H^T G^T-view   (m = D, n = V, k = rows)
        //   dH^T[D][rows] = W^T G-view   (m = D, n = rows, k = V)
        p.write_g = 0;
        const size_t blas_ws = std::max((size_t)big::DH_SPLITS * chunk * a.D * sizeof(float), blas::WS_BYTES);
        QPAM_CHECK_HIP(hipFuncSetAttribute(gkern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gsmem));
        for (int r0 = 0; r0 < a.N; r0 += chunk) {
            p.row0 = r0;
            p.rows = std::min(chunk, a.N - r0);
            p.Rp = round_up(p.rows, big::BTM);
            int st = launch_grad();
            if (st) return st;
            st = blas::gemm_bf16(false, false, a.D, a.V, p.rows, (const U *)a.h + (int64_t)r0 * a.ldh, a.ldh,
                                 p.gtbuf, p.Rp, dw_write ? 0.f : 1.f, a.dw, a.lddw, !(dw_write && a.dw_out == 1),
                                 q.dh_part, blas_ws, stream);
            if (st) return st;
            st = blas::gemm_bf16(false, true, a.D, p.rows, a.V, a.w, a.ldw, p.gtbuf, p.Rp, 0.f,
                                 (U *)a.dh + (int64_t)r0 * a.lddh, a.lddh, false, q.dh_part, blas_ws, stream);
            if (st) return st;
        }
        return QPAM_OK;
    }
    p.wt = ws;
    p.gbuf = ws + (int64_t)a.D * p.Vp;
    p.gtbuf = (U *)p.gbuf + (int64_t)chunk * p.Vp;
    p.ht = (U *)p.gtbuf + (int64_t)p.Vp * Rmax;
    q.dh_part = (float *)(((uintptr_t)((U *)p.ht + (int64_t)a.D * Rmax) + 255) & ~(uintptr_t)255);
    p.write_g = 1;
    QPAM_CHECK_HIP(hipFuncSetAttribute(gkern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)gsmem));
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)big::dw_gemm_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)big::dh_gemm_kernel,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    hipLaunchKernelGGL(transpose_kernel<U>, dim3((a.D + 63) / 64, (p.Vp + 63) / 64), dim3(THREADS), 0, stream,
                       (const U *)a.w, a.ldw, a.V, a.D, (U *)p.wt, (int64_t)p.Vp, a.D, p.Vp);
    int st = launch_status("transpose_kernel(W)");
    if (st) return st;
    q.dw_ntiles_n = (a.D + big::BTN - 1) / big::BTN;
    q.n_dw = ((a.V + big::BTM - 1) / big::BTM) * q.dw_ntiles_n;
    q.dh_ntiles_n = q.dw_ntiles_n;
    q.splits = big::DH_SPLITS;
    q.ksplit = round_up((p.Vp + q.splits - 1) / q.splits, BK);
    for (int r0 = 0; r0 < a.N; r0 += chunk) {
        p.row0 = r0;
        p.rows = std::min(chunk, a.N - r0);
        p.Rp = round_up(p.rows, big::BTM);
        hipLaunchKernelGGL(transpose_kernel<U>, dim3((a.D + 63) / 64, (p.Rp + 63) / 64), dim3(THREADS), 0, stream,
                           (const U *)a.h + (int64_t)r0 * a.ldh, a.ldh, p.rows, a.D, (U *)p.ht, (int64_t)p.Rp, a.D,
                           p.Rp);
        st = launch_status("transpose_kernel(H)");
        if (st) return st;
        st = launch_grad();
        if (st) return st;
        q.dh_ntiles_m = (p.rows + big::BTM - 1) / big::BTM;
        hipLaunchKernelGGL(big::dw_gemm_kernel, dim3(big::xcd_grid(q.n_dw)), dim3(THREADS), smem, stream, q);
        st = launch_status("ce dw_gemm_kernel (bf16)");
        if (st) return st;
        hipLaunchKernelGGL(big::dh_gemm_kernel, dim3(big::xcd_grid(q.splits * q.dh_ntiles_m * q.dh_ntiles_n)),
                           dim3(THREADS), smem, stream, q);
        st = launch_status("ce dh_gemm_kernel (bf16)");
        if (st) return st;
        hipLaunchKernelGGL(big::dh_reduce_kernel, dim3(1024), dim3(THREADS), 0, stream, q);
        st = launch_status("ce dh_reduce_kernel");
        if (st) return st;
    }
    return QPAM_OK;
}

template <typename T>
int run_bwd(const qpam_ce_bwd_args &a, hipStream_t stream) {
    if (is_bf<T>()) return run_bwd_bf16(a, stream);
    BwdParams p;
    p.a = a;
    p.write_g = 1;
    p.Vp = round_up(a.V, VT);
    const int chunk = pass_rows(a);
    const int Rmax = round_up(chunk, BM);
    T *ws = (T *)a.workspace;
    p.wt = ws;
    p.gbuf = ws + (int64_t)a.D * p.Vp;
    p.gtbuf = (T *)p.gbuf + (int64_t)chunk * p.Vp;
    p.ht = (T *)p.gtbuf + (int64_t)p.Vp * Rmax;
    const size_t smem = gemm_smem<T>();
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)ce_grad_tile_kernel<T>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)ce_gemm_kernel<T, false>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    QPAM_CHECK_HIP(hipFuncSetAttribute((const void *)ce_gemm_kernel<T, true>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem));
    // W^T [D][Vp] (zero-padded vocab columns)
    hipLaunchKernelGGL(transpose_kernel<T>, dim3((a.D + 63) / 64, (p.Vp + 63) / 64), dim3(THREADS), 0, stream,
                       (const T *)a.w, a.ldw, a.V, a.D, (T *)p.wt, (int64_t)p.Vp, a.D, p.Vp);
    int st = launch_status("transpose_kernel(W)");
    if (st) return st;
    for (int r0 = 0; r0 < a.N; r0 += chunk) {
        p.row0 = r0;
        p.rows = std::min(chunk, a.N - r0);
        p.Rp = round_up(p.rows, BM);
        // H^T [D][Rp] of this chunk
        hipLaunchKernelGGL(transpose_kernel<T>, dim3((a.D + 63) / 64, (p.Rp + 63) / 64), dim3(THREADS), 0, stream,
                           (const T *)a.h + (int64_t)r0 * a.ldh, a.ldh, p.rows, a.D, (T *)p.ht, (int64_t)p.Rp, a.D,
                           p.Rp);
        st = launch_status("transpose_kernel(H)");
        if (st) return st;
        hipLaunchKernelGGL(ce_grad_tile_kernel<T>, dim3(p.Vp / VT, p.Rp / BM), dim3(THREADS), smem, stream, p);
        st = launch_status("ce_grad_tile_kernel");
        if (st) return st;
        // dH[r0 .. r0+rows] = G [rows][Vp] * (W^T [D][Vp])^T
        hipLaunchKernelGGL((ce_gemm_kernel<T, false>), dim3((a.D + BN - 1) / BN, (p.rows + BM - 1) / BM),
                           dim3(THREADS), smem, stream, (const T *)p.gbuf, (int64_t)p.Vp, p.rows, (const T *)p.wt,
                           (int64_t)p.Vp, a.D, p.Vp, (void *)((T *)a.dh + (int64_t)r0 * a.lddh), a.lddh);
        st = launch_status("ce_gemm_kernel(dH)");
        if (st) return st;
        // dW [V][D] += G^T [Vp][Rp] * (H^T [D][Rp])^T
        hipLaunchKernelGGL((ce_gemm_kernel<T, true>), dim3((a.D + BN - 1) / BN, (a.V + BM - 1) / BM),
                           dim3(THREADS), smem, stream, (const T *)p.gtbuf, (int64_t)p.Rp, a.V, (const T *)p.ht,
                           (int64_t)p.Rp, a.D, p.Rp, (void *)a.dw, a.lddw);
        st = launch_status("ce_gemm_kernel(dW)");
        if (st) return st;
    }
    return QPAM_OK;
}

int validate_common(int N, int V, int D, int dtype, const void *h, int64_t ldh, const void *w, int64_t ldw,
                    const int64_t *targets, const char *who) {
    QPAM_REQUIRE(N >= 1 && V >= 1 && D >= 1, "%s: bad sizes N=%d V=%d D=%d", who, N, V, D);
    QPAM_REQUIRE(dtype == QPAM_F32 || dtype == QPAM_BF16, "%s: dtype %d", who, dtype);
    QPAM_REQUIRE(D % BK == 0, "%s: hidden size %d must be a multiple of %d", who, D, BK);
    QPAM_REQUIRE(h && w && targets, "%s: null pointer", who);
    const int vec = dtype == QPAM_F32 ? 4 : 8;
    QPAM_REQUIRE(((uintptr_t)h % 16) == 0 && ((uintptr_t)w % 16) == 0 && ldh % vec == 0 && ldw % vec == 0 &&
                     ldh >= D && ldw >= D,
                 "%s: H and W must be 16-byte aligned with leading dims multiple of %d and >= D", who, vec);
    return QPAM_OK;
}

}  // namespace
}  // namespace ce
}  // namespace qpam

extern "C" size_t qpam_ce_fwd_workspace_size(const qpam_ce_fwd_args *a) {
    using namespace qpam::ce;
    if (!a) return 0;
    return a->dtype == QPAM_BF16 ? fwd_ws<unsigned short>(*a) : fwd_ws<float>(*a);
}

extern "C" int qpam_ce_fwd(const qpam_ce_fwd_args *a, void *stream) {
    using namespace qpam;
    using namespace qpam::ce;
    QPAM_REQUIRE(a != nullptr, "qpam_ce_fwd: null args");
    int st = validate_common(a->N, a->V, a->D, a->dtype, a->h, a->ldh, a->w, a->ldw, a->targets, "qpam_ce_fwd");
    if (st) return st;
    QPAM_REQUIRE(a->lse && a->loss, "qpam_ce_fwd: lse and loss outputs are required");
    const size_t need = qpam_ce_fwd_workspace_size(a);
    QPAM_REQUIRE(a->workspace && a->workspace_bytes >= need && ((uintptr_t)a->workspace % 16) == 0,
                 "qpam_ce_fwd: workspace needs %zu bytes (got %zu)", need, a->workspace_bytes);
    QPAM_REQUIRE((a->N + BM - 1) / BM <= 65535, "qpam_ce_fwd: too many rows");
    return a->dtype == QPAM_BF16 ? run_fwd<unsigned short>(*a, (hipStream_t)stream)
                                 : run_fwd<float>(*a, (hipStream_t)stream);
}

extern "C" size_t qpam_ce_bwd_workspace_size(const qpam_ce_bwd_args *a) {
    using namespace qpam::ce;
    if (!a || a->chunk < 1) return 0;
    return a->dtype == QPAM_BF16 ? bwd_ws<unsigned short>(*a) : bwd_ws<float>(*a);
}

extern "C" int qpam_ce_bwd(const qpam_ce_bwd_args *a, void *stream) {
    using namespace qpam;
    using namespace qpam::ce;
    QPAM_REQUIRE(a != nullptr, "qpam_ce_bwd: null args");
    int st = validate_common(a->N, a->V, a->D, a->dtype, a->h, a->ldh, a->w, a->ldw, a->targets, "qpam_ce_bwd");
    if (st) return st;
    QPAM_REQUIRE(a->lse && a->grad_scale && a->dh && a->dw, "qpam_ce_bwd: null lse/grad_scale/dh/dw");
    QPAM_REQUIRE(a->chunk >= 1, "qpam_ce_bwd: chunk must be >= 1");
    QPAM_REQUIRE(a->lddh >= a->D && a->lddw >= a->D, "qpam_ce_bwd: output leading dims must be >= D");
    QPAM_REQUIRE(a->dw_out >= 0 && a->dw_out <= 2, "qpam_ce_bwd: dw_out must be 0, 1 or 2");
    const size_t need = qpam_ce_bwd_workspace_size(a);
    QPAM_REQUIRE(a->workspace && a->workspace_bytes >= need && ((uintptr_t)a->workspace % 16) == 0,
                 "qpam_ce_bwd: workspace needs %zu bytes (got %zu)", need, a->workspace_bytes);
    hipStream_t s = (hipStream_t)stream;
    if (a->dw_out == 0) return a->dtype == QPAM_BF16 ? run_bwd<unsigned short>(*a, s) : run_bwd<float>(*a, s);
    if (dw_direct(*a)) return run_bwd_bf16(*a, s, true);
    // dW accumulated in fp32 -- dw itself when it is fp32, else the workspace's tail -- from zero
    qpam_ce_bwd_args b = *a;
    b.dw_out = 0;
    float *acc = static_cast<float *>(a->dw);
    int64_t ld = a->lddw;
    const bool convert = a->dw_out == 1 && a->dtype == QPAM_BF16;
    if (convert) {
        acc = (float *)(((uintptr_t)a->workspace + bwd_ws_base<unsigned short>(b) + 255) & ~(uintptr_t)255);
        ld = a->D;
    }
    const int64_t n = (int64_t)a->V * a->D;
    const dim3 grid((unsigned)std::min<int64_t>((n + THREADS - 1) / THREADS, 65536));
    hipLaunchKernelGGL(dw_fill_kernel, grid, dim3(THREADS), 0, s, acc, (int64_t)a->V, a->D, ld);
    st = launch_status("ce dw_fill_kernel");
    if (st) return st;
    b.dw = acc;
    b.lddw = ld;
    st = a->dtype == QPAM_BF16 ? run_bwd<unsigned short>(b, s) : run_bwd<float>(b, s);
    if (st || !convert) return st;
    hipLaunchKernelGGL(dw_cast_kernel, grid, dim3(THREADS), 0, s, (const float *)acc, ld, (unsigned short *)a->dw,
                       a->lddw, (int64_t)a->V, a->D);
    return launch_status("ce dw_cast_kernel");
}
