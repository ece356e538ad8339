/*
 * qpam.h -- C ABI of the MI355X (gfx950) Phase-Associative-Memory hot path.
 *
 * Plain C: POD argument structs of dimensions, strides (in elements) and
 * device pointers; every entry point launches asynchronously on the HIP
 * stream passed as `stream` (NULL = the null stream), performs no host
 * synchronisation and returns a qpam_status.  qpam_last_error() returns a
 * thread-local message for the last non-zero status on the calling thread.
 * The caller owns every input, output and workspace buffer.  The library
 * itself holds, per device and until the process ends: a hipBLASLt handle and
 * its plan cache (created by the first LM-head backward that uses hipBLASLt),
 * one extra default-priority stream with two events (created by the first
 * call that forks work onto it), and the statically allocated 64 MiB scratch
 * array of qpam_scan_fwd_noalloc (a module-scope device array, present from
 * load).  No other entry point allocates device memory.
 *
 * Complex tensors are planar: separate real and imaginary planes that share
 * one set of strides, innermost axis contiguous.  The decode state is the one
 * exception: it keeps the reference's interleaved [..., d, d, 2] layout so the
 * decode drop-in needs no conversion.
 *
 * Reference interfaces replaced (paths relative to gowrav-vishwakarma/qllm2):
 *   qpam_decode_step    v11/model.py:927-965  V11PAMLayer._recur_step_additive
 *   qpam_decode_step_bwd v11/model.py:927-965 its gradient (torch autograd there)
 *                       v11/model.py:845-925  V11PAMLayer._recurrent (token
 *                       step over K states with the e^{i phi} rotation)
 *   qpam_scan_fwd       v11/model.py:378-417  _forward_chunked_head,
 *                       v11/model.py:354-376  _dual_form_block (T <= C),
 *                       v11/flash_pam.py:56-152 flash_pam_chunked_head,
 *                       v11/model.py:657-781  _fused_chunk_step /
 *                                             _forward_multistate_fused
 *   qpam_scan_bwd       the autograd backward of the same functions (the
 *                       reference differentiates them with torch autograd and
 *                       v11/triton_kernels.py:447-480 for the decay matrix)
 *   qpam_decay_matrix   v11/triton_kernels.py:570-573 fused_decay_matrix
 *                       (forward, v11/triton_kernels.py:170-202, 420-445)
 *   qpam_cplx_fwd       v11/triton_kernels.py:489-520 public fused_complex_norm,
 *                       fused_mod_swish, fused_mod_relu, fused_cgu_gate
 *                       (forward kernels :48-166)
 *   qpam_cplx_bwd       their autograd backward (v11/triton_kernels.py:209-395)
 *   qpam_ce_fwd         v11/fused_ce.py:28-53   _FusedLinearCE.forward
 *                       v11/fused_ce.py:98-141  linear_ce_per_token /
 *                                               linear_ce_stats
 *   qpam_ce_bwd         v11/fused_ce.py:56-82   _FusedLinearCE.backward
 *   qpam_prologue_fwd   the elementwise steps of V11PAMLayer between the
 *                       projections and the scan: _project's RoPE / qk-norm
 *                       (v11/model.py:290-305), _gamma_all_and_vprime /
 *                       _gamma_and_vprime (:630-655, :309-347, floor :193-201)
 *                       and the rotations of _phase_and_alpha (:230-257,
 *                       consumed at :741-746)
 *   qpam_prologue_bwd   their autograd backward
 *   qpam_delta_fwd      v11/model.py:491-576  V11PAMLayer._forward_delta (E2
 *                       delta write; its solve v11/model.py:1005-1016) and
 *                       v11/model.py:967-1002 _recur_step_delta
 *   qpam_delta_bwd      their autograd backward
 *   qpam_cabs_fwd/_bwd  cabs (v11/complex_ops.py:86-87) feeding the gate and
 *                       phase projections (v11/model.py:228, 646)
 *   qpam_cweight_pack   ComplexLinear's weights (v11/complex_ops.py:146-172)
 *                       as the real operand of one GEMM: the layer's qkv_proj
 *                       with dt_proj (v11/model.py:280, 636) and o_proj (:836)
 *   qpam_cweight_unpack its backward (the weights' gradients)
 *   qpam_slice_sum      the gate projections' weight gradient (v11/model.py:228,
 *                       646) summed over row slices and cast
 *   qpam_resid_norm     the decode's residual adds and pre-norms, V11Block.forward
 *                       (v11/model.py:1039-1049) with ComplexNorm
 *                       (v11/complex_ops.py:188-189)
 *   qpam_cgu_mix        the CGU's activation and gate between its projections,
 *                       ComplexGatedUnit.forward (v11/complex_ops.py:216-220;
 *                       activations :102-143)
 */
#ifndef QPAM_H
#define QPAM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    QPAM_OK = 0,
    QPAM_ERR_ARG = 1,         /* invalid dimensions, strides or pointers */
    QPAM_ERR_UNSUPPORTED = 2, /* valid request this build does not implement */
    QPAM_ERR_HIP = 3,         /* a HIP runtime call failed */
    QPAM_ERR_WORKSPACE = 4    /* workspace missing or too small */
} qpam_status;

typedef enum { QPAM_F32 = 0, QPAM_BF16 = 1 } qpam_dtype;

/* Library version and the last error message of the calling thread. */
int qpam_version(void);
const char *qpam_last_error(void);

/* Profiling helpers (no reference counterpart): timing events that the
 * entry points with a prof_ev[2] field record around their dominant kernel,
 * so a benchmark can time that kernel alone on the launch stream. */
int qpam_event_create(void **ev);
int qpam_event_destroy(void *ev);
int qpam_event_elapsed_ms(void *ev0, void *ev1, float *ms);

/* ---------------------------------------------------------------- decode --
 * One O(1)/token recurrent step over a ragged pool of sequence slots.
 * For every listed slot a and every group g (= layer*heads + head) and state m:
 *     S[a,g,m] <- gamma[a,g,m] * S[a,g,m] + v[a,g] (x) conj(k[a,g])
 *     y[a,g]    = sum_m rot[a,g,m] * (S[a,g,m] @ (q_scale * q[a,g]))
 * (update before read, v11/model.py:948-964).  Slots not listed are neither
 * read nor written; ids outside [0, n_slots) are skipped.  rot may be NULL
 * (all ones).  S is interleaved complex fp32 [d][d][2]; q, k, v, y are
 * interleaved [d][2] (q, k, v optionally planar, see q_im); rot is interleaved
 * [2].  d in {16, 32, 64, 128}.
 */
typedef struct {
    int32_t n_slots;        /* size of the slot axis of every operand */
    int32_t n_active;       /* entries in `active` (or n_slots if active == NULL) */
    const int32_t *active;  /* device list of slot ids, or NULL for all slots */
    int32_t n_groups;       /* layers * heads per slot */
    int32_t n_states;       /* M >= 1 matrix states per group */
    int32_t d;              /* head dim */
    float q_scale;          /* 1.0 when q is already scaled */
    float *state;           /* updated in place */
    int64_t st_slot, st_group, st_state;  /* float strides of S */
    const float *q, *k, *v;
    int64_t sq_slot, sq_group, sk_slot, sk_group, sv_slot, sv_group;
    const float *gamma;
    int64_t sg_slot, sg_group, sg_state;
    const float *rot;       /* optional */
    int64_t sr_slot, sr_group, sr_state;
    float *y;
    int64_t sy_slot, sy_group;
    /* optional per-slot rotary position (the reference's _project rotation,
     * v11/model.py:290-301, with one offset per slot instead of one step_offset):
     * q and k of slot a are multiplied, feature by feature, by the complex
     * rope[pos[a]][j] before the update; rope is [rope_len][d][2] fp32 (the
     * build_rope_cache table, v11/complex_ops.py:261-266), positions are clamped
     * to [0, rope_len). */
    const float *rope;      /* NULL = no rotation */
    const int32_t *pos;     /* [n_slots] device positions */
    int32_t rope_len;
    /* 0: q, k, v, gamma, rot, y are indexed by slot id (rows of unlisted slots
     * are ignored / left alone).  1: they are compact, row i belonging to the
     * slot active[i] (n_active rows); S and pos stay indexed by slot id. */
    int32_t vec_by_rank;
    /* optional planar q, k, v (ABI 7): when set (all three), q, k, v point at the
     * real planes and these at the imaginary planes, rows of d floats with the
     * same strides (a prologue's output planes need no interleaving copy);
     * NULL = interleaved [d][2] rows. */
    const float *q_im, *k_im, *v_im;
    /* optional planar rotation (ABI 7): rot points at the real plane and rot_im at
     * the imaginary one, same strides; NULL = interleaved [2] entries. */
    const float *rot_im;
    /* 0: one decay per (slot, group, state); 1 (ABI 9): d decays there, one per
     * key channel j (contiguous), S[i][j] <- gamma[j] S[i][j] + v_i conj(k_j) --
     * the per-channel branch of _recur_step_additive (v11/model.py:952-954). */
    int32_t gamma_per_channel;
    /* qpam_dtype of y (ABI 9): QPAM_F32, or QPAM_BF16 (rounded once from the fp32
     * sums; `y` then points at bf16 elements with the same element strides) */
    int32_t y_dtype;
    /* optional (ABI 12): the decode prologue fused into the update (d = 64, head
     * decay).  With proj set, q, k, v, gamma and rot are ignored and formed per
     * (row, group g) from the layer's projection row proj[row][proj_ld]
     * (proj_dtype): q, k, v real planes at columns (0, G, 2G) d + g d, their
     * imaginary planes at (3G, 4G, 5G) d + g d, G = n_groups, the decay logit
     * at 6 G d + g -- the layout qpam_prologue_fwd reads -- and from the gate
     * logits gate[row][gate_ld] (proj_dtype, optional): protect at
     * protect_col + g, phase of state m at phase_col + g M + m (-1: absent).
     * As qpam_prologue_fwd computes them (without its RoPE, which rope / pos
     * apply here): q, k normalised per element when qk_norm,
     * p = sigmoid(protect), v' = v (1 - p), gamma_m = base_m (1 - p) + p with
     * base_m = exp(-softplus(dt + dt_bias[g] + state_offset[m])) lifted onto
     * [gamma_floor, 1) when gamma_floor > 0, rot_m = e^{i phase_m}. */
    const void *proj;
    int32_t proj_dtype;
    int32_t qk_norm;
    int64_t proj_ld;
    const void *gate;
    int64_t gate_ld;
    int32_t protect_col, phase_col;
    const float *dt_bias;               /* [G] fp32 */
    const float *state_offset;          /* [M] fp32, optional */
    float gamma_floor;
} qpam_decode_args;

int qpam_decode_step(const qpam_decode_args *a, void *stream);

/* Backward of one decode step, the gradient of _recur_step_additive
 * (v11/model.py:927-965, which the reference differentiates with torch
 * autograd) for n independent (slot, head) states of one matrix state each:
 *   S' = gamma (.) S + v (x) conj(k),  y = S' q   (q already scaled)
 * with gamma one decay per state or (gamma_per_channel) one per key column.
 * In: the state before the step `state` [n][d][d][2], gamma [n] or [n][d],
 * q, k, v, dy [n][d][2], dstate_new [n][d][d][2] (the gradient of S'; NULL =
 * zero).  Out: dstate (gradient of S) [n][d][d][2], dgamma (shape of gamma),
 * dq, dk, dv [n][d][2].  fp32, contiguous; d in {16, 32, 64, 128}.
 * Deterministic (fixed-order reductions). */
typedef struct {
    int64_t n;
    int32_t d, gamma_per_channel;
    const float *state, *gamma, *q, *k, *v, *dy, *dstate_new;
    float *dstate, *dgamma, *dq, *dk, *dv;
} qpam_decode_bwd_args;

int qpam_decode_step_bwd(const qpam_decode_bwd_args *a, void *stream);

/* ------------------------------------------------------------------ scan --
 * Chunked dual-form PAM scan with M >= 1 states per head (E3 when M > 1):
 *     q~ = q_scale * q;  D_m, cum_m, total_m from c = cumsum(-log(gamma_m+1e-6))
 *     Y[t]  = sum_{s<=t} (sum_m r_m[t] D_m[t,s]) (q~_t . k_s*) v_s
 *           + sum_m r_m[t] cum_m[t] (S_m,in @ q~_t)
 *     S_m  <- total_m S_m + sum_s D_m[C-1,s] v_s (x) k_s*
 * q, k, v: planar [B,H,T,d] (strides s0=b, s1=h, s2=t), fp32 or bf16.
 * gamma: fp32 [M,B,H,T]; rot (r_m, optional, NULL = 1): planar fp32 [M,B,H,T].
 * s0: optional initial state, planar fp32 [M,B,H,d,d] contiguous.
 * y: planar fp32 (or bf16, y_dtype) [B,H,T,d]; s_out: final state planar fp32 [M,B,H,d,d].
 * The workspace keeps the state entering every chunk, planar fp32
 * [M,B,H,n_chunks,d,d]; qpam_scan_bwd reads it.  d == 64, C in {16,32,64}.
 */
typedef struct {
    const void *re, *im;
    int64_t s0, s1, s2;
} qpam_cview;

typedef struct {
    float *re, *im;
    int64_t s0, s1, s2;
} qpam_mview;

typedef struct {
    int32_t B, H, T, d, C, M;
    int32_t dtype;          /* qpam_dtype of q, k, v (and of dq, dk, dv) */
    float q_scale;
    int32_t y_dtype;        /* qpam_dtype of y: QPAM_F32, or QPAM_BF16 for bf16 inputs with C == 64
                               (y rounded once from the fp32 result) */
    int32_t reserved0;
    qpam_cview q, k, v;
    const float *gamma;
    int64_t sg_m, sg_b, sg_h, sg_t;
    const float *rot_re, *rot_im;          /* optional */
    int64_t sr_m, sr_b, sr_h, sr_t;
    const float *s0_re, *s0_im;            /* optional */
    qpam_mview y;
    float *s_re, *s_im;
    void *workspace;
    size_t workspace_bytes;
    void *prof_ev[2];       /* optional hipEvent_t pair recorded around the
                               chunk-output kernel (the dominant launch) */
} qpam_scan_args;

size_t qpam_scan_workspace_size(const qpam_scan_args *a);
int qpam_scan_fwd(const qpam_scan_args *a, void *stream);

/* Allocation-free variant of qpam_scan_fwd.  It has no counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, kernels and results as qpam_scan_fwd, except that
 * `workspace` / `workspace_bytes` are ignored: the per-chunk states live in a
 * device array of QPAM_SCAN_FWD_NOALLOC_MAX_BYTES bytes inside the library
 * (one per GPU, held until the process ends).  A call whose states need more
 * (qpam_scan_workspace_size) fails with QPAM_ERR_WORKSPACE before any launch;
 * 64 MiB covers one 2048-token sequence of 12 heads with up to 4 fp32 states.
 * Every call on a GPU shares that GPU's array and it keeps only the last
 * call's states: calls that overlap on one GPU would race, and no
 * qpam_scan_bwd can follow (training uses qpam_scan_fwd).  Each call records
 * an event on its stream after its launches; a call on another stream while
 * that event is still pending fails with QPAM_ERR_ARG (checked with
 * hipEventQuery, no host wait; not checked under HIP graph capture, where the
 * caller orders the graph's replays).  The first call on a device sets up the
 * symbol address and that event; no call allocates device memory (no
 * hipMalloc, no library allocation). */
#define QPAM_SCAN_FWD_NOALLOC_MAX_BYTES (64u << 20)
int qpam_scan_fwd_noalloc(const qpam_scan_args *a, void *stream);

/* Backward of qpam_scan_fwd.  `fwd` must describe the same call whose
 * workspace still holds the per-chunk states.  dy: planar fp32 (or bf16, dy_dtype) [B,H,T,d];
 * ds: optional gradient of the final state, planar fp32 [M,B,H,d,d].
 * Outputs dq, dk, dv (dtype of q) planar [B,H,T,d]; dgamma fp32 [M,B,H,T]
 * with the strides of gamma; drot (optional) planar fp32 with rot's strides;
 * ds0 (optional) planar fp32 [M,B,H,d,d].  bwd_workspace holds per-chunk
 * state gradients, size from qpam_scan_bwd_workspace_size.  With bf16 q/k/v
 * and C == 64, dq/dk/dv planes must be 8-byte aligned with strides that are
 * multiples of 4 elements (their rows are stored in 8-byte runs). */
typedef struct {
    const qpam_scan_args *fwd;
    qpam_cview dy;
    int32_t dy_dtype;       /* qpam_dtype of dy: QPAM_F32, or QPAM_BF16 for bf16 inputs with C == 64 */
    int32_t reserved0;
    const float *ds_re, *ds_im;            /* optional */
    qpam_mview dq, dk, dv;
    float *dgamma;
    float *drot_re, *drot_im;              /* optional */
    float *ds0_re, *ds0_im;                /* optional */
    void *workspace;
    size_t workspace_bytes;
} qpam_scan_bwd_args;

size_t qpam_scan_bwd_workspace_size(const qpam_scan_bwd_args *a);
int qpam_scan_bwd(const qpam_scan_bwd_args *a, void *stream);

/* Decay matrix of fused_decay_matrix: gamma [N, T] fp32 (row stride ldg) ->
 * D [N, T, T] fp32 contiguous, D[t,s] = exp(min(c_s - c_t, 0)) for s <= t
 * else 0, c = cumsum(-log(gamma + 1e-6)).  T <= 4096. */
int qpam_decay_matrix(int32_t n, int32_t t, const float *gamma, int64_t ldg, float *out, void *stream);

/* ------------------------------------------------ PAM layer prologue -----
 * One pass from the layer's projections to the scan's inputs:
 *   q' = nrm(q * rope[rope_offset + t]),  k' = nrm(k * rope[rope_offset + t])
 *   p  = sigmoid(protect[b,t,h])                     (GSP; p = 0 without it)
 *   base_m = exp(-softplus(dt[b,t,h] + dt_bias[h] + dt_bias2[h] + state_offset[m]))
 *   base_m <- floor + (1 - floor) base_m             (only when floor > 0)
 *   gamma[m,b,h,t] = base_m (1 - p) + p,   v' = v (1 - p)
 *   rot[m,b,h,t] = routing[b,t,h,m] e^{i phase[b,t,h,m]}
 * with complex products per element, nrm(z) = z / sqrt(re^2 + im^2 + 1e-8)
 * when qk_norm (else the identity), softplus(x) = x for x > 20 else
 * log(1 + e^x).  q, k, v: planar views [B,T,H,d] (strides sx_b, sx_t, sx_h
 * shared by the six planes, d contiguous; the columns of one projection GEMM
 * [B*T, (re|im) x (q|k|v) x H x d] give them without copies), in_dtype; the
 * logits dt, protect, phase and routing are in in_dtype too (any strides).
 * q', k', v': planar [B,H,T,d] contiguous in out_dtype -- the scan's q, k, v.
 * gamma, rot: fp32 [M,B,H,T] contiguous -- the scan's gamma and rot.
 * d in {16, 32, 64, 128}, 1 <= M <= 4.  Rope rows past rope_len - 1 are
 * clamped to the last row (size the table to cover rope_offset + T).
 * dt_bias, dt_bias2 (an nn.Linear's own bias, optional) and state_offset are
 * read in param_dtype and summed in fp32 (ABI 11; param_dtype 0 = fp32 as
 * before).
 */
typedef struct {
    int32_t B, T, H, d, M;
    int32_t in_dtype, out_dtype;        /* qpam_dtype */
    int32_t qk_norm;
    float gamma_floor;
    int32_t rope_offset, rope_len;
    const float *rope;                  /* [rope_len][d][2], optional (NULL = none) */
    const void *q_re, *q_im, *k_re, *k_im, *v_re, *v_im;
    int64_t sx_b, sx_t, sx_h;
    const void *dt;                     /* [B,T,H] pre-bias decay logits */
    int64_t sd_b, sd_t, sd_h;
    const void *dt_bias;                /* [H] param_dtype */
    const void *state_offset;           /* [M] param_dtype, optional (NULL = 0) */
    const void *protect;                /* [B,T,H] protect-gate logits, optional */
    int64_t sp_b, sp_t, sp_h;
    const void *phase;                  /* [B,T,H,M], optional (NULL = no rot) */
    const void *routing;                /* [B,T,H,M], optional (NULL = 1) */
    int64_t sr_b, sr_t, sr_h, sr_m;     /* shared by phase and routing */
    void *oq_re, *oq_im, *ok_re, *ok_im, *ov_re, *ov_im;
    float *gamma;
    float *rot_re, *rot_im;             /* required when phase is given */
    int32_t param_dtype;                /* qpam_dtype of dt_bias, dt_bias2, state_offset */
    const void *dt_bias2;               /* [H] param_dtype, optional (NULL = 0) */
} qpam_prologue_args;

int qpam_prologue_fwd(const qpam_prologue_args *a, void *stream);

/* Backward of qpam_prologue_fwd (`fwd` describes the forward call; its
 * outputs are not read).  In: gradients of q', k', v' ([B,H,T,d] contiguous,
 * out_dtype), of gamma and (when phase) rot ([M,B,H,T] fp32).  Out: the
 * gradients of the projections q, k, v (planar views [B,T,H,d] with strides
 * sg_b, sg_t, sg_h, in_dtype); dpre [B,T,H,M] fp32 = dL/d(dt + dt_bias +
 * state_offset_m) (dt_bias's and state_offset's gradients are its sums over
 * the other axes); optionally ddt [B,T,H] (strides sdd_*, in_dtype) = the sum
 * of dpre over m, dt's gradient; dprotect [B,T,H] fp32 (when protect); dphase
 * and, optionally, drouting [B,T,H,M] fp32 (when phase) -- the layouts of the
 * logits they are the gradients of.  16 * H * (2 + 4 M) * 4 <= 65536.
 * ABI 11: dprotect, dphase and drouting are written in dlogit_dtype (0 = fp32)
 * with strides sdp_* (dprotect) and sdq_* (dphase, drouting), all zero meaning
 * the contiguous layouts above (so the gradients of logits that are columns of
 * one matrix land in that matrix's gradient directly); ddt_pad zero columns are
 * written after ddt's H (stride sdd_h); dbias [H] and doffset [M] (param_dtype,
 * optional) receive the sums of dpre over (b, t, m) and (b, t, h), formed in a
 * fixed order -- dpre is then scratch (per-block partial sums) and does not
 * hold dpre after the call.  dbias is the gradient of dt_bias and of
 * dt_bias2 alike. */
typedef struct {
    const qpam_prologue_args *fwd;
    const void *gq_re, *gq_im, *gk_re, *gk_im, *gv_re, *gv_im;
    const float *ggamma;
    const float *grot_re, *grot_im;     /* required when phase is given */
    void *dq_re, *dq_im, *dk_re, *dk_im, *dv_re, *dv_im;
    int64_t sg_b, sg_t, sg_h;
    float *dpre;
    void *ddt;                          /* optional */
    int64_t sdd_b, sdd_t, sdd_h;
    void *dprotect;
    void *dphase, *drouting;
    int32_t dlogit_dtype;
    int32_t ddt_pad;
    int64_t sdp_b, sdp_t, sdp_h;
    int64_t sdq_b, sdq_t, sdq_h, sdq_m;
    void *dbias;                        /* optional */
    void *doffset;                      /* optional (with state_offset) */
} qpam_prologue_bwd_args;

int qpam_prologue_bwd(const qpam_prologue_bwd_args *a, void *stream);

/* cabs (v11/complex_ops.py:86-87), the magnitudes the layer's gates read
 * (v11/model.py:228, 646): mag[i] = sqrt(z[i][0]^2 + z[i][1]^2 + 1e-8) over n
 * interleaved complex elements (n a multiple of 4, buffers 16-byte aligned
 * for fp32, 8-byte for bf16; mag in the dtype of z); the backward writes
 * gz[i] = gmag[i] z[i] / mag[i]. */
int qpam_cabs_fwd(int32_t dtype, int64_t n, const void *z, void *mag, void *stream);
int qpam_cabs_bwd(int32_t dtype, int64_t n, const void *z, const void *mag, const void *gmag, void *gz, void *stream);
/* The same backward added into gz (gz[i] += gmag[i] z[i] / mag[i]): the
 * layer input's gradient from its projections already in gz, its gradient
 * through the gates' magnitudes accumulated in the same pass (ABI 11). */
int qpam_cabs_bwd_acc(int32_t dtype, int64_t n, const void *z, const void *mag, const void *gmag, void *gz,
                      void *stream);

/* Complex linear weights as one real GEMM operand (ComplexLinear,
 * v11/complex_ops.py:146-172: re = Wr xr - Wi xi, im = Wi xr + Wr xi; the PAM
 * layer's qkv_proj and dt_proj, v11/model.py:280, 636, and o_proj, :836).
 * wr, wi [R][C] (row-major, contiguous) make W, with p the output part and q
 * the input part (0 = re, 1 = im) and the value wr, -wi, wi, wr at
 * (p, q) = (0,0), (0,1), (1,0), (1,1):
 *   QPAM_CW_IN  W[p R + r][2 c + q]  (interleaved input, outputs as a real then
 *               an imaginary block; C a multiple of 4), followed by tail_rows
 *               real rows W[2R + h][2 c + q] = tail[h][q C + c] (an nn.Linear
 *               over [xr | xi] reordered to the interleaved input) and
 *               zero_rows rows of zeros;
 *   QPAM_CW_OUT W[2 r + p][q C + c]  (input as two blocks, interleaved outputs;
 *               C a multiple of 8, no tail or zero rows).
 * W rows are ldw elements apart (ldw >= 2C, a multiple of 8); W, wr, wi, tail in
 * `dtype`; every pointer 16-byte aligned.
 * qpam_cweight_unpack is the backward: the gradient of W is the sum of `slices`
 * W-shaped matrices in g (g_dtype, slice_stride elements apart, summed in fp32
 * in slice order, e.g. the per-slice products of a row-sliced g^T x); it writes
 * g_wr, g_wi [R][C] and g_tail [tail_rows][2C] in `dtype`. */
enum { QPAM_CW_IN = 0, QPAM_CW_OUT = 1 };
typedef struct {
    int32_t dtype;
    int32_t layout;
    int64_t R, C;
    const void *wr, *wi;
    const void *tail;
    int64_t tail_rows, zero_rows;
    void *w;
    int64_t ldw;
    const void *g;
    int32_t g_dtype;
    int32_t slices;
    int64_t slice_stride;
    void *g_wr, *g_wi, *g_tail;
} qpam_cweight_args;

int qpam_cweight_pack(const qpam_cweight_args *a, void *stream);
int qpam_cweight_unpack(const qpam_cweight_args *a, void *stream);

/* out[i] = sum over s < slices of in[s * stride + i], i < n (fp32, in slice
 * order, rounded once to out_dtype): the row-sliced weight-gradient products
 * of an nn.Linear (the layer's gate projections over |x|, v11/model.py:228,
 * 646) reduced and cast in one pass (ABI 11).  n and stride multiples of 8,
 * in and out 16-byte aligned. */
int qpam_slice_sum(int32_t in_dtype, int32_t out_dtype, int32_t slices, int64_t n, int64_t stride, const void *in,
                   void *out, void *stream);

/* Gate logits of the decode step from |x| (v11/model.py:228, 646: protect_gate
 * and phase_proj applied to cabs(x), two nn.Linear on the same magnitudes, in
 * one call): out[r][g] = bias[g] + sum_j w[g][j] |z[r][j]| with
 * |z| = sqrt(re^2 + im^2 + 1e-8), z interleaved complex rows [rows][dim][2]
 * (dtype), w fp32 [G][dim] row-major, bias fp32 [G] or NULL, out [rows][ld_out]
 * (out_dtype).  dim <= 4096.  Inference only (no backward). */
int qpam_mag_linear(int32_t dtype, int32_t out_dtype, int64_t rows, int32_t dim, int32_t G, const void *z,
                    const float *w, const float *bias, void *out, int64_t ld_out, void *stream);

/* ---------------------------------------------------------- E2 delta rule --
 * Gated delta-rule write, per (b, h) over t (one state, head-scalar decay):
 *   S <- (gamma_t + gamma_eps) S;  u = beta_t (v_t - S k_t);
 *   S <- S + u (x) conj(k_t);      y_t = S (q_scale q_t)
 * -- the result of _forward_delta's chunked UT solve with gamma_eps = 1e-6
 * (its per-step factor gamma + 1e-6), of _recur_step_delta with 0.  q, k, v
 * fp32 planar [B,H,T,d] (strides b, h, t); gamma, beta fp32 [B,H,T] sharing
 * strides sg_*; s0 optional fp32 planar [B,H,d,d] contiguous; y fp32 planar
 * [B,H,T,d]; s_re/s_im the final state [B,H,d,d].  The workspace (size from
 * qpam_delta_workspace_size, or NULL when no backward follows) keeps, per
 * chunk, the entering state, the solved U and the chunk's triangular products
 * for the backward.  d == 64.  The chunked form follows the reference's chunks
 * of `chunk` steps (v11/model.py:494), its decay matrix exp(min(L_t - L_s, 0))
 * and its state-write weight alpha_last / (alpha_s + 1e-12)
 * (v11/model.py:508-510, 565-566); gamma + gamma_eps is kept at or above the
 * smallest normal float.
 */
typedef struct {
    int32_t B, H, T, d;
    float q_scale;
    float gamma_eps;
    int32_t chunk;                         /* steps per chunk of the chunked form: the reference's
                                              delta_chunk, 1..64 (0 = 64) */
    int32_t exact_write;                   /* 1: state-write weight exp(L_last - L_s) (the token
                                              recurrence, _recur_step_delta) instead of the chunked
                                              form's alpha_last / (alpha_s + 1e-12) */
    qpam_cview q, k, v;
    const float *gamma, *beta;
    int64_t sg_b, sg_h, sg_t;
    const float *s0_re, *s0_im;            /* optional */
    qpam_mview y;
    float *s_re, *s_im;
    void *workspace;
    size_t workspace_bytes;
    void *scratch;                         /* qpam_delta_scratch_size bytes: the forward's per-chunk
                                              products (always required by qpam_delta_fwd) */
    size_t scratch_bytes;
} qpam_delta_args;

size_t qpam_delta_workspace_size(const qpam_delta_args *a);
size_t qpam_delta_scratch_size(const qpam_delta_args *a);
int qpam_delta_fwd(const qpam_delta_args *a, void *stream);

/* Backward of qpam_delta_fwd (`fwd` describes the forward call; its
 * workspace still holds the per-chunk records).  dy fp32 planar [B,H,T,d]; ds
 * optional gradient of the final state.  Out: dq, dk, dv planar fp32; dgamma,
 * dbeta [B,H,T] with the strides of gamma; ds0 optional [B,H,d,d].
 * Deterministic (fixed-order reductions). */
typedef struct {
    const qpam_delta_args *fwd;
    qpam_cview dy;
    const float *ds_re, *ds_im;            /* optional */
    qpam_mview dq, dk, dv;
    float *dgamma, *dbeta;
    float *ds0_re, *ds0_im;                /* optional */
    void *workspace;
    size_t workspace_bytes;
} qpam_delta_bwd_args;

size_t qpam_delta_bwd_workspace_size(const qpam_delta_bwd_args *a);
int qpam_delta_bwd(const qpam_delta_bwd_args *a, void *stream);

/* ------------------------------------------------ E1 per-channel decay --
 * The per-channel pieces of V11PAMLayer._forward_chunked_perchannel
 * (v11/model.py:421-489); its chunk-parallel complex products are plain
 * batched GEMMs on the caller's side.
 *
 * qpam_pc_fold_fwd: per chunk of `chunk` steps and key channel j, with
 *   L_t = max(sum_{u<=t} log(max(gamma_u, 1e-6)), -30)   (v11/model.py:436-438)
 * writes qf = q e^{L_t} q_scale, kf = k e^{-L_t}, wf = k e^{L_last - L_t}
 * (L_last at the chunk's last step) and atot = e^{L_last}
 * (v11/model.py:439-450, 480); rows past T are zero.  q, k interleaved complex
 * [B,H,T,d,2] in `dtype` (element strides b, h, t; d and the pair contiguous);
 * gamma [B,H,T,d] in `g_dtype` (strides g_*).  Outputs fp32, contiguous:
 * qf, kf, wf [B*H][n][chunk][d][2], atot [B*H][n][d], n = ceil(T / chunk).
 * qpam_pc_fold_bwd: from the gradients of those four (each may be NULL for
 * zero) writes dq, dk (contiguous [B,H,T,d,2], `dtype`) and dgamma
 * (contiguous [B,H,T,d], `g_dtype`), through both clamps as torch's
 * clamp_min / clamp pass gradients (at or above the bound). */
typedef struct {
    int32_t dtype, g_dtype;
    int64_t B, H, T, d;
    int32_t chunk;                         /* the reference's chunk_size, 1..64 */
    float q_scale;
    const void *q, *k;
    int64_t q_sb, q_sh, q_st, k_sb, k_sh, k_st;
    const void *gamma;
    int64_t g_sb, g_sh, g_st;
    float *qf, *kf, *wf, *atot;            /* forward outputs */
    const float *dqf, *dkf, *dwf, *datot;  /* backward inputs (optional) */
    void *dq, *dk, *dgamma;                /* backward outputs */
} qpam_pc_fold_args;

int qpam_pc_fold_fwd(const qpam_pc_fold_args *a, void *stream);
int qpam_pc_fold_bwd(const qpam_pc_fold_args *a, void *stream);

/* The per-column decayed state scan of the per-channel chunks
 * (v11/model.py:486): state S [d][d] complex per chain, column j decayed by
 * a[c][j] at each step c; out[c] = S before step c, then S <- a[c] (.) S + x[c];
 * fin = S after the last step.  reverse = 1 walks c from n-1 down to 0 (the
 * gradient of the forward scan: x = the gradient of out, init = that of fin,
 * out = the gradient of x).  fp32, contiguous: x, out [N][n][d][d][2],
 * a [N][n][d], init, fin [N][d][d][2] (init NULL = zero, fin optional). */
typedef struct {
    int64_t N, n, d;
    const float *x, *a;
    float *out;
    const float *init;
    float *fin;
    int32_t reverse;
} qpam_pc_scan_args;

int qpam_pc_scan(const qpam_pc_scan_args *a, void *stream);

/* ------------------------------------------------ complex elementwise -----
 * Split-real complex tensors [rows, dim, 2] (interleaved re/im, contiguous),
 * fp32 or bf16; per-column parameters fp32 [dim].  Ops (z = gate for the CGU):
 *   NORM       out = z/(|z|+1e-8) * (|z|/rms) * scale, rms = sqrt(mean|z|^2 + eps)
 *   MOD_SWISH  out = z/(|z|+1e-8) * |z| sigmoid(beta |z| + bias)
 *   MOD_RELU   out = z/(|z|+1e-8) * relu(|z| + bias)
 *   CGU_GATE   out = sigmoid(|z|) * (z/(|z|+1e-8)) * up
 * with |z| = sqrt(re^2 + im^2 + 1e-8).  The backward writes gz (and gup), and
 * the parameter gradients gp0 (scale / bias) and gp1 (beta) as fp32 column
 * sums (deterministic: per-block partials in the workspace, summed in order).
 * dim * (number of parameters) <= 8192. */
enum { QPAM_CPLX_NORM = 0, QPAM_CPLX_MOD_SWISH = 1, QPAM_CPLX_MOD_RELU = 2, QPAM_CPLX_CGU_GATE = 3 };

typedef struct {
    int32_t op;            /* QPAM_CPLX_* */
    int32_t dtype;         /* of z, up, out and the tensor gradients */
    int64_t rows;
    int32_t dim;
    float eps;             /* NORM */
    const void *z;         /* [rows][dim][2] (the gate of CGU_GATE) */
    const void *up;        /* CGU_GATE */
    const float *p0;       /* NORM: scale; MOD_*: bias */
    const float *p1;       /* MOD_SWISH: beta */
    void *out;             /* forward output */
    const void *gout;      /* backward: gradient of out */
    void *gz, *gup;        /* backward: gradients of z / up */
    float *gp0, *gp1;      /* backward: parameter gradients [dim] */
    void *workspace;       /* backward: qpam_cplx_workspace_size bytes */
    size_t workspace_bytes;
} qpam_cplx_args;

size_t qpam_cplx_workspace_size(const qpam_cplx_args *a);
int qpam_cplx_fwd(const qpam_cplx_args *a, void *stream);
int qpam_cplx_bwd(const qpam_cplx_args *a, void *stream);

/* --------------------------------------------- decode block glue (ABI 13) --
 * Inference only: the work between the GEMMs of a V11 block in the model-level
 * decode, one launch each (the reference runs each as its own torch ops).
 *
 * qpam_resid_norm: the residual add then the next pre-norm (V11Block.forward,
 * v11/model.py:1039-1049; ComplexNorm, v11/complex_ops.py:188-189):
 *   x <- x + y * y_scale[0]        (when y is given; fp32 product and sum)
 *   out = ComplexNorm(x; norm_scale, eps) in out_dtype
 * x fp32 [rows][dim][2] (row stride ldx floats) is updated in place; y in y_dtype
 * (row stride ldy elements); y_scale is a device fp32 scalar (the block's
 * cgu_scale / pam_scale parameter: a captured graph follows weight updates);
 * norm_scale fp32 [dim].  dim a multiple of 4, at most 2048; row starts 16-byte
 * aligned.  out may not alias x or y. */
typedef struct {
    int64_t rows;
    int32_t dim;
    float eps;
    float *x;
    int64_t ldx;
    const void *y;          /* NULL: no residual, out = ComplexNorm(x) */
    int32_t y_dtype;
    int64_t ldy;
    const float *y_scale;
    const float *norm_scale;
    void *out;
    int32_t out_dtype;
    int64_t ldo;
} qpam_resid_norm_args;

int qpam_resid_norm(const qpam_resid_norm_args *a, void *stream);

/* qpam_cgu_mix: ComplexGatedUnit.forward between its projections
 * (v11/complex_ops.py:216-220): gu [rows][4 hid] in gu_dtype (row stride ldg
 * elements) holds the gate projection's hid complex values (re, im
 * interleaved) and then the up projection's;
 *   out = cgu_gate(gate, act(up))  in out_dtype [rows][hid][2] (row stride ldo)
 * with the formulas of qpam_cplx_fwd and act (parameters fp32 [hid]):
 *   MOD_RELU   bias                           (beta NULL)
 *   MOD_SWISH  bias, beta                     (phase_alpha, phase_beta NULL)
 *   phase-modulated (PhaseModulatedActivation, v11/complex_ops.py:125-143):
 *              bias, beta, phase_alpha, phase_beta: ModSwish's magnitude with
 *              the phase turned by phase_alpha |u| + phase_beta.
 * hid a multiple of 4; row starts and parameters 16-byte aligned. */
typedef struct {
    int64_t rows;
    int32_t hid;
    const void *gu;
    int32_t gu_dtype;
    int64_t ldg;
    const float *bias;
    const float *beta;
    const float *phase_alpha;
    const float *phase_beta;
    void *out;
    int32_t out_dtype;
    int64_t ldo;
} qpam_cgu_mix_args;

int qpam_cgu_mix(const qpam_cgu_mix_args *a, void *stream);

/* -------------------------------------------------------------------- CE --
 * Tied complex LM-head cross-entropy over hidden rows H [N, D] and weights
 * W [V, D] (row-major, leading dims ldh/ldw, bf16 or fp32), logits H W^T.
 * Forward writes per-row lse [N] and per-row loss [N] (0 on ignored rows and
 * on targets outside [0, V); times mask if given) and, if `correct` is
 * non-NULL, the argmax == target flag per row; loss_sum (optional, device
 * float[2]) receives {sum(loss), denominator}, the denominator being
 * sum(mask) or the number of rows whose target != ignore_index.  D must be a
 * multiple of 32.
 * Backward computes dH = G W, dW += G^T H with G = (softmax - onehot) *
 * grad_scale[row] (grad_scale = g/denom * mask, 0 on ignored rows), processing
 * `chunk` rows at a time through a bf16 G buffer in the workspace.
 */
typedef struct {
    int32_t N, V, D;
    int32_t dtype;                 /* of H and W */
    const void *h; int64_t ldh;
    const void *w; int64_t ldw;
    const int64_t *targets;        /* [N] */
    const float *mask;             /* optional [N] */
    int64_t ignore_index;
    float *lse;                    /* [N] */
    float *loss;                   /* [N] */
    float *correct;                /* optional [N], 1.0 where argmax == target */
    float *loss_sum;               /* optional device float[2] */
    void *workspace;
    size_t workspace_bytes;
} qpam_ce_fwd_args;

size_t qpam_ce_fwd_workspace_size(const qpam_ce_fwd_args *a);
int qpam_ce_fwd(const qpam_ce_fwd_args *a, void *stream);

typedef struct {
    int32_t N, V, D;
    int32_t dtype;
    const void *h; int64_t ldh;
    const void *w; int64_t ldw;
    const int64_t *targets;
    const float *mask;             /* optional */
    int64_t ignore_index;
    const float *lse;              /* from qpam_ce_fwd */
    const float *grad_scale;       /* device scalar: grad_output / denom */
    void *dh; int64_t lddh;        /* dtype of h */
    void *dw; int64_t lddw;        /* dw_out 0: fp32, accumulated (the caller zeroes it);
                                      1: written, in dtype; 2: written, fp32 */
    int32_t chunk;                 /* the reference's row chunk: one pass covers as many rows
                                      as fit the bytes the reference keeps alive for `chunk`
                                      rows (fp32 logits and softmax): 4 chunk rows with bf16
                                      inputs and the library GEMMs (G^T only), 2 chunk rows
                                      with the hand-written GEMMs (G and G^T), chunk rows fp32 */
    void *workspace;
    size_t workspace_bytes;
    int32_t dw_out;                /* ABI 14: 0 = dw accumulated in fp32 as above; 1 = dw written
                                      (not accumulated) in dtype -- with bf16 inputs the weight
                                      gradient leaves in bf16 from the fp32 sums, with no
                                      conversion pass after the call; 2 = dw written in fp32 (an
                                      fp32 master weight run on its bf16 copy), no zero fill */
} qpam_ce_bwd_args;

size_t qpam_ce_bwd_workspace_size(const qpam_ce_bwd_args *a);
int qpam_ce_bwd(const qpam_ce_bwd_args *a, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* QPAM_H */
