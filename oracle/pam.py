"""CPU restatement of the QLLM v11 PAM scan and decode (test infrastructure only).

Every function restates the reference algorithm in torch-on-CPU, keeping the
reference's numerical conventions:
  * split-real interleaved complex tensors ``[..., 2]`` (v11/complex_ops.py:29-45),
  * log-decay ``log(gamma + 1e-6)`` and the ``-1e4`` causal mask before
    ``clamp(max=0)`` (v11/flash_pam.py:40-52, v11/triton_kernels.py:522-528),
  * queries scaled by ``head_dim ** -0.5`` before chunking (v11/model.py:381-382).

Backward passes are torch autograd through these forward restatements, exactly
as the reference obtains its gradients (it has no hand-written PAM backward
apart from the decay-matrix closed form, v11/triton_kernels.py:447-480, which
equals autograd of the PyTorch fallback away from clamp ties).

Independent pins (brute-force complex128 recurrences, textbook outer-product
updates) live at the bottom of this file; tests/test_oracle_pam.py checks the
restatement against them.
"""

import math

import numpy as np
import torch

EPS = 1e-6  # v11/flash_pam.py:45, v11/model.py:395


# ---------------------------------------------------------------- helpers ----

def _re(z):
    return z[..., 0]


def _im(z):
    return z[..., 1]


def _stack(r, i):
    return torch.stack([r, i], dim=-1)


def cmul(a, b):
    """(a_r + i a_i)(b_r + i b_i) on split-real tensors (v11/complex_ops.py:73-79)."""
    return _stack(_re(a) * _re(b) - _im(a) * _im(b), _re(a) * _im(b) + _im(a) * _re(b))


def to_planar(z):
    """[..., d, 2] interleaved -> (re, im) contiguous planes."""
    return z[..., 0].contiguous(), z[..., 1].contiguous()


def from_planar(re, im):
    return torch.stack([re, im], dim=-1)


# ------------------------------------------------------ a1: decay matrices ----

def decay_matrices(decay_gamma, chunk_len=None):
    """[N, C] -> (D [N,C,C], cum [N,C], total [N], decay_last [N,C]).

    Follows v11/flash_pam.py:32-53 (and the PyTorch fallback
    v11/triton_kernels.py:522-528 for D):
      c      = cumsum(-log(gamma + 1e-6))
      D[t,s] = exp(min(c[s] - c[t], 0)) for s <= t, exp(-1e4) = 0 otherwise
      cum[t] = exp(cumsum(log(gamma + 1e-6)))[t],  total = cum[C-1]
      decay_last[s] = D[C-1, s]
    bf16/fp16 gamma is computed in fp32 (v11/flash_pam.py:40-44).
    """
    chunk_len = decay_gamma.shape[-1] if chunk_len is None else chunk_len
    compute_dtype = (torch.float32 if decay_gamma.dtype in (torch.bfloat16, torch.float16)
                     else decay_gamma.dtype)
    log_decay = torch.log(decay_gamma.to(compute_dtype) + EPS)
    cum_neg = torch.cumsum(-log_decay, dim=-1)
    log_d = (cum_neg.unsqueeze(-1) - cum_neg.unsqueeze(-2)).transpose(-1, -2)
    causal = torch.tril(torch.ones(chunk_len, chunk_len, dtype=compute_dtype, device=decay_gamma.device))
    log_d = log_d * causal + (1 - causal) * (-1e4)
    d_mat = torch.exp(log_d.clamp(max=0.0))
    cum = torch.exp(torch.cumsum(log_decay, dim=-1))
    return d_mat, cum, cum[..., -1], d_mat[..., -1, :]


def decay_matrix(decay_gamma, seq_len):
    """fused_decay_matrix semantics (v11/triton_kernels.py:570-573 -> 522-528)."""
    return decay_matrices(decay_gamma, seq_len)[0].to(decay_gamma.dtype)


# ------------------------------------------------- a2: dual-form block -------

def dual_form_block(scaled_queries, keys, protected_values, decay_gamma):
    """One chunk, zero incoming state (v11/model.py:354-376).

    scaled_queries, keys, protected_values: [B,H,C,d,2]; decay_gamma [B,H,C].
    Returns output [B,H,C,d,2] and chunk state [B,H,d,d,2] (S[i,j] = value i, key j).
    """
    b, h, c = decay_gamma.shape
    d_mat = decay_matrix(decay_gamma.reshape(b * h, c), c).reshape(b, h, c, c)
    qr, qi = _re(scaled_queries), _im(scaled_queries)
    kr, ki = _re(keys), _im(keys)
    w_r = qr @ kr.transpose(-1, -2) + qi @ ki.transpose(-1, -2)
    w_i = qi @ kr.transpose(-1, -2) - qr @ ki.transpose(-1, -2)
    a_r, a_i = w_r * d_mat, w_i * d_mat
    vr, vi = _re(protected_values), _im(protected_values)
    out = _stack(a_r @ vr - a_i @ vi, a_r @ vi + a_i @ vr)
    last = d_mat[:, :, -1, :].unsqueeze(-1)
    wvr, wvi = vr * last, vi * last
    s_r = wvr.transpose(-1, -2) @ kr + wvi.transpose(-1, -2) @ ki
    s_i = wvi.transpose(-1, -2) @ kr - wvr.transpose(-1, -2) @ ki
    return out, _stack(s_r, s_i)


# ------------------------------------------ a3: chunked head (one state) -----

def chunked_head(queries, keys, protected_values, decay_gamma, head_dim, chunk_size):
    """V11PAMLayer._forward_chunked_head (v11/model.py:378-417).

    queries NOT pre-scaled.  Per chunk c with S_0 = 0:
      Y_c[t] = sum_{s<=t} D[t,s] (q~_t . k_s*) v_s + cum[t] * S_{c-1} q~_t
      S_c    = total_c * S_{c-1} + sum_s D[C-1,s] v_s (x) k_s*
    The last chunk may be ragged.
    """
    b, h, t = queries.shape[:3]
    sq = queries * head_dim ** -0.5
    state = queries.new_zeros(b, h, head_dim, head_dim, 2)
    outs = []
    for c0 in range(0, t, chunk_size):
        c1 = min(c0 + chunk_size, t)
        q_c, k_c, v_c, g_c = sq[:, :, c0:c1], keys[:, :, c0:c1], protected_values[:, :, c0:c1], decay_gamma[:, :, c0:c1]
        out_c, ds = dual_form_block(q_c, k_c, v_c, g_c)
        cum = torch.exp(torch.cumsum(torch.log(g_c + EPS), dim=-1))
        if c0 > 0:
            sr, si = _re(state), _im(state)
            qr, qi = _re(q_c), _im(q_c)
            car_r = (sr @ qr.transpose(-1, -2) - si @ qi.transpose(-1, -2)).transpose(-1, -2)
            car_i = (sr @ qi.transpose(-1, -2) + si @ qr.transpose(-1, -2)).transpose(-1, -2)
            ce = cum.unsqueeze(-1)
            out_c = out_c + _stack(car_r * ce, car_i * ce)
        outs.append(out_c)
        state = state * cum[:, :, -1][..., None, None, None] + ds
    return torch.cat(outs, dim=2), state


def forward_head(queries, keys, protected_values, decay_gamma, head_dim, chunk_size):
    """Single-state prefill dispatch of V11PAMLayer.forward (v11/model.py:818-829):
    chunked when T > C, one dual-form block otherwise."""
    t = queries.shape[2]
    if chunk_size > 0 and t > chunk_size:
        return chunked_head(queries, keys, protected_values, decay_gamma, head_dim, chunk_size)
    return dual_form_block(queries * head_dim ** -0.5, keys, protected_values, decay_gamma)


# ------------------------------------------ E1: per-channel decay ------------

def chunked_perchannel(queries, keys, protected_values, decay_gamma, head_dim, chunk_size):
    """V11PAMLayer._forward_chunked_perchannel (v11/model.py:421-489).

    decay_gamma [B,H,T,d]: one decay per key channel j, S[i,j] <- g_j S[i,j]
    + v_i conj(k_j).  Per chunk the decay is folded into the operands: with
    L = max(cumsum(log max(g, 1e-6)), -30) (inclusive), queries carry e^{L}
    and keys e^{-L}, so the masked score (q e^L)(k e^-L)* is the decayed
    score; the carried read is (q e^L) S^T, and the state update weights each
    key by e^{L_last - L} and decays S's columns by e^{L_last}.  Queries are
    unscaled on entry (scaled by head_dim**-0.5 here)."""
    b, h, t = queries.shape[:3]
    scale = head_dim ** -0.5
    state = queries.new_zeros(b, h, head_dim, head_dim, 2)
    outs = []
    for c0 in range(0, t, chunk_size):
        c1 = min(c0 + chunk_size, t)
        n = c1 - c0
        q_c, k_c, v_c = queries[:, :, c0:c1], keys[:, :, c0:c1], protected_values[:, :, c0:c1]
        lg = torch.log(decay_gamma[:, :, c0:c1].clamp_min(1e-6)).float()
        cl = torch.cumsum(lg, dim=2).clamp(min=-30.0)                     # [B,H,n,d]
        a = torch.exp(cl).to(queries.dtype)
        inv = torch.exp(-cl).to(queries.dtype)
        tail = torch.exp(cl[:, :, -1:] - cl).to(queries.dtype)
        a_tot = torch.exp(cl[:, :, -1]).to(queries.dtype)                 # [B,H,d]
        fq = q_c * (a * scale).unsqueeze(-1)
        fk = k_c * inv.unsqueeze(-1)
        w_r = _re(fq) @ _re(fk).transpose(-1, -2) + _im(fq) @ _im(fk).transpose(-1, -2)
        w_i = _im(fq) @ _re(fk).transpose(-1, -2) - _re(fq) @ _im(fk).transpose(-1, -2)
        mask = torch.tril(torch.ones(n, n, dtype=w_r.dtype, device=w_r.device))
        w_r, w_i = w_r * mask, w_i * mask
        vr, vi = _re(v_c), _im(v_c)
        out = _stack(w_r @ vr - w_i @ vi, w_r @ vi + w_i @ vr)
        if c0 > 0:
            sr, si = _re(state), _im(state)
            out = out + _stack(_re(fq) @ sr.transpose(-1, -2) - _im(fq) @ si.transpose(-1, -2),
                               _re(fq) @ si.transpose(-1, -2) + _im(fq) @ sr.transpose(-1, -2))
        outs.append(out)
        dk = k_c * tail.unsqueeze(-1)
        s_r = vr.transpose(-1, -2) @ _re(dk) + vi.transpose(-1, -2) @ _im(dk)
        s_i = vi.transpose(-1, -2) @ _re(dk) - vr.transpose(-1, -2) @ _im(dk)
        state = state * a_tot[:, :, None, :, None] + _stack(s_r, s_i)
    return torch.cat(outs, dim=2), state


# ------------------------------------------ a4: flash_pam_chunked_head -------

def flash_pam_chunked_head(queries, keys, protected_values, decay_gamma, head_dim, chunk_size):
    """v11/flash_pam.py:56-152: pads q/k/v with 0 and gamma with 1 to a chunk
    multiple, runs all intra-chunk products at once, then the sequential carry."""
    b, h, t = queries.shape[:3]
    c = chunk_size
    n = (t + c - 1) // c
    pad = n * c - t
    sq = queries * head_dim ** -0.5
    k, v, g = keys, protected_values, decay_gamma
    if pad:
        sq = torch.nn.functional.pad(sq, (0, 0, 0, 0, 0, pad))
        k = torch.nn.functional.pad(k, (0, 0, 0, 0, 0, pad))
        v = torch.nn.functional.pad(v, (0, 0, 0, 0, 0, pad))
        g = torch.nn.functional.pad(g, (0, pad), value=1.0)
    nb = b * h * n
    qc = sq.reshape(nb, c, head_dim, 2)
    kc = k.reshape(nb, c, head_dim, 2)
    vc = v.reshape(nb, c, head_dim, 2)
    d_mat, cum, total, last = decay_matrices(g.reshape(nb, c), c)
    qr, qi, kr, ki, vr, vi = _re(qc), _im(qc), _re(kc), _im(kc), _re(vc), _im(vc)
    w_r = torch.bmm(qr, kr.transpose(-1, -2)) + torch.bmm(qi, ki.transpose(-1, -2))
    w_i = torch.bmm(qi, kr.transpose(-1, -2)) - torch.bmm(qr, ki.transpose(-1, -2))
    d_t = d_mat.to(w_r.dtype)
    a_r, a_i = w_r * d_t, w_i * d_t
    intra = _stack(torch.bmm(a_r, vr) - torch.bmm(a_i, vi), torch.bmm(a_r, vi) + torch.bmm(a_i, vr))
    le = last.unsqueeze(-1).to(vr.dtype)
    wvr, wvi = vr * le, vi * le
    s_r = torch.bmm(wvr.transpose(-1, -2), kr) + torch.bmm(wvi.transpose(-1, -2), ki)
    s_i = torch.bmm(wvi.transpose(-1, -2), kr) - torch.bmm(wvr.transpose(-1, -2), ki)
    ds = _stack(s_r, s_i).view(b, h, n, head_dim, head_dim, 2)
    intra = intra.view(b, h, n, c, head_dim, 2)
    cum = cum.view(b, h, n, c).to(queries.dtype)
    total = total.view(b, h, n).to(queries.dtype)
    sqc = sq.view(b, h, n, c, head_dim, 2)
    state = queries.new_zeros(b, h, head_dim, head_dim, 2)
    outs = []
    for ci in range(n):
        o = intra[:, :, ci]
        if ci > 0:
            sr, si = _re(state), _im(state)
            q_r, q_i = sqc[:, :, ci, ..., 0], sqc[:, :, ci, ..., 1]
            car_r = (sr @ q_r.transpose(-1, -2) - si @ q_i.transpose(-1, -2)).transpose(-1, -2)
            car_i = (sr @ q_i.transpose(-1, -2) + si @ q_r.transpose(-1, -2)).transpose(-1, -2)
            ce = cum[:, :, ci].unsqueeze(-1)
            o = o + _stack(car_r * ce, car_i * ce)
        outs.append(o)
        state = state * total[:, :, ci][..., None, None, None] + ds[:, :, ci]
    out = torch.cat(outs, dim=2)
    return (out[:, :, :t] if pad else out), state


# ------------------------------------------ a5: E3 fused multistate ----------

def fused_chunk_step(q_c, k_c, v_c, gamma_c, phase_c, routing_c, state, is_first):
    """V11PAMLayer._fused_chunk_step (v11/model.py:657-737).

    q_c (scaled), k_c, v_c: [B,H,C,d,2]; gamma_c, phase_c, routing_c: [M,B,H,C];
    state [M,B,H,d,d,2].  D~ = sum_m r_m D_m with r_m = routing_m e^{i phase_m}.
    """
    m, b, h, c = gamma_c.shape
    qr, qi, kr, ki = _re(q_c), _im(q_c), _re(k_c), _im(k_c)
    w_r = qr @ kr.transpose(-1, -2) + qi @ ki.transpose(-1, -2)
    w_i = qi @ kr.transpose(-1, -2) - qr @ ki.transpose(-1, -2)
    d_mat = decay_matrix(gamma_c.reshape(m * b * h, c), c).reshape(m, b, h, c, c)
    cos_p, sin_p = torch.cos(phase_c), torch.sin(phase_c)
    dt_r = ((routing_c * cos_p).unsqueeze(-1) * d_mat).sum(0)
    dt_i = ((routing_c * sin_p).unsqueeze(-1) * d_mat).sum(0)
    a_r = w_r * dt_r - w_i * dt_i
    a_i = w_r * dt_i + w_i * dt_r
    vr, vi = _re(v_c), _im(v_c)
    out = _stack(a_r @ vr - a_i @ vi, a_r @ vi + a_i @ vr)
    cum = torch.exp(torch.cumsum(torch.log(gamma_c + EPS), dim=-1))
    if not is_first:
        sr, si = _re(state), _im(state)
        qrs, qis = qr.unsqueeze(0), qi.unsqueeze(0)
        car_r = (sr @ qrs.transpose(-1, -2) - si @ qis.transpose(-1, -2)).transpose(-1, -2)
        car_i = (sr @ qis.transpose(-1, -2) + si @ qrs.transpose(-1, -2)).transpose(-1, -2)
        comb_r = (routing_c * cos_p * cum).unsqueeze(-1)
        comb_i = (routing_c * sin_p * cum).unsqueeze(-1)
        out = out + _stack((car_r * comb_r - car_i * comb_i).sum(0), (car_r * comb_i + car_i * comb_r).sum(0))
    last = d_mat[:, :, :, -1, :].unsqueeze(-1)
    wvr, wvi = vr.unsqueeze(0) * last, vi.unsqueeze(0) * last
    krs, kis = kr.unsqueeze(0), ki.unsqueeze(0)
    s_r = wvr.transpose(-1, -2) @ krs + wvi.transpose(-1, -2) @ kis
    s_i = wvi.transpose(-1, -2) @ krs - wvr.transpose(-1, -2) @ kis
    new_state = state * cum[..., -1][..., None, None, None] + _stack(s_r, s_i)
    return out, new_state


def multistate_fused(queries, keys, protected_values, gamma_all, phase, routing, head_dim, chunk_size,
                     state=None):
    """Chunk loop of V11PAMLayer._forward_multistate_fused (v11/model.py:739-781),
    with the per-state decay gamma_all [M,B,H,T], phase and routing [M,B,H,T]
    already produced by the layer's prologue.  Returns (Y, S [M,B,H,d,d,2])."""
    m = gamma_all.shape[0]
    b, h, t = queries.shape[:3]
    c = chunk_size if chunk_size > 0 else t
    sq = queries * head_dim ** -0.5
    first = state is None
    if state is None:
        state = queries.new_zeros(m, b, h, head_dim, head_dim, 2)
    outs = []
    for c0 in range(0, t, c):
        c1 = min(c0 + c, t)
        o, state = fused_chunk_step(sq[:, :, c0:c1], keys[:, :, c0:c1], protected_values[:, :, c0:c1],
                                    gamma_all[..., c0:c1], phase[..., c0:c1], routing[..., c0:c1],
                                    state, first and c0 == 0)
        outs.append(o)
    return torch.cat(outs, dim=2), state


# ------------------------------------------ a6: K-loop multistate ------------

def multistate_loop(queries, keys, protected_values, gamma_all, phase, routing, head_dim, chunk_size):
    """V11PAMLayer._forward_multistate (v11/model.py:580-614): one single-state
    scan per state, outputs rotated by routing*e^{i phase} and summed."""
    m = gamma_all.shape[0]
    total = None
    states = []
    for s in range(m):
        y, st = forward_head(queries, keys, protected_values, gamma_all[s], head_dim, chunk_size)
        rot = _stack(routing[s] * torch.cos(phase[s]), routing[s] * torch.sin(phase[s]))
        y = cmul(y, rot.unsqueeze(-2))
        total = y if total is None else total + y
        states.append(st)
    return total, torch.stack(states, dim=0)


# ------------------------------------------ a7: recurrent decode -------------

def recur_step_additive(state, decay_gamma, value_t, key_t, query_t):
    """V11PAMLayer._recur_step_additive (v11/model.py:927-965).

    state [..., d, d, 2]; decay_gamma [...] (head scalar) or [..., d] (E1: one
    decay per key channel j, v11/model.py:948-954); value_t/key_t/query_t
    [..., d, 2] (query already scaled).  S <- gamma*S + v (x) k*;  y = S q
    (update before read).
    """
    kc = _stack(_re(key_t), -_im(key_t)).unsqueeze(-3)
    vr, vi = _re(value_t).unsqueeze(-1), _im(value_t).unsqueeze(-1)
    outer = _stack(vr * _re(kc) - vi * _im(kc), vr * _im(kc) + vi * _re(kc))
    if decay_gamma.dim() == state.dim() - 3:
        state = state * decay_gamma[..., None, None, None] + outer
    else:
        state = state * decay_gamma[..., None, :, None] + outer
    qr, qi = _re(query_t).unsqueeze(-2), _im(query_t).unsqueeze(-2)
    y = _stack((_re(state) * qr - _im(state) * qi).sum(-1), (_re(state) * qi + _im(state) * qr).sum(-1))
    return y, state


def recurrent(queries, keys, protected_values, gamma_all, head_dim, phase=None, routing=None, state=None):
    """Token loop of V11PAMLayer._recurrent (v11/model.py:845-925) for the
    additive head-decay write, M >= 1 states.

    queries/keys/protected_values [B,H,T,d,2] (queries unscaled); gamma_all
    [M,B,H,T]; optional phase/routing [M,B,H,T] rotate each state's read.
    Returns (Y [B,H,T,d,2], state [M,B,H,d,d,2]).
    """
    m = gamma_all.shape[0]
    b, h, t, d = queries.shape[:4]
    if state is None:
        state = queries.new_zeros(m, b, h, d, d, 2)
    scale = head_dim ** -0.5
    ys = []
    for ti in range(t):
        acc = None
        new_states = []
        for s in range(m):
            y, st = recur_step_additive(state[s], gamma_all[s, :, :, ti], protected_values[:, :, ti],
                                        keys[:, :, ti], queries[:, :, ti] * scale)
            if phase is not None:
                rot = _stack(routing[s, :, :, ti] * torch.cos(phase[s, :, :, ti]),
                             routing[s, :, :, ti] * torch.sin(phase[s, :, :, ti]))
                y = cmul(y, rot.unsqueeze(-2))
            acc = y if acc is None else acc + y
            new_states.append(st)
        ys.append(acc)
        state = torch.stack(new_states, 0)
    return torch.stack(ys, dim=2), state


def rope_table(max_len, head_dim):
    """e^{i m theta_j}, theta_j = 10000^(-j/head_dim), [max_len, head_dim, 2] in
    float64 (v11/complex_ops.py:261-266 computes the same angles in fp32)."""
    j = np.arange(head_dim, dtype=np.float64)
    inv = 1.0 / (10000.0 ** (j / head_dim))
    ang = np.arange(max_len, dtype=np.float64)[:, None] * inv[None, :]
    return torch.from_numpy(np.stack([np.cos(ang), np.sin(ang)], -1))


def decode_slots(state, active, q, k, v, gamma, q_scale, rot=None, rope=None, pos=None):
    """One continuous-batching decode step over a slot pool (config 4 semantics).

    state [S, G, M, d, d, 2] (G = layers*heads groups, M states), active: 1-D
    int tensor of slot ids, q/k/v [S, G, d, 2] (q unscaled), gamma [S, G, M],
    rot optional [S, G, M, 2].  With rope [P, d, 2] and pos [S], q and k of
    slot a are first multiplied by rope[pos[a]] (the reference's
    cmul(queries, rope_cache[step_offset]), v11/model.py:290-301, with one
    offset per slot).  For every active slot and group applies
    recur_step_additive per state, rotates, sums over M.  Returns (y [S,G,d,2]
    with zeros for inactive slots, new state) -- inactive slots untouched.
    """
    state = state.clone()
    y = torch.zeros_like(q)
    for sl in active.tolist():
        acc = None
        qs, ks = q[sl], k[sl]
        if rope is not None:
            r = rope[int(pos[sl])].to(q.dtype)
            qs, ks = cmul(qs, r), cmul(ks, r)
        for m in range(state.shape[2]):
            ym, st = recur_step_additive(state[sl, :, m], gamma[sl, :, m], v[sl], ks, qs * q_scale)
            state[sl, :, m] = st
            if rot is not None:
                ym = cmul(ym, rot[sl, :, m].unsqueeze(-2))
            acc = ym if acc is None else acc + ym
        y[sl] = acc
    return y, state


# ------------------------------------------ independent pins -----------------

def brute_force_scan(q, k, v, gamma, scale, eps=0.0, state0=None):
    """Textbook recurrence in complex128 numpy, independent of the chunked code:
        S_t = (gamma_t + eps) S_{t-1} + v_t k_t^H,   y_t = S_t (scale q_t)
    q,k,v: complex arrays [..., T, d]; gamma [..., T].  Returns (y, S_T).
    (memory_probes/core.py:92-101 states the same update.)"""
    q = np.asarray(q, dtype=np.complex128)
    k = np.asarray(k, dtype=np.complex128)
    v = np.asarray(v, dtype=np.complex128)
    g = np.asarray(gamma, dtype=np.float64) + eps
    t, d = q.shape[-2], q.shape[-1]
    s = np.zeros(q.shape[:-2] + (d, d), np.complex128) if state0 is None else np.array(state0, np.complex128)
    y = np.zeros_like(q)
    for ti in range(t):
        s = g[..., ti, None, None] * s + v[..., ti, :, None] * np.conj(k[..., ti, None, :])
        y[..., ti, :] = np.einsum('...ij,...j->...i', s, scale * q[..., ti, :])
    return y, s


def brute_force_perchannel(q, k, v, gamma, scale):
    """E1 textbook recurrence in complex128 numpy: one decay per key channel,
        S_t[i, j] = gamma_t[j] S_{t-1}[i, j] + v_t[i] conj(k_t[j]),  y_t = S_t (scale q_t).
    q,k,v complex [..., T, d]; gamma [..., T, d].  Returns (y, S_T)."""
    q = np.asarray(q, dtype=np.complex128)
    k = np.asarray(k, dtype=np.complex128)
    v = np.asarray(v, dtype=np.complex128)
    g = np.asarray(gamma, dtype=np.float64)
    t, d = q.shape[-2], q.shape[-1]
    s = np.zeros(q.shape[:-2] + (d, d), np.complex128)
    y = np.zeros_like(q)
    for ti in range(t):
        s = g[..., ti, None, :] * s + v[..., ti, :, None] * np.conj(k[..., ti, None, :])
        y[..., ti, :] = np.einsum('...ij,...j->...i', s, scale * q[..., ti, :])
    return y, s


def to_complex(z):
    """split-real torch tensor [..., 2] -> complex128 numpy."""
    z = z.detach().to(torch.float64).numpy()
    return z[..., 0] + 1j * z[..., 1]


def from_complex(a, dtype=torch.float64):
    return torch.from_numpy(np.stack([a.real, a.imag], axis=-1)).to(dtype)


# ------------------------------------------ synthetic inputs (BASELINE) -----

def make_scan_inputs(B, H, T, d, seed, *, m_states=1, unit_qk=False, gamma_mu=3.0,
                     gamma_mu_step=0.0, qkv_std=1.0, dtype=torch.float32):
    """Seeded CPU inputs drawn in float64 in the order q, k, v, gamma-logits
    (then cast): complex Gaussians with independent re/im ~N(0, qkv_std^2),
    optional unit L2 norm per (b,h,t) head vector for q and k, and
    gamma_m = sigmoid(N(gamma_mu + m*gamma_mu_step, 1)) per (m,b,h,t)."""
    g = torch.Generator('cpu').manual_seed(seed)

    def cg():
        return torch.randn(B, H, T, d, 2, generator=g, dtype=torch.float64) * qkv_std

    q, k, v = cg(), cg(), cg()
    if unit_qk:
        q = q / q.square().sum(dim=(-1, -2), keepdim=True).sqrt()
        k = k / k.square().sum(dim=(-1, -2), keepdim=True).sqrt()
    logits = torch.randn(m_states, B, H, T, generator=g, dtype=torch.float64)
    mu = gamma_mu + gamma_mu_step * torch.arange(m_states, dtype=torch.float64).view(-1, 1, 1, 1)
    gamma = torch.sigmoid(logits + mu)
    return q.to(dtype), k.to(dtype), v.to(dtype), gamma.to(dtype)


def scan_flops(B, H, T, d, C, M=1, backward=False):
    """Algorithmic FLOPs of the chunked scan, dense-chunk convention, 8 flops
    per complex MAC: per chunk 16 C^2 d (score + intra read) + 16 M C d^2
    (carried read + state write); backward doubles it."""
    n = math.ceil(T / C)
    f = B * H * n * (16 * C * C * d + 16 * M * C * d * d)
    return 3 * f if backward else f
