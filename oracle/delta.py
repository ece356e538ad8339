"""CPU restatement of the QLLM v11 E2 delta-rule write (test infrastructure
only: the product never imports this module).

delta_chunked     V11PAMLayer._forward_delta (v11/model.py:491-576): per chunk
                  the UT-transform solve (I + M) U = W (_complex_triangular_solve,
                  v11/model.py:1005-1016) with M[t,s] = beta_t D[t,s] (k_t . k_s*)
                  strictly lower, W = beta (V - alpha S k), then the dual-form
                  read, the carried read and the state write.
recur_step_delta  V11PAMLayer._recur_step_delta (v11/model.py:967-1002): one
                  token, S <- g S; u = beta (v - S k); S <- S + u (x) k*; y = S q.
delta_recurrent   the token loop of _recur_step_delta with the decay the
                  chunked form uses (g + 1e-6), the independent pin of
                  delta_chunked.
Tensors are split-real [..., d, 2]; queries unscaled (scaled by head_dim^-1/2
inside, as the reference).
"""

import torch

from . import pam as O

EPS = O.EPS


def _csolve_unit_lower(m_re, m_im, w_re, w_im):
    """(I + M) U = W for complex M strictly lower triangular, as the reference
    does it: the real 2C x 2C block system [[I+Mr, -Mi], [Mi, I+Mr]] through
    torch.linalg.solve in float (v11/model.py:1005-1016)."""
    c = m_re.shape[-1]
    eye = torch.eye(c, dtype=m_re.dtype, device=m_re.device)
    top = torch.cat([eye + m_re, -m_im], dim=-1)
    bot = torch.cat([m_im, eye + m_re], dim=-1)
    sol = torch.linalg.solve(torch.cat([top, bot], dim=-2), torch.cat([w_re, w_im], dim=-2))
    return sol[..., :c, :], sol[..., c:, :]


def delta_chunked(queries, keys, values, gamma, beta, head_dim, chunk_size, state=None):
    """_forward_delta.  queries/keys/values [B,H,T,d,2], gamma/beta [B,H,T],
    state optional [B,H,d,d,2] (the reference starts from zero; a nonzero start
    is the same algebra with the carried terms on the first chunk).
    Returns (Y [B,H,T,d,2], S [B,H,d,d,2])."""
    b, h, t, d = queries.shape[:4]
    scale = head_dim ** -0.5
    s = state.clone() if state is not None else queries.new_zeros(b, h, d, d, 2)
    has_state = state is not None
    outs = []
    for c0 in range(0, t, chunk_size):
        c1 = min(c0 + chunk_size, t)
        n = c1 - c0
        q, k, v = queries[:, :, c0:c1], keys[:, :, c0:c1], values[:, :, c0:c1]
        g, bt = gamma[:, :, c0:c1], beta[:, :, c0:c1]
        dmat = O.decay_matrix(g.reshape(b * h, n), n).reshape(b, h, n, n)      # D[t,s]
        alpha = torch.exp(torch.cumsum(torch.log(g + EPS), dim=-1))            # prod_{0..t}
        kr, ki, qr, qi = k[..., 0], k[..., 1], q[..., 0], q[..., 1]
        gram_r = kr @ kr.transpose(-1, -2) + ki @ ki.transpose(-1, -2)
        gram_i = ki @ kr.transpose(-1, -2) - kr @ ki.transpose(-1, -2)
        strict = torch.tril(torch.ones(n, n, dtype=q.dtype, device=q.device), -1)
        m_re = bt.unsqueeze(-1) * dmat * strict * gram_r
        m_im = bt.unsqueeze(-1) * dmat * strict * gram_i
        vr, vi = v[..., 0], v[..., 1]
        if c0 > 0 or has_state:
            sr, si = s[..., 0], s[..., 1]
            sk_r = (kr @ sr.transpose(-1, -2) - ki @ si.transpose(-1, -2)) * alpha.unsqueeze(-1)
            sk_i = (kr @ si.transpose(-1, -2) + ki @ sr.transpose(-1, -2)) * alpha.unsqueeze(-1)
            w_re, w_im = bt.unsqueeze(-1) * (vr - sk_r), bt.unsqueeze(-1) * (vi - sk_i)
        else:
            w_re, w_im = bt.unsqueeze(-1) * vr, bt.unsqueeze(-1) * vi
        u_re, u_im = _csolve_unit_lower(m_re, m_im, w_re, w_im)
        qk_r = qr @ kr.transpose(-1, -2) + qi @ ki.transpose(-1, -2)
        qk_i = qi @ kr.transpose(-1, -2) - qr @ ki.transpose(-1, -2)
        causal = torch.tril(torch.ones(n, n, dtype=q.dtype, device=q.device))
        p_r, p_i = dmat * causal * qk_r, dmat * causal * qk_i
        y = torch.stack([(p_r @ u_re - p_i @ u_im) * scale, (p_r @ u_im + p_i @ u_re) * scale], -1)
        if c0 > 0 or has_state:
            sr, si = s[..., 0], s[..., 1]
            sq_r, sq_i = qr * scale * alpha.unsqueeze(-1), qi * scale * alpha.unsqueeze(-1)
            y = y + torch.stack([sq_r @ sr.transpose(-1, -2) - sq_i @ si.transpose(-1, -2),
                                 sq_r @ si.transpose(-1, -2) + sq_i @ sr.transpose(-1, -2)], -1)
        outs.append(y)
        total = alpha[:, :, -1:]
        tail = total / (alpha + 1e-12)
        ud_r, ud_i = u_re * tail.unsqueeze(-1), u_im * tail.unsqueeze(-1)
        ns_r = ud_r.transpose(-1, -2) @ kr + ud_i.transpose(-1, -2) @ ki
        ns_i = ud_i.transpose(-1, -2) @ kr - ud_r.transpose(-1, -2) @ ki
        s = s * total.unsqueeze(-1).unsqueeze(-1) + torch.stack([ns_r, ns_i], -1)
    return torch.cat(outs, dim=2), s


def recur_step_delta(state, gamma_t, value_t, key_t, query_t, beta_t):
    """_recur_step_delta (v11/model.py:967-1002).  state [..., d, d, 2],
    gamma_t/beta_t [...], value/key/query [..., d, 2] (query already scaled)."""
    s = state * gamma_t[..., None, None, None]
    kr, ki = key_t[..., 0].unsqueeze(-2), key_t[..., 1].unsqueeze(-2)
    pred_r = (s[..., 0] * kr - s[..., 1] * ki).sum(-1)
    pred_i = (s[..., 0] * ki + s[..., 1] * kr).sum(-1)
    bt = beta_t.unsqueeze(-1)
    u_r, u_i = bt * (value_t[..., 0] - pred_r), bt * (value_t[..., 1] - pred_i)
    cr, ci = key_t[..., 0].unsqueeze(-2), -key_t[..., 1].unsqueeze(-2)
    s = s + torch.stack([u_r.unsqueeze(-1) * cr - u_i.unsqueeze(-1) * ci,
                         u_r.unsqueeze(-1) * ci + u_i.unsqueeze(-1) * cr], -1)
    qr, qi = query_t[..., 0].unsqueeze(-2), query_t[..., 1].unsqueeze(-2)
    y = torch.stack([(s[..., 0] * qr - s[..., 1] * qi).sum(-1), (s[..., 0] * qi + s[..., 1] * qr).sum(-1)], -1)
    return y, s


def delta_recurrent(queries, keys, values, gamma, beta, head_dim, state=None, eps=EPS):
    """Token loop of recur_step_delta with decay gamma + eps (the chunked form's
    per-step factor).  Returns (Y, S) like delta_chunked."""
    b, h, t, d = queries.shape[:4]
    s = state.clone() if state is not None else queries.new_zeros(b, h, d, d, 2)
    scale = head_dim ** -0.5
    ys = []
    for ti in range(t):
        y, s = recur_step_delta(s, gamma[:, :, ti] + eps, values[:, :, ti], keys[:, :, ti],
                                queries[:, :, ti] * scale, beta[:, :, ti])
        ys.append(y)
    return torch.stack(ys, 2), s


def make_delta_inputs(B, H, T, d, seed, dtype=torch.float64, unit_keys=True):
    """Seeded inputs: complex N(0,1) q, v; keys normalised to unit norm per
    token (the reference feeds cnormalize'd or RMS-scaled keys; unit keys keep
    the delta rule's (I + M) well conditioned); gamma in (0.5, 1), beta in
    (0, 1)."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, T, d, 2, generator=g, dtype=torch.float64)
    k = torch.randn(B, H, T, d, 2, generator=g, dtype=torch.float64)
    v = torch.randn(B, H, T, d, 2, generator=g, dtype=torch.float64)
    if unit_keys:
        k = k / k.square().sum((-1, -2), keepdim=True).sqrt()
    gamma = 0.5 + 0.5 * torch.sigmoid(torch.randn(B, H, T, generator=g, dtype=torch.float64) + 2)
    beta = torch.sigmoid(torch.randn(B, H, T, generator=g, dtype=torch.float64))
    return tuple(x.to(dtype) for x in (q, k, v, gamma, beta))
