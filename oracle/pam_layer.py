"""CPU restatement of the V11PAMLayer forward around the scan (test
infrastructure only: the product never imports this module).

Follows v11/model.py for the production prefill path (head decay, additive
write; E3 fused for n_states > 1):
  _project                  271-306  fused QKV complex projection, RoPE cmul,
                                     optional cnormalize
  _apply_gamma_floor        193-201
  _gamma_and_vprime         309-347  (single state, state_offset = 0)
  _gamma_all_and_vprime     630-655  (E3: one offset per state)
  _phase_and_alpha          230-257  phases [B,T,H,K], routing 1 or K*softmax
  forward                   785-843  dispatch, head merge, o_proj
with ComplexLinear (v11/complex_ops.py:165-172), cabs / cnormalize /
to_real_concat (v11/complex_ops.py:86-97) and build_rope_cache
(v11/complex_ops.py:261-266) restated.  Every function works in the dtype of
its inputs (float64 in the tests).
"""

import torch
import torch.nn.functional as F

from . import pam as O


def cabs(z):
    """v11/complex_ops.py:86-87."""
    return torch.sqrt(z[..., 0].square() + z[..., 1].square() + 1e-8)


def cnormalize(z):
    """v11/complex_ops.py:91-92."""
    return z / cabs(z).unsqueeze(-1)


def to_real_concat(z):
    """v11/complex_ops.py:95-97."""
    return torch.cat([z[..., 0], z[..., 1]], dim=-1)


def complex_linear(z, w_re, w_im, b_re=None, b_im=None):
    """ComplexLinear.forward (v11/complex_ops.py:165-172)."""
    xr, xi = z[..., 0], z[..., 1]
    re = xr @ w_re.T - xi @ w_im.T
    im = xr @ w_im.T + xi @ w_re.T
    if b_re is not None:
        re, im = re + b_re, im + b_im
    return torch.stack([re, im], dim=-1)


def prologue(q, k, v, dt, dt_bias, state_offset, protect, phase, routing, rope, rope_offset, qk_norm,
             gamma_floor):
    """The elementwise steps between the projections and the scan.

    q, k, v: [B,T,H,d,2] projection outputs; dt, protect: [B,T,H] logits
    (protect None = no GSP); state_offset [M] or None (one state, offset 0);
    phase, routing [B,T,H,M] or None; rope [P,d,2] or None.
    Returns q', k', v' [B,H,T,d,2], gamma [M,B,H,T] and (phase, routing)
    permuted to [M,B,H,T] (routing of ones when None), or None without phase.
    """
    q, k, v = (x.transpose(1, 2) for x in (q, k, v))                     # v11/model.py:285-287
    t = q.shape[2]
    if rope is not None:                                                  # :290-301
        r = rope[rope_offset:rope_offset + t].to(q.dtype)
        q, k = O.cmul(q, r), O.cmul(k, r)
    if qk_norm:                                                           # :303-305
        q, k = cnormalize(q), cnormalize(k)
    offs = state_offset.view(-1, 1, 1, 1) if state_offset is not None else torch.zeros(1, 1, 1, 1, dtype=dt.dtype)
    softplus_dt = F.softplus(dt + dt_bias + offs).permute(0, 1, 3, 2)      # [M,B,H,T]  :640-643
    base = torch.exp(-softplus_dt)
    if gamma_floor and gamma_floor > 0.0:                                 # :193-201
        base = gamma_floor + (1.0 - gamma_floor) * base
    if protect is not None:                                               # :644-651
        p = torch.sigmoid(protect).transpose(1, 2)                        # [B,H,T]
        gamma = base * (1 - p) + p
        v = v * (1 - p)[..., None, None]
    else:
        gamma = base
    rot = None
    if phase is not None:                                                 # :741-743
        ph = phase.permute(3, 0, 2, 1)
        ro = routing.permute(3, 0, 2, 1) if routing is not None else torch.ones_like(ph)
        rot = (ph, ro)
    return q, k, v, gamma, rot


def layer_forward(p, cfg, x, step_offset=0):
    """V11PAMLayer.forward for a prefill (state None, T > 1), head decay and
    additive write.  p: parameters by the reference's attribute names
    ('qkv_proj.weight_real', ..., 'dt_proj.weight', 'dt_proj.bias', 'dt_bias',
    'protect_gate.weight/bias', 'state_dt_offset', 'phase_proj.weight/bias',
    'score_proj.weight/bias', 'o_proj.weight_real/imag'); cfg: n_heads,
    head_dim, n_states, chunk_size, use_rope, use_gsp, qk_norm, gamma_floor,
    gate_content_aware, routing_content_aware, state_compete, max_seq_len.
    Returns (out [B,T,dim,2], state)."""
    b, t = x.shape[:2]
    h, d, m = cfg["n_heads"], cfg["head_dim"], cfg["n_states"]
    qkv = complex_linear(x, p["qkv_proj.weight_real"], p["qkv_proj.weight_imag"]).view(b, t, 3, h, d, 2)
    q, k, v = qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2]
    rope = None
    if cfg["use_rope"]:
        rope = O.rope_table(max(cfg["max_seq_len"], 2 * (step_offset + t)), d).to(x.dtype)
    dt = to_real_concat(x) @ p["dt_proj.weight"].T + p["dt_proj.bias"]
    protect = None
    if cfg["use_gsp"]:
        gate_in = to_real_concat(x) if cfg["gate_content_aware"] else cabs(x)
        protect = gate_in @ p["protect_gate.weight"].T + p["protect_gate.bias"]
    phase = routing = None
    offs = None
    if m > 1:
        route_in = to_real_concat(x) if cfg["routing_content_aware"] else cabs(x)
        phase = (route_in @ p["phase_proj.weight"].T + p["phase_proj.bias"]).view(b, t, h, m)
        if cfg["state_compete"]:
            scores = (route_in @ p["score_proj.weight"].T + p["score_proj.bias"]).view(b, t, h, m)
            routing = F.softmax(scores, dim=-1) * m
        offs = p["state_dt_offset"]
    q, k, v, gamma, rot = prologue(q, k, v, dt, p["dt_bias"], offs, protect, phase, routing, rope, step_offset,
                                   cfg["qk_norm"], cfg["gamma_floor"])
    if m > 1:
        y, s = O.multistate_fused(q, k, v, gamma, rot[0], rot[1], d, cfg["chunk_size"])
    else:
        y, s = O.forward_head(q, k, v, gamma[0], d, cfg["chunk_size"])
    y = y.transpose(1, 2).reshape(b, t, h * d, 2)                         # :834-835
    out = complex_linear(y, p["o_proj.weight_real"], p["o_proj.weight_imag"])
    return out, s


def layer_decode(p, cfg, x, step_offset, state):
    """V11PAMLayer.forward in decode form (v11/model.py:830-832 -> _recurrent
    :845-925 for the additive head-decay write): the same projections and
    prologue at position step_offset + t, then the token recurrence.  state:
    [M,B,H,d,d,2] (or None).  Returns (out, state)."""
    b, t = x.shape[:2]
    h, d, m = cfg["n_heads"], cfg["head_dim"], cfg["n_states"]
    qkv = complex_linear(x, p["qkv_proj.weight_real"], p["qkv_proj.weight_imag"]).view(b, t, 3, h, d, 2)
    rope = O.rope_table(2 * (step_offset + t) + 1, d).to(x.dtype) if cfg["use_rope"] else None
    dt = to_real_concat(x) @ p["dt_proj.weight"].T + p["dt_proj.bias"]
    protect = None
    if cfg["use_gsp"]:
        gate_in = to_real_concat(x) if cfg["gate_content_aware"] else cabs(x)
        protect = gate_in @ p["protect_gate.weight"].T + p["protect_gate.bias"]
    phase = routing = offs = None
    if m > 1:
        route_in = to_real_concat(x) if cfg["routing_content_aware"] else cabs(x)
        phase = (route_in @ p["phase_proj.weight"].T + p["phase_proj.bias"]).view(b, t, h, m)
        if cfg["state_compete"]:
            scores = (route_in @ p["score_proj.weight"].T + p["score_proj.bias"]).view(b, t, h, m)
            routing = F.softmax(scores, dim=-1) * m
        offs = p["state_dt_offset"]
    q, k, v, gamma, rot = prologue(qkv[:, :, 0], qkv[:, :, 1], qkv[:, :, 2], dt, p["dt_bias"], offs, protect, phase,
                                   routing, rope, step_offset, cfg["qk_norm"], cfg["gamma_floor"])
    phase_p, routing_p = rot if rot is not None else (None, None)
    y, state = O.recurrent(q, k, v, gamma, d, phase_p, routing_p, state=state)
    y = y.transpose(1, 2).reshape(b, t, h * d, 2)
    return complex_linear(y, p["o_proj.weight_real"], p["o_proj.weight_imag"]), state


def make_layer_params(cfg, dim, seed, dtype=torch.float64):
    """Seeded parameters of the shapes V11PAMLayer.__init__ creates
    (v11/model.py:129-178), drawn at scales that keep the decays and gates
    away from saturation."""
    g = torch.Generator().manual_seed(seed)
    h, d, m = cfg["n_heads"], cfg["head_dim"], cfg["n_states"]
    inner = h * d

    def rn(*shape, std=1.0):
        return (torch.randn(*shape, generator=g) * std).to(dtype)

    p = {
        "qkv_proj.weight_real": rn(3 * inner, dim, std=dim ** -0.5),
        "qkv_proj.weight_imag": rn(3 * inner, dim, std=dim ** -0.5),
        "o_proj.weight_real": rn(dim, inner, std=inner ** -0.5),
        "o_proj.weight_imag": rn(dim, inner, std=inner ** -0.5),
        "dt_proj.weight": rn(h, 2 * dim, std=0.3 * (2 * dim) ** -0.5),
        "dt_proj.bias": rn(h, std=0.1),
        "dt_bias": rn(h, std=0.5) - 2.0,
    }
    if cfg["use_gsp"]:
        gin = 2 * dim if cfg["gate_content_aware"] else dim
        p["protect_gate.weight"] = rn(h, gin, std=gin ** -0.5)
        p["protect_gate.bias"] = rn(h, std=0.1) - 1.0
    if m > 1:
        rin = 2 * dim if cfg["routing_content_aware"] else dim
        p["state_dt_offset"] = torch.linspace(-1.0, 1.0, m, dtype=dtype) + rn(m, std=0.1)
        p["phase_proj.weight"] = rn(h * m, rin, std=rin ** -0.5)
        p["phase_proj.bias"] = rn(h * m, std=1.0)
        if cfg["state_compete"]:
            p["score_proj.weight"] = rn(h * m, rin, std=rin ** -0.5)
            p["score_proj.bias"] = rn(h * m, std=0.1)
    return p
