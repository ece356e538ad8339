"""Class-shaped CPU restatement of V11PAMLayer (test infrastructure only: the
product never imports this module).

The reference's drop-in boundary is a set of methods of one class,
V11PAMLayer (v11/model.py:99-1002), so install() is tested on a class with
the same attribute and method names whose bodies restate the reference's
algorithm on top of the oracle functions (oracle/pam.py, oracle/delta.py,
oracle/pam_layer.py).  The prefill dispatch of forward (785-843), the K-loop
(580-614), the fused E3 chunk loop (739-781) and the decode loop of
_recurrent (845-925) call the layer's own methods, as the reference does, so
a subclass whose methods install() rebinds runs the rebound ones.

Method -> reference lines:
  _apply_gamma_floor 193-201, _phase_and_alpha 230-257, _route_balance_loss
  259-268, _project 271-306, _gamma_and_vprime 309-347, _dual_form_block
  354-376, _forward_chunked_head 378-417, _forward_chunked_perchannel 421-489,
  _forward_delta 491-576, _forward_multistate 580-614, _gamma_all_and_vprime
  630-655, _fused_chunk_step 657-737, _forward_multistate_fused 739-781,
  forward 785-843, _recurrent 845-925, _recur_step_additive 927-965,
  _recur_step_delta 967-1002.

Parameters keep the reference's names (qkv_proj.weight_real/imag,
o_proj.weight_real/imag, dt_proj.weight/bias, dt_bias, protect_gate.*,
beta_proj.*, state_dt_offset, phase_proj.*, score_proj.*).  The module runs
in the dtype and on the device of its parameters; dropout is the identity
(the reference's self-test runs with dropout 0).
"""

import torch
import torch.nn.functional as F
from torch import nn

from . import delta as OD
from . import pam as O
from . import pam_layer as L

DEFAULTS = dict(dim=32, n_heads=2, head_dim=16, n_states=1, chunk_size=24, use_rope=True, use_gsp=True,
                qk_norm=False, gamma_floor=0.0, gate_content_aware=False, routing_content_aware=False,
                state_compete=False, max_seq_len=512, decay_mode="head", write_mode="additive", delta_chunk=64,
                fused_e3=True, route_balance_lambda=0.0)


def config(**overrides):
    c = dict(DEFAULTS)
    c.update(overrides)
    return c


def make_params(cfg, seed, dtype=torch.float64):
    """Seeded parameters by the reference's names: oracle/pam_layer.py's
    make_layer_params, plus the E1 decay projection (H*d outputs, bias [H,d],
    v11/model.py:142-147) and the E2 write-strength projection (:156-158)."""
    p = L.make_layer_params(cfg, cfg["dim"], seed, dtype)
    g = torch.Generator().manual_seed(seed + 7919)
    h, d, dim = cfg["n_heads"], cfg["head_dim"], cfg["dim"]
    if cfg["decay_mode"] == "per_channel":
        p["dt_proj.weight"] = (torch.randn(h * d, 2 * dim, generator=g, dtype=torch.float64)
                               * 0.3 * (2 * dim) ** -0.5).to(dtype)
        p["dt_proj.bias"] = (torch.randn(h * d, generator=g, dtype=torch.float64) * 0.1).to(dtype)
        p["dt_bias"] = (torch.randn(h, d, generator=g, dtype=torch.float64) * 0.5 - 2.0).to(dtype)
    if cfg["write_mode"] == "delta":
        # the delta write S <- S - beta (S k) k* is stable for beta |k|^2 < 2: keys of
        # squared norm ~0.5 at inputs of scale 0.5
        for name in ("qkv_proj.weight_real", "qkv_proj.weight_imag"):
            p[name] = p[name] * (0.7 * d ** -0.5)
        p["beta_proj.weight"] = (torch.randn(h, dim, generator=g, dtype=torch.float64) * dim ** -0.5).to(dtype)
        p["beta_proj.bias"] = torch.zeros(h, dtype=dtype)
    return p


class ComplexLinear(nn.Module):
    """ComplexLinear without bias (v11/complex_ops.py:146-172)."""

    def __init__(self, w_re, w_im):
        super().__init__()
        self.weight_real = nn.Parameter(w_re.clone())
        self.weight_imag = nn.Parameter(w_im.clone())
        self.bias_real = None
        self.bias_imag = None

    def forward(self, z):
        return L.complex_linear(z, self.weight_real, self.weight_imag)


def _linear(w, b):
    m = nn.Linear(w.shape[1], w.shape[0], dtype=w.dtype)
    m.weight = nn.Parameter(w.clone())
    m.bias = nn.Parameter(b.clone())
    return m


class V11PAMLayer(nn.Module):
    """V11PAMLayer restated; cfg: the keys of DEFAULTS (a subset of V11Config)."""

    def __init__(self, cfg=None, params=None, seed=0, dtype=torch.float64):
        super().__init__()
        c = config(**(cfg or {}))
        self.cfg = c
        p = params if params is not None else make_params(c, seed, dtype)
        h, d, m = c["n_heads"], c["head_dim"], c["n_states"]
        self.num_heads, self.head_dim, self.n_states = h, d, m
        self.inner_dim, self.dim = h * d, c["dim"]
        self.fused_qkv = True
        for key in ("use_rope", "use_gsp", "qk_norm", "decay_mode", "write_mode", "delta_chunk", "fused_e3",
                    "gamma_floor", "gate_content_aware", "routing_content_aware", "state_compete",
                    "route_balance_lambda", "chunk_size"):
            setattr(self, key, c[key])
        self.recompute_pam_chunks = False
        self.gate_surprisal_lambda = 0.0
        self.qkv_proj = ComplexLinear(p["qkv_proj.weight_real"], p["qkv_proj.weight_imag"])
        self.o_proj = ComplexLinear(p["o_proj.weight_real"], p["o_proj.weight_imag"])
        self.dt_proj = _linear(p["dt_proj.weight"], p["dt_proj.bias"])
        self.dt_bias = nn.Parameter(p["dt_bias"].clone())
        if self.use_gsp:
            self.protect_gate = _linear(p["protect_gate.weight"], p["protect_gate.bias"])
        if self.write_mode == "delta":
            self.beta_proj = _linear(p["beta_proj.weight"], p["beta_proj.bias"])
        if m > 1:
            self.state_dt_offset = nn.Parameter(p["state_dt_offset"].clone())
            self.phase_proj = _linear(p["phase_proj.weight"], p["phase_proj.bias"])
            if self.state_compete:
                self.score_proj = _linear(p["score_proj.weight"], p["score_proj.bias"])
        if self.use_rope:
            self.register_buffer("rope_cache", O.rope_table(c["max_seq_len"], d).to(dtype), persistent=False)
        self.dropout = nn.Dropout(0.0)
        causal = self.chunk_size if self.chunk_size > 0 else c["max_seq_len"]
        self.register_buffer("_causal", torch.tril(torch.ones(causal, causal, dtype=dtype)), persistent=False)
        self._route_aux = None
        self._gate_prob_bt = None

    # ---------------------------------------------------------- prologue helpers

    def _apply_gamma_floor(self, base_decay):
        if self.gamma_floor and self.gamma_floor > 0.0:
            return self.gamma_floor + (1.0 - self.gamma_floor) * base_decay
        return base_decay

    def _routing_input(self, x):
        return L.to_real_concat(x) if self.routing_content_aware else L.cabs(x)

    def _phase_and_alpha(self, x):
        b, t = x.shape[:2]
        h, m = self.num_heads, self.n_states
        r_in = self._routing_input(x)
        phase = self.phase_proj(r_in).view(b, t, h, m)
        if self.state_compete:
            weights = F.softmax(self.score_proj(r_in).view(b, t, h, m), dim=-1) * m
        else:
            weights = torch.ones(b, t, h, m, device=x.device, dtype=x.dtype)
        return phase, weights

    def _route_balance_loss(self, routing_weights):
        if self.route_balance_lambda <= 0 or not self.state_compete or not self.training:
            return None
        prob = (routing_weights / self.n_states).mean(dim=(0, 1))
        entropy = -(prob * (prob + 1e-8).log()).sum(dim=-1)
        return -self.route_balance_lambda * entropy.mean()

    def _project(self, x, step_offset):
        b, t = x.shape[:2]
        h, d = self.num_heads, self.head_dim
        qkv = self.qkv_proj(x).view(b, t, 3, h, d, 2)
        q, k, v = (qkv[:, :, i].transpose(1, 2).contiguous() for i in range(3))
        if self.use_rope:
            end = step_offset + t
            if end > self.rope_cache.shape[0]:
                self.register_buffer("rope_cache", O.rope_table(end * 2, d).to(self.rope_cache),
                                     persistent=False)
            r = self.rope_cache[step_offset:end].to(dtype=x.dtype)
            q, k = O.cmul(q, r), O.cmul(k, r)
        if self.qk_norm:
            q, k = L.cnormalize(q), L.cnormalize(k)
        return q, k, v

    def _gamma_and_vprime(self, x, values, state_offset=0.0):
        b, t = x.shape[:2]
        h, d = self.num_heads, self.head_dim
        x_flat = L.to_real_concat(x)
        if self.decay_mode == "per_channel":
            logits = self.dt_proj(x_flat).view(b, t, h, d)
            sp = F.softplus(logits + self.dt_bias + state_offset).permute(0, 2, 1, 3).contiguous()
        else:
            sp = F.softplus(self.dt_proj(x_flat) + self.dt_bias + state_offset).transpose(1, 2).contiguous()
        base = self._apply_gamma_floor(torch.exp(-sp))
        if not self.use_gsp:
            return base, values
        gate_in = L.to_real_concat(x) if self.gate_content_aware else L.cabs(x)
        p = torch.sigmoid(self.protect_gate(gate_in)).transpose(1, 2)        # [B,H,T]
        pe = p.unsqueeze(-1) if self.decay_mode == "per_channel" else p
        return base * (1 - pe) + pe, values * (1 - p)[..., None, None]

    def _gamma_all_and_vprime(self, x, values):
        x_flat = L.to_real_concat(x)
        offs = self.state_dt_offset.view(self.n_states, 1, 1, 1)
        sp = F.softplus(self.dt_proj(x_flat) + self.dt_bias + offs).permute(0, 1, 3, 2).contiguous()
        base = self._apply_gamma_floor(torch.exp(-sp))                        # [K,B,H,T]
        if not self.use_gsp:
            return base, values
        gate_in = L.to_real_concat(x) if self.gate_content_aware else L.cabs(x)
        p = torch.sigmoid(self.protect_gate(gate_in)).transpose(1, 2)
        return base * (1 - p) + p, values * (1 - p)[..., None, None]

    # ---------------------------------------------------------- scans

    @staticmethod
    def _dual_form_block(scaled_queries, keys, protected_values, decay_gamma, causal_mask):
        return O.dual_form_block(scaled_queries, keys, protected_values, decay_gamma)

    def _forward_chunked_head(self, queries, keys, protected_values, decay_gamma, head_dim):
        return O.chunked_head(queries, keys, protected_values, decay_gamma, head_dim, self.chunk_size)

    def _forward_chunked_perchannel(self, queries, keys, protected_values, decay_gamma, head_dim):
        return O.chunked_perchannel(queries, keys, protected_values, decay_gamma, head_dim, self.chunk_size)

    def _forward_delta(self, queries, keys, protected_values, decay_gamma, write_beta, head_dim):
        return OD.delta_chunked(queries, keys, protected_values, decay_gamma, write_beta, head_dim,
                                self.delta_chunk)

    def _forward_multistate(self, x, queries, keys, protected_values, head_dim):
        t = x.shape[1]
        phase, weights = self._phase_and_alpha(x)
        phase, weights = phase.permute(0, 2, 3, 1), weights.permute(0, 2, 3, 1)     # [B,H,K,T]
        self._route_aux = self._route_balance_loss(weights.permute(0, 3, 1, 2))
        total, states = None, []
        for s in range(self.n_states):
            g, pv = self._gamma_and_vprime(x, protected_values, state_offset=self.state_dt_offset[s])
            if self.decay_mode == "per_channel":
                y, st = self._forward_chunked_perchannel(queries, keys, pv, g, head_dim)
            elif self.chunk_size > 0 and t > self.chunk_size:
                y, st = self._forward_chunked_head(queries, keys, pv, g, head_dim)
            else:
                y, st = self._dual_form_block(queries * head_dim ** -0.5, keys, pv, g, self._causal[:t, :t])
            rot = torch.stack([weights[:, :, s] * torch.cos(phase[:, :, s]),
                               weights[:, :, s] * torch.sin(phase[:, :, s])], -1)
            y = O.cmul(y, rot.unsqueeze(-2))
            total = y if total is None else total + y
            states.append(st)
        return total, torch.stack(states, dim=0)

    def _fused_chunk_step(self, queries_chunk, keys_chunk, protected_values_chunk, decay_gamma_chunk,
                          retrieval_phase_chunk, routing_weights_chunk, memory_state, is_first_chunk):
        return O.fused_chunk_step(queries_chunk, keys_chunk, protected_values_chunk, decay_gamma_chunk,
                                  retrieval_phase_chunk, routing_weights_chunk, memory_state, is_first_chunk)

    def _forward_multistate_fused(self, x, queries, keys, values, head_dim):
        b, t = x.shape[:2]
        chunk = self.chunk_size if self.chunk_size > 0 else t
        phase, weights = self._phase_and_alpha(x)
        phase, weights = phase.permute(3, 0, 2, 1), weights.permute(3, 0, 2, 1)      # [K,B,H,T]
        self._route_aux = self._route_balance_loss(weights.permute(1, 3, 2, 0))
        gamma_all, pv = self._gamma_all_and_vprime(x, values)
        sq = queries * head_dim ** -0.5
        state = queries.new_zeros(self.n_states, b, self.num_heads, head_dim, head_dim, 2)
        outs = []
        for c0 in range(0, t, chunk):
            c1 = min(c0 + chunk, t)
            y, state = self._fused_chunk_step(sq[:, :, c0:c1], keys[:, :, c0:c1], pv[:, :, c0:c1],
                                              gamma_all[..., c0:c1], phase[..., c0:c1], weights[..., c0:c1],
                                              state, c0 == 0)
            outs.append(y)
        return torch.cat(outs, dim=2), state

    # ---------------------------------------------------------- forward

    def forward(self, x, state=None, step_offset=0):
        b, t = x.shape[:2]
        d = self.head_dim
        q, k, v = self._project(x, step_offset)
        if state is None and t > 1:
            if self.n_states > 1:
                if self.fused_e3 and self.decay_mode != "per_channel" and self.write_mode == "additive":
                    y, new_state = self._forward_multistate_fused(x, q, k, v, d)
                else:
                    y, new_state = self._forward_multistate(x, q, k, v, d)
            elif self.write_mode == "delta":
                g, pv = self._gamma_and_vprime(x, v)
                beta = torch.sigmoid(self.beta_proj(L.cabs(x))).transpose(1, 2)
                y, new_state = self._forward_delta(q, k, pv, g, beta, d)
            elif self.decay_mode == "per_channel":
                g, pv = self._gamma_and_vprime(x, v)
                y, new_state = self._forward_chunked_perchannel(q, k, pv, g, d)
            else:
                g, pv = self._gamma_and_vprime(x, v)
                if self.chunk_size > 0 and t > self.chunk_size:
                    y, new_state = self._forward_chunked_head(q, k, pv, g, d)
                else:
                    y, new_state = self._dual_form_block(q * d ** -0.5, k, pv, g, self._causal[:t, :t])
        else:
            y, new_state = self._recurrent(x, q, k, v, state, d)
        y = y.transpose(1, 2).contiguous().view(b, t, self.inner_dim, 2)
        return self.o_proj(y), new_state

    # ---------------------------------------------------------- decode

    def _recurrent(self, x, queries, keys, values, state, head_dim):
        b, t = x.shape[:2]
        h, m = self.num_heads, self.n_states
        scale = head_dim ** -0.5
        beta = None
        if self.write_mode == "delta":
            beta = torch.sigmoid(self.beta_proj(L.cabs(x))).transpose(1, 2)
        if m > 1:
            phase, weights = self._phase_and_alpha(x)
            phase, weights = phase.permute(0, 2, 3, 1), weights.permute(0, 2, 3, 1)  # [B,H,K,T]
            self._route_aux = self._route_balance_loss(weights.permute(0, 3, 1, 2))
        if state is None:
            shape = (m, b, h, head_dim, head_dim, 2) if m > 1 else (b, h, head_dim, head_dim, 2)
            state = torch.zeros(shape, device=x.device, dtype=x.dtype)
        outs = []
        for ti in range(t):
            tok = x[:, ti:ti + 1]
            k_t, q_t, v_t = keys[:, :, ti], queries[:, :, ti] * scale, values[:, :, ti]
            if m > 1:
                acc, new_states = None, []
                for s in range(m):
                    g, pv = self._gamma_and_vprime(tok, values[:, :, ti:ti + 1], state_offset=self.state_dt_offset[s])
                    y, st = self._recur_step_additive(state[s], g[:, :, 0], pv[:, :, 0], k_t, q_t)
                    rot = torch.stack([weights[:, :, s, ti] * torch.cos(phase[:, :, s, ti]),
                                       weights[:, :, s, ti] * torch.sin(phase[:, :, s, ti])], -1)
                    y = O.cmul(y, rot.unsqueeze(-2))
                    acc = y if acc is None else acc + y
                    new_states.append(st)
                outs.append(acc)
                state = torch.stack(new_states, dim=0)
                continue
            g, pv = self._gamma_and_vprime(tok, values[:, :, ti:ti + 1])
            if self.write_mode == "delta":
                y, state = self._recur_step_delta(state, g[:, :, 0], pv[:, :, 0], k_t, q_t, beta[:, :, ti])
            else:
                y, state = self._recur_step_additive(state, g[:, :, 0], pv[:, :, 0], k_t, q_t)
            outs.append(y)
        return torch.stack(outs, dim=2), state

    def _recur_step_additive(self, memory_state, decay_gamma, value_t, key_t, query_t):
        return O.recur_step_additive(memory_state, decay_gamma, value_t, key_t, query_t)

    def _recur_step_delta(self, memory_state, decay_gamma, value_t, key_t, query_t, write_beta_t):
        return OD.recur_step_delta(memory_state, decay_gamma, value_t, key_t, query_t, write_beta_t)
