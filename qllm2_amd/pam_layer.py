"""HIP implementations of the V11PAMLayer hot-path methods, with the
reference's signatures and return tuples, and install() to bind them.

Reference methods replaced (v11/model.py):
  _dual_form_block          354-376  (static; T <= C prefill and chunk body)
  _forward_chunked_head     378-417  (single-state chunked prefill)
  _fused_chunk_step         657-737  (one E3 chunk with carried state)
  _forward_multistate_fused 739-781  (E3 prefill: all chunks in one scan)
  _recur_step_additive      927-965  (one decode step)
  _recurrent                845-925  (decode token loop; all K states of a
                                      token in one kernel launch)

Every replacement keeps the layer's own projections/gates (_phase_and_alpha,
_gamma_all_and_vprime, _gamma_and_vprime) and replaces only the PAM math.
Modes outside the hot path (E1 per-channel decay, E2 delta write) keep the
reference methods: install() leaves them reachable as the saved originals.
"""

import sys

import torch

from . import decode as _decode
from . import fused_ce as _fused_ce
from . import flash_pam as _flash_pam
from . import triton_kernels as _tk
from .pam_scan import pam_scan_interleaved


def _cat_rot(phase, routing):
    """(re, im) planes of r = routing * e^{i phase} (autograd flows to both)."""
    return routing * torch.cos(phase), routing * torch.sin(phase)


def dual_form_block(scaled_queries, keys, protected_values, decay_gamma, causal_mask=None):
    """V11PAMLayer._dual_form_block: one block with zero incoming state; queries
    already scaled.  Returns (output [B,H,C,d,2], chunk state [B,H,d,d,2])."""
    d = scaled_queries.shape[-2]
    y, s = pam_scan_interleaved(scaled_queries, keys, protected_values, decay_gamma.unsqueeze(0), d,
                                scaled_queries.shape[2], scale_queries=False)
    return y, s[0]


def forward_chunked_head(self, queries, keys, protected_values, decay_gamma, head_dim):
    """V11PAMLayer._forward_chunked_head (queries unscaled)."""
    y, s = pam_scan_interleaved(queries, keys, protected_values, decay_gamma.unsqueeze(0), head_dim,
                                self.chunk_size)
    return y, s[0]


def fused_chunk_step(self, queries_chunk, keys_chunk, protected_values_chunk, decay_gamma_chunk,
                     retrieval_phase_chunk, routing_weights_chunk, memory_state, is_first_chunk):
    """V11PAMLayer._fused_chunk_step: queries scaled; decay/phase/routing
    [K,B,H,C]; memory_state [K,B,H,d,d,2] (ignored when is_first_chunk)."""
    d = queries_chunk.shape[-2]
    rot = _cat_rot(retrieval_phase_chunk, routing_weights_chunk)
    s0 = None if is_first_chunk else memory_state
    y, s = pam_scan_interleaved(queries_chunk, keys_chunk, protected_values_chunk, decay_gamma_chunk, d,
                                queries_chunk.shape[2], rot=rot, s0=s0, scale_queries=False)
    if is_first_chunk and memory_state is not None:
        # the reference skips the carried read on the first chunk but still
        # decays the (zero-initialised) incoming state into the new one
        total = torch.exp(torch.log(decay_gamma_chunk.float() + 1e-6).sum(-1))
        s = s + (total[..., None, None, None] * memory_state.float()).to(s.dtype)
    return y, s


def forward_multistate_fused(self, x, queries, keys, values, head_dim):
    """V11PAMLayer._forward_multistate_fused: the layer's own prologue, then
    one E3 scan over every chunk.  Returns (output, state [K,B,H,d,d,2])."""
    retrieval_phase, routing_weights = self._phase_and_alpha(x)
    retrieval_phase = retrieval_phase.permute(3, 0, 2, 1)
    routing_weights = routing_weights.permute(3, 0, 2, 1)
    self._route_aux = self._route_balance_loss(routing_weights.permute(1, 3, 2, 0))
    decay_gamma_all, protected_values = self._gamma_all_and_vprime(x, values)
    chunk = self.chunk_size if self.chunk_size > 0 else x.shape[1]
    return pam_scan_interleaved(queries, keys, protected_values, decay_gamma_all, head_dim, chunk,
                                rot=_cat_rot(retrieval_phase, routing_weights))


def recur_step_additive(self, memory_state, decay_gamma, value_t, key_t, query_t):
    """V11PAMLayer._recur_step_additive (head-scalar decay)."""
    return _decode.recur_step_additive(memory_state, decay_gamma, value_t, key_t, query_t)


def recurrent(self, x, queries, keys, values, state, head_dim):
    """V11PAMLayer._recurrent for the additive head-decay write: per token one
    qpam_decode_step launch updates all K states and sums the rotated reads."""
    if self.write_mode != 'additive' or self.decay_mode == 'per_channel' or torch.is_grad_enabled():
        return _ORIGINALS['_recurrent'](self, x, queries, keys, values, state, head_dim)
    b, t = x.shape[0], x.shape[1]
    h, k_states, d = self.num_heads, self.n_states, head_dim
    scale = head_dim ** -0.5
    if k_states > 1:
        phase, routing = self._phase_and_alpha(x)            # [B,T,H,K]
        self._route_aux = self._route_balance_loss(routing)
        rot = torch.stack([routing * torch.cos(phase), routing * torch.sin(phase)], -1)  # [B,T,H,K,2]
    if state is None:
        shape = (k_states, b, h, d, d, 2) if k_states > 1 else (b, h, d, d, 2)
        state = torch.zeros(shape, device=x.device, dtype=x.dtype)
    # pool layout [slot=b, group=h, state=k, d, d, 2]
    pool = (state if k_states > 1 else state.unsqueeze(0)).permute(1, 2, 0, 3, 4, 5).to(torch.float32).contiguous()
    ys = []
    for ti in range(t):
        tok = x[:, ti:ti + 1]
        gam = []
        v_t = None
        for kk in range(k_states):
            off = self.state_dt_offset[kk] if k_states > 1 else 0.0
            g_k, pv = self._gamma_and_vprime(tok, values[:, :, ti:ti + 1], state_offset=off)
            gam.append(g_k[:, :, 0])
            v_t = pv[:, :, 0]
        gamma = torch.stack(gam, -1).float().contiguous()                     # [B,H,K]
        r = rot[:, ti].float().contiguous() if k_states > 1 else None         # [B,H,K,2]
        y = _decode.decode_step(pool, queries[:, :, ti].float().contiguous(), keys[:, :, ti].float().contiguous(),
                                v_t.float().contiguous(), gamma, rot=r, q_scale=scale)
        ys.append(y.to(x.dtype))
    out = torch.stack(ys, dim=2)
    new_state = pool.permute(2, 0, 1, 3, 4, 5).to(x.dtype)
    return out, (new_state if k_states > 1 else new_state[0])


_ORIGINALS = {}

_METHODS = {
    "_forward_chunked_head": forward_chunked_head,
    "_fused_chunk_step": fused_chunk_step,
    "_forward_multistate_fused": forward_multistate_fused,
    "_recur_step_additive": recur_step_additive,
    "_recurrent": recurrent,
}


def install(model_module=None):
    """Bind the HIP implementations into the reference's v11 package.

    model_module: the imported v11.model module (default: sys.modules['v11.model']).
    Rebinds the V11PAMLayer methods above (and the static _dual_form_block),
    replaces the module-level fused_decay_matrix name v11/model.py:40 bound at
    import, and aliases v11.flash_pam / v11.triton_kernels / v11.fused_ce to this
    package's modules so later imports (v11/model.py:1182, v7/train.py:301,350)
    resolve here.  Returns the dict of replaced originals."""
    mod = model_module if model_module is not None else sys.modules["v11.model"]
    layer = mod.V11PAMLayer
    for name, fn in _METHODS.items():
        if name not in _ORIGINALS and hasattr(layer, name):
            _ORIGINALS[name] = getattr(layer, name)
        setattr(layer, name, fn)
    if "_dual_form_block" not in _ORIGINALS and hasattr(layer, "_dual_form_block"):
        _ORIGINALS["_dual_form_block"] = layer.__dict__.get("_dual_form_block", layer._dual_form_block)
    layer._dual_form_block = staticmethod(dual_form_block)
    if hasattr(mod, "fused_decay_matrix"):
        mod.fused_decay_matrix = _tk.fused_decay_matrix
    pkg = mod.__name__.rsplit(".", 1)[0] if "." in mod.__name__ else "v11"
    for sub, m in (("flash_pam", _flash_pam), ("triton_kernels", _tk), ("fused_ce", _fused_ce)):
        sys.modules[f"{pkg}.{sub}"] = m
        parent = sys.modules.get(pkg)
        if parent is not None:
            setattr(parent, sub, m)
    # v11.complex_ops bound the four elementwise ops from v11.triton_kernels at its
    # own import (v11/complex_ops.py:19-24); its layers look them up at call time
    cops = sys.modules.get(f"{pkg}.complex_ops")
    if cops is not None:
        for name in _COMPLEX_OPS:
            if hasattr(cops, name):
                _ORIGINALS.setdefault(f"complex_ops.{name}", getattr(cops, name))
                setattr(cops, name, getattr(_tk, name))
    return dict(_ORIGINALS)


_COMPLEX_OPS = ("fused_complex_norm", "fused_mod_swish", "fused_mod_relu", "fused_cgu_gate")
