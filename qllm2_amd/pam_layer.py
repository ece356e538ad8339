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
  _forward_chunked_perchannel 421-489 (E1 per-channel decay: the fold and the
                                      state scan as HIP kernels, the chunk
                                      products as batched complex GEMMs)
  _forward_delta            491-576  (E2 delta write; HIP token recurrence
                                      instead of the per-chunk solve)
  _recur_step_delta         967-1002 (one E2 decode token)

  forward                   785-843  prefill of the production modes (head
                                      decay, additive write, E3 fused or one
                                      state, head_dim 16/32/64/128): projections as
                                      planar GEMMs, one prologue kernel, the
                                      scan writing Y head-merged, o_proj on the
                                      planar Y; other calls go to the original

The method replacements keep the layer's own projections/gates
(_phase_and_alpha, _gamma_all_and_vprime, _gamma_and_vprime) and replace only
the PAM math; the forward replacement fuses those elementwise steps into the
prologue kernel (qpam_prologue_fwd).

install() keeps the class's own methods as `_qpam_originals` on that class,
and every replacement hands a call to the saved method when the kernels do
not cover it, so the installed layer computes what the reference computes in
every mode:
  * CPU tensors (the reference computes on CPU through its torch code);
  * the E2 delta write with head dims above 64 (its key dim is one 64-wide
    tile; smaller head dims are zero-padded).
The HIP library itself has no CPU path: the replacements raise for GPU
tensors if it cannot load.
"""

import importlib
import sys

import torch
import torch.nn.functional as F

from . import _lib
from . import _reference
from . import cproj as _cproj
from . import decode as _decode
from . import pam_delta as _delta
from . import fused_ce as _fused_ce
from . import flash_pam as _flash_pam
from . import triton_kernels as _tk
from .pam_perchannel import perchannel_chunked
from .pam_prologue import HEAD_DIMS as _PROLOGUE_DIMS, cabs, pam_prologue, proj_columns
from .pam_scan import chunk_for, pam_scan_interleaved, pam_scan_planar


def _cat_rot(phase, routing):
    """(re, im) planes of r = routing * e^{i phase} (autograd flows to both)."""
    return routing * torch.cos(phase), routing * torch.sin(phase)


def _originals(owner):
    """The methods install() saved from `owner`'s class (or the class itself)."""
    cls = owner if isinstance(owner, type) else type(owner)
    table = getattr(cls, "_qpam_originals", None)
    if table is None:
        raise RuntimeError(f"qpam: {cls.__name__} was not set up by qllm2_amd.pam_layer.install(), so a call "
                           "the HIP kernels do not cover has no reference method to run")
    return table


def _original(self, name):
    return _originals(self)[name]


def _scan_covers(t, head_dim, n_states=1):
    """True when the HIP scan takes this call: a GPU tensor (every head dim and
    state count: head dims below 64 are zero-padded, larger ones run as 64 x 64
    state blocks, states beyond 4 in groups)."""
    return t.is_cuda and head_dim >= 1 and n_states >= 1


def dual_form_block(scaled_queries, keys, protected_values, decay_gamma, causal_mask=None):
    """V11PAMLayer._dual_form_block: one block with zero incoming state; queries
    already scaled.  Returns (output [B,H,C,d,2], chunk state [B,H,d,d,2])."""
    d = scaled_queries.shape[-2]
    y, s = pam_scan_interleaved(scaled_queries, keys, protected_values, decay_gamma.unsqueeze(0), d,
                                scaled_queries.shape[2], scale_queries=False)
    return y, s[0]


def _dual_form_block_for(original):
    """The static _dual_form_block install() binds: the HIP block, or the saved
    reference block for calls the scan does not take."""
    def _dual_form_block(scaled_queries, keys, protected_values, decay_gamma, causal_mask=None):
        if not _scan_covers(scaled_queries, scaled_queries.shape[-2]) and original is not None:
            return original(scaled_queries, keys, protected_values, decay_gamma, causal_mask)
        return dual_form_block(scaled_queries, keys, protected_values, decay_gamma, causal_mask)
    _dual_form_block.__doc__ = dual_form_block.__doc__
    _dual_form_block.__wrapped__ = dual_form_block
    return _dual_form_block


def forward_chunked_head(self, queries, keys, protected_values, decay_gamma, head_dim):
    """V11PAMLayer._forward_chunked_head (queries unscaled)."""
    if not _scan_covers(queries, head_dim):
        return _original(self, "_forward_chunked_head")(self, queries, keys, protected_values, decay_gamma,
                                                        head_dim)
    y, s = pam_scan_interleaved(queries, keys, protected_values, decay_gamma.unsqueeze(0), head_dim,
                                self.chunk_size)
    return y, s[0]


def fused_chunk_step(self, queries_chunk, keys_chunk, protected_values_chunk, decay_gamma_chunk,
                     retrieval_phase_chunk, routing_weights_chunk, memory_state, is_first_chunk):
    """V11PAMLayer._fused_chunk_step: queries scaled; decay/phase/routing
    [K,B,H,C]; memory_state [K,B,H,d,d,2] (ignored when is_first_chunk)."""
    d = queries_chunk.shape[-2]
    if not _scan_covers(queries_chunk, d, decay_gamma_chunk.shape[0]):
        return _original(self, "_fused_chunk_step")(
            self, queries_chunk, keys_chunk, protected_values_chunk, decay_gamma_chunk, retrieval_phase_chunk,
            routing_weights_chunk, memory_state, is_first_chunk)
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
    if not _scan_covers(queries, head_dim, self.n_states):
        return _original(self, "_forward_multistate_fused")(self, x, queries, keys, values, head_dim)
    retrieval_phase, routing_weights = self._phase_and_alpha(x)
    retrieval_phase = retrieval_phase.permute(3, 0, 2, 1)
    routing_weights = routing_weights.permute(3, 0, 2, 1)
    self._route_aux = self._route_balance_loss(routing_weights.permute(1, 3, 2, 0))
    decay_gamma_all, protected_values = self._gamma_all_and_vprime(x, values)
    chunk = self.chunk_size if self.chunk_size > 0 else x.shape[1]
    return pam_scan_interleaved(queries, keys, protected_values, decay_gamma_all, head_dim, chunk,
                                rot=_cat_rot(retrieval_phase, routing_weights))


def forward_delta(self, queries, keys, protected_values, decay_gamma, write_beta, head_dim):
    """V11PAMLayer._forward_delta (E2 delta write, head-scalar decay): the HIP
    delta-rule kernels (head dims up to 64) over the layer's chunks of
    delta_chunk steps (v11/model.py:494); per-channel decay, larger head dims
    or chunks above 64 steps keep the original."""
    chunk = int(getattr(self, "delta_chunk", 64))
    if decay_gamma.dim() != 3 or head_dim > 64 or not queries.is_cuda or not 1 <= chunk <= 64:
        return _original(self, "_forward_delta")(self, queries, keys, protected_values, decay_gamma, write_beta,
                                                 head_dim)
    return _delta.forward_delta(queries, keys, protected_values, decay_gamma, write_beta, head_dim, chunk=chunk)


def recur_step_delta(self, memory_state, decay_gamma, value_t, key_t, query_t, write_beta_t):
    """V11PAMLayer._recur_step_delta (one decode token of the E2 write; the HIP
    step is differentiable)."""
    if decay_gamma.dim() != 2 or memory_state.shape[-2] > 64 or not memory_state.is_cuda:
        return _original(self, "_recur_step_delta")(self, memory_state, decay_gamma, value_t, key_t, query_t,
                                                    write_beta_t)
    return _delta.recur_step_delta(memory_state, decay_gamma, value_t, key_t, query_t, write_beta_t)


_DECODE_MAX = _decode.KERNEL_DIMS[-1]  # head dims up to this decode on the kernels (others padded)


def forward_chunked_perchannel(self, queries, keys, protected_values, decay_gamma, head_dim):
    """V11PAMLayer._forward_chunked_perchannel (E1, v11/model.py:421-489) on
    the GPU (qllm2_amd/pam_perchannel.py), differentiable; CPU tensors and
    chunk sizes outside 1..64 run the saved reference method."""
    if not queries.is_cuda or not 1 <= int(self.chunk_size) <= 64:
        return _original(self, "_forward_chunked_perchannel")(self, queries, keys, protected_values, decay_gamma,
                                                              head_dim)
    return perchannel_chunked(queries, keys, protected_values, decay_gamma, head_dim, self.chunk_size)


def recur_step_additive(self, memory_state, decay_gamma, value_t, key_t, query_t):
    """V11PAMLayer._recur_step_additive: the HIP decode step for head or
    per-channel decay (decay_gamma [...] or [..., d]), differentiable (the
    backward is a HIP kernel as well; head dims other than 16/32/64/128 run
    zero-padded to the next of them); CPU tensors and head dims above 128 run
    the saved reference step (v11/model.py:927-965)."""
    if (not memory_state.is_cuda or decay_gamma.dim() not in (memory_state.dim() - 3, memory_state.dim() - 2)
            or memory_state.shape[-2] > _DECODE_MAX):
        return _original(self, "_recur_step_additive")(self, memory_state, decay_gamma, value_t, key_t, query_t)
    return _decode.recur_step_additive(memory_state, decay_gamma, value_t, key_t, query_t)


def recurrent(self, x, queries, keys, values, state, head_dim):
    """V11PAMLayer._recurrent for the additive write (head or per-channel
    decay): per token one qpam_decode_step launch updates all K states and sums
    the rotated reads (head dims other than 16/32/64/128 on the next of them,
    the state pool and each token's q, k, v zero-padded).  The E2 mode, grad
    mode, CPU tensors and head dims above 128 run the saved reference loop
    (which then calls the replaced steps where they apply)."""
    if (self.write_mode != 'additive' or torch.is_grad_enabled()
            or not x.is_cuda or head_dim > _DECODE_MAX):
        return _original(self, "_recurrent")(self, x, queries, keys, values, state, head_dim)
    b, t = x.shape[0], x.shape[1]
    h, k_states, d = self.num_heads, self.n_states, head_dim
    kd = _decode.kernel_dim(d)
    pad = (lambda z: F.pad(z, (0, 0, 0, kd - d))) if kd != d else (lambda z: z)  # [..., d, 2] -> [..., kd, 2]
    scale = head_dim ** -0.5
    if k_states > 1:
        phase, routing = self._phase_and_alpha(x)            # [B,T,H,K]
        self._route_aux = self._route_balance_loss(routing)
        rot = torch.stack([routing * torch.cos(phase), routing * torch.sin(phase)], -1)  # [B,T,H,K,2]
    if state is None:
        shape = (k_states, b, h, d, d, 2) if k_states > 1 else (b, h, d, d, 2)
        state = torch.zeros(shape, device=x.device, dtype=x.dtype)
    # pool layout [slot=b, group=h, state=k, d, d, 2] (zero-padded to the kernel's head dim)
    pool = (state if k_states > 1 else state.unsqueeze(0)).permute(1, 2, 0, 3, 4, 5).to(torch.float32)
    pool = (F.pad(pool, (0, 0, 0, kd - d, 0, kd - d)) if kd != d else pool).contiguous()
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
        gamma = torch.stack(gam, 2).float()                                   # [B,H,K] or [B,H,K,d]
        if kd != d and gamma.dim() == 4:
            gamma = F.pad(gamma, (0, kd - d), value=1.0)  # padded key columns: any finite decay
        r = rot[:, ti].float().contiguous() if k_states > 1 else None         # [B,H,K,2]
        y = _decode.decode_step(pool, pad(queries[:, :, ti].float()).contiguous(),
                                pad(keys[:, :, ti].float()).contiguous(), pad(v_t.float()).contiguous(),
                                gamma.contiguous(), rot=r, q_scale=scale)
        ys.append(y[..., :d, :].to(x.dtype))
    out = torch.stack(ys, dim=2)
    new_state = pool[..., :d, :d, :].permute(2, 0, 1, 3, 4, 5).to(x.dtype)
    return out, (new_state if k_states > 1 else new_state[0])


def _in_weight(self, h, d, cols):
    """Weight [cols, 2 dim] and bias [cols] (None when the QKV projection
    has none) of the one GEMM that maps the interleaved input x.view(N, 2 dim)
    (re, im per feature) to `proj`: the real planes of q, k, v
    (ComplexLinear: re = Wr xr - Wi xi, v11/complex_ops.py:165-172), their
    imaginary planes (im = Wi xr + Wr xi), dt_proj's logits without its bias
    (v11/model.py:636, its [xr | xi] columns reordered to the interleaved
    input), zero padding."""
    if self.fused_qkv:
        mods = [self.qkv_proj]
    else:
        mods = [self.q_proj, self.k_proj, self.v_proj]
    wr = torch.cat([m.weight_real for m in mods], 0) if len(mods) > 1 else mods[0].weight_real
    wi = torch.cat([m.weight_imag for m in mods], 0) if len(mods) > 1 else mods[0].weight_imag
    rows, dim = wr.shape
    w_dt = self.dt_proj.weight.view(h, 2, dim).transpose(1, 2).reshape(h, 2 * dim)
    pad = cols - 2 * rows - h
    parts = [torch.stack([wr, -wi], -1).view(rows, 2 * dim), torch.stack([wi, wr], -1).view(rows, 2 * dim), w_dt]
    if pad:
        parts.append(w_dt.new_zeros(pad, 2 * dim))
    w = torch.cat(parts, 0)
    if all(getattr(m, "bias_real", None) is None for m in mods):
        return w, None      # dt_proj's bias joins dt_bias in the prologue instead
    br = torch.cat([m.bias_real if m.bias_real is not None else wr.new_zeros(m.weight_real.shape[0]) for m in mods])
    bi = torch.cat([m.bias_imag if m.bias_imag is not None else wr.new_zeros(m.weight_real.shape[0]) for m in mods])
    return w, torch.cat([br, bi, wr.new_zeros(h + pad)])


_ONES = {}


def _ones(x):
    """A [1,1,1,1] tensor of ones in x's device and dtype, made once."""
    key = (x.device, x.dtype)
    t = _ONES.get(key)
    if t is None:
        t = _ONES[key] = torch.ones(1, 1, 1, 1, device=x.device, dtype=x.dtype)
    return t


def _packed_in(self, x2, h, cols, with_mag):
    """proj [B,T,cols] from the packed input projection (qkv_proj, or q/k/v_proj,
    and dt_proj's logits without its bias in one GEMM, the weight packed and its
    gradient split on the HIP library), with_mag: (proj, cabs(x)), or None where
    that path does not apply (projection biases, mixed dtypes, autocast)."""
    mods = [self.qkv_proj] if self.fused_qkv else [self.q_proj, self.k_proj, self.v_proj]
    if any(getattr(m, "bias_real", None) is not None or getattr(m, "bias_imag", None) is not None for m in mods):
        return None
    wr = torch.cat([m.weight_real for m in mods], 0) if len(mods) > 1 else mods[0].weight_real
    wi = torch.cat([m.weight_imag for m in mods], 0) if len(mods) > 1 else mods[0].weight_imag
    tail = self.dt_proj.weight
    if tail.shape != (h, x2.shape[-1]) or not _cproj.supported(x2, wr, wi, tail, layout=_lib.QPAM_CW_IN):
        return None
    return _cproj.linear_in(x2, wr, wi, tail, cols, with_mag)


def _out_weight(mod):
    """Weight [2 dim, 2 inner] (and bias) of the o_proj GEMM from the
    per-token [y_re | y_im] planes to the interleaved output (re_o, im_o)."""
    wr, wi = mod.weight_real, mod.weight_imag
    dim = wr.shape[0]
    w = torch.stack([torch.cat([wr, -wi], 1), torch.cat([wi, wr], 1)], 1).view(2 * dim, -1)
    bias = None
    if getattr(mod, "bias_real", None) is not None:
        bias = torch.stack([mod.bias_real, mod.bias_imag], 1).view(2 * dim)
    return w, bias


def _fused_prefill(self, x, state):
    return (state is None and x.dim() == 4 and x.shape[1] > 1 and x.is_cuda
            and getattr(self, "decay_mode", "head") != "per_channel" and self.write_mode == "additive"
            and self.head_dim in _PROLOGUE_DIMS and 1 <= self.n_states <= 4
            and (self.n_states == 1 or getattr(self, "fused_e3", True)))


class _TallKLinear(torch.autograd.Function):
    """F.linear whose weight gradient g^T x contracts over all N = B T rows in
    row slices: one batched product [S, in, N/S] x [S, N/S, out] and a sum of
    the S partial products (in fp32 for 16-bit weights).  A weight gradient with a small output (the
    gate logits: out = H or H + H K) or a square one (o_proj) gives the library
    GEMM a few hundred output tiles at most for a K of N; the slices give it
    S times as many."""

    @staticmethod
    def forward(ctx, x, w, b, splits):
        ctx.save_for_backward(x, w)
        ctx.splits, ctx.has_bias = splits, b is not None
        return F.linear(x, w, b)

    @staticmethod
    def backward(ctx, gy):
        x, w = ctx.saved_tensors
        gx = gw = gb = None
        g2 = gy.reshape(-1, w.shape[0])
        acc = torch.float32 if w.dtype in (torch.float16, torch.bfloat16) else w.dtype
        if ctx.needs_input_grad[0]:
            gx = (g2 @ w).view(x.shape)
        if ctx.needs_input_grad[1]:
            x2, n, s = x.reshape(-1, w.shape[1]), g2.shape[0], ctx.splits
            # g^T x as (x^T g)^T: the right operand of the batched product stays a
            # contiguous slice (no copy of either operand)
            gwt = torch.bmm(x2.view(s, n // s, -1).transpose(1, 2), g2.view(s, n // s, -1))
            gw = gwt.sum(0, dtype=acc).t().contiguous().to(w.dtype)
        if ctx.has_bias and ctx.needs_input_grad[2]:
            gb = g2.sum(0, dtype=acc).to(w.dtype)
        return gx, gw, gb, None


def _linear_tall_k(x, w, b):
    """F.linear for N = x.numel() / in rows with the sliced weight gradient when
    the library GEMM would see few output tiles (fewer than 512 of 128 x 128) and
    N splits into slices of at least 512 rows; plain F.linear otherwise (and
    under autocast or mixed dtypes)."""
    n = x.numel() // w.shape[1]
    tiles = -(-w.shape[0] // 128) * -(-w.shape[1] // 128)
    s = 1
    while s * tiles < 512 and n % (2 * s) == 0 and n // (2 * s) >= 512:
        s *= 2
    if s == 1 or torch.is_autocast_enabled() or x.dtype != w.dtype or not torch.is_grad_enabled():
        return F.linear(x, w, b)
    return _TallKLinear.apply(x if x.is_contiguous() else x.contiguous(), w, b, s)


def forward(self, x, state=None, step_offset: int = 0):
    """V11PAMLayer.forward (v11/model.py:785-843) for a prefill of the
    production modes; everything else runs the original forward.

    x [B,T,dim,2] -> (out [B,T,dim,2], state [K,B,H,d,d,2] or [B,H,d,d,2]).
    Three GEMMs and two HIP launches instead of the reference's chain of
    elementwise passes: (1) one GEMM from x viewed as [N, 2 dim] (no copy) to
    the q, k, v planes and the decay logits; (2) one GEMM from |x| to the
    protect-gate and phase logits; qpam_prologue_fwd turns those and the RoPE
    table into the scan's operands; the scan writes Y as [B,T,2,H,d]; (3) one
    GEMM from Y viewed as [N, 2 H d] straight to the interleaved output."""
    if not _fused_prefill(self, x, state):
        return _original(self, "forward")(self, x, state, step_offset)
    b, t, dim = x.shape[0], x.shape[1], x.shape[2]
    h, d, m = self.num_heads, self.head_dim, self.n_states
    n = b * t
    xc = x if x.is_contiguous() else x.contiguous()
    cols = proj_columns(h, d)
    need_mag = (self.use_gsp and not self.gate_content_aware) or (m > 1 and not (self.routing_content_aware
                                                                               or self.state_compete))
    packed = _packed_in(self, xc.view(b, t, 2 * dim), h, cols, need_mag)
    mag = None
    if packed is not None:
        proj, mag = packed if need_mag else (packed, None)               # mag [B,T,dim] = cabs(x)
    else:
        w_in, b_in = _in_weight(self, h, d, cols)
        proj = F.linear(xc.view(b, t, 2 * dim), w_in, b_in)             # [B,T,cols]
    if proj.dtype not in (torch.float32, torch.bfloat16):
        proj = proj.float()
    rope = None
    if self.use_rope:
        end = step_offset + t
        if end > self.rope_cache.shape[0]:  # grown as the reference does (v11/model.py:291-297)
            self.register_buffer("rope_cache", _decode.build_rope_cache(end * 2, d, device=x.device),
                                 persistent=False)
        rope = self.rope_cache.float()
    if need_mag and mag is None:
        mag = cabs(xc)                                                   # [B,T,dim]
    protect = phase = routing = offsets = None
    g_w, g_b, g_parts = [], [], []
    if self.use_gsp:
        if self.gate_content_aware:
            protect = self.protect_gate(torch.cat([xc[..., 0], xc[..., 1]], -1))
        else:
            g_w.append(self.protect_gate.weight), g_b.append(self.protect_gate.bias), g_parts.append("protect")
    if m > 1:
        offsets = self.state_dt_offset
        if self.routing_content_aware or self.state_compete:
            phase, routing_w = self._phase_and_alpha(x)                  # [B,T,H,K]
            self._route_aux = self._route_balance_loss(routing_w)
            routing = routing_w if self.state_compete else None
        else:
            g_w.append(self.phase_proj.weight), g_b.append(self.phase_proj.bias), g_parts.append("phase")
            self._route_aux = self._route_balance_loss(_ones(x).expand(b, t, h, m))
    gate_kw = {}
    if g_parts:
        if _cproj.gate_supported(mag, g_w, g_b):
            gl = _cproj.gate_linear(mag, g_w, g_b)                       # [B,T,H (+H K)]
        else:
            gl = _linear_tall_k(mag, torch.cat(g_w, 0), torch.cat(g_b, 0))
        col, cols_of = 0, {}
        for part in g_parts:
            cols_of[part] = col
            if part == "protect":
                protect, col = gl[..., col:col + h], col + h
            else:
                phase, col = gl[..., col:col + h * m].view(b, t, h, m), col + h * m
        if routing is None and (protect is None or "protect" in cols_of) and (phase is None or "phase" in cols_of):
            # the prologue reads the logits as columns of gl and returns gl's gradient whole
            gate_kw = dict(gate=gl, protect_col=cols_of.get("protect", -1), phase_col=cols_of.get("phase", -1))
    if protect is not None and self.gate_surprisal_lambda > 0 and self.training:
        self._gate_prob_bt = torch.sigmoid(protect.float()).mean(dim=2)  # [B,T]
    (qr, qi), (kr, ki), (vr, vi), gamma, rot = pam_prologue(
        proj, self.dt_bias, dt_bias2=self.dt_proj.bias, n_heads=h, n_states=m, state_offset=offsets,
        protect=None if gate_kw else protect, phase=None if gate_kw else phase, routing=routing, rope=rope,
        rope_offset=step_offset, qk_norm=self.qk_norm, gamma_floor=self.gamma_floor or 0.0, head_dim=d, **gate_kw)
    o_dtype = self.o_proj.weight_real.dtype
    ck = chunk_for(self.chunk_size, t)
    # bf16 o_proj: the scan writes Y in bf16 itself (and reads its gradient in bf16)
    y_bf16 = (qr.dtype == torch.bfloat16 and ck == 64 and o_dtype == torch.bfloat16
              and not torch.is_autocast_enabled())
    y, _, s_re, s_im = pam_scan_planar(qr, qi, kr, ki, vr, vi, gamma, q_scale=d ** -0.5, chunk=ck, rot=rot,
                                       y_layout="bt2hd_bf16" if y_bf16 else "bt2hd")
    y = y.view(b, t, 2 * h * d)
    if o_dtype != torch.float32 and not torch.is_autocast_enabled():
        y = y.to(o_dtype)
    wr_o, wi_o = self.o_proj.weight_real, self.o_proj.weight_imag
    if getattr(self.o_proj, "bias_real", None) is None and _cproj.supported(y, wr_o, wi_o, layout=_lib.QPAM_CW_OUT):
        out = _cproj.linear_out(y, wr_o, wi_o).view(b, t, dim, 2)
    else:
        w_out, b_out = _out_weight(self.o_proj)
        out = _linear_tall_k(y, w_out, b_out).view(b, t, dim, 2)
    if self.training:
        # one keep-mask per complex value (as_complex_dropout_mask, v11/complex_ops.py:59-66)
        mask = self.dropout(torch.ones(out.shape[:-1], device=out.device, dtype=out.dtype))
        out = out * mask.unsqueeze(-1)
    new_state = torch.view_as_real(torch.complex(s_re, s_im)).to(x.dtype)
    return out, (new_state if m > 1 else new_state[0])


_METHODS = {
    "forward": forward,
    "_forward_chunked_head": forward_chunked_head,
    "_fused_chunk_step": fused_chunk_step,
    "_forward_multistate_fused": forward_multistate_fused,
    "_recur_step_additive": recur_step_additive,
    "_forward_delta": forward_delta,
    "_recur_step_delta": recur_step_delta,
    "_recurrent": recurrent,
    "_forward_chunked_perchannel": forward_chunked_perchannel,
}

# module-level functions of the reference's v11 package that this package
# replaces, kept for CPU calls (qllm2_amd/_reference.py)
_MODULE_FUNCS = {
    "flash_pam": ("flash_pam_chunked_head", "_chunk_decay_matrices"),
    "triton_kernels": ("fused_decay_matrix", "fused_complex_norm", "fused_mod_swish", "fused_mod_relu",
                       "fused_cgu_gate"),
    "fused_ce": ("fused_linear_cross_entropy", "linear_ce_per_token", "linear_ce_stats"),
}

_COMPLEX_OPS = ("fused_complex_norm", "fused_mod_swish", "fused_mod_relu", "fused_cgu_gate")


def install(model_module=None):
    """Bind the HIP implementations into the reference's v11 package.

    model_module: the imported v11.model module (default: sys.modules['v11.model']).
    Rebinds the V11PAMLayer methods above (and the static _dual_form_block)
    after keeping the class's own methods as V11PAMLayer._qpam_originals (the
    replacements hand them the calls the kernels do not cover), replaces the
    module-level fused_decay_matrix name v11/model.py:40 bound at import, and
    aliases v11.flash_pam / v11.triton_kernels / v11.fused_ce to this
    package's modules so later imports (v11/model.py:1182, v7/train.py:301,350)
    resolve here; the reference functions they replace are kept for CPU
    tensors.  Calling it again is harmless.  Returns the saved originals."""
    mod = model_module if model_module is not None else sys.modules["v11.model"]
    layer = mod.V11PAMLayer
    table = layer.__dict__.get("_qpam_originals")
    if table is None:
        table = {name: getattr(layer, name) for name in _METHODS if hasattr(layer, name)}
        if hasattr(layer, "_dual_form_block"):
            table["_dual_form_block"] = getattr(layer, "_dual_form_block")   # the static function itself
        layer._qpam_originals = table
    for name, fn in _METHODS.items():
        if name in table:
            setattr(layer, name, fn)
    layer._dual_form_block = staticmethod(_dual_form_block_for(table.get("_dual_form_block")))
    if hasattr(mod, "fused_decay_matrix"):
        _reference.save("triton_kernels.fused_decay_matrix", mod.fused_decay_matrix)
        mod.fused_decay_matrix = _tk.fused_decay_matrix
    pkg = mod.__name__.rsplit(".", 1)[0] if "." in mod.__name__ else "v11"
    ours = {"flash_pam": _flash_pam, "triton_kernels": _tk, "fused_ce": _fused_ce}
    saved = dict(table)
    for sub, m in ours.items():
        ref = sys.modules.get(f"{pkg}.{sub}")
        if ref is None:
            try:
                ref = importlib.import_module(f"{pkg}.{sub}")
            except ImportError:
                ref = None
        if ref is not None and ref is not m:
            for name in _MODULE_FUNCS[sub]:
                _reference.save(f"{sub}.{name}", getattr(ref, name, None))
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
                if _reference.saved(f"triton_kernels.{name}") is None:
                    _reference.save(f"triton_kernels.{name}", getattr(cops, name))
                setattr(cops, name, getattr(_tk, name))
    for sub, names in _MODULE_FUNCS.items():
        for name in names:
            fn = _reference.saved(f"{sub}.{name}")
            if fn is not None:
                saved[f"{sub}.{name}"] = fn
    return saved
