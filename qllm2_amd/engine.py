"""Continuous-batching decode of a stack of PAM layers on the HIP kernels.

Replaces the decode loop of V11LM.generate (v11/model.py:1207-1245) and of
bench_infer's PAM loop (v11/bench_infer.py:167-193) for the PAM layers: the
reference runs one forward per token for a fixed batch whose sequences share
one step_offset, calling V11PAMLayer.forward -> _project -> _recurrent
(v11/model.py:785-925) per layer.  Here sequences join and leave between
steps, each keeps its own position, and a step of one layer runs only on the
live sequences:

  * one GEMM from the live rows x [n, dim, 2] (read interleaved, no copy) to
    the q, k, v planes and the decay logits (the fused-prefill projection,
    pam_layer._in_weight), one GEMM per gate input for the GSP protect gate and
    the E3 phase / score projections (v11/model.py:230-257, 309-347);
  * the prologue kernel (qpam_prologue_fwd: decay, GSP blend, gamma floor,
    qk-norm, rotations) on that [n, 1] batch;
  * one decode launch (qpam_decode_step, compact rows, per-slot RoPE in the
    kernel: the rotation has unit modulus per feature, so it commutes with
    the qk-norm the prologue applied first) that updates the live slots'
    states in the SlotPool and reads y;
  * one GEMM from the interleaved y to the interleaved o_proj output.

Prefill stays the fused layer forward (pam_layer.forward); its per-layer
states enter the pool through `admit`.  The layers must use head-scalar decay,
the additive write and head_dim 64 (the production presets); the engine reads
their parameters by the reference's names.  Everything runs in fp32.
"""

import torch
import torch.nn.functional as F

from .decode import SlotPool
from .pam_layer import _in_weight
from .pam_prologue import HEAD_DIM, cabs, pam_prologue, proj_columns


def _cat_planes(x):
    return torch.cat([x[..., 0], x[..., 1]], dim=-1)


class DecodeEngine:
    """Decode state and per-step work of `layers` (V11PAMLayer modules, or any
    module with their attributes) for up to `n_slots` concurrent sequences."""

    def __init__(self, layers, n_slots, *, max_len=4096):
        self.layers = list(layers)
        l0 = self.layers[0]
        self.n_heads, self.head_dim, self.n_states = l0.num_heads, l0.head_dim, l0.n_states
        for layer in self.layers:
            if (layer.num_heads, layer.head_dim, layer.n_states) != (self.n_heads, self.head_dim, self.n_states):
                raise ValueError("DecodeEngine: every layer needs the same heads, head_dim and state count")
            if getattr(layer, "decay_mode", "head") != "head" or getattr(layer, "write_mode", "additive") != "additive":
                raise NotImplementedError("DecodeEngine runs the head-decay additive write (E1 / E2 layers decode "
                                          "through the reference's _recurrent)")
            if layer.head_dim != HEAD_DIM or not 1 <= layer.n_states <= 4:
                raise NotImplementedError("DecodeEngine needs head_dim 64 and 1 to 4 states")
        device = l0.qkv_proj.weight_real.device
        self.pool = SlotPool(n_slots, len(self.layers), self.n_heads, self.head_dim, self.n_states, device=device,
                             max_len=max_len)
        self.refresh_weights()

    # ------------------------------------------------------------ weights
    def refresh_weights(self):
        """Rebuild the GEMM weights from the layers' parameters (call after
        changing them)."""
        h, d = self.n_heads, self.head_dim
        cols = proj_columns(h)
        self._w = []
        with torch.no_grad():
            for layer in self.layers:
                w_in, b_in = _in_weight(layer, h, d, cols)
                wr, wi = layer.o_proj.weight_real, layer.o_proj.weight_imag
                dim = wr.shape[0]
                # y interleaved [n, H d, 2] -> out interleaved [n, dim, 2]
                w_out = torch.stack([torch.stack([wr, -wi], -1), torch.stack([wi, wr], -1)], 1).reshape(2 * dim, -1)
                b_out = None
                if getattr(layer.o_proj, "bias_real", None) is not None:
                    b_out = torch.stack([layer.o_proj.bias_real, layer.o_proj.bias_imag], 1).reshape(2 * dim)
                self._w.append(dict(w_in=w_in.float().contiguous(), b_in=None if b_in is None else b_in.float(),
                                    w_out=w_out.float().contiguous(),
                                    b_out=None if b_out is None else b_out.float(), dim=dim))

    # ------------------------------------------------------------ slots
    def admit(self, position, states=None):
        """A sequence whose next token is at `position` joins; `states` are the
        per-layer states of its prefill (pam_layer.forward with B = 1: each
        [K, 1, H, d, d, 2], or [1, H, d, d, 2] for one state), or None for an
        empty memory.  Returns its slot id."""
        per_layer = None
        if states is not None:
            if len(states) != len(self.layers):
                raise ValueError(f"states for {len(states)} layers, engine has {len(self.layers)}")
            per_layer = []
            for st in states:
                st = st.float()
                if self.n_states > 1 or st.dim() == 6:
                    st = st[:, 0] if st.dim() == 6 else st     # [K, H, d, d, 2]
                else:
                    st = st[0]                                 # [H, d, d, 2]
                per_layer.append(st)
        return self.pool.acquire(position, per_layer)

    def release(self, slot):
        self.pool.release(slot)

    def layer_state(self, layer_idx, slot):
        """State of one sequence in one layer as the reference holds it:
        [K, 1, H, d, d, 2] (or [1, H, d, d, 2] for one state)."""
        st = self.pool.state[slot, layer_idx].permute(1, 0, 2, 3, 4)      # [H, K, d, d, 2] -> [K, H, d, d, 2]
        return st.unsqueeze(1) if self.n_states > 1 else st[0].unsqueeze(0)

    # ------------------------------------------------------------ step
    def _gates(self, layer, x):
        """protect logits [n, H], phase and routing [n, H, K] of the live rows."""
        n, h, m = x.shape[0], self.n_heads, self.n_states
        mag = None
        protect = phase = routing = None
        if layer.use_gsp:
            if layer.gate_content_aware:
                protect = layer.protect_gate(_cat_planes(x))
            else:
                mag = cabs(x)
                protect = layer.protect_gate(mag)
        if m > 1:
            if layer.routing_content_aware:
                r_in = _cat_planes(x)
            else:
                r_in = mag if mag is not None else cabs(x)
            phase = layer.phase_proj(r_in).view(n, h, m)
            if layer.state_compete:
                routing = F.softmax(layer.score_proj(r_in).view(n, h, m), dim=-1) * m
        return protect, phase, routing

    @torch.no_grad()
    def layer_step(self, layer_idx, x, slots):
        """One token of the listed sequences through layer `layer_idx`.
        x [n, dim, 2] (fp32, row i belongs to slots[i]); slots: int32 device
        tensor of n distinct live slot ids.  Updates those slots' states and
        returns the layer's output [n, dim, 2]."""
        layer, w = self.layers[layer_idx], self._w[layer_idx]
        n, dim = x.shape[0], w["dim"]
        h, d, m = self.n_heads, self.head_dim, self.n_states
        if n == 0:
            return x.new_zeros(0, dim, 2)
        x = x.float().contiguous()
        proj = F.linear(x.view(n, 2 * dim), w["w_in"], w["b_in"]).view(n, 1, -1)
        protect, phase, routing = self._gates(layer, x)
        dt_bias = layer.dt_bias if layer.dt_proj.bias is None else layer.dt_bias + layer.dt_proj.bias
        (qr, qi), (kr, ki), (vr, vi), gamma, rot = pam_prologue(
            proj, dt_bias, n_heads=h, n_states=m, state_offset=layer.state_dt_offset if m > 1 else None,
            protect=None if protect is None else protect.view(n, 1, h),
            phase=None if phase is None else phase.view(n, 1, h, m),
            routing=None if routing is None else routing.view(n, 1, h, m),
            rope=None, qk_norm=layer.qk_norm, gamma_floor=layer.gamma_floor or 0.0)
        q = torch.stack([qr[:, :, 0], qi[:, :, 0]], -1)                      # [n, H, d, 2]
        k = torch.stack([kr[:, :, 0], ki[:, :, 0]], -1)
        v = torch.stack([vr[:, :, 0], vi[:, :, 0]], -1)
        g = gamma[..., 0].permute(1, 2, 0)                                    # [n, H, K] view
        r = torch.stack([rot[0][..., 0], rot[1][..., 0]], -1).permute(1, 2, 0, 3) if rot is not None else None
        if not layer.use_rope:
            raise NotImplementedError("DecodeEngine applies RoPE per slot; layers without RoPE are not supported")
        y = self.pool.step(layer_idx, q, k, v, g, slots, rot=r, q_scale=d ** -0.5, compact=True)
        return F.linear(y.view(n, 2 * h * d), w["w_out"], w["b_out"]).view(n, dim, 2)

    def step(self, x, slots, between=None, host_slots=None):
        """One token of the listed sequences through every layer in order:
        x [n, dim, 2] enters layer 0, each layer's output (passed through
        `between(layer_idx, out)` when given: the model's own residual / norm /
        channel-mix work) enters the next; then the positions advance.
        slots: int32 device tensor of the live slot ids (row order of x);
        host_slots: the same ids as a host list, if the caller has them (no
        read-back).  Returns the last layer's output."""
        for li in range(len(self.layers)):
            x = self.layer_step(li, x, slots)
            if between is not None:
                x = between(li, x)
        self.pool.advance(slots, host_slots)
        return x
