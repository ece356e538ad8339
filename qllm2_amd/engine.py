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
  * one decode launch (qpam_decode_step, compact rows, planar q, k, v as the
    prologue wrote them, per-slot RoPE in the kernel: the rotation has unit
    modulus per feature, so it commutes with the qk-norm the prologue applied
    first) that updates the live slots' states in the SlotPool and reads y;
  * one GEMM from the interleaved y to the interleaved o_proj output.

With `graphs=True` the per-token work of all layers is captured once per
batch-size bucket (live rows rounded up to a multiple of `graph_bucket`) in a
HIP graph and replayed: one launch per step instead of about a dozen per
layer, so the host's dispatch of the small GEMMs and kernels no longer sets
the step time.  The padded rows point at reserved scratch slots (zero input,
their states are never read).  The first step of each bucket runs eagerly on
the padded batch (so library work done on a shape's first use, such as GEMM
autotuning, happens outside the capture) and captures the graph; a grown RoPE
table or new weights start new graphs.

Prefill stays the fused layer forward (pam_layer.forward); its per-layer
states enter the pool through `admit`.  The layers must use head-scalar decay,
the additive write and head_dim 16, 32, 64 or 128 (64 in the production
presets: its decode kernel forms q, k, v and the gates itself; the others run
the prologue kernel before the decode kernel); the engine reads their
parameters by the reference's names.  The states, the prologue and the
decode kernel run in fp32; the projection and o_proj GEMMs run in fp32 or,
with dtype=torch.bfloat16, on bf16 copies of the weights and inputs with fp32
accumulation (the gates' small GEMMs stay fp32).
"""

import torch
import torch.nn.functional as F

from .decode import SlotPool
from .pam_layer import _in_weight
from .pam_prologue import HEAD_DIM, HEAD_DIMS, cabs, mag_linear, prologue_decode, proj_columns


def _cat_planes(x):
    return torch.cat([x[..., 0], x[..., 1]], dim=-1)


class DecodeEngine:
    """Decode state and per-step work of `layers` (V11PAMLayer modules, or any
    module with their attributes) for up to `n_slots` concurrent sequences."""

    MAX_GRAPHS = 64  # captured graphs kept at once (each holds its own buffers)

    def __init__(self, layers, n_slots, *, max_len=4096, graphs=False, graph_bucket=16, dtype=torch.float32):
        if dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("DecodeEngine: dtype must be float32 or bfloat16")
        self.dtype = dtype
        self.layers = list(layers)
        l0 = self.layers[0]
        self.n_heads, self.head_dim, self.n_states = l0.num_heads, l0.head_dim, l0.n_states
        for layer in self.layers:
            if (layer.num_heads, layer.head_dim, layer.n_states) != (self.n_heads, self.head_dim, self.n_states):
                raise ValueError("DecodeEngine: every layer needs the same heads, head_dim and state count")
            if getattr(layer, "decay_mode", "head") != "head" or getattr(layer, "write_mode", "additive") != "additive":
                raise NotImplementedError("DecodeEngine runs the head-decay additive write (E1 / E2 layers decode "
                                          "through the reference's _recurrent)")
            if layer.head_dim not in HEAD_DIMS or not 1 <= layer.n_states <= 4:
                raise NotImplementedError(f"DecodeEngine needs a head_dim in {HEAD_DIMS} and 1 to 4 states")
        device = l0.qkv_proj.weight_real.device
        self.graph_bucket = int(graph_bucket) if graphs else 0
        if graphs and self.graph_bucket < 1:
            raise ValueError("graph_bucket must be at least 1")
        self.n_slots = n_slots
        self.pool = SlotPool(n_slots + max(self.graph_bucket - 1, 0), len(self.layers), self.n_heads,
                             self.head_dim, self.n_states, device=device, max_len=max_len)
        # scratch slots for the padded rows of a graph replay (bucket - 1 at most)
        scratch = self.pool.reserve(max(self.graph_bucket - 1, 0))
        self._scratch = torch.tensor(scratch, dtype=torch.int32, device=device) if scratch else None
        self._graphs = {}
        self._wver = 0
        self.refresh_weights()

    # ------------------------------------------------------------ weights
    def refresh_weights(self):
        """Rebuild the GEMM weights (and the summed decay bias) from the
        layers' parameters (call after changing them)."""
        h, d = self.n_heads, self.head_dim
        cols = proj_columns(h, d)
        self._graphs = {}  # captured graphs hold the old weight tensors
        self._wver += 1
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
                dt = self.dtype  # the projection and o_proj GEMMs' dtype
                entry = dict(w_in=w_in.to(dt).contiguous(), b_in=None if b_in is None else b_in.to(dt),
                             w_out=w_out.to(dt).contiguous(), b_out=None if b_out is None else b_out.to(dt),
                             dim=dim, w_mag=None,
                             dt_bias=(layer.dt_bias if layer.dt_proj.bias is None
                                      else layer.dt_bias + layer.dt_proj.bias).float().contiguous(),
                             state_offset=(layer.state_dt_offset.float().contiguous() if self.n_states > 1
                                           else None))
                # the protect gate and the phase projection both read |x|: one GEMM for both
                if (layer.use_gsp and not layer.gate_content_aware and self.n_states > 1
                        and not layer.routing_content_aware):
                    lin = (layer.protect_gate, layer.phase_proj)
                    entry["w_mag"] = torch.cat([m.weight for m in lin], 0).float().contiguous()
                    entry["b_mag"] = (torch.cat([m.bias if m.bias is not None else m.weight.new_zeros(m.weight.shape[0])
                                                 for m in lin]).float()
                                      if any(m.bias is not None for m in lin) else None)
                self._w.append(entry)

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
    def _gates(self, layer, x, w):
        """protect logits [n, H], phase and routing [n, H, K] of the live rows."""
        n, h, m = x.shape[0], self.n_heads, self.n_states
        mag = None
        protect = phase = routing = None
        if w["w_mag"] is not None:  # protect gate and phase projection from |x| in one launch
            gl = mag_linear(x, w["w_mag"], w["b_mag"], out_dtype=self.dtype)
            protect, phase = gl[:, :h], gl[:, h:].reshape(n, h, m)
            if layer.state_compete:
                routing = F.softmax(layer.score_proj(cabs(x).float()).view(n, h, m), dim=-1) * m
            return protect, phase, routing
        xf = x.float()
        if layer.use_gsp:
            if layer.gate_content_aware:
                protect = layer.protect_gate(_cat_planes(xf))
            else:
                mag = cabs(xf)
                protect = layer.protect_gate(mag)
        if m > 1:
            if layer.routing_content_aware:
                r_in = _cat_planes(xf)
            else:
                r_in = mag if mag is not None else cabs(xf)
            phase = layer.phase_proj(r_in).view(n, h, m)
            if layer.state_compete:
                routing = F.softmax(layer.score_proj(r_in).view(n, h, m), dim=-1) * m
        return protect, phase, routing

    @torch.no_grad()
    def layer_step(self, layer_idx, x, slots):
        """One token of the listed sequences through layer `layer_idx`.
        x [n, dim, 2] (fp32 or bf16, row i belongs to slots[i]); slots: int32
        device tensor of n distinct live slot ids.  Updates those slots' states
        and returns the layer's output [n, dim, 2] in the GEMM dtype (a bf16
        output feeds the next layer's bf16 projection with no conversion)."""
        layer, w = self.layers[layer_idx], self._w[layer_idx]
        n, dim = x.shape[0], w["dim"]
        h, d, m = self.n_heads, self.head_dim, self.n_states
        if n == 0:
            return x.new_zeros(0, dim, 2)
        x = x.contiguous() if x.dtype in (torch.float32, torch.bfloat16) else x.float().contiguous()
        proj = F.linear(x.view(n, 2 * dim).to(self.dtype), w["w_in"], w["b_in"]).view(n, 1, -1)
        if not layer.use_rope:
            raise NotImplementedError("DecodeEngine applies RoPE per slot; layers without RoPE are not supported")
        out = torch.empty(n, h, d, 2, device=x.device, dtype=self.dtype)
        if w["w_mag"] is not None and not layer.state_compete and d == HEAD_DIM:
            # the gate logits from |x| in one launch, the prologue inside the decode kernel
            gl = mag_linear(x, w["w_mag"], w["b_mag"], out_dtype=self.dtype)
            y = self.pool.step_proj(layer_idx, proj.view(n, -1), w["dt_bias"], slots, q_scale=d ** -0.5,
                                    compact=True, out=out, gate=gl, protect_col=0 if layer.use_gsp else -1,
                                    phase_col=(h if layer.use_gsp else 0) if m > 1 else -1,
                                    state_offset=w["state_offset"], qk_norm=layer.qk_norm,
                                    gamma_floor=layer.gamma_floor or 0.0)
            return F.linear(y.view(n, 2 * h * d), w["w_out"], w["b_out"]).view(n, dim, 2)
        protect, phase, routing = self._gates(layer, x, w)
        # the prologue writes fp32 planes (what the decode kernel reads) from a bf16 or fp32 projection
        (qr, qi), (kr, ki), (vr, vi), gamma, rot = prologue_decode(
            proj, w["dt_bias"], n_heads=h, n_states=m, state_offset=layer.state_dt_offset if m > 1 else None,
            protect=None if protect is None else protect.view(n, 1, h),
            phase=None if phase is None else phase.view(n, 1, h, m),
            routing=None if routing is None else routing.view(n, 1, h, m),
            qk_norm=layer.qk_norm, gamma_floor=layer.gamma_floor or 0.0, head_dim=d)
        # the prologue's planes go to the decode kernel as they are ([n, H, d] views)
        q, k, v = ((re[:, :, 0], im[:, :, 0]) for re, im in ((qr, qi), (kr, ki), (vr, vi)))
        g = gamma[..., 0].permute(1, 2, 0)                                    # [n, H, K] view
        r = tuple(x[..., 0].permute(1, 2, 0) for x in rot) if rot is not None else None  # planar [n, H, K] views
        # every listed slot is live, so the kernel writes every row of y: no zero fill
        # y in the GEMM dtype straight from the decode kernel (no conversion pass before o_proj)
        y = self.pool.step(layer_idx, q, k, v, g, slots, rot=r, q_scale=d ** -0.5, compact=True, out=out)
        return F.linear(y.view(n, 2 * h * d), w["w_out"], w["b_out"]).view(n, dim, 2)

    def _layers(self, x, slots, between):
        for li in range(len(self.layers)):
            x = self.layer_step(li, x, slots)
            if between is not None:
                x = between(li, x)
        return x

    def step(self, x, slots, between=None, host_slots=None):
        """One token of the listed sequences through every layer in order:
        x [n, dim, 2] enters layer 0, each layer's output (passed through
        `between(layer_idx, out)` when given: the model's own residual / norm /
        channel-mix work) enters the next; then the positions advance.
        slots: int32 device tensor of the live slot ids (row order of x);
        host_slots: the same ids as a host list, if the caller has them (no
        read-back).  Returns the last layer's output.

        With graphs, `between` is captured into the graph with the layers (it
        must be capturable: device work only, no host reads; pass the same
        callable every step, graphs are cached per callable) and the returned
        tensor is a view of the graph's output buffer, valid until the next
        step of the same bucket."""
        if not self.graph_bucket:
            x = self._layers(x, slots, between)
            self.pool.advance(slots, host_slots)
            return x
        n = x.shape[0]
        if n > self.n_slots:
            raise ValueError(f"DecodeEngine: {n} rows for {self.n_slots} slots")
        if host_slots is None:
            host_slots = slots.tolist()
        if self.pool.live:  # grow the rotary table as SlotPool.step would, before any capture or replay
            self.pool.ensure_len(max(self.pool._host_pos[s] for s in self.pool.live))
        nb = -(-n // self.graph_bucket) * self.graph_bucket
        rope = self.pool.rope.data_ptr()
        if self._graphs and next(iter(self._graphs))[2] != rope:
            self._graphs = {}  # graphs of the old rotary table are never replayed again
        key = (nb, id(between), rope, self._wver)
        entry = self._graphs.get(key) if n else None
        if entry is not None and entry["between"] is not between:
            # an id can be reused once its object is gone; each entry holds its own
            # callable (so the id stays taken while the entry lives), and a graph
            # is replayed only for the very callable it captured
            entry = None
        if entry is None:
            if n and nb > n:  # run the padded batch eagerly: the capture then meets only shapes already run
                x = torch.cat([x, x.new_zeros(nb - n, *x.shape[1:])])
                slots = torch.cat([slots.to(torch.int32), self._scratch[:nb - n]])
            out = self._layers(x, slots, between)[:n]
            if n:
                if len(self._graphs) >= self.MAX_GRAPHS:  # e.g. a new `between` callable every step
                    self._graphs = {}
                self._graphs[key] = self._capture(nb, between)
            self.pool.advance(slots[:n], host_slots)
            return out
        entry["x"][:n].copy_(x)
        entry["slots"][:n].copy_(slots)
        if nb > n:
            entry["x"][n:].zero_()
            entry["slots"][n:].copy_(self._scratch[:nb - n])
        entry["graph"].replay()
        self.pool.advance(slots, host_slots)
        return entry["out"][:n]

    def _capture(self, nb, between):
        """Capture the layers' work for `nb` rows (static input, slot-id and
        output buffers; nothing runs during the capture)."""
        dim = self._w[0]["dim"]
        dev = self.pool.device
        x = torch.zeros(nb, dim, 2, device=dev, dtype=torch.float32)
        slots = torch.zeros(nb, device=dev, dtype=torch.int32)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = self._layers(x, slots, between)
        return {"graph": graph, "x": x, "slots": slots, "out": out, "between": between}
