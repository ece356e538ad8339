"""O(1)/token recurrent PAM decode on the HIP kernel (qpam_decode_step).

Reference: V11PAMLayer._recur_step_additive (v11/model.py:927-965) and the
per-token state loop of V11PAMLayer._recurrent (v11/model.py:845-925).

`decode_step` is the continuous-batching form: one call updates every listed
slot of a state pool in place, all layers/heads/states at once, optionally
rotating q and k by each slot's own RoPE position.  `SlotPool` is the decode
engine around it (V11LM.generate, v11/model.py:1207-1245, without the batch-1
loop): per-layer states of many sequences, joined and released between steps.
`recur_step_additive` keeps the reference method's signature and functional
(non-mutating) semantics.  The kernels are built for head dims 16, 32, 64 and
128; a smaller head dim of another size runs on the next of them with zero
padding (the padded rows and columns of the state stay zero, since the padded
entries of v and k are zero, and the padded columns of q add nothing to y).
"""

import torch
import torch.nn.functional as F

from . import _lib

KERNEL_DIMS = (16, 32, 64, 128)


def kernel_dim(d):
    """The kernels' head dim that runs head dim d (d itself, or the next
    larger one with zero padding); None above 128."""
    return next((k for k in KERNEL_DIMS if k >= d), None)


def _check_cuda(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("qpam decode: tensors must be on the GPU (no CPU path in this library)")


def decode_step(state, q, k, v, gamma, *, active=None, rot=None, q_scale=1.0, out=None, rope=None, pos=None,
                compact=False):
    """In-place ragged decode step over a slot pool.

    state  [S, G, M, d, d, 2] fp32 (G = layers*heads, M states), updated in place
    q,k,v  [R, G, d, 2] fp32 (q unscaled; multiplied by q_scale), or all three
           as planar (re, im) pairs of [R, G, d] fp32 tensors with equal strides
    gamma  [R, G, M] fp32 (any strides), or [R, G, M, d] with the last dim
           contiguous: one decay per key channel (E1 per-channel decay)
    active optional int32 [n] slot ids (others untouched); None = all slots
    rot    optional [R, G, M, 2] fp32 complex rotation of each state's read, or a
           planar (re, im) pair of [R, G, M] fp32 tensors with equal strides
    rope   optional [P, d, 2] fp32 rotary table (build_rope_cache) with
    pos    int32 [S] per-slot positions: q and k of slot a are rotated by rope[pos[a]]
    compact False: R = S, row a of q, k, v, gamma, rot, y belongs to slot a
           True:  R = n, row i belongs to slot active[i] (the live batch of an engine)
    out    optional y buffer [R, G, d, 2], fp32 or bf16 (the kernel rounds the fp32
           sums once)
    Returns y [R, G, d, 2] (without `compact`, rows of unlisted slots are left
    as in `out` / zero).
    """
    planar = isinstance(q, (tuple, list))
    if any(isinstance(t, (tuple, list)) != planar for t in (k, v)):
        raise ValueError("q, k and v must all be interleaved tensors or all (re, im) plane pairs")
    planes = [x for t in (q, k, v) for x in t] if planar else [q, k, v]
    _check_cuda(state, *planes, gamma, active, *(rot if isinstance(rot, (tuple, list)) else (rot,)), rope, pos)
    if state.dim() != 6 or state.shape[-1] != 2 or state.shape[-2] != state.shape[-3]:
        raise ValueError(f"state must be [S,G,M,d,d,2], got {tuple(state.shape)}")
    n_slots, n_groups, n_states, d = state.shape[:4]
    if compact and active is None:
        raise ValueError("compact rows need the active slot list")
    rows = active.numel() if compact else n_slots
    want = (rows, n_groups, d) if planar else (rows, n_groups, d, 2)
    for name, t in zip(("q_re", "q_im", "k_re", "k_im", "v_re", "v_im") if planar else ("q", "k", "v"), planes):
        if tuple(t.shape) != want:
            raise ValueError(f"{name} must be {list(want)}, got {tuple(t.shape)}")
    per_channel = gamma.dim() == 4
    if tuple(gamma.shape) != ((rows, n_groups, n_states, d) if per_channel else (rows, n_groups, n_states)):
        raise ValueError(f"gamma must be [{rows},{n_groups},{n_states}] or [{rows},{n_groups},{n_states},{d}], "
                         f"got {tuple(gamma.shape)}")
    if per_channel and gamma.stride(-1) != 1:
        gamma = gamma.contiguous()
    rot_pl = isinstance(rot, (tuple, list))
    rots = list(rot) if rot_pl else ([rot] if rot is not None else [])
    for t in [state, gamma] + planes + rots:
        if t.dtype != torch.float32:
            raise ValueError("qpam decode works on fp32 tensors")
    if state.stride()[-3:] != (2 * d, 2, 1):
        raise ValueError("state matrices must be contiguous [d, d, 2]")
    if planar:
        pairs = []
        for re, im in (q, k, v):
            if re.stride(-1) != 1 or re.stride() != im.stride():
                re, im = re.contiguous(), im.contiguous()
            pairs.append((re, im))
        (q, q_im), (k, k_im), (v, v_im) = pairs
    else:
        q, k, v = (t if t.stride()[-2:] == (2, 1) else t.contiguous() for t in (q, k, v))
    rot_im = None
    if rot_pl:
        rot, rot_im = rots
        for t in (rot, rot_im):
            if tuple(t.shape) != (rows, n_groups, n_states):
                raise ValueError(f"rot planes must be [{rows},{n_groups},{n_states}]")
        if rot.stride() != rot_im.stride():
            rot, rot_im = rot.contiguous(), rot_im.contiguous()
    elif rot is not None:
        if tuple(rot.shape) != (rows, n_groups, n_states, 2):
            raise ValueError(f"rot must be [{rows},{n_groups},{n_states},2]")
        rot = rot if rot.stride(-1) == 1 else rot.contiguous()
    y = out if out is not None else torch.zeros(rows, n_groups, d, 2, device=state.device, dtype=torch.float32)
    if y.dtype not in (torch.float32, torch.bfloat16) or tuple(y.shape) != (rows, n_groups, d, 2) \
            or y.stride()[-2:] != (2, 1):
        raise ValueError(f"out must be fp32 or bf16 [{rows},{n_groups},{d},2] with contiguous rows")
    if active is not None:
        if active.dtype != torch.int32:
            active = active.to(torch.int32)
        active = active.contiguous()
        n_active = active.numel()
    else:
        n_active = n_slots
    a = _lib.DecodeArgs()
    a.n_slots, a.n_active, a.n_groups, a.n_states, a.d = n_slots, n_active, n_groups, n_states, d
    a.vec_by_rank = int(bool(compact))
    a.active = active.data_ptr() if active is not None else None
    a.q_scale = float(q_scale)
    a.state = state.data_ptr()
    a.st_slot, a.st_group, a.st_state = state.stride(0), state.stride(1), state.stride(2)
    a.q, a.k, a.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    if planar:
        a.q_im, a.k_im, a.v_im = q_im.data_ptr(), k_im.data_ptr(), v_im.data_ptr()
    a.sq_slot, a.sq_group = q.stride(0), q.stride(1)
    a.sk_slot, a.sk_group = k.stride(0), k.stride(1)
    a.sv_slot, a.sv_group = v.stride(0), v.stride(1)
    a.gamma = gamma.data_ptr()
    a.sg_slot, a.sg_group, a.sg_state = gamma.stride()[:3]
    a.gamma_per_channel = int(per_channel)
    if rot is not None:
        a.rot = rot.data_ptr()
        a.sr_slot, a.sr_group, a.sr_state = rot.stride(0), rot.stride(1), rot.stride(2)
        if rot_im is not None:
            a.rot_im = rot_im.data_ptr()
    a.y = y.data_ptr()
    a.sy_slot, a.sy_group = y.stride(0), y.stride(1)
    a.y_dtype = _lib.QPAM_BF16 if y.dtype == torch.bfloat16 else _lib.QPAM_F32
    if rope is not None:
        if pos is None:
            raise ValueError("rope needs per-slot positions `pos`")
        if rope.dtype != torch.float32 or tuple(rope.shape[1:]) != (d, 2):
            raise ValueError(f"rope must be fp32 [P, {d}, 2], got {rope.dtype} {tuple(rope.shape)}")
        rope = rope.contiguous()
        pos = pos.to(torch.int32).contiguous()
        if pos.numel() != n_slots:
            raise ValueError(f"pos must hold one position per slot ({n_slots}), got {pos.numel()}")
        a.rope, a.pos, a.rope_len = rope.data_ptr(), pos.data_ptr(), rope.shape[0]
    L = _lib.lib()
    with torch.cuda.device(state.device):
        _lib.check(L.qpam_decode_step(a, _lib.stream_ptr(state.device)), "qpam_decode_step")
    return y


def decode_step_proj(state, proj, dt_bias, *, gate=None, protect_col=-1, phase_col=-1, state_offset=None,
                     qk_norm=False, gamma_floor=0.0, active=None, q_scale=1.0, out=None, rope=None, pos=None,
                     compact=False):
    """decode_step with the decode prologue fused (d = 64, head decay): q, k,
    v, the decays and the rotations of each (row, head) are formed in the kernel
    from the layer's projection row and gate logits, as pam_prologue computes
    them (qk-norm, GSP blend, softplus decay with floor, rotation e^{i phase}),
    then RoPE at each slot's position and the update.

    state  [S, G, M, 64, 64, 2] fp32, updated in place (G heads of one layer)
    proj   [R, C] fp32 or bf16, the prologue's layout: q, k, v real planes
           ([G, 64] each), their imaginary planes, G decay logits (C >= 6 G 64 + G)
    dt_bias [G] fp32 (the summed decay biases); state_offset [M] fp32 or None
    gate   [R, W] in proj's dtype or None: protect logits at protect_col + g,
           phase of state m at phase_col + g M + m (-1: absent)
    Other arguments and the return value as decode_step."""
    _check_cuda(state, proj, dt_bias, gate, state_offset, active, rope, pos)
    if state.dim() != 6 or state.shape[-1] != 2 or state.shape[3] != 64 or state.shape[4] != 64:
        raise ValueError(f"state must be [S,G,M,64,64,2], got {tuple(state.shape)}")
    n_slots, n_groups, n_states, d = state.shape[:4]
    if compact and active is None:
        raise ValueError("compact rows need the active slot list")
    rows = active.numel() if compact else n_slots
    if proj.dim() != 2 or proj.shape[0] != rows or proj.shape[1] < 6 * n_groups * d + n_groups \
            or proj.stride(1) != 1 or proj.dtype not in (torch.float32, torch.bfloat16):
        raise ValueError(f"proj must be fp32/bf16 [{rows}, >= {6 * n_groups * d + n_groups}] with contiguous rows")
    if gate is not None and (gate.dim() != 2 or gate.shape[0] != rows or gate.stride(1) != 1
                             or gate.dtype != proj.dtype):
        raise ValueError(f"gate must be [{rows}, W] in proj's dtype with contiguous rows")
    if state.dtype != torch.float32 or state.stride()[-3:] != (2 * d, 2, 1):
        raise ValueError("state must be fp32 with contiguous [d, d, 2] matrices")
    # the gate columns the kernel reads must lie inside the gate matrix
    width = gate.shape[1] if gate is not None else 0
    if protect_col >= 0 and protect_col + n_groups > width:
        raise ValueError(f"protect columns {protect_col}..{protect_col + n_groups - 1} outside the gate's {width}")
    if phase_col >= 0 and phase_col + n_groups * n_states > width:
        raise ValueError(f"phase columns {phase_col}..{phase_col + n_groups * n_states - 1} outside the gate's "
                         f"{width}")
    if dt_bias.numel() != n_groups or (state_offset is not None and state_offset.numel() != n_states):
        raise ValueError(f"dt_bias must have {n_groups} elements and state_offset {n_states}")
    dt_bias = dt_bias.float().contiguous()
    state_offset = state_offset.float().contiguous() if state_offset is not None else None
    y = out if out is not None else torch.zeros(rows, n_groups, d, 2, device=state.device, dtype=torch.float32)
    if y.dtype not in (torch.float32, torch.bfloat16) or tuple(y.shape) != (rows, n_groups, d, 2) \
            or y.stride()[-2:] != (2, 1):
        raise ValueError(f"out must be fp32 or bf16 [{rows},{n_groups},{d},2] with contiguous rows")
    if active is not None:
        active = active.to(torch.int32).contiguous()
    a = _lib.DecodeArgs()
    a.n_slots, a.n_active, a.n_groups, a.n_states, a.d = n_slots, (active.numel() if active is not None else
                                                                    n_slots), n_groups, n_states, d
    a.vec_by_rank = int(bool(compact))
    a.active = active.data_ptr() if active is not None else None
    a.q_scale = float(q_scale)
    a.state = state.data_ptr()
    a.st_slot, a.st_group, a.st_state = state.stride(0), state.stride(1), state.stride(2)
    a.proj, a.proj_dtype, a.proj_ld = proj.data_ptr(), _lib.QPAM_BF16 if proj.dtype == torch.bfloat16 else \
        _lib.QPAM_F32, proj.stride(0)
    a.qk_norm, a.gamma_floor = int(bool(qk_norm)), float(gamma_floor)
    a.protect_col, a.phase_col = int(protect_col), int(phase_col)
    if gate is not None:
        a.gate, a.gate_ld = gate.data_ptr(), gate.stride(0)
    a.dt_bias = dt_bias.data_ptr()
    if state_offset is not None:
        a.state_offset = state_offset.data_ptr()
    a.y = y.data_ptr()
    a.sy_slot, a.sy_group = y.stride(0), y.stride(1)
    a.y_dtype = _lib.QPAM_BF16 if y.dtype == torch.bfloat16 else _lib.QPAM_F32
    if rope is not None:
        if pos is None:
            raise ValueError("rope needs per-slot positions `pos`")
        if rope.dtype != torch.float32 or tuple(rope.shape[1:]) != (d, 2):
            raise ValueError(f"rope must be fp32 [P, {d}, 2], got {rope.dtype} {tuple(rope.shape)}")
        rope = rope.contiguous()
        pos = pos.to(torch.int32).contiguous()
        if pos.numel() != n_slots:
            raise ValueError(f"pos must hold one position per slot ({n_slots}), got {pos.numel()}")
        a.rope, a.pos, a.rope_len = rope.data_ptr(), pos.data_ptr(), rope.shape[0]
    with torch.cuda.device(state.device):
        _lib.check(_lib.lib().qpam_decode_step(a, _lib.stream_ptr(state.device)), "qpam_decode_step")
    return y


class _DecodeStep(torch.autograd.Function):
    """One decode step of n independent single-state (slot, head) rows, out of
    place and differentiable: (state [n,d,d,2], gamma [n] or [n,d], v, k, q
    [n,d,2], q scaled) -> (y [n,d,2], new state).  Forward: qpam_decode_step;
    backward: qpam_decode_step_bwd."""

    @staticmethod
    def forward(ctx, state, gamma, v, k, q):
        n, d = state.shape[0], state.shape[1]
        per_channel = gamma.dim() == 2
        new = state.clone()
        y = decode_step(new.view(n, 1, 1, d, d, 2), q.view(n, 1, d, 2), k.view(n, 1, d, 2), v.view(n, 1, d, 2),
                        gamma.view(n, 1, 1, d) if per_channel else gamma.view(n, 1, 1), q_scale=1.0)
        ctx.save_for_backward(state, gamma, q, k, v)
        return y.view(n, d, 2), new

    @staticmethod
    def backward(ctx, dy, dnew):
        state, gamma, q, k, v = ctx.saved_tensors
        dy = dy.contiguous() if dy is not None else torch.zeros_like(q)
        dnew = dnew.contiguous() if dnew is not None else None
        dstate, dgamma = torch.empty_like(state), torch.empty_like(gamma)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        a = _lib.DecodeBwdArgs()
        a.n, a.d, a.gamma_per_channel = state.shape[0], state.shape[1], int(gamma.dim() == 2)
        a.state, a.gamma, a.q, a.k, a.v, a.dy = (t.data_ptr() for t in (state, gamma, q, k, v, dy))
        a.dstate_new = dnew.data_ptr() if dnew is not None else None
        a.dstate, a.dgamma, a.dq, a.dk, a.dv = (t.data_ptr() for t in (dstate, dgamma, dq, dk, dv))
        with torch.cuda.device(state.device):
            _lib.check(_lib.lib().qpam_decode_step_bwd(a, _lib.stream_ptr(state.device)), "qpam_decode_step_bwd")
        return dstate, dgamma, dv, dk, dq


def recur_step_additive(memory_state, decay_gamma, value_t, key_t, query_t):
    """Drop-in for V11PAMLayer._recur_step_additive (v11/model.py:927-965).
    memory_state [..., d, d, 2]; decay_gamma [...] (head decay) or [..., d]
    (per-channel decay, one per key column); value_t/key_t/query_t [..., d, 2]
    (query already scaled).  Returns (output [..., d, 2], new memory_state);
    the input is not modified.  Differentiable in every input (the backward is
    qpam_decode_step_bwd)."""
    per_channel = decay_gamma.dim() == memory_state.dim() - 2
    if not per_channel and decay_gamma.dim() != memory_state.dim() - 3:
        raise ValueError(f"decay_gamma must be [...] or [..., d] for a state {tuple(memory_state.shape)}")
    lead = memory_state.shape[:-3]
    d = memory_state.shape[-2]
    kd = kernel_dim(d)
    if kd is None:
        raise ValueError(f"qpam decode: head dim {d} (at most {KERNEL_DIMS[-1]})")
    n = memory_state[..., 0, 0, 0].numel()
    f32 = lambda t, *shape: t.to(torch.float32).contiguous().view(n, *shape)  # noqa: E731
    st, gam = f32(memory_state, d, d, 2), f32(decay_gamma, d) if per_channel else f32(decay_gamma)
    v, k, q = f32(value_t, d, 2), f32(key_t, d, 2), f32(query_t, d, 2)
    if kd != d:  # zero padding to the kernel's head dim (differentiable: the gradients come back sliced)
        p = kd - d
        st = F.pad(st, (0, 0, 0, p, 0, p))
        v, k, q = (F.pad(t, (0, 0, 0, p)) for t in (v, k, q))
        if per_channel:
            gam = F.pad(gam, (0, p), value=1.0)
    y, new_state = _DecodeStep.apply(st, gam, v, k, q)
    if kd != d:
        y, new_state = y[:, :d], new_state[:, :d, :d]
    return (y.reshape(*lead, d, 2).to(memory_state.dtype),
            new_state.reshape(*lead, d, d, 2).to(memory_state.dtype))


def build_rope_cache(max_len, head_dim, device=None):
    """Complex RoPE table e^{i m theta_j} [max_len, head_dim, 2] fp32, the
    reference's build_rope_cache (v11/complex_ops.py:261-266):
    theta_j = 10000^(-j / head_dim), computed in fp32 as there."""
    inverse_freqs = 1.0 / (10000.0 ** (torch.arange(head_dim, device=device).float() / head_dim))
    positions = torch.arange(max_len, device=device).float()
    angles = positions.unsqueeze(1) * inverse_freqs.unsqueeze(0)
    return torch.stack([angles.cos(), angles.sin()], dim=-1)


class SlotPool:
    """PAM state of a continuous-batching decode: `n_slots` sequence slots, each
    with per-layer fp32 states [layers, heads, states, d, d, 2] and its own
    position for the rotary offset.

    Replaces the per-sequence state lists and the single step_offset of the
    reference's batch loop (V11LM.generate, v11/model.py:1207-1245): sequences
    join (acquire, optionally with the states a prefill produced) and leave
    (release) between steps, and one `step` per layer updates every listed slot
    with one kernel launch (qpam_decode_step with per-slot RoPE); `advance`
    moves the listed slots' positions by one token.
    """

    def __init__(self, n_slots, n_layers, n_heads, head_dim, n_states=1, device="cuda", max_len=4096):
        self.n_slots, self.n_layers, self.n_heads, self.head_dim, self.n_states = (
            n_slots, n_layers, n_heads, head_dim, n_states)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("qpam SlotPool: the pool lives on the GPU (no CPU path in this library)")
        self.state = torch.zeros(n_slots, n_layers, n_heads, n_states, head_dim, head_dim, 2,
                                 device=self.device, dtype=torch.float32)
        self.pos = torch.zeros(n_slots, device=self.device, dtype=torch.int32)
        self._host_pos = [0] * n_slots       # host copy of pos: the table is grown before a step needs it
        self.rope = build_rope_cache(max_len, head_dim, device=self.device)
        self._free = list(range(n_slots - 1, -1, -1))
        self.live = set()

    def reserve(self, count):
        """Take the `count` highest free slot ids out of circulation for good
        (scratch rows: a padded batch points its extra rows at them).  Returns
        the ids."""
        if count > len(self._free):
            raise RuntimeError("SlotPool: not enough free slots to reserve")
        ids, self._free = sorted(self._free[:count]), self._free[count:]
        return ids

    def acquire(self, position=0, states=None):
        """Take a free slot for a sequence whose next token is at `position`.
        states: optional per-layer prefill states, each [n_states, n_heads, d, d, 2]
        (the reference's [K, B=1, H, d, d, 2] with the batch axis dropped) or
        [n_heads, d, d, 2] when n_states == 1.  Returns the slot id."""
        if not self._free:
            raise RuntimeError("SlotPool: no free slot")
        slot = self._free.pop()
        self.live.add(slot)
        self.pos[slot] = int(position)
        self._host_pos[slot] = int(position)
        if states is None:
            self.state[slot].zero_()
        else:
            for layer, st in enumerate(states):
                st = st.to(self.device, torch.float32)
                if st.dim() == 4:
                    st = st.unsqueeze(0)
                # [M, H, d, d, 2] -> [H, M, d, d, 2]
                self.state[slot, layer].copy_(st.permute(1, 0, 2, 3, 4))
        return slot

    def release(self, slot):
        self.live.discard(slot)
        self._free.append(slot)

    def layer_state(self, layer):
        """View [n_slots, n_heads, n_states, d, d, 2] of one layer (no copy)."""
        return self.state[:, layer]

    def ensure_len(self, max_pos):
        """Grow the rotary table (doubling, as the reference's rope cache) to cover max_pos."""
        if max_pos >= self.rope.shape[0]:
            self.rope = build_rope_cache(2 * (max_pos + 1), self.head_dim, device=self.device)

    def step(self, layer, q, k, v, gamma, active, rot=None, q_scale=None, out=None, compact=False):
        """One token for the listed slots on one layer: q, k, v [n_slots, heads, d, 2]
        (or planar (re, im) pairs of [n_slots, heads, d], as decode_step takes)
        (rows of unlisted slots ignored; q unscaled), gamma [n_slots, heads, states],
        rot optional [n_slots, heads, states, 2]; with `compact` the rows are those of
        the listed slots in order ([n_active, ...]).  RoPE at each slot's position; the
        table is grown first (doubling) when a live slot's position passes its end."""
        scale = self.head_dim ** -0.5 if q_scale is None else q_scale
        if self.live:
            self.ensure_len(max(self._host_pos[s] for s in self.live))
        return decode_step(self.layer_state(layer), q, k, v, gamma, active=active, rot=rot, q_scale=scale,
                           out=out, rope=self.rope, pos=self.pos, compact=compact)

    def step_proj(self, layer, proj, dt_bias, active, q_scale=None, out=None, compact=False, **prologue):
        """step with the decode prologue fused (decode_step_proj): proj
        [rows, C] the layer's projection rows, prologue keywords as
        decode_step_proj takes them (gate, protect_col, phase_col,
        state_offset, qk_norm, gamma_floor)."""
        scale = self.head_dim ** -0.5 if q_scale is None else q_scale
        if self.live:
            self.ensure_len(max(self._host_pos[s] for s in self.live))
        return decode_step_proj(self.layer_state(layer), proj, dt_bias, active=active, q_scale=scale, out=out,
                                rope=self.rope, pos=self.pos, compact=compact, **prologue)

    def advance(self, active, host_ids=None):
        """Move the listed slots one token on.  active: an int tensor or a list
        of slot ids; host_ids: the same ids as a host list when `active` is a
        device tensor (saves reading it back, a host synchronisation)."""
        if host_ids is None:
            host_ids = active.tolist() if torch.is_tensor(active) else list(active)
        for s in host_ids:
            self._host_pos[int(s)] += 1
        if torch.is_tensor(active):
            idx = active.to(self.device, torch.long)
        else:
            idx = torch.tensor(host_ids, dtype=torch.long).to(self.device)
        self.pos[idx] += 1

