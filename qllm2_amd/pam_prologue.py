"""PAM layer prologue on the HIP kernel (qpam_prologue_fwd / _bwd).

One pass from the layer's projections to the scan's inputs, replacing the
elementwise steps of V11PAMLayer (v11/model.py) between its projections and
its chunk loop: RoPE and qk-norm of _project (:290-305), the decay / GSP
blend of _gamma_all_and_vprime and _gamma_and_vprime (:630-655, :309-347,
gamma floor :193-201) and the state rotations of _phase_and_alpha
(:230-257, :741-746), with the [B,T,H] -> [B,H,T] transposes folded into the
kernel's addressing.

`pam_prologue` is differentiable (torch.library custom op with a registered
autograd formula); gradients of the decay logits, dt_bias and state offsets
come from one per-element tensor dpre that torch sums over the broadcast axes.
"""

from typing import List, Optional

import torch
from torch import Tensor

from . import _lib


def _dt_code(t):
    if t.dtype == torch.float32:
        return _lib.QPAM_F32
    if t.dtype == torch.bfloat16:
        return _lib.QPAM_BF16
    raise ValueError(f"qpam prologue: projections must be fp32 or bf16, got {t.dtype}")


def _fill(qkv_re, qkv_im, dt, dt_bias, state_offset, protect, phase, routing, rope, M, rope_offset, qk_norm,
          gamma_floor):
    if not qkv_re.is_cuda:
        raise ValueError("qpam prologue: tensors must be on the GPU (no CPU path in this library)")
    if qkv_re.dim() != 5 or qkv_re.shape[2] != 3 or qkv_re.shape != qkv_im.shape:
        raise ValueError(f"qkv planes must be [B,T,3,H,d], got {tuple(qkv_re.shape)} / {tuple(qkv_im.shape)}")
    B, T, _, H, d = qkv_re.shape
    if d != 64:
        raise NotImplementedError("the HIP prologue supports head_dim 64")
    if not 1 <= M <= 4:
        raise NotImplementedError("the HIP prologue supports 1 to 4 states")
    if qkv_re.stride() != qkv_im.stride() or qkv_re.stride(-1) != 1:
        raise ValueError("qkv planes must share strides with a contiguous last axis")
    for name, t, shape in (("dt", dt, (B, T, H)), ("protect", protect, (B, T, H)), ("phase", phase, (B, T, H, M)),
                           ("routing", routing, (B, T, H, M)), ("dt_bias", dt_bias, (H,)),
                           ("state_offset", state_offset, (M,))):
        if t is not None and (tuple(t.shape) != shape or t.dtype != torch.float32):
            raise ValueError(f"{name} must be fp32 {list(shape)}, got {t.dtype} {tuple(t.shape)}")
    if routing is not None and (phase is None or routing.stride() != phase.stride()):
        routing = routing.contiguous()
        if phase is not None:
            phase = phase.contiguous()
    if rope is not None:
        if rope.dtype != torch.float32 or tuple(rope.shape[1:]) != (d, 2):
            raise ValueError(f"rope must be fp32 [P, {d}, 2]")
        rope = rope.contiguous()
    a = _lib.PrologueArgs()
    a.B, a.T, a.H, a.d, a.M = B, T, H, d, M
    a.in_dtype = a.out_dtype = _dt_code(qkv_re)
    a.qk_norm = int(bool(qk_norm))
    a.gamma_floor = float(gamma_floor)
    keep = [rope, dt_bias, state_offset, protect, phase, routing]
    if rope is not None:
        a.rope, a.rope_offset, a.rope_len = rope.data_ptr(), int(rope_offset), rope.shape[0]
    es = qkv_re.element_size()
    a.q_re, a.q_im = qkv_re.data_ptr(), qkv_im.data_ptr()
    a.k_re, a.k_im = a.q_re + qkv_re.stride(2) * es, a.q_im + qkv_re.stride(2) * es
    a.v_re, a.v_im = a.q_re + 2 * qkv_re.stride(2) * es, a.q_im + 2 * qkv_re.stride(2) * es
    a.sx_b, a.sx_t, a.sx_h = qkv_re.stride(0), qkv_re.stride(1), qkv_re.stride(3)
    a.dt = dt.data_ptr()
    a.sd_b, a.sd_t, a.sd_h = dt.stride()
    dt_bias = dt_bias.contiguous()
    keep.append(dt_bias)
    a.dt_bias = dt_bias.data_ptr()
    if state_offset is not None:
        state_offset = state_offset.contiguous()
        keep.append(state_offset)
        a.state_offset = state_offset.data_ptr()
    if protect is not None:
        a.protect = protect.data_ptr()
        a.sp_b, a.sp_t, a.sp_h = protect.stride()
    if phase is not None:
        a.phase = phase.data_ptr()
        a.sr_b, a.sr_t, a.sr_h, a.sr_m = phase.stride()
        if routing is not None:
            a.routing = routing.data_ptr()
    return a, keep


@torch.library.custom_op("qpam::prologue_fwd", mutates_args=())
def prologue_fwd_op(qkv_re: Tensor, qkv_im: Tensor, dt: Tensor, dt_bias: Tensor, state_offset: Optional[Tensor],
                    protect: Optional[Tensor], phase: Optional[Tensor], routing: Optional[Tensor],
                    rope: Optional[Tensor], M: int, rope_offset: int, qk_norm: bool,
                    gamma_floor: float) -> List[Tensor]:
    """Returns [q_re, q_im, k_re, k_im, v_re, v_im] ([B,H,T,d], qkv dtype), gamma
    [M,B,H,T] and rot_re, rot_im [M,B,H,T] (empty without phase)."""
    a, keep = _fill(qkv_re, qkv_im, dt, dt_bias, state_offset, protect, phase, routing, rope, M, rope_offset,
                    qk_norm, gamma_floor)
    B, T, _, H, d = qkv_re.shape
    dev = qkv_re.device
    outs = [torch.empty(B, H, T, d, device=dev, dtype=qkv_re.dtype) for _ in range(6)]
    a.oq_re, a.oq_im, a.ok_re, a.ok_im, a.ov_re, a.ov_im = (o.data_ptr() for o in outs)
    gamma = torch.empty(M, B, H, T, device=dev, dtype=torch.float32)
    a.gamma = gamma.data_ptr()
    if phase is not None:
        rot = [torch.empty_like(gamma), torch.empty_like(gamma)]
        a.rot_re, a.rot_im = rot[0].data_ptr(), rot[1].data_ptr()
    else:
        rot = [gamma.new_empty(0), gamma.new_empty(0)]
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().qpam_prologue_fwd(a, _lib.stream_ptr(dev)), "qpam_prologue_fwd")
    del keep
    return outs + [gamma] + rot


@prologue_fwd_op.register_fake
def _(qkv_re, qkv_im, dt, dt_bias, state_offset, protect, phase, routing, rope, M, rope_offset, qk_norm,
      gamma_floor):
    B, T, _, H, d = qkv_re.shape
    outs = [qkv_re.new_empty(B, H, T, d) for _ in range(6)]
    gamma = dt.new_empty(M, B, H, T)
    rot = [dt.new_empty(M, B, H, T) if phase is not None else dt.new_empty(0) for _ in range(2)]
    return outs + [gamma] + rot


@torch.library.custom_op("qpam::prologue_bwd", mutates_args=())
def prologue_bwd_op(qkv_re: Tensor, qkv_im: Tensor, dt: Tensor, dt_bias: Tensor, state_offset: Optional[Tensor],
                    protect: Optional[Tensor], phase: Optional[Tensor], routing: Optional[Tensor],
                    rope: Optional[Tensor], M: int, rope_offset: int, qk_norm: bool, gamma_floor: float,
                    grads: List[Tensor], want_routing: bool) -> List[Tensor]:
    """grads: the 9 output gradients (rot's empty without phase).  Returns
    [dqkv_re, dqkv_im ([B,T,3,H,d]), dpre [M,B,H,T], dprotect [B,H,T],
    dphase, drouting [M,B,H,T]] (empty where not applicable)."""
    a, keep = _fill(qkv_re, qkv_im, dt, dt_bias, state_offset, protect, phase, routing, rope, M, rope_offset,
                    qk_norm, gamma_floor)
    B, T, _, H, d = qkv_re.shape
    dev = qkv_re.device
    g = _lib.PrologueBwdArgs()
    g.fwd = _lib.ctypes.pointer(a)
    gs = [x.contiguous() for x in grads]
    g.gq_re, g.gq_im, g.gk_re, g.gk_im, g.gv_re, g.gv_im = (x.data_ptr() for x in gs[:6])
    g.ggamma = gs[6].data_ptr()
    if phase is not None:
        g.grot_re, g.grot_im = gs[7].data_ptr(), gs[8].data_ptr()
    dre = torch.empty(B, T, 3, H, d, device=dev, dtype=qkv_re.dtype)
    dim = torch.empty_like(dre)
    es = dre.element_size()
    g.dq_re, g.dq_im = dre.data_ptr(), dim.data_ptr()
    g.dk_re, g.dk_im = g.dq_re + dre.stride(2) * es, g.dq_im + dre.stride(2) * es
    g.dv_re, g.dv_im = g.dq_re + 2 * dre.stride(2) * es, g.dq_im + 2 * dre.stride(2) * es
    g.sg_b, g.sg_t, g.sg_h = dre.stride(0), dre.stride(1), dre.stride(3)
    dpre = torch.empty(M, B, H, T, device=dev, dtype=torch.float32)
    g.dpre = dpre.data_ptr()
    # distinct (never aliased) empty tensors stand for the gradients that do not apply
    dprotect = torch.empty(B, H, T, device=dev, dtype=torch.float32) if protect is not None else dpre.new_empty(0)
    if protect is not None:
        g.dprotect = dprotect.data_ptr()
    dphase = torch.empty_like(dpre) if phase is not None else dpre.new_empty(0)
    drouting = torch.empty_like(dpre) if (phase is not None and want_routing) else dpre.new_empty(0)
    if phase is not None:
        g.dphase = dphase.data_ptr()
        if want_routing:
            g.drouting = drouting.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().qpam_prologue_bwd(g, _lib.stream_ptr(dev)), "qpam_prologue_bwd")
    del keep, gs
    return [dre, dim, dpre, dprotect, dphase, drouting]


@prologue_bwd_op.register_fake
def _(qkv_re, qkv_im, dt, dt_bias, state_offset, protect, phase, routing, rope, M, rope_offset, qk_norm,
      gamma_floor, grads, want_routing):
    B, T, _, H, d = qkv_re.shape
    dre = qkv_re.new_empty(B, T, 3, H, d)
    dpre = dt.new_empty(M, B, H, T)
    dprotect = dt.new_empty(B, H, T) if protect is not None else dt.new_empty(0)
    dphase = dt.new_empty(M, B, H, T) if phase is not None else dt.new_empty(0)
    drouting = dt.new_empty(M, B, H, T) if (phase is not None and want_routing) else dt.new_empty(0)
    return [dre, torch.empty_like(dre), dpre, dprotect, dphase, drouting]


def _setup(ctx, inputs, output):
    (qkv_re, qkv_im, dt, dt_bias, state_offset, protect, phase, routing, rope, M, rope_offset, qk_norm,
     gamma_floor) = inputs
    ctx.save_for_backward(qkv_re, qkv_im, dt, dt_bias, state_offset, protect, phase, routing, rope)
    ctx.cfg = (M, rope_offset, qk_norm, gamma_floor)
    ctx.set_materialize_grads(False)


def _backward(ctx, grads):
    qkv_re, qkv_im, dt, dt_bias, state_offset, protect, phase, routing, rope = ctx.saved_tensors
    M, rope_offset, qk_norm, gamma_floor = ctx.cfg
    B, T, _, H, d = qkv_re.shape
    dev = qkv_re.device
    full = []
    for i, gr in enumerate(grads):
        if gr is not None:
            full.append(gr)
        elif i < 6:
            full.append(torch.zeros(B, H, T, d, device=dev, dtype=qkv_re.dtype))
        elif i == 6 or phase is not None:
            full.append(torch.zeros(M, B, H, T, device=dev, dtype=torch.float32))
        else:
            full.append(torch.empty(0, device=dev))
    want_routing = routing is not None
    dre, dim, dpre, dprotect, dphase, drouting = prologue_bwd_op(
        qkv_re, qkv_im, dt, dt_bias, state_offset, protect, phase, routing, rope, M, rope_offset, qk_norm,
        gamma_floor, full, want_routing)
    d_dt = dpre.sum(0).transpose(1, 2)                                   # [B,T,H]
    d_bias = dpre.sum((0, 1, 3))
    d_off = dpre.sum((1, 2, 3)) if state_offset is not None else None
    d_protect = dprotect.transpose(1, 2) if protect is not None else None
    d_phase = dphase.permute(1, 3, 2, 0) if phase is not None else None   # [B,T,H,M]
    d_routing = drouting.permute(1, 3, 2, 0) if want_routing else None
    return (dre, dim, d_dt, d_bias, d_off, d_protect, d_phase, d_routing, None, None, None, None, None)


prologue_fwd_op.register_autograd(_backward, setup_context=_setup)


def pam_prologue(qkv_re, qkv_im, dt, dt_bias, *, n_states=1, state_offset=None, protect=None, phase=None,
                 routing=None, rope=None, rope_offset=0, qk_norm=False, gamma_floor=0.0):
    """Differentiable prologue.  qkv_re, qkv_im: planar projection outputs
    [B,T,3,H,d] (fp32 or bf16); dt, protect: [B,T,H] logits; dt_bias [H];
    state_offset [M]; phase, routing [B,T,H,M]; rope [P,d,2] fp32 covering
    rope_offset + T.  The small tensors are used in fp32 (cast here).
    Returns (q, k, v) as planar pairs [B,H,T,d], gamma [M,B,H,T] and rot
    (re, im) [M,B,H,T] or None."""
    f32 = (lambda t: t.float() if t is not None and t.dtype != torch.float32 else t)
    if rope is not None and rope_offset + qkv_re.shape[1] > rope.shape[0]:
        raise ValueError(f"rope table of {rope.shape[0]} rows does not cover positions up to "
                         f"{rope_offset + qkv_re.shape[1]}")
    out = prologue_fwd_op(qkv_re, qkv_im, f32(dt), f32(dt_bias), f32(state_offset), f32(protect), f32(phase),
                          f32(routing), rope, int(n_states), int(rope_offset), bool(qk_norm), float(gamma_floor))
    rot = (out[7], out[8]) if phase is not None else None
    return (out[0], out[1]), (out[2], out[3]), (out[4], out[5]), out[6], rot
