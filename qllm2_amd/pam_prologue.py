"""PAM layer prologue on the HIP kernel (qpam_prologue_fwd / _bwd).

One pass from the layer's projections to the scan's inputs, replacing the
elementwise steps of V11PAMLayer (v11/model.py) between its projections and
its chunk loop: RoPE and qk-norm of _project (:290-305), the decay / GSP
blend of _gamma_all_and_vprime and _gamma_and_vprime (:630-655, :309-347,
gamma floor :193-201) and the state rotations of _phase_and_alpha
(:230-257, :741-746), with the [B,T,H] -> [B,H,T] transposes folded into the
kernel's addressing.

The projections arrive as one matrix `proj` [B, T, C], the output of a single
GEMM: columns [0, 3 H d) hold the real planes of q, k, v ([3, H, d] per
token), [3 H d, 6 H d) the imaginary planes, [6 H d, 6 H d + H) the decay
logits dt, and the rest (up to a multiple of 8 columns) padding.  Its
gradient is produced whole by the backward kernel, so autograd hands it to
the GEMM's backward without assembling slices.

`pam_prologue` is differentiable (torch.library custom op with a registered
autograd formula); the gradients of dt_bias and the state offsets are sums of
the kernel's per-element dpre over the broadcast axes.  The backward writes
the logits' gradients in the logits' own [B,T,H(,M)] layouts.
"""

from typing import List, Optional

import torch
from torch import Tensor

from . import _lib

HEAD_DIM = 64                       # the layer's production head dim (the fused decode prologue's)
HEAD_DIMS = (16, 32, 64, 128)       # head dims of the prologue kernels


def proj_columns(n_heads, head_dim=HEAD_DIM):
    """Width of `proj` for n_heads heads of head_dim: q, k, v planes, dt, padding to 8."""
    return 6 * n_heads * head_dim + (n_heads + 7) // 8 * 8


def _dt_code(t):
    if t.dtype == torch.float32:
        return _lib.QPAM_F32
    if t.dtype == torch.bfloat16:
        return _lib.QPAM_BF16
    raise ValueError(f"qpam prologue: projections must be fp32 or bf16, got {t.dtype}")


def _param_code(t):
    return _lib.QPAM_BF16 if t.dtype == torch.bfloat16 else _lib.QPAM_F32


def _gate_views(gate, protect_col, phase_col, H, M):
    """(pointer offset in elements, strides) of the protect and phase logits
    read as columns of the gate-logit matrix `gate` [B, T, W]."""
    sb, st = gate.stride(0), gate.stride(1)
    prot = (protect_col, (sb, st, 1)) if protect_col >= 0 else None
    ph = (phase_col, (sb, st, M, 1)) if phase_col >= 0 else None
    return prot, ph


def _fill(proj, protect, phase, routing, dt_bias, dt_bias2, state_offset, rope, H, M, D, rope_offset, qk_norm,
          gamma_floor, gate=None, protect_col=-1, phase_col=-1):
    if not proj.is_cuda:
        raise ValueError("qpam prologue: tensors must be on the GPU (no CPU path in this library)")
    if D not in HEAD_DIMS:
        raise NotImplementedError(f"the HIP prologue takes head dims {HEAD_DIMS}, not {D}")
    d = D
    if proj.dim() != 3 or proj.shape[2] < 6 * H * d + H or proj.stride(2) != 1:
        raise ValueError(f"proj must be [B, T, >= {6 * H * d + H}] with contiguous columns, got {tuple(proj.shape)}")
    if not 1 <= M <= 4:
        raise NotImplementedError("the HIP prologue supports 1 to 4 states")
    B, T = proj.shape[0], proj.shape[1]
    for name, t, shape in (("protect", protect, (B, T, H)), ("phase", phase, (B, T, H, M)),
                           ("routing", routing, (B, T, H, M))):
        if t is not None and (tuple(t.shape) != shape or t.dtype != proj.dtype):
            raise ValueError(f"{name} must be {proj.dtype} {list(shape)}, got {t.dtype} {tuple(t.shape)}")
    if gate is not None:
        width = (H if protect_col >= 0 else 0) + (H * M if phase_col >= 0 else 0)
        if (protect is not None or phase is not None or routing is not None or gate.dim() != 3
                or tuple(gate.shape[:2]) != (B, T) or gate.dtype != proj.dtype or gate.stride(2) != 1
                or max(protect_col + H, phase_col + H * M) > gate.shape[2] or width == 0):
            raise ValueError("gate: [B, T, W] logits in proj's dtype with contiguous columns holding protect "
                             "(H columns at protect_col) and/or phase (H * M at phase_col), given instead of "
                             "protect / phase / routing")
    pdt = dt_bias.dtype
    for name, t, shape in (("dt_bias", dt_bias, (H,)), ("dt_bias2", dt_bias2, (H,)), ("state_offset", state_offset, (M,))):
        if t is not None and (tuple(t.shape) != shape or t.dtype != pdt or pdt not in (torch.float32, torch.bfloat16)):
            raise ValueError(f"{name} must be {list(shape)} in dt_bias's dtype (fp32 or bf16)")
    if routing is not None and routing.stride() != phase.stride():
        routing, phase = routing.contiguous(), phase.contiguous()
    if rope is not None:
        if rope.dtype != torch.float32 or tuple(rope.shape[1:]) != (d, 2):
            raise ValueError(f"rope must be fp32 [P, {d}, 2]")
        rope = rope.contiguous()
    dt_bias = dt_bias.contiguous()
    dt_bias2 = dt_bias2.contiguous() if dt_bias2 is not None else None
    state_offset = state_offset.contiguous() if state_offset is not None else None
    a = _lib.PrologueArgs()
    a.B, a.T, a.H, a.d, a.M = B, T, H, d, M
    a.in_dtype = a.out_dtype = _dt_code(proj)
    a.qk_norm = int(bool(qk_norm))
    a.gamma_floor = float(gamma_floor)
    a.param_dtype = _param_code(dt_bias)
    keep = [proj, rope, dt_bias, dt_bias2, state_offset, protect, phase, routing, gate]
    if rope is not None:
        a.rope, a.rope_offset, a.rope_len = rope.data_ptr(), int(rope_offset), rope.shape[0]
    es, base, plane = proj.element_size(), proj.data_ptr(), H * d
    a.q_re, a.k_re, a.v_re = (base + i * plane * es for i in range(3))
    a.q_im, a.k_im, a.v_im = (base + (3 + i) * plane * es for i in range(3))
    a.sx_b, a.sx_t, a.sx_h = proj.stride(0), proj.stride(1), d
    a.dt = base + 6 * plane * es
    a.sd_b, a.sd_t, a.sd_h = proj.stride(0), proj.stride(1), 1
    a.dt_bias = dt_bias.data_ptr()
    if dt_bias2 is not None:
        a.dt_bias2 = dt_bias2.data_ptr()
    if state_offset is not None:
        a.state_offset = state_offset.data_ptr()
    if gate is not None:
        prot, ph = _gate_views(gate, protect_col, phase_col, H, M)
        if prot is not None:
            a.protect = gate.data_ptr() + prot[0] * gate.element_size()
            a.sp_b, a.sp_t, a.sp_h = prot[1]
        if ph is not None:
            a.phase = gate.data_ptr() + ph[0] * gate.element_size()
            a.sr_b, a.sr_t, a.sr_h, a.sr_m = ph[1]
        return a, keep
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
def prologue_fwd_op(proj: Tensor, protect: Optional[Tensor], phase: Optional[Tensor], routing: Optional[Tensor],
                    dt_bias: Tensor, dt_bias2: Optional[Tensor], state_offset: Optional[Tensor],
                    rope: Optional[Tensor], H: int, M: int, D: int, rope_offset: int, qk_norm: bool,
                    gamma_floor: float, gate: Optional[Tensor], protect_col: int, phase_col: int) -> List[Tensor]:
    """Returns [q_re, q_im, k_re, k_im, v_re, v_im] ([B,H,T,d], proj dtype),
    gamma [M,B,H,T] and rot_re, rot_im [M,B,H,T] (empty without phase).  With
    `gate` the protect and phase logits are its columns from protect_col /
    phase_col (-1: absent) and protect / phase / routing are None."""
    a, keep = _fill(proj, protect, phase, routing, dt_bias, dt_bias2, state_offset, rope, H, M, D, rope_offset, qk_norm,
                    gamma_floor, gate, protect_col, phase_col)
    B, T = proj.shape[0], proj.shape[1]
    dev = proj.device
    outs = [torch.empty(B, H, T, D, device=dev, dtype=proj.dtype) for _ in range(6)]
    a.oq_re, a.oq_im, a.ok_re, a.ok_im, a.ov_re, a.ov_im = (o.data_ptr() for o in outs)
    gamma = torch.empty(M, B, H, T, device=dev, dtype=torch.float32)
    a.gamma = gamma.data_ptr()
    if a.phase:
        rot = [torch.empty_like(gamma), torch.empty_like(gamma)]
        a.rot_re, a.rot_im = rot[0].data_ptr(), rot[1].data_ptr()
    else:
        rot = [gamma.new_empty(0), gamma.new_empty(0)]
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().qpam_prologue_fwd(a, _lib.stream_ptr(dev)), "qpam_prologue_fwd")
    del keep
    return outs + [gamma] + rot


@prologue_fwd_op.register_fake
def _(proj, protect, phase, routing, dt_bias, dt_bias2, state_offset, rope, H, M, D, rope_offset, qk_norm, gamma_floor,
      gate, protect_col, phase_col):
    B, T = proj.shape[0], proj.shape[1]
    outs = [proj.new_empty(B, H, T, D) for _ in range(6)]
    gamma = proj.new_empty(M, B, H, T, dtype=torch.float32)
    has_phase = phase is not None or (gate is not None and phase_col >= 0)
    rot = [gamma.new_empty(M, B, H, T) if has_phase else gamma.new_empty(0) for _ in range(2)]
    return outs + [gamma] + rot


def _gate_covered(gate, protect_col, phase_col, H, M):
    """Whether the protect and phase columns cover every column of `gate`."""
    spans = sorted(s for s in ((protect_col, H), (phase_col, H * M)) if s[0] >= 0)
    end = 0
    for start, n in spans:
        if start != end:
            return False
        end = start + n
    return end == gate.shape[2]


@torch.library.custom_op("qpam::prologue_bwd", mutates_args=())
def prologue_bwd_op(proj: Tensor, protect: Optional[Tensor], phase: Optional[Tensor], routing: Optional[Tensor],
                    dt_bias: Tensor, dt_bias2: Optional[Tensor], state_offset: Optional[Tensor],
                    rope: Optional[Tensor], H: int, M: int, D: int, rope_offset: int, qk_norm: bool,
                    gamma_floor: float, gate: Optional[Tensor], protect_col: int, phase_col: int,
                    grads: List[Tensor]) -> List[Tensor]:
    """grads: the 9 output gradients (rot's empty without phase).  Returns
    [dproj ([B,T,C], padding columns zero), dprotect [B,T,H], dphase,
    drouting [B,T,H,M] (in the logits' dtype, empty where not applicable),
    dgate (gate's layout, or empty), dbias [H] (the gradient of dt_bias and of
    dt_bias2), doffset [M] (or empty), both in dt_bias's dtype]."""
    a, keep = _fill(proj, protect, phase, routing, dt_bias, dt_bias2, state_offset, rope, H, M, D, rope_offset, qk_norm,
                    gamma_floor, gate, protect_col, phase_col)
    B, T, C = proj.shape
    dev = proj.device
    g = _lib.PrologueBwdArgs()
    g.fwd = _lib.ctypes.pointer(a)
    gs = [x.contiguous() for x in grads]
    g.gq_re, g.gq_im, g.gk_re, g.gk_im, g.gv_re, g.gv_im = (x.data_ptr() for x in gs[:6])
    g.ggamma = gs[6].data_ptr()
    if a.phase:
        g.grot_re, g.grot_im = gs[7].data_ptr(), gs[8].data_ptr()
    dproj = torch.empty(B, T, C, device=dev, dtype=proj.dtype)
    used = 6 * H * D + H
    g.ddt_pad = C - used                       # the kernel zeroes the padding columns
    es, base, plane = dproj.element_size(), dproj.data_ptr(), H * D
    g.dq_re, g.dk_re, g.dv_re = (base + i * plane * es for i in range(3))
    g.dq_im, g.dk_im, g.dv_im = (base + (3 + i) * plane * es for i in range(3))
    g.sg_b, g.sg_t, g.sg_h = dproj.stride(0), dproj.stride(1), D
    g.ddt = base + 6 * plane * es
    g.sdd_b, g.sdd_t, g.sdd_h = dproj.stride(0), dproj.stride(1), 1
    # scratch for the per-block partial sums of the decay-logit gradient
    scratch = torch.empty(max(1, B * T * H * M), device=dev, dtype=torch.float32)
    g.dpre = scratch.data_ptr()
    dbias = torch.empty(H, device=dev, dtype=dt_bias.dtype)
    g.dbias = dbias.data_ptr()
    doffset = torch.empty(M, device=dev, dtype=dt_bias.dtype) if state_offset is not None else dbias.new_empty(0)
    if state_offset is not None:
        g.doffset = doffset.data_ptr()
    g.dlogit_dtype = _dt_code(proj)
    # distinct (never aliased) empty tensors stand for the gradients that do not apply
    dprotect, dphase, drouting, dgate = (proj.new_empty(0) for _ in range(4))
    if gate is not None:
        dgate = torch.empty_like(gate) if _gate_covered(gate, protect_col, phase_col, H, M) else torch.zeros_like(gate)
        prot, ph = _gate_views(dgate, protect_col, phase_col, H, M)
        if prot is not None:
            g.dprotect = dgate.data_ptr() + prot[0] * dgate.element_size()
            g.sdp_b, g.sdp_t, g.sdp_h = prot[1]
        if ph is not None:
            g.dphase = dgate.data_ptr() + ph[0] * dgate.element_size()
            g.sdq_b, g.sdq_t, g.sdq_h, g.sdq_m = ph[1]
    else:
        if protect is not None:
            dprotect = torch.empty(B, T, H, device=dev, dtype=proj.dtype)
            g.dprotect = dprotect.data_ptr()
        if phase is not None:
            dphase = torch.empty(B, T, H, M, device=dev, dtype=proj.dtype)
            g.dphase = dphase.data_ptr()
            if routing is not None:
                drouting = torch.empty_like(dphase)
                g.drouting = drouting.data_ptr()
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().qpam_prologue_bwd(g, _lib.stream_ptr(dev)), "qpam_prologue_bwd")
    del keep, gs
    return [dproj, dprotect, dphase, drouting, dgate, dbias, doffset]


@prologue_bwd_op.register_fake
def _(proj, protect, phase, routing, dt_bias, dt_bias2, state_offset, rope, H, M, D, rope_offset, qk_norm, gamma_floor,
      gate, protect_col, phase_col, grads):
    B, T, C = proj.shape
    e = proj.new_empty(0)
    return [proj.new_empty(B, T, C), proj.new_empty(B, T, H) if protect is not None else e,
            proj.new_empty(B, T, H, M) if phase is not None else e,
            proj.new_empty(B, T, H, M) if routing is not None else e,
            torch.empty_like(gate) if gate is not None else e, dt_bias.new_empty(H),
            dt_bias.new_empty(M) if state_offset is not None else dt_bias.new_empty(0)]


def _setup(ctx, inputs, output):
    (proj, protect, phase, routing, dt_bias, dt_bias2, state_offset, rope, H, M, D, rope_offset, qk_norm, gamma_floor,
     gate, protect_col, phase_col) = inputs
    ctx.save_for_backward(proj, protect, phase, routing, dt_bias, dt_bias2, state_offset, rope, gate)
    ctx.cfg = (H, M, D, rope_offset, qk_norm, gamma_floor, protect_col, phase_col)
    ctx.set_materialize_grads(False)


def _backward(ctx, grads):
    proj, protect, phase, routing, dt_bias, dt_bias2, state_offset, rope, gate = ctx.saved_tensors
    H, M, D, rope_offset, qk_norm, gamma_floor, protect_col, phase_col = ctx.cfg
    B, T = proj.shape[0], proj.shape[1]
    dev = proj.device
    has_phase = phase is not None or (gate is not None and phase_col >= 0)
    full = []
    for i, gr in enumerate(grads):
        if gr is not None:
            full.append(gr)
        elif i < 6:
            full.append(torch.zeros(B, H, T, D, device=dev, dtype=proj.dtype))
        elif i == 6 or has_phase:
            full.append(torch.zeros(M, B, H, T, device=dev, dtype=torch.float32))
        else:
            full.append(torch.empty(0, device=dev))
    dproj, dprotect, dphase, drouting, dgate, dbias, doffset = prologue_bwd_op(
        proj, protect, phase, routing, dt_bias, dt_bias2, state_offset, rope, H, M, D, rope_offset, qk_norm,
        gamma_floor, gate, protect_col, phase_col, full)
    return (dproj, dprotect if protect is not None else None, dphase if phase is not None else None,
            drouting if routing is not None else None, dbias, dbias if dt_bias2 is not None else None,
            doffset if state_offset is not None else None, None, None, None, None, None, None, None,
            dgate if gate is not None else None, None, None)


prologue_fwd_op.register_autograd(_backward, setup_context=_setup)


def pam_prologue(proj, dt_bias, *, n_heads, n_states=1, state_offset=None, protect=None, phase=None, routing=None,
                 rope=None, rope_offset=0, qk_norm=False, gamma_floor=0.0, dt_bias2=None, gate=None,
                 protect_col=-1, phase_col=-1, head_dim=HEAD_DIM):
    """Differentiable prologue.  proj [B,T,C] (fp32 or bf16, layout above);
    protect [B,T,H] and phase, routing [B,T,H,M] (cast to proj's dtype; any
    strides), or `gate` [B,T,W] holding the protect logits in columns
    protect_col.. and the phase logits in phase_col.. (-1: absent), whose
    gradient then comes back as one tensor; dt_bias [H], dt_bias2 [H]
    (optional, added to dt_bias) and state_offset [M] in one dtype (fp32 or
    bf16; mixed dtypes are read in fp32); rope [P,d,2] fp32 covering
    rope_offset + T; head_dim 16, 32, 64 or 128.  Returns (q, k, v) as planar
    pairs [B,H,T,d], gamma [M,B,H,T] and rot (re, im) [M,B,H,T] or None."""
    if rope is not None and rope_offset + proj.shape[1] > rope.shape[0]:
        raise ValueError(f"rope table of {rope.shape[0]} rows does not cover positions up to "
                         f"{rope_offset + proj.shape[1]}")
    cast = (lambda t: t.to(proj.dtype) if t is not None and t.dtype != proj.dtype else t)
    params = [t for t in (dt_bias, dt_bias2, state_offset) if t is not None]
    if len({t.dtype for t in params}) != 1 or params[0].dtype not in (torch.float32, torch.bfloat16):
        f32 = (lambda t: t.float() if t is not None else None)
        dt_bias, dt_bias2, state_offset = f32(dt_bias), f32(dt_bias2), f32(state_offset)
    if gate is not None:
        gate = cast(gate)
        if gate.stride(-1) != 1:
            gate = gate.contiguous()
    out = prologue_fwd_op(proj, cast(protect), cast(phase), cast(routing), dt_bias, dt_bias2, state_offset, rope,
                          int(n_heads), int(n_states), int(head_dim), int(rope_offset), bool(qk_norm),
                          float(gamma_floor), gate, int(protect_col), int(phase_col))
    rot = (out[7], out[8]) if phase is not None or (gate is not None and phase_col >= 0) else None
    return (out[0], out[1]), (out[2], out[3]), (out[4], out[5]), out[6], rot


def prologue_decode(proj, dt_bias, *, n_heads, n_states=1, state_offset=None, protect=None, phase=None,
                    routing=None, qk_norm=False, gamma_floor=0.0, head_dim=HEAD_DIM):
    """Inference form of pam_prologue for the decode step (no autograd, no
    RoPE): the q, k, v planes come out in fp32 whatever proj's dtype (fp32 or
    bf16), which is what the decode kernel reads, so a bf16 projection needs no
    widening pass.  protect / phase / routing as in pam_prologue."""
    cast = (lambda t: t.to(proj.dtype) if t is not None and t.dtype != proj.dtype else t)
    f32 = (lambda t: t.float() if t is not None and t.dtype != torch.float32 else t)
    a, keep = _fill(proj, cast(protect), cast(phase), cast(routing), f32(dt_bias), None, f32(state_offset), None,
                    int(n_heads), int(n_states), int(head_dim), 0, bool(qk_norm), float(gamma_floor))
    a.out_dtype = _lib.QPAM_F32
    B, T, H, M = proj.shape[0], proj.shape[1], int(n_heads), int(n_states)
    dev = proj.device
    outs = [torch.empty(B, H, T, int(head_dim), device=dev, dtype=torch.float32) for _ in range(6)]
    a.oq_re, a.oq_im, a.ok_re, a.ok_im, a.ov_re, a.ov_im = (o.data_ptr() for o in outs)
    gamma = torch.empty(M, B, H, T, device=dev, dtype=torch.float32)
    a.gamma = gamma.data_ptr()
    rot = None
    if phase is not None:
        rot = (torch.empty_like(gamma), torch.empty_like(gamma))
        a.rot_re, a.rot_im = rot[0].data_ptr(), rot[1].data_ptr()
    with torch.cuda.device(dev):
        _lib.check(_lib.lib().qpam_prologue_fwd(a, _lib.stream_ptr(dev)), "qpam_prologue_fwd")
    del keep
    return (outs[0], outs[1]), (outs[2], outs[3]), (outs[4], outs[5]), gamma, rot


def mag_linear(z, weight, bias=None, out_dtype=torch.float32):
    """Gate logits from |z| in one launch (inference): z [n, dim, 2] (fp32 or
    bf16, contiguous), weight fp32 [G, dim], bias fp32 [G] or None ->
    out [n, G] = |z| weight^T + bias in out_dtype (|z| as cabs)."""
    if not z.is_cuda:
        raise ValueError("qpam mag_linear: tensors must be on the GPU (no CPU path in this library)")
    if not (z.dim() == 3 and z.shape[2] == 2 and z.dtype in (torch.float32, torch.bfloat16)):
        raise ValueError("qpam mag_linear: z must be a float32 or bfloat16 [n, dim, 2] tensor")
    z = z.contiguous()
    n, dim = z.shape[0], z.shape[1]
    if not (weight.dim() == 2 and weight.shape[1] == dim and weight.device == z.device):
        raise ValueError(f"qpam mag_linear: weight must be [G, {dim}] on {z.device}")
    G = weight.shape[0]
    if bias is not None and not (bias.numel() == G and bias.device == z.device):
        raise ValueError(f"qpam mag_linear: bias must have {G} elements on {z.device}")
    w = weight.float().contiguous()
    b = bias.float().contiguous() if bias is not None else None
    out = torch.empty(n, G, device=z.device, dtype=out_dtype)
    with torch.cuda.device(z.device):
        _lib.check(_lib.lib().qpam_mag_linear(_dt_code(z), _dt_code(out), n, dim, G, z.data_ptr(), w.data_ptr(),
                                              b.data_ptr() if b is not None else None, out.data_ptr(), G,
                                              _lib.stream_ptr(z.device)), "qpam_mag_linear")
    return out


@torch.library.custom_op("qpam::cabs", mutates_args=())
def cabs_op(z: Tensor) -> Tensor:
    """|z| = sqrt(re^2 + im^2 + 1e-8) of a complex [..., 2] tensor (fp32 or bf16)."""
    if not z.is_cuda:
        raise ValueError("qpam cabs: tensors must be on the GPU (no CPU path in this library)")
    zc = z.contiguous()
    mag = torch.empty(z.shape[:-1], device=z.device, dtype=z.dtype)
    with torch.cuda.device(z.device):
        _lib.check(_lib.lib().qpam_cabs_fwd(_dt_code(z), mag.numel(), zc.data_ptr(), mag.data_ptr(),
                                            _lib.stream_ptr(z.device)), "qpam_cabs_fwd")
    return mag


@cabs_op.register_fake
def _(z):
    return z.new_empty(z.shape[:-1])


@torch.library.custom_op("qpam::cabs_bwd", mutates_args=())
def cabs_bwd_op(z: Tensor, mag: Tensor, gmag: Tensor) -> Tensor:
    zc, gc = z.contiguous(), gmag.contiguous()
    gz = torch.empty_like(zc)
    with torch.cuda.device(z.device):
        _lib.check(_lib.lib().qpam_cabs_bwd(_dt_code(z), mag.numel(), zc.data_ptr(), mag.data_ptr(), gc.data_ptr(),
                                            gz.data_ptr(), _lib.stream_ptr(z.device)), "qpam_cabs_bwd")
    return gz


@cabs_bwd_op.register_fake
def _(z, mag, gmag):
    return torch.empty_like(z)


def _cabs_setup(ctx, inputs, output):
    ctx.save_for_backward(inputs[0], output)


def _cabs_backward(ctx, g):
    z, mag = ctx.saved_tensors
    return cabs_bwd_op(z, mag, g.to(mag.dtype))


cabs_op.register_autograd(_cabs_backward, setup_context=_cabs_setup)


def cabs(z):
    """Differentiable complex magnitude on the HIP kernel (cabs of
    v11/complex_ops.py:86-87); the element count must be a multiple of 4."""
    if z.dtype not in (torch.float32, torch.bfloat16) or z.shape[-1] != 2 or (z.numel() // 2) % 4:
        raise ValueError("qpam cabs: fp32/bf16 [..., 2] tensors with a multiple of 4 complex elements")
    return cabs_op(z)
