"""Drop-in for the public API of v11/triton_kernels.py (no Triton inside).

fused_decay_matrix (v11/triton_kernels.py:570-573) runs the HIP decay-matrix
kernel (qpam_decay_matrix) for the forward; its backward is the reference's
closed form (v11/triton_kernels.py:447-480: grad_cum = column sums - row sums
of dD . D over the unclamped causal entries, reverse cumsum, divided by
-(gamma + 1e-6)).  The PAM scan kernels never call it: they rebuild D from
log-decay prefix sums in registers.

The complex elementwise ops (fused_complex_norm, fused_mod_swish,
fused_mod_relu, fused_cgu_gate; v11/triton_kernels.py:48-166 forward,
:209-395 autograd backward) run HIP kernels for the forward and the backward
(qpam_cplx_fwd / qpam_cplx_bwd, csrc/complex_ops.hip) on fp32 and bf16
tensors; other floating dtypes are computed in fp32 and cast back.

set_triton_enabled / triton_enabled keep their names; they switch the HIP
kernels on or off (off = the reference's PyTorch formulas, its `_pt_*`
functions, v11/triton_kernels.py:489-520, on the GPU).  HAS_TRITON is False:
this module has no Triton.  CPU tensors raise, except after
pam_layer.install(), which keeps the reference's own functions for them
(the reference computes on CPU through its `_pt_*` forms).
"""

import ctypes
from typing import List, Optional

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib, _reference

__all__ = ["fused_decay_matrix", "fused_complex_norm", "fused_mod_swish", "fused_mod_relu", "fused_cgu_gate",
           "set_triton_enabled", "triton_enabled", "HAS_TRITON", "HAS_HIP"]

HAS_TRITON = False
HAS_HIP = True
_use_hip = True


def set_triton_enabled(enabled: bool) -> None:
    """Toggle the HIP decay-matrix forward (name kept from the reference API)."""
    global _use_hip
    _use_hip = bool(enabled)


def triton_enabled() -> bool:
    return _use_hip


# ---------------------------------------------------------------- PyTorch forms (reference formulas)

def _pt_complex_norm(z: Tensor, scale: Tensor, eps: float = 1e-6) -> Tensor:
    mag = torch.sqrt(z[..., 0].square() + z[..., 1].square() + 1e-8)
    rms = torch.sqrt(mag.square().mean(dim=-1, keepdim=True) + eps)
    return (z / (mag.unsqueeze(-1) + 1e-8)) * ((mag / rms) * scale).unsqueeze(-1)


def _pt_mod_swish(z: Tensor, bias: Tensor, beta: Tensor) -> Tensor:
    mag = torch.sqrt(z[..., 0].square() + z[..., 1].square() + 1e-8)
    return (z / (mag.unsqueeze(-1) + 1e-8)) * (mag * torch.sigmoid(beta * mag + bias)).unsqueeze(-1)


def _pt_mod_relu(z: Tensor, bias: Tensor) -> Tensor:
    mag = torch.sqrt(z[..., 0].square() + z[..., 1].square() + 1e-8)
    return (z / (mag.unsqueeze(-1) + 1e-8)) * F.relu(mag + bias).unsqueeze(-1)


def _pt_cgu_gate(gate: Tensor, up: Tensor) -> Tensor:
    gmag = torch.sqrt(gate[..., 0].square() + gate[..., 1].square() + 1e-8)
    gm = torch.sigmoid(gmag)
    pr, pi = gate[..., 0] / (gmag + 1e-8), gate[..., 1] / (gmag + 1e-8)
    ur, ui = up[..., 0], up[..., 1]
    return torch.stack([(pr * ur - pi * ui) * gm, (pr * ui + pi * ur) * gm], dim=-1)


def _pt_decay_matrix(decay_gamma: Tensor, seq_len: int) -> Tensor:
    log_gamma = torch.log(decay_gamma + 1e-6)
    c = torch.cumsum(-log_gamma, dim=-1)
    log_d = (c.unsqueeze(-1) - c.unsqueeze(-2)).transpose(-1, -2)
    causal = torch.tril(torch.ones(seq_len, seq_len, device=decay_gamma.device, dtype=decay_gamma.dtype))
    log_d = log_d * causal + (1 - causal) * (-1e4)
    return torch.exp(log_d.clamp(max=0.0))


# ---------------------------------------------------------------- decay matrix (HIP forward)

@torch.library.custom_op("qpam::decay_matrix", mutates_args=())
def decay_matrix_op(decay_gamma: Tensor, seq_len: int) -> Tensor:
    g = decay_gamma.to(torch.float32).contiguous()
    n = g.shape[0]
    out = torch.empty(n, seq_len, seq_len, device=g.device, dtype=torch.float32)
    L = _lib.lib()
    with torch.cuda.device(g.device):
        _lib.check(L.qpam_decay_matrix(n, seq_len, g.data_ptr(), g.stride(0), out.data_ptr(),
                                       _lib.stream_ptr(g.device)), "qpam_decay_matrix")
    return out


@decay_matrix_op.register_fake
def _(decay_gamma, seq_len):
    return decay_gamma.new_empty(decay_gamma.shape[0], seq_len, seq_len, dtype=torch.float32)


def _decay_setup(ctx, inputs, output):
    decay_gamma, seq_len = inputs
    ctx.save_for_backward(decay_gamma, output)


def _decay_backward(ctx, grad):
    """Closed form of v11/triton_kernels.py:447-480."""
    decay_gamma, d_mat = ctx.saved_tensors
    g = decay_gamma.float()
    c = torch.cumsum(-torch.log(g + 1e-6), dim=-1)
    t = d_mat.shape[-1]
    causal = torch.tril(torch.ones(t, t, device=g.device, dtype=torch.bool))
    not_clamped = causal & ((c.unsqueeze(-2) - c.unsqueeze(-1)) <= 0)
    gl = grad.float() * d_mat * not_clamped.float()
    grad_c = gl.sum(dim=-2) - gl.sum(dim=-1)
    grad_neg_log = grad_c.flip(-1).cumsum(-1).flip(-1)
    return (-grad_neg_log / (g + 1e-6)).to(decay_gamma.dtype), None


decay_matrix_op.register_autograd(_decay_backward, setup_context=_decay_setup)


def fused_decay_matrix(decay_gamma: Tensor, seq_len: int, block: int = 64) -> Tensor:
    """D[t,s] = exp(min(c_s - c_t, 0)) for s <= t else 0, c = cumsum(-log(gamma+1e-6)),
    gamma [N, T] -> [N, T, T] in gamma's dtype (v11/triton_kernels.py:570-573)."""
    if not decay_gamma.is_cuda:
        return _reference.on_cpu("triton_kernels.fused_decay_matrix", "fused_decay_matrix", decay_gamma, seq_len,
                                 block)
    if _use_hip:
        # a registered custom op (fake + autograd): torch.compile traces it as one node
        return decay_matrix_op(decay_gamma, seq_len).to(decay_gamma.dtype)
    return _pt_decay_matrix(decay_gamma, seq_len)


# ---------------------------------------------------------------- complex elementwise ops (HIP)

_NATIVE = {torch.float32: _lib.QPAM_F32, torch.bfloat16: _lib.QPAM_BF16}
_N_PARAMS = {_lib.QPAM_CPLX_NORM: 1, _lib.QPAM_CPLX_MOD_SWISH: 2, _lib.QPAM_CPLX_MOD_RELU: 1,
             _lib.QPAM_CPLX_CGU_GATE: 0}


def _cplx_args(op, z, up, p0, p1, eps):
    a = _lib.CplxArgs()
    a.op, a.dtype = op, _NATIVE[z.dtype]
    a.dim = z.shape[-2]
    a.rows = z.numel() // (2 * a.dim)
    a.eps = eps
    a.z, a.up, a.p0, a.p1 = _lib.ptr(z), _lib.ptr(up), _lib.ptr(p0), _lib.ptr(p1)
    return a


def _none_if_empty(t):
    return t if t.numel() else None


@torch.library.custom_op("qpam::cplx_fwd", mutates_args=())
def cplx_fwd_op(op: int, z: Tensor, up: Optional[Tensor], p0: Optional[Tensor], p1: Optional[Tensor],
                eps: float) -> Tensor:
    out = torch.empty_like(z)
    a = _cplx_args(op, z, up, p0, p1, eps)
    a.out = _lib.ptr(out)
    with torch.cuda.device(z.device):
        _lib.check(_lib.lib().qpam_cplx_fwd(ctypes.byref(a), _lib.stream_ptr(z.device)), "qpam_cplx_fwd")
    return out


@cplx_fwd_op.register_fake
def _(op, z, up, p0, p1, eps):
    return torch.empty_like(z)


@torch.library.custom_op("qpam::cplx_bwd", mutates_args=())
def cplx_bwd_op(op: int, z: Tensor, up: Optional[Tensor], p0: Optional[Tensor], p1: Optional[Tensor], eps: float,
                gout: Tensor) -> List[Tensor]:
    """[d z, d up, d p0, d p1]; the entries an op has no input for are empty."""
    gz = torch.empty_like(z)
    gup = torch.empty_like(up) if up is not None else z.new_empty(0)
    dim, np_ = z.shape[-2], _N_PARAMS[op]
    gp0 = torch.empty(dim, device=z.device, dtype=torch.float32) if np_ >= 1 else z.new_empty(0, dtype=torch.float32)
    gp1 = torch.empty(dim, device=z.device, dtype=torch.float32) if np_ >= 2 else z.new_empty(0, dtype=torch.float32)
    a = _cplx_args(op, z, up, p0, p1, eps)
    a.gout, a.gz = _lib.ptr(gout), _lib.ptr(gz)
    a.gup = _lib.ptr(gup if up is not None else None)
    a.gp0, a.gp1 = _lib.ptr(gp0 if np_ >= 1 else None), _lib.ptr(gp1 if np_ >= 2 else None)
    L = _lib.lib()
    ws = torch.empty(max(1, (L.qpam_cplx_workspace_size(ctypes.byref(a)) + 3) // 4), device=z.device,
                     dtype=torch.float32)
    a.workspace, a.workspace_bytes = _lib.ptr(ws), ws.numel() * 4
    with torch.cuda.device(z.device):
        _lib.check(L.qpam_cplx_bwd(ctypes.byref(a), _lib.stream_ptr(z.device)), "qpam_cplx_bwd")
    return [gz, gup, gp0, gp1]


@cplx_bwd_op.register_fake
def _(op, z, up, p0, p1, eps, gout):
    dim, np_ = z.shape[-2], _N_PARAMS[op]
    f32 = torch.float32
    return [torch.empty_like(z), torch.empty_like(up) if up is not None else z.new_empty(0),
            z.new_empty(dim if np_ >= 1 else 0, dtype=f32), z.new_empty(dim if np_ >= 2 else 0, dtype=f32)]


def _cplx_setup(ctx, inputs, output):
    op, z, up, p0, p1, eps = inputs
    ctx.op, ctx.eps = op, eps
    ctx.save_for_backward(z, up, p0, p1)


def _cplx_backward(ctx, gout):
    z, up, p0, p1 = ctx.saved_tensors
    gz, gup, gp0, gp1 = cplx_bwd_op(ctx.op, z, up, p0, p1, ctx.eps, gout.contiguous())
    return None, gz, _none_if_empty(gup), _none_if_empty(gp0), _none_if_empty(gp1), None


cplx_fwd_op.register_autograd(_cplx_backward, setup_context=_cplx_setup)


def _run_cplx(op, z, up=None, p0=None, p1=None, eps=0.0):
    if not z.is_cuda:
        raise ValueError("qpam complex ops: tensors must be on the GPU (no CPU path in this library)")
    if z.dim() < 2 or z.shape[-1] != 2:
        raise ValueError(f"qpam complex ops: expected [..., dim, 2], got {tuple(z.shape)}")
    dtype = z.dtype
    work = dtype if dtype in _NATIVE else torch.float32
    zc = z.to(work).contiguous()
    upc = up.to(work).contiguous() if up is not None else None
    if upc is not None and upc.shape != zc.shape:
        raise ValueError(f"qpam fused_cgu_gate: gate {tuple(zc.shape)} and up {tuple(upc.shape)} differ")
    dim = zc.shape[-2]
    prm = []
    for p in (p0, p1):
        if p is None:
            prm.append(None)
            continue
        if p.numel() != dim:
            raise ValueError(f"qpam complex ops: parameter of {p.numel()} entries for dim {dim}")
        prm.append(p.reshape(dim).to(torch.float32).contiguous())  # differentiable cast: grads return in p's dtype
    out = cplx_fwd_op(op, zc, upc, prm[0], prm[1], float(eps))
    return out if out.dtype == dtype else out.to(dtype)


def fused_complex_norm(z: Tensor, scale: Tensor, eps: float = 1e-6) -> Tensor:
    """ComplexNorm forward (v11/triton_kernels.py:48-79, backward :209-260)."""
    if not z.is_cuda:
        return _reference.on_cpu("triton_kernels.fused_complex_norm", "fused_complex_norm", z, scale, eps)
    if _use_hip:
        return _run_cplx(_lib.QPAM_CPLX_NORM, z, p0=scale, eps=eps)
    return _pt_complex_norm(z, scale, eps)


def fused_mod_swish(z: Tensor, bias: Tensor, beta: Tensor) -> Tensor:
    """ModSwish forward (v11/triton_kernels.py:83-108, backward :263-304)."""
    if not z.is_cuda:
        return _reference.on_cpu("triton_kernels.fused_mod_swish", "fused_mod_swish", z, bias, beta)
    if _use_hip:
        return _run_cplx(_lib.QPAM_CPLX_MOD_SWISH, z, p0=bias, p1=beta)
    return _pt_mod_swish(z, bias, beta)


def fused_mod_relu(z: Tensor, bias: Tensor) -> Tensor:
    """ModReLU forward (v11/triton_kernels.py:112-135, backward :307-345)."""
    if not z.is_cuda:
        return _reference.on_cpu("triton_kernels.fused_mod_relu", "fused_mod_relu", z, bias)
    if _use_hip:
        return _run_cplx(_lib.QPAM_CPLX_MOD_RELU, z, p0=bias)
    return _pt_mod_relu(z, bias)


def fused_cgu_gate(gate: Tensor, up: Tensor) -> Tensor:
    """CGU gate sigmoid(|g|) * phase(g) * up (v11/triton_kernels.py:139-166, backward :348-395)."""
    if not gate.is_cuda:
        return _reference.on_cpu("triton_kernels.fused_cgu_gate", "fused_cgu_gate", gate, up)
    if _use_hip:
        return _run_cplx(_lib.QPAM_CPLX_CGU_GATE, gate, up=up)
    return _pt_cgu_gate(gate, up)
