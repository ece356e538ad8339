"""Drop-in for the public API of v11/triton_kernels.py (no Triton inside).

fused_decay_matrix (v11/triton_kernels.py:570-573) runs the HIP decay-matrix
kernel (qpam_decay_matrix) for the forward; its backward is the reference's
closed form (v11/triton_kernels.py:447-480: grad_cum = column sums - row sums
of dD . D over the unclamped causal entries, reverse cumsum, divided by
-(gamma + 1e-6)).  The PAM scan kernels never call it: they rebuild D from
log-decay prefix sums in registers.

The complex elementwise ops (fused_complex_norm, fused_mod_swish,
fused_mod_relu, fused_cgu_gate) are outside the PAM scan / decode / CE hot
path; they keep the reference's PyTorch formulas (its `_pt_*` functions,
v11/triton_kernels.py:489-520) until their HIP kernels land.

set_triton_enabled / triton_enabled keep their names; they switch the HIP
decay-matrix forward on or off (off = the PyTorch formula).  HAS_TRITON is
False: this module has no Triton.
"""

import torch
import torch.nn.functional as F
from torch import Tensor

from . import _lib

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
    if decay_gamma.is_cuda and _use_hip and not torch.compiler.is_compiling():
        return decay_matrix_op(decay_gamma, seq_len).to(decay_gamma.dtype)
    if decay_gamma.is_cuda or torch.compiler.is_compiling():
        return _pt_decay_matrix(decay_gamma, seq_len)
    raise ValueError("qpam fused_decay_matrix: tensors must be on the GPU (no CPU path in this library)")


def fused_complex_norm(z: Tensor, scale: Tensor, eps: float = 1e-6) -> Tensor:
    return _pt_complex_norm(z, scale, eps)


def fused_mod_swish(z: Tensor, bias: Tensor, beta: Tensor) -> Tensor:
    return _pt_mod_swish(z, bias, beta)


def fused_mod_relu(z: Tensor, bias: Tensor) -> Tensor:
    return _pt_mod_relu(z, bias)


def fused_cgu_gate(gate: Tensor, up: Tensor) -> Tensor:
    return _pt_cgu_gate(gate, up)
