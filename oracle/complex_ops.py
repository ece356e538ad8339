"""CPU restatement of the complex elementwise layers (test infrastructure only).

Split-real tensors [..., dim, 2] with |z| = sqrt(re^2 + im^2 + 1e-8), as the
reference's PyTorch forms (v11/triton_kernels.py:489-520; the same formulas as
ComplexNorm / ModSwish / ModReLU / CGU in v11/complex_ops.py):
  complex_norm  z / (|z| + 1e-8) * (|z| / rms) * scale,  rms = sqrt(mean_dim |z|^2 + eps)
  mod_swish     z / (|z| + 1e-8) * |z| * sigmoid(beta |z| + bias)
  mod_relu      z / (|z| + 1e-8) * relu(|z| + bias)
  cgu_gate      sigmoid(|g|) * (g / (|g| + 1e-8)) (x) up          (complex product)
  phase_mod     (z / (|z| + 1e-8)) (x) e^{i (alpha |z| + beta_ph)} * |z| * sigmoid(beta |z| + bias)
Gradients are torch autograd through these forms.  The *_backward functions
restate the closed forms of the reference's autograd Functions
(v11/triton_kernels.py:209-395) so that tests can check the two agree.
"""

import torch
import torch.nn.functional as F


def _mag(z):
    return torch.sqrt(z[..., 0].square() + z[..., 1].square() + 1e-8)


def complex_norm(z, scale, eps=1e-6):
    """v11/triton_kernels.py:489-494 (_pt_complex_norm)."""
    mag = _mag(z)
    rms = torch.sqrt(mag.square().mean(dim=-1, keepdim=True) + eps)
    return (z / (mag.unsqueeze(-1) + 1e-8)) * ((mag / rms) * scale).unsqueeze(-1)


def mod_swish(z, bias, beta):
    """v11/triton_kernels.py:497-501 (_pt_mod_swish)."""
    mag = _mag(z)
    return (z / (mag.unsqueeze(-1) + 1e-8)) * (mag * torch.sigmoid(beta * mag + bias)).unsqueeze(-1)


def mod_relu(z, bias):
    """v11/triton_kernels.py:504-508 (_pt_mod_relu)."""
    mag = _mag(z)
    return (z / (mag.unsqueeze(-1) + 1e-8)) * F.relu(mag + bias).unsqueeze(-1)


def phase_mod(z, bias, beta, phase_alpha, phase_beta):
    """PhaseModulatedActivation.forward (v11/complex_ops.py:135-143): ModSwish's
    magnitude; the unit phase z / (|z| + 1e-8) turned by the angle
    phase_alpha |z| + phase_beta (a complex product with (cos, sin))."""
    mag = _mag(z)
    act = mag * torch.sigmoid(beta * mag + bias)
    pr, pi = z[..., 0] / (mag + 1e-8), z[..., 1] / (mag + 1e-8)
    ang = phase_alpha * mag + phase_beta
    c, s = torch.cos(ang), torch.sin(ang)
    return torch.stack([(pr * c - pi * s) * act, (pr * s + pi * c) * act], dim=-1)


def cgu_gate(gate, up):
    """v11/triton_kernels.py:511-520 (_pt_cgu_gate)."""
    gmag = _mag(gate)
    gm = torch.sigmoid(gmag)
    pr, pi = gate[..., 0] / (gmag + 1e-8), gate[..., 1] / (gmag + 1e-8)
    ur, ui = up[..., 0], up[..., 1]
    return torch.stack([(pr * ur - pi * ui) * gm, (pr * ui + pi * ur) * gm], dim=-1)


def _batch_dims(z):
    return tuple(range(z.dim() - 2))


def complex_norm_backward(z, scale, gout, eps=1e-6):
    """Closed form of _FusedComplexNormFn.backward (v11/triton_kernels.py:230-260)."""
    zr, zi = z[..., 0], z[..., 1]
    mag = _mag(z)
    rms = torch.sqrt(mag.square().mean(dim=-1, keepdim=True) + eps)
    inv_mag, inv_rms = 1.0 / (mag + 1e-8), 1.0 / rms
    ur, ui = zr * inv_mag, zi * inv_mag
    smag = mag * inv_rms * scale
    gr, gi = gout[..., 0], gout[..., 1]
    gs = gr * ur + gi * ui
    g_scale = (gs * mag * inv_rms).sum(dim=_batch_dims(z))
    gnm = gs * scale
    gmag = gnm * inv_rms
    g_rms = -(gnm * mag * inv_rms * inv_rms).sum(-1, keepdim=True)
    gmag = gmag + g_rms * mag / (z.shape[-2] * rms)
    pr, pi = gr * smag, gi * smag
    dot = pr * ur + pi * ui
    gz = torch.stack([(pr - ur * dot) * inv_mag + gmag * zr / mag, (pi - ui * dot) * inv_mag + gmag * zi / mag], -1)
    return gz, g_scale


def mod_swish_backward(z, bias, beta, gout):
    """Closed form of _FusedModSwishFn.backward (v11/triton_kernels.py:280-304)."""
    zr, zi = z[..., 0], z[..., 1]
    mag = _mag(z)
    inv_mag = 1.0 / (mag + 1e-8)
    ur, ui = zr * inv_mag, zi * inv_mag
    sig = torch.sigmoid(beta * mag + bias)
    act = mag * sig
    gr, gi = gout[..., 0], gout[..., 1]
    da = gr * ur + gi * ui
    sd = sig * (1.0 - sig)
    dmag = da * (sig + mag * beta * sd)
    d_bias = (da * mag * sd).sum(dim=_batch_dims(z))
    d_beta = (da * mag * mag * sd).sum(dim=_batch_dims(z))
    pr, pi = gr * act, gi * act
    dot = pr * ur + pi * ui
    gz = torch.stack([(pr - ur * dot) * inv_mag + dmag * zr / mag, (pi - ui * dot) * inv_mag + dmag * zi / mag], -1)
    return gz, d_bias, d_beta


def mod_relu_backward(z, bias, gout):
    """Closed form of _FusedModReluFn.backward (v11/triton_kernels.py:322-345)."""
    zr, zi = z[..., 0], z[..., 1]
    mag = _mag(z)
    inv_mag = 1.0 / (mag + 1e-8)
    ur, ui = zr * inv_mag, zi * inv_mag
    act = F.relu(mag + bias)
    active = (mag + bias > 0).to(z.dtype)
    gr, gi = gout[..., 0], gout[..., 1]
    da = gr * ur + gi * ui
    dmag = da * active
    d_bias = dmag.sum(dim=_batch_dims(z))
    pr, pi = gr * act, gi * act
    dot = pr * ur + pi * ui
    gz = torch.stack([(pr - ur * dot) * inv_mag + dmag * zr / mag, (pi - ui * dot) * inv_mag + dmag * zi / mag], -1)
    return gz, d_bias


def cgu_gate_backward(gate, up, gout):
    """Closed form of _FusedCGUGateFn.backward (v11/triton_kernels.py:364-395)."""
    gr_, gi_ = gate[..., 0], gate[..., 1]
    ur, ui = up[..., 0], up[..., 1]
    dr, di = gout[..., 0], gout[..., 1]
    gmag = _mag(gate)
    gm = torch.sigmoid(gmag)
    inv = 1.0 / (gmag + 1e-8)
    pr, pi = gr_ * inv, gi_ * inv
    cr, ci = pr * ur - pi * ui, pr * ui + pi * ur
    dgm = (dr * cr + di * ci) * gm * (1.0 - gm)
    dcr, dci = dr * gm, di * gm
    d_up = torch.stack([dcr * pr + dci * pi, -dcr * pi + dci * pr], -1)
    dpr, dpi = dcr * ur + dci * ui, -dcr * ui + dci * ur
    dot = dpr * pr + dpi * pi
    d_gate = torch.stack([(dpr - pr * dot) * inv + dgm * gr_ / gmag, (dpi - pi * dot) * inv + dgm * gi_ / gmag], -1)
    return d_gate, d_up
