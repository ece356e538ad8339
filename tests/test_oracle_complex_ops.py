"""Pins the CPU restatement of the complex elementwise layers (oracle/complex_ops.py)
by what the mathematics fixes — phase preservation, RMS normalisation, the relu
threshold, the swish limits, complex-product phases — and checks that the
restated closed-form backward formulas of the reference's autograd Functions
agree with autograd of the forward forms (fp64)."""

import math

import pytest
import torch

from oracle import complex_ops as O


def _z(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, 2, generator=g, dtype=torch.float64) * scale


def _angle(z):
    return torch.atan2(z[..., 1], z[..., 0])


def _abs(z):
    return torch.sqrt(z[..., 0] ** 2 + z[..., 1] ** 2)


def _wrap(a):
    return torch.remainder(a + math.pi, 2 * math.pi) - math.pi


def test_complex_norm_preserves_phase_and_normalises_rms():
    z = _z((5, 7, 48), 1)
    out = O.complex_norm(z, torch.ones(48, dtype=torch.float64), eps=0.0)
    assert _wrap(_angle(out) - _angle(z)).abs().max() < 1e-12
    # unit RMS magnitude over the feature axis (up to the 1e-8 terms)
    rms = _abs(out).square().mean(-1).sqrt()
    assert (rms - 1).abs().max() < 1e-6
    # a per-feature scale multiplies the magnitudes
    s = torch.linspace(0.5, 2.0, 48, dtype=torch.float64)
    out2 = O.complex_norm(z, s, eps=0.0)
    assert torch.allclose(_abs(out2), _abs(out) * s, rtol=1e-12, atol=0)


def test_mod_relu_threshold_and_phase():
    z = _z((3, 64), 2)
    b = torch.full((64,), -0.7, dtype=torch.float64)
    out = O.mod_relu(z, b)
    small = _abs(z) < 0.7 - 1e-6
    assert torch.all(out[small] == 0)
    big = _abs(z) > 0.7 + 1e-6
    assert torch.allclose(_abs(out)[big], (_abs(z) - 0.7)[big], rtol=1e-6)
    assert _wrap(_angle(out) - _angle(z))[big].abs().max() < 1e-12


def test_mod_swish_limits():
    z = _z((4, 32), 3)
    zero = torch.zeros(32, dtype=torch.float64)
    # beta = 0, bias = 0: sigmoid(0) = 1/2 on the magnitude
    assert torch.allclose(O.mod_swish(z, zero, zero), z * 0.5, rtol=1e-6, atol=1e-9)
    # very large bias: the gate opens fully
    assert torch.allclose(O.mod_swish(z, zero + 60.0, zero), z, rtol=1e-6, atol=1e-9)


def test_cgu_gate_is_a_phase_rotation_times_sigmoid_magnitude():
    g, u = _z((6, 40), 4), _z((6, 40), 5)
    out = O.cgu_gate(g, u)
    assert torch.allclose(_abs(out), torch.sigmoid(_abs(g)) * _abs(u), rtol=1e-5)  # 1e-8 terms of |g|
    assert _wrap(_angle(out) - _angle(g) - _angle(u)).abs().max() < 1e-9


def test_phase_mod_is_mod_swish_turned_by_its_angle():
    """The phase-modulated activation keeps ModSwish's magnitude and turns its
    phase by alpha |z| + beta_ph: with both phase parameters zero it is ModSwish
    exactly; otherwise the magnitudes agree and the angle difference is
    alpha |z| + beta_ph (|z| with its 1e-8 term), checked against complex128
    polar arithmetic."""
    z = _z((5, 48), 11)
    g = torch.Generator().manual_seed(12)
    bias, beta = torch.randn(48, generator=g, dtype=torch.float64) * 0.3, 1 + torch.randn(48, generator=g, dtype=torch.float64) * 0.2
    pa, pb = torch.randn(48, generator=g, dtype=torch.float64), torch.randn(48, generator=g, dtype=torch.float64) * 2
    zero = torch.zeros(48, dtype=torch.float64)
    assert torch.equal(O.phase_mod(z, bias, beta, zero, zero), O.mod_swish(z, bias, beta))
    out = O.phase_mod(z, bias, beta, pa, pb)
    sw = O.mod_swish(z, bias, beta)
    assert torch.allclose(_abs(out), _abs(sw), rtol=1e-12, atol=0)
    mag = torch.sqrt(_abs(z) ** 2 + 1e-8)
    assert _wrap(_angle(out) - _angle(z) - (pa * mag + pb)).abs().max() < 1e-9
    want = torch.complex(sw[..., 0], sw[..., 1]) * torch.polar(torch.ones_like(mag), pa * mag + pb)
    assert torch.allclose(torch.view_as_real(want), out, rtol=0, atol=1e-12)


@pytest.mark.parametrize("name", ["norm", "swish", "relu", "cgu"])
def test_closed_form_backward_matches_autograd(name):
    torch.manual_seed(7)
    z = _z((3, 5, 24), 8).requires_grad_(True)
    gout = _z((3, 5, 24), 9)
    if name == "norm":
        p = torch.linspace(0.5, 1.5, 24, dtype=torch.float64).requires_grad_(True)
        O.complex_norm(z, p).backward(gout)
        gz, gp = O.complex_norm_backward(z.detach(), p.detach(), gout)
        pairs = [(gz, z.grad), (gp, p.grad)]
    elif name == "swish":
        b = torch.linspace(-1, 1, 24, dtype=torch.float64).requires_grad_(True)
        be = torch.linspace(0.2, 2, 24, dtype=torch.float64).requires_grad_(True)
        O.mod_swish(z, b, be).backward(gout)
        gz, gb, gbe = O.mod_swish_backward(z.detach(), b.detach(), be.detach(), gout)
        pairs = [(gz, z.grad), (gb, b.grad), (gbe, be.grad)]
    elif name == "relu":
        b = torch.linspace(-1, 0.5, 24, dtype=torch.float64).requires_grad_(True)
        O.mod_relu(z, b).backward(gout)
        gz, gb = O.mod_relu_backward(z.detach(), b.detach(), gout)
        pairs = [(gz, z.grad), (gb, b.grad)]
    else:
        u = _z((3, 5, 24), 10).requires_grad_(True)
        O.cgu_gate(z, u).backward(gout)
        gz, gu = O.cgu_gate_backward(z.detach(), u.detach(), gout)
        pairs = [(gz, z.grad), (gu, u.grad)]
    for a, b in pairs:
        assert (a - b).abs().max() <= 1e-6 * b.abs().max()


def test_forms_pass_gradcheck():
    z = _z((2, 6), 11).requires_grad_(True)
    p = torch.linspace(0.3, 1.3, 6, dtype=torch.float64).requires_grad_(True)
    q = torch.linspace(0.5, 1.5, 6, dtype=torch.float64).requires_grad_(True)
    u = _z((2, 6), 12).requires_grad_(True)
    assert torch.autograd.gradcheck(lambda a, b: O.complex_norm(a, b), (z, p))
    assert torch.autograd.gradcheck(lambda a, b, c: O.mod_swish(a, b, c), (z, p, q))
    assert torch.autograd.gradcheck(lambda a, b: O.mod_relu(a, b), (z, p - 1.0))
    assert torch.autograd.gradcheck(lambda a, b: O.cgu_gate(a, b), (z, u))
