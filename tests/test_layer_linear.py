"""The fused layer's linear with the sliced weight gradient
(qllm2_amd/pam_layer.py: _linear_tall_k) against F.linear on the CPU.

The forward is F.linear itself; the backward's weight gradient is a sum of
per-slice products, so in float64 it equals F.linear's gradient to rounding,
and the input and bias gradients are the same products as F.linear's."""

import pytest
import torch
import torch.nn.functional as F

from qllm2_amd.pam_layer import _linear_tall_k


@pytest.mark.parametrize("shape,n_in,n_out,bias", [((8, 2048), 96, 48, True),     # sliced, gate-like
                                                    ((4, 1024), 64, 64, False),   # sliced, square
                                                    ((3, 333), 32, 8, True),      # rows do not split: plain
                                                    ((2, 64), 16, 1024, True)])   # many tiles: plain
def test_matches_f_linear_float64(shape, n_in, n_out, bias):
    g = torch.Generator().manual_seed(sum(shape) + n_in + n_out)
    x = torch.randn(*shape, n_in, generator=g, dtype=torch.float64, requires_grad=True)
    w = torch.randn(n_out, n_in, generator=g, dtype=torch.float64, requires_grad=True)
    b = torch.randn(n_out, generator=g, dtype=torch.float64, requires_grad=True) if bias else None
    dy = torch.randn(*shape, n_out, generator=g, dtype=torch.float64)
    ins = [x, w] + ([b] if bias else [])
    y = _linear_tall_k(x, w, b)
    ref = F.linear(x, w, b)
    assert torch.equal(y, ref)
    got = torch.autograd.grad(y, ins, dy)
    exp = torch.autograd.grad(ref, ins, dy)
    for a, e in zip(got, exp):
        assert a.shape == e.shape and a.is_contiguous()
        assert ((a - e).abs().max() / e.abs().max()).item() < 1e-13


def test_bf16_weight_gradient_within_bf16_rounding():
    """16-bit weights: partial products come back in bf16 and are summed in
    fp32; the result stays within bf16 rounding of the float64 product."""
    g = torch.Generator().manual_seed(7)
    x = torch.randn(16384, 96, generator=g)
    dy = torch.randn(16384, 48, generator=g)
    w = torch.randn(48, 96, generator=g)
    xb, wb = x.bfloat16().requires_grad_(True), w.bfloat16().requires_grad_(True)
    y = _linear_tall_k(xb, wb, None)
    (gw,) = torch.autograd.grad(y, [wb], dy.bfloat16())
    exact = dy.bfloat16().double().t() @ xb.detach().double()
    assert gw.dtype == torch.bfloat16
    assert ((gw.double() - exact).abs().max() / exact.abs().max()).item() < 2e-2
