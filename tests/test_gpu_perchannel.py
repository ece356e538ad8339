"""GPU parity of the E1 per-channel chunked scan (qllm2_amd/pam_perchannel.py:
HIP fold and state-scan kernels around batched complex GEMMs) against the
oracle's restatement of V11PAMLayer._forward_chunked_perchannel
(oracle/pam.py: chunked_perchannel, pinned to the textbook per-channel
recurrence), float64 on the CPU: outputs, final state and the gradients of q,
k, v and gamma by float64 autograd of the oracle.  Shapes cover ragged last
chunks, head dims 16 / 64 / 96, chunks 16 / 24 / 64, decays strong enough that
the chunk's log-decay prefix reaches the -30 clamp, gammas under the 1e-6
floor, and bf16 inputs.  Bars: rel <= 1e-4 (fp32), 2e-2 (bf16), per (b, h)
slice relative to that slice's largest reference value."""

import pytest
import torch

from oracle import pam as O

pytestmark = pytest.mark.gpu

CASES = [  # (B, H, T, d, C, gamma regime)
    (2, 3, 100, 16, 24, "mild"),
    (1, 2, 130, 64, 64, "mild"),
    (1, 1, 70, 96, 16, "mild"),
    (2, 2, 96, 32, 32, "strong"),   # prefixes reach -30 inside a chunk
    (1, 2, 64, 16, 64, "tiny"),     # gammas below the 1e-6 floor
]


def _inputs(B, H, T, d, regime, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn(B, H, T, d, 2, generator=g, dtype=torch.float64) * (2 * d) ** -0.5 for _ in range(3))
    x = torch.randn(B, H, T, d, generator=g, dtype=torch.float64)
    if regime == "mild":
        gamma = torch.sigmoid(x + 3.0)
    elif regime == "strong":
        gamma = torch.sigmoid(x - 1.5)            # log gamma ~ -1.7 per step: -30 within ~18 steps
    else:
        gamma = torch.where(x > 0.5, torch.full_like(x, 3e-7), torch.sigmoid(x + 2.0))
    return q, k, v, gamma


def _rel(got, ref):
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    err = (got - ref).abs().flatten(2).max(-1).values
    scale = ref.abs().flatten(2).max(-1).values + 1e-30
    return (err / scale).max().item()


@pytest.mark.parametrize("B,H,T,d,C,regime", CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_perchannel_matches_oracle(gpu_lib, B, H, T, d, C, regime, dtype):
    from qllm2_amd.pam_perchannel import perchannel_chunked
    print(f"case B={B} H={H} T={T} d={d} C={C} {regime} {dtype}", flush=True)
    q, k, v, gamma = _inputs(B, H, T, d, regime, 900 + T + d)
    if dtype == torch.bfloat16:  # the oracle sees the rounded inputs
        q, k, v = (t.to(torch.bfloat16).double() for t in (q, k, v))
    gen = torch.Generator().manual_seed(901)
    dy = torch.randn(B, H, T, d, 2, generator=gen, dtype=torch.float64)
    ds = torch.randn(B, H, d, d, 2, generator=gen, dtype=torch.float64) * 0.1
    leaves_r = [t.clone().requires_grad_(True) for t in (q, k, v, gamma)]
    y_r, s_r = O.chunked_perchannel(*leaves_r, d, C)
    ((y_r * dy).sum() + (s_r * ds).sum()).backward()
    dev = torch.device("cuda")
    leaves = [q.to(dtype), k.to(dtype), v.to(dtype), gamma.float()]
    leaves = [t.to(dev).requires_grad_(True) for t in leaves]
    y, s = perchannel_chunked(*leaves, d, C)
    assert y.dtype == dtype and s.dtype == dtype
    ((y.float() * dy.float().to(dev)).sum() + (s.float() * ds.float().to(dev)).sum()).backward()
    torch.cuda.synchronize()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert _rel(y, y_r) < tol, f"y {_rel(y, y_r):.2e}"
    assert _rel(s, s_r) < tol, f"state {_rel(s, s_r):.2e}"
    for name, a, b in zip("qkvg", leaves, leaves_r):
        assert _rel(a.grad, b.grad) < tol, f"d{name} {_rel(a.grad, b.grad):.2e}"


def test_perchannel_deterministic(gpu_lib):
    """Two runs of forward + backward give bit-identical results."""
    from qllm2_amd.pam_perchannel import perchannel_chunked
    q, k, v, gamma = _inputs(2, 3, 200, 64, "mild", 77)
    dev = torch.device("cuda")
    outs = []
    for _ in range(2):
        leaves = [t.float().to(dev).requires_grad_(True) for t in (q, k, v, gamma)]
        y, s = perchannel_chunked(*leaves, 64, 64)
        (y.square().sum() + s.square().sum()).backward()
        outs.append([y.detach(), s.detach()] + [t.grad for t in leaves])
    torch.cuda.synchronize()
    for a, b in zip(*outs):
        assert torch.equal(a, b)
