"""GPU parity of the chunked scan forward (qpam_scan_fwd) against the CPU oracle.

Tolerances (north star): fp32 inputs rel <= 1e-4 on Y and S; bf16 inputs with
fp32 state rel <= 2e-2.  The oracle runs in float64 on the same (rounded)
inputs; for bf16 it consumes the bf16-rounded values.
"""

import math

import pytest
import torch

from oracle import pam as O

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return ((a.double() - b.double()).abs().max() / (b.double().abs().max() + 1e-30)).item()


def _rel_heads(a, b, lead):
    """Largest per-head relative error: max |a - b| / max |b| within each slice
    over the first `lead` dimensions ((b, h) for Y, (m, b, h) for S), then the
    max over slices."""
    a, b = a.double(), b.double()
    err = (a - b).abs().flatten(lead).amax(-1)
    ref = b.abs().flatten(lead).amax(-1)
    return (err / (ref + 1e-30)).max().item()


def _close(y, y_ref, s, s_ref, tol):
    """Y [B,H,T,d,2] and S [M,B,H,d,d,2]: whole-tensor and worst-head relative error."""
    assert _rel(y, y_ref) < tol, f"y rel {_rel(y, y_ref):.2e}"
    assert _rel_heads(y, y_ref, 2) < tol, f"y worst head rel {_rel_heads(y, y_ref, 2):.2e}"
    assert _rel(s, s_ref) < tol, f"s rel {_rel(s, s_ref):.2e}"
    assert _rel_heads(s, s_ref, 3) < tol, f"s worst head rel {_rel_heads(s, s_ref, 3):.2e}"


def _planes(x, dtype):
    return x[..., 0].contiguous().to(dtype).cuda(), x[..., 1].contiguous().to(dtype).cuda()


def _run(q, k, v, gamma, d, chunk, dtype=torch.float32, rot=None, s0=None):
    from qllm2_amd.pam_scan import pam_scan_planar
    qr, qi = _planes(q, dtype)
    kr, ki = _planes(k, dtype)
    vr, vi = _planes(v, dtype)
    rotp = (rot[0].float().cuda(), rot[1].float().cuda()) if rot is not None else None
    s0p = (s0[..., 0].float().cuda().contiguous(), s0[..., 1].float().cuda().contiguous()) if s0 is not None else None
    y_re, y_im, s_re, s_im = pam_scan_planar(qr, qi, kr, ki, vr, vi, gamma.float().cuda(), q_scale=d ** -0.5,
                                             chunk=chunk, rot=rotp, s0=s0p)
    torch.cuda.synchronize()
    return (torch.stack([y_re, y_im], -1).cpu(), torch.stack([s_re, s_im], -1).cpu())


def test_config1_parity_chunked_and_recurrent(gpu_lib):
    """Config 1: B=1, T=128, H=4, d=32, C=32, fp32; chunked oracle and the exact
    recurrence (which differs from the chunked form by the reference's +1e-6)."""
    B, H, T, d, C = 1, 4, 128, 32, 32
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 1001, qkv_std=1 / math.sqrt(2 * d), dtype=torch.float32)
    y, s = _run(q, k, v, gamma, d, C)
    y_ref, s_ref = O.chunked_head(q.double(), k.double(), v.double(), gamma[0].double(), d, C)
    assert _rel(y, y_ref) < 1e-4 and _rel(s[0], s_ref) < 1e-4
    yb, _ = O.brute_force_scan(O.to_complex(q), O.to_complex(k), O.to_complex(v), gamma[0].double().numpy(),
                               d ** -0.5)
    assert _rel(y, O.from_complex(yb)) < 1e-4


@pytest.mark.parametrize("T,C", [(64, 64), (200, 64), (100, 32), (70, 16), (2048, 64)])
def test_single_state_fp32(gpu_lib, T, C):
    B, H, d = 2, 3, 64
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 2000 + T + C, unit_qk=True, dtype=torch.float32)
    y, s = _run(q, k, v, gamma, d, C)
    y_ref, s_ref = O.chunked_head(q.double(), k.double(), v.double(), gamma[0].double(), d, C)
    assert _rel(y, y_ref) < 1e-4
    assert _rel(s[0], s_ref) < 1e-4


def test_multistate_rotation_and_initial_state_fp32(gpu_lib):
    M, B, H, T, d, C = 3, 2, 2, 150, 64, 64
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 31, m_states=M, gamma_mu=2.0, gamma_mu_step=1.0,
                                        unit_qk=True, dtype=torch.float32)
    g = torch.Generator().manual_seed(5)
    phase = torch.randn(M, B, H, T, generator=g)
    routing = torch.rand(M, B, H, T, generator=g) + 0.5
    s0 = torch.randn(M, B, H, d, d, 2, generator=g) * 0.1
    rot = (routing * torch.cos(phase), routing * torch.sin(phase))
    y, s = _run(q, k, v, gamma, d, C, rot=rot, s0=s0)
    y_ref, s_ref = O.multistate_fused(q.double(), k.double(), v.double(), gamma.double(), phase.double(),
                                      routing.double(), d, C, state=s0.double())
    _close(y, y_ref, s, s_ref, 1e-4)


def test_config2_full_size_fp32(gpu_lib):
    """Config 2: B=8, T=2048, H=12, d=64, C=64, unit-norm q,k, fp32 planar."""
    B, H, T, d, C = 8, 12, 2048, 64, 64
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 1002, unit_qk=True, dtype=torch.float32)
    y, s = _run(q, k, v, gamma, d, C)
    y_ref, s_ref = O.chunked_head(q.double(), k.double(), v.double(), gamma[0].double(), d, C)
    _close(y, y_ref, s, s_ref.unsqueeze(0), 1e-4)


def test_e3_bf16_inputs(gpu_lib):
    """Config-3 shape family (smaller B): M=3, bf16 q/k/v, fp32 state, rel 2e-2."""
    M, B, H, T, d, C = 3, 2, 2, 512, 64, 64
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 1003, m_states=M, gamma_mu=2.0, gamma_mu_step=1.0,
                                        unit_qk=True, dtype=torch.float32)
    qb, kb, vb = (x.to(torch.bfloat16) for x in (q, k, v))
    y, s = _run(qb, kb, vb, gamma, d, C, dtype=torch.bfloat16)
    ones, zeros = torch.ones_like(gamma), torch.zeros_like(gamma)
    y_ref, s_ref = O.multistate_fused(qb.double(), kb.double(), vb.double(), gamma.double(), zeros.double(),
                                      ones.double(), d, C)
    _close(y, y_ref, s, s_ref, 2e-2)


@pytest.mark.parametrize("B,T", [(2, 0), (0, 16)])
def test_empty_batch_or_sequence_raises(gpu_lib, B, T):
    """The reference's chunk loop concatenates an empty list at T = 0 and
    raises (v11/model.py:385, 417); the HIP scan rejects zero sizes with an
    error too, before any launch."""
    from qllm2_amd._lib import QpamError
    from qllm2_amd.pam_scan import pam_scan_planar

    def call(b, t):
        z = torch.zeros(b, 2, t, 64, device="cuda")
        return pam_scan_planar(z, z, z, z, z, z, torch.full((1, b, 2, t), 0.9, device="cuda"), q_scale=0.125,
                               chunk=16)

    y_re = call(2, 16)[0]  # the same arguments at a nonzero size are accepted
    assert y_re.shape == (2, 2, 16, 64)
    with pytest.raises((QpamError, ValueError, RuntimeError)):
        call(B, T)
    torch.cuda.synchronize()


def _rel_per_chain(a, b):
    """Max over (b, h) chains of that chain's max error over its max reference
    value: a chain with small values cannot hide behind another's scale."""
    a, b = a.double().flatten(0, 1).flatten(1), b.double().flatten(0, 1).flatten(1)
    return ((a - b).abs().max(1).values / (b.abs().max(1).values + 1e-30)).max().item()


@pytest.mark.parametrize("T,C,with_s0", [(64 * 37 + 13, 64, True), (64 * 37 + 13, 64, False), (40, 64, True),
                                         (64, 64, False), (32 * 9 + 5, 32, True), (16 * 7, 16, False)])
def test_fp32_state_pass_entering_states(gpu_lib, T, C, with_s0):
    """fp32, one state: the state pass (the carried state of each chain walking
    its chunks in registers) and the output kernel.  Y and the final state per
    (b, h) chain against the oracle (with an initial state through the fused-E3
    restatement, M = 1, no rotation), and the state entering every sampled chunk
    -- what the output kernel and the backward read -- against the oracle's
    state after that prefix."""
    from qllm2_amd import pam_scan
    B, H, d = 2, 3, 64
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 4100 + T, unit_qk=True, dtype=torch.float32)
    g = torch.Generator().manual_seed(4101)
    s0 = torch.randn(1, B, H, d, d, 2, generator=g) * 0.1 if with_s0 else None
    pl = [x[..., i].contiguous().cuda() for x in (q, k, v) for i in (0, 1)]
    s0p = (s0[..., 0].contiguous().cuda(), s0[..., 1].contiguous().cuda()) if with_s0 else (None, None)
    out = pam_scan.scan_fwd_op(*pl, gamma.cuda(), None, None, *s0p, d ** -0.5, C, 0)
    torch.cuda.synchronize()
    y = torch.stack([out[0], out[1]], -1).cpu()
    s = torch.stack([out[2], out[3]], -1).cpu()[0]
    ws = out[4]

    def oracle(t_end):
        zero = torch.zeros(1, B, H, t_end)
        return O.multistate_fused(q[:, :, :t_end].double(), k[:, :, :t_end].double(), v[:, :, :t_end].double(),
                                  gamma[:, :, :, :t_end].double(), zero.double(), (zero + 1).double(), d, C,
                                  state=s0.double() if with_s0 else None)

    y_ref, s_ref = oracle(T)
    assert _rel_per_chain(y, y_ref) < 1e-4, f"y {_rel_per_chain(y, y_ref):.2e}"
    assert _rel_per_chain(s, s_ref[0]) < 1e-4, f"s {_rel_per_chain(s, s_ref[0]):.2e}"
    n = (T + C - 1) // C
    states = ws[:B * H * n * 2 * d * d].view(B, H, n, 2, d, d).cpu()
    for c in sorted({1, 2, n // 2, n - 1} & set(range(1, n))):
        _, s_c = oracle(c * C)
        got = torch.stack([states[:, :, c, 0], states[:, :, c, 1]], -1)
        assert _rel_per_chain(got, s_c[0]) < 1e-4, f"entering state of chunk {c}"
    if with_s0:
        got = torch.stack([states[:, :, 0, 0], states[:, :, 0, 1]], -1)
        assert torch.equal(got, s0[0]), "the state entering chunk 0 is s0"
