"""CPU checks of the scan wrapper's host-side decomposition (no GPU call).

pam_scan_planar takes any head dim and state count by handing the d = 64,
M <= 4 kernel op pieces of the problem: head dims below 64 zero-padded, head
dims above 64 as 64 x 64 state blocks run as extra heads, more than four states
in groups.  Here the kernel op is replaced by a float64 stand-in built on the
oracle (it checks that every piece it receives is a shape the kernels take),
so the reshapes, sums and concatenations are compared with the oracle at the
full shape, values and gradients.
"""

import pytest
import torch

from oracle import pam as O
from qllm2_amd import pam_scan


def _stand_in(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, q_scale, chunk,
              y_layout):
    assert q_re.shape[-1] == 64 and 1 <= gamma.shape[0] <= pam_scan.MAX_STATES and y_layout == 0
    M, B, H, T = gamma.shape
    q = torch.stack([q_re, q_im], -1) * (q_scale / 64 ** -0.5)  # the oracle scales by 64^-0.5
    k, v = torch.stack([k_re, k_im], -1), torch.stack([v_re, v_im], -1)
    if rot_re is None:
        phase, routing = gamma.new_zeros(M, B, H, T), gamma.new_ones(M, B, H, T)
    else:
        phase, routing = torch.atan2(rot_im, rot_re), torch.sqrt(rot_re ** 2 + rot_im ** 2)
    s0 = torch.stack([s0_re, s0_im], -1) if s0_re is not None else None
    y, s = O.multistate_fused(q, k, v, gamma, phase, routing, 64, chunk, state=s0)
    return [y[..., 0], y[..., 1], s[..., 0], s[..., 1], gamma.new_zeros(1)]


@pytest.fixture
def stand_in(monkeypatch):
    monkeypatch.setattr(pam_scan, "scan_fwd_op", _stand_in)


@pytest.mark.parametrize("M,d,with_rot,with_s0", [
    (1, 128, False, True), (2, 96, True, True), (1, 48, False, False), (6, 64, True, True),
    (5, 128, True, True), (9, 32, True, False),
])
def test_decomposition_matches_oracle(stand_in, M, d, with_rot, with_s0):
    B, H, T, C = 1, 2, 40, 16
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 90 + M + d, m_states=M, gamma_mu=2.0, gamma_mu_step=0.5,
                                        unit_qk=True, dtype=torch.float64)
    g = torch.Generator().manual_seed(91 + M + d)
    phase = torch.randn(M, B, H, T, generator=g, dtype=torch.float64)
    routing = torch.rand(M, B, H, T, generator=g, dtype=torch.float64) + 0.5
    if not with_rot:
        phase, routing = torch.zeros_like(phase), torch.ones_like(routing)
    s0 = torch.randn(M, B, H, d, d, 2, generator=g, dtype=torch.float64) * 0.1 if with_s0 else None
    dy = torch.randn(B, H, T, d, 2, generator=g, dtype=torch.float64)
    ds = torch.randn(M, B, H, d, d, 2, generator=g, dtype=torch.float64)

    leaves = [x.clone().requires_grad_(True) for x in (q, k, v, gamma, phase, routing)]
    s0l = s0.clone().requires_grad_(True) if s0 is not None else None
    y_ref, s_ref = O.multistate_fused(*leaves, d, C, state=s0l)
    ((y_ref * dy).sum() + (s_ref * ds).sum()).backward()
    ref_grads = [x.grad for x in leaves] + [s0l.grad if s0l is not None else None]

    ql, kl, vl, gl, pl, rl = [x.clone().requires_grad_(True) for x in (q, k, v, gamma, phase, routing)]
    s0p = None
    if s0 is not None:
        s0p = (s0[..., 0].clone().requires_grad_(True), s0[..., 1].clone().requires_grad_(True))
    rot = (rl * torch.cos(pl), rl * torch.sin(pl)) if with_rot else None
    y_re, y_im, s_re, s_im = pam_scan.pam_scan_planar(ql[..., 0], ql[..., 1], kl[..., 0], kl[..., 1], vl[..., 0],
                                                      vl[..., 1], gl, q_scale=d ** -0.5, chunk=C, rot=rot, s0=s0p)
    y, s = torch.stack([y_re, y_im], -1), torch.stack([s_re, s_im], -1)
    assert y.shape == y_ref.shape and s.shape == s_ref.shape
    assert torch.allclose(y, y_ref, rtol=0, atol=1e-10 * y_ref.abs().max().item())
    assert torch.allclose(s, s_ref, rtol=0, atol=1e-10 * s_ref.abs().max().item())
    ((y * dy).sum() + (s * ds).sum()).backward()
    got = [ql.grad, kl.grad, vl.grad, gl.grad]
    if with_rot:
        got += [pl.grad, rl.grad]
    got.append(torch.stack([s0p[0].grad, s0p[1].grad], -1) if s0p is not None else None)
    want = ref_grads[:4] + (ref_grads[4:6] if with_rot else []) + [ref_grads[6]]
    for a, b in zip(got, want):
        if b is None:
            assert a is None
            continue
        assert torch.allclose(a, b, rtol=0, atol=1e-9 * b.abs().max().item())


def test_state_groups_are_balanced(stand_in, monkeypatch):
    """Nine states run as three kernel calls of three states each (no call of one)."""
    sizes = []

    def counting(*args):
        sizes.append(args[6].shape[0])
        return _stand_in(*args)

    monkeypatch.setattr(pam_scan, "scan_fwd_op", counting)
    B, H, T, d, M = 1, 1, 8, 64, 9
    planes = [torch.randn(B, H, T, d, dtype=torch.float64) for _ in range(6)]
    gamma = torch.full((M, B, H, T), 0.9, dtype=torch.float64)
    pam_scan.pam_scan_planar(*planes, gamma, q_scale=0.125, chunk=16)
    assert sizes == [3, 3, 3]
