"""GPU parity of the reference-API mirrors (flash_pam, triton_kernels,
pam_layer methods) against the CPU oracle.  The layer methods are exercised
through a minimal object that provides the attributes and prologue methods
the reference V11PAMLayer hands to them (chunk_size, n_states, gates)."""

import types

import pytest
import torch

from oracle import pam as O

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def test_fused_decay_matrix_forward_and_backward(gpu_lib):
    from qllm2_amd.triton_kernels import fused_decay_matrix
    g = torch.Generator().manual_seed(0)
    gamma = torch.sigmoid(torch.randn(6, 40, generator=g) + 2)
    gamma[0, 5] = 1.0  # a clamped entry (log(1 + 1e-6) > 0)
    up = torch.randn(6, 40, 40, generator=g)
    gc = gamma.cuda().requires_grad_(True)
    d = fused_decay_matrix(gc, 40)
    (d * up.cuda()).sum().backward()
    gr = gamma.double().requires_grad_(True)
    dr = O.decay_matrix(gr, 40)
    (dr * up.double()).sum().backward()
    assert _rel(d, dr) < 1e-5
    assert _rel(gc.grad, gr.grad) < 1e-4


def test_chunk_decay_matrices(gpu_lib):
    from qllm2_amd.flash_pam import _chunk_decay_matrices
    gamma = torch.sigmoid(torch.randn(5, 16, generator=torch.Generator().manual_seed(1)) + 3)
    got = _chunk_decay_matrices(gamma.cuda(), 16)
    ref = O.decay_matrices(gamma.double(), 16)
    for a, b in zip(got, ref):
        assert _rel(a, b) < 1e-5


def test_flash_pam_chunked_head(gpu_lib):
    from qllm2_amd.flash_pam import flash_pam_chunked_head
    B, H, T, d, C = 2, 3, 200, 64, 64
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 41, unit_qk=True)
    xs = [x.cuda().requires_grad_(True) for x in (q, k, v, gamma[0])]
    y, s = flash_pam_chunked_head(*xs, d, C)
    dy = torch.randn(B, H, T, d, 2, generator=torch.Generator().manual_seed(2))
    (y * dy.cuda()).sum().backward()
    rs = [x.double().requires_grad_(True) for x in (q, k, v, gamma[0])]
    yr, sr = O.flash_pam_chunked_head(*rs, d, C)
    (yr * dy.double()).sum().backward()
    assert _rel(y, yr) < 1e-4
    _, s_chunked = O.chunked_head(q.double(), k.double(), v.double(), gamma[0].double(), d, C)
    assert _rel(s, s_chunked) < 1e-4
    for a, b in zip(xs, rs):
        assert _rel(a.grad, b.grad) < 1e-4


def test_dual_form_block_and_chunked_head_methods(gpu_lib):
    from qllm2_amd import pam_layer as PL
    B, H, T, d = 1, 2, 48, 16
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 43)
    sq = q * d ** -0.5
    y, s = PL.dual_form_block(sq.cuda(), k.cuda(), v.cuda(), gamma[0].cuda(), None)
    yr, sr = O.dual_form_block(sq.double(), k.double(), v.double(), gamma[0].double())
    assert _rel(y, yr) < 1e-4 and _rel(s, sr) < 1e-4
    layer = types.SimpleNamespace(chunk_size=24)
    y2, s2 = PL.forward_chunked_head(layer, q.cuda(), k.cuda(), v.cuda(), gamma[0].cuda(), d)
    y2r, s2r = O.chunked_head(q.double(), k.double(), v.double(), gamma[0].double(), d, 24)
    assert _rel(y2, y2r) < 1e-4 and _rel(s2, s2r) < 1e-4


def test_fused_chunk_step_method(gpu_lib):
    from qllm2_amd import pam_layer as PL
    M, B, H, C, d = 3, 2, 2, 24, 16
    q, k, v, gamma = O.make_scan_inputs(B, H, C, d, 44, m_states=M, gamma_mu=2.0, gamma_mu_step=1.0)
    g = torch.Generator().manual_seed(3)
    phase, routing = torch.randn(M, B, H, C, generator=g), torch.rand(M, B, H, C, generator=g) + 0.5
    state = torch.randn(M, B, H, d, d, 2, generator=g) * 0.1
    sq = q * d ** -0.5
    for first in (True, False):
        st = torch.zeros_like(state) if first else state
        y, s = PL.fused_chunk_step(None, sq.cuda(), k.cuda(), v.cuda(), gamma.cuda(), phase.cuda(), routing.cuda(),
                                   st.cuda(), first)
        yr, sr = O.fused_chunk_step(sq.double(), k.double(), v.double(), gamma.double(), phase.double(),
                                    routing.double(), st.double(), first)
        assert _rel(y, yr) < 1e-4 and _rel(s, sr) < 1e-4


class _StandInLayer:
    """The attributes and prologue methods V11PAMLayer passes to the PAM math,
    returning precomputed per-token tensors (x[b, t, 0, 0] carries t)."""

    def __init__(self, gamma_all, phase, routing, values_scale, chunk):
        self.gamma_all, self.phase, self.routing, self.vs = gamma_all, phase, routing, values_scale
        self.chunk_size, self.n_states = chunk, gamma_all.shape[0]
        self.num_heads = gamma_all.shape[2]
        self.write_mode, self.decay_mode = 'additive', 'head'
        self.state_dt_offset = torch.arange(self.n_states, dtype=torch.float32)
        self._route_aux = None

    def _t(self, x):
        return x[:, :, 0, 0].long()[0]

    def _phase_and_alpha(self, x):
        t = self._t(x)
        return self.phase[..., t].permute(1, 3, 2, 0), self.routing[..., t].permute(1, 3, 2, 0)  # [B,T,H,K]

    def _route_balance_loss(self, r):
        return None

    def _gamma_all_and_vprime(self, x, values):
        return self.gamma_all, values * self.vs

    def _gamma_and_vprime(self, x, values, state_offset=0.0):
        t = self._t(x)
        m = int(round(float(state_offset)))
        return self.gamma_all[m][..., t], values * self.vs


def test_multistate_fused_and_recurrent_methods(gpu_lib):
    from qllm2_amd import pam_layer as PL
    M, B, H, T, d, C = 3, 2, 2, 40, 16, 16
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 45, m_states=M, gamma_mu=2.0, gamma_mu_step=1.0)
    g = torch.Generator().manual_seed(4)
    phase, routing = torch.randn(M, B, H, T, generator=g), torch.rand(M, B, H, T, generator=g) + 0.5
    x = torch.arange(T, dtype=torch.float32).view(1, T, 1, 1).expand(B, T, 1, 2).contiguous()
    layer = _StandInLayer(gamma.cuda(), phase.cuda(), routing.cuda(), 0.7, C)
    y, s = PL.forward_multistate_fused(layer, x.cuda(), q.cuda(), k.cuda(), v.cuda(), d)
    yr, sr = O.multistate_fused(q.double(), k.double(), (0.7 * v).double(), gamma.double(), phase.double(),
                                routing.double(), d, C)
    assert _rel(y, yr) < 1e-4 and _rel(s, sr) < 1e-4
    # recurrent token loop (decode path): no +1e-6 in the recurrence (v11/model.py:948-954)
    with torch.no_grad():
        y2, s2 = PL.recurrent(layer, x.cuda(), q.cuda(), k.cuda(), v.cuda(), None, d)
    y2r, s2r = O.recurrent(q.double(), k.double(), (0.7 * v).double(), gamma.double(), d, phase.double(),
                           routing.double())
    assert _rel(y2, y2r) < 1e-4 and _rel(s2, s2r) < 1e-4
