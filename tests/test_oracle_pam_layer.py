"""Pins the CPU restatement of the PAM layer forward (oracle/pam_layer.py)
against closed forms and against the layer's own token recurrence.

The prologue is pinned by closed forms of its scalar maps (exp(-softplus(x)) =
1/(1+e^x), the GSP blend, the gamma floor), ComplexLinear by complex128
matrix products, the RoPE placement by the relative-position property (the
layer's output does not depend on step_offset from a zero state), and the
whole prefill by the reference's decode path (the same projections and
prologue at positions step_offset + t, then the exact token recurrence).
"""

import pytest
import torch

from oracle import pam as O
from oracle import pam_layer as L


def _cfg(**kw):
    c = dict(n_heads=2, head_dim=8, n_states=3, chunk_size=16, use_rope=True, use_gsp=True, qk_norm=False,
             gamma_floor=0.0, gate_content_aware=False, routing_content_aware=False, state_compete=False,
             max_seq_len=64)
    c.update(kw)
    return c


def _c(z):
    return torch.complex(z[..., 0], z[..., 1])


def _x(b, t, dim, seed):
    return torch.randn(b, t, dim, 2, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


def test_prologue_scalar_closed_forms():
    """gamma = (1-p)/(1+e^pre) + p with pre = dt + dt_bias + offset_m and
    p = 1/(1+e^-protect); the floor maps base -> f + (1-f) base; v' = (1-p) v;
    no GSP leaves gamma = 1/(1+e^pre) and v unchanged."""
    g = torch.Generator().manual_seed(3)
    B, T, H, d, M = 2, 5, 3, 4, 3
    q, k, v = (torch.randn(B, T, H, d, 2, generator=g, dtype=torch.float64) for _ in range(3))
    dt = torch.randn(B, T, H, generator=g, dtype=torch.float64) * 4
    dt[0, 0, 0] = 30.0  # softplus threshold branch
    bias = torch.randn(H, generator=g, dtype=torch.float64)
    off = torch.tensor([-1.0, 0.0, 2.0], dtype=torch.float64)
    prot = torch.randn(B, T, H, generator=g, dtype=torch.float64)
    _, _, v2, gamma, rot = L.prologue(q, k, v, dt, bias, off, prot, None, None, None, 0, False, 0.0)
    pre = (dt + bias)[None] + off[:, None, None, None]                  # [M,B,T,H]
    p = 1 / (1 + torch.exp(-prot))
    ref = (1 - p) / (1 + torch.exp(pre)) + p
    assert torch.allclose(gamma, ref.permute(0, 1, 3, 2), rtol=1e-12, atol=1e-15)
    assert torch.allclose(v2, (v * (1 - p)[..., None, None]).transpose(1, 2), atol=1e-15)
    assert rot is None
    _, _, _, gf, _ = L.prologue(q, k, v, dt, bias, off, prot, None, None, None, 0, False, 0.9)
    base = 0.9 + 0.1 / (1 + torch.exp(pre))
    assert torch.allclose(gf, ((1 - p) * base + p).permute(0, 1, 3, 2), rtol=1e-12)
    _, _, v3, g3, _ = L.prologue(q, k, v, dt, bias, None, None, None, None, None, 0, False, 0.0)
    assert g3.shape == (1, B, H, T)
    assert torch.allclose(g3[0], (1 / (1 + torch.exp(dt + bias))).transpose(1, 2), rtol=1e-12, atol=1e-15)
    assert torch.equal(v3, v.transpose(1, 2))


def test_prologue_rope_and_norm():
    """q' = q e^{i (offset + t) theta_j}; with qk_norm every complex element of
    q', k' has modulus 1 and the phase of the rotated element."""
    g = torch.Generator().manual_seed(4)
    B, T, H, d = 1, 6, 2, 8
    q, k, v = (torch.randn(B, T, H, d, 2, generator=g, dtype=torch.float64) for _ in range(3))
    dt = torch.zeros(B, T, H, dtype=torch.float64)
    rope = O.rope_table(40, d)
    q2, k2, _, _, _ = L.prologue(q, k, v, dt, torch.zeros(H, dtype=torch.float64), None, None, None, None, rope, 9,
                                 False, 0.0)
    qc, rc = _c(q.transpose(1, 2)), _c(rope[9:9 + T])
    assert torch.allclose(_c(q2), qc * rc, atol=1e-14)
    q3, k3, _, _, _ = L.prologue(q, k, v, dt, torch.zeros(H, dtype=torch.float64), None, None, None, None, rope, 9,
                                 True, 0.0)
    z = _c(q3)
    assert torch.allclose(z.abs(), torch.ones_like(z.abs()), atol=1e-7)
    assert torch.allclose(torch.angle(z), torch.angle(qc * rc), atol=1e-9)


def test_complex_linear_is_complex_matmul():
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 4, 6, 2, generator=g, dtype=torch.float64)
    wr, wi = torch.randn(5, 6, generator=g, dtype=torch.float64), torch.randn(5, 6, generator=g, dtype=torch.float64)
    br, bi = torch.randn(5, generator=g, dtype=torch.float64), torch.randn(5, generator=g, dtype=torch.float64)
    got = _c(L.complex_linear(x, wr, wi, br, bi))
    ref = _c(x) @ torch.complex(wr, wi).T + torch.complex(br, bi)
    assert torch.allclose(got, ref, atol=1e-12)


@pytest.mark.parametrize("m,compete", [(3, False), (3, True), (1, False)])
def test_layer_output_independent_of_step_offset(m, compete):
    """RoPE rotates q and k by the same per-position phases and PAM reads
    q . k*, so from a zero state the layer's output depends on position
    differences only."""
    cfg = _cfg(n_states=m, state_compete=compete)
    p = L.make_layer_params(cfg, 6, 11 + m)
    x = _x(2, 40, 6, 12)
    y0, s0 = L.layer_forward(p, cfg, x, step_offset=0)
    y1, s1 = L.layer_forward(p, cfg, x, step_offset=23)
    assert torch.allclose(y0, y1, atol=1e-11)
    # the final state keeps the absolute phases of the keys, so it does move: the rotation is live
    assert not torch.allclose(s0, s1, atol=1e-6)


@pytest.mark.parametrize("m,compete,floor,qk_norm", [(3, True, 0.0, False), (2, False, 0.5, True),
                                                     (1, False, 0.0, False)])
def test_layer_prefill_equals_token_decode(m, compete, floor, qk_norm):
    """Chunked prefill (E3 fused or single-state chunked) against the
    reference's decode path run token by token with step_offset = t: same
    output and final state up to the (gamma + 1e-6) of the chunked form."""
    cfg = _cfg(n_states=m, state_compete=compete, gamma_floor=floor, qk_norm=qk_norm)
    p = L.make_layer_params(cfg, 6, 21 + m)
    x = _x(2, 37, 6, 22)
    y, s = L.layer_forward(p, cfg, x)
    st = None
    ys = []
    for t in range(x.shape[1]):
        yt, st = L.layer_decode(p, cfg, x[:, t:t + 1], t, st)
        ys.append(yt)
    yd = torch.cat(ys, 1)
    rel = ((y - yd).abs().max() / yd.abs().max()).item()
    assert rel < 1e-4, rel
    s = s if m > 1 else s.unsqueeze(0)
    assert ((s - st).abs().max() / st.abs().max()).item() < 1e-4
