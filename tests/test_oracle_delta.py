"""Pins the CPU restatement of the E2 delta rule (oracle/delta.py).

The chunked UT-transform form is pinned against the reference's token
recurrence (_recur_step_delta run with the chunked form's gamma + 1e-6),
which is in turn pinned by closed-form properties of the delta rule: with
beta = 1 and orthonormal keys each write stores v exactly (S k = v), beta = 0
leaves a decayed state untouched, and the state is linear in the values for
fixed keys/gates."""

import pytest
import torch

from oracle import delta as D


@pytest.fixture(autouse=True)
def _f64():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


@pytest.mark.parametrize("T,C,with_state", [(40, 16, False), (64, 64, False), (70, 32, True), (9, 64, True)])
def test_chunked_equals_token_recurrence(T, C, with_state):
    q, k, v, g, b = D.make_delta_inputs(2, 2, T, 8, 100 + T + C)
    s0 = torch.randn(2, 2, 8, 8, 2, generator=torch.Generator().manual_seed(5)) * 0.3 if with_state else None
    y1, s1 = D.delta_chunked(q, k, v, g, b, 8, C, state=s0)
    y2, s2 = D.delta_recurrent(q, k, v, g, b, 8, state=s0)
    assert torch.allclose(y1, y2, atol=1e-9, rtol=1e-9)
    assert torch.allclose(s1, s2, atol=1e-9, rtol=1e-9)


def test_beta_one_orthonormal_keys_recall_exactly():
    """beta = 1, gamma ~ 1 (no decay): writing v_t under orthonormal keys makes
    S k_t = v_t for every stored t (the delta rule overwrites, the additive
    rule would sum)."""
    d, T = 8, 6
    qk = torch.linalg.qr(torch.randn(d, d, generator=torch.Generator().manual_seed(1)))[0]
    keys = torch.zeros(1, 1, T, d, 2)
    keys[0, 0, :, :, 0] = qk[:T]
    v = torch.randn(1, 1, T, d, 2, generator=torch.Generator().manual_seed(2))
    s = torch.zeros(1, 1, d, d, 2)
    for t in range(T):
        _, s = D.recur_step_delta(s, torch.ones(1, 1), v[:, :, t], keys[:, :, t], torch.zeros(1, 1, d, 2),
                                  torch.ones(1, 1))
    for t in range(T):
        sk_r = (s[..., 0] * keys[:, :, t, :, 0].unsqueeze(-2)).sum(-1)
        sk_i = (s[..., 1] * keys[:, :, t, :, 0].unsqueeze(-2)).sum(-1)
        assert torch.allclose(torch.stack([sk_r, sk_i], -1), v[:, :, t], atol=1e-12)
    # overwrite: a second write to key 0 replaces, not adds
    v2 = torch.randn(1, 1, d, 2, generator=torch.Generator().manual_seed(3))
    _, s = D.recur_step_delta(s, torch.ones(1, 1), v2, keys[:, :, 0], torch.zeros(1, 1, d, 2), torch.ones(1, 1))
    sk = torch.stack([(s[..., 0] * keys[:, :, 0, :, 0].unsqueeze(-2)).sum(-1),
                      (s[..., 1] * keys[:, :, 0, :, 0].unsqueeze(-2)).sum(-1)], -1)
    assert torch.allclose(sk, v2, atol=1e-12)


def test_beta_zero_only_decays_and_reads():
    q, k, v, g, _ = D.make_delta_inputs(1, 2, 12, 8, 7)
    s0 = torch.randn(1, 2, 8, 8, 2, generator=torch.Generator().manual_seed(8))
    y, s = D.delta_chunked(q, k, v, g, torch.zeros_like(g), 8, 4, state=s0)
    decay = torch.cumprod(g + D.EPS, dim=-1)
    assert torch.allclose(s, s0 * decay[..., -1, None, None, None], atol=1e-12)
    # y_t = decay_t S0 q~_t
    sq = torch.einsum("bhij,bhtj->bhti", torch.complex(s0[..., 0], s0[..., 1]),
                      torch.complex(q[..., 0], q[..., 1])) * 8 ** -0.5
    ref = sq * decay.unsqueeze(-1)
    assert torch.allclose(torch.complex(y[..., 0], y[..., 1]), ref, atol=1e-12)


def test_linear_in_values():
    q, k, v, g, b = D.make_delta_inputs(1, 1, 20, 8, 9)
    v2 = torch.randn(v.shape, generator=torch.Generator().manual_seed(10))
    y1, s1 = D.delta_chunked(q, k, v, g, b, 8, 8)
    y2, s2 = D.delta_chunked(q, k, v2, g, b, 8, 8)
    y3, s3 = D.delta_chunked(q, k, 2 * v - 3 * v2, g, b, 8, 8)
    assert torch.allclose(y3, 2 * y1 - 3 * y2, atol=1e-10) and torch.allclose(s3, 2 * s1 - 3 * s2, atol=1e-10)


def test_chunked_gradcheck():
    q, k, v, g, b = D.make_delta_inputs(1, 1, 6, 3, 11)
    xs = [x.clone().requires_grad_(True) for x in (q, k, v, g, b)]
    assert torch.autograd.gradcheck(lambda *a: D.delta_chunked(*a, 3, 4)[0], xs, eps=1e-6, atol=1e-6)


def test_chunked_form_edge_weights_closed_form():
    """Where the reference's chunked form departs from the token recurrence by
    construction (v11/model.py:508-510, 565-566), pinned by closed forms with
    orthonormal keys (then M = 0 and U = beta V):
    * strong decay: the state write weights u_s by alpha_last / (alpha_s + 1e-12),
      not alpha_last / alpha_s, once alpha_s (a prefix product of gamma + 1e-6)
      is near 1e-12;
    * gamma = 1: log(gamma + 1e-6) > 0, and the decay matrix clamps
      exp(min(L_t - L_s, 0)) to 1 where the recurrence grows by (1 + 1e-6)^(t-s)."""
    d, T = 8, 6
    qk = torch.linalg.qr(torch.randn(d, d, generator=torch.Generator().manual_seed(11)))[0]
    keys = torch.zeros(1, 1, T, d, 2)
    keys[0, 0, :, :, 0] = qk[:T]
    v = torch.randn(1, 1, T, d, 2, generator=torch.Generator().manual_seed(12))
    q = torch.randn(1, 1, T, d, 2, generator=torch.Generator().manual_seed(13))
    beta = torch.ones(1, 1, T)
    # strong decay: alpha runs 1e-3 .. 1e-18
    gamma = torch.full((1, 1, T), 1e-3)
    _, s = D.delta_chunked(q, keys, v, gamma, beta, d, 64)
    alpha = torch.cumprod(gamma[0, 0] + D.EPS, 0)
    tail = alpha[-1] / (alpha + 1e-12)
    want = torch.zeros(d, d, 2)
    for t in range(T):
        kt = keys[0, 0, t, :, 0]
        want[..., 0] += tail[t] * torch.outer(v[0, 0, t, :, 0], kt)
        want[..., 1] += tail[t] * torch.outer(v[0, 0, t, :, 1], kt)
    assert torch.allclose(s[0, 0], want, rtol=1e-10, atol=1e-300)
    exact = alpha[-1] / alpha
    assert (tail[4:] / exact[4:]).max() < 1e-2  # alpha_s <= 1e-15 there: the weights differ by construction
    # gamma = 1: y_t = q~_t . sum_{s <= t} (k_s* . q~_t) v_s with unit decay (clamped)
    gamma = torch.ones(1, 1, T)
    y, _ = D.delta_chunked(q, keys, v, gamma, beta, d, 64)
    qs = q[0, 0] * d ** -0.5
    for t in range(T):
        acc = torch.zeros(d, 2)
        for s_ in range(t + 1):
            w_r = (qs[t, :, 0] * keys[0, 0, s_, :, 0]).sum()  # keys are real here
            w_i = (qs[t, :, 1] * keys[0, 0, s_, :, 0]).sum()
            acc[:, 0] += w_r * v[0, 0, s_, :, 0] - w_i * v[0, 0, s_, :, 1]
            acc[:, 1] += w_r * v[0, 0, s_, :, 1] + w_i * v[0, 0, s_, :, 0]
        assert torch.allclose(y[0, 0, t], acc, rtol=1e-10, atol=1e-12)
