"""Pins the CPU PAM oracle against closed forms and brute-force recurrences.

The reference's own tests are self-consistency checks in float64
(v11/selftest.py:16-99, memory_probes/interference.py:158-225,
v11/bench_flash_pam.py:41-70); these tests restate them against independent
formulas so that a dropped term, a wrong sign or a transposed operand in the
oracle fails here.
"""

import math

import numpy as np
import pytest
import torch

from oracle import pam as O



@pytest.fixture(autouse=True)
def _float64_default():
    # the oracle pins run in float64; restore the default so other test modules are unaffected
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def _inputs(B, H, T, d, seed, **kw):
    return O.make_scan_inputs(B, H, T, d, seed, dtype=torch.float64, **kw)


def test_decay_matrices_closed_form():
    g = torch.Generator().manual_seed(0)
    for c in (1, 2, 5, 8):
        gamma = torch.sigmoid(torch.randn(3, c, generator=g) + 1.0)
        d_mat, cum, total, last = O.decay_matrices(gamma)
        ge = gamma + O.EPS
        for n in range(3):
            for t in range(c):
                assert math.isclose(cum[n, t].item(), torch.prod(ge[n, :t + 1]).item(), rel_tol=1e-12)
                for s in range(c):
                    want = torch.prod(ge[n, s + 1:t + 1]).item() if s <= t else 0.0
                    assert math.isclose(d_mat[n, t, s].item(), want, rel_tol=1e-12, abs_tol=1e-300)
            assert total[n].item() == cum[n, -1].item()
            assert torch.equal(last[n], d_mat[n, -1])


def test_decay_matrix_clamp_on_growth():
    # gamma = 1 makes log(gamma+1e-6) > 0: the clamp pins D to 1 (v11/flash_pam.py:49)
    gamma = torch.ones(1, 4)
    d_mat = O.decay_matrices(gamma)[0]
    assert torch.equal(d_mat[0], torch.tril(torch.ones(4, 4)))


def test_dual_form_block_vs_recurrence():
    q, k, v, gamma = _inputs(2, 3, 16, 8, 1)
    sq = q * 8 ** -0.5
    y, s = O.dual_form_block(sq, k, v, gamma[0])
    yb, sb = O.brute_force_scan(O.to_complex(q), O.to_complex(k), O.to_complex(v), gamma[0].numpy(),
                                8 ** -0.5, eps=O.EPS)
    np.testing.assert_allclose(O.to_complex(y), yb, rtol=0, atol=1e-12)
    np.testing.assert_allclose(O.to_complex(s), sb, rtol=0, atol=1e-12)


@pytest.mark.parametrize("T,C", [(128, 32), (80, 24), (64, 64), (17, 1), (40, 7)])
def test_chunked_head_vs_recurrence(T, C):
    B, H, d = 1, 4, 32 if T == 128 else 8
    q, k, v, gamma = _inputs(B, H, T, d, 1000 + T + C)
    y, s = O.chunked_head(q, k, v, gamma[0], d, C)
    yb, sb = O.brute_force_scan(O.to_complex(q), O.to_complex(k), O.to_complex(v), gamma[0].numpy(),
                                d ** -0.5, eps=O.EPS)
    scale = np.abs(yb).max()
    assert np.abs(O.to_complex(y) - yb).max() <= 1e-12 * scale
    assert np.abs(O.to_complex(s) - sb).max() <= 1e-12 * np.abs(sb).max()


def test_config1_chunked_vs_exact_recurrence_tolerance():
    """Config 1: chunked (with the reference's +1e-6) vs the exact recurrence.

    Each decay factor differs by 1e-6/gamma, so over the effective memory window
    1/(1-gamma) (gamma ~ sigmoid(3) = 0.95 -> ~20 steps) Y differs by
    ~20 * 1e-6 / 0.95 ~ 2e-5 relative, inside the rel 1e-4 bar."""
    B, H, T, d, C = 1, 4, 128, 32, 32
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 1001, qkv_std=1 / math.sqrt(2 * d), dtype=torch.float64)
    y, _ = O.chunked_head(q, k, v, gamma[0], d, C)
    yb, _ = O.brute_force_scan(O.to_complex(q), O.to_complex(k), O.to_complex(v), gamma[0].numpy(), d ** -0.5)
    rel = np.abs(O.to_complex(y) - yb).max() / np.abs(yb).max()
    assert rel < 1e-4
    assert rel > 1e-8  # the epsilon is really there


def test_gamma_one_is_causal_prefix_sum():
    B, H, T, d, C = 1, 2, 24, 4, 8
    q, k, v, _ = _inputs(B, H, T, d, 5)
    gamma = torch.ones(B, H, T)
    y, _ = O.chunked_head(q, k, v, gamma, d, C)
    qc, kc, vc = O.to_complex(q) * d ** -0.5, O.to_complex(k), O.to_complex(v)
    score = np.einsum('bhtj,bhsj->bhts', qc, np.conj(kc))
    # D is clamped at 1 when log(1+1e-6) > 0 (v11/flash_pam.py:49); cum is not
    d_intra = np.tril(np.ones((T, T)))
    want = np.zeros_like(qc)
    for c0 in range(0, T, C):
        for t in range(c0, c0 + C):
            acc = np.einsum('bhs,bhsi->bhi', score[:, :, t, c0:t + 1] * d_intra[t, c0:t + 1], vc[:, :, c0:t + 1])
            # carried part: previous chunks enter with cum factors (1+eps)^(pos in chunk + 1)
            if c0 > 0:
                # state after previous chunks, with the chunk totals (1+eps)^C and last-row D=1
                st = np.zeros((B, H, d, d), complex)
                for p0 in range(0, c0, C):
                    st = st * (1 + O.EPS) ** C + np.einsum('bhsi,bhsj->bhij', vc[:, :, p0:p0 + C],
                                                           np.conj(kc[:, :, p0:p0 + C]))
                acc = acc + (1 + O.EPS) ** (t - c0 + 1) * np.einsum('bhij,bhj->bhi', st, qc[:, :, t])
            want[:, :, t] = acc
    np.testing.assert_allclose(O.to_complex(y), want, rtol=0, atol=1e-11 * np.abs(want).max())


def test_flash_equals_chunked_ragged():
    B, H, T, d, C = 2, 2, 50, 8, 16
    q, k, v, gamma = _inputs(B, H, T, d, 7)
    y1, s1 = O.chunked_head(q, k, v, gamma[0], d, C)
    y2, s2 = O.flash_pam_chunked_head(q, k, v, gamma[0], d, C)
    assert (y1 - y2).abs().max() < 1e-12
    # the padded tail multiplies the final state by (1+1e-6)^pad and shifts decay_last by the same
    assert (s1 - s2).abs().max() < 1e-4 * s1.abs().max()
    y3, s3 = O.flash_pam_chunked_head(q[:, :, :48], k[:, :, :48], v[:, :, :48], gamma[0, :, :, :48], d, C)
    y4, s4 = O.chunked_head(q[:, :, :48], k[:, :, :48], v[:, :, :48], gamma[0, :, :, :48], d, C)
    assert (y3 - y4).abs().max() < 1e-12 and (s3 - s4).abs().max() < 1e-12


def _routing(M, B, H, T, seed):
    g = torch.Generator().manual_seed(seed)
    phase = torch.randn(M, B, H, T, generator=g)
    routing = torch.rand(M, B, H, T, generator=g) + 0.5
    return phase, routing


def test_multistate_fused_equals_loop_and_brute_force():
    M, B, H, T, d, C = 3, 2, 2, 40, 8, 16
    q, k, v, gamma = _inputs(B, H, T, d, 9, m_states=M, gamma_mu=2.0, gamma_mu_step=1.0)
    phase, routing = _routing(M, B, H, T, 3)
    y1, s1 = O.multistate_fused(q, k, v, gamma, phase, routing, d, C)
    y2, s2 = O.multistate_loop(q, k, v, gamma, phase, routing, d, C)
    assert (y1 - y2).abs().max() < 1e-10 and (s1 - s2).abs().max() < 1e-10
    want = 0
    for m in range(M):
        yb, sb = O.brute_force_scan(O.to_complex(q), O.to_complex(k), O.to_complex(v), gamma[m].numpy(),
                                    d ** -0.5, eps=O.EPS)
        r = routing[m].numpy() * np.exp(1j * phase[m].numpy())
        want = want + yb * r[..., None]
        np.testing.assert_allclose(O.to_complex(s1[m]), sb, atol=1e-11 * np.abs(sb).max(), rtol=0)
    np.testing.assert_allclose(O.to_complex(y1), want, atol=1e-11 * np.abs(want).max(), rtol=0)


def test_multistate_single_state_reduces_to_chunked():
    B, H, T, d, C = 1, 2, 33, 8, 8
    q, k, v, gamma = _inputs(B, H, T, d, 11)
    ones, zeros = torch.ones_like(gamma), torch.zeros_like(gamma)
    y1, s1 = O.multistate_fused(q, k, v, gamma, zeros, ones, d, C)
    y2, s2 = O.chunked_head(q, k, v, gamma[0], d, C)
    assert (y1 - y2).abs().max() < 1e-12 and (s1[0] - s2).abs().max() < 1e-12


def test_recurrent_matches_numpy_textbook_step():
    # memory_probes/core.py:92-101 + interference.py:206-223: S = g S + v (x) k*
    B, H, d = 2, 3, 6
    g = torch.Generator().manual_seed(2)
    s = torch.randn(B, H, d, d, 2, generator=g)
    v, k, q = (torch.randn(B, H, d, 2, generator=g) for _ in range(3))
    gam = torch.rand(B, H, generator=g)
    y, s2 = O.recur_step_additive(s, gam, v, k, q)
    sc, vc, kc, qc = O.to_complex(s), O.to_complex(v), O.to_complex(k), O.to_complex(q)
    want_s = gam.numpy()[..., None, None] * sc + vc[..., :, None] * np.conj(kc[..., None, :])
    np.testing.assert_allclose(O.to_complex(s2), want_s, atol=1e-13, rtol=0)
    np.testing.assert_allclose(O.to_complex(y), np.einsum('...ij,...j->...i', want_s, qc), atol=1e-12, rtol=0)


def test_recurrent_token_loop_vs_chunked_e3():
    M, B, H, T, d, C = 2, 1, 2, 20, 4, 8
    q, k, v, gamma = _inputs(B, H, T, d, 13, m_states=M)
    phase, routing = _routing(M, B, H, T, 4)
    y1, s1 = O.multistate_fused(q, k, v, gamma, phase, routing, d, C)
    y2, s2 = O.recurrent(q, k, v, gamma + O.EPS, d, phase, routing)
    assert (y1 - y2).abs().max() < 1e-11 * y1.abs().max()
    assert (s1 - s2).abs().max() < 1e-11 * s1.abs().max()


def test_decode_slots_matches_recurrent():
    S, G, M, d = 5, 3, 2, 4
    g = torch.Generator().manual_seed(8)
    state = torch.randn(S, G, M, d, d, 2, generator=g)
    q, k, v = (torch.randn(S, G, d, 2, generator=g) for _ in range(3))
    gamma = torch.rand(S, G, M, generator=g)
    rot = torch.randn(S, G, M, 2, generator=g)
    active = torch.tensor([4, 0, 2])
    y, st = O.decode_slots(state, active, q, k, v, gamma, 0.5, rot)
    for sl in range(S):
        if sl not in (0, 2, 4):
            assert torch.equal(st[sl], state[sl]) and torch.all(y[sl] == 0)
            continue
        # recurrent() with T=1, state layout [M,B=G,H=1,...]
        yy, ss = O.recurrent(q[sl][:, None, None], k[sl][:, None, None], v[sl][:, None, None],
                             gamma[sl].T[:, :, None, None], 4, None, None,
                             state=state[sl].transpose(0, 1)[:, :, None])
        del yy
        assert torch.allclose(st[sl].transpose(0, 1)[:, :, None], ss, atol=1e-13)
        acc = 0
        for m in range(M):
            ym, _ = O.recur_step_additive(state[sl, :, m], gamma[sl, :, m], v[sl], k[sl], q[sl] * 0.5)
            acc = acc + O.cmul(ym, rot[sl, :, m].unsqueeze(-2))
        assert torch.allclose(y[sl], acc, atol=1e-12)


def test_chunked_grads_gradcheck():
    B, H, T, d, C = 1, 1, 10, 3, 4
    q, k, v, gamma = _inputs(B, H, T, d, 21)
    args = [x.clone().requires_grad_(True) for x in (q, k, v, gamma[0])]
    assert torch.autograd.gradcheck(lambda a, b, c, g: O.chunked_head(a, b, c, g, d, C), args,
                                    eps=1e-6, atol=1e-6)


def test_multistate_grads_match_recurrence_autograd():
    """Autograd through the chunked E3 oracle == autograd through the token loop."""
    M, B, H, T, d, C = 3, 1, 2, 18, 4, 8
    q, k, v, gamma = _inputs(B, H, T, d, 23, m_states=M)
    phase, routing = _routing(M, B, H, T, 5)
    dy = torch.randn(B, H, T, d, 2, generator=torch.Generator().manual_seed(1))

    def grads(fn):
        xs = [x.clone().requires_grad_(True) for x in (q, k, v, gamma, phase, routing)]
        y, s = fn(*xs)
        (y * dy).sum().backward()
        return [x.grad for x in xs]

    g1 = grads(lambda a, b, c, g, p, r: O.multistate_fused(a, b, c, g, p, r, d, C))
    g2 = grads(lambda a, b, c, g, p, r: O.recurrent(a, b, c, g + O.EPS, d, p, r))
    for a, b in zip(g1, g2):
        assert (a - b).abs().max() <= 1e-10 * (b.abs().max() + 1e-30)


def test_rope_table_closed_form():
    """RoPE table: rope[0] = 1, unit modulus, band 0 turns 1 rad per position,
    band d/2 turns 10000^(-1/2) = 0.01 rad, and rope[a + b] = rope[a] * rope[b]
    (angles linear in the position)."""
    d, P = 64, 300
    r = O.rope_table(P, d)
    assert torch.allclose(r[0], torch.stack([torch.ones(d), torch.zeros(d)], -1), atol=0)
    assert torch.allclose(r.square().sum(-1), torch.ones(P, d), atol=1e-14)
    m = torch.arange(P, dtype=torch.float64)
    assert torch.allclose(r[:, 0, 0], torch.cos(m)) and torch.allclose(r[:, 0, 1], torch.sin(m))
    assert torch.allclose(r[:, d // 2, 1], torch.sin(0.01 * m), atol=1e-13)
    for a, b in ((3, 5), (17, 200), (0, 99)):
        assert torch.allclose(r[a + b], O.cmul(r[a], r[b]), atol=1e-12)


def test_build_rope_cache_matches_table():
    """The library's fp32 table (computed as the reference does, in fp32) against
    the float64 closed form: angle error bounded by fp32 rounding of m * theta."""
    from qllm2_amd.decode import build_rope_cache
    P, d = 4096, 64
    got = build_rope_cache(P, d)
    assert got.dtype == torch.float32 and tuple(got.shape) == (P, d, 2)
    ref = O.rope_table(P, d)
    assert (got.double() - ref).abs().max() < 2e-3
    assert (got.double()[:64] - ref[:64]).abs().max() < 1e-5


def test_decode_rope_is_relative():
    """PAM reads S q with S = sum gamma^.. v k*: with q and k rotated by the same
    per-position phases the output depends only on position differences, so
    decoding a sequence at offset 0 and at offset 37 gives the same outputs
    from a zero state.  A rotation of only q (or a missing conjugate on k)
    breaks this.  Position 0 is the identity rotation."""
    S, G, M, d, T = 2, 3, 2, 8, 6
    g = torch.Generator().manual_seed(21)
    rope = O.rope_table(64, d)
    seq = [tuple(torch.randn(S, G, d, 2, generator=g) for _ in range(3)) for _ in range(T)]
    gamma = torch.rand(S, G, M, generator=g)
    rot = torch.randn(S, G, M, 2, generator=g)
    active = torch.arange(S)

    def run(off, q_only=False):
        st = torch.zeros(S, G, M, d, d, 2)
        ys = []
        for t, (q, k, v) in enumerate(seq):
            if q_only:
                y, st = O.decode_slots(st, active, O.cmul(q, rope[off + t]), k, v, gamma, 0.3, rot)
            else:
                y, st = O.decode_slots(st, active, q, k, v, gamma, 0.3, rot, rope=rope, pos=torch.full((S,), off + t))
            ys.append(y)
        return torch.stack(ys)

    assert torch.allclose(run(0), run(37), atol=1e-12)
    assert not torch.allclose(run(0, True), run(37, True), atol=1e-3)
    st0 = torch.randn(S, G, M, d, d, 2, generator=g)
    q, k, v = seq[0]
    a = O.decode_slots(st0, active, q, k, v, gamma, 0.3, rot, rope=rope, pos=torch.zeros(S, dtype=torch.long))
    b = O.decode_slots(st0, active, q, k, v, gamma, 0.3, rot)
    assert torch.allclose(a[0], b[0], atol=1e-14) and torch.allclose(a[1], b[1], atol=1e-14)
