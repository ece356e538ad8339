"""CPU pins of the class-shaped V11PAMLayer restatement (oracle/v11_layer.py)
and of the E1 per-channel chunked form it needs:

  * chunked_perchannel == the textbook per-channel recurrence (complex128
    brute force), ragged chunks;
  * the class's prefill == the functional layer oracle (oracle/pam_layer.py,
    pinned in test_oracle_pam_layer.py) for the production modes;
  * parallel prefill == token-by-token decode through the class's own
    forward (the reference's v11/selftest.py:16-38 check) in every mode the
    self-test runs (v11/selftest.py:193-204: baseline, E1, E2, E3, E1+E3) plus
    the E3 K-loop, at the self-test's shape and bar (atol 2e-3 in float64);
  * fused E3 == K-loop to < 1e-10, output, state and input gradient
    (v11/selftest.py:65-99)."""

import pytest
import torch

from oracle import pam as O
from oracle import pam_layer as L
from oracle import v11_layer as V

MODES = {
    "baseline": {},
    "E1": dict(decay_mode="per_channel"),
    "E2": dict(write_mode="delta", delta_chunk=20),
    "E3": dict(n_states=2),
    "E3_loop": dict(n_states=2, fused_e3=False),
    "E1+E3": dict(decay_mode="per_channel", n_states=2),
}


def test_perchannel_chunked_matches_brute_force():
    g = torch.Generator().manual_seed(3)
    B, H, T, d, C = 2, 2, 45, 8, 16
    q, k, v = (torch.randn(B, H, T, d, 2, generator=g, dtype=torch.float64) for _ in range(3))
    gamma = 0.6 + 0.4 * torch.rand(B, H, T, d, generator=g, dtype=torch.float64)
    y, s = O.chunked_perchannel(q, k, v, gamma, d, C)
    y_ref, s_ref = O.brute_force_perchannel(O.to_complex(q), O.to_complex(k), O.to_complex(v), gamma.numpy(),
                                            d ** -0.5)
    # the reference takes the log-decay in fp32 (v11/model.py:433): ~1e-7 relative
    assert (O.to_complex(y) - y_ref).__abs__().max() / abs(y_ref).max() < 1e-5
    assert (O.to_complex(s) - s_ref).__abs__().max() / abs(s_ref).max() < 1e-5


def test_perchannel_decode_step_decays_key_columns():
    """_recur_step_additive with gamma [..., d]: column j of S decays by gamma_j."""
    g = torch.Generator().manual_seed(4)
    s = torch.randn(2, 3, 4, 4, 2, generator=g, dtype=torch.float64)
    gam = torch.rand(2, 3, 4, generator=g, dtype=torch.float64)
    zero = torch.zeros(2, 3, 4, 2, dtype=torch.float64)
    _, s1 = O.recur_step_additive(s, gam, zero, zero, zero)
    assert torch.equal(s1, s * gam[:, :, None, :, None])


@pytest.mark.parametrize("over", [dict(n_states=3), dict(n_states=1), dict(n_states=3, state_compete=True,
                                                                            routing_content_aware=True)])
def test_class_prefill_matches_functional_oracle(over):
    cfg = V.config(head_dim=16, chunk_size=24, **over)
    p = V.make_params(cfg, 11)
    layer = V.V11PAMLayer(cfg, p)
    x = torch.randn(2, 60, cfg["dim"], 2, generator=torch.Generator().manual_seed(12), dtype=torch.float64) * 0.5
    y, s = layer(x)
    y_ref, s_ref = L.layer_forward(p, cfg, x)
    assert (y - y_ref).abs().max() < 1e-12
    assert (s - s_ref).abs().max() < 1e-12


def run_mode(layer, x):
    """(parallel output, token-by-token output) of one layer, as v11/selftest.py:16-38."""
    with torch.no_grad():
        par, _ = layer(x, state=None, step_offset=0)
        outs, state = [], None
        for t in range(x.shape[1]):
            o, state = layer(x[:, t:t + 1], state=state, step_offset=t)
            outs.append(o)
    return par, torch.cat(outs, dim=1), state


@pytest.mark.parametrize("mode", list(MODES))
def test_class_parallel_equals_recurrent(mode):
    cfg = V.config(**MODES[mode])
    layer = V.V11PAMLayer(cfg, seed=20).eval()
    x = torch.randn(2, 80, cfg["dim"], 2, generator=torch.Generator().manual_seed(21), dtype=torch.float64) * 0.5
    par, rec, _ = run_mode(layer, x)
    diff = (par - rec).abs().max().item()
    assert diff < 2e-3, f"{mode}: max|diff| {diff:.2e}"
    assert diff / par.abs().max().item() < 1e-3


def test_class_fused_e3_equals_k_loop():
    cfg = V.config(n_states=3, gate_content_aware=True, head_dim=16, chunk_size=24)
    p = V.make_params(cfg, 30)
    fused = V.V11PAMLayer(cfg, p)
    loop = V.V11PAMLayer(dict(cfg, fused_e3=False), p)
    x = torch.randn(2, 80, cfg["dim"], 2, generator=torch.Generator().manual_seed(31), dtype=torch.float64) * 0.5
    x1, x2 = x.clone().requires_grad_(True), x.clone().requires_grad_(True)
    y1, s1 = fused(x1)
    y2, s2 = loop(x2)
    (y1 ** 2).sum().backward()
    (y2 ** 2).sum().backward()
    assert (y1 - y2).abs().max() < 1e-10
    assert (s1 - s2).abs().max() < 1e-10
    assert (x1.grad - x2.grad).abs().max() < 1e-10
