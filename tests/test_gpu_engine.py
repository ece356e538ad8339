"""GPU parity of the continuous-batching decode engine (qllm2_amd/engine.py)
against per-sequence float64 oracles.

Two stacked PAM layers (E3 with three states, GSP, state competition, gamma
floor; and a one-state stack with qk-norm) decode five sequences that join and
leave on a pool of four slots (a leaving sequence's slot is reused), in an
unsorted live order, with prompts long enough to grow the pool's RoPE table.
Each sequence is prefilled on the GPU by the fused layer forward
(pam_layer.forward) and admitted with its per-layer states; every decoded
output and each sequence's states before it leaves are compared with the
oracle: V11PAMLayer.forward's prefill restatement (oracle/pam_layer.py
layer_forward) and its decode form (layer_decode) chained over the layers,
fp32 rel <= 1e-4."""

import pytest
import torch

from oracle import pam_layer as L
from oracle import v11_layer as V

pytestmark = pytest.mark.gpu

CFGS = {
    "e3": dict(dim=64, n_heads=2, head_dim=64, n_states=3, chunk_size=64, state_compete=True, gamma_floor=0.2),
    "one_state": dict(dim=64, n_heads=2, head_dim=64, n_states=1, chunk_size=64, qk_norm=True),
}
# (prompt length, join step, tokens decoded)
SEQS = [(5, 0, 5), (12, 0, 9), (3, 1, 4), (20, 3, 7), (8, 6, 5)]


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


@pytest.mark.parametrize("graphs", [False, True])
@pytest.mark.parametrize("name", list(CFGS))
def test_engine_matches_per_sequence_oracle(gpu_lib, name, graphs):
    """Eager steps, and HIP-graph replays (graph_bucket 2: odd live counts pad
    one row onto a scratch slot; each bucket is captured on its first step and
    replayed on later ones, with admissions, releases and a RoPE-table growth
    in between)."""
    from qllm2_amd import pam_layer
    from qllm2_amd.engine import DecodeEngine
    cfg = V.config(**CFGS[name])
    n_layers, dim = 2, cfg["dim"]
    params = [V.make_params(cfg, 800 + i) for i in range(n_layers)]
    layers = [V.V11PAMLayer(cfg, {k: v.float() for k, v in p.items()}, dtype=torch.float32).cuda().eval()
              for p in params]
    engine = DecodeEngine(layers, n_slots=4, max_len=16, graphs=graphs, graph_bucket=2)
    g = torch.Generator().manual_seed(810)
    prompts = [torch.randn(1, t, dim, 2, generator=g, dtype=torch.float64) * 0.5 for t, _, _ in SEQS]
    tokens = [torch.randn(n, dim, 2, generator=g, dtype=torch.float64) * 0.5 for _, _, n in SEQS]

    # oracle, per sequence: prefill then token decode, chained over the layers
    ref_out, ref_state = [], []
    for (t0, _, n), xp, xt in zip(SEQS, prompts, tokens):
        states, x = [], xp
        for p in params:
            x, s = L.layer_forward(p, cfg, x)
            states.append(s if cfg["n_states"] > 1 else s.unsqueeze(0))    # [M, B, H, d, d, 2]
        outs = []
        for i in range(n):
            x = xt[i].view(1, 1, dim, 2)
            for li, p in enumerate(params):
                x, states[li] = L.layer_decode(p, cfg, x, t0 + i, states[li])
            outs.append(x[0, 0])
        ref_out.append(torch.stack(outs))
        ref_state.append(states)

    slot_of, done, got = {}, set(), [[] for _ in SEQS]
    step = 0
    while len(done) < len(SEQS):
        for si, (t0, join, n) in enumerate(SEQS):
            if join == step:
                with torch.no_grad():       # prefill on the GPU: the fused layer forward
                    x, states = prompts[si].float().cuda(), []
                    for layer in layers:
                        x, s = pam_layer.forward(layer, x, None, 0)
                        states.append(s)
                slot_of[si] = engine.admit(t0, states)
        live = [si for si in sorted(slot_of, reverse=True) if si not in done]
        slots = torch.tensor([slot_of[si] for si in live], dtype=torch.int32, device="cuda")
        x = torch.stack([tokens[si][len(got[si])] for si in live]).float().cuda()
        y = engine.step(x, slots)
        for row, si in enumerate(live):
            got[si].append(y[row].cpu())
            if len(got[si]) == SEQS[si][2]:
                for li in range(n_layers):
                    st = engine.layer_state(li, slot_of[si]).reshape(-1)
                    want = ref_state[si][li].reshape(-1)
                    assert _rel(st, want) < 1e-4, f"seq {si} layer {li} state {_rel(st, want):.2e}"
                engine.release(slot_of[si])
                done.add(si)
                del slot_of[si]
        step += 1
    assert engine.pool.rope.shape[0] > 16, "the RoPE table should have grown past its initial 16 rows"
    if graphs:
        assert len(engine._graphs) >= 2, "both buckets should have been captured"
    for si in range(len(SEQS)):
        out = torch.stack(got[si])
        assert _rel(out, ref_out[si]) < 1e-4, f"seq {si}: {_rel(out, ref_out[si]):.2e}"
