"""GPU parity of the continuous-batching decode engine (qllm2_amd/engine.py)
against per-sequence float64 oracles.

Two stacked PAM layers (E3 with three states, GSP, state competition, gamma
floor; a one-state stack with qk-norm; at head dim 64, and E3 at 32 and one
state at 128, whose steps run the prologue kernel before the decode kernel)
decode five sequences that join and
leave on a pool of four slots (a leaving sequence's slot is reused), in an
unsorted live order, with prompts long enough to grow the pool's RoPE table.
Each sequence is prefilled on the GPU by the fused layer forward
(pam_layer.forward) and admitted with its per-layer states; every decoded
output and each sequence's states before it leaves are compared with the
oracle: V11PAMLayer.forward's prefill restatement (oracle/pam_layer.py
layer_forward) and its decode form (layer_decode) chained over the layers,
fp32 rel <= 1e-4; with bf16 GEMMs (the projection read by the prologue in
bf16, at head dims 64, 32 and 128) rel <= 5e-2: each decoded layer rounds to
bf16 six times (its input, the two GEMMs' weights, the projection, y and the
o_proj output, 2^-8 each), about 2.3e-2 to first order per layer, two layers."""

import pytest
import torch

from oracle import pam_layer as L
from oracle import v11_layer as V

pytestmark = pytest.mark.gpu

CFGS = {
    "e3": dict(dim=64, n_heads=2, head_dim=64, n_states=3, chunk_size=64, state_compete=True, gamma_floor=0.2),
    "one_state": dict(dim=64, n_heads=2, head_dim=64, n_states=1, chunk_size=64, qk_norm=True),
    "e3_hd32": dict(dim=64, n_heads=2, head_dim=32, n_states=2, chunk_size=32, state_compete=True),
    "hd128": dict(dim=128, n_heads=1, head_dim=128, n_states=1, chunk_size=64),
}
# (prompt length, join step, tokens decoded)
SEQS = [(5, 0, 5), (12, 0, 9), (3, 1, 4), (20, 3, 7), (8, 6, 5)]


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


@pytest.mark.parametrize("graphs", [False, True])
@pytest.mark.parametrize("name,dtype", [(n, torch.float32) for n in CFGS] +
                         [(n, torch.bfloat16) for n in ("e3", "e3_hd32", "hd128")])
def test_engine_matches_per_sequence_oracle(gpu_lib, name, dtype, graphs):
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
    engine = DecodeEngine(layers, n_slots=4, max_len=16, graphs=graphs, graph_bucket=2, dtype=dtype)
    tol = 1e-4 if dtype == torch.float32 else 5e-2
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
                    assert _rel(st, want) < tol, f"seq {si} layer {li} state {_rel(st, want):.2e}"
                engine.release(slot_of[si])
                done.add(si)
                del slot_of[si]
        step += 1
    assert engine.pool.rope.shape[0] > 16, "the RoPE table should have grown past its initial 16 rows"
    if graphs:
        assert len(engine._graphs) >= 2, "both buckets should have been captured"
    for si in range(len(SEQS)):
        out = torch.stack(got[si])
        assert _rel(out, ref_out[si]) < tol, f"seq {si}: {_rel(out, ref_out[si]):.2e}"


def test_engine_graph_replay_with_between_hook(gpu_lib):
    """A `between` hook (the model's own work between layers: here a residual
    scale and a per-feature gain, device work only) is captured into the graph
    with the layers: graph replays over changing live sets give the eager
    engine's outputs and states (rel 1e-6: the padded batches may run the GEMMs
    with other tilings)."""
    from qllm2_amd.engine import DecodeEngine
    cfg = V.config(**CFGS["e3"])
    dim = cfg["dim"]
    params = [V.make_params(cfg, 830 + i) for i in range(2)]
    layers = [V.V11PAMLayer(cfg, {k: v.float() for k, v in p.items()}, dtype=torch.float32).cuda().eval()
              for p in params]
    gain = torch.linspace(0.5, 1.5, dim, device="cuda").view(1, dim, 1)
    hook = (lambda li, out: out * gain + 0.1 * li)
    engines = [DecodeEngine(layers, n_slots=6, max_len=64, graphs=gr, graph_bucket=4) for gr in (False, True)]
    g = torch.Generator().manual_seed(831)
    for e in engines:
        for pos in (3, 9, 0, 5, 12):
            e.admit(pos)
    live_sets = [[0, 1, 2, 3, 4], [4, 2, 0], [1, 3], [0, 1, 2, 3, 4], [3, 1], [4, 2, 0]]
    for live in live_sets:
        x = torch.randn(len(live), dim, 2, generator=g).cuda()
        slots = torch.tensor(live, dtype=torch.int32, device="cuda")
        ys = [e.step(x, slots, between=hook, host_slots=live).clone() for e in engines]
        torch.cuda.synchronize()
        assert _rel(ys[1], ys[0]) < 1e-6, f"live {live}: {_rel(ys[1], ys[0]):.2e}"
    for slot in range(5):
        for li in range(2):
            a, b = (e.layer_state(li, slot) for e in engines)
            assert _rel(b, a) < 1e-6
    assert len(engines[1]._graphs) == 2  # buckets of 4 and 8 rows


def test_engine_graph_fresh_closure_each_step(gpu_lib):
    """A new `between` closure every step, each with its own gain (ids of freed
    closures are reused by CPython): every step runs its own closure's work, so
    the graph engine matches the eager engine step by step."""
    from qllm2_amd.engine import DecodeEngine
    cfg = V.config(**CFGS["e3"])
    dim = cfg["dim"]
    params = [V.make_params(cfg, 840 + i) for i in range(2)]
    layers = [V.V11PAMLayer(cfg, {k: v.float() for k, v in p.items()}, dtype=torch.float32).cuda().eval()
              for p in params]
    engines = [DecodeEngine(layers, n_slots=6, max_len=64, graphs=gr, graph_bucket=4) for gr in (False, True)]
    g = torch.Generator().manual_seed(841)
    for e in engines:
        for pos in (2, 7, 4):
            e.admit(pos)
    live = [0, 1, 2]
    for step in range(6):
        x = torch.randn(len(live), dim, 2, generator=g).cuda()
        slots = torch.tensor(live, dtype=torch.int32, device="cuda")
        ys = []
        for e in engines:
            scale = torch.full((1, dim, 1), 0.5 + 0.25 * step, device="cuda")
            ys.append(e.step(x, slots, between=(lambda li, out, s=scale: out * s), host_slots=live).clone())
        torch.cuda.synchronize()
        assert _rel(ys[1], ys[0]) < 1e-6, f"step {step}: {_rel(ys[1], ys[0]):.2e}"
