"""GPU parity of the model-level decoder (qllm2_amd/model_decode.py) against
the float64 oracle model (oracle/v11_model.py V11LM: embedding, blocks of
ComplexNorm -> CGU -> residual -> ComplexNorm -> PAM -> residual, output norm,
LM-head projection and norm, tied logits).

Two blocks decode five sequences that join and leave on four slots (a leaving
sequence's slot is reused), in an unsorted live order, with prompts long
enough to grow the pool's RoPE table; each sequence is admitted with its
prompt's prefill (the fused PAM prefill on the GPU) and fed fixed
continuation tokens.  The logits of the prompt's last token and of every
decoded token are compared with the oracle's per-sequence prefill + decode,
per row relative to the row's largest logit: fp32 GEMMs rel <= 1e-4; bf16
GEMMs (bf16 weights and inputs, fp32 accumulation, 7 GEMMs per block) rel <=
3e-2.  Eager steps and HIP-graph replays (bucket 2)."""

import pytest
import torch

from oracle import v11_model as VM

pytestmark = pytest.mark.gpu

CFGS = {
    "e3_swish": (dict(dim=128, n_heads=2, head_dim=64, n_states=3, chunk_size=64, state_compete=True,
                      gamma_floor=0.2), "swish"),
    "one_state_relu": (dict(dim=128, n_heads=2, head_dim=64, n_states=1, chunk_size=64, qk_norm=True), "relu"),
    "one_state_phase_mod": (dict(dim=128, n_heads=2, head_dim=64, n_states=1, chunk_size=64), "phase_mod"),
}
VOCAB = 300
# (prompt length, join step, tokens decoded)
SEQS = [(5, 0, 5), (12, 0, 9), (3, 1, 4), (20, 3, 7), (8, 6, 5)]


def _row_rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().amax(-1) / b.abs().amax(-1)).max().item()


@pytest.mark.parametrize("graphs", [False, True])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("name", list(CFGS))
def test_model_decoder_matches_per_sequence_oracle(gpu_lib, name, dtype, graphs):
    from qllm2_amd.model_decode import ModelDecoder
    cfg, act = CFGS[name]
    n_layers = 2
    p = VM.make_model_params(cfg, n_layers, VOCAB, 900, activation=act)
    ref_model = VM.V11LM(cfg, n_layers, p, activation=act).eval()
    gpu_model = VM.V11LM(cfg, n_layers, {k: v.float() for k, v in p.items()}, activation=act,
                         dtype=torch.float32).cuda().eval()
    dec = ModelDecoder(gpu_model, n_slots=4, max_len=16, dtype=dtype, graphs=graphs, graph_bucket=2)
    g = torch.Generator().manual_seed(901)
    prompts = [torch.randint(0, VOCAB, (t,), generator=g) for t, _, _ in SEQS]
    conts = [torch.randint(0, VOCAB, (n,), generator=g) for _, _, n in SEQS]

    ref = []  # per sequence: logits after the prompt, then after each continuation token
    with torch.no_grad():
        for (t0, _, n), pr, ct in zip(SEQS, prompts, conts):
            logits, states = ref_model(pr.view(1, -1))
            rows = [logits[0, -1]]
            for i in range(n - 1):
                lg, states = ref_model(ct[i].view(1, 1), states=states, step_offset=t0 + i)
                rows.append(lg[0, 0])
            ref.append(torch.stack(rows))

    tol = 1e-4 if dtype == torch.float32 else 3e-2
    slot_of, done, got = {}, set(), [[] for _ in SEQS]
    step = 0
    while len(done) < len(SEQS):
        for si, (t0, join, n) in enumerate(SEQS):
            if join == step:
                slot, logits = dec.admit(prompts[si].cuda())
                slot_of[si] = slot
                got[si].append(logits.cpu())
        live = [si for si in sorted(slot_of, reverse=True) if si not in done and len(got[si]) < SEQS[si][2]]
        if live:
            slots = torch.tensor([slot_of[si] for si in live], dtype=torch.int32, device="cuda")
            ids = torch.stack([conts[si][len(got[si]) - 1] for si in live]).cuda()
            logits = dec.step(ids, slots)
            for row, si in enumerate(live):
                got[si].append(logits[row].cpu())
        for si in list(slot_of):
            if si not in done and len(got[si]) == SEQS[si][2]:
                dec.release(slot_of[si])
                done.add(si)
                del slot_of[si]
        step += 1
    for si in range(len(SEQS)):
        r = _row_rel(torch.stack(got[si]), ref[si])
        assert r < tol, f"seq {si}: rel {r:.2e}"
    if graphs:
        assert len(dec._graphs) >= 2, "both buckets should have been captured"


def test_model_decoder_sampling(gpu_lib):
    """Greedy picks the argmax; top-k sampling never leaves the k largest logits."""
    from qllm2_amd.model_decode import ModelDecoder
    logits = torch.randn(6, 50, generator=torch.Generator().manual_seed(3)).cuda()
    assert torch.equal(ModelDecoder.sample(logits, temperature=0), logits.argmax(-1))
    top = logits.topk(5).indices
    gen = torch.Generator(device="cuda").manual_seed(4)
    for _ in range(20):
        pick = ModelDecoder.sample(logits, temperature=0.7, top_k=5, generator=gen)
        assert all(pick[i] in top[i] for i in range(6))
