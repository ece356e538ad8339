"""CPU checks of the model-level oracle (oracle/v11_model.py: V11LM, V11Block,
ComplexGatedUnit restated around the PAM layer), float64:

  * the prefill of a prompt then token-by-token decode gives the logits of one
    prefill over the whole sequence (the PAM layer's chunked form and its
    recurrent form agree up to the chunked form's gamma + 1e-6: derived bound
    T * 1e-6 relative per decayed term, 1e-4 here);
  * with both residual scales at zero the blocks pass the embedding through,
    and the tied logits equal Re(lm conj(E)) computed in complex128 from the
    head's output;
  * the CGU sub-block is linear in the down projection (scaling its weights
    scales the block's channel-mix contribution exactly)."""

import torch

from oracle import complex_ops as C
from oracle import pam_layer as L
from oracle import v11_model as VM

CFG = dict(dim=32, n_heads=2, head_dim=16, n_states=3, chunk_size=8, state_compete=True, gamma_floor=0.2)


def _model(seed=5, n_layers=2, vocab=60, **over):
    p = VM.make_model_params(CFG, n_layers, vocab, seed)
    p.update(over)
    return VM.V11LM(CFG, n_layers, p).eval(), p


def _rel(a, b):
    return ((a - b).abs().max() / b.abs().max()).item()


def test_prefill_then_decode_equals_full_prefill():
    model, _ = _model()
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, 60, (1, 21), generator=g)
    with torch.no_grad():
        full, _ = model(ids)
        logits, states = model(ids[:, :13])
        assert _rel(logits, full[:, :13]) < 1e-12
        for t in range(13, 21):
            step, states = model(ids[:, t:t + 1], states=states, step_offset=t)
            assert _rel(step[:, 0], full[:, t]) < 1e-4, t


def test_zero_residual_scales_and_tied_logits():
    n_layers = 2
    zero = torch.tensor(0.0, dtype=torch.float64)
    over = {f"blocks.{i}.{s}": zero for i in range(n_layers) for s in ("cgu_scale", "pam_scale")}
    model, p = _model(n_layers=n_layers, **over)
    ids = torch.tensor([[3, 17, 42, 5, 0, 59]])
    with torch.no_grad():
        logits, _ = model(ids)
        z = model.embed_norm(model.embed(ids))
        lm = model.lm_head_norm(model.lm_head_proj(model.output_norm(z)))
    e = torch.complex(p["embed.embed_real.weight"], p["embed.embed_imag.weight"])
    want = (torch.complex(lm[..., 0], lm[..., 1]) @ e.conj().T).real
    assert _rel(logits, want) < 1e-12


def test_channel_mix_linear_in_down_projection():
    model, p = _model(seed=9)
    blk = model.blocks[0]
    x = torch.randn(1, 4, CFG["dim"], 2, generator=torch.Generator().manual_seed(10), dtype=torch.float64)
    with torch.no_grad():
        h = blk.norm1(x)
        a = blk.cgu(h)
        blk.cgu.down_proj.weight_real.mul_(2.5)
        blk.cgu.down_proj.weight_imag.mul_(2.5)
        b = blk.cgu(h)
        # the same through the oracle's own pieces
        gate = L.complex_linear(h, p["blocks.0.cgu.gate_proj.weight_real"], p["blocks.0.cgu.gate_proj.weight_imag"])
        up = C.mod_swish(L.complex_linear(h, p["blocks.0.cgu.up_proj.weight_real"],
                                          p["blocks.0.cgu.up_proj.weight_imag"]),
                         p["blocks.0.cgu.act.bias"], p["blocks.0.cgu.act.beta"])
        want = L.complex_linear(C.cgu_gate(gate, up), p["blocks.0.cgu.down_proj.weight_real"],
                                p["blocks.0.cgu.down_proj.weight_imag"])
    assert _rel(b, 2.5 * a) < 1e-12
    assert _rel(a, want) < 1e-12


def test_phase_mod_block_prefill_then_decode():
    """A model with the phase-modulated CGU activation: decode after a prefill
    gives the logits of one prefill over the whole sequence, and its
    activation is not ModSwish's (the phase parameters are used)."""
    p = VM.make_model_params(CFG, 2, 60, 8, activation="phase_mod")
    model = VM.V11LM(CFG, 2, p, activation="phase_mod").eval()
    swish = VM.V11LM(CFG, 2, p, activation="swish").eval()
    ids = torch.randint(0, 60, (1, 17), generator=torch.Generator().manual_seed(9))
    with torch.no_grad():
        full, _ = model(ids)
        logits, states = model(ids[:, :11])
        for t in range(11, 17):
            step, states = model(ids[:, t:t + 1], states=states, step_offset=t)
            assert _rel(step[:, 0], full[:, t]) < 1e-4, t
        assert _rel(swish(ids)[0], full) > 1e-3
