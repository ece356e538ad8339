"""Class-shaped CPU restatement of the QLLM v11 language model around the PAM
layer (test infrastructure only: the product never imports this module).

V11LM (v11/model.py:1052-1146): ComplexEmbed -> ComplexNorm -> [V11Block] x N
-> output ComplexNorm -> lm_head_proj (ComplexLinear with bias) -> lm_head_norm
-> tied logits Re(lm . conj(E)) = lm_re E_re^T + lm_im E_im^T.
V11Block (v11/model.py:1021-1049): pre-norm residuals, channel mix first,
    x = x + cgu_scale * CGU(norm1(x));  x = x + pam_scale * PAM(norm2(x)).
ComplexGatedUnit (v11/complex_ops.py:200-220): gate = gate_proj(z), up =
act(up_proj(z)), down_proj(cgu_gate(gate, up)), the projections without bias.

Modules keep the reference's attribute names (embed.embed_real / embed_imag,
embed_norm, blocks[i].norm1 / cgu / cgu_scale / norm2 / pam / pam_scale,
output_norm, lm_head_proj, lm_head_norm) so a model-level decoder can read a
reference V11LM and this class alike.  The PAM layer is oracle/v11_layer.py's
V11PAMLayer; the complex elementwise ops are oracle/complex_ops.py's forms of
the reference's PyTorch paths.  Learned position embeddings (use_learned_pos)
and dropout are not restated (the decode path runs without either).
"""

import torch
from torch import nn

from . import complex_ops as C
from . import pam_layer as L
from . import v11_layer as V


class ComplexLinear(nn.Module):
    """ComplexLinear (v11/complex_ops.py:146-172), optional bias."""

    def __init__(self, w_re, w_im, b_re=None, b_im=None):
        super().__init__()
        self.weight_real = nn.Parameter(w_re.clone())
        self.weight_imag = nn.Parameter(w_im.clone())
        self.bias_real = nn.Parameter(b_re.clone()) if b_re is not None else None
        self.bias_imag = nn.Parameter(b_im.clone()) if b_im is not None else None

    def forward(self, z):
        return L.complex_linear(z, self.weight_real, self.weight_imag, self.bias_real, self.bias_imag)


class ComplexNorm(nn.Module):
    """ComplexNorm (v11/complex_ops.py:175-192)."""

    def __init__(self, scale, eps=1e-6):
        super().__init__()
        self.scale = nn.Parameter(scale.clone())
        self.eps = eps

    def forward(self, z):
        return C.complex_norm(z, self.scale, self.eps)


class ModSwish(nn.Module):
    """ModSwish (v11/complex_ops.py:113-123)."""

    def __init__(self, bias, beta):
        super().__init__()
        self.bias = nn.Parameter(bias.clone())
        self.beta = nn.Parameter(beta.clone())

    def forward(self, z):
        return C.mod_swish(z, self.bias, self.beta)


class ModReLU(nn.Module):
    """ModReLU (v11/complex_ops.py:102-110)."""

    def __init__(self, bias):
        super().__init__()
        self.bias = nn.Parameter(bias.clone())

    def forward(self, z):
        return C.mod_relu(z, self.bias)


class PhaseModulatedActivation(nn.Module):
    """PhaseModulatedActivation (v11/complex_ops.py:125-143)."""

    def __init__(self, bias, beta, phase_alpha, phase_beta):
        super().__init__()
        self.bias = nn.Parameter(bias.clone())
        self.beta = nn.Parameter(beta.clone())
        self.phase_alpha = nn.Parameter(phase_alpha.clone())
        self.phase_beta = nn.Parameter(phase_beta.clone())

    def forward(self, z):
        return C.phase_mod(z, self.bias, self.beta, self.phase_alpha, self.phase_beta)


class ComplexGatedUnit(nn.Module):
    """ComplexGatedUnit (v11/complex_ops.py:200-220)."""

    def __init__(self, p, prefix, activation):
        super().__init__()
        lin = lambda name: ComplexLinear(p[f"{prefix}.{name}.weight_real"], p[f"{prefix}.{name}.weight_imag"])
        self.gate_proj, self.up_proj, self.down_proj = lin("gate_proj"), lin("up_proj"), lin("down_proj")
        # _build_activation (v11/complex_ops.py:192-197): 'swish', 'phase_mod', else ModReLU
        if activation == "swish":
            self.act = ModSwish(p[f"{prefix}.act.bias"], p[f"{prefix}.act.beta"])
        elif activation == "phase_mod":
            self.act = PhaseModulatedActivation(p[f"{prefix}.act.bias"], p[f"{prefix}.act.beta"],
                                                p[f"{prefix}.act.phase_alpha"], p[f"{prefix}.act.phase_beta"])
        else:
            self.act = ModReLU(p[f"{prefix}.act.bias"])

    def forward(self, z):
        gate = self.gate_proj(z)
        up = self.act(self.up_proj(z))
        return self.down_proj(C.cgu_gate(gate, up))


class V11Block(nn.Module):
    """V11Block (v11/model.py:1021-1049), dropout the identity."""

    def __init__(self, cfg, p, prefix, activation, dtype):
        super().__init__()
        self.norm1 = ComplexNorm(p[f"{prefix}.norm1.scale"])
        self.cgu = ComplexGatedUnit(p, f"{prefix}.cgu", activation)
        self.cgu_scale = nn.Parameter(p[f"{prefix}.cgu_scale"].clone())
        self.norm2 = ComplexNorm(p[f"{prefix}.norm2.scale"])
        pam_p = {k[len(prefix) + 5:]: v for k, v in p.items() if k.startswith(f"{prefix}.pam.")}
        self.pam = V.V11PAMLayer(cfg, pam_p, dtype=dtype)
        self.pam_scale = nn.Parameter(p[f"{prefix}.pam_scale"].clone())

    def forward(self, x, pam_state=None, step_offset=0):
        x = x + self.cgu(self.norm1(x)) * self.cgu_scale
        pam_out, new_state = self.pam(self.norm2(x), state=pam_state, step_offset=step_offset)
        return x + pam_out * self.pam_scale, new_state


class _Embedding(nn.Module):
    def __init__(self, w):
        super().__init__()
        self.weight = nn.Parameter(w.clone())

    def forward(self, ids):
        return self.weight[ids]


class ComplexEmbed(nn.Module):
    """ComplexEmbed (v11/complex_ops.py:223-235)."""

    def __init__(self, w_re, w_im):
        super().__init__()
        self.embed_real, self.embed_imag = _Embedding(w_re), _Embedding(w_im)

    def forward(self, ids):
        return torch.stack([self.embed_real(ids), self.embed_imag(ids)], dim=-1)


def make_model_params(cfg, n_layers, vocab, seed, expand=2, activation="swish", dtype=torch.float64):
    """Seeded parameters of an n_layers model by the reference's names (PAM
    layers from oracle/v11_layer.make_params; the other weights are scaled so
    that activations stay O(1) through the stack; the residual scales are off
    their init values so that every path matters)."""
    cfg = V.config(**cfg)
    g = torch.Generator().manual_seed(seed)
    dim = cfg["dim"]
    hid = dim * expand

    def rn(*shape, std):
        return (torch.randn(*shape, generator=g, dtype=torch.float64) * std).to(dtype)

    p = {"embed.embed_real.weight": rn(vocab, dim, std=0.5), "embed.embed_imag.weight": rn(vocab, dim, std=0.5),
         "embed_norm.scale": 1.0 + rn(dim, std=0.1), "output_norm.scale": 1.0 + rn(dim, std=0.1),
         "lm_head_proj.weight_real": rn(dim, dim, std=dim ** -0.5),
         "lm_head_proj.weight_imag": rn(dim, dim, std=dim ** -0.5),
         "lm_head_proj.bias_real": rn(dim, std=0.1), "lm_head_proj.bias_imag": rn(dim, std=0.1),
         "lm_head_norm.scale": 1.0 + rn(dim, std=0.1)}
    for i in range(n_layers):
        b = f"blocks.{i}"
        p[f"{b}.norm1.scale"] = 1.0 + rn(dim, std=0.1)
        p[f"{b}.norm2.scale"] = 1.0 + rn(dim, std=0.1)
        for name, (o, n_in) in (("gate_proj", (hid, dim)), ("up_proj", (hid, dim)), ("down_proj", (dim, hid))):
            p[f"{b}.cgu.{name}.weight_real"] = rn(o, n_in, std=(2 * n_in) ** -0.5)
            p[f"{b}.cgu.{name}.weight_imag"] = rn(o, n_in, std=(2 * n_in) ** -0.5)
        p[f"{b}.cgu.act.bias"] = rn(hid, std=0.1) - (0.0 if activation in ("swish", "phase_mod") else 0.1)
        if activation in ("swish", "phase_mod"):
            p[f"{b}.cgu.act.beta"] = 1.0 + rn(hid, std=0.2)
        if activation == "phase_mod":  # angles of a radian or so, so that the rotation matters
            p[f"{b}.cgu.act.phase_alpha"] = rn(hid, std=0.5)
            p[f"{b}.cgu.act.phase_beta"] = rn(hid, std=1.0)
        p[f"{b}.cgu_scale"] = torch.tensor(0.7, dtype=dtype)
        p[f"{b}.pam_scale"] = torch.tensor(0.6, dtype=dtype)
        for k, v in V.make_params(cfg, seed + 31 * (i + 1), dtype).items():
            p[f"{b}.pam.{k}"] = v
    return p


class V11LM(nn.Module):
    """V11LM (v11/model.py:1052-1146) without learned position embeddings."""

    def __init__(self, cfg, n_layers, p, activation="swish", dtype=torch.float64):
        super().__init__()
        c = V.config(**cfg)
        self.embed = ComplexEmbed(p["embed.embed_real.weight"], p["embed.embed_imag.weight"])
        self.pos_embed = None
        self.embed_norm = ComplexNorm(p["embed_norm.scale"])
        self.blocks = nn.ModuleList([V11Block(c, p, f"blocks.{i}", activation, dtype) for i in range(n_layers)])
        self.output_norm = ComplexNorm(p["output_norm.scale"])
        self.lm_head_proj = ComplexLinear(p["lm_head_proj.weight_real"], p["lm_head_proj.weight_imag"],
                                          p["lm_head_proj.bias_real"], p["lm_head_proj.bias_imag"])
        self.lm_head_norm = ComplexNorm(p["lm_head_norm.scale"])

    def forward(self, input_ids, states=None, step_offset=0):
        """input_ids [B, T] -> (logits [B, T, V], per-layer PAM states)."""
        z = self.embed_norm(self.embed(input_ids))
        new_states = []
        for i, block in enumerate(self.blocks):
            z, s = block(z, pam_state=states[i] if states is not None else None, step_offset=step_offset)
            new_states.append(s)
        lm = self.lm_head_norm(self.lm_head_proj(self.output_norm(z)))
        logits = lm[..., 0] @ self.embed.embed_real.weight.T + lm[..., 1] @ self.embed.embed_imag.weight.T
        return logits, new_states
