"""CPU checks of install() (no GPU call).

* It rebinds the V11PAMLayer hot-path methods of a v11.model-like module,
  keeps the class's own methods on that class, replaces the module-level
  fused_decay_matrix name, aliases v11.flash_pam / triton_kernels / fused_ce
  and rebinds the elementwise ops v11.complex_ops imported.
* After install(), a layer on CPU tensors computes exactly what the
  un-installed layer computes, in every mode (prefill and decode, forward and
  gradients): the replacements hand CPU calls to the saved reference methods.
  The stand-in reference class is the oracle's V11PAMLayer restatement.
* The replaced module functions hand CPU calls to the reference functions
  install() found, and raise without them.
"""

import sys
import types

import pytest
import torch

from oracle import ce as OC
from oracle import complex_ops as OX
from oracle import pam as O
from oracle import v11_layer as V
from qllm2_amd import _reference, fused_ce, flash_pam, pam_layer, triton_kernels

_SUBS = ("model", "flash_pam", "triton_kernels", "fused_ce", "complex_ops")


@pytest.fixture
def fake_pkg():
    """A v11-like package whose model module holds a subclass of the oracle's
    V11PAMLayer (so install() leaves the oracle class itself untouched), and
    whose flash_pam / triton_kernels / fused_ce / complex_ops hold the oracle's
    restatements of the reference functions."""
    name = "v11fake"
    pkg = types.ModuleType(name)
    mod = types.ModuleType(f"{name}.model")

    class V11PAMLayer(V.V11PAMLayer):
        pass

    mod.V11PAMLayer = V11PAMLayer
    decay = lambda gamma, seq_len, block=64: O.decay_matrix(gamma, seq_len)  # noqa: E731 (reference signature)
    mod.fused_decay_matrix = decay
    fp = types.ModuleType(f"{name}.flash_pam")
    fp.flash_pam_chunked_head = O.flash_pam_chunked_head
    fp._chunk_decay_matrices = O.decay_matrices
    tk = types.ModuleType(f"{name}.triton_kernels")
    tk.fused_decay_matrix = decay
    tk.fused_complex_norm, tk.fused_mod_swish = OX.complex_norm, OX.mod_swish
    tk.fused_mod_relu, tk.fused_cgu_gate = OX.mod_relu, OX.cgu_gate
    ce = types.ModuleType(f"{name}.fused_ce")
    ce.fused_linear_cross_entropy = lambda h, w, t, mask=None, chunk=4096, ignore_index=-100: OC.ce_forward(
        h, w, t, mask=mask, chunk=chunk, ignore_index=ignore_index)[0]
    ce.linear_ce_per_token = OC.ce_per_token
    ce.linear_ce_stats = OC.ce_stats
    cops = types.ModuleType(f"{name}.complex_ops")  # imported the ops by name before install()
    for op in ("fused_complex_norm", "fused_mod_swish", "fused_mod_relu", "fused_cgu_gate"):
        setattr(cops, op, getattr(tk, op))
    for sub, m in zip(_SUBS, (mod, fp, tk, ce, cops)):
        sys.modules[f"{name}.{sub}"] = m
    sys.modules[name] = pkg
    saved = dict(_reference._SAVED)
    _reference._SAVED.clear()
    try:
        yield pkg, mod, (fp, tk, ce, cops)
    finally:
        _reference._SAVED.clear()
        _reference._SAVED.update(saved)
        for sub in _SUBS:
            sys.modules.pop(f"{name}.{sub}", None)
        sys.modules.pop(name, None)


def test_install_rebinds_methods_and_aliases(fake_pkg):
    pkg, mod, (fp, tk, ce, cops) = fake_pkg
    layer = mod.V11PAMLayer
    originals = pam_layer.install(mod)
    assert layer.forward is pam_layer.forward
    assert layer._forward_chunked_head is pam_layer.forward_chunked_head
    assert layer._fused_chunk_step is pam_layer.fused_chunk_step
    assert layer._forward_multistate_fused is pam_layer.forward_multistate_fused
    assert layer._recur_step_additive is pam_layer.recur_step_additive
    assert layer._recurrent is pam_layer.recurrent
    assert layer._forward_delta is pam_layer.forward_delta
    assert layer._recur_step_delta is pam_layer.recur_step_delta
    assert layer._dual_form_block.__wrapped__ is pam_layer.dual_form_block   # staticmethod unwraps
    # the class's own methods are kept on it; the oracle base class is untouched
    assert layer._qpam_originals["_recurrent"] is V.V11PAMLayer._recurrent
    assert layer._qpam_originals["_dual_form_block"] is V.V11PAMLayer._dual_form_block
    assert V.V11PAMLayer.forward is not pam_layer.forward
    assert mod.fused_decay_matrix is triton_kernels.fused_decay_matrix
    assert sys.modules["v11fake.flash_pam"] is flash_pam
    assert sys.modules["v11fake.triton_kernels"] is triton_kernels
    assert sys.modules["v11fake.fused_ce"] is fused_ce
    assert pkg.fused_ce is fused_ce
    assert set(originals) >= {"forward", "_forward_chunked_head", "_recurrent", "_dual_form_block",
                              "fused_ce.fused_linear_cross_entropy", "flash_pam.flash_pam_chunked_head"}
    for name in ("fused_complex_norm", "fused_mod_swish", "fused_mod_relu", "fused_cgu_gate"):
        assert getattr(cops, name) is getattr(triton_kernels, name)
    # a second install() keeps the first originals (never saves its own replacements)
    pam_layer.install(mod)
    assert layer._qpam_originals["_recurrent"] is V.V11PAMLayer._recurrent
    assert _reference.saved("flash_pam.flash_pam_chunked_head") is O.flash_pam_chunked_head


MODES = {
    "baseline": {},
    "E1": dict(decay_mode="per_channel"),
    "E2": dict(write_mode="delta", delta_chunk=20),
    "E3": dict(n_states=2),
    "E3_loop": dict(n_states=2, fused_e3=False),
    "E1+E3": dict(decay_mode="per_channel", n_states=2),
    "E3_hd64": dict(n_states=3, head_dim=64, chunk_size=64),
}


@pytest.mark.parametrize("mode", list(MODES))
def test_installed_layer_on_cpu_is_the_reference(fake_pkg, mode):
    """Prefill, token decode and a grad-mode T = 1 step on CPU: bit-identical
    to the un-installed class (outputs, states and every gradient)."""
    _, mod, _ = fake_pkg
    pam_layer.install(mod)
    cfg = V.config(**MODES[mode])
    p = V.make_params(cfg, 40)
    ref = V.V11PAMLayer(cfg, p).eval()
    inst = mod.V11PAMLayer(cfg, p).eval()
    x = torch.randn(2, 30, cfg["dim"], 2, generator=torch.Generator().manual_seed(41), dtype=torch.float64) * 0.5
    with torch.no_grad():
        for layer_pair in ((ref, inst),):
            outs = []
            for layer in layer_pair:
                y, s = layer(x)
                st, ys = None, []
                for t in range(6):
                    o, st = layer(x[:, t:t + 1], state=st, step_offset=t)
                    ys.append(o)
                outs.append((y, s, torch.cat(ys, 1), st))
            for a, b in zip(*outs):
                assert torch.equal(a, b)
    # grad mode: a T = 1 step carrying a state
    grads = []
    for layer in (ref, inst):
        layer.zero_grad()
        with torch.no_grad():
            _, st = layer(x[:, :5])
        st = st.clone().requires_grad_(True)
        xt = x[:, 5:6].clone().requires_grad_(True)
        y, s2 = layer(xt, state=st, step_offset=5)
        ((y ** 2).sum() + (s2 ** 2).sum()).backward()
        grads.append([xt.grad, st.grad] + [prm.grad for prm in layer.parameters()])
    for a, b in zip(*grads):
        assert (a is None and b is None) or torch.equal(a, b)


def test_module_functions_cpu_after_install(fake_pkg):
    _, mod, (fp, tk, ce, cops) = fake_pkg
    g = torch.Generator().manual_seed(50)
    gamma = torch.rand(4, 16, generator=g, dtype=torch.float64)
    q, k, v = (torch.randn(1, 2, 20, 8, 2, generator=g, dtype=torch.float64) for _ in range(3))
    gam = torch.rand(1, 2, 20, generator=g, dtype=torch.float64)
    h = torch.randn(12, 16, generator=g, dtype=torch.float64)
    w = torch.randn(30, 16, generator=g, dtype=torch.float64)
    tgt = torch.randint(0, 30, (12,), generator=g)
    z = torch.randn(5, 8, 2, generator=g, dtype=torch.float64)
    scale = torch.rand(8, generator=g, dtype=torch.float64)
    with pytest.raises(ValueError, match="GPU"):
        triton_kernels.fused_decay_matrix(gamma, 16)
    with pytest.raises(ValueError, match="GPU"):
        fused_ce.fused_linear_cross_entropy(h, w, tgt)
    pam_layer.install(mod)
    assert torch.equal(triton_kernels.fused_decay_matrix(gamma, 16), O.decay_matrix(gamma, 16))
    assert torch.equal(cops.fused_complex_norm(z, scale), OX.complex_norm(z, scale))
    y, s = flash_pam.flash_pam_chunked_head(q, k, v, gam, 8, 8)
    y_ref, s_ref = O.flash_pam_chunked_head(q, k, v, gam, 8, 8)
    assert torch.equal(y, y_ref) and torch.equal(s, s_ref)
    assert torch.equal(fused_ce.fused_linear_cross_entropy(h, w, tgt), ce.fused_linear_cross_entropy(h, w, tgt))
    assert torch.equal(fused_ce.linear_ce_per_token(h, w, tgt), OC.ce_per_token(h, w, tgt))
