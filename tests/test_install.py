"""CPU check of install(): it rebinds the V11PAMLayer hot-path methods of a
v11.model-like module, replaces the module-level fused_decay_matrix name,
aliases the v11.flash_pam / triton_kernels / fused_ce modules and rebinds the
elementwise ops v11.complex_ops imported (no GPU call)."""

import sys
import types

from qllm2_amd import fused_ce, flash_pam, pam_layer, triton_kernels


def test_install_rebinds_methods_and_aliases():
    pkg = types.ModuleType("v11x")
    mod = types.ModuleType("v11x.model")

    class V11PAMLayer:
        def forward(self, *a):
            return "orig"

        @staticmethod
        def _dual_form_block(*a):
            return "orig"

        def _forward_chunked_head(self, *a):
            return "orig"

        def _fused_chunk_step(self, *a):
            return "orig"

        def _forward_multistate_fused(self, *a):
            return "orig"

        def _recur_step_additive(self, *a):
            return "orig"

        def _recurrent(self, *a):
            return "orig"

        def _forward_delta(self, *a):
            return "orig"

        def _recur_step_delta(self, *a):
            return "orig"

    mod.V11PAMLayer = V11PAMLayer
    mod.fused_decay_matrix = lambda *a: "orig"
    cops = types.ModuleType("v11x.complex_ops")  # imported the ops by name before install()
    for name in ("fused_complex_norm", "fused_mod_swish", "fused_mod_relu", "fused_cgu_gate"):
        setattr(cops, name, lambda *a: "orig")
    sys.modules["v11x"] = pkg
    sys.modules["v11x.model"] = mod
    sys.modules["v11x.complex_ops"] = cops
    saved = dict(pam_layer._ORIGINALS)
    pam_layer._ORIGINALS.clear()
    try:
        originals = pam_layer.install(mod)
        assert V11PAMLayer.forward is pam_layer.forward
        assert V11PAMLayer._forward_chunked_head is pam_layer.forward_chunked_head
        assert V11PAMLayer._fused_chunk_step is pam_layer.fused_chunk_step
        assert V11PAMLayer._forward_multistate_fused is pam_layer.forward_multistate_fused
        assert V11PAMLayer._recur_step_additive is pam_layer.recur_step_additive
        assert V11PAMLayer._recurrent is pam_layer.recurrent
        assert V11PAMLayer._forward_delta is pam_layer.forward_delta
        assert V11PAMLayer._recur_step_delta is pam_layer.recur_step_delta
        assert V11PAMLayer._dual_form_block is pam_layer.dual_form_block  # staticmethod unwraps
        assert mod.fused_decay_matrix is triton_kernels.fused_decay_matrix
        assert sys.modules["v11x.flash_pam"] is flash_pam
        assert sys.modules["v11x.triton_kernels"] is triton_kernels
        assert sys.modules["v11x.fused_ce"] is fused_ce
        assert pkg.fused_ce is fused_ce
        assert set(originals) >= {"forward", "_forward_chunked_head", "_recurrent", "_dual_form_block"}
        for name in ("fused_complex_norm", "fused_mod_swish", "fused_mod_relu", "fused_cgu_gate"):
            assert getattr(cops, name) is getattr(triton_kernels, name)
    finally:
        pam_layer._ORIGINALS.clear()
        pam_layer._ORIGINALS.update(saved)
        for k in ("v11x", "v11x.model", "v11x.flash_pam", "v11x.triton_kernels", "v11x.fused_ce", "v11x.complex_ops"):
            sys.modules.pop(k, None)
