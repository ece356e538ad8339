"""GPU parity of the drop-in as a whole: install() on a V11PAMLayer-shaped
class, then the reference's own layer-level checks run through it.

The class is the oracle's restatement of V11PAMLayer (oracle/v11_layer.py:
same attributes, same method names, the reference's dispatch in forward and
_recurrent); install() rebinds a subclass of it, so the saved originals are
the restated reference methods.  For every mode of the reference's self-test
(v11/selftest.py:193-204: baseline, E1 per-channel, E2 delta, E3 multistate,
E1+E3) plus the E3 K-loop, at head_dim 16 (the self-test's shape) and 64, and
the shapes the kernels take in pieces (six states, head_dim 128 and 96):

  * the installed layer on the GPU (fp32) against the float64 oracle layer on
    the CPU: parallel prefill, token-by-token decode and the final state, rel
    <= 1e-4 (max error over max reference value, per batch row);
  * parallel == recurrent on the GPU within the self-test's bar (atol 2e-3,
    v11/selftest.py:16-38);
  * the HIP kernels ran where they apply: counters on the saved originals show
    the head-decay scans, the delta write and the decode steps never fell
    back (decode at head dims 96 and 48 runs zero-padded on the 128- and
    64-wide kernels, with per-channel decays in the E1 mode);
  * grad mode: a T = 1 step carrying a state (the reference's recurrent
    branch, v11/model.py:830-832; the decode step and its backward as HIP
    kernels) and a prefill, every gradient (input, state, each parameter)
    against float64 autograd of the oracle layer, rel <= 1e-4.
"""

import collections
import sys
import types

import pytest
import torch

from oracle import v11_layer as V

pytestmark = pytest.mark.gpu

DIM16 = dict(dim=32, n_heads=2, head_dim=16, chunk_size=24)
DIM64 = dict(dim=64, n_heads=2, head_dim=64, chunk_size=64)
MODES = {
    "baseline": dict(DIM16),
    "E1": dict(DIM16, decay_mode="per_channel"),
    "E2": dict(DIM16, write_mode="delta", delta_chunk=20),
    "E3": dict(DIM16, n_states=2),
    "E3_loop": dict(DIM16, n_states=2, fused_e3=False),
    "E1+E3": dict(DIM16, decay_mode="per_channel", n_states=2),
    "baseline_hd64": dict(DIM64),
    "E2_hd64": dict(DIM64, write_mode="delta", delta_chunk=64),
    "E3_hd64": dict(DIM64, n_states=3, state_compete=True, gamma_floor=0.2),
    "E3_6states": dict(DIM16, n_states=6),
    "baseline_hd128": dict(dim=128, n_heads=1, head_dim=128, chunk_size=64),
    "E3_hd96": dict(dim=96, n_heads=1, head_dim=96, chunk_size=32, n_states=2),
    "E1_hd48": dict(dim=96, n_heads=2, head_dim=48, chunk_size=32, decay_mode="per_channel"),
}
# reference methods that must not run (the HIP path covers the call) per mode
HIP_ONLY = {
    "baseline": ("_forward_chunked_head", "_recurrent", "_recur_step_additive"),
    "E3": ("_forward_multistate_fused", "_fused_chunk_step", "_recurrent", "_recur_step_additive"),
    "E3_loop": ("_forward_chunked_head", "_recurrent", "_recur_step_additive"),
    "baseline_hd64": ("_forward_chunked_head", "_recurrent", "_recur_step_additive"),
    "E2_hd64": ("_forward_delta", "_recur_step_delta"),
    "E3_hd64": ("_forward_multistate_fused", "_recurrent", "_recur_step_additive"),
    "E2": ("_forward_delta", "_recur_step_delta"),
    "E3_6states": ("_forward_multistate_fused", "_fused_chunk_step", "_recurrent", "_recur_step_additive"),
    "baseline_hd128": ("_forward_chunked_head", "_recurrent", "_recur_step_additive"),
    "E3_hd96": ("_forward_multistate_fused", "_fused_chunk_step", "_recurrent", "_recur_step_additive"),
    "E1_hd48": ("_forward_chunked_perchannel", "_recurrent", "_recur_step_additive"),
    "E1": ("_forward_chunked_perchannel", "_recurrent", "_recur_step_additive"),
    "E1+E3": ("_forward_chunked_perchannel", "_recurrent", "_recur_step_additive"),
}


@pytest.fixture(scope="module")
def installed():
    from qllm2_amd import _reference, pam_layer
    name = "v11gpu"
    pkg, mod = types.ModuleType(name), types.ModuleType(f"{name}.model")

    class V11PAMLayer(V.V11PAMLayer):
        pass

    mod.V11PAMLayer = V11PAMLayer
    sys.modules[name], sys.modules[f"{name}.model"] = pkg, mod
    saved = dict(_reference._SAVED)
    try:
        pam_layer.install(mod)
        calls = collections.Counter()
        table = V11PAMLayer._qpam_originals

        def counted(key, fn):
            def run(*a, **k):
                calls[key] += 1
                return fn(*a, **k)
            return run

        for key in list(table):
            table[key] = counted(key, table[key])
        yield V11PAMLayer, calls
    finally:
        _reference._SAVED.clear()
        _reference._SAVED.update(saved)
        for sub in ("model", "flash_pam", "triton_kernels", "fused_ce"):
            sys.modules.pop(f"{name}.{sub}", None)
        sys.modules.pop(name, None)


def _rel(got, ref):
    """Max over batch rows of (max error / max reference value) of that row."""
    got, ref = got.detach().double().cpu(), ref.detach().double().cpu()
    err = (got - ref).abs().flatten(1).max(1).values
    scale = ref.abs().flatten(1).max(1).values + 1e-30
    return (err / scale).max().item()


def _pair(installed, mode, seed):
    cls, calls = installed
    cfg = V.config(**MODES[mode])
    p = V.make_params(cfg, seed)
    ref = V.V11PAMLayer(cfg, p).eval()
    gpu = cls(cfg, {k: v.float() for k, v in p.items()}, dtype=torch.float32).cuda().eval()
    return cfg, ref, gpu, calls


def _run_mode(layer, x):
    with torch.no_grad():
        par, s_par = layer(x, state=None, step_offset=0)
        outs, state = [], None
        for t in range(x.shape[1]):
            o, state = layer(x[:, t:t + 1], state=state, step_offset=t)
            outs.append(o)
    return par, s_par, torch.cat(outs, dim=1), state


@pytest.mark.parametrize("mode", list(MODES))
def test_installed_selftest_matches_oracle(installed, mode):
    cfg, ref, gpu, calls = _pair(installed, mode, 60)
    x = torch.randn(2, 80, cfg["dim"], 2, generator=torch.Generator().manual_seed(61), dtype=torch.float64) * 0.5
    par_r, s_par_r, rec_r, s_rec_r = _run_mode(ref, x)
    calls.clear()
    par, s_par, rec, s_rec = _run_mode(gpu, x.float().cuda())
    torch.cuda.synchronize()
    print(f"{mode}: reference methods run {dict(calls)}")
    assert _rel(par, par_r) < 1e-4, f"parallel {_rel(par, par_r):.2e}"
    assert _rel(rec, rec_r) < 1e-4, f"recurrent {_rel(rec, rec_r):.2e}"
    assert _rel(s_par, s_par_r) < 1e-4, f"prefill state {_rel(s_par, s_par_r):.2e}"
    assert _rel(s_rec, s_rec_r) < 1e-4, f"decode state {_rel(s_rec, s_rec_r):.2e}"
    assert (par - rec).abs().max().item() < 2e-3
    for name in HIP_ONLY.get(mode, ()):
        assert calls[name] == 0, f"{mode}: the reference's {name} ran {calls[name]} times"


GRAD_MODES = ["baseline", "E1", "E3", "E1+E3", "E2_hd64", "baseline_hd64", "E3_hd64", "E2", "E3_6states",
              "baseline_hd128", "E3_hd96", "E1_hd48"]


def _grads(layer, x, step_offset, state, loss_fn):
    layer.zero_grad()
    x = x.clone().requires_grad_(True)
    st = state.clone().requires_grad_(True) if state is not None else None
    y, s = layer(x, state=st, step_offset=step_offset)
    loss_fn(y, s).backward()
    named = {n: p.grad for n, p in layer.named_parameters()}
    return y, s, x.grad, (st.grad if st is not None else None), named


@pytest.mark.parametrize("mode", GRAD_MODES)
def test_installed_grad_mode_matches_oracle(installed, mode):
    """A T = 1 step carrying a prefill state under grad mode (the reference's
    recurrent branch; a training forward of one token) and a prefill, both
    differentiated: outputs, states and every gradient."""
    cfg, ref, gpu, _ = _pair(installed, mode, 70)
    g = torch.Generator().manual_seed(71)
    x = torch.randn(2, 40, cfg["dim"], 2, generator=g, dtype=torch.float64) * 0.5
    dy = torch.randn(2, 40, cfg["dim"], 2, generator=g, dtype=torch.float64)
    with torch.no_grad():
        _, st_r = ref(x[:, :33])
        _, st_g = gpu(x[:, :33].float().cuda())

    def step_loss(dyt):
        return lambda y, s: (y * dyt).sum() + (s * s).sum()

    ra = _grads(ref, x[:, 33:34], 33, st_r, step_loss(dy[:, 33:34]))
    calls = installed[1]
    calls.clear()
    ga = _grads(gpu, x[:, 33:34].float().cuda(), 33, st_g, step_loss(dy[:, 33:34].float().cuda()))
    if not mode.startswith("E2"):  # the additive step and its backward ran as HIP kernels
        assert calls["_recur_step_additive"] == 0, f"{mode}: the reference step ran {calls['_recur_step_additive']} times"
    names = ["y", "state", "dx", "dstate"]
    for nm, a, b in zip(names, ga[:4], ra[:4]):
        assert _rel(a, b) < 1e-4, f"step {nm}: {_rel(a, b):.2e}"
    for nm, b in ra[4].items():
        a = ga[4][nm]
        assert (a is None) == (b is None), nm
        if b is not None:
            assert _rel(a.reshape(1, -1), b.reshape(1, -1)) < 1e-4, f"step d{nm}: {_rel(a.reshape(1, -1), b.reshape(1, -1)):.2e}"
    # prefill with gradients
    loss = lambda y, s: (y * dy).sum() if y.device.type == "cpu" else (y * dy.float().cuda()).sum()  # noqa: E731
    ra = _grads(ref, x, 0, None, loss)
    ga = _grads(gpu, x.float().cuda(), 0, None, loss)
    assert _rel(ga[0], ra[0]) < 1e-4, f"prefill y {_rel(ga[0], ra[0]):.2e}"
    assert _rel(ga[2], ra[2]) < 1e-4, f"prefill dx {_rel(ga[2], ra[2]):.2e}"
    for nm, b in ra[4].items():
        a = ga[4][nm]
        if b is not None:
            assert _rel(a.reshape(1, -1), b.reshape(1, -1)) < 1e-4, f"prefill d{nm}: {_rel(a.reshape(1, -1), b.reshape(1, -1)):.2e}"
