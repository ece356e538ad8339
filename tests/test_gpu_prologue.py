"""GPU parity of the PAM layer prologue (qpam_prologue_fwd / _bwd) and of the
fused layer forward (pam_layer.forward: planar projections, prologue kernel,
scan writing head-merged Y, planar o_proj) against the CPU oracle
(oracle/pam_layer.py) in float64, forward and every gradient.

Tolerances: fp32 rel <= 1e-5 on the prologue outputs and <= 1e-4 on every
gradient and on the layer; bf16 projections rel <= 2e-2 (oracle fed the
bf16-rounded values)."""

import math

import pytest
import torch

from oracle import pam as O
from oracle import pam_layer as L

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


CASES = [  # (M, rope_offset or None, gsp, phase, routing, qk_norm, floor, T)
    (3, 0, True, True, False, False, 0.0, 130),
    (3, 57, True, True, True, False, 0.0, 64),
    (1, None, True, False, False, True, 0.5, 100),
    (2, 5, False, True, False, True, 0.0, 37),
    (4, 1000, True, True, True, False, 0.25, 200),
]


def _inputs(M, use_rope, gsp, phase, routing, T, seed, B=2, H=3, d=64):
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(B, T, 3, H, d, 2, generator=g)
    dt = torch.randn(B, T, H, generator=g) * 3
    dt[0, 0, 0] = 25.0  # softplus threshold branch
    bias = torch.randn(H, generator=g) - 2
    off = torch.linspace(-1, 1, M) + 0.1 * torch.randn(M, generator=g) if M > 1 else None
    prot = torch.randn(B, T, H, generator=g) if gsp else None
    ph = torch.randn(B, T, H, M, generator=g) * 2 if phase else None
    ro = torch.rand(B, T, H, M, generator=g) * 2 if routing else None
    return qkv, dt, bias, off, prot, ph, ro


def _oracle(qkv, dt, bias, off, prot, ph, ro, rope, offset, qk_norm, floor):
    """float64 oracle forward; returns leaves (for grads) and outputs."""
    leaves = [x.double().requires_grad_(True) if x is not None else None for x in (qkv, dt, bias, off, prot, ph, ro)]
    q, k, v = leaves[0][:, :, 0], leaves[0][:, :, 1], leaves[0][:, :, 2]
    q2, k2, v2, gamma, rot = L.prologue(q, k, v, leaves[1], leaves[2], leaves[3], leaves[4], leaves[5], leaves[6],
                                        rope.double() if rope is not None else None, offset, qk_norm, floor)
    rr = (rot[1] * torch.cos(rot[0]), rot[1] * torch.sin(rot[0])) if rot is not None else None
    return leaves, (q2, k2, v2, gamma, rr)


@pytest.mark.parametrize("d", [64, 16, 32, 128])
@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prologue_matches_oracle(gpu_lib, case, dtype, d):
    """The prologue op on a projection matrix [B,T,C] (q, k, v re planes, im
    planes, dt, padding) against the oracle's prologue: outputs, and the
    gradients of the projection matrix (its padding columns zero), dt_bias,
    the state offsets, protect, phase and routing; head dims 16 to 128 (a
    token row of d / 4 lanes in the kernels)."""
    from qllm2_amd.decode import build_rope_cache
    from qllm2_amd.pam_prologue import pam_prologue, proj_columns
    M, offset, gsp, phase, routing, qk_norm, floor, T = case
    B, H = 2, 3
    qkv, dt, bias, off, prot, ph, ro = _inputs(M, offset is not None, gsp, phase, routing, T, 500 + M + T + d, d=d)
    rnd = (lambda t: t.to(dtype).float() if t is not None else None)
    qkv, dt, prot, ph, ro = rnd(qkv), rnd(dt), rnd(prot), rnd(ph), rnd(ro)   # values both sides see
    rope = build_rope_cache(offset + T + 3, d) if offset is not None else None
    leaves, ref = _oracle(qkv, dt, bias, off, prot, ph, ro, rope, offset or 0, qk_norm, floor)
    dev = torch.device("cuda")
    C = proj_columns(H, d)
    proj = torch.cat([qkv[..., 0].reshape(B, T, 3 * H * d), qkv[..., 1].reshape(B, T, 3 * H * d), dt,
                      torch.zeros(B, T, C - 6 * H * d - H)], -1)
    proj = proj.to(dtype).to(dev).requires_grad_(True)
    gl = [x.to(dev).to(dtype if i >= 2 else torch.float32).requires_grad_(True) if x is not None else None
          for i, x in enumerate((bias, off, prot, ph, ro))]
    q, k, v, gamma, rot = pam_prologue(proj, gl[0], n_heads=H, n_states=M, state_offset=gl[1], protect=gl[2],
                                       phase=gl[3], routing=gl[4], rope=rope.to(dev) if rope is not None else None,
                                       rope_offset=offset or 0, qk_norm=qk_norm, gamma_floor=floor, head_dim=d)
    tol_f = 1e-5 if dtype == torch.float32 else 2e-2
    tol_g = 1e-4 if dtype == torch.float32 else 2e-2
    for name, got, want in (("q", q, ref[0]), ("k", k, ref[1]), ("v", v, ref[2])):
        assert got[0].dtype == dtype
        assert _rel(torch.stack([got[0].float(), got[1].float()], -1), want) < tol_f, name
    assert _rel(gamma, ref[3]) < tol_f
    if phase:
        assert _rel(rot[0], ref[4][0]) < tol_f and _rel(rot[1], ref[4][1]) < tol_f
    else:
        assert rot is None
    # one seeded cotangent per output
    g = torch.Generator().manual_seed(77)
    cot = [torch.randn(x.shape, generator=g, dtype=torch.float64) for x in (ref[0], ref[1], ref[2], ref[3])]
    loss_ref = sum((a * c).sum() for a, c in zip(ref[:4], cot))
    loss = sum((torch.stack([p[0].float(), p[1].float()], -1) * c.to(dev).float()).sum()
               for p, c in zip((q, k, v), cot[:3])) + (gamma * cot[3].to(dev).float()).sum()
    if phase:
        cr = [torch.randn(ref[4][0].shape, generator=g, dtype=torch.float64) for _ in range(2)]
        loss_ref = loss_ref + (ref[4][0] * cr[0]).sum() + (ref[4][1] * cr[1]).sum()
        loss = loss + (rot[0] * cr[0].to(dev).float()).sum() + (rot[1] * cr[1].to(dev).float()).sum()
    loss_ref.backward()
    loss.backward()
    dp = proj.grad.float().cpu()
    assert proj.grad.dtype == dtype
    n = 3 * H * d
    got_qkv = torch.stack([dp[..., :n].reshape(B, T, 3, H, d), dp[..., n:2 * n].reshape(B, T, 3, H, d)], -1)
    assert _rel(got_qkv, leaves[0].grad) < tol_g, "dqkv"
    assert _rel(dp[..., 2 * n:2 * n + H], leaves[1].grad) < tol_g, "ddt"
    assert torch.all(dp[..., 2 * n + H:] == 0), "padding columns"
    names = ["dbias", "doffset", "dprotect", "dphase", "drouting"]
    for name, a, b in zip(names, gl, leaves[2:]):
        if a is None:
            continue
        assert math.isfinite(a.grad.float().abs().sum().item()), name
        assert _rel(a.grad, b.grad) < tol_g, f"{name}: {_rel(a.grad, b.grad):.2e}"


@pytest.mark.parametrize("case", [CASES[0], CASES[2], CASES[3]])
@pytest.mark.parametrize("pdtype", [torch.float32, torch.bfloat16])
def test_prologue_gate_matrix_and_params(gpu_lib, case, pdtype):
    """The layer's form of the call: protect and phase as columns of one gate
    matrix whose gradient comes back whole, the decay bias given as two
    vectors (dt_bias and the dt projection's own bias, summed in the kernel),
    dt_bias / dt_bias2 / state_offset in fp32 or bf16 with their gradients in
    that dtype (formed by the in-call fixed-order reduction)."""
    from qllm2_amd.decode import build_rope_cache
    from qllm2_amd.pam_prologue import pam_prologue, proj_columns
    M, offset, gsp, phase, routing, qk_norm, floor, T = case
    B, H, d, dtype = 2, 3, 64, torch.bfloat16
    qkv, dt, bias, off, prot, ph, ro = _inputs(M, offset is not None, gsp, phase, routing, T, 900 + M + T)
    rnd = (lambda t: t.to(dtype).float() if t is not None else None)
    qkv, dt, prot, ph = rnd(qkv), rnd(dt), rnd(prot), rnd(ph)
    b1 = (0.6 * bias).to(pdtype).float()
    b2 = (0.4 * bias).to(pdtype).float()
    off = off.to(pdtype).float() if off is not None else None
    rope = build_rope_cache(offset + T + 3, 64) if offset is not None else None
    leaves, ref = _oracle(qkv, dt, b1 + b2, off, prot, ph, None, rope, offset or 0, qk_norm, floor)
    dev = torch.device("cuda")
    C = proj_columns(H)
    proj = torch.cat([qkv[..., 0].reshape(B, T, 3 * H * d), qkv[..., 1].reshape(B, T, 3 * H * d), dt,
                      torch.zeros(B, T, C - 6 * H * d - H)], -1).to(dtype).to(dev).requires_grad_(True)
    cols = ([prot] if gsp else []) + ([ph.reshape(B, T, H * M)] if phase else [])
    gate = torch.cat(cols, -1).to(dtype).to(dev).requires_grad_(True)
    pcol, fcol = (0, H if gsp else 0) if phase else (0, -1)
    if not gsp:
        pcol = -1
    pb1, pb2 = (x.to(pdtype).to(dev).requires_grad_(True) for x in (b1, b2))
    poff = off.to(pdtype).to(dev).requires_grad_(True) if off is not None else None
    q, k, v, gamma, rot = pam_prologue(proj, pb1, dt_bias2=pb2, n_heads=H, n_states=M, state_offset=poff,
                                       gate=gate, protect_col=pcol, phase_col=fcol,
                                       rope=rope.to(dev) if rope is not None else None, rope_offset=offset or 0,
                                       qk_norm=qk_norm, gamma_floor=floor)
    for name, got, want in (("q", q, ref[0]), ("k", k, ref[1]), ("v", v, ref[2])):
        assert _rel(torch.stack([got[0].float(), got[1].float()], -1), want) < 2e-2, name
    assert _rel(gamma, ref[3]) < 2e-2
    g = torch.Generator().manual_seed(78)
    cot = [torch.randn(x.shape, generator=g, dtype=torch.float64) for x in (ref[0], ref[1], ref[2], ref[3])]
    loss_ref = sum((a * c).sum() for a, c in zip(ref[:4], cot))
    loss = sum((torch.stack([p[0].float(), p[1].float()], -1) * c.to(dev).float()).sum()
               for p, c in zip((q, k, v), cot[:3])) + (gamma * cot[3].to(dev).float()).sum()
    if phase:
        assert rot is not None and _rel(rot[0], ref[4][0]) < 2e-2
        cr = [torch.randn(ref[4][0].shape, generator=g, dtype=torch.float64) for _ in range(2)]
        loss_ref = loss_ref + (ref[4][0] * cr[0]).sum() + (ref[4][1] * cr[1]).sum()
        loss = loss + (rot[0] * cr[0].to(dev).float()).sum() + (rot[1] * cr[1].to(dev).float()).sum()
    else:
        assert rot is None
    loss_ref.backward()
    loss.backward()
    dp = proj.grad.float().cpu()
    assert torch.all(dp[..., 6 * H * d + H:] == 0), "padding columns"
    assert _rel(dp[..., 6 * H * d:6 * H * d + H], leaves[1].grad) < 2e-2, "ddt"
    assert gate.grad.dtype == dtype and gate.grad.shape == gate.shape
    gg = gate.grad.float().cpu()
    if gsp:
        assert _rel(gg[..., pcol:pcol + H], leaves[4].grad) < 2e-2, "dprotect"
    if phase:
        assert _rel(gg[..., fcol:fcol + H * M].reshape(B, T, H, M), leaves[5].grad) < 2e-2, "dphase"
    for got in (pb1.grad, pb2.grad):
        assert got.dtype == pdtype
        assert _rel(got, leaves[2].grad) < 2e-2, "dbias"
    if poff is not None:
        assert poff.grad.dtype == pdtype and _rel(poff.grad, leaves[3].grad) < 2e-2, "doffset"


class _Lin(torch.nn.Module):
    def __init__(self, wr, wi):
        super().__init__()
        self.weight_real = torch.nn.Parameter(wr.clone())
        self.weight_imag = torch.nn.Parameter(wi.clone())
        self.bias_real = None


class _Layer(torch.nn.Module):
    """The attributes and the two helper methods of V11PAMLayer that the fused
    forward reads, holding the oracle's parameters."""

    def __init__(self, cfg, p, max_len=64):
        super().__init__()
        from qllm2_amd.decode import build_rope_cache
        h, d, m = cfg["n_heads"], cfg["head_dim"], cfg["n_states"]
        self.num_heads, self.head_dim, self.n_states = h, d, m
        self.inner_dim = h * d
        self.chunk_size, self.use_rope, self.use_gsp, self.qk_norm = (cfg["chunk_size"], cfg["use_rope"],
                                                                       cfg["use_gsp"], cfg["qk_norm"])
        self.gamma_floor, self.gate_content_aware = cfg["gamma_floor"], cfg["gate_content_aware"]
        self.routing_content_aware, self.state_compete = cfg["routing_content_aware"], cfg["state_compete"]
        self.fused_qkv, self.decay_mode, self.write_mode, self.fused_e3 = True, "head", "additive", True
        self.gate_surprisal_lambda = 0.0
        f = lambda t: t.float().clone()  # noqa: E731
        self.qkv_proj = _Lin(f(p["qkv_proj.weight_real"]), f(p["qkv_proj.weight_imag"]))
        self.o_proj = _Lin(f(p["o_proj.weight_real"]), f(p["o_proj.weight_imag"]))
        self.dt_proj = torch.nn.Linear(1, 1)
        self.dt_proj.weight = torch.nn.Parameter(f(p["dt_proj.weight"]))
        self.dt_proj.bias = torch.nn.Parameter(f(p["dt_proj.bias"]))
        self.dt_bias = torch.nn.Parameter(f(p["dt_bias"]))
        if cfg["use_gsp"]:
            self.protect_gate = torch.nn.Linear(1, 1)
            self.protect_gate.weight = torch.nn.Parameter(f(p["protect_gate.weight"]))
            self.protect_gate.bias = torch.nn.Parameter(f(p["protect_gate.bias"]))
        if m > 1:
            self.state_dt_offset = torch.nn.Parameter(f(p["state_dt_offset"]))
            self.phase_proj = torch.nn.Linear(1, 1)
            self.phase_proj.weight = torch.nn.Parameter(f(p["phase_proj.weight"]))
            self.phase_proj.bias = torch.nn.Parameter(f(p["phase_proj.bias"]))
            if cfg["state_compete"]:
                self.score_proj = torch.nn.Linear(1, 1)
                self.score_proj.weight = torch.nn.Parameter(f(p["score_proj.weight"]))
                self.score_proj.bias = torch.nn.Parameter(f(p["score_proj.bias"]))
        self.register_buffer("rope_cache", build_rope_cache(max_len, d), persistent=False)
        self.dropout = torch.nn.Dropout(0.0)

    def _phase_and_alpha(self, x):
        b, t = x.shape[:2]
        mag = torch.sqrt(x[..., 0].square() + x[..., 1].square() + 1e-8)
        r_in = torch.cat([x[..., 0], x[..., 1]], -1) if self.routing_content_aware else mag
        phase = self.phase_proj(r_in).view(b, t, self.num_heads, self.n_states)
        if self.state_compete:
            w = torch.softmax(self.score_proj(r_in).view(b, t, self.num_heads, self.n_states), -1) * self.n_states
        else:
            w = torch.ones_like(phase)
        return phase, w

    def _route_balance_loss(self, w):
        return None

    def forward(self, x, state=None, step_offset=0):
        from qllm2_amd import pam_layer
        return pam_layer.forward(self, x, state, step_offset)


LAYER_CASES = [  # cfg overrides, T, step_offset, tolerance
    (dict(n_states=3), 200, 0, 1e-4),
    (dict(n_states=3, state_compete=True, gamma_floor=0.3), 150, 40, 1e-4),
    (dict(n_states=1, qk_norm=True), 130, 7, 1e-4),
    (dict(n_states=1, chunk_size=256), 100, 0, 1e-4),
    (dict(n_states=3, head_dim=32), 100, 3, 1e-4),
    # qk-norm's backward over 128-wide rows: the oracle's own fp32 dx is 2.1e-4
    # from its float64 dx here, so fp32 parity is 2x that
    (dict(n_states=1, head_dim=128, qk_norm=True), 130, 0, 4e-4),
    (dict(n_states=2, head_dim=16, state_compete=True), 70, 5, 1e-4),
]


def _layer_cfg(**kw):
    c = dict(n_heads=2, head_dim=64, n_states=3, chunk_size=64, use_rope=True, use_gsp=True, qk_norm=False,
             gamma_floor=0.0, gate_content_aware=False, routing_content_aware=False, state_compete=False,
             max_seq_len=64)
    c.update(kw)
    return c


@pytest.mark.parametrize("over,T,offset,tol", LAYER_CASES)
def test_fused_layer_forward_matches_oracle(gpu_lib, over, T, offset, tol):
    """pam_layer.forward against the oracle's V11PAMLayer.forward restatement:
    output, final state, dL/dx and every parameter gradient (fp32; head dims
    16 to 128 on the prologue kernel)."""
    cfg = _layer_cfg(**over)
    dim = 48
    p = L.make_layer_params(cfg, dim, 900 + T)
    x = torch.randn(2, T, dim, 2, generator=torch.Generator().manual_seed(901 + T))
    dy = torch.randn(2, T, dim, 2, generator=torch.Generator().manual_seed(902 + T))
    pr = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    xr = x.double().requires_grad_(True)
    y_ref, s_ref = L.layer_forward(pr, cfg, xr, step_offset=offset)
    (y_ref * dy.double()).sum().backward()
    layer = _Layer(cfg, p).cuda()
    xc = x.cuda().requires_grad_(True)
    y, s = layer(xc, None, offset)
    (y * dy.cuda()).sum().backward()
    torch.cuda.synchronize()
    assert _rel(y, y_ref) < tol, f"y {_rel(y, y_ref):.2e}"
    assert _rel(s, s_ref) < tol, f"state {_rel(s, s_ref):.2e}"
    assert _rel(xc.grad, xr.grad) < tol, f"dx {_rel(xc.grad, xr.grad):.2e}"
    params = dict(layer.named_parameters())
    for name, ref_leaf in pr.items():
        got = params[name].grad
        assert got is not None, name
        assert _rel(got, ref_leaf.grad) < tol, f"{name}: {_rel(got, ref_leaf.grad):.2e}"


@pytest.mark.parametrize("head_dim,n_states", [(64, 3), (32, 3), (128, 1)])
def test_fused_layer_bf16(gpu_lib, head_dim, n_states):
    """The layer in bf16 (parameters and activations): bf16 projections, bf16
    scan operands with fp32 state; output and gradients within 2e-2 of the
    float64 oracle on the bf16-rounded parameters and input."""
    cfg = _layer_cfg(n_states=n_states, head_dim=head_dim)
    dim = 64
    p = {k: v.to(torch.bfloat16).double() for k, v in L.make_layer_params(cfg, dim, 950).items()}
    x = torch.randn(2, 256, dim, 2, generator=torch.Generator().manual_seed(951)).to(torch.bfloat16)
    dy = torch.randn(2, 256, dim, 2, generator=torch.Generator().manual_seed(952))
    pr = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    xr = x.double().requires_grad_(True)
    y_ref, _ = L.layer_forward(pr, cfg, xr)
    (y_ref * dy.double()).sum().backward()
    layer = _Layer(cfg, p).cuda().to(torch.bfloat16)
    layer.rope_cache = layer.rope_cache.float()
    xc = x.cuda().requires_grad_(True)
    y, _ = layer(xc)
    (y.float() * dy.cuda()).sum().backward()
    assert y.dtype == torch.bfloat16
    assert _rel(y, y_ref) < 2e-2
    assert _rel(xc.grad, xr.grad) < 2e-2
    params = dict(layer.named_parameters())
    for name in ("qkv_proj.weight_real", "o_proj.weight_imag", "dt_bias", "state_dt_offset", "phase_proj.weight",
                 "protect_gate.weight"):
        if name in pr:  # the one-state layer has no state offsets or phase projection
            assert _rel(params[name].grad, pr[name].grad) < 2e-2, name


def test_fused_layer_graph_capture(gpu_lib):
    """The fused layer's forward and backward captured in one HIP graph: three
    replays on new inputs (copied into the captured input buffer), with eager
    steps and host synchronisations between them, each give the eager output,
    dx and parameter gradients of the same input (fp32, rel 1e-6: the scan's
    reductions run in a fixed order; a wrong replay would be off by the size of
    the values)."""
    cfg = _layer_cfg(n_states=3)
    dim = 48
    p = L.make_layer_params(cfg, dim, 970)
    layer = _Layer(cfg, p).cuda()
    params = list(layer.parameters())
    gen = torch.Generator().manual_seed(971)
    dy = torch.randn(2, 128, dim, 2, generator=gen).cuda()

    def eager(x):
        xx = x.clone().requires_grad_(True)
        y, _ = layer(xx)
        return [y.detach()] + list(torch.autograd.grad(y, [xx] + params, dy))

    static_x = torch.randn(2, 128, dim, 2, generator=gen).cuda().requires_grad_(True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            y, _ = layer(static_x)
            torch.autograd.grad(y, [static_x] + params, dy)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        y_static, _ = layer(static_x)
        g_static = torch.autograd.grad(y_static, [static_x] + params, dy)
    for i in range(3):
        x = torch.randn(2, 128, dim, 2, generator=gen).cuda()
        want = eager(x)
        torch.cuda.synchronize()
        static_x.data.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        got = [y_static] + list(g_static)
        for a, b in zip(got, want):
            assert _rel(a, b) < 1e-6, f"replay {i}: {_rel(a, b):.2e}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cabs_matches_oracle(gpu_lib, dtype):
    """The cabs kernel (|z| with the reference's +1e-8) and its backward
    against the oracle's cabs under float64 autograd; a zero element keeps a
    finite gradient (|z| >= 1e-4)."""
    from qllm2_amd.pam_prologue import cabs
    g = torch.Generator().manual_seed(31)
    z = torch.randn(3, 50, 16, 2, generator=g).to(dtype).float()
    z[0, 0, 0] = 0.0
    gm = torch.randn(3, 50, 16, generator=g)
    zr = z.double().requires_grad_(True)
    mr = L.cabs(zr)
    (mr * gm.double()).sum().backward()
    zc = z.to(dtype).cuda().requires_grad_(True)
    m = cabs(zc)
    (m.float() * gm.cuda()).sum().backward()
    tol = 1e-6 if dtype == torch.float32 else 1e-2
    assert m.dtype == dtype and _rel(m, mr) < tol
    assert zc.grad.dtype == dtype and _rel(zc.grad, zr.grad) < tol
    assert torch.isfinite(zc.grad.float()).all()


@pytest.mark.parametrize("dtype,out_dtype", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                             (torch.bfloat16, torch.float32)])
def test_mag_linear_matches_oracle(gpu_lib, dtype, out_dtype):
    """The decode step's gate logits from |x| (qpam_mag_linear: cabs then the
    protect-gate and phase rows in one launch) against the oracle's cabs and a
    float64 matmul; rows of odd length, with and without bias."""
    from qllm2_amd.pam_prologue import mag_linear
    g = torch.Generator().manual_seed(41)
    for n, dim, G, bias in ((193, 768, 48, True), (5, 100, 7, False), (1, 1536, 12, True)):
        z = torch.randn(n, dim, 2, generator=g).to(dtype)
        w = torch.randn(G, dim, generator=g) * dim ** -0.5
        b = torch.randn(G, generator=g) if bias else None
        ref = L.cabs(z.double()) @ w.double().T + (b.double() if bias else 0.0)
        out = mag_linear(z.cuda(), w.cuda(), b.cuda() if bias else None, out_dtype=out_dtype)
        assert out.dtype == out_dtype and tuple(out.shape) == (n, G)
        tol = 1e-5 if out_dtype == torch.float32 else 1e-2
        assert _rel(out, ref) < tol, f"n={n} dim={dim}: {_rel(out, ref):.2e}"
