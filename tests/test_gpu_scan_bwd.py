"""GPU parity of the scan backward (qpam_scan_bwd through torch autograd)
against autograd of the CPU oracle, the way the reference gets its gradients.

Loss = sum(Y * dY) + sum(S * dS) with seeded dY, dS.  Tolerances (north
star): fp32 inputs rel <= 1e-4 on every gradient (max-abs relative to the
reference gradient); bf16 inputs with fp32 state rel <= 2e-2.
"""

import math

import pytest
import torch

from oracle import pam as O

pytestmark = pytest.mark.gpu


def _rel(a, b):
    return ((a.double() - b.double()).abs().max() / (b.double().abs().max() + 1e-30)).item()


def _rel_heads(a, b, lead):
    """Largest per-head relative error: max |a - b| / max |b| within each slice
    over the first `lead` dimensions ((b, h) or (m, b, h)), then the max over
    slices."""
    a, b = a.double(), b.double()
    err = (a - b).abs().flatten(lead).amax(-1)
    ref = b.abs().flatten(lead).amax(-1)
    return (err / (ref + 1e-30)).max().item()


# leading (per-head) dimensions of each gradient: dq, dk, dv [B,H,T,d,2];
# dgamma, dphase, drouting [M,B,H,T]; ds0 [M,B,H,d,d,2]
LEAD = [2, 2, 2, 3, 3, 3, 3]


def _check(got, ref, tol, names=None):
    for name, lead, a, b in zip(names or NAMES, LEAD, got, ref):
        if a is None or b is None:
            continue
        assert math.isfinite(a.abs().sum().item()), name
        assert _rel(a, b) < tol, f"{name}: rel {_rel(a, b):.2e}"
        assert _rel_heads(a, b, lead) < tol, f"{name}: worst head rel {_rel_heads(a, b, lead):.2e}"


def _case(M, B, H, T, d, seed, with_rot, with_s0, dtype):
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, seed, m_states=M, gamma_mu=2.0 if M > 1 else 3.0,
                                        gamma_mu_step=1.0 if M > 1 else 0.0, unit_qk=True, dtype=torch.float32)
    q, k, v = (x.to(dtype).to(torch.float32) for x in (q, k, v))  # rounded values both sides see
    g = torch.Generator().manual_seed(seed + 1)
    dy = torch.randn(B, H, T, d, 2, generator=g)
    ds = torch.randn(M, B, H, d, d, 2, generator=g) * 0.1
    phase = torch.randn(M, B, H, T, generator=g) if with_rot else torch.zeros(M, B, H, T)
    routing = (torch.rand(M, B, H, T, generator=g) + 0.5) if with_rot else torch.ones(M, B, H, T)
    s0 = torch.randn(M, B, H, d, d, 2, generator=g) * 0.1 if with_s0 else None
    return q, k, v, gamma, dy, ds, phase, routing, s0


def _oracle_grads(q, k, v, gamma, dy, ds, phase, routing, s0, d, C):
    xs = [x.double().clone().requires_grad_(True) for x in (q, k, v, gamma, phase, routing)]
    s0d = s0.double().clone().requires_grad_(True) if s0 is not None else None
    y, s = O.multistate_fused(xs[0], xs[1], xs[2], xs[3], xs[4], xs[5], d, C, state=s0d)
    ((y * dy.double()).sum() + (s * ds.double()).sum()).backward()
    out = [x.grad for x in xs]
    out.append(s0d.grad if s0d is not None else None)
    return out


def _gpu_grads(q, k, v, gamma, dy, ds, phase, routing, s0, d, C, dtype, with_rot, outs=None):
    from qllm2_amd.pam_scan import pam_scan_planar
    dev = torch.device("cuda")

    def leaf(x):
        return x.to(dev).requires_grad_(True)

    planes = [leaf(x[..., i].contiguous().to(dtype)) for x in (q, k, v) for i in (0, 1)]
    gam = leaf(gamma.float())
    ph, ro = leaf(phase.float()), leaf(routing.float())
    rot = (ro * torch.cos(ph), ro * torch.sin(ph)) if with_rot else None
    s0p = None
    if s0 is not None:
        s0r, s0i = leaf(s0[..., 0].contiguous()), leaf(s0[..., 1].contiguous())
        s0p = (s0r, s0i)
    y_re, y_im, s_re, s_im = pam_scan_planar(*planes, gam, q_scale=d ** -0.5, chunk=C, rot=rot, s0=s0p)
    if outs is not None:
        outs["y"] = torch.stack([y_re, y_im], -1).detach().float().cpu()
        outs["s"] = torch.stack([s_re, s_im], -1).detach().float().cpu()
    dyd, dsd = dy.to(dev), ds.to(dev)
    loss = ((y_re * dyd[..., 0]).sum() + (y_im * dyd[..., 1]).sum() + (s_re * dsd[..., 0]).sum()
            + (s_im * dsd[..., 1]).sum())
    loss.backward()
    torch.cuda.synchronize()

    def cpx(a, b):
        return torch.stack([a.grad.float(), b.grad.float()], -1).cpu()

    out = [cpx(planes[0], planes[1]), cpx(planes[2], planes[3]), cpx(planes[4], planes[5]), gam.grad.cpu()]
    out += [ph.grad.cpu() if with_rot else None, ro.grad.cpu() if with_rot else None]
    out.append(torch.stack([s0p[0].grad, s0p[1].grad], -1).cpu() if s0 is not None else None)
    return out


NAMES = ["dq", "dk", "dv", "dgamma", "dphase", "drouting", "ds0"]


@pytest.mark.parametrize("M,T,C,with_rot,with_s0", [
    (1, 64, 64, False, False), (1, 200, 64, False, False), (1, 100, 32, False, True),
    (3, 150, 64, True, True), (2, 70, 16, True, False),
])
def test_scan_backward_fp32(gpu_lib, M, T, C, with_rot, with_s0):
    B, H, d = 2, 2, 64
    case = _case(M, B, H, T, d, 3000 + M * 7 + T + C, with_rot, with_s0, torch.float32)
    ref = _oracle_grads(*case, d, C)
    got = _gpu_grads(*case, d, C, torch.float32, with_rot)
    _check(got, ref, 1e-4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_scan_backward_strided_gamma_and_rot(gpu_lib, dtype):
    """gamma and the rotation planes as permuted views of [B,T,H,M] tensors (the
    layout V11PAMLayer._forward_multistate_fused hands over, v11/model.py:746-748):
    dgamma, dphase and drouting against oracle autograd."""
    M, B, H, T, d, C = 2, 2, 3, 40, 64, 64
    case = list(_case(M, B, H, T, d, 3400, True, False, dtype))
    ref = _oracle_grads(*case, d, C)
    from qllm2_amd.pam_scan import pam_scan_planar
    dev = torch.device("cuda")
    q, k, v, gamma, dy, ds, phase, routing, _ = case
    planes = [x[..., i].contiguous().to(dtype).to(dev).requires_grad_(True) for x in (q, k, v) for i in (0, 1)]
    # [B,T,H,M] storage, [M,B,H,T] views
    gam = gamma.permute(1, 3, 2, 0).contiguous().to(dev).requires_grad_(True)
    ph = phase.permute(1, 3, 2, 0).contiguous().to(dev).requires_grad_(True)
    ro = routing.permute(1, 3, 2, 0).contiguous().to(dev).requires_grad_(True)
    g4, p4, r4 = (x.permute(3, 0, 2, 1) for x in (gam, ph, ro))
    assert not g4.is_contiguous()
    rot = (r4 * torch.cos(p4), r4 * torch.sin(p4))
    y_re, y_im, s_re, s_im = pam_scan_planar(*planes, g4, q_scale=d ** -0.5, chunk=C, rot=rot)
    dyd, dsd = dy.to(dev), ds.to(dev)
    ((y_re * dyd[..., 0]).sum() + (y_im * dyd[..., 1]).sum() + (s_re * dsd[..., 0]).sum()
     + (s_im * dsd[..., 1]).sum()).backward()
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    for name, got, want in (("dgamma", gam.grad, ref[3]), ("dphase", ph.grad, ref[4]), ("drouting", ro.grad, ref[5])):
        got = got.permute(3, 0, 2, 1).cpu()
        assert _rel(got, want) < tol, f"{name}: rel {_rel(got, want):.2e}"


@pytest.mark.parametrize("M,d,T,C,dtype,with_rot,with_s0", [
    (1, 128, 150, 64, torch.float32, False, True),   # 2 x 2 state blocks of 64 x 64
    (2, 96, 100, 32, torch.float32, True, True),     # padded to 128
    (1, 48, 90, 16, torch.float32, False, True),     # padded to 64 (48 does not divide 64)
    (6, 64, 130, 64, torch.float32, True, True),     # two kernel calls of three states
    (5, 64, 200, 64, torch.bfloat16, True, True),    # bf16 segment kernels, groups of 3 + 2 states
    (2, 128, 200, 64, torch.bfloat16, True, False),
    (5, 128, 70, 32, torch.float32, True, True),     # both
])
def test_scan_any_head_dim_and_state_count(gpu_lib, M, d, T, C, dtype, with_rot, with_s0):
    """Head dims other than 64 and more than four states (the reference's layer
    takes any head_dim and n_states, v11/model.py:45-97): Y, the final state
    and every gradient against oracle autograd at the true head dim."""
    B, H = 2, 2
    case = _case(M, B, H, T, d, 3600 + M * 13 + d + T, with_rot, with_s0, dtype)
    q, k, v, gamma, dy, ds, phase, routing, s0 = case
    with torch.no_grad():
        y_ref, s_ref = O.multistate_fused(q.double(), k.double(), v.double(), gamma.double(), phase.double(),
                                          routing.double(), d, C,
                                          state=s0.double() if s0 is not None else None)
    ref = _oracle_grads(*case, d, C)
    outs = {}
    got = _gpu_grads(*case, d, C, dtype, with_rot, outs)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert outs["y"].shape == y_ref.shape and outs["s"].shape == s_ref.shape
    assert _rel(outs["y"], y_ref) < tol and _rel_heads(outs["y"], y_ref, 2) < tol
    assert _rel(outs["s"], s_ref) < tol and _rel_heads(outs["s"], s_ref, 3) < tol
    _check(got, ref, tol)


@pytest.mark.parametrize("M,d", [(5, 64), (2, 128), (5, 96)])
def test_scan_head_merged_y_any_shape(gpu_lib, M, d):
    """The head-merged layouts for shapes the kernels take in pieces: 'bt2hd'
    holds the [B,H,T,d] planes moved into [B,T,2,H,d] (the kernels may sum in
    another order per layout: rel 1e-6), and 'bt2hd_bf16' is that fp32 tensor
    rounded once (the state groups are summed in fp32)."""
    from qllm2_amd.pam_scan import pam_scan_planar
    g = torch.Generator().manual_seed(71 + M + d)
    B, H, T = 2, 2, 150
    planes = [(torch.randn(B, H, T, d, generator=g) * 0.5).to(torch.bfloat16).cuda() for _ in range(6)]
    gamma = (0.8 + 0.19 * torch.rand(M, B, H, T, generator=g)).cuda()
    rot = tuple(torch.randn(M, B, H, T, generator=g).cuda() for _ in range(2))
    with torch.no_grad():
        y_re, y_im, s_re, _ = pam_scan_planar(*planes, gamma, q_scale=d ** -0.5, chunk=64, rot=rot)
        y32, none32, s32, _ = pam_scan_planar(*planes, gamma, q_scale=d ** -0.5, chunk=64, rot=rot,
                                              y_layout="bt2hd")
        y16, none16, s16, _ = pam_scan_planar(*planes, gamma, q_scale=d ** -0.5, chunk=64, rot=rot,
                                              y_layout="bt2hd_bf16")
    assert none32 is None and none16 is None
    assert y32.shape == (B, T, 2, H, d) and y16.dtype == torch.bfloat16
    assert _rel(y32, torch.stack([y_re.transpose(1, 2), y_im.transpose(1, 2)], 2)) < 1e-6
    assert torch.equal(y16, y32.to(torch.bfloat16))
    assert _rel(s32, s_re) < 1e-6 and torch.equal(s16, s32)


def test_scan_backward_bf16_e3(gpu_lib):
    M, B, H, T, d, C = 3, 2, 2, 512, 64, 64
    case = _case(M, B, H, T, d, 3303, False, False, torch.bfloat16)
    ref = _oracle_grads(*case, d, C)
    got = _gpu_grads(*case, d, C, torch.bfloat16, False)
    _check(got, ref, 2e-2)


@pytest.mark.parametrize("M,T,with_rot,with_s0", [
    (3, 40, True, True),     # one partial chunk
    (3, 150, True, True),    # odd chunk count, ragged last chunk
    (1, 200, False, False),  # even chunk count, ragged last chunk, no rotation
    (2, 128, True, False),   # two full chunks
    (3, 64 * 6 + 10, True, True),  # seven chunks: a full segment of four, then a segment of three
    (2, 64 * 9, True, True),       # nine chunks: the last segment holds one chunk
])
def test_scan_backward_bf16_ragged(gpu_lib, M, T, with_rot, with_s0):
    """bf16 inputs (the segment kernels, four 64-step chunks per segment) at
    sequence lengths that are not a multiple of the chunk, chunk counts of 1, 2,
    odd and even, and segment counts with a partial last segment: every gradient
    against oracle autograd."""
    B, H, d, C = 2, 2, 64, 64
    case = _case(M, B, H, T, d, 3500 + M * 11 + T, with_rot, with_s0, torch.bfloat16)
    ref = _oracle_grads(*case, d, C)
    got = _gpu_grads(*case, d, C, torch.bfloat16, with_rot)
    _check(got, ref, 2e-2)


def test_scan_backward_config3_full_size(gpu_lib):
    """Config 3: E3 M=3, B=8, T=2048, H=12, d=64, C=64, bf16 q/k/v, fp32 state,
    dY complex N(0,1); oracle autograd in fp32 on the bf16-rounded inputs."""
    M, B, H, T, d, C = 3, 8, 12, 2048, 64, 64
    q, k, v, gamma = O.make_scan_inputs(B, H, T, d, 1003, m_states=M, gamma_mu=2.0, gamma_mu_step=1.0,
                                        unit_qk=True, dtype=torch.float32)
    q, k, v = (x.to(torch.bfloat16).to(torch.float32) for x in (q, k, v))
    g = torch.Generator().manual_seed(1003 + 1)
    dy = torch.randn(B, H, T, d, 2, generator=g)
    ds = torch.zeros(M, B, H, d, d, 2)
    phase, routing = torch.zeros(M, B, H, T), torch.ones(M, B, H, T)
    xs = [x.clone().requires_grad_(True) for x in (q, k, v, gamma)]
    y, s = O.multistate_fused(xs[0], xs[1], xs[2], xs[3], phase, routing, d, C)
    (y * dy).sum().backward()
    ref = [x.grad for x in xs]
    y_ref, s_ref = y.detach(), s.detach()
    del y, s
    outs = {}
    got = _gpu_grads(q, k, v, gamma, dy, ds, phase, routing, None, d, C, torch.bfloat16, False, outs)
    assert _rel(outs["y"], y_ref) < 2e-2 and _rel_heads(outs["y"], y_ref, 2) < 2e-2
    assert _rel(outs["s"], s_ref) < 2e-2 and _rel_heads(outs["s"], s_ref, 3) < 2e-2
    _check(got[:4], ref, 2e-2, NAMES[:4])


def test_scan_bf16_e3_decay_regimes(gpu_lib):
    """One E3 call whose chunks take both decay paths of the bf16 kernels: chunks
    where every log(gamma + 1e-6) <= 0 with a moderate range (factorised decay)
    and chunks that need the per-element exact form -- gamma = 1 (the clamp of
    min(L_t - L_s, 0) is active) and gamma = 0.05 (cumulative decay beyond the
    factorisation range).  Forward Y, S and every gradient against the oracle."""
    from qllm2_amd.pam_scan import pam_scan_planar
    M, B, H, T, d, C = 3, 1, 2, 320, 64, 64
    case = list(_case(M, B, H, T, d, 3404, True, True, torch.bfloat16))
    gamma = case[3].clone()
    gamma[:, :, :, 64:128] = 1.0       # chunk 1: clamp regime in every state
    gamma[:, :, 1, 128:192] = 0.05     # chunk 2, head 1: exp(-L) would overflow
    gamma[0, :, 0, 192:256] = 1.0      # chunk 3, head 0: one state clamps, the others factorise
    case[3] = gamma
    ref = _oracle_grads(*case, d, C)
    got = _gpu_grads(*case, d, C, torch.bfloat16, True)
    for name, a, b in zip(NAMES, got, ref):
        if a is None or b is None:
            continue
        assert math.isfinite(a.abs().sum().item()), name
        assert _rel(a, b) < 2e-2, f"{name}: rel {_rel(a, b):.2e}"
    q, k, v, gamma, dy, ds, phase, routing, s0 = case
    y_ref, s_ref = O.multistate_fused(q.double(), k.double(), v.double(), gamma.double(), phase.double(),
                                      routing.double(), d, C, state=s0.double())
    dev = torch.device("cuda")
    planes = [x[..., i].contiguous().to(torch.bfloat16).to(dev) for x in (q, k, v) for i in (0, 1)]
    rot = ((routing * torch.cos(phase)).to(dev), (routing * torch.sin(phase)).to(dev))
    s0p = (s0[..., 0].contiguous().to(dev), s0[..., 1].contiguous().to(dev))
    with torch.no_grad():
        y_re, y_im, s_re, s_im = pam_scan_planar(*planes, gamma.float().to(dev), q_scale=d ** -0.5, chunk=C,
                                                 rot=rot, s0=s0p)
    y = torch.stack([y_re, y_im], -1).cpu()
    s = torch.stack([s_re, s_im], -1).cpu()
    assert _rel(y, y_ref) < 2e-2, f"y: rel {_rel(y, y_ref):.2e}"
    assert _rel(s, s_ref) < 2e-2, f"s: rel {_rel(s, s_ref):.2e}"


@pytest.mark.parametrize("T", [200, 2048])
def test_bf16_head_merged_y_equals_rounded_fp32(gpu_lib, T):
    """y_layout 'bt2hd_bf16' (E3, bf16 inputs, chunk 64): y is the fp32
    result rounded once, so it equals the 'bt2hd' fp32 y rounded to bf16 bit
    for bit; a bf16 dy gives the gradients of the same dy widened to fp32 (the
    backward's LDS partial sums may add in another order: rel 1e-6)."""
    from qllm2_amd.pam_scan import pam_scan_planar
    g = torch.Generator().manual_seed(31 + T)
    M, B, H, d = 3, 2, 2, 64
    planes = [(torch.randn(B, H, T, d, generator=g) * 0.5).to(torch.bfloat16).cuda() for _ in range(6)]
    gamma = (0.8 + 0.19 * torch.rand(M, B, H, T, generator=g)).cuda()
    rot = tuple(torch.randn(M, B, H, T, generator=g).cuda() for _ in range(2))
    dy = (torch.randn(B, T, 2, H, d, generator=g)).to(torch.bfloat16).cuda()

    def run(layout, dy_in):
        ins = [p.clone().requires_grad_(True) for p in planes]
        gm = gamma.clone().requires_grad_(True)
        rr = [r.clone().requires_grad_(True) for r in rot]
        y, _, s_re, s_im = pam_scan_planar(*ins, gm, q_scale=d ** -0.5, chunk=64, rot=tuple(rr), y_layout=layout)
        grads = torch.autograd.grad(y, ins + [gm] + rr, dy_in)
        torch.cuda.synchronize()
        return y, s_re, grads

    y32, s32, g32 = run("bt2hd", dy.float())
    y16, s16, g16 = run("bt2hd_bf16", dy)
    assert y16.dtype == torch.bfloat16 and y16.shape == (B, T, 2, H, d)
    assert torch.equal(y16, y32.to(torch.bfloat16))
    assert torch.equal(s16, s32)
    for a, b in zip(g16, g32):
        assert a.dtype == b.dtype
        assert _rel(a, b) < 1e-6


def _random_cases(n, seed):
    g = torch.Generator().manual_seed(seed)
    pick = (lambda xs: xs[int(torch.randint(len(xs), (1,), generator=g))])
    cases = []
    for i in range(n):
        cases.append((pick([1, 2, 3, 4, 5, 6]), pick([16, 32, 48, 64, 80, 128]), int(torch.randint(1, 260, (1,), generator=g)),
                      pick([16, 32, 64]), pick(["f32", "bf16"]), bool(torch.randint(2, (1,), generator=g)),
                      bool(torch.randint(2, (1,), generator=g))))
    return cases


@pytest.mark.parametrize("M,d,T,C,dt,with_rot,with_s0", _random_cases(10, 4242))
def test_scan_seeded_random_shapes(gpu_lib, M, d, T, C, dt, with_rot, with_s0):
    """Seeded random shapes across every axis the scan takes (states 1-6, head
    dims below, at and above 64, lengths 1-259, chunks 16/32/64, fp32 and bf16,
    with and without rotations and a start state): Y, S and every gradient
    against oracle autograd."""
    dtype = torch.float32 if dt == "f32" else torch.bfloat16
    B, H = 1, 2
    case = _case(M, B, H, T, d, 4300 + M * 17 + d + T + C, with_rot, with_s0, dtype)
    q, k, v, gamma, dy, ds, phase, routing, s0 = case
    with torch.no_grad():
        y_ref, s_ref = O.multistate_fused(q.double(), k.double(), v.double(), gamma.double(), phase.double(),
                                          routing.double(), d, C,
                                          state=s0.double() if s0 is not None else None)
    ref = _oracle_grads(*case, d, C)
    outs = {}
    got = _gpu_grads(*case, d, C, dtype, with_rot, outs)
    tol = 1e-4 if dtype == torch.float32 else 2e-2
    assert _rel(outs["y"], y_ref) < tol and _rel_heads(outs["y"], y_ref, 2) < tol
    assert _rel(outs["s"], s_ref) < tol and _rel_heads(outs["s"], s_ref, 3) < tol
    _check(got, ref, tol)


@pytest.mark.parametrize("dtype,M,T,C", [(torch.bfloat16, 3, 1024, 64), (torch.float32, 2, 300, 64),
                                         (torch.float32, 3, 200, 32)])
def test_scan_backward_deterministic(gpu_lib, dtype, M, T, C):
    """Two backward passes over the same inputs give bit-identical gradients
    (the kernels' reductions run in a fixed order, no floating-point atomics):
    the E3 bf16 path at B=4, H=12 (many blocks in flight at once) and the fp32
    paths with 64- and 32-step chunks."""
    B, H, d = 4, 12, 64
    case = _case(M, B, H, T, d, 5100 + M + T + C, True, True, dtype)
    runs = [_gpu_grads(*case, d, C, dtype, True) for _ in range(2)]
    for name, a, b in zip(NAMES, runs[0], runs[1]):
        if a is not None:
            assert torch.equal(a, b), f"{name}: differs between two runs"
