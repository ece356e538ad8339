"""GPU parity of the E2 delta-rule kernels (qpam_delta_fwd / qpam_delta_bwd)
against the CPU oracle (oracle/delta.py: the reference's chunked UT-transform
form and its token recurrence) in float64, fp32 rel <= 1e-4 on Y, S and every
gradient (dq, dk, dv, dgamma, dbeta, ds0)."""

import math

import pytest
import torch

from oracle import delta as D

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def _run(q, k, v, g, b, s0, dy, ds, eps, d=64):
    from qllm2_amd.pam_delta import delta_planar
    dev = torch.device("cuda")
    planes = [x[..., i].contiguous().float().to(dev).requires_grad_(True) for x in (q, k, v) for i in (0, 1)]
    gg, bb = g.float().to(dev).requires_grad_(True), b.float().to(dev).requires_grad_(True)
    s0p = None
    if s0 is not None:
        s0p = tuple(s0[..., i].contiguous().float().to(dev).requires_grad_(True) for i in (0, 1))
    y_re, y_im, s_re, s_im = delta_planar(*planes, gg, bb, q_scale=d ** -0.5, gamma_eps=eps, s0=s0p)
    loss = (y_re * dy[..., 0].to(dev)).sum() + (y_im * dy[..., 1].to(dev)).sum()
    if ds is not None:
        loss = loss + (s_re * ds[..., 0].to(dev)).sum() + (s_im * ds[..., 1].to(dev)).sum()
    loss.backward()
    torch.cuda.synchronize()
    cpx = (lambda a, b: torch.stack([a.grad, b.grad], -1).cpu())
    grads = [cpx(planes[0], planes[1]), cpx(planes[2], planes[3]), cpx(planes[4], planes[5]), gg.grad.cpu(),
             bb.grad.cpu(), cpx(*s0p) if s0p is not None else None]
    return torch.stack([y_re, y_im], -1).detach().cpu(), torch.stack([s_re, s_im], -1).detach().cpu(), grads


def _ref(q, k, v, g, b, s0, dy, ds, chunked, d=64):
    xs = [x.double().clone().requires_grad_(True) for x in (q, k, v, g, b)]
    s0r = s0.double().clone().requires_grad_(True) if s0 is not None else None
    if chunked:
        y, s = D.delta_chunked(*xs, d, 64, state=s0r)
    else:
        y, s = D.delta_recurrent(*xs, d, state=s0r, eps=0.0)
    loss = (y * dy.double()).sum() + ((s * ds.double()).sum() if ds is not None else 0)
    loss.backward()
    return y.detach(), s.detach(), [x.grad for x in xs] + [s0r.grad if s0r is not None else None]


NAMES = ["dq", "dk", "dv", "dgamma", "dbeta", "ds0"]


@pytest.mark.parametrize("T,with_s0,with_ds", [(64, False, False), (100, True, True), (37, False, True),
                                               (1, True, False), (16, False, False), (130, True, False)])
def test_delta_matches_chunked_oracle(gpu_lib, T, with_s0, with_ds):
    """The reference's chunked UT-transform form (delta_chunk 64) in float64
    against the kernels with gamma + 1e-6: outputs, final state, all gradients;
    ragged T (a partial last 64-step chunk, T below one chunk)."""
    B, H, d = 2, 3, 64
    q, k, v, g, b = D.make_delta_inputs(B, H, T, d, 600 + T)
    gen = torch.Generator().manual_seed(601 + T)
    s0 = torch.randn(B, H, d, d, 2, generator=gen, dtype=torch.float64) * 0.05 if with_s0 else None
    dy = torch.randn(B, H, T, d, 2, generator=gen, dtype=torch.float64)
    ds = torch.randn(B, H, d, d, 2, generator=gen, dtype=torch.float64) * 0.1 if with_ds else None
    y, s, grads = _run(q, k, v, g, b, s0, dy, ds, 1e-6)
    yr, sr, rgrads = _ref(q, k, v, g, b, s0, dy, ds, chunked=True)
    assert _rel(y, yr) < 1e-4, f"y {_rel(y, yr):.2e}"
    assert _rel(s, sr) < 1e-4, f"s {_rel(s, sr):.2e}"
    for name, a, r in zip(NAMES, grads, rgrads):
        if a is None or r is None:
            continue
        assert math.isfinite(a.abs().sum().item()), name
        assert _rel(a, r) < 1e-4, f"{name}: {_rel(a, r):.2e}"


@pytest.mark.parametrize("d,T", [(32, 100), (16, 70), (48, 130)])
def test_delta_small_head_dims(gpu_lib, d, T):
    """Head dims below 64 (the reference's small presets use 32) run zero-padded
    to 64 and sliced back: Y, S and every gradient against the chunked oracle
    at the true head dim (its own query scale d^-0.5)."""
    B, H = 2, 2
    q, k, v, g, b = D.make_delta_inputs(B, H, T, d, 660 + d + T)
    gen = torch.Generator().manual_seed(661 + d + T)
    s0 = torch.randn(B, H, d, d, 2, generator=gen, dtype=torch.float64) * 0.05
    dy = torch.randn(B, H, T, d, 2, generator=gen, dtype=torch.float64)
    ds = torch.randn(B, H, d, d, 2, generator=gen, dtype=torch.float64) * 0.1
    y, s, grads = _run(q, k, v, g, b, s0, dy, ds, 1e-6, d=d)
    yr, sr, rgrads = _ref(q, k, v, g, b, s0, dy, ds, chunked=True, d=d)
    assert y.shape == yr.shape and s.shape == sr.shape
    assert _rel(y, yr) < 1e-4, f"y {_rel(y, yr):.2e}"
    assert _rel(s, sr) < 1e-4, f"s {_rel(s, sr):.2e}"
    for name, a, r in zip(NAMES, grads, rgrads):
        assert a.shape == r.shape, name
        assert _rel(a, r) < 1e-4, f"{name}: {_rel(a, r):.2e}"


def test_delta_strided_gamma_and_beta(gpu_lib):
    """gamma and beta as transposed views of [B,T,H] tensors with equal strides
    (the layout of the reference's write_beta, v11/model.py:807): dgamma and
    dbeta against the chunked oracle."""
    from qllm2_amd.pam_delta import delta_planar
    B, H, T, d = 2, 3, 50, 64
    q, k, v, g, b = D.make_delta_inputs(B, H, T, d, 640)
    dy = torch.randn(B, H, T, d, 2, generator=torch.Generator().manual_seed(641), dtype=torch.float64)
    _, _, rgrads = _ref(q, k, v, g, b, None, dy, None, chunked=True)
    dev = torch.device("cuda")
    planes = [x[..., i].contiguous().float().to(dev) for x in (q, k, v) for i in (0, 1)]
    gt = g.transpose(1, 2).contiguous().float().to(dev).requires_grad_(True)   # [B,T,H] storage
    bt = b.transpose(1, 2).contiguous().float().to(dev).requires_grad_(True)
    gv, bv = gt.transpose(1, 2), bt.transpose(1, 2)
    assert not gv.is_contiguous() and gv.stride() == bv.stride()
    y_re, y_im, _, _ = delta_planar(*planes, gv, bv, q_scale=64 ** -0.5, gamma_eps=1e-6)
    ((y_re * dy[..., 0].to(dev)).sum() + (y_im * dy[..., 1].to(dev)).sum()).backward()
    assert _rel(gt.grad.transpose(1, 2), rgrads[3]) < 1e-4, "dgamma"
    assert _rel(bt.grad.transpose(1, 2), rgrads[4]) < 1e-4, "dbeta"


def test_delta_step_matches_reference_step(gpu_lib):
    """recur_step_delta (the decode drop-in, gamma without the chunked form's
    1e-6) against the reference step, several tokens in a row."""
    from qllm2_amd.pam_delta import recur_step_delta
    B, H, d = 2, 2, 64
    q, k, v, g, b = D.make_delta_inputs(B, H, 5, d, 650)
    s = torch.randn(B, H, d, d, 2, generator=torch.Generator().manual_seed(651), dtype=torch.float64) * 0.1
    sc = s.float().cuda()
    for t in range(5):
        qt = q[:, :, t] * d ** -0.5
        yr, s = D.recur_step_delta(s, g[:, :, t], v[:, :, t], k[:, :, t], qt, b[:, :, t])
        y, sc = recur_step_delta(sc, g[:, :, t].float().cuda(), v[:, :, t].float().cuda(), k[:, :, t].float().cuda(),
                                 qt.float().cuda(), b[:, :, t].float().cuda())
        assert _rel(y, yr) < 1e-4 and _rel(sc, s) < 1e-4


@pytest.mark.parametrize("chunk", [32, 20])
def test_delta_reference_chunk_length_strong_decay(gpu_lib, chunk):
    """The chunked form with the reference's own chunk length (delta_chunk 32,
    the tiny_e2 preset, v11/model.py:1326; 20, its self-test) under strong decay
    (gamma in 0.3..0.6: over 32-64 steps the within-chunk decay falls below the
    state-write weight's 1e-12, where the chunk boundaries change the result):
    y, the final state and every gradient against the chunked oracle run with
    the same chunk length, per (b, h)."""
    from qllm2_amd.pam_delta import delta_planar
    B, H, T, d = 2, 3, 150, 64
    q, k, v, g, b = D.make_delta_inputs(B, H, T, d, 700 + chunk)
    g = 0.3 + 0.3 * torch.rand(B, H, T, generator=torch.Generator().manual_seed(701), dtype=torch.float64)
    dy = torch.randn(B, H, T, d, 2, generator=torch.Generator().manual_seed(702), dtype=torch.float64)
    leaves = [x.clone().requires_grad_(True) for x in (q, k, v, g, b)]
    yr, sr = D.delta_chunked(*leaves[:3], leaves[3], leaves[4], d, chunk)
    (yr * dy).sum().backward()
    rgrads = [x.grad for x in leaves]
    # the 64-step form differs here (the check that the chunk length matters)
    y64, _ = D.delta_chunked(q, k, v, g, b, d, 64)
    assert _rel(y64, yr.detach()) > 1e-3
    dev = torch.device("cuda")
    planes = [x[..., i].contiguous().float().to(dev).requires_grad_(True) for x in (q, k, v) for i in (0, 1)]
    gg, bb = g.float().to(dev).requires_grad_(True), b.float().to(dev).requires_grad_(True)
    y_re, y_im, s_re, s_im = delta_planar(*planes, gg, bb, q_scale=d ** -0.5, gamma_eps=1e-6, chunk=chunk)
    ((y_re * dy[..., 0].to(dev)).sum() + (y_im * dy[..., 1].to(dev)).sum()).backward()
    assert _rel_heads(torch.stack([y_re, y_im], -1), yr) < 1e-4, "y"
    assert _rel_heads(torch.stack([s_re, s_im], -1), sr) < 1e-4, "s"
    for name, (re, im), r in zip(("dq", "dk", "dv"), ((planes[0], planes[1]), (planes[2], planes[3]),
                                                       (planes[4], planes[5])), rgrads[:3]):
        assert _rel_heads(torch.stack([re.grad, im.grad], -1), r) < 1e-4, name
    assert _rel_heads(gg.grad, rgrads[3]) < 1e-4, "dgamma"
    assert _rel_heads(bb.grad, rgrads[4]) < 1e-4, "dbeta"


def test_delta_step_tiny_gamma(gpu_lib):
    """recur_step_delta with gamma <= 1e-10 (and exactly 0): the step's write
    keeps weight 1 as in the reference step (v11/model.py:967-1002), so the
    state is the write alone; y, the state and the gradients of the step
    against the reference step under autograd."""
    from qllm2_amd.pam_delta import recur_step_delta
    B, H, d = 2, 2, 64
    q, k, v, g, b = D.make_delta_inputs(B, H, 1, d, 710)
    g = torch.tensor([[1e-10, 0.0], [3e-12, 1e-10]], dtype=torch.float64)
    s = torch.randn(B, H, d, d, 2, generator=torch.Generator().manual_seed(711), dtype=torch.float64) * 0.1
    qt = q[:, :, 0] * d ** -0.5
    leaves = [x.clone().requires_grad_(True) for x in (s, v[:, :, 0], k[:, :, 0], qt, b[:, :, 0])]
    yr, sr = D.recur_step_delta(leaves[0], g, leaves[1], leaves[2], leaves[3], leaves[4])
    gy = torch.randn(yr.shape, generator=torch.Generator().manual_seed(712), dtype=torch.float64)
    ((yr * gy).sum() + sr.sum()).backward()
    dev = torch.device("cuda")
    cl = [x.detach().float().to(dev).requires_grad_(True) for x in (s, v[:, :, 0], k[:, :, 0], qt, b[:, :, 0])]
    y, sc = recur_step_delta(cl[0], g.float().to(dev), cl[1], cl[2], cl[3], cl[4])
    assert torch.isfinite(y).all() and torch.isfinite(sc).all()
    assert _rel(y, yr) < 1e-4 and _rel(sc, sr) < 1e-4
    ((y * gy.float().to(dev)).sum() + sc.sum()).backward()
    for name, a, r in zip(("ds", "dv", "dk", "dq", "dbeta"), cl, leaves):
        assert torch.isfinite(a.grad).all(), name
        assert _rel(a.grad, r.grad) < 1e-4, f"{name}: {_rel(a.grad, r.grad):.2e}"


def test_delta_long_sequence_properties(gpu_lib):
    """T = 2048 (the config-3 length, 32 chunks), B=1, H=4: output
    and final state of the first head against the oracle's token recurrence."""
    from qllm2_amd.pam_delta import delta_planar
    B, H, T, d = 1, 4, 2048, 64
    q, k, v, g, b = D.make_delta_inputs(B, H, T, d, 660, dtype=torch.float32)
    dev = torch.device("cuda")
    planes = [x[..., i].contiguous().to(dev) for x in (q, k, v) for i in (0, 1)]
    with torch.no_grad():
        y_re, y_im, s_re, s_im = delta_planar(*planes, g.to(dev), b.to(dev), q_scale=d ** -0.5, gamma_eps=1e-6)
    yr, sr = D.delta_recurrent(q[:, :1].double(), k[:, :1].double(), v[:, :1].double(), g[:, :1].double(),
                               b[:, :1].double(), d)
    y = torch.stack([y_re, y_im], -1)[:, :1].cpu()
    assert _rel(y, yr) < 1e-4
    assert _rel(torch.stack([s_re, s_im], -1)[:, :1].cpu(), sr) < 1e-4


def _rel_heads(a, b):
    """max over (batch, head) of that head's max-abs error over its own max-abs
    reference value (floored at 1e-6 of the global one, for heads whose exact
    gradient is zero): a head whose values are small cannot hide behind another."""
    a, b = a.detach().double().cpu(), b.detach().double().cpu()
    err = (a - b).abs().flatten(2).amax(-1)
    ref = b.abs().flatten(2).amax(-1).clamp_min(1e-6 * b.abs().max().item() + 1e-300)
    return (err / ref).max().item()


def test_delta_multichunk_per_head(gpu_lib):
    """Five chunks (T = 300, ragged last chunk) with s0 and ds, every output and
    gradient normalised per (b, h) against the chunked oracle in float64."""
    B, H, T, d = 2, 3, 300, 64
    q, k, v, g, b = D.make_delta_inputs(B, H, T, d, 670)
    gen = torch.Generator().manual_seed(671)
    s0 = torch.randn(B, H, d, d, 2, generator=gen, dtype=torch.float64) * 0.05
    dy = torch.randn(B, H, T, d, 2, generator=gen, dtype=torch.float64)
    ds = torch.randn(B, H, d, d, 2, generator=gen, dtype=torch.float64) * 0.1
    y, s, grads = _run(q, k, v, g, b, s0, dy, ds, 1e-6)
    yr, sr, rgrads = _ref(q, k, v, g, b, s0, dy, ds, chunked=True)
    assert _rel_heads(y, yr) < 1e-4, f"y {_rel_heads(y, yr):.2e}"
    assert _rel_heads(s, sr) < 1e-4, f"s {_rel_heads(s, sr):.2e}"
    for name, a, r in zip(NAMES, grads, rgrads):
        assert _rel_heads(a, r) < 1e-4, f"{name}: {_rel_heads(a, r):.2e}"


def test_delta_decay_regimes(gpu_lib):
    """Per head a different regime: strong decay (gamma in (0.01, 0.3): the
    within-chunk alpha = e^L underflows in fp32), gamma = 1 exactly (no decay),
    beta = 0 (no write) and beta = 1 (full overwrite), over three chunks; outputs
    and gradients per (b, h) against the chunked oracle."""
    B, H, T, d = 1, 4, 160, 64
    q, k, v, g, b = D.make_delta_inputs(B, H, T, d, 680)
    gen = torch.Generator().manual_seed(681)
    g = g.clone()
    b = b.clone()
    g[:, 0] = 0.01 + 0.29 * torch.rand(B, T, generator=gen, dtype=torch.float64)
    g[:, 1] = 1.0
    b[:, 2] = 0.0
    b[:, 3] = 1.0
    dy = torch.randn(B, H, T, d, 2, generator=gen, dtype=torch.float64)
    y, s, grads = _run(q, k, v, g, b, None, dy, None, 1e-6)
    yr, sr, rgrads = _ref(q, k, v, g, b, None, dy, None, chunked=True)
    assert _rel_heads(y, yr) < 1e-4, f"y {_rel_heads(y, yr):.2e}"
    assert _rel_heads(s, sr) < 1e-4, f"s {_rel_heads(s, sr):.2e}"
    for name, a, r in zip(NAMES[:5], grads[:5], rgrads[:5]):
        assert _rel_heads(a, r) < 1e-4, f"{name}: {_rel_heads(a, r):.2e}"


def _delta_cases(n, seed):
    g = torch.Generator().manual_seed(seed)
    return [([16, 32, 48, 64][int(torch.randint(4, (1,), generator=g))], int(torch.randint(1, 300, (1,), generator=g)),
             bool(torch.randint(2, (1,), generator=g)), bool(torch.randint(2, (1,), generator=g))) for _ in range(n)]


@pytest.mark.parametrize("d,T,with_s0,with_ds", _delta_cases(8, 777))
def test_delta_seeded_random_shapes(gpu_lib, d, T, with_s0, with_ds):
    """Seeded random head dims (16-64), lengths (1-299: partial and multiple
    chunks), start states and state gradients: Y, S and every gradient against
    the chunked oracle."""
    B, H = 1, 2
    q, k, v, g, b = D.make_delta_inputs(B, H, T, d, 780 + d + T)
    gen = torch.Generator().manual_seed(781 + d + T)
    s0 = torch.randn(B, H, d, d, 2, generator=gen, dtype=torch.float64) * 0.05 if with_s0 else None
    dy = torch.randn(B, H, T, d, 2, generator=gen, dtype=torch.float64)
    ds = torch.randn(B, H, d, d, 2, generator=gen, dtype=torch.float64) * 0.1 if with_ds else None
    y, s, grads = _run(q, k, v, g, b, s0, dy, ds, 1e-6, d=d)
    yr, sr, rgrads = _ref(q, k, v, g, b, s0, dy, ds, chunked=True, d=d)
    assert _rel(y, yr) < 1e-4, f"y {_rel(y, yr):.2e}"
    assert _rel(s, sr) < 1e-4, f"s {_rel(s, sr):.2e}"
    for name, a, r in zip(NAMES, grads, rgrads):
        if a is None or r is None:
            continue
        assert _rel(a, r) < 1e-4, f"{name}: {_rel(a, r):.2e}"
