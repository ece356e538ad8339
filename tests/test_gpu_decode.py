"""GPU parity of the ragged decode kernel (qpam_decode_step) against the CPU
oracle (oracle/pam.py: recur_step_additive, decode_slots), fp32, rel <= 1e-4
(observed ~1e-6: only the summation order of S q differs)."""

import math

import pytest
import torch

from oracle import pam as O

pytestmark = pytest.mark.gpu

REL = 1e-4


def _rel(a, b):
    return ((a.double() - b.double()).abs().max() / (b.double().abs().max() + 1e-30)).item()


def _pool(S, G, M, d, seed):
    g = torch.Generator().manual_seed(seed)
    state = torch.randn(S, G, M, d, d, 2, generator=g) * 0.01
    q, k, v = (torch.randn(S, G, d, 2, generator=g) for _ in range(3))
    gamma = torch.sigmoid(torch.randn(S, G, M, generator=g) + 3)
    rot = torch.randn(S, G, M, 2, generator=g)
    return state, q, k, v, gamma, rot


@pytest.mark.parametrize("d", [16, 32, 64, 128])
@pytest.mark.parametrize("M,use_rot", [(1, False), (1, True), (2, True), (3, True), (4, False), (5, True)])
def test_decode_step_matches_oracle(gpu_lib, d, M, use_rot):
    S, G = 6, 5
    state, q, k, v, gamma, rot = _pool(S, G, M, d, 100 + d + M)
    active = torch.tensor([5, 1, 3], dtype=torch.int32)
    scale = d ** -0.5
    y_ref, s_ref = O.decode_slots(state.double(), active.long(), q.double(), k.double(), v.double(),
                                  gamma.double(), scale, rot.double() if use_rot else None)
    from qllm2_amd.decode import decode_step
    st = state.cuda()
    y = decode_step(st, q.cuda(), k.cuda(), v.cuda(), gamma.cuda(), active=active.cuda(),
                    rot=rot.cuda() if use_rot else None, q_scale=scale)
    torch.cuda.synchronize()
    st, y = st.cpu(), y.cpu()
    for sl in (0, 2, 4):  # unlisted slots: bit-identical, y untouched (zero)
        assert torch.equal(st[sl], state[sl]) and torch.all(y[sl] == 0)
    for sl in (1, 3, 5):
        assert _rel(st[sl], s_ref[sl]) < REL
        assert _rel(y[sl], y_ref[sl]) < REL


def test_decode_all_slots_and_empty_list(gpu_lib):
    from qllm2_amd.decode import decode_step
    state, q, k, v, gamma, _ = _pool(4, 3, 1, 64, 7)
    st = state.cuda()
    y = decode_step(st, q.cuda(), k.cuda(), v.cuda(), gamma.cuda(), q_scale=0.125)
    y_ref, s_ref = O.decode_slots(state.double(), torch.arange(4), q.double(), k.double(), v.double(),
                                  gamma.double(), 0.125)
    assert _rel(st.cpu(), s_ref) < REL and _rel(y.cpu(), y_ref) < REL
    st2 = st.clone()
    decode_step(st2, q.cuda(), k.cuda(), v.cuda(), gamma.cuda(), active=torch.empty(0, dtype=torch.int32).cuda())
    assert torch.equal(st2, st)
    # out-of-range ids are skipped, not faulted on
    bad = torch.tensor([-1, 4, 1000], dtype=torch.int32).cuda()
    decode_step(st2, q.cuda(), k.cuda(), v.cuda(), gamma.cuda(), active=bad)
    torch.cuda.synchronize()
    assert torch.equal(st2, st)


def test_recur_step_additive_dropin(gpu_lib):
    from qllm2_amd.decode import recur_step_additive
    g = torch.Generator().manual_seed(3)
    B, H, d = 2, 3, 16
    s = torch.randn(B, H, d, d, 2, generator=g)
    v, k, q = (torch.randn(B, H, d, 2, generator=g) for _ in range(3))
    gam = torch.rand(B, H, generator=g)
    y_ref, s_ref = O.recur_step_additive(s.double(), gam.double(), v.double(), k.double(), q.double())
    sc = s.cuda()
    y, s2 = recur_step_additive(sc, gam.cuda(), v.cuda(), k.cuda(), q.cuda())
    assert torch.equal(sc.cpu(), s)  # functional: input untouched
    assert _rel(y.cpu(), y_ref) < REL and _rel(s2.cpu(), s_ref) < REL


def test_decode_config4_full_pool_properties(gpu_lib):
    """Config 4 at full size: 256 slots x 16 layers x 12 heads, d=64, ~75% active,
    two consecutive steps with fresh q, k, v.  After each step every inactive
    slot is bit-identical to its state before the step, and every active slot's
    state and output match the oracle's step (oracle/pam.py recur_step_additive,
    float64 on the CPU) applied to that slot's previous GPU state, with the
    worst slot's relative error reported."""
    from qllm2_amd.decode import decode_step
    S, G, d = 256, 16 * 12, 64
    gen = torch.Generator().manual_seed(1004)
    dev = torch.device("cuda")
    state = (torch.randn(S, G, 1, d, d, 2, generator=gen) * 0.01).to(dev)
    gamma = torch.sigmoid(torch.randn(S, G, 1, generator=gen) + 3).to(dev)
    mask = torch.rand(S, generator=gen) < 0.75
    active = torch.nonzero(mask).flatten().to(torch.int32)
    inactive = torch.nonzero(~mask).flatten().to(dev)
    for step in range(2):
        q, k, v = ((torch.randn(S, G, d, 2, generator=gen)).to(dev) for _ in range(3))
        before = state.clone()
        y = decode_step(state, q, k, v, gamma, active=active.to(dev), q_scale=d ** -0.5)
        torch.cuda.synchronize()
        assert torch.equal(state[inactive], before[inactive]), f"step {step}: an inactive slot changed"
        assert math.isfinite(y.abs().sum().item())
        worst_s = worst_y = 0.0
        for group in active.split(32):
            g = group.long()
            b0, gm = before[g.to(dev), :, 0].double().cpu(), gamma[g.to(dev), :, 0].double().cpu()
            ys, ss = O.recur_step_additive(b0, gm, v[g.to(dev)].double().cpu(), k[g.to(dev)].double().cpu(),
                                           (q[g.to(dev)] * d ** -0.5).double().cpu())
            got_s, got_y = state[g.to(dev), :, 0].double().cpu(), y[g.to(dev)].double().cpu()
            for i in range(len(g)):
                worst_s = max(worst_s, _rel(got_s[i], ss[i]))
                worst_y = max(worst_y, _rel(got_y[i], ys[i]))
        assert worst_s < REL and worst_y < REL, f"step {step}: worst slot state {worst_s:.2e}, output {worst_y:.2e}"
        del before


@pytest.mark.parametrize("d", [16, 64, 128])
@pytest.mark.parametrize("M,use_rot", [(1, False), (3, True)])
def test_decode_rope_per_slot(gpu_lib, d, M, use_rot):
    """Per-slot rotary positions inside the decode kernel against the oracle's
    cmul(q, rope[pos]), cmul(k, rope[pos]) (one offset per slot)."""
    from qllm2_amd.decode import decode_step
    S, G = 7, 4
    state, q, k, v, gamma, rot = _pool(S, G, M, d, 300 + d + M)
    rope = O.rope_table(1000, d)
    pos = torch.tensor([0, 999, 5, 123, 77, 1, 640], dtype=torch.int32)
    active = torch.tensor([6, 0, 1, 3, 4], dtype=torch.int32)
    scale = d ** -0.5
    y_ref, s_ref = O.decode_slots(state.double(), active.long(), q.double(), k.double(), v.double(),
                                  gamma.double(), scale, rot.double() if use_rot else None, rope=rope, pos=pos)
    st = state.cuda()
    y = decode_step(st, q.cuda(), k.cuda(), v.cuda(), gamma.cuda(), active=active.cuda(),
                    rot=rot.cuda() if use_rot else None, q_scale=scale, rope=rope.float().cuda(), pos=pos.cuda())
    torch.cuda.synchronize()
    st, y = st.cpu(), y.cpu()
    for sl in (2, 5):
        assert torch.equal(st[sl], state[sl]) and torch.all(y[sl] == 0)
    for sl in (0, 1, 3, 4, 6):
        assert _rel(st[sl], s_ref[sl]) < REL
        assert _rel(y[sl], y_ref[sl]) < REL


def test_slot_pool_e3_continuous_batching(gpu_lib):
    """SlotPool over 2 layers x 3 heads x 3 states, d=64: sequences join with a
    prefill state at their own position, leave, and their slots are reused, over
    12 steps.  Every live sequence's outputs and states are checked each step
    against its own oracle decode (per-sequence state, per-sequence position)."""
    from qllm2_amd.decode import SlotPool
    L, H, M, d, S = 2, 3, 3, 64, 5
    pool = SlotPool(S, L, H, d, n_states=M, max_len=256)
    g = torch.Generator().manual_seed(77)
    scale = d ** -0.5
    rope = O.rope_table(256, d)
    seqs = {}  # seq id -> dict(slot, pos, states [L] of [H, M, d, d, 2] float64)
    schedule = {0: [("join", 0, 10), ("join", 1, 0), ("join", 2, 50)], 3: [("leave", 1), ("join", 3, 7)],
                5: [("join", 4, 200), ("join", 5, 3)], 7: [("leave", 0), ("leave", 4)], 8: [("join", 6, 1)]}
    for step in range(12):
        for ev in schedule.get(step, []):
            if ev[0] == "join":
                _, sid, p0 = ev
                pre = [torch.randn(M, H, d, d, 2, generator=g) * 0.02 for _ in range(L)]
                slot = pool.acquire(position=p0, states=pre)
                seqs[sid] = dict(slot=slot, pos=p0, st=[x.permute(1, 0, 2, 3, 4).double() for x in pre])
            else:
                pool.release(seqs.pop(ev[1])["slot"])
        active = torch.tensor(sorted(s["slot"] for s in seqs.values()), dtype=torch.int32)
        for layer in range(L):
            q, k, v = (torch.randn(S, H, d, 2, generator=g) for _ in range(3))
            gamma = torch.sigmoid(torch.randn(S, H, M, generator=g) + 2)
            rot = torch.randn(S, H, M, 2, generator=g)
            y = pool.step(layer, q.cuda(), k.cuda(), v.cuda(), gamma.cuda(), active.cuda(), rot=rot.cuda())
            y = y.cpu()
            for sid, s in seqs.items():
                sl = s["slot"]
                yr, sr = O.decode_slots(s["st"][layer][None], torch.tensor([0]), q[sl:sl + 1].double(),
                                        k[sl:sl + 1].double(), v[sl:sl + 1].double(), gamma[sl:sl + 1].double(),
                                        scale, rot[sl:sl + 1].double(), rope=rope, pos=torch.tensor([s["pos"]]))
                s["st"][layer] = sr[0]
                assert _rel(y[sl], yr[0]) < REL, (step, layer, sid)
                assert _rel(pool.state[sl, layer].cpu(), sr[0]) < REL, (step, layer, sid)
        pool.advance(active.cuda())
        for s in seqs.values():
            s["pos"] += 1
        assert pool.pos.cpu()[active.long()].tolist() == [
            s["pos"] for s in sorted(seqs.values(), key=lambda s: s["slot"])]


@pytest.mark.parametrize("d,M,use_rot", [(64, 1, False), (64, 3, True), (32, 5, True), (128, 1, True),
                                         (16, 2, False)])
def test_decode_planar_inputs_equal_interleaved(gpu_lib, d, M, use_rot):
    """q, k, v (and the rotations) handed over as planar (re, im) planes (the
    engine passes the prologue's planes) give the interleaved call's y and state
    bit for bit: the
    kernels read the same values, only through 8-byte instead of 16-byte loads;
    compact rows with per-slot RoPE, every kernel variant (one state, several,
    the general state loop)."""
    from qllm2_amd.decode import build_rope_cache, decode_step
    S, G = 7, 3
    state, q, k, v, gamma, rot = _pool(S, G, M, d, 900 + d + M)
    active = torch.tensor([6, 0, 2, 4], dtype=torch.int32).cuda()
    n = active.numel()
    qc, kc, vc = (x[:n].cuda() for x in (q, k, v))
    gc, rc = gamma[:n].cuda(), rot[:n].cuda() if use_rot else None
    rope = build_rope_cache(32, d, device="cuda")
    pos = torch.tensor([3, 30, 1, 0, 9, 2, 17], dtype=torch.int32).cuda()
    runs = []
    for planar in (False, True):
        st = state.cuda()
        qkv = [(x[..., 0].contiguous(), x[..., 1].contiguous()) for x in (qc, kc, vc)] if planar else [qc, kc, vc]
        r = (rc[..., 0].contiguous(), rc[..., 1].contiguous()) if planar and rc is not None else rc
        y = decode_step(st, *qkv, gc, active=active, rot=r, q_scale=d ** -0.5, rope=rope, pos=pos, compact=True)
        torch.cuda.synchronize()
        runs.append((y.cpu(), st.cpu()))
    assert torch.equal(runs[0][0], runs[1][0]) and torch.equal(runs[0][1], runs[1][1])


def test_decode_planar_inputs_rejected_when_mixed(gpu_lib):
    from qllm2_amd.decode import decode_step
    state, q, k, v, gamma, _ = _pool(2, 1, 1, 16, 5)
    st, q, k, v, gamma = (x.cuda() for x in (state, q, k, v, gamma))
    with pytest.raises(ValueError, match="plane pairs"):
        decode_step(st, (q[..., 0], q[..., 1]), k, v, gamma)


@pytest.mark.parametrize("d", [16, 32, 64, 128])
@pytest.mark.parametrize("M,use_rot", [(1, False), (2, True), (3, True), (5, True)])
def test_decode_per_channel_decay_matches_textbook_recurrence(gpu_lib, d, M, use_rot):
    """E1 per-channel decay (gamma [R, G, M, d], one per key column) through
    every decode kernel: T steps from a zero state on two of four slots equal
    the oracle's textbook per-channel recurrence (brute_force_perchannel,
    complex128) per state, rotated and summed; the other slots stay zero."""
    from qllm2_amd.decode import decode_step
    S, G, T = 4, 3, 6
    g = torch.Generator().manual_seed(300 + d + M)
    q, k, v = (torch.randn(T, S, G, d, 2, generator=g, dtype=torch.float64) for _ in range(3))
    gamma = torch.sigmoid(torch.randn(T, S, G, M, d, generator=g, dtype=torch.float64) + 1.0)
    rot = torch.randn(T, S, G, M, 2, generator=g, dtype=torch.float64)
    active = torch.tensor([3, 1], dtype=torch.int32)
    scale = d ** -0.5
    st = torch.zeros(S, G, M, d, d, 2, device="cuda")
    ys = []
    for t in range(T):
        ys.append(decode_step(st, q[t].float().cuda(), k[t].float().cuda(), v[t].float().cuda(),
                              gamma[t].float().cuda(), active=active.cuda(), q_scale=scale,
                              rot=rot[t].float().cuda() if use_rot else None).cpu())
    torch.cuda.synchronize()
    for s in active.tolist():
        y_ref = 0
        for m in range(M):
            y_m, s_m = O.brute_force_perchannel(O.to_complex(q[:, s]).transpose(1, 0, 2),
                                                O.to_complex(k[:, s]).transpose(1, 0, 2),
                                                O.to_complex(v[:, s]).transpose(1, 0, 2),
                                                gamma[:, s, :, m].numpy().transpose(1, 0, 2), scale)
            r = O.to_complex(rot[:, s, :, m]).T[:, :, None] if use_rot else 1.0   # [G, T, 1]
            y_ref = y_ref + r * y_m
            got_s = st[s, :, m].cpu()
            assert _rel(got_s, O.from_complex(s_m)) < REL
        got_y = torch.stack([y[s] for y in ys], 1)                    # [G, T, d, 2]
        assert _rel(got_y, O.from_complex(y_ref)) < REL
    for s in (0, 2):
        assert st[s].abs().max().item() == 0.0


@pytest.mark.parametrize("d", [16, 32, 64, 128, 24, 48, 96])
@pytest.mark.parametrize("per_channel", [False, True])
@pytest.mark.parametrize("with_dstate", [False, True])
def test_decode_step_backward_matches_autograd(gpu_lib, d, per_channel, with_dstate):
    """qpam_decode_step_bwd through recur_step_additive's autograd: the
    gradients of the state, gamma, v, k and q for a loss on y (and on the new
    state) equal float64 autograd of the oracle step (the reference's
    _recur_step_additive restated) over [2, 3] (slot, head) rows.  Head dims
    24, 48 and 96 run zero-padded on the 32-, 64- and 128-wide kernels."""
    from qllm2_amd.decode import recur_step_additive
    g = torch.Generator().manual_seed(500 + d + 7 * per_channel + with_dstate)
    state = torch.randn(2, 3, d, d, 2, generator=g, dtype=torch.float64) * 0.1
    gam = torch.sigmoid(torch.randn(*((2, 3, d) if per_channel else (2, 3)), generator=g, dtype=torch.float64) + 2)
    v, k, q = (torch.randn(2, 3, d, 2, generator=g, dtype=torch.float64) for _ in range(3))
    q = q * d ** -0.5
    dy = torch.randn(2, 3, d, 2, generator=g, dtype=torch.float64)
    ds = torch.randn(2, 3, d, d, 2, generator=g, dtype=torch.float64) * 0.1 if with_dstate else None
    leaves_r = [t.clone().requires_grad_(True) for t in (state, gam, v, k, q)]
    y_r, s_r = O.recur_step_additive(*leaves_r)
    loss = (y_r * dy).sum() + ((s_r * ds).sum() if ds is not None else 0)
    loss.backward()
    leaves = [t.float().cuda().requires_grad_(True) for t in (state, gam, v, k, q)]
    y, s = recur_step_additive(*leaves)
    loss = (y * dy.float().cuda()).sum() + ((s * ds.float().cuda()).sum() if ds is not None else 0)
    loss.backward()
    torch.cuda.synchronize()
    assert _rel(y.detach().cpu(), y_r.detach()) < REL
    assert _rel(s.detach().cpu(), s_r.detach()) < REL
    for name, a, b in zip(("state", "gamma", "v", "k", "q"), leaves, leaves_r):
        assert _rel(a.grad.cpu(), b.grad) < REL, f"d{name} {_rel(a.grad.cpu(), b.grad):.2e}"


@pytest.mark.parametrize("d", [16, 64, 128])
@pytest.mark.parametrize("M,use_rot", [(1, False), (3, True), (5, True)])
def test_decode_bf16_output_equals_rounded_fp32(gpu_lib, d, M, use_rot):
    """y written in bf16 by the kernel (y_dtype) equals the fp32 y of the same
    step rounded to bf16, bit for bit, and the states agree exactly (single,
    multi-state and general kernels)."""
    from qllm2_amd.decode import decode_step
    S, G = 5, 4
    state, q, k, v, gamma, rot = _pool(S, G, M, d, 700 + d + M)
    active = torch.tensor([4, 0, 2], dtype=torch.int32).cuda()
    outs = []
    for dt in (torch.float32, torch.bfloat16):
        st = state.clone().cuda()
        y = torch.empty(3, G, d, 2, device="cuda", dtype=dt)
        decode_step(st, q[[4, 0, 2]].cuda(), k[[4, 0, 2]].cuda(), v[[4, 0, 2]].cuda(), gamma[[4, 0, 2]].cuda(),
                    active=active, rot=rot[[4, 0, 2]].cuda() if use_rot else None, q_scale=d ** -0.5, out=y,
                    compact=True)
        outs.append((y, st))
    torch.cuda.synchronize()
    assert torch.equal(outs[1][0], outs[0][0].to(torch.bfloat16))
    assert torch.equal(outs[1][1], outs[0][1])


@pytest.mark.parametrize("M,qk_norm,floor,gsp,dtype", [(3, False, 0.0, True, torch.bfloat16), (3, True, 0.25, True, torch.float32),
                                                       (1, False, 0.0, False, torch.bfloat16), (4, True, 0.0, False, torch.float32)])
def test_decode_step_proj_matches_prologue_then_decode(M, qk_norm, floor, gsp, dtype):
    """The decode prologue fused into the kernel (decode_step_proj) against the
    separate inference prologue (prologue_decode) followed by decode_step on the
    same projection rows, gate logits, states and positions."""
    from qllm2_amd.decode import build_rope_cache, decode_step, decode_step_proj
    from qllm2_amd.pam_prologue import prologue_decode, proj_columns
    dev = "cuda"
    S, H, d, n = 11, 5, 64, 7
    g = torch.Generator(device=dev).manual_seed(M * 10 + int(qk_norm))
    C = proj_columns(H)
    proj = (torch.randn(n, C, device=dev, generator=g) * 0.5).to(dtype)
    W = (H if gsp else 0) + (H * M if M > 1 else 0)
    gate = (torch.randn(n, max(W, 1), device=dev, generator=g) * 1.5).to(dtype)
    dt_bias = torch.randn(H, device=dev, generator=g) - 1.0
    off = torch.linspace(-0.5, 0.5, M, device=dev) if M > 1 else None
    state0 = torch.randn(S, H, M, d, d, 2, device=dev, generator=g) * 0.1
    active = torch.tensor([9, 0, 4, 10, 2, 7, 5], device=dev, dtype=torch.int32)
    rope = build_rope_cache(64, d, device=dev)
    pos = torch.randint(0, 60, (S,), device=dev, generator=g, dtype=torch.int32)
    pcol = 0 if gsp else -1
    fcol = (H if gsp else 0) if M > 1 else -1
    st_a = state0.clone()
    y_a = decode_step_proj(st_a, proj, dt_bias, gate=gate if W else None, protect_col=pcol, phase_col=fcol,
                           state_offset=off, qk_norm=qk_norm, gamma_floor=floor, active=active, q_scale=d ** -0.5,
                           rope=rope, pos=pos, compact=True)
    prot = gate[:, :H].view(n, 1, H) if gsp else None
    ph = gate[:, fcol:fcol + H * M].view(n, 1, H, M) if M > 1 else None
    (qr, qi), (kr, ki), (vr, vi), gamma, rot = prologue_decode(proj.view(n, 1, C), dt_bias, n_heads=H, n_states=M,
                                                                state_offset=off, protect=prot, phase=ph,
                                                                qk_norm=qk_norm, gamma_floor=floor)
    q, k, v = ((re[:, :, 0], im[:, :, 0]) for re, im in ((qr, qi), (kr, ki), (vr, vi)))
    gm = gamma[..., 0].permute(1, 2, 0)
    r = tuple(x[..., 0].permute(1, 2, 0) for x in rot) if rot is not None else None
    st_b = state0.clone()
    y_b = decode_step(st_b, q, k, v, gm, active=active, rot=r, q_scale=d ** -0.5, rope=rope, pos=pos, compact=True)
    scale = lambda t: t.abs().max().clamp_min(1e-6)
    assert ((y_a - y_b).abs().max() / scale(y_b)).item() < 1e-5
    assert ((st_a - st_b).abs().max() / scale(st_b)).item() < 1e-5
    untouched = [s for s in range(S) if s not in active.tolist()]
    assert torch.equal(st_a[untouched], state0[untouched])


def test_decode_step_proj_checks_arguments(gpu_lib):
    """The fused-prologue decode wrapper refuses gate columns outside the gate
    matrix, decay-bias / state-offset vectors of the wrong length and a RoPE
    table of another head dim, before any launch."""
    from qllm2_amd.decode import decode_step_proj
    S, G, M, d = 2, 2, 2, 64
    state = torch.zeros(S, G, M, d, d, 2, device="cuda")
    proj = torch.zeros(S, 6 * G * d + G, device="cuda")
    gate = torch.zeros(S, G + G * M, device="cuda")
    dt_bias, off = torch.zeros(G, device="cuda"), torch.zeros(M, device="cuda")
    ok = dict(gate=gate, protect_col=0, phase_col=G, state_offset=off)
    with pytest.raises(ValueError, match="protect columns"):
        decode_step_proj(state, proj, dt_bias, **{**ok, "protect_col": G + G * M - 1})
    with pytest.raises(ValueError, match="phase columns"):
        decode_step_proj(state, proj, dt_bias, **{**ok, "phase_col": G + 1})
    with pytest.raises(ValueError, match="phase columns"):
        decode_step_proj(state, proj, dt_bias, phase_col=0)  # no gate matrix at all
    with pytest.raises(ValueError, match="dt_bias"):
        decode_step_proj(state, proj, torch.zeros(G + 1, device="cuda"), **ok)
    with pytest.raises(ValueError, match="state_offset"):
        decode_step_proj(state, proj, dt_bias, **{**ok, "state_offset": torch.zeros(M + 1, device="cuda")})
    with pytest.raises(ValueError, match="rope"):
        decode_step_proj(state, proj, dt_bias, **ok, rope=torch.zeros(8, 32, 2, device="cuda"),
                         pos=torch.zeros(S, dtype=torch.int32, device="cuda"))
    y = decode_step_proj(state, proj, dt_bias, **ok)  # the valid call runs
    torch.cuda.synchronize()
    assert y.shape == (S, G, d, 2)
