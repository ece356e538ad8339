"""GPU parity of the fused tied LM-head cross-entropy (qpam_ce_fwd/bwd) against
the CPU oracle (oracle/ce.py, the reference's chunk loop) in float64.

Tolerances: fp32 operands rel <= 1e-4 on loss, dH, dW; bf16 operands
(fp32 accumulation) rel <= 2e-2, oracle fed the bf16-rounded values.
"""

import pytest
import torch

from oracle import ce as O

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = torch.as_tensor(a).double(), torch.as_tensor(b).double()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def _data(n, d, v, seed, dtype, e_std=1.0):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, d, generator=g).to(dtype)
    w = (torch.randn(v, d, generator=g) * e_std).to(dtype)
    t = torch.randint(0, v, (n,), generator=g)
    return h, w, t


def _gpu(h, w, t, mask=None, chunk=4096, ignore_index=-100, grad_output=1.0):
    from qllm2_amd.fused_ce import fused_linear_cross_entropy
    hc = h.cuda().requires_grad_(True)
    wc = w.cuda().requires_grad_(True)
    loss = fused_linear_cross_entropy(hc, wc, t.cuda(), mask=mask.cuda() if mask is not None else None,
                                      chunk=chunk, ignore_index=ignore_index)
    (loss * grad_output).backward()
    torch.cuda.synchronize()
    return loss.detach().cpu(), hc.grad.cpu(), wc.grad.cpu()


@pytest.mark.parametrize("n,chunk", [(200, 32), (300, 4096), (129, 128)])
def test_ce_fp32_ignore_index(gpu_lib, n, chunk):
    h, w, t = _data(n, 64, 512, 10 + n, torch.float32)
    t[::7] = -100
    loss, dh, dw = _gpu(h, w, t, chunk=chunk)
    ref, denom = O.ce_forward(h.double(), w.double(), t, chunk=chunk)
    rdh, rdw = O.ce_backward(h.double(), w.double(), t, denom, chunk=chunk)
    assert _rel(loss, ref) < 1e-5
    assert _rel(dh, rdh) < 1e-4 and _rel(dw, rdw) < 1e-4


def test_ce_fp32_mask_and_grad_output(gpu_lib):
    h, w, t = _data(200, 96, 700, 3, torch.float32)
    mask = (torch.rand(200, generator=torch.Generator().manual_seed(4)) > 0.3).float()
    loss, dh, dw = _gpu(h, w, t, mask=mask, chunk=64, ignore_index=-1, grad_output=2.5)
    ref, denom = O.ce_forward(h.double(), w.double(), t, mask=mask.double(), chunk=64, ignore_index=-1)
    rdh, rdw = O.ce_backward(h.double(), w.double(), t, denom, grad_output=2.5, mask=mask.double(), chunk=64,
                             ignore_index=-1)
    assert _rel(loss, ref) < 1e-5
    assert _rel(dh, rdh) < 1e-4 and _rel(dw, rdw) < 1e-4


def test_ce_all_rows_ignored(gpu_lib):
    h, w, t = _data(40, 32, 100, 5, torch.float32)
    t[:] = -100
    loss, dh, dw = _gpu(h, w, t)
    assert loss.item() == 0.0 and torch.all(dh == 0) and torch.all(dw == 0)


# bf16 backward GEMMs: hipBLASLt (default) or the hand-written kernels (QPAM_CE_GEMM=hip)
GEMM_PATHS = ["library", "hip"]


def _select_gemm(monkeypatch, path):
    if path == "hip":
        monkeypatch.setenv("QPAM_CE_GEMM", "hip")
    else:
        monkeypatch.delenv("QPAM_CE_GEMM", raising=False)


@pytest.mark.parametrize("path", GEMM_PATHS)
@pytest.mark.parametrize("chunk", [384, 64])
def test_ce_bf16(gpu_lib, monkeypatch, path, chunk):
    """bf16 operands; chunk 64 makes the backward take several passes (256 rows
    each on the library GEMMs, 128 on the hand-written ones)."""
    _select_gemm(monkeypatch, path)
    h, w, t = _data(1000, 128, 3000, 6, torch.bfloat16, e_std=0.1)
    t[::10] = -100
    loss, dh, dw = _gpu(h, w, t, chunk=chunk)
    ref, denom = O.ce_forward(h.double(), w.double(), t, chunk=384)
    rdh, rdw = O.ce_backward(h.double(), w.double(), t, denom, chunk=384)
    assert dh.dtype == torch.bfloat16 and dw.dtype == torch.bfloat16
    assert _rel(loss, ref) < 2e-2
    assert _rel(dh, rdh) < 2e-2 and _rel(dw, rdw) < 2e-2


@pytest.mark.parametrize("path", GEMM_PATHS)
def test_ce_fp32_master_weight(gpu_lib, monkeypatch, path):
    """bf16 hidden rows with an fp32 master embedding (config 5's E): the GEMMs run
    on a bf16 copy of E, the loss and dH match the oracle on the bf16-rounded
    values, and dE comes back in fp32 (the gradient of the bf16 copy), over
    several backward passes."""
    _select_gemm(monkeypatch, path)
    h, w, t = _data(1000, 128, 3000, 16, torch.bfloat16, e_std=0.1)
    w = w.float() + torch.randn(w.shape, generator=torch.Generator().manual_seed(17)) * 1e-3  # not bf16-exact
    t[::10] = -100
    loss, dh, dw = _gpu(h, w, t, chunk=64)
    wb = w.to(torch.bfloat16).double()
    ref, denom = O.ce_forward(h.double(), wb, t, chunk=384)
    rdh, rdw = O.ce_backward(h.double(), wb, t, denom, chunk=384)
    assert dh.dtype == torch.bfloat16 and dw.dtype == torch.float32
    assert _rel(loss, ref) < 2e-2
    assert _rel(dh, rdh) < 2e-2 and _rel(dw, rdw) < 2e-2


@pytest.mark.parametrize("d", [128, 96])
def test_ce_bf16_tile_paths(gpu_lib, monkeypatch, d):
    """bf16 hidden sizes that take the 256 x 256 logits tiles (d % 64 == 0) and the
    256 x 128 tiles (d = 96): loss, gradients through the hand-written backward
    GEMMs, per-token losses and the argmax-based accuracy counts."""
    from qllm2_amd.fused_ce import linear_ce_per_token, linear_ce_stats
    _select_gemm(monkeypatch, "hip")
    h, w, t = _data(300, d, 700, 11 + d, torch.bfloat16, e_std=0.1)
    t[::9] = -100
    loss, dh, dw = _gpu(h, w, t, chunk=256)
    ref, denom = O.ce_forward(h.double(), w.double(), t, chunk=256)
    rdh, rdw = O.ce_backward(h.double(), w.double(), t, denom, chunk=256)
    assert _rel(loss, ref) < 2e-2
    assert _rel(dh, rdh) < 2e-2 and _rel(dw, rdw) < 2e-2
    per = linear_ce_per_token(h.cuda(), w.cuda(), t.cuda()).float().cpu()
    assert _rel(per, O.ce_per_token(h.double(), w.double(), t)) < 2e-2
    t2 = (h.float() @ w.float().T).argmax(-1)
    _, corr, tok = linear_ce_stats(h.cuda(), w.cuda(), t2.cuda())
    assert tok == 300 and corr >= 297  # bf16 logits may reorder near-ties


def test_ce_per_token_and_stats(gpu_lib):
    from qllm2_amd.fused_ce import linear_ce_per_token, linear_ce_stats
    h, w, t = _data(150, 64, 400, 7, torch.float32)
    t[::5] = -100
    per = linear_ce_per_token(h.cuda(), w.cuda(), t.cuda()).cpu()
    assert _rel(per, O.ce_per_token(h, w, t)) < 1e-5
    ls, corr, tok = linear_ce_stats(h.cuda(), w.cuda(), t.cuda())
    rls, rcorr, rtok = O.ce_stats(h, w, t)
    assert abs(ls - rls) <= 1e-4 * abs(rls) and corr == rcorr and tok == rtok
    # a row whose target is the argmax counts as correct
    t2 = (h @ w.T).argmax(-1)
    _, corr2, tok2 = linear_ce_stats(h.cuda(), w.cuda(), t2.cuda())
    assert corr2 == tok2 == 150


_CFG5 = {}


def _config5_reference():
    """Config 5 inputs and the fp32 CPU row log-sum-exps on the bf16 values,
    computed once for the module's full-size tests."""
    if not _CFG5:
        N, d_model, V = 16384, 512, 50261
        h, w, t = O.make_ce_inputs(N, d_model, V, 1005, dtype=torch.bfloat16)
        hf, wf = h.float(), w.float()
        lse = torch.empty(N)
        for c0 in range(0, N, 2048):
            lse[c0:c0 + 2048] = torch.logsumexp(hf[c0:c0 + 2048] @ wf.T, dim=-1)
        _CFG5.update(h=h, w=w, t=t, lse=lse)
    return _CFG5


def _check_config5(loss, dh, dw, n_rows, n_cols, seed):
    """Loss on all rows; dH on n_rows sampled rows and dW on n_cols sampled
    vocabulary rows, against fp32 CPU math on the bf16 values."""
    c = _config5_reference()
    h, w, t, lse = c["h"], c["w"], c["t"], c["lse"]
    hf, wf = h.float(), w.float()
    N, V = hf.shape[0], wf.shape[0]
    valid = t != -100
    tl = (hf[valid] * wf[t[valid]]).sum(-1)
    denom = valid.sum()
    ref_loss = (lse[valid] - tl).sum() / denom
    assert _rel(loss, ref_loss) < 2e-2
    g = torch.Generator().manual_seed(seed)
    rows = torch.randperm(N, generator=g)[:n_rows]
    p = torch.softmax(hf[rows] @ wf.T, -1)
    tv = t[rows]
    ok = tv != -100
    p[ok, tv[ok]] -= 1
    p[~ok] = 0
    p /= denom
    assert _rel(dh[rows], p @ wf) < 2e-2
    cols = torch.randperm(V, generator=g)[:n_cols]
    gcols = torch.exp(hf @ wf[cols].T - lse[:, None])
    onehot = (t[:, None] == cols[None, :]).float()
    gcols = (gcols - onehot) * valid[:, None].float() / denom
    assert _rel(dw[cols], gcols.T @ hf) < 2e-2


@pytest.mark.parametrize("path", GEMM_PATHS)
def test_ce_config5_full_size(gpu_lib, monkeypatch, path):
    """Config 5: N=16384, d_model=512 (D=1024 real-concat), V=50261, bf16 h ~N(0,1),
    E ~N(0, 0.02^2), 10% ignore.  Loss checked on all rows, dH on 256 sampled
    rows, dW on 1024 sampled vocab rows, against fp32 CPU math on the bf16 values."""
    _select_gemm(monkeypatch, path)
    c = _config5_reference()
    loss, dh, dw = _gpu(c["h"], c["w"], c["t"])
    _check_config5(loss, dh, dw, 256, 1024, 9)


def test_ce_config5_full_size_fp32_master(gpu_lib, monkeypatch):
    """Config 5 with its stated E: an fp32 master embedding (every entry off the
    bf16 grid by a quarter of a bf16 ulp, so its bf16 operand copy is the bf16 E
    of the reference values), bf16 h: the loss, dH (bf16) and dE (fp32, the
    gradient of the bf16 copy) at full size on the default backward path, dH on
    512 sampled rows and dE on 2048 sampled vocabulary rows."""
    _select_gemm(monkeypatch, GEMM_PATHS[0])
    c = _config5_reference()
    wb = c["w"].float()
    ulp = torch.where(wb != 0, torch.exp2(torch.floor(torch.log2(wb.abs().clamp_min(1e-30))) - 7), torch.zeros_like(wb))
    sign = torch.randint(0, 2, wb.shape, generator=torch.Generator().manual_seed(33)).float() * 2 - 1
    master = wb + 0.25 * ulp * sign
    assert torch.equal(master.to(torch.bfloat16), c["w"]) and not torch.equal(master, wb)
    loss, dh, dw = _gpu(c["h"], master, c["t"])
    assert dh.dtype == torch.bfloat16 and dw.dtype == torch.float32
    _check_config5(loss, dh, dw, 512, 2048, 19)


def _config5_full_gradients_fp32(h, w, t):
    """Every row of dH and every vocabulary row of dW of config 5 by torch
    float32 GEMMs on the GPU over 2048-row slices (the fp32 reference of the
    same op on the bf16 values; 2D products only)."""
    hf, wf, tc = h.float().cuda(), w.float().cuda(), t.cuda()
    valid = tc != -100
    denom = valid.sum().float()
    dh = torch.empty_like(hf)
    dw = torch.zeros_like(wf)
    for c0 in range(0, hf.shape[0], 2048):
        hs, ts, vs = hf[c0:c0 + 2048], tc[c0:c0 + 2048], valid[c0:c0 + 2048]
        p = torch.softmax(hs @ wf.T, -1)
        idx = torch.nonzero(vs).flatten()
        p[idx, ts[idx]] -= 1
        p[~vs] = 0
        p /= denom
        dh[c0:c0 + 2048] = p @ wf
        dw += p.T.contiguous() @ hs
    torch.cuda.synchronize()
    return dh.cpu(), dw.cpu()


def test_ce_config5_every_gradient_row(gpu_lib, monkeypatch):
    """Config 5 at full size on the default backward path: every row of dH and
    every vocabulary row of dE against torch float32 GEMMs on the same bf16
    values (rel <= 2e-2 of each tensor's largest entry, and per dE row of that
    row's largest reference entry over the rows whose reference is not tiny)."""
    _select_gemm(monkeypatch, GEMM_PATHS[0])
    c = _config5_reference()
    loss, dh, dw = _gpu(c["h"], c["w"], c["t"])
    ref_dh, ref_dw = _config5_full_gradients_fp32(c["h"], c["w"], c["t"])
    assert _rel(dh, ref_dh) < 2e-2, f"dH {_rel(dh, ref_dh):.2e}"
    assert _rel(dw, ref_dw) < 2e-2, f"dW {_rel(dw, ref_dw):.2e}"
    row_max = ref_dw.abs().max(-1).values
    big = row_max > 1e-3 * row_max.max()
    row_err = (dw.float() - ref_dw).abs().max(-1).values
    assert (row_err[big] / row_max[big]).max().item() < 5e-2
