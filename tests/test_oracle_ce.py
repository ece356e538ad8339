"""Pins the CPU cross-entropy oracle against F.cross_entropy on full logits
(the reference's own check, v11/fused_ce.py:144-186 and v11/selftest.py:102-126),
with closed-form gradients (softmax - onehot)/denom."""

import torch
import torch.nn.functional as F

from oracle import ce as O


def _data(n=200, d=48, v=512, seed=0):
    g = torch.Generator().manual_seed(seed)
    h = torch.randn(n, d, generator=g, dtype=torch.float64)
    w = torch.randn(v, d, generator=g, dtype=torch.float64)
    t = torch.randint(0, v, (n,), generator=g)
    return h, w, t


def test_ce_forward_backward_ignore_index():
    h, w, t = _data()
    t[::7] = -100
    hr, wr = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    ref = F.cross_entropy(hr @ wr.T, t, ignore_index=-100)
    ref.backward()
    loss, denom = O.ce_forward(h, w, t, chunk=32)
    assert abs(loss.item() - ref.item()) < 1e-12
    d_h, d_w = O.ce_backward(h, w, t, denom, chunk=32)
    assert (d_h - hr.grad).abs().max() < 1e-12
    assert (d_w - wr.grad).abs().max() < 1e-12
    # closed form: G = (softmax - onehot)/denom on valid rows
    p = torch.softmax(h @ w.T, -1)
    valid = t != -100
    p[valid, t[valid]] -= 1
    p[~valid] = 0
    p /= valid.sum()
    assert (d_h - p @ w).abs().max() < 1e-12 and (d_w - p.T @ h).abs().max() < 1e-12


def test_ce_mask_and_grad_output():
    h, w, t = _data(seed=1)
    mask = (torch.rand(h.shape[0], generator=torch.Generator().manual_seed(3)) > 0.3).double()
    hr, wr = h.clone().requires_grad_(True), w.clone().requires_grad_(True)
    per = F.cross_entropy(hr @ wr.T, t, reduction='none')
    ref = (per * mask).sum() / mask.sum().clamp_min(1)
    (2.5 * ref).backward()
    loss, denom = O.ce_forward(h, w, t, mask=mask, chunk=64, ignore_index=-1)
    assert abs(loss.item() - ref.item()) < 1e-12
    d_h, d_w = O.ce_backward(h, w, t, denom, grad_output=2.5, mask=mask, chunk=64, ignore_index=-1)
    assert (d_h - hr.grad).abs().max() < 1e-12 and (d_w - wr.grad).abs().max() < 1e-12


def test_ce_all_ignored_denominator_clamps():
    h, w, t = _data(n=10)
    t[:] = -100
    loss, denom = O.ce_forward(h, w, t)
    assert loss.item() == 0.0 and denom.item() == 1
    d_h, d_w = O.ce_backward(h, w, t, denom)
    assert torch.all(d_h == 0) and torch.all(d_w == 0)


def test_ce_per_token_and_stats():
    h, w, t = _data(n=64, seed=4)
    t[::5] = -100
    logits = (h @ w.T).float()
    per = O.ce_per_token(h, w, t, chunk=24)
    ref = F.cross_entropy(logits, t, ignore_index=-100, reduction='none')
    assert torch.allclose(per, ref, atol=1e-5)
    loss_sum, correct, tokens = O.ce_stats(h, w, t, chunk=24)
    valid = t != -100
    assert tokens == valid.sum().item()
    assert abs(loss_sum - ref[valid].sum().item()) < 1e-3
    assert correct == ((logits.argmax(-1) == t) & valid).sum().item()
    # logsumexp identity
    assert torch.allclose(per[valid], torch.logsumexp(logits, -1)[valid] - logits[valid, t[valid]], atol=1e-5)
