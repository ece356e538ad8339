"""CPU restatement of the tied complex LM-head cross-entropy (test infrastructure only).

Follows v11/fused_ce.py:26-141 and V11LM.ce_from_lm (v11/model.py:1175-1190):
  hidden_rows = [lm_r | lm_i]  [N, 2d],  weight_matrix = [E_r | E_i]  [V, 2d]
  logits      = hidden_rows @ weight_matrix.T = Re(h . conj(E)^T)
  loss        = sum_n CE_n * mask_n / denom,
  denom       = mask.sum().clamp_min(1) or #(targets != ignore).clamp_min(1)
Forward and backward are the reference's row-chunk loops computed in fp32
(`.float()`), gradient = (softmax - onehot) * grad/denom (* mask), zeroed on
ignore rows.
"""

import torch
import torch.nn.functional as F


def ce_forward(hidden_rows, weight_matrix, targets, mask=None, chunk=4096, ignore_index=-100):
    """_FusedLinearCE.forward (v11/fused_ce.py:28-53).  Returns (loss, denom)."""
    n = hidden_rows.shape[0]
    loss_sum = torch.zeros((), dtype=torch.float32 if hidden_rows.dtype != torch.float64 else torch.float64)
    if mask is not None:
        denom = mask.sum().clamp_min(1.0)
    else:
        denom = (targets != ignore_index).sum().clamp_min(1).to(loss_sum.dtype)
    acc = torch.float64 if hidden_rows.dtype == torch.float64 else torch.float32
    for c0 in range(0, n, chunk):
        c1 = min(c0 + chunk, n)
        logits = hidden_rows[c0:c1].to(acc) @ weight_matrix.to(acc).T
        per = F.cross_entropy(logits, targets[c0:c1], ignore_index=ignore_index, reduction='none')
        if mask is not None:
            per = per * mask[c0:c1].to(acc)
        loss_sum = loss_sum + per.sum()
    return loss_sum / denom, denom


def ce_backward(hidden_rows, weight_matrix, targets, denom, grad_output=1.0, mask=None, chunk=4096,
                ignore_index=-100):
    """_FusedLinearCE.backward (v11/fused_ce.py:56-82).  Returns (dH, dW) in the
    input dtypes (the reference casts each chunk's products back)."""
    n = hidden_rows.shape[0]
    acc = torch.float64 if hidden_rows.dtype == torch.float64 else torch.float32
    scale = grad_output / denom
    d_h = torch.zeros_like(hidden_rows)
    d_w = torch.zeros_like(weight_matrix)
    w = weight_matrix.to(acc)
    for c0 in range(0, n, chunk):
        c1 = min(c0 + chunk, n)
        h = hidden_rows[c0:c1].to(acc)
        p = torch.softmax(h @ w.T, dim=-1)
        tgt = targets[c0:c1]
        valid = tgt != ignore_index
        safe = torch.where(valid, tgt, torch.zeros_like(tgt))
        p.scatter_add_(1, safe.unsqueeze(1), -torch.ones_like(safe, dtype=p.dtype).unsqueeze(1))
        if mask is not None:
            p = p * (scale * mask[c0:c1].to(acc)).unsqueeze(1)
        else:
            p = p * scale
        p = p * valid.unsqueeze(1).to(acc)
        d_h[c0:c1] = (p @ w).to(d_h.dtype)
        d_w += (p.T @ h).to(d_w.dtype)
    return d_h, d_w


def ce_per_token(hidden_rows, weight_matrix, targets, chunk=4096, ignore_index=-100):
    """linear_ce_per_token (v11/fused_ce.py:98-115): per-row CE, 0 on ignore rows."""
    out = torch.zeros(hidden_rows.shape[0], dtype=torch.float32)
    for c0 in range(0, hidden_rows.shape[0], chunk):
        c1 = min(c0 + chunk, hidden_rows.shape[0])
        logits = hidden_rows[c0:c1].float() @ weight_matrix.float().T
        out[c0:c1] = F.cross_entropy(logits, targets[c0:c1], ignore_index=ignore_index, reduction='none')
    return out


def ce_stats(hidden_rows, weight_matrix, targets, mask=None, chunk=4096, ignore_index=-100):
    """linear_ce_stats (v11/fused_ce.py:118-141): (loss_sum, correct, tokens)."""
    loss_sum = correct = tokens = 0.0
    for c0 in range(0, hidden_rows.shape[0], chunk):
        c1 = min(c0 + chunk, hidden_rows.shape[0])
        logits = hidden_rows[c0:c1].float() @ weight_matrix.float().T
        tgt = targets[c0:c1]
        per = F.cross_entropy(logits, tgt, ignore_index=ignore_index, reduction='none')
        ok = (logits.argmax(dim=-1) == tgt).float()
        tm = mask[c0:c1].float() if mask is not None else (tgt != ignore_index).float()
        loss_sum += (per * tm).sum().item()
        correct += (ok * tm).sum().item()
        tokens += tm.sum().item()
    return loss_sum, correct, tokens


def make_ce_inputs(N, d_model, V, seed, *, ignore_frac=0.1, ignore_index=-100, e_std=0.02,
                   dtype=torch.bfloat16):
    """Seeded config-5 style inputs drawn in float64 on the CPU: h complex
    ~N(0,1) per part, E complex ~N(0, e_std^2), labels U[0,V) with a fraction
    set to ignore_index.  Returns real-concat hidden [N, 2d], weight [V, 2d]
    (cast to `dtype`) and int64 targets."""
    g = torch.Generator('cpu').manual_seed(seed)
    h = torch.randn(N, 2 * d_model, generator=g, dtype=torch.float64)
    e = torch.randn(V, 2 * d_model, generator=g, dtype=torch.float64) * e_std
    tgt = torch.randint(0, V, (N,), generator=g)
    drop = torch.rand(N, generator=g, dtype=torch.float64) < ignore_frac
    tgt = torch.where(drop, torch.full_like(tgt, ignore_index), tgt)
    return h.to(dtype), e.to(dtype), tgt


def ce_flops(N, V, D):
    """Algorithmic FLOPs of fwd+bwd (logit recompute excluded): 3 GEMMs of 2*N*V*D."""
    return 3 * 2 * N * V * D
