"""Fused tied LM-head cross-entropy on the HIP kernels (qpam_ce_fwd / qpam_ce_bwd).

Same functions, arguments and autograd contract as the reference module
v11/fused_ce.py (fused_linear_cross_entropy 85-94, linear_ce_per_token 98-115,
linear_ce_stats 118-141): hidden_rows [N, 2d] = [lm_r | lm_i], weight_matrix
[V, 2d] = [E_r | E_i], logits = hidden_rows @ weight_matrix.T, mean (or
mask-weighted) cross-entropy with ignore_index; gradients flow to
hidden_rows and weight_matrix only.

Precision: if either operand is bf16 the GEMMs run on bf16 MFMA with fp32
accumulation (the other operand is cast to bf16); two fp32 operands run on
fp32 MFMA.  dW is accumulated in fp32 and cast to the weight dtype; dH is
written in the hidden dtype.  Targets outside [0, V) that are not
ignore_index contribute zero loss (the reference raises for them).  CPU
tensors raise, except after pam_layer.install(), which keeps the reference's
own functions for them.
"""

from typing import List, Optional

import torch
from torch import Tensor

from . import _lib, _reference

__all__ = ["fused_linear_cross_entropy", "linear_ce_per_token", "linear_ce_stats"]


def _operands(hidden_rows, weight_matrix):
    if not (hidden_rows.is_cuda and weight_matrix.is_cuda):
        raise ValueError("qpam fused CE: tensors must be on the GPU (no CPU path in this library)")
    if hidden_rows.dim() != 2 or weight_matrix.dim() != 2 or hidden_rows.shape[1] != weight_matrix.shape[1]:
        raise ValueError(f"hidden_rows [N, D] and weight_matrix [V, D] expected, got "
                         f"{tuple(hidden_rows.shape)} and {tuple(weight_matrix.shape)}")
    if hidden_rows.shape[1] % 32:
        raise NotImplementedError("qpam fused CE needs D % 32 == 0")
    work = torch.bfloat16 if torch.bfloat16 in (hidden_rows.dtype, weight_matrix.dtype) else torch.float32
    h = hidden_rows.to(work)
    w = weight_matrix.to(work)
    vec = 8 if work == torch.bfloat16 else 4
    if h.stride(1) != 1 or h.stride(0) % vec or h.data_ptr() % 16:
        h = h.contiguous()
    if w.stride(1) != 1 or w.stride(0) % vec or w.data_ptr() % 16:
        w = w.contiguous()
    return h, w, (_lib.QPAM_BF16 if work == torch.bfloat16 else _lib.QPAM_F32)


def _fwd_args(h, w, dtype, targets, mask, ignore_index):
    a = _lib.CeFwdArgs()
    a.N, a.V, a.D, a.dtype = h.shape[0], w.shape[0], h.shape[1], dtype
    a.h, a.ldh, a.w, a.ldw = h.data_ptr(), h.stride(0), w.data_ptr(), w.stride(0)
    a.targets = targets.data_ptr()
    a.mask = mask.data_ptr() if mask is not None else None
    a.ignore_index = int(ignore_index)
    return a


def _run_fwd(h, w, dtype, targets, mask, ignore_index, want_correct):
    n = h.shape[0]
    dev = h.device
    lse = torch.empty(n, device=dev, dtype=torch.float32)
    loss = torch.empty(n, device=dev, dtype=torch.float32)
    correct = torch.empty(n, device=dev, dtype=torch.float32) if want_correct else None
    red = torch.empty(2, device=dev, dtype=torch.float32)
    a = _fwd_args(h, w, dtype, targets, mask, ignore_index)
    a.lse, a.loss, a.loss_sum = lse.data_ptr(), loss.data_ptr(), red.data_ptr()
    a.correct = correct.data_ptr() if correct is not None else None
    L = _lib.lib()
    nbytes = L.qpam_ce_fwd_workspace_size(a)
    ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    with torch.cuda.device(dev):
        _lib.check(L.qpam_ce_fwd(a, _lib.stream_ptr(dev)), "qpam_ce_fwd")
    return lse, loss, correct, red


def _prep_targets(targets, mask, n):
    if targets.shape != (n,):
        raise ValueError(f"targets must be [{n}]")
    targets = targets.to(torch.int64).contiguous()
    if mask is not None:
        mask = mask.to(torch.float32).contiguous()
        if mask.shape != (n,):
            raise ValueError(f"mask must be [{n}]")
    return targets, mask


@torch.library.custom_op("qpam::ce_fwd", mutates_args=())
def ce_fwd_op(hidden_rows: Tensor, weight_matrix: Tensor, targets: Tensor, mask: Optional[Tensor],
              ignore_index: int) -> List[Tensor]:
    """Returns [loss (0-d fp32, as the reference's fp32 chunk sums), lse [N] fp32, denom (0-d fp32)]."""
    h, w, dtype = _operands(hidden_rows, weight_matrix)
    targets, mask = _prep_targets(targets, mask, h.shape[0])
    lse, _, _, red = _run_fwd(h, w, dtype, targets, mask, ignore_index, False)
    denom = red[1].clamp_min(1.0)
    loss = red[0] / denom
    return [loss, lse, denom]


@ce_fwd_op.register_fake
def _(hidden_rows, weight_matrix, targets, mask, ignore_index):
    n = hidden_rows.shape[0]
    return [hidden_rows.new_empty((), dtype=torch.float32), hidden_rows.new_empty(n, dtype=torch.float32),
            hidden_rows.new_empty((), dtype=torch.float32)]


@torch.library.custom_op("qpam::ce_bwd", mutates_args=())
def ce_bwd_op(hidden_rows: Tensor, weight_matrix: Tensor, targets: Tensor, mask: Optional[Tensor],
              ignore_index: int, lse: Tensor, grad_scale: Tensor, chunk: int, dw_fp32: bool = False) -> List[Tensor]:
    """Returns [d hidden_rows, d weight_matrix] in the input dtypes (d
    weight_matrix in fp32 with dw_fp32: the gradient of an fp32 master weight
    whose bf16 copy is weight_matrix)."""
    h, w, dtype = _operands(hidden_rows, weight_matrix)
    targets, mask = _prep_targets(targets, mask, h.shape[0])
    dev = h.device
    dh = torch.empty_like(h)
    # the weight's own dtype is the working one: the library writes dW in it (no
    # zero fill, no conversion pass); an fp32 master weight run on its bf16 copy
    # keeps the fp32 accumulation
    # fp32 dW written (no zero fill) for an fp32 master weight: dw_fp32, or an fp32
    # weight_matrix run on its bf16 copy here
    fp32_dw = dw_fp32 or weight_matrix.dtype != w.dtype
    dw = torch.empty(w.shape, device=dev, dtype=torch.float32 if fp32_dw else w.dtype)
    gs = grad_scale.to(torch.float32).reshape(1).contiguous()
    a = _lib.CeBwdArgs()
    a.N, a.V, a.D, a.dtype = h.shape[0], w.shape[0], h.shape[1], dtype
    a.h, a.ldh, a.w, a.ldw = h.data_ptr(), h.stride(0), w.data_ptr(), w.stride(0)
    a.targets = targets.data_ptr()
    a.mask = mask.data_ptr() if mask is not None else None
    a.ignore_index = int(ignore_index)
    a.lse, a.grad_scale = lse.data_ptr(), gs.data_ptr()
    a.dh, a.lddh, a.dw, a.lddw = dh.data_ptr(), dh.stride(0), dw.data_ptr(), dw.stride(0)
    a.chunk = int(max(1, min(chunk, h.shape[0])))
    a.dw_out = 2 if fp32_dw else 1
    L = _lib.lib()
    nbytes = L.qpam_ce_bwd_workspace_size(a)
    ws = torch.empty(nbytes, device=dev, dtype=torch.uint8)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    with torch.cuda.device(dev):
        _lib.check(L.qpam_ce_bwd(a, _lib.stream_ptr(dev)), "qpam_ce_bwd")
    return [dh.to(hidden_rows.dtype), dw if fp32_dw else dw.to(weight_matrix.dtype)]


@ce_bwd_op.register_fake
def _(hidden_rows, weight_matrix, targets, mask, ignore_index, lse, grad_scale, chunk, dw_fp32=False):
    return [torch.empty_like(hidden_rows),
            torch.empty_like(weight_matrix, dtype=torch.float32 if dw_fp32 else weight_matrix.dtype)]


class _FusedLinearCE(torch.autograd.Function):
    """Autograd wrapper with the reference's signature (v11/fused_ce.py:26-82)."""

    @staticmethod
    def forward(ctx, hidden_rows, weight_matrix, targets, mask, chunk, ignore_index):
        # an fp32 master weight with bf16 rows: one bf16 copy serves the forward and the backward
        master = weight_matrix.dtype == torch.float32 and hidden_rows.dtype == torch.bfloat16
        w_op = weight_matrix.to(torch.bfloat16) if master else weight_matrix
        loss, lse, denom = ce_fwd_op(hidden_rows, w_op, targets, mask, ignore_index)
        ctx.save_for_backward(hidden_rows, w_op, targets, mask, lse, denom)
        ctx.chunk, ctx.ignore_index, ctx.master = chunk, ignore_index, master
        return loss

    @staticmethod
    def backward(ctx, grad_output):
        hidden_rows, w_op, targets, mask, lse, denom = ctx.saved_tensors
        grad_scale = grad_output.to(torch.float32) / denom
        dh, dw = ce_bwd_op(hidden_rows, w_op, targets, mask, ctx.ignore_index, lse, grad_scale, ctx.chunk,
                           ctx.master)
        return dh, dw, None, None, None, None


def fused_linear_cross_entropy(hidden_rows: Tensor, weight_matrix: Tensor, targets: Tensor,
                               mask: Optional[Tensor] = None, chunk: int = 4096,
                               ignore_index: int = -100) -> Tensor:
    """Mean cross-entropy of (hidden_rows @ weight_matrix.T) vs targets
    (v11/fused_ce.py:85-94).  `chunk` bounds the backward's live gradient
    memory as in the reference (fp32 logits and softmax of `chunk` rows, 8
    bytes per row and vocabulary entry): with bf16 operands one pass holds a
    bf16 gradient of 4 x chunk rows (2 x chunk with QPAM_CE_GEMM=hip), the
    same bytes.  An fp32 weight_matrix with bf16 hidden_rows (fp32 master
    embedding) runs on a bf16 copy of the weights and returns an fp32
    gradient."""
    if not hidden_rows.is_cuda:
        return _reference.on_cpu("fused_ce.fused_linear_cross_entropy", "fused_linear_cross_entropy", hidden_rows,
                                 weight_matrix, targets, mask=mask, chunk=chunk, ignore_index=ignore_index)
    return _FusedLinearCE.apply(hidden_rows, weight_matrix, targets, mask, chunk, ignore_index)


@torch.no_grad()
def linear_ce_per_token(hidden_rows, weight_matrix, targets, chunk: int = 4096, ignore_index: int = -100):
    """Per-row cross-entropy [N], 0.0 on ignore rows (v11/fused_ce.py:98-115)."""
    if not hidden_rows.is_cuda:
        return _reference.on_cpu("fused_ce.linear_ce_per_token", "linear_ce_per_token", hidden_rows, weight_matrix,
                                 targets, chunk=chunk, ignore_index=ignore_index)
    h, w, dtype = _operands(hidden_rows, weight_matrix)
    targets, _ = _prep_targets(targets, None, h.shape[0])
    _, loss, _, _ = _run_fwd(h, w, dtype, targets, None, ignore_index, False)
    return loss.to(hidden_rows.dtype)


@torch.no_grad()
def linear_ce_stats(hidden_rows, weight_matrix, targets, mask=None, chunk: int = 4096, ignore_index: int = -100):
    """(loss_sum, correct, tokens) as Python floats (v11/fused_ce.py:118-141)."""
    if not hidden_rows.is_cuda:
        return _reference.on_cpu("fused_ce.linear_ce_stats", "linear_ce_stats", hidden_rows, weight_matrix, targets,
                                 mask=mask, chunk=chunk, ignore_index=ignore_index)
    h, w, dtype = _operands(hidden_rows, weight_matrix)
    targets, maskf = _prep_targets(targets, mask, h.shape[0])
    _, loss, correct, _ = _run_fwd(h, w, dtype, targets, None, ignore_index, True)
    if maskf is not None:
        token_mask = maskf
    else:
        token_mask = (targets != ignore_index).to(torch.float32)
    vals = torch.stack([(loss * token_mask).sum(), (correct * token_mask).sum(), token_mask.sum()]).tolist()
    return vals[0], vals[1], vals[2]
