"""E2 delta-rule write on the HIP kernels (qpam_delta_fwd / qpam_delta_bwd).

Reference: V11PAMLayer._forward_delta (v11/model.py:491-576, the chunked
UT-transform form with _complex_triangular_solve, :1005-1016) and
_recur_step_delta (:967-1002).  Both compute the token recurrence

    S <- g~ S;  u = beta (v - S k);  S <- S + u (x) k*;  y = S q~

with g~ = gamma + 1e-6 in the chunked form (its log(gamma + 1e-6) decays) and
g~ = gamma in the single step; the kernels compute the chunked form itself on
fp32 MFMA, forward and backward, over the reference's chunks of delta_chunk
steps (its clamped decay matrix and state-write weights included); the single
step uses the recurrence's exact write weight.

`delta_planar` is differentiable (torch.library custom op with a registered
autograd formula); `forward_delta` and `recur_step_delta` keep the reference
methods' split-real signatures.
"""

from typing import List, Optional

import torch
from torch import Tensor

from . import _lib
from .pam_scan import _cview, _mview

CHUNK_EPS = 1e-6


def _plane(t):
    t = t if t.dtype == torch.float32 else t.float()
    ok = t.stride(-1) == 1 and all(s % 4 == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0
    return t if ok else t.contiguous()


def _fill(q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im, q_scale, gamma_eps, chunk, exact_write):
    for t in (q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta):
        if not t.is_cuda:
            raise ValueError("qpam delta: tensors must be on the GPU (no CPU path in this library)")
    B, H, T, d = q_re.shape
    if d != 64:
        raise NotImplementedError("the HIP delta rule supports head_dim 64")
    for t in (q_re, q_im, k_re, k_im, v_re, v_im):
        if tuple(t.shape) != (B, H, T, d):
            raise ValueError(f"q/k/v planes must be [B,H,T,d] = {(B, H, T, d)}, got {tuple(t.shape)}")
    if tuple(gamma.shape) != (B, H, T) or gamma.shape != beta.shape:
        raise ValueError("gamma and beta must be [B, H, T]")
    if not 1 <= chunk <= 64:
        raise NotImplementedError(f"the HIP delta rule runs chunks of 1..64 steps, got {chunk}")
    a = _lib.DeltaArgs()
    a.B, a.H, a.T, a.d = B, H, T, d
    a.q_scale, a.gamma_eps = float(q_scale), float(gamma_eps)
    a.chunk, a.exact_write = int(chunk), int(bool(exact_write))
    keep = []
    for name, (re, im) in (("q", (q_re, q_im)), ("k", (k_re, k_im)), ("v", (v_re, v_im))):
        view, re, im = _cview(_plane(re), _plane(im))
        keep += [re, im]
        setattr(a, name, view)
    gamma, beta = gamma.float(), beta.float()
    if gamma.stride() != beta.stride():
        gamma, beta = gamma.contiguous(), beta.contiguous()
    keep += [gamma, beta]
    a.gamma, a.beta = gamma.data_ptr(), beta.data_ptr()
    a.sg_b, a.sg_h, a.sg_t = gamma.stride()
    if s0_re is not None:
        s0_re, s0_im = s0_re.float().contiguous(), s0_im.float().contiguous()
        keep += [s0_re, s0_im]
        a.s0_re, a.s0_im = s0_re.data_ptr(), s0_im.data_ptr()
    return a, keep


@torch.library.custom_op("qpam::delta_fwd", mutates_args=())
def delta_fwd_op(q_re: Tensor, q_im: Tensor, k_re: Tensor, k_im: Tensor, v_re: Tensor, v_im: Tensor,
                 gamma: Tensor, beta: Tensor, s0_re: Optional[Tensor], s0_im: Optional[Tensor], q_scale: float,
                 gamma_eps: float, chunk: int, exact_write: bool, keep_workspace: bool) -> List[Tensor]:
    """Returns [y_re, y_im ([B,H,T,d] fp32), s_re, s_im ([B,H,d,d]), workspace]."""
    a, keep = _fill(q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im, q_scale, gamma_eps, chunk,
                    exact_write)
    B, H, T, d = q_re.shape
    dev = q_re.device
    y_re = torch.empty(B, H, T, d, device=dev, dtype=torch.float32)
    y_im = torch.empty_like(y_re)
    s_re = torch.empty(B, H, d, d, device=dev, dtype=torch.float32)
    s_im = torch.empty_like(s_re)
    a.y = _mview(y_re, y_im)
    a.s_re, a.s_im = s_re.data_ptr(), s_im.data_ptr()
    L = _lib.lib()
    if keep_workspace:
        nbytes = L.qpam_delta_workspace_size(a)
        ws = torch.empty((nbytes + 3) // 4, device=dev, dtype=torch.float32)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * 4
    else:
        ws = torch.empty(0, device=dev, dtype=torch.float32)
    if T > 0 and B > 0:
        # the forward's per-chunk products (freed when the call returns; the
        # caching allocator keeps the block for the next call)
        scratch = torch.empty((L.qpam_delta_scratch_size(a) + 3) // 4, device=dev, dtype=torch.float32)
        a.scratch, a.scratch_bytes = scratch.data_ptr(), scratch.numel() * 4
        with torch.cuda.device(dev):
            _lib.check(L.qpam_delta_fwd(a, _lib.stream_ptr(dev)), "qpam_delta_fwd")
        del scratch
    else:
        y_re.zero_(), y_im.zero_()
        if s0_re is not None:
            s_re.copy_(s0_re), s_im.copy_(s0_im)
        else:
            s_re.zero_(), s_im.zero_()
    del keep
    return [y_re, y_im, s_re, s_im, ws]


# floats of one (b, h, chunk) record of the forward's workspace: entering state and U
# (2 x 2 d^2), four triangular products of 10 blocks x 512 floats, L (64)
_WS_REC = 4 * 64 * 64 + 4 * 10 * 512 + 64


def _ws_bytes(B, H, T, d=64, chunk=64):
    return B * H * ((T + chunk - 1) // chunk) * _WS_REC * 4


@delta_fwd_op.register_fake
def _(q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im, q_scale, gamma_eps, chunk, exact_write,
      keep_workspace):
    B, H, T, d = q_re.shape
    y = q_re.new_empty(B, H, T, d, dtype=torch.float32)
    s = q_re.new_empty(B, H, d, d, dtype=torch.float32)
    ws = q_re.new_empty(_ws_bytes(B, H, T, d, chunk) // 4 if keep_workspace else 0, dtype=torch.float32)
    return [y, torch.empty_like(y), s, torch.empty_like(s), ws]


@torch.library.custom_op("qpam::delta_bwd", mutates_args=())
def delta_bwd_op(q_re: Tensor, q_im: Tensor, k_re: Tensor, k_im: Tensor, v_re: Tensor, v_im: Tensor,
                 gamma: Tensor, beta: Tensor, s0_re: Optional[Tensor], s0_im: Optional[Tensor], q_scale: float,
                 gamma_eps: float, chunk: int, exact_write: bool, ws: Tensor, dy_re: Tensor, dy_im: Tensor,
                 ds_re: Optional[Tensor], ds_im: Optional[Tensor]) -> List[Tensor]:
    """Returns [dq_re, dq_im, dk_re, dk_im, dv_re, dv_im, dgamma, dbeta, ds0_re, ds0_im]
    (ds0 empty without s0)."""
    # the kernels write dgamma and dbeta with gamma's strides: contiguous planes,
    # matching the gradients allocated below
    gamma, beta = gamma.contiguous(), beta.contiguous()
    a, keep = _fill(q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im, q_scale, gamma_eps, chunk,
                    exact_write)
    B, H, T, d = q_re.shape
    dev = q_re.device
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * 4
    g = _lib.DeltaBwdArgs()
    g.fwd = _lib.ctypes.pointer(a)
    dy_re, dy_im = dy_re.float().contiguous(), dy_im.float().contiguous()
    g.dy, _, _ = _cview(dy_re, dy_im)
    if ds_re is not None:
        ds_re, ds_im = ds_re.float().contiguous(), ds_im.float().contiguous()
        g.ds_re, g.ds_im = ds_re.data_ptr(), ds_im.data_ptr()
    outs = [torch.empty(B, H, T, d, device=dev, dtype=torch.float32) for _ in range(6)]
    g.dq, g.dk, g.dv = _mview(outs[0], outs[1]), _mview(outs[2], outs[3]), _mview(outs[4], outs[5])
    dgamma = torch.empty(B, H, T, device=dev, dtype=torch.float32)
    dbeta = torch.empty_like(dgamma)
    g.dgamma, g.dbeta = dgamma.data_ptr(), dbeta.data_ptr()
    if s0_re is not None:
        ds0 = [torch.empty(B, H, d, d, device=dev, dtype=torch.float32) for _ in range(2)]
        g.ds0_re, g.ds0_im = ds0[0].data_ptr(), ds0[1].data_ptr()
    else:
        ds0 = [dgamma.new_empty(0), dgamma.new_empty(0)]
    L = _lib.lib()
    nbytes = L.qpam_delta_bwd_workspace_size(g)
    ws2 = torch.empty((nbytes + 3) // 4 + 4, device=dev, dtype=torch.float32)
    g.workspace, g.workspace_bytes = ws2.data_ptr(), ws2.numel() * 4
    with torch.cuda.device(dev):
        _lib.check(L.qpam_delta_bwd(g, _lib.stream_ptr(dev)), "qpam_delta_bwd")
    del keep
    return outs + [dgamma, dbeta] + ds0


@delta_bwd_op.register_fake
def _(q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im, q_scale, gamma_eps, chunk, exact_write, ws,
      dy_re, dy_im, ds_re, ds_im):
    B, H, T, d = q_re.shape
    outs = [q_re.new_empty(B, H, T, d, dtype=torch.float32) for _ in range(6)]
    dg = gamma.new_empty(B, H, T, dtype=torch.float32)
    ds0 = [gamma.new_empty(B, H, d, d, dtype=torch.float32) if s0_re is not None else gamma.new_empty(0)
           for _ in range(2)]
    return outs + [dg, torch.empty_like(dg)] + ds0


def _setup(ctx, inputs, output):
    (q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im, q_scale, gamma_eps, chunk, exact_write,
     keep_ws) = inputs
    ctx.save_for_backward(q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im, output[4])
    ctx.q_scale, ctx.gamma_eps, ctx.keep = q_scale, gamma_eps, keep_ws
    ctx.chunk, ctx.exact_write = chunk, exact_write
    ctx.set_materialize_grads(False)


def _backward(ctx, grads):
    q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im, ws = ctx.saved_tensors
    if not ctx.keep:
        raise RuntimeError("qpam delta: the forward ran without its backward workspace (keep_workspace=False)")
    dy_re, dy_im, ds_re, ds_im = grads[0], grads[1], grads[2], grads[3]
    if dy_re is None:
        dy_re = torch.zeros_like(q_re, dtype=torch.float32)
    if dy_im is None:
        dy_im = torch.zeros_like(q_re, dtype=torch.float32)
    if ds_re is None and ds_im is None:
        ds = (None, None)
    else:
        ds = (ds_re if ds_re is not None else torch.zeros_like(ds_im), ds_im if ds_im is not None else torch.zeros_like(ds_re))
    g = delta_bwd_op(q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im, ctx.q_scale, ctx.gamma_eps,
                     ctx.chunk, ctx.exact_write, ws, dy_re, dy_im, ds[0], ds[1])
    cast = (lambda x, like: x.to(like.dtype) if x.dtype != like.dtype else x)
    out = [cast(g[i], t) for i, t in enumerate((q_re, q_im, k_re, k_im, v_re, v_im))]
    out += [cast(g[6], gamma), cast(g[7], beta)]
    out += [g[8], g[9]] if s0_re is not None else [None, None]
    return tuple(out) + (None, None, None, None, None)


delta_fwd_op.register_autograd(_backward, setup_context=_setup)


def delta_planar(q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, *, q_scale, gamma_eps=CHUNK_EPS, s0=None,
                 chunk=64, exact_write=False):
    """Differentiable delta-rule scan on planar [B,H,T,d] planes, d <= 64
    (computed in fp32).  gamma, beta [B,H,T]; s0 optional (re, im) [B,H,d,d].
    `chunk` is the chunked form's chunk length (the reference's delta_chunk,
    1..64); exact_write uses the token recurrence's state-write weight (1 on
    the step itself) instead of the chunked form's alpha_last / (alpha_s + 1e-12).
    Returns (y_re, y_im, s_re, s_im).

    d < 64 is zero-padded to 64 and sliced back, which is exact: padded key
    columns add nothing to k.k*, S k or q.k*, and padded value rows of the
    update (beta (v - S k)) and of the state stay zero."""
    s0_re, s0_im = s0 if s0 is not None else (None, None)
    d = q_re.shape[-1]
    if d < 64:
        pad = 64 - d
        q_re, q_im, k_re, k_im, v_re, v_im = (torch.nn.functional.pad(x, (0, pad))
                                              for x in (q_re, q_im, k_re, k_im, v_re, v_im))
        if s0_re is not None:
            s0_re, s0_im = (torch.nn.functional.pad(x, (0, pad, 0, pad)) for x in (s0_re, s0_im))
        s0p = (s0_re, s0_im) if s0_re is not None else None
        y_re, y_im, s_re, s_im = delta_planar(q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, q_scale=q_scale,
                                              gamma_eps=gamma_eps, s0=s0p, chunk=chunk, exact_write=exact_write)
        return y_re[..., :d], y_im[..., :d], s_re[..., :d, :d], s_im[..., :d, :d]
    keep = torch.is_grad_enabled() and any(
        t is not None and t.requires_grad for t in (q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im))
    out = delta_fwd_op(q_re, q_im, k_re, k_im, v_re, v_im, gamma, beta, s0_re, s0_im, float(q_scale),
                       float(gamma_eps), int(chunk), bool(exact_write), bool(keep))
    return out[0], out[1], out[2], out[3]


def forward_delta(queries, keys, protected_values, decay_gamma, write_beta, head_dim, state=None, chunk=64):
    """V11PAMLayer._forward_delta (v11/model.py:491-576) on split-real
    [B,H,T,d,2] tensors (queries unscaled), decay_gamma / write_beta [B,H,T],
    chunks of `chunk` steps (the layer's delta_chunk, v11/model.py:494).
    Returns (output [B,H,T,d,2], memory_state [B,H,d,d,2]) in the input dtype."""
    dtype = queries.dtype
    planes = [x[..., i] for x in (queries, keys, protected_values) for i in (0, 1)]
    s0 = (state[..., 0], state[..., 1]) if state is not None else None
    y_re, y_im, s_re, s_im = delta_planar(*planes, decay_gamma, write_beta, q_scale=head_dim ** -0.5,
                                          gamma_eps=CHUNK_EPS, s0=s0, chunk=chunk)
    return torch.stack([y_re, y_im], -1).to(dtype), torch.stack([s_re, s_im], -1).to(dtype)


def recur_step_delta(memory_state, decay_gamma, value_t, key_t, query_t, write_beta_t):
    """V11PAMLayer._recur_step_delta (v11/model.py:967-1002): one token,
    memory_state [B,H,d,d,2], decay_gamma / write_beta_t [B,H], value/key/query
    [B,H,d,2] (query already scaled).  Returns (output [B,H,d,2], new state);
    the input state is not modified.  The step's write has weight 1 (the
    exact recurrence) and gamma is used as given (no 1e-6 shift)."""
    dtype = memory_state.dtype
    planes = [x[..., i].unsqueeze(2) for x in (query_t, key_t, value_t) for i in (0, 1)]
    y_re, y_im, s_re, s_im = delta_planar(*planes, decay_gamma.unsqueeze(-1), write_beta_t.unsqueeze(-1),
                                          q_scale=1.0, gamma_eps=0.0, exact_write=True,
                                          s0=(memory_state[..., 0], memory_state[..., 1]))
    return torch.stack([y_re[:, :, 0], y_im[:, :, 0]], -1).to(dtype), torch.stack([s_re, s_im], -1).to(dtype)
