"""Chunked dual-form PAM scan on the HIP kernels (qpam_scan_fwd / qpam_scan_bwd).

Planar API: every complex tensor is a pair of real planes.  q, k, v are
[B, H, T, d] (any strides with d contiguous), fp32 or bf16; gamma is fp32
[M, B, H, T]; optional rot (r_m = alpha_m e^{i phi_m}) is a pair of fp32
[M, B, H, T] planes; optional s0 is a pair of fp32 [M, B, H, d, d] planes.
Outputs Y (fp32 planes [B, H, T, d]) and the final state S (fp32 planes
[M, B, H, d, d]).  Math: v11/model.py:378-417 (M = 1) and 657-781 (M > 1).

The ops are registered with torch.library (custom_op + register_fake +
register_autograd) so autograd and torch.compile see them as single nodes.

Chunking: the kernels run chunks of 16, 32 or 64 steps.  With gamma + 1e-6 < 1
the chunked result does not depend on the chunk length (every term is a
product of (gamma + 1e-6) factors), so a reference chunk_size outside
{16, 32} runs with 64-step chunks; see chunk_for().
"""

from typing import List, Optional, Tuple

import torch
from torch import Tensor

from . import _lib

KERNEL_CHUNKS = (16, 32, 64)
SEG = 4  # 64-step chunks per segment of the bf16 kernels (workspace layout)

# Optional EventPair whose events the next forward records around its
# dominant (chunk-output) kernel; set by benchmarks, cleared after use.
_PROFILE = {"fwd": None}


def set_profile_events(pair):
    """Arm a _lib.EventPair to be recorded around the next forward's
    chunk-output kernel (benchmark instrumentation)."""
    _PROFILE["fwd"] = pair


def chunk_for(chunk_size: int, seq_len: int) -> int:
    """Kernel chunk length used for a reference chunk_size."""
    if chunk_size in (16, 32):
        return chunk_size
    return 64


def _dtype_code(t):
    if t.dtype == torch.float32:
        return _lib.QPAM_F32
    if t.dtype == torch.bfloat16:
        return _lib.QPAM_BF16
    raise ValueError(f"qpam scan: q/k/v must be fp32 or bf16, got {t.dtype}")


def _aligned_plane(t):
    vec = 4 if t.dtype == torch.float32 else 8
    ok = t.stride(-1) == 1 and all(s % vec == 0 for s in t.stride()[:-1]) and t.data_ptr() % 16 == 0
    return t if ok else t.contiguous()


def _cview(re, im):
    if re.stride() != im.stride():
        im = im.contiguous() if re.is_contiguous() else im
        re = re.contiguous()
        im = im.contiguous()
    v = _lib.CView()
    v.re, v.im = re.data_ptr(), im.data_ptr()
    v.s0, v.s1, v.s2 = re.stride(0), re.stride(1), re.stride(2)
    return v, re, im


def _mview(re, im):
    v = _lib.MView()
    v.re, v.im = re.data_ptr(), im.data_ptr()
    v.s0, v.s1, v.s2 = re.stride(0), re.stride(1), re.stride(2)
    return v


def _fill_args(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, q_scale, chunk):
    M, B, H, T = gamma.shape
    d = q_re.shape[-1]
    a = _lib.ScanArgs()
    a.B, a.H, a.T, a.d, a.C, a.M = B, H, T, d, chunk, M
    a.dtype = _dtype_code(q_re)
    a.q_scale = float(q_scale)
    keep = []
    for name, (re, im) in (("q", (q_re, q_im)), ("k", (k_re, k_im)), ("v", (v_re, v_im))):
        view, re, im = _cview(_aligned_plane(re), _aligned_plane(im))
        keep += [re, im]
        setattr(a, name, view)
    a.gamma = gamma.data_ptr()
    a.sg_m, a.sg_b, a.sg_h, a.sg_t = gamma.stride()
    if rot_re is not None:
        if rot_re.stride() != rot_im.stride():
            rot_re, rot_im = rot_re.contiguous(), rot_im.contiguous()
        keep += [rot_re, rot_im]
        a.rot_re, a.rot_im = rot_re.data_ptr(), rot_im.data_ptr()
        a.sr_m, a.sr_b, a.sr_h, a.sr_t = rot_re.stride()
    if s0_re is not None:
        s0_re, s0_im = s0_re.contiguous(), s0_im.contiguous()
        keep += [s0_re, s0_im]
        a.s0_re, a.s0_im = s0_re.data_ptr(), s0_im.data_ptr()
    return a, keep


def _validate(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, chunk):
    if chunk not in KERNEL_CHUNKS:
        raise ValueError(f"kernel chunk must be one of {KERNEL_CHUNKS}")
    if gamma.dim() != 4:
        raise ValueError("gamma must be [M, B, H, T]")
    M, B, H, T = gamma.shape
    for t in (q_re, q_im, k_re, k_im, v_re, v_im):
        if t.dim() != 4 or tuple(t.shape[:3]) != (B, H, T):
            raise ValueError(f"q/k/v planes must be [B={B}, H={H}, T={T}, d], got {tuple(t.shape)}")
        if t.dtype != q_re.dtype:
            raise ValueError("q, k, v must share one dtype")
        if not t.is_cuda:
            raise ValueError("qpam scan: tensors must be on the GPU (no CPU path in this library)")
    if gamma.dtype != torch.float32:
        raise ValueError("gamma must be fp32")
    if q_re.shape[-1] != 64:
        raise NotImplementedError("the HIP scan supports head_dim 64")
    if M > 4:
        raise NotImplementedError("the HIP scan supports up to 4 states")
    for t in (rot_re, rot_im):
        if t is not None and (tuple(t.shape) != (M, B, H, T) or t.dtype != torch.float32):
            raise ValueError("rot planes must be fp32 [M, B, H, T]")
    for t in (s0_re, s0_im):
        if t is not None and (tuple(t.shape) != (M, B, H, 64, 64) or t.dtype != torch.float32):
            raise ValueError("s0 planes must be fp32 [M, B, H, 64, 64]")


@torch.library.custom_op("qpam::scan_fwd", mutates_args=())
def scan_fwd_op(q_re: Tensor, q_im: Tensor, k_re: Tensor, k_im: Tensor, v_re: Tensor, v_im: Tensor,
                gamma: Tensor, rot_re: Optional[Tensor], rot_im: Optional[Tensor], s0_re: Optional[Tensor],
                s0_im: Optional[Tensor], q_scale: float, chunk: int, y_layout: int) -> List[Tensor]:
    """Returns [y_re, y_im, s_re, s_im, workspace]; the workspace keeps the
    per-chunk entering states for the backward.  y_layout 0: y planes
    [B,H,T,d]; 1: [B,T,H,d] (head-merged); 2: one tensor [B,T,2,H,d] in the
    y_re slot (re and im planes of a token side by side, the [N, 2 H d] input
    of one output-projection GEMM) and an empty y_im; 3: layout 2 in bf16 (bf16
    inputs, chunk 64: the kernel rounds y once from its fp32 result)."""
    _validate(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, chunk)
    M, B, H, T = gamma.shape
    d = q_re.shape[-1]
    dev = q_re.device
    a, keep = _fill_args(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, q_scale, chunk)
    if y_layout in (2, 3):
        y_re = torch.empty(B, T, 2, H, d, device=dev, dtype=torch.bfloat16 if y_layout == 3 else torch.float32)
        y_im = y_re.new_empty(0)
        a.y = _mview(y_re[:, :, 0].transpose(1, 2), y_re[:, :, 1].transpose(1, 2))
        a.y_dtype = 1 if y_layout == 3 else 0
    else:
        y_re = torch.empty((B, T, H, d) if y_layout == 1 else (B, H, T, d), device=dev, dtype=torch.float32)
        y_im = torch.empty_like(y_re)
        a.y = _mview(y_re.transpose(1, 2), y_im.transpose(1, 2)) if y_layout == 1 else _mview(y_re, y_im)
    s_re = torch.empty(M, B, H, d, d, device=dev, dtype=torch.float32)
    s_im = torch.empty_like(s_re)
    a.s_re, a.s_im = s_re.data_ptr(), s_im.data_ptr()
    L = _lib.lib()
    nbytes = L.qpam_scan_workspace_size(a)
    ws = torch.empty((nbytes + 3) // 4, device=dev, dtype=torch.float32)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * 4
    prof = _PROFILE["fwd"]
    if prof is not None:
        a.prof_ev[0], a.prof_ev[1] = prof.ev[0], prof.ev[1]
        _PROFILE["fwd"] = None
    with torch.cuda.device(dev):
        _lib.check(L.qpam_scan_fwd(a, _lib.stream_ptr(dev)), "qpam_scan_fwd")
    del keep
    return [y_re, y_im, s_re, s_im, ws]


def fwd_workspace_bytes(M, B, H, T, chunk, bf16, d=64):
    """Forward workspace size, as qpam_scan_workspace_size computes it: fp32
    per-chunk states (fp32 inputs) and chunk totals; with bf16 inputs and chunk
    64 also the segment totals, two per-step segment weights and the backward's
    per-step complex weights conj(rho_m[t]) q_scale, then at a
    256-byte aligned offset the bf16 snapshots of the entering states and the
    fp32 segment states; with fp32 inputs and chunk 64, at that offset the
    state pass's per-chunk decay weights."""
    chains, n = M * B * H, (T + chunk - 1) // chunk
    snap = bf16 and chunk == 64
    if snap:
        n_segs = (n + SEG - 1) // SEG
        floats = chains * n + chains * n_segs + 4 * chains * n * 64
        off = (floats * 4 + 255) & ~255
        return off + chains * n * 2 * d * d * 2 + chains * n_segs * 2 * d * d * 4
    off = ((chains * n * 2 * d * d + chains * n) * 4 + 255) & ~255
    return off + (chains * n * 64 * 4 if chunk == 64 else 0)


@scan_fwd_op.register_fake
def _(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, q_scale, chunk, y_layout):
    M, B, H, T = gamma.shape
    d = q_re.shape[-1]
    s = q_re.new_empty(M, B, H, d, d, dtype=torch.float32)
    nbytes = fwd_workspace_bytes(M, B, H, T, chunk, q_re.dtype == torch.bfloat16, d)
    ws = q_re.new_empty((nbytes + 3) // 4, dtype=torch.float32)
    if y_layout in (2, 3):
        yd = torch.bfloat16 if y_layout == 3 else torch.float32
        return [q_re.new_empty(B, T, 2, H, d, dtype=yd), q_re.new_empty(0, dtype=yd), s, torch.empty_like(s), ws]
    y = q_re.new_empty((B, T, H, d) if y_layout == 1 else (B, H, T, d), dtype=torch.float32)
    return [y, torch.empty_like(y), s, torch.empty_like(s), ws]


@torch.library.custom_op("qpam::scan_bwd", mutates_args=())
def scan_bwd_op(q_re: Tensor, q_im: Tensor, k_re: Tensor, k_im: Tensor, v_re: Tensor, v_im: Tensor,
                gamma: Tensor, rot_re: Optional[Tensor], rot_im: Optional[Tensor], s0_re: Optional[Tensor],
                s0_im: Optional[Tensor], q_scale: float, chunk: int, ws: Tensor, dy_re: Tensor, dy_im: Tensor,
                ds_re: Optional[Tensor], ds_im: Optional[Tensor], y_layout: int) -> List[Tensor]:
    """Returns [dq_re, dq_im, dk_re, dk_im, dv_re, dv_im, dgamma, drot_re, drot_im, ds0_re, ds0_im]
    (drot/ds0 are empty tensors when rot/s0 were not given); dy in y's layout."""
    M, B, H, T = gamma.shape
    d = q_re.shape[-1]
    dev = q_re.device
    # the kernels write dgamma and drot with the strides of gamma and rot: hand
    # them contiguous planes so those strides match the gradients allocated here
    gamma = gamma.contiguous()
    if rot_re is not None:
        rot_re, rot_im = rot_re.contiguous(), rot_im.contiguous()
    a, keep = _fill_args(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, q_scale, chunk)
    a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel() * 4
    bw = _lib.ScanBwdArgs()
    bw.fwd = _lib.ctypes.pointer(a)
    if y_layout in (2, 3):  # one [B,T,2,H,d] gradient in dy_re (bf16 for layout 3)
        dy = dy_re.contiguous()
        bw.dy_dtype = 1 if y_layout == 3 else 0
        dy_re, dy_im = dy[:, :, 0].transpose(1, 2), dy[:, :, 1].transpose(1, 2)
    else:
        dy_re, dy_im = dy_re.contiguous(), dy_im.contiguous()
        if y_layout == 1:
            dy_re, dy_im = dy_re.transpose(1, 2), dy_im.transpose(1, 2)
    bw.dy, _, _ = _cview(dy_re, dy_im)
    if ds_re is not None:
        ds_re, ds_im = ds_re.contiguous(), ds_im.contiguous()
        bw.ds_re, bw.ds_im = ds_re.data_ptr(), ds_im.data_ptr()
    outs = [torch.empty(B, H, T, d, device=dev, dtype=q_re.dtype) for _ in range(6)]
    bw.dq = _mview(outs[0], outs[1])
    bw.dk = _mview(outs[2], outs[3])
    bw.dv = _mview(outs[4], outs[5])
    dgamma = torch.empty(M, B, H, T, device=dev, dtype=torch.float32)
    bw.dgamma = dgamma.data_ptr()
    if rot_re is not None:
        drot_re = torch.empty(M, B, H, T, device=dev, dtype=torch.float32)
        drot_im = torch.empty_like(drot_re)
        bw.drot_re, bw.drot_im = drot_re.data_ptr(), drot_im.data_ptr()
    else:
        drot_re, drot_im = torch.empty(0, device=dev), torch.empty(0, device=dev)
    if s0_re is not None:
        ds0_re = torch.empty(M, B, H, d, d, device=dev, dtype=torch.float32)
        ds0_im = torch.empty_like(ds0_re)
        bw.ds0_re, bw.ds0_im = ds0_re.data_ptr(), ds0_im.data_ptr()
    else:
        ds0_re, ds0_im = torch.empty(0, device=dev), torch.empty(0, device=dev)
    L = _lib.lib()
    nbytes = L.qpam_scan_bwd_workspace_size(bw)
    ws2 = torch.empty((nbytes + 3) // 4 + 1, device=dev, dtype=torch.float32)
    bw.workspace, bw.workspace_bytes = ws2.data_ptr(), ws2.numel() * 4
    with torch.cuda.device(dev):
        _lib.check(L.qpam_scan_bwd(bw, _lib.stream_ptr(dev)), "qpam_scan_bwd")
    del keep
    return outs + [dgamma, drot_re, drot_im, ds0_re, ds0_im]


@scan_bwd_op.register_fake
def _(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, q_scale, chunk, ws, dy_re,
      dy_im, ds_re, ds_im, y_layout):
    M, B, H, T = gamma.shape
    d = q_re.shape[-1]
    outs = [q_re.new_empty(B, H, T, d) for _ in range(6)]
    dg = gamma.new_empty(M, B, H, T)
    dr = [gamma.new_empty(M, B, H, T) if rot_re is not None else gamma.new_empty(0) for _ in range(2)]
    d0 = [gamma.new_empty(M, B, H, d, d) if s0_re is not None else gamma.new_empty(0) for _ in range(2)]
    return outs + [dg] + dr + d0


def _setup_context(ctx, inputs, output):
    (q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, q_scale, chunk, y_layout) = inputs
    ctx.save_for_backward(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, output[4])
    ctx.q_scale, ctx.chunk, ctx.y_layout = q_scale, chunk, y_layout
    # outputs without an incoming gradient arrive as None (the workspace output
    # never has one): no zero-filled gradient buffers
    ctx.set_materialize_grads(False)


def _backward(ctx, grads):
    (q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, ws) = ctx.saved_tensors
    dy_re, dy_im, ds_re, ds_im = grads[0], grads[1], grads[2], grads[3]
    B, H, T, d = q_re.shape
    if ctx.y_layout in (2, 3):
        if dy_re is None:
            dy_re = q_re.new_zeros((B, T, 2, H, d), dtype=torch.bfloat16 if ctx.y_layout == 3 else torch.float32)
        dy_im = dy_re
    else:
        yshape = (B, T, H, d) if ctx.y_layout == 1 else (B, H, T, d)
        if dy_re is None:
            dy_re = q_re.new_zeros(yshape, dtype=torch.float32)
        if dy_im is None:
            dy_im = q_re.new_zeros(yshape, dtype=torch.float32)
    if ds_re is None and ds_im is None:
        ds_re_t = ds_im_t = None
    else:
        ds_re_t = ds_re if ds_re is not None else torch.zeros_like(ds_im)
        ds_im_t = ds_im if ds_im is not None else torch.zeros_like(ds_re)
    g = scan_bwd_op(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im, ctx.q_scale,
                    ctx.chunk, ws, dy_re, dy_im, ds_re_t, ds_im_t, ctx.y_layout)
    drot = (g[7], g[8]) if rot_re is not None else (None, None)
    ds0 = (g[9], g[10]) if s0_re is not None else (None, None)
    return (g[0], g[1], g[2], g[3], g[4], g[5], g[6], drot[0], drot[1], ds0[0], ds0[1], None, None, None)


scan_fwd_op.register_autograd(_backward, setup_context=_setup_context)


MAX_STATES = 4  # states one kernel call carries (the E3 kernels are built for M = 1..4)


def pam_scan_planar(q_re, q_im, k_re, k_im, v_re, v_im, gamma, *, q_scale, chunk=64, rot=None, s0=None,
                    y_layout="bhtd"):
    """Differentiable planar scan.  Returns (y_re, y_im, s_re, s_im); y is
    [B,H,T,d], or [B,T,H,d] with y_layout="bthd", or with y_layout="bt2hd"
    one tensor [B,T,2,H,d] returned as y_re (y_im None): the kernel writes y
    in that layout and reads its gradient in it, no transposes.
    y_layout="bt2hd_bf16" is the same tensor in bf16 (bf16 q, k, v and chunk
    64): y is rounded once from the fp32 result and the gradient is read in
    bf16, which equals rounding an fp32 y afterwards and widening a bf16 dy.

    Any head dim and state count (the reference's layer takes any, v11/model.py:45-97):
      * d < 64 is zero-padded to 64 and sliced back (exact: padded key/query
        columns add nothing to q.k*, padded value rows stay zero);
      * d > 64 is padded to a multiple of 64 and split into 64 x 64 blocks of
        the state: block (i, j) (value rows 64 i.., key columns 64 j..) evolves
        on its own, S_ij <- gamma S_ij + v_i (x) conj(k_j), and y_i = sum_j S_ij q_j,
        so the blocks run as n^2 heads of the d = 64 kernels and y sums over j;
      * more than 4 states run in groups of at most 4 (Y is the sum of the
        states' reads, the states are independent chains)."""
    layouts = {"bhtd": 0, "bthd": 1, "bt2hd": 2, "bt2hd_bf16": 3}
    if y_layout not in layouts:
        raise ValueError(f"y_layout must be one of {list(layouts)}")
    if y_layout == "bt2hd_bf16" and (q_re.dtype != torch.bfloat16 or chunk != 64):
        raise ValueError("y_layout 'bt2hd_bf16' needs bf16 q, k, v and chunk 64")
    if gamma.dim() == 4 and gamma.shape[0] > MAX_STATES:
        return _scan_state_groups(q_re, q_im, k_re, k_im, v_re, v_im, gamma, q_scale, chunk, rot, s0, y_layout)
    if q_re.shape[-1] > 64:
        return _scan_blocks(q_re, q_im, k_re, k_im, v_re, v_im, gamma, q_scale, chunk, rot, s0, y_layout)
    rot_re, rot_im = rot if rot is not None else (None, None)
    s0_re, s0_im = s0 if s0 is not None else (None, None)
    d = q_re.shape[-1]
    if d < 64 and y_layout in ("bt2hd", "bt2hd_bf16"):
        y_re, y_im, s_re, s_im = pam_scan_planar(q_re, q_im, k_re, k_im, v_re, v_im, gamma, q_scale=q_scale,
                                                 chunk=chunk, rot=rot, s0=s0)
        return _to_bt2hd(y_re, y_im, y_layout), None, s_re, s_im
    if d < 64:
        pad = 64 - d
        q_re, q_im, k_re, k_im, v_re, v_im = (torch.nn.functional.pad(x, (0, pad))
                                              for x in (q_re, q_im, k_re, k_im, v_re, v_im))
        if s0_re is not None:
            s0_re, s0_im = (torch.nn.functional.pad(x, (0, pad, 0, pad)) for x in (s0_re, s0_im))
    out = scan_fwd_op(q_re, q_im, k_re, k_im, v_re, v_im, gamma, rot_re, rot_im, s0_re, s0_im,
                      float(q_scale), int(chunk), layouts[y_layout])
    y_re, y_im, s_re, s_im = out[0], out[1], out[2], out[3]
    if y_layout in ("bt2hd", "bt2hd_bf16"):
        return y_re, None, s_re, s_im
    if d < 64:
        y_re, y_im = y_re[..., :d], y_im[..., :d]
        s_re, s_im = s_re[..., :d, :d], s_im[..., :d, :d]
    return y_re, y_im, s_re, s_im


def _to_bt2hd(y_re, y_im, y_layout):
    """[B,H,T,d] planes -> one [B,T,2,H,d] tensor (bf16 for 'bt2hd_bf16')."""
    y = torch.stack([y_re.transpose(1, 2), y_im.transpose(1, 2)], dim=2)
    return y.to(torch.bfloat16) if y_layout == "bt2hd_bf16" else y


def _scan_state_groups(q_re, q_im, k_re, k_im, v_re, v_im, gamma, q_scale, chunk, rot, s0, y_layout):
    """More than MAX_STATES states: near-equal groups of at most MAX_STATES,
    one scan each; Y is summed over the groups (in fp32, rounded once for the
    bf16 layout) and the final states are concatenated."""
    M = gamma.shape[0]
    n_groups = -(-M // MAX_STATES)
    bounds = [round(i * M / n_groups) for i in range(n_groups + 1)]
    layout = "bt2hd" if y_layout == "bt2hd_bf16" else y_layout
    y_re = y_im = None
    s_re, s_im = [], []
    for m0, m1 in zip(bounds[:-1], bounds[1:]):
        rot_g = (rot[0][m0:m1], rot[1][m0:m1]) if rot is not None else None
        s0_g = (s0[0][m0:m1], s0[1][m0:m1]) if s0 is not None else None
        yr, yi, sr, si = pam_scan_planar(q_re, q_im, k_re, k_im, v_re, v_im, gamma[m0:m1], q_scale=q_scale,
                                         chunk=chunk, rot=rot_g, s0=s0_g, y_layout=layout)
        y_re = yr if y_re is None else y_re + yr
        if yi is not None:
            y_im = yi if y_im is None else y_im + yi
        s_re.append(sr)
        s_im.append(si)
    if y_layout == "bt2hd_bf16":
        y_re = y_re.to(torch.bfloat16)
    return y_re, y_im, torch.cat(s_re, 0), torch.cat(s_im, 0)


def _scan_blocks(q_re, q_im, k_re, k_im, v_re, v_im, gamma, q_scale, chunk, rot, s0, y_layout):
    """Head dim d > 64: d is zero-padded to 64 n and the d x d state splits into
    n x n blocks of 64 x 64, each an independent chain with the head's decay:
    block (i, j) reads value block i and key/query block j, and y_i = sum_j of
    the blocks' reads.  The n^2 blocks of every head run as extra heads of one
    d = 64 scan (q and k repeated over i, v over j, gamma and rot over both)."""
    B, H, T, d = q_re.shape
    M = gamma.shape[0]
    n = -(-d // 64)
    dp = 64 * n

    def padded(x):
        return torch.nn.functional.pad(x, (0, dp - d)) if dp != d else x

    def key_side(x):  # [B,H,T,d] -> [B, H n n, T, 64], entry (i, j) = column block j
        xb = padded(x).reshape(B, H, T, n, 64).permute(0, 1, 3, 2, 4)
        return xb.unsqueeze(2).expand(B, H, n, n, T, 64).reshape(B, H * n * n, T, 64)

    def value_side(x):  # entry (i, j) = column block i
        xb = padded(x).reshape(B, H, T, n, 64).permute(0, 1, 3, 2, 4)
        return xb.unsqueeze(3).expand(B, H, n, n, T, 64).reshape(B, H * n * n, T, 64)

    def per_block(x):  # [M,B,H,T] -> [M, B, H n n, T]
        return x.unsqueeze(3).expand(M, B, H, n * n, T).reshape(M, B, H * n * n, T)

    def state_blocks(x):  # [M,B,H,d,d] -> [M, B, H n n, 64, 64]
        if dp != d:
            x = torch.nn.functional.pad(x, (0, dp - d, 0, dp - d))
        return x.reshape(M, B, H, n, 64, n, 64).permute(0, 1, 2, 3, 5, 4, 6).reshape(M, B, H * n * n, 64, 64)

    rot_b = (per_block(rot[0]), per_block(rot[1])) if rot is not None else None
    s0_b = (state_blocks(s0[0]), state_blocks(s0[1])) if s0 is not None else None
    y_re, y_im, s_re, s_im = pam_scan_planar(
        key_side(q_re), key_side(q_im), key_side(k_re), key_side(k_im), value_side(v_re), value_side(v_im),
        per_block(gamma), q_scale=q_scale, chunk=chunk, rot=rot_b, s0=s0_b)

    def gather_y(y):  # [B, H n n, T, 64] -> [B,H,T,d]
        y = y.view(B, H, n, n, T, 64).sum(3)
        return y.permute(0, 1, 3, 2, 4).reshape(B, H, T, dp)[..., :d]

    def gather_s(s):  # [M, B, H n n, 64, 64] -> [M,B,H,d,d]
        s = s.view(M, B, H, n, n, 64, 64).permute(0, 1, 2, 3, 5, 4, 6).reshape(M, B, H, dp, dp)
        return s[..., :d, :d]

    y_re, y_im, s_re, s_im = gather_y(y_re), gather_y(y_im), gather_s(s_re), gather_s(s_im)
    if y_layout == "bthd":
        return y_re.transpose(1, 2), y_im.transpose(1, 2), s_re, s_im
    if y_layout in ("bt2hd", "bt2hd_bf16"):
        return _to_bt2hd(y_re, y_im, y_layout), None, s_re, s_im
    return y_re, y_im, s_re, s_im


def _planes(z):
    return z[..., 0], z[..., 1]


def pam_scan_interleaved(queries, keys, values, gamma_all, head_dim, chunk_size, *, rot=None, s0=None,
                         scale_queries=True):
    """Split-real [..., d, 2] front end: queries/keys/values [B,H,T,d,2],
    gamma_all [M,B,H,T]; rot optional (re, im) planes [M,B,H,T]; s0 optional
    [M,B,H,d,d,2].  Returns (Y [B,H,T,d,2], S [M,B,H,d,d,2]) in the input dtype."""
    dtype = queries.dtype
    work = torch.bfloat16 if dtype == torch.bfloat16 else torch.float32
    qr, qi = (x.to(work) for x in _planes(queries))
    kr, ki = (x.to(work) for x in _planes(keys))
    vr, vi = (x.to(work) for x in _planes(values))
    s0p = None
    if s0 is not None:
        s0p = (s0[..., 0].float(), s0[..., 1].float())
    rotp = (rot[0].float(), rot[1].float()) if rot is not None else None
    t = queries.shape[2]
    y_re, y_im, s_re, s_im = pam_scan_planar(
        qr, qi, kr, ki, vr, vi, gamma_all.float(), q_scale=head_dim ** -0.5 if scale_queries else 1.0,
        chunk=chunk_for(chunk_size, t), rot=rotp, s0=s0p)
    y = torch.stack([y_re, y_im], dim=-1).to(dtype)
    s = torch.stack([s_re, s_im], dim=-1).to(dtype)
    return y, s
