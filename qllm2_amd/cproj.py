"""The PAM layer's complex projections as single real GEMMs over a packed
weight, with the packing and the weight-gradient split on the HIP library
(qpam_cweight_pack / qpam_cweight_unpack).

ComplexLinear (v11/complex_ops.py:146-172) computes re = Wr xr - Wi xi and
im = Wi xr + Wr xi.  The layer's fused forward runs its input projection
(qkv_proj plus dt_proj's logits, v11/model.py:280, 636) as one GEMM from x
viewed as [N, 2 dim] (re, im per feature) and its output projection (o_proj,
v11/model.py:836) as one GEMM from the scan's [N, 2 H d] planes to the
interleaved output.  Each needs the weights rearranged into one real matrix
W; built from torch passes, that took five to seven small launches per
projection forward and as many backward.  Here:

  * linear_in:  proj [N, cols] = x2 W^T with W in layout QPAM_CW_IN
    (W[p R + r][2c + q], then dt_proj's rows, then zero rows up to `cols`);
    backward: gx = g W, gW = g^T x2 (one GEMM), split by one unpack launch;
  * linear_out: out [N, 2 dim] = y2 W^T with W in layout QPAM_CW_OUT
    (W[2r + p][q C + c]); backward: gx = g W, the weight gradient as a
    batched product over row slices of N (the library GEMM sees few output
    tiles for a K of N otherwise) whose slices the unpack launch sums in fp32
    in slice order.

The weight gradients are formed in fp32 from the bf16 (or fp32) GEMM outputs
and rounded once to the weights' dtype.  linear_in can also return cabs(x)
(the gates' input, v11/model.py:228, 646) and then adds the gradient that
comes back through it into x's gradient in the same pass as the projection's
(qpam_cabs_bwd_acc), instead of a separate gradient and a sum.  gate_linear
runs the gate projections over |x| (protect_gate and phase_proj stacked) with
their weight gradient reduced over row slices and cast by one launch
(qpam_slice_sum) and their bias gradient as one product with a ones row.
"""

import ctypes

import torch
import torch.nn.functional as F

from . import _lib


def _code(t):
    if t.dtype == torch.float32:
        return _lib.QPAM_F32
    if t.dtype == torch.bfloat16:
        return _lib.QPAM_BF16
    raise ValueError(f"qpam complex projection: dtype {t.dtype} is not supported (fp32 or bf16)")


def _aligned(*ts):
    return all(t is None or (t.is_contiguous() and t.data_ptr() % 16 == 0) for t in ts)


def supported(x2, wr, wi, tail=None, layout=_lib.QPAM_CW_IN):
    """Whether the packed path applies: GPU tensors of one dtype (fp32 or
    bf16), contiguous 16-byte aligned weights, feature counts the kernels'
    vector width divides, no autocast."""
    ts = [x2, wr, wi] + ([tail] if tail is not None else [])
    if not all(t.is_cuda and t.dtype == x2.dtype for t in ts) or x2.dtype not in (torch.float32, torch.bfloat16):
        return False
    if torch.is_autocast_enabled() or not _aligned(wr, wi, tail):
        return False
    C = wr.shape[1]
    return C % (4 if layout == _lib.QPAM_CW_IN else 8) == 0 and wr.shape == wi.shape


def _args(layout, wr, wi, tail, zero_rows, ldw):
    a = _lib.CWeightArgs()
    a.dtype, a.layout = _code(wr), layout
    a.R, a.C = wr.shape
    a.wr, a.wi = wr.data_ptr(), wi.data_ptr()
    if tail is not None:
        a.tail, a.tail_rows = tail.data_ptr(), tail.shape[0]
    a.zero_rows, a.ldw = zero_rows, ldw
    return a


def _pack(layout, wr, wi, tail=None, rows=None):
    R, C = wr.shape
    tail_rows = tail.shape[0] if tail is not None else 0
    rows = rows if rows is not None else 2 * R + tail_rows
    w = torch.empty(rows, 2 * C, device=wr.device, dtype=wr.dtype)
    a = _args(layout, wr, wi, tail, rows - 2 * R - tail_rows, 2 * C)
    a.w = w.data_ptr()
    with torch.cuda.device(wr.device):
        _lib.check(_lib.lib().qpam_cweight_pack(ctypes.byref(a), _lib.stream_ptr(wr.device)), "qpam_cweight_pack")
    return w


def _unpack(layout, g, slices, wr, wi, tail, rows):
    R, C = wr.shape
    tail_rows = tail.shape[0] if tail is not None else 0
    g_wr, g_wi = torch.empty_like(wr), torch.empty_like(wi)
    g_tail = torch.empty_like(tail) if tail is not None else None
    a = _args(layout, wr, wi, tail, rows - 2 * R - tail_rows, 2 * C)
    a.g, a.g_dtype, a.slices, a.slice_stride = g.data_ptr(), _code(g), slices, rows * 2 * C
    a.g_wr, a.g_wi = g_wr.data_ptr(), g_wi.data_ptr()
    if tail is not None:
        a.g_tail = g_tail.data_ptr()
    with torch.cuda.device(wr.device):
        _lib.check(_lib.lib().qpam_cweight_unpack(ctypes.byref(a), _lib.stream_ptr(wr.device)), "qpam_cweight_unpack")
    return g_wr, g_wi, g_tail


def _cabs(x2):
    """|z| per complex feature of x2 [..., 2C] (qpam_cabs_fwd, cabs of
    v11/complex_ops.py:86-87) -> [..., C] in x2's dtype."""
    mag = torch.empty(x2.shape[:-1] + (x2.shape[-1] // 2,), device=x2.device, dtype=x2.dtype)
    with torch.cuda.device(x2.device):
        _lib.check(_lib.lib().qpam_cabs_fwd(_code(x2), mag.numel(), x2.data_ptr(), mag.data_ptr(),
                                            _lib.stream_ptr(x2.device)), "qpam_cabs_fwd")
    return mag


class _LinearIn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x2, wr, wi, tail, cols, with_mag):
        w = _pack(_lib.QPAM_CW_IN, wr, wi, tail, cols)
        out = F.linear(x2, w)
        mag = _cabs(x2) if with_mag else x2.new_empty(0)
        ctx.save_for_backward(x2, w, wr, wi, tail, mag if with_mag else None)
        if not with_mag:
            ctx.mark_non_differentiable(mag)
        return out, mag

    @staticmethod
    def backward(ctx, g, g_mag):
        x2, w, wr, wi, tail, mag = ctx.saved_tensors
        g2 = g.reshape(-1, w.shape[0])
        if not g2.is_contiguous():
            g2 = g2.contiguous()
        gx = None
        if ctx.needs_input_grad[0]:
            gx = (g2 @ w).view(x2.shape)
            if mag is not None and g_mag is not None:
                # the gradient through |x| added into the projections' in one pass
                gm = g_mag.to(mag.dtype).contiguous()
                with torch.cuda.device(x2.device):
                    _lib.check(_lib.lib().qpam_cabs_bwd_acc(_code(x2), mag.numel(), x2.data_ptr(), mag.data_ptr(),
                                                            gm.data_ptr(), gx.data_ptr(),
                                                            _lib.stream_ptr(x2.device)), "qpam_cabs_bwd_acc")
        g_wr = g_wi = g_tail = None
        if any(ctx.needs_input_grad[1:4]):
            gw = g2.t() @ x2.reshape(-1, w.shape[1])                  # [cols, 2 dim]
            g_wr, g_wi, g_tail = _unpack(_lib.QPAM_CW_IN, gw, 1, wr, wi, tail, w.shape[0])
        return gx, g_wr, g_wi, g_tail, None, None


def linear_in(x2, wr, wi, tail, cols, with_mag=False):
    """x2 [..., 2C] (features interleaved (re, im)), complex weights wr, wi
    [R, C], tail [Tr, 2C] real rows over [xr | xi] (or None) -> [..., cols]:
    columns [0, R) the real outputs, [R, 2R) the imaginary outputs, then the
    tail's outputs, then zeros.  with_mag also returns |x| [..., C] (cabs) and
    adds its gradient into x's own in the backward: (proj, mag)."""
    out, mag = _LinearIn.apply(x2, wr, wi, tail, int(cols), bool(with_mag))
    return (out, mag) if with_mag else out


def _splits(n, out, inp):
    """Row slices of N for a weight gradient with out x in outputs: enough for
    512 output tiles of 128 x 128, each slice at least 512 rows."""
    tiles = -(-out // 128) * -(-inp // 128)
    s = 1
    while s * tiles < 512 and n % (2 * s) == 0 and n // (2 * s) >= 512:
        s *= 2
    return s


class _LinearOut(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y2, wr, wi):
        w = _pack(_lib.QPAM_CW_OUT, wr, wi)
        ctx.save_for_backward(y2, w, wr, wi)
        return F.linear(y2, w)

    @staticmethod
    def backward(ctx, g):
        y2, w, wr, wi = ctx.saved_tensors
        out, inp = w.shape
        g2 = g.reshape(-1, out)
        if not g2.is_contiguous():
            g2 = g2.contiguous()
        gx = (g2 @ w).view(y2.shape) if ctx.needs_input_grad[0] else None
        g_wr = g_wi = None
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            n = g2.shape[0]
            s = _splits(n, out, inp)
            y2f = y2.reshape(n, inp)
            # g^T y per row slice: [S, out, in]; the right operand is a contiguous slice
            gws = torch.bmm(g2.view(s, n // s, out).transpose(1, 2), y2f.view(s, n // s, inp))
            g_wr, g_wi, _ = _unpack(_lib.QPAM_CW_OUT, gws, s, wr, wi, None, out)
        return gx, g_wr, g_wi


def linear_out(y2, wr, wi):
    """y2 [..., 2C] (a real then an imaginary block of C features), complex
    weights wr, wi [R, C] -> [..., 2R] with the outputs interleaved (re, im)."""
    return _LinearOut.apply(y2, wr, wi)


_ONES = {}


def _ones_row(n, like):
    key = (n, like.device, like.dtype)
    t = _ONES.get(key)
    if t is None:
        if len(_ONES) > 16:
            _ONES.clear()
        t = _ONES[key] = torch.ones(1, n, device=like.device, dtype=like.dtype)
    return t


class _GateLinear(torch.autograd.Function):
    """F.linear over the gate rows of several nn.Linear stacked: the weight
    gradient as a batched product over row slices of N summed and cast by one
    launch (qpam_slice_sum), the bias gradient as one product with a ones row."""

    @staticmethod
    def forward(ctx, x, n_parts, *params):
        ws, bs = params[:n_parts], params[n_parts:]
        w = torch.cat(ws, 0) if n_parts > 1 else ws[0]
        b = torch.cat(bs, 0) if n_parts > 1 else bs[0]
        ctx.save_for_backward(x, w)
        ctx.rows = [t.shape[0] for t in ws]
        ctx.b_dtype = b.dtype
        return F.linear(x, w, b)

    @staticmethod
    def backward(ctx, g):
        x, w = ctx.saved_tensors
        out, inp = w.shape
        g2 = g.reshape(-1, out)
        if not g2.is_contiguous():
            g2 = g2.contiguous()
        n = g2.shape[0]
        gx = (g2 @ w).view(x.shape) if ctx.needs_input_grad[0] else None
        x2 = x.reshape(n, inp)
        s = _splits(n, out, inp)
        gws = torch.bmm(g2.view(s, n // s, out).transpose(1, 2), x2.view(s, n // s, inp))   # [S, out, in]
        gw = torch.empty(out, inp, device=w.device, dtype=w.dtype)
        with torch.cuda.device(w.device):
            _lib.check(_lib.lib().qpam_slice_sum(_code(gws), _code(gw), s, out * inp, out * inp, gws.data_ptr(),
                                                 gw.data_ptr(), _lib.stream_ptr(w.device)), "qpam_slice_sum")
        gb = (_ones_row(n, g2) @ g2).view(out).to(ctx.b_dtype)
        gws_parts = list(torch.split(gw, ctx.rows, 0))
        gbs_parts = list(torch.split(gb, ctx.rows, 0))
        return (gx, None, *gws_parts, *gbs_parts)


def gate_supported(x, weights, biases):
    """The gate path applies: biases present, one dtype (fp32 or bf16) for x,
    weights and biases, feature counts the slice-sum vector width divides."""
    ts = [x] + list(weights) + list(biases)
    if any(t is None for t in biases) or torch.is_autocast_enabled():
        return False
    if not all(t.is_cuda and t.dtype == x.dtype for t in ts) or x.dtype not in (torch.float32, torch.bfloat16):
        return False
    return (sum(w.shape[0] for w in weights) * x.shape[-1]) % 8 == 0


def gate_linear(x, weights, biases):
    """F.linear(x, cat(weights), cat(biases)) with the weight gradients formed
    by a sliced product reduced in one launch (see _GateLinear)."""
    return _GateLinear.apply(x, len(weights), *weights, *biases)
