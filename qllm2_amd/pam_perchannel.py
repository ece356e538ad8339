"""E1 per-channel decay on the GPU: V11PAMLayer._forward_chunked_perchannel
(v11/model.py:421-489) with the reference's signature and return tuple.

Per chunk of `chunk` steps the reference folds the decay into the operands
(L = max(cumsum(log max(gamma, 1e-6)), -30) per key channel): queries carry
e^{L} q_scale, keys e^{-L}, the state-write keys e^{L_last - L}, and the state
decays column j by e^{L_last[j]}.  Here:

  * the fold runs in one HIP kernel over all chunks at once (qpam_pc_fold_fwd;
    its backward, qpam_pc_fold_bwd, forms dq, dk and dgamma through both
    clamps);
  * the chunk-parallel products -- the masked score Q K^H, its read of V, the
    chunk's state increment V^T conj(W) and the carried read Q S^T -- are
    batched complex GEMMs over every (b, h, chunk) at once (the library GEMM,
    fp32 complex);
  * the state entering each chunk comes from the per-column decayed scan over
    the chunks (qpam_pc_scan; backward: the same kernel in reverse).

Autograd runs through the GEMMs and the two custom functions, so the layer's
training forward has gradients for q, k, v and gamma.  The whole computation
is fp32 (the reference computes in the input dtype); outputs are cast back to
the input dtype.
"""

import ctypes

import torch

from . import _lib

_MASKS = {}


def _mask(c, device):
    key = (c, device)
    m = _MASKS.get(key)
    if m is None:
        m = torch.tril(torch.ones(c, c, device=device, dtype=torch.float32))
        _MASKS[key] = m
    return m


def _dt(t):
    if t.dtype == torch.float32:
        return _lib.QPAM_F32
    if t.dtype == torch.bfloat16:
        return _lib.QPAM_BF16
    raise ValueError(f"qpam per-channel scan: dtype {t.dtype} is not supported (fp32 or bf16)")


def _pairs(x):
    """x [..., d, 2] with the last two dims contiguous (a copy otherwise)."""
    return x if (x.stride(-1) == 1 and x.stride(-2) == 2) else x.contiguous()


def _ptr(t):
    return t.data_ptr() if t is not None else None


class _Fold(torch.autograd.Function):
    """(q, k [B,H,T,d,2], gamma [B,H,T,d]) -> qf, kf, wf [B*H, n, C, d, 2] fp32
    and atot [B*H, n, d]: the folded operands of every chunk."""

    @staticmethod
    def forward(ctx, q, k, gamma, chunk, q_scale):
        if q.dim() != 5 or q.shape[-1] != 2 or k.shape != q.shape or gamma.shape != q.shape[:4]:
            raise ValueError(f"qpam per-channel fold: q, k [B,H,T,d,2] and gamma [B,H,T,d] expected, got "
                             f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(gamma.shape)}")
        q, k = _pairs(q), _pairs(k.to(q.dtype))
        gamma = gamma if gamma.stride(-1) == 1 else gamma.contiguous()
        B, H, T, d = q.shape[:4]
        n = -(-T // chunk)
        dev = q.device
        qf, kf, wf = (torch.empty(B * H, n, chunk, d, 2, device=dev, dtype=torch.float32) for _ in range(3))
        atot = torch.empty(B * H, n, d, device=dev, dtype=torch.float32)
        a = _Fold._args(q, k, gamma, chunk, q_scale)
        a.qf, a.kf, a.wf, a.atot = qf.data_ptr(), kf.data_ptr(), wf.data_ptr(), atot.data_ptr()
        with torch.cuda.device(dev):
            _lib.check(_lib.lib().qpam_pc_fold_fwd(ctypes.byref(a), _lib.stream_ptr(dev)), "qpam_pc_fold_fwd")
        ctx.save_for_backward(q, k, gamma)
        ctx.chunk, ctx.q_scale = chunk, q_scale
        return qf, kf, wf, atot

    @staticmethod
    def _args(q, k, gamma, chunk, q_scale):
        B, H, T, d = q.shape[:4]
        a = _lib.PcFoldArgs()
        a.dtype, a.g_dtype = _dt(q), _dt(gamma)
        a.B, a.H, a.T, a.d = B, H, T, d
        a.chunk, a.q_scale = int(chunk), float(q_scale)
        a.q, a.k, a.gamma = q.data_ptr(), k.data_ptr(), gamma.data_ptr()
        a.q_sb, a.q_sh, a.q_st = q.stride(0), q.stride(1), q.stride(2)
        a.k_sb, a.k_sh, a.k_st = k.stride(0), k.stride(1), k.stride(2)
        a.g_sb, a.g_sh, a.g_st = gamma.stride(0), gamma.stride(1), gamma.stride(2)
        return a

    @staticmethod
    def backward(ctx, dqf, dkf, dwf, datot):
        q, k, gamma = ctx.saved_tensors
        dq, dk = torch.empty(q.shape, device=q.device, dtype=q.dtype), torch.empty(k.shape, device=k.device,
                                                                                     dtype=q.dtype)
        dgamma = torch.empty(gamma.shape, device=gamma.device, dtype=gamma.dtype)
        grads = [g.contiguous() if g is not None else None for g in (dqf, dkf, dwf, datot)]
        a = _Fold._args(q, k, gamma, ctx.chunk, ctx.q_scale)
        a.dqf, a.dkf, a.dwf, a.datot = (_ptr(g) for g in grads)
        a.dq, a.dk, a.dgamma = dq.data_ptr(), dk.data_ptr(), dgamma.data_ptr()
        with torch.cuda.device(q.device):
            _lib.check(_lib.lib().qpam_pc_fold_bwd(ctypes.byref(a), _lib.stream_ptr(q.device)), "qpam_pc_fold_bwd")
        return dq, dk, dgamma, None, None


def _scan(x, a, out, init, fin, reverse):
    N, n, d = a.shape
    s = _lib.PcScanArgs()
    s.N, s.n, s.d = N, n, d
    s.x, s.a, s.out, s.init, s.fin = x.data_ptr(), a.data_ptr(), out.data_ptr(), _ptr(init), _ptr(fin)
    s.reverse = 1 if reverse else 0
    with torch.cuda.device(x.device):
        _lib.check(_lib.lib().qpam_pc_scan(ctypes.byref(s), _lib.stream_ptr(x.device)), "qpam_pc_scan")


class _Scan(torch.autograd.Function):
    """(x [N,n,d,d,2] chunk increments, a [N,n,d] column decays) -> (state
    entering each chunk [N,n,d,d,2], final state [N,d,d,2])."""

    @staticmethod
    def forward(ctx, x, a):
        if a.dim() != 3 or x.shape != (*a.shape, a.shape[2], 2):
            raise ValueError(f"qpam per-channel scan: x [N,n,d,d,2] and a [N,n,d] expected, got "
                             f"{tuple(x.shape)}, {tuple(a.shape)}")
        x, a = x.contiguous(), a.contiguous()
        N, n, d = a.shape
        out = torch.empty_like(x)
        fin = torch.empty(N, d, d, 2, device=x.device, dtype=torch.float32)
        _scan(x, a, out, None, fin, False)
        ctx.save_for_backward(a, out)
        return out, fin

    @staticmethod
    def backward(ctx, dout, dfin):
        a, out = ctx.saved_tensors
        dout = dout.contiguous() if dout is not None else torch.zeros_like(out)
        dfin = dfin.contiguous() if dfin is not None else None
        dx = torch.empty_like(out)
        _scan(dout, a, dx, dfin, None, True)
        # d a[c][j] = sum_i Re(conj(S_in[c][i][j]) dx[c][i][j])
        da = (out * dx).sum(-1).sum(-2)
        return dx, da


def perchannel_chunked(queries, keys, protected_values, decay_gamma, head_dim, chunk_size):
    """V11PAMLayer._forward_chunked_perchannel (v11/model.py:421-489):
    queries, keys, protected_values [B,H,T,d,2], decay_gamma [B,H,T,d] (CUDA,
    fp32 or bf16) -> (y [B,H,T,d,2], final state [B,H,d,d,2]) in the input
    dtype; differentiable in all four inputs."""
    if not queries.is_cuda:
        raise ValueError("qpam per-channel scan: tensors must be on the GPU (no CPU path in this library)")
    B, H, T, d = queries.shape[:4]
    C = int(chunk_size)
    if not 1 <= C <= 64:
        raise ValueError(f"qpam per-channel scan: chunk_size {C} outside 1..64")
    n = -(-T // C)
    qf, kf, wf, atot = _Fold.apply(queries, keys, decay_gamma, C, head_dim ** -0.5)
    Q, K, W = (torch.view_as_complex(t) for t in (qf, kf, wf))   # [N, n, C, d]
    v = protected_values.float()
    if n * C != T:
        v = torch.nn.functional.pad(v, (0, 0, 0, 0, 0, n * C - T))
    V = torch.view_as_complex(v.reshape(B * H, n, C, d, 2).contiguous())
    # the right operands of the products as contiguous tensors
    P = (Q @ K.conj().transpose(-1, -2).contiguous()) * _mask(C, queries.device)   # masked score [N,n,C,C]
    Y = P @ V
    dS = V.transpose(-1, -2).contiguous() @ W.conj().resolve_conj()                # sum_s v_s[i] conj(w_s[j])
    s_in, s_fin = _Scan.apply(torch.view_as_real(dS), atot)
    Y = Y + Q @ torch.view_as_complex(s_in).transpose(-1, -2).contiguous()      # carried read q' S^T
    y = torch.view_as_real(Y).reshape(B, H, n * C, d, 2)[:, :, :T]
    return y.to(queries.dtype), s_fin.reshape(B, H, d, d, 2).to(queries.dtype)
