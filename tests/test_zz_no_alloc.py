"""GPU check of the allocation-free scan forward (qpam_scan_fwd_noalloc)
through the C ABI: on two calls in a row, the second with a smaller input,
its outputs equal qpam_scan_fwd's with a caller workspace bit for bit (the
same kernels on the same inputs), for the fp32 path and the bf16 E3 path; a
call whose states exceed the library's scratch is refused before any launch."""

import ctypes
import math

import pytest
import torch

from oracle import pam as O

pytestmark = pytest.mark.gpu


def _inputs(B, H, T, M, dtype, seed, rot, s0):
    q, k, v, gamma = O.make_scan_inputs(B, H, T, 64, seed, m_states=M, unit_qk=True, gamma_mu_step=1.0)
    dev = torch.device("cuda")
    planes = [x[..., i].contiguous().to(dtype).to(dev) for x in (q, k, v) for i in (0, 1)]
    g = torch.Generator().manual_seed(seed + 1)
    rr = ri = s0r = s0i = None
    if rot:
        ph = torch.rand(M, B, H, T, generator=g) * 2 * math.pi
        rr, ri = torch.cos(ph).to(dev), torch.sin(ph).to(dev)
    if s0:
        s0r, s0i = (torch.randn(M, B, H, 64, 64, generator=g).mul(0.05).to(dev) for _ in range(2))
    return planes, gamma.to(dev), rr, ri, s0r, s0i


def _run(entry, planes, gamma, rr, ri, s0r, s0i, chunk):
    from qllm2_amd import _lib
    from qllm2_amd.pam_scan import _fill_args, _mview
    M, B, H, T = gamma.shape
    a, keep = _fill_args(*planes, gamma, rr, ri, s0r, s0i, 0.125, chunk)
    y_re = torch.empty(B, H, T, 64, device="cuda")
    y_im = torch.empty_like(y_re)
    s_re = torch.empty(M, B, H, 64, 64, device="cuda")
    s_im = torch.empty_like(s_re)
    a.y = _mview(y_re, y_im)
    a.s_re, a.s_im = s_re.data_ptr(), s_im.data_ptr()
    L = _lib.lib()
    ws = None
    if entry == "qpam_scan_fwd":
        ws = torch.empty(L.qpam_scan_workspace_size(a), device="cuda", dtype=torch.uint8)
        a.workspace, a.workspace_bytes = ws.data_ptr(), ws.numel()
    else:
        assert L.qpam_scan_workspace_size(a) <= _lib.QPAM_SCAN_FWD_NOALLOC_MAX_BYTES
    _lib.check(getattr(L, entry)(ctypes.byref(a), _lib.stream_ptr()), entry)
    torch.cuda.synchronize()
    del keep, ws
    return y_re, y_im, s_re, s_im


CALLS = [  # (B, H, T, M, dtype, rot, s0, chunk): each pair runs large, then smaller
    [(2, 6, 1024, 3, torch.bfloat16, True, True, 64), (1, 3, 200, 1, torch.float32, False, False, 64)],
    [(2, 4, 777, 2, torch.float32, True, True, 64), (1, 2, 90, 2, torch.bfloat16, False, True, 64)],
    [(1, 12, 2048, 1, torch.float32, False, False, 64), (2, 2, 48, 1, torch.float32, False, False, 16)],
]


@pytest.mark.parametrize("calls", CALLS)
def test_noalloc_matches_workspace_entry(gpu_lib, calls):
    for i, (B, H, T, M, dtype, rot, s0, chunk) in enumerate(calls):
        print(f"call {i}: B={B} H={H} T={T} M={M} {dtype} rot={rot} s0={s0} C={chunk}", flush=True)
        args = _inputs(B, H, T, M, dtype, 300 + 10 * i + B + T, rot, s0)
        want = _run("qpam_scan_fwd", *args, chunk)
        got = _run("qpam_scan_fwd_noalloc", *args, chunk)
        for g, w in zip(got, want):
            assert torch.equal(g, w)


def test_noalloc_refuses_calls_beyond_its_scratch(gpu_lib):
    """fp32, one state, 12 heads, 12800 tokens: 2400 chunk states of 32 KiB
    (78.6 MB) exceed the 64 MiB scratch: QPAM_ERR_WORKSPACE, no launch."""
    from qllm2_amd import _lib
    from qllm2_amd.pam_scan import _fill_args, _mview
    B, H, T, M = 1, 12, 12800, 1
    planes = [torch.zeros(B, H, T, 64, device="cuda") for _ in range(6)]
    gamma = torch.full((M, B, H, T), 0.9, device="cuda")
    a, keep = _fill_args(*planes, gamma, None, None, None, None, 0.125, 64)
    y = torch.empty(B, H, T, 64, device="cuda")
    s = torch.empty(M, B, H, 64, 64, device="cuda")
    a.y = _mview(y, y)
    a.s_re, a.s_im = s.data_ptr(), s.data_ptr()
    L = _lib.lib()
    assert L.qpam_scan_workspace_size(a) > _lib.QPAM_SCAN_FWD_NOALLOC_MAX_BYTES
    st = L.qpam_scan_fwd_noalloc(ctypes.byref(a), _lib.stream_ptr())
    assert st == _lib.QPAM_ERR_WORKSPACE
    assert b"scratch" in L.qpam_last_error()


def test_noalloc_refuses_overlapping_call_on_another_stream(gpu_lib):
    """A call on stream A is held behind a bounded spin kernel; a call on stream
    B issued meanwhile would share the scratch with it and is refused
    (QPAM_ERR_ARG) with no launch; once A has finished, the same call on B runs
    and equals the workspace entry's result."""
    from qllm2_amd import _lib
    from qllm2_amd.pam_scan import _fill_args, _mview
    planes, gamma, rr, ri, s0r, s0i = _inputs(1, 4, 512, 1, torch.float32, 377, False, False)
    want = _run("qpam_scan_fwd", planes, gamma, rr, ri, s0r, s0i, 64)
    L = _lib.lib()
    M, B, H, T = gamma.shape

    def args():
        a, keep = _fill_args(*planes, gamma, None, None, None, None, 0.125, 64)
        y_re, y_im = torch.empty(B, H, T, 64, device="cuda"), torch.empty(B, H, T, 64, device="cuda")
        s_re, s_im = torch.empty(M, B, H, 64, 64, device="cuda"), torch.empty(M, B, H, 64, 64, device="cuda")
        a.y = _mview(y_re, y_im)
        a.s_re, a.s_im = s_re.data_ptr(), s_im.data_ptr()
        return a, keep, (y_re, y_im, s_re, s_im)

    sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
    aa, ka, _ = args()
    ab, kb, outs_b = args()
    torch.cuda.synchronize()
    with torch.cuda.stream(sa):
        torch.cuda._sleep(200_000_000)  # a bounded spin (about 0.1 s) ahead of the call on A
        assert L.qpam_scan_fwd_noalloc(ctypes.byref(aa), ctypes.c_void_p(sa.cuda_stream)) == _lib.QPAM_OK
    st = L.qpam_scan_fwd_noalloc(ctypes.byref(ab), ctypes.c_void_p(sb.cuda_stream))
    assert st == _lib.QPAM_ERR_ARG, st
    assert b"another stream" in L.qpam_last_error()
    torch.cuda.synchronize()
    assert L.qpam_scan_fwd_noalloc(ctypes.byref(ab), ctypes.c_void_p(sb.cuda_stream)) == _lib.QPAM_OK
    torch.cuda.synchronize()
    for g, w in zip(outs_b, want):
        assert torch.equal(g, w)
    del ka, kb
