"""GPU parity of the complex elementwise layers (qpam_cplx_fwd / qpam_cplx_bwd
behind qllm2_amd.triton_kernels.fused_*) against autograd of the CPU oracle
(oracle/complex_ops.py, the reference's PyTorch forms) in float64 on the same
inputs.  Tolerances: fp32 rel <= 1e-5 forward, 1e-4 on every gradient; bf16
tensors (fp32 math inside) rel <= 2e-2.  Shapes include the reference's own
check sizes (B=3, T=128, D=384 and D_hidden=1152, v11/triton_kernels.py:600-640),
a dim that is not a multiple of 64 and a single row."""

import pytest
import torch

from oracle import complex_ops as O

pytestmark = pytest.mark.gpu


def _rel(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return ((a - b).abs().max() / (b.abs().max() + 1e-30)).item()


def _inputs(shape, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(*shape, 2, generator=g).to(dtype)
    up = torch.randn(*shape, 2, generator=g).to(dtype)
    gout = torch.randn(*shape, 2, generator=g).to(dtype)
    dim = shape[-1]
    p0 = torch.rand(dim, generator=g) + 0.5
    p1 = torch.rand(dim, generator=g) * 2.0
    return z, up, gout, p0, p1


def _oracle(name, z, up, gout, p0, p1):
    zz = z.double().requires_grad_(True)
    uu = up.double().requires_grad_(True)
    a, b = p0.double().requires_grad_(True), p1.double().requires_grad_(True)
    if name == "norm":
        out, params = O.complex_norm(zz, a), [a]
    elif name == "swish":
        out, params = O.mod_swish(zz, a - 1.0, b), [a, b]
    elif name == "relu":
        out, params = O.mod_relu(zz, a - 1.2), [a]
    else:
        out, params = O.cgu_gate(zz, uu), []
    out.backward(gout.double())
    grads = [zz.grad] + ([uu.grad] if name == "cgu" else []) + [p.grad for p in params]
    return out.detach(), grads


def _gpu(name, z, up, gout, p0, p1):
    from qllm2_amd import triton_kernels as tk
    dev = torch.device("cuda")
    zz = z.to(dev).requires_grad_(True)
    uu = up.to(dev).requires_grad_(True)
    a, b = p0.to(dev).requires_grad_(True), p1.to(dev).requires_grad_(True)
    if name == "norm":
        out, params = tk.fused_complex_norm(zz, a), [a]
    elif name == "swish":
        out, params = tk.fused_mod_swish(zz, a - 1.0, b), [a, b]
    elif name == "relu":
        out, params = tk.fused_mod_relu(zz, a - 1.2), [a]
    else:
        out, params = tk.fused_cgu_gate(zz, uu), []
    assert out.dtype == z.dtype and out.shape == z.shape
    out.backward(gout.to(dev))
    torch.cuda.synchronize()
    grads = [zz.grad] + ([uu.grad] if name == "cgu" else []) + [p.grad for p in params]
    return out.detach(), grads


OPS = ["norm", "swish", "relu", "cgu"]
# dims: 768 / 1024 / 256 / 2048 (dim / 4 a multiple of 64) take the row-team kernels
# (row counts below, at and off a multiple of the rows per iteration, a single row);
# 384 / 1152 / 100 / 64 the register-row kernels (1, 2, 8 groups of four columns per
# lane), 2304 the LDS-accumulating kernels, 7 and 50 the scalar path
SHAPES = [(3, 37, 768), (5, 26, 1024), (1, 256), (2, 2048), (3, 128, 384), (3, 128, 1152), (5, 100), (1, 64),
          (2, 3, 7), (4, 2304), (6, 50)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("name", OPS)
def test_complex_ops_fp32(gpu_lib, name, shape):
    z, up, gout, p0, p1 = _inputs(shape, 100 + len(shape) * 7 + shape[-1], torch.float32)
    ref_out, ref_grads = _oracle(name, z, up, gout, p0, p1)
    out, grads = _gpu(name, z, up, gout, p0, p1)
    assert _rel(out, ref_out) < 1e-5, f"{name} fwd rel {_rel(out, ref_out):.2e}"
    for i, (g, r) in enumerate(zip(grads, ref_grads)):
        assert g is not None and g.dtype == torch.float32
        assert _rel(g, r) < 1e-4, f"{name} grad {i} rel {_rel(g, r):.2e}"


@pytest.mark.parametrize("shape", [(3, 128, 384), (3, 45, 1024)])
@pytest.mark.parametrize("name", OPS)
def test_complex_ops_bf16(gpu_lib, name, shape):
    z, up, gout, p0, p1 = _inputs(shape, 200 + shape[-1], torch.bfloat16)
    ref_out, ref_grads = _oracle(name, z, up, gout, p0, p1)
    out, grads = _gpu(name, z, up, gout, p0, p1)
    assert _rel(out, ref_out) < 2e-2, f"{name} fwd rel {_rel(out, ref_out):.2e}"
    for i, (g, r) in enumerate(zip(grads, ref_grads)):
        assert _rel(g, r) < 2e-2, f"{name} grad {i} rel {_rel(g, r):.2e}"


def test_complex_ops_zero_rows_and_pytorch_toggle(gpu_lib):
    from qllm2_amd import triton_kernels as tk
    z = torch.zeros(0, 16, 2, device="cuda", requires_grad=True)
    s = torch.ones(16, device="cuda", requires_grad=True)
    tk.fused_complex_norm(z, s).sum().backward()
    assert s.grad is not None and torch.all(s.grad == 0)
    # the toggle selects the reference's PyTorch forms (on the GPU); same values
    zz, _, _, p0, _ = _inputs((4, 96), 5, torch.float32)
    zz, p0 = zz.cuda(), p0.cuda()
    hip = tk.fused_complex_norm(zz, p0)
    tk.set_triton_enabled(False)
    try:
        pt = tk.fused_complex_norm(zz, p0)
    finally:
        tk.set_triton_enabled(True)
    assert _rel(hip, pt) < 1e-5


@pytest.mark.parametrize("dtype,rows", [(torch.bfloat16, 70000), (torch.float32, 36000)])
def test_cgu_gate_grid_stride_rows(gpu_lib, dtype, rows):
    """The CGU gate's flat kernels (forward and backward) launch one 16-byte
    group per thread up to 65536 blocks of 256 threads and loop over the rest:
    [rows, 1024] complex tensors with more groups than that (bf16: 4 complex
    per group, 67.1 M elements; fp32: 2 per group, 33.6 M) reach the loop.
    Output and both gradients against the oracle on row ranges served by the
    first pass (the first rows), around the first row the loop serves, and at
    the end (the gate is row-local, so a slice of rows is checked exactly)."""
    from qllm2_amd import triton_kernels as tk
    dim = 1024
    per_group = 4 if dtype == torch.bfloat16 else 2
    assert rows * dim // per_group > 65536 * 256
    first_loop_row = 65536 * 256 * per_group // dim
    g = torch.Generator(device="cuda").manual_seed(77)
    z = torch.randn(rows, dim, 2, device="cuda", generator=g).to(dtype).requires_grad_(True)
    up = torch.randn(rows, dim, 2, device="cuda", generator=g).to(dtype).requires_grad_(True)
    gout = torch.randn(rows, dim, 2, device="cuda", generator=g).to(dtype)
    out = tk.fused_cgu_gate(z, up)
    out.backward(gout)
    torch.cuda.synchronize()
    tol = 2e-2 if dtype == torch.bfloat16 else 1e-5
    for r0, r1 in ((0, 64), (first_loop_row - 40, first_loop_row + 40), (rows - 64, rows)):
        zs, us, gs = (x[r0:r1].detach().cpu() for x in (z, up, gout))
        ones = torch.ones(dim)
        ref_out, ref_grads = _oracle("cgu", zs, us, gs, ones, ones)
        assert _rel(out[r0:r1], ref_out) < tol, f"rows {r0}..{r1}: fwd"
        assert _rel(z.grad[r0:r1], ref_grads[0]) < max(tol, 1e-4), f"rows {r0}..{r1}: dz"
        assert _rel(up.grad[r0:r1], ref_grads[1]) < max(tol, 1e-4), f"rows {r0}..{r1}: dup"
