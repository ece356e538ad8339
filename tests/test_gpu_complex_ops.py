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


# ------------------------------------------------ decode block glue (inference)

@pytest.mark.parametrize("dim,rows", [(768, 211), (64, 5), (1000, 3), (2048, 17)])
@pytest.mark.parametrize("ydt,odt", [(None, torch.float32), (torch.float32, torch.float32),
                                     (torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16),
                                     (torch.bfloat16, torch.float32)])
def test_resid_norm_matches_add_then_norm(gpu_lib, dim, rows, ydt, odt):
    """qpam_resid_norm: x += y * s in place (bit-equal to torch's fp32 product
    then sum), then ComplexNorm of the new x against the float64 oracle (fp32
    out rel <= 1e-5, bf16 out rel <= 2^-8 per element of the row scale); with no
    y and a dim the norm's row-team path takes (768), bit-equal to
    qpam_cplx_fwd's ComplexNorm.  x rows strided inside a wider buffer."""
    from qllm2_amd import triton_kernels as tk
    from qllm2_amd.model_decode import resid_norm
    g = torch.Generator().manual_seed(dim + rows)
    xs = (torch.randn(rows, dim + 8, 2, generator=g) * 1.5).cuda()
    x = xs[:, :dim]
    y = torch.randn(rows, dim, 2, generator=g).cuda().to(ydt) if ydt is not None else None
    scale = (torch.rand(dim, generator=g) + 0.5).cuda()
    s = torch.tensor(0.7, device="cuda")
    x0 = x.clone()
    want_x = x0 + y.float() * s if y is not None else x0
    out = resid_norm(x, scale, 1e-6, y=y, y_scale=s, out_dtype=odt)
    assert torch.equal(x, want_x)
    assert out.dtype == odt and out.shape == (rows, dim, 2)
    ref = O.complex_norm(want_x.double().cpu(), scale.double().cpu(), 1e-6)
    err = (out.double().cpu() - ref).abs().amax((-1, -2)) / ref.abs().amax((-1, -2))
    assert err.max().item() < (1e-5 if odt == torch.float32 else 2 ** -8)
    if y is None and dim == 768:
        assert torch.equal(out.float(), tk.fused_complex_norm(x0.contiguous(), scale, 1e-6).to(odt).float())


@pytest.mark.parametrize("act", ["swish", "relu", "phase_mod"])
@pytest.mark.parametrize("gdt,odt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.bfloat16, torch.float32)])
@pytest.mark.parametrize("hid,rows", [(2304, 130), (36, 3)])
def test_cgu_mix_matches_oracle(gpu_lib, act, gdt, odt, hid, rows):
    """qpam_cgu_mix: cgu_gate(gate, act(up)) from the [gate | up] GEMM output
    against the float64 oracle on the same (dtype-rounded) inputs: fp32 rel <=
    1e-5 of each row's largest output, bf16 output rel <= 2^-8; gu rows strided
    inside a wider buffer; the fp32 result also against the HIP ops one at a
    time (fused_mod_* then fused_cgu_gate)."""
    from qllm2_amd import triton_kernels as tk
    from qllm2_amd.model_decode import cgu_mix
    g = torch.Generator().manual_seed(hid + rows)
    gus = (torch.randn(rows, 4 * hid + 16, generator=g) * 1.3).cuda().to(gdt)
    gu = gus[:, :4 * hid]
    bias = (torch.randn(hid, generator=g) * 0.3).cuda()
    beta = (1 + torch.randn(hid, generator=g) * 0.2).cuda() if act != "relu" else None
    pa = torch.randn(hid, generator=g).cuda() if act == "phase_mod" else None
    pb = (torch.randn(hid, generator=g) * 2).cuda() if act == "phase_mod" else None
    out = cgu_mix(gu, hid, bias, beta, pa, pb, out_dtype=odt)
    assert out.dtype == odt and out.shape == (rows, hid, 2)
    gd = gu.double().cpu()
    gate, up = gd[:, :2 * hid].reshape(rows, hid, 2), gd[:, 2 * hid:].reshape(rows, hid, 2)
    b64 = bias.double().cpu()
    if act == "swish":
        u = O.mod_swish(up, b64, beta.double().cpu())
    elif act == "relu":
        u = O.mod_relu(up, b64)
    else:
        u = O.phase_mod(up, b64, beta.double().cpu(), pa.double().cpu(), pb.double().cpu())
    ref = O.cgu_gate(gate, u)
    err = (out.double().cpu() - ref).abs().amax((-1, -2)) / ref.abs().amax((-1, -2))
    assert err.max().item() < (1e-5 if odt == torch.float32 else 2 ** -8)
    if act != "phase_mod" and gdt == torch.float32:
        gf, uf = gu[:, :2 * hid].reshape(rows, hid, 2).contiguous(), gu[:, 2 * hid:].reshape(rows, hid, 2).contiguous()
        ua = tk.fused_mod_swish(uf, bias, beta) if act == "swish" else tk.fused_mod_relu(uf, bias)
        assert _rel(out, tk.fused_cgu_gate(gf, ua)) < 1e-6


def test_block_glue_rejects_bad_arguments(gpu_lib):
    from qllm2_amd import _lib
    from qllm2_amd.model_decode import cgu_mix, resid_norm
    x = torch.randn(4, 18, 2, device="cuda")
    with pytest.raises(_lib.QpamError, match="multiple of 4"):
        resid_norm(x, torch.ones(18, device="cuda"), 1e-6)
    x = torch.randn(4, 4096, 2, device="cuda")
    with pytest.raises(_lib.QpamError, match="at most"):
        resid_norm(x, torch.ones(4096, device="cuda"), 1e-6)
    gu = torch.randn(3, 4 * 8, device="cuda")
    with pytest.raises(_lib.QpamError, match="given together"):
        cgu_mix(gu, 8, torch.zeros(8, device="cuda"), torch.ones(8, device="cuda"), torch.zeros(8, device="cuda"), None)


def test_block_glue_wrappers_check_parameters(gpu_lib):
    """The host wrappers refuse parameter vectors the kernels would misread
    (wrong length, dtype or device) before any launch."""
    from qllm2_amd.model_decode import cgu_mix, resid_norm
    x = torch.randn(4, 16, 2, device="cuda")
    with pytest.raises(ValueError, match="scale"):
        resid_norm(x, torch.ones(8, device="cuda"), 1e-6)
    with pytest.raises(ValueError, match="scale"):
        resid_norm(x, torch.ones(16, device="cuda", dtype=torch.bfloat16), 1e-6)
    with pytest.raises(ValueError, match="scale"):
        resid_norm(x, torch.ones(16), 1e-6)
    with pytest.raises(ValueError, match="y_scale"):
        resid_norm(x, torch.ones(16, device="cuda"), 1e-6, y=x.clone(), y_scale=torch.ones(2, device="cuda"))
    gu = torch.randn(3, 4 * 8, device="cuda")
    with pytest.raises(ValueError, match="bias"):
        cgu_mix(gu, 8, torch.zeros(4, device="cuda"))
    with pytest.raises(ValueError, match="beta"):
        cgu_mix(gu, 8, torch.zeros(8, device="cuda"), torch.ones(8, device="cuda", dtype=torch.float64))
