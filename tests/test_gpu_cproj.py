"""Packed complex projections (qpam_cweight_pack / _unpack, qllm2_amd/cproj.py)
against the torch assembly of the same real weight (ComplexLinear,
v11/complex_ops.py:146-172: re = Wr xr - Wi xi, im = Wi xr + Wr xi) and
against ComplexLinear itself through autograd."""

import pytest
import torch

pytestmark = pytest.mark.gpu


def _dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return "cuda"


def _w_in_torch(wr, wi, tail, cols):
    """The input projection's weight as torch ops: [wr, -wi] and [wi, wr]
    interleaved per input feature, the tail reordered to the interleaved
    input, zero rows up to cols."""
    R, C = wr.shape
    parts = [torch.stack([wr, -wi], -1).view(R, 2 * C), torch.stack([wi, wr], -1).view(R, 2 * C)]
    if tail is not None:
        parts.append(tail.view(tail.shape[0], 2, C).transpose(1, 2).reshape(tail.shape[0], 2 * C))
    rows = sum(p.shape[0] for p in parts)
    if cols > rows:
        parts.append(wr.new_zeros(cols - rows, 2 * C))
    return torch.cat(parts, 0)


def _w_out_torch(wr, wi):
    R = wr.shape[0]
    return torch.stack([torch.cat([wr, -wi], 1), torch.cat([wi, wr], 1)], 1).view(2 * R, -1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("R,C,H,pad", [(96, 64, 3, 5), (2304, 768, 12, 4), (8, 4, 0, 0)])
def test_pack_in_bit_exact(dtype, R, C, H, pad):
    from qllm2_amd import _lib, cproj
    dev = _dev()
    g = torch.Generator(device=dev).manual_seed(R + C)
    wr, wi = (torch.randn(R, C, device=dev, generator=g).to(dtype) for _ in range(2))
    tail = torch.randn(H, 2 * C, device=dev, generator=g).to(dtype) if H else None
    cols = 2 * R + H + pad
    w = cproj._pack(_lib.QPAM_CW_IN, wr, wi, tail, cols)
    assert torch.equal(w, _w_in_torch(wr, wi, tail, cols))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("R,C", [(768, 768), (40, 24), (8, 8)])
def test_pack_out_bit_exact(dtype, R, C):
    from qllm2_amd import _lib, cproj
    dev = _dev()
    g = torch.Generator(device=dev).manual_seed(R * 7 + C)
    wr, wi = (torch.randn(R, C, device=dev, generator=g).to(dtype) for _ in range(2))
    assert torch.equal(cproj._pack(_lib.QPAM_CW_OUT, wr, wi), _w_out_torch(wr, wi))


@pytest.mark.parametrize("wdt,gdt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16),
                                     (torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16)])
def test_unpack_in_is_the_adjoint(wdt, gdt):
    """The unpack is the transpose of the pack: its outputs are the gradients of
    <W(wr, wi, tail), G> by autograd through the torch assembly, formed in fp32
    and rounded once."""
    from qllm2_amd import _lib, cproj
    dev = _dev()
    R, C, H, cols = 192, 128, 6, 192 * 2 + 6 + 2
    gen = torch.Generator(device=dev).manual_seed(3)
    wr, wi = (torch.randn(R, C, device=dev, generator=gen).to(wdt) for _ in range(2))
    tail = torch.randn(H, 2 * C, device=dev, generator=gen).to(wdt)
    G = torch.randn(cols, 2 * C, device=dev, generator=gen).to(gdt)
    g_wr, g_wi, g_tail = cproj._unpack(_lib.QPAM_CW_IN, G, 1, wr, wi, tail, cols)
    leaves = [x.float().requires_grad_(True) for x in (wr, wi, tail)]
    (_w_in_torch(*leaves, cols) * G.float()).sum().backward()
    for got, leaf in zip((g_wr, g_wi, g_tail), leaves):
        assert got.dtype == wdt
        assert torch.equal(got, leaf.grad.to(wdt))


@pytest.mark.parametrize("wdt,gdt", [(torch.float32, torch.float32), (torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("slices", [1, 4])
def test_unpack_out_sums_slices(wdt, gdt, slices):
    from qllm2_amd import _lib, cproj
    dev = _dev()
    R, C = 96, 64
    gen = torch.Generator(device=dev).manual_seed(11 + slices)
    wr, wi = (torch.randn(R, C, device=dev, generator=gen).to(wdt) for _ in range(2))
    Gs = torch.randn(slices, 2 * R, 2 * C, device=dev, generator=gen).to(gdt)
    g_wr, g_wi, _ = cproj._unpack(_lib.QPAM_CW_OUT, Gs, slices, wr, wi, None, 2 * R)
    G = Gs[0].float()
    for s in range(1, slices):  # slice order, as the kernel sums
        G = G + Gs[s].float()
    leaves = [x.float().requires_grad_(True) for x in (wr, wi)]
    (_w_out_torch(*leaves) * G).sum().backward()
    for got, leaf in zip((g_wr, g_wi), leaves):
        assert torch.equal(got, leaf.grad.to(wdt))


def _clinear(x, wr, wi):
    """ComplexLinear (v11/complex_ops.py:165-172) on [..., C, 2] -> [..., R, 2]."""
    re = x[..., 0] @ wr.t() - x[..., 1] @ wi.t()
    im = x[..., 0] @ wi.t() + x[..., 1] @ wr.t()
    return torch.stack([re, im], -1)


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-5), (torch.bfloat16, 2e-2)])
def test_linear_in_matches_complex_linear(dtype, tol):
    from qllm2_amd import cproj
    dev = _dev()
    B, T, C, R, H = 2, 384, 128, 96, 4
    cols = 2 * R + H + 4
    gen = torch.Generator(device=dev).manual_seed(5)
    x = torch.randn(B, T, C, 2, device=dev, generator=gen)
    wr, wi = (torch.randn(R, C, device=dev, generator=gen) * C ** -0.5 for _ in range(2))
    tail = torch.randn(H, 2 * C, device=dev, generator=gen) * C ** -0.5
    gout = torch.randn(B, T, cols, device=dev, generator=gen)
    p = [t.to(dtype).requires_grad_(True) for t in (x, wr, wi, tail)]
    y = cproj.linear_in(p[0].view(B, T, 2 * C), p[1], p[2], p[3], cols)
    y.backward(gout.to(dtype))
    # reference in fp32 on the same (rounded) inputs
    q = [t.detach().float().requires_grad_(True) for t in p]
    z = _clinear(q[0], q[1], q[2])
    dt = torch.cat([q[0][..., 0], q[0][..., 1]], -1) @ q[3].t()
    ref = torch.cat([z[..., 0], z[..., 1], dt, torch.zeros(B, T, cols - 2 * R - H, device=dev)], -1)
    ref.backward(gout.to(dtype).float())
    scale = lambda r: r.abs().max().clamp_min(1e-6)
    assert ((y.float() - ref).abs().max() / scale(ref)) < tol
    for a, b in zip(p, q):
        assert ((a.grad.float() - b.grad).abs().max() / scale(b.grad)) < tol


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("N", [8192, 1000])
def test_linear_out_matches_complex_linear(dtype, tol, N):
    """N = 8192 runs the sliced weight gradient (4 slices of 2048 rows), N = 1000
    one slice."""
    from qllm2_amd import cproj
    dev = _dev()
    C, R = 256, 128
    gen = torch.Generator(device=dev).manual_seed(N)
    y2 = torch.randn(N, 2 * C, device=dev, generator=gen)
    wr, wi = (torch.randn(R, C, device=dev, generator=gen) * C ** -0.5 for _ in range(2))
    gout = torch.randn(N, 2 * R, device=dev, generator=gen)
    p = [t.to(dtype).requires_grad_(True) for t in (y2, wr, wi)]
    out = cproj.linear_out(*p)
    out.backward(gout.to(dtype))
    q = [t.detach().float().requires_grad_(True) for t in p]
    xin = torch.stack([q[0][:, :C], q[0][:, C:]], -1)
    ref = _clinear(xin, q[1], q[2]).reshape(N, 2 * R)
    ref.backward(gout.to(dtype).float())
    scale = lambda r: r.abs().max().clamp_min(1e-6)
    assert ((out.float() - ref).abs().max() / scale(ref)) < tol
    for a, b in zip(p, q):
        assert ((a.grad.float() - b.grad).abs().max() / scale(b.grad)) < tol


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-5), (torch.bfloat16, 2e-2)])
def test_linear_in_with_mag(dtype, tol):
    """proj and cabs(x) from one call; x's gradient sums the projection's and
    the one through |x| (cabs, v11/complex_ops.py:86-87)."""
    from qllm2_amd import cproj
    dev = _dev()
    B, T, C, R, H = 2, 256, 64, 48, 3
    cols = 2 * R + H + 5
    gen = torch.Generator(device=dev).manual_seed(8)
    x = torch.randn(B, T, C, 2, device=dev, generator=gen)
    wr, wi = (torch.randn(R, C, device=dev, generator=gen) * C ** -0.5 for _ in range(2))
    tail = torch.randn(H, 2 * C, device=dev, generator=gen) * C ** -0.5
    g1 = torch.randn(B, T, cols, device=dev, generator=gen)
    g2 = torch.randn(B, T, C, device=dev, generator=gen)
    p = [t.to(dtype).requires_grad_(True) for t in (x, wr, wi, tail)]
    y, mag = cproj.linear_in(p[0].view(B, T, 2 * C), p[1], p[2], p[3], cols, with_mag=True)
    torch.autograd.backward([y, mag], [g1.to(dtype), g2.to(dtype)])
    q = [t.detach().float().requires_grad_(True) for t in p]
    z = _clinear(q[0], q[1], q[2])
    dt = torch.cat([q[0][..., 0], q[0][..., 1]], -1) @ q[3].t()
    ref = torch.cat([z[..., 0], z[..., 1], dt, torch.zeros(B, T, cols - 2 * R - H, device=dev)], -1)
    mref = torch.sqrt(q[0][..., 0] ** 2 + q[0][..., 1] ** 2 + 1e-8)
    torch.autograd.backward([ref, mref], [g1.to(dtype).float(), g2.to(dtype).float()])
    scale = lambda r: r.abs().max().clamp_min(1e-6)
    assert ((mag.float() - mref).abs().max() / scale(mref)) < tol
    for a, b in zip(p, q):
        assert ((a.grad.float() - b.grad).abs().max() / scale(b.grad)) < tol


@pytest.mark.parametrize("dtype,tol", [(torch.float32, 2e-5), (torch.bfloat16, 2e-2)])
@pytest.mark.parametrize("parts", [1, 2])
def test_gate_linear_matches_linear(dtype, tol, parts):
    """Stacked nn.Linear rows over one input (N = 16384 runs 32 row slices in
    the weight gradient) against torch autograd through F.linear."""
    from qllm2_amd import cproj
    dev = _dev()
    N, D = 16384, 256
    rows = [12, 36][:parts]
    gen = torch.Generator(device=dev).manual_seed(parts)
    x = torch.rand(N, D, device=dev, generator=gen)
    ws = [torch.randn(r, D, device=dev, generator=gen) * D ** -0.5 for r in rows]
    bs = [torch.randn(r, device=dev, generator=gen) for r in rows]
    g = torch.randn(N, sum(rows), device=dev, generator=gen)
    p = [t.to(dtype).requires_grad_(True) for t in [x] + ws + bs]
    assert cproj.gate_supported(p[0], p[1:1 + parts], p[1 + parts:])
    out = cproj.gate_linear(p[0], p[1:1 + parts], p[1 + parts:])
    out.backward(g.to(dtype))
    q = [t.detach().float().requires_grad_(True) for t in p]
    ref = torch.nn.functional.linear(q[0], torch.cat(q[1:1 + parts]), torch.cat(q[1 + parts:]))
    ref.backward(g.to(dtype).float())
    scale = lambda r: r.abs().max().clamp_min(1e-6)
    assert ((out.float() - ref).abs().max() / scale(ref)) < tol
    for a, b in zip(p, q):
        assert a.grad.dtype == a.dtype
        assert ((a.grad.float() - b.grad).abs().max() / scale(b.grad)) < tol
