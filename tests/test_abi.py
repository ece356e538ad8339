"""CPU checks of the C ABI boundary: the built library loads (no GPU needed to
dlopen it), exports every function include/qpam.h declares, the ctypes
structures match the header's field lists, and the product path refuses CPU
tensors instead of falling back."""

import ctypes
import os
import re

import pytest
import torch

from qllm2_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "qpam.h")


def _header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(qpam_\w+)\s*\(", text, flags=re.M)))


def _header_struct_fields(name):
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    m = re.search(r"typedef struct \{([^{}]*)\}\s*" + name + ";", text)
    assert m, name
    fields = []
    for decl in m.group(1).split(";"):
        decl = decl.strip()
        if not decl:
            continue
        decl = re.sub(r"^(const\s+)?\w+\s*", "", decl)
        for part in decl.split(","):
            part = part.strip().lstrip("*").strip()
            part = re.sub(r"\[.*\]", "", part)
            fields.append(part)
    return fields


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.lib()
    names = _header_functions()
    assert "qpam_decode_step" in names and "qpam_scan_fwd" in names and "qpam_ce_fwd" in names
    for n in names:
        assert hasattr(lib, n), f"libqpam.so does not export {n}"
        assert n in _lib.SIGNATURES, f"ctypes binding misses {n}"
    assert set(_lib.SIGNATURES) == set(names)
    assert lib.qpam_version() == _lib.ABI_VERSION


@pytest.mark.parametrize("cname,pyname", [
    ("qpam_decode_args", "DecodeArgs"), ("qpam_scan_args", "ScanArgs"), ("qpam_scan_bwd_args", "ScanBwdArgs"),
    ("qpam_ce_fwd_args", "CeFwdArgs"), ("qpam_ce_bwd_args", "CeBwdArgs"), ("qpam_cplx_args", "CplxArgs"),
    ("qpam_pc_fold_args", "PcFoldArgs"), ("qpam_pc_scan_args", "PcScanArgs"),
    ("qpam_cweight_args", "CWeightArgs"), ("qpam_prologue_args", "PrologueArgs"),
    ("qpam_prologue_bwd_args", "PrologueBwdArgs"), ("qpam_resid_norm_args", "ResidNormArgs"),
    ("qpam_cgu_mix_args", "CguMixArgs"),
])
def test_ctypes_structs_match_header(cname, pyname):
    py = [f[0] for f in getattr(_lib, pyname)._fields_]
    assert py == _header_struct_fields(cname)


def test_errors_surface_as_exceptions_without_gpu():
    lib = _lib.lib()
    a = _lib.DecodeArgs()  # all zero: invalid sizes -> status, message, no launch
    st = lib.qpam_decode_step(ctypes.byref(a), None)
    assert st != 0
    assert b"qpam_decode_step" in lib.qpam_last_error()
    with pytest.raises(_lib.QpamError):
        _lib.check(st, "qpam_decode_step")


def test_complex_op_argument_errors_without_gpu():
    """Bad op, missing parameter and oversized dim come back as errors before any launch."""
    lib = _lib.lib()
    a = _lib.CplxArgs()
    a.op, a.dtype, a.rows, a.dim = 7, _lib.QPAM_F32, 4, 8
    assert lib.qpam_cplx_fwd(ctypes.byref(a), None) != 0 and b"unknown op" in lib.qpam_last_error()
    a.op = _lib.QPAM_CPLX_MOD_SWISH
    a.z, a.out, a.p0 = 16, 16, 16  # p1 (beta) missing
    assert lib.qpam_cplx_fwd(ctypes.byref(a), None) != 0 and b"beta" in lib.qpam_last_error()
    a.op, a.dim = _lib.QPAM_CPLX_NORM, 9000
    assert lib.qpam_cplx_fwd(ctypes.byref(a), None) != 0 and b"too large" in lib.qpam_last_error()
    a.dim = 8
    assert lib.qpam_cplx_workspace_size(ctypes.byref(a)) == 1 * 1 * 8 * 4  # one block, one parameter


@pytest.mark.parametrize("d", [8, 24, 48, 96, 256])
def test_prologue_refuses_head_dims_outside_its_kernels(d):
    """The prologue's C entry points take exactly the head dims the Python side
    dispatches to them (pam_prologue.HEAD_DIMS); any other is an error before
    any launch, forward and backward."""
    from qllm2_amd.pam_prologue import HEAD_DIMS
    assert HEAD_DIMS == (16, 32, 64, 128)
    lib = _lib.lib()
    a = _lib.PrologueArgs()
    a.B, a.T, a.H, a.M, a.d = 1, 1, 1, 1, d
    assert lib.qpam_prologue_fwd(ctypes.byref(a), None) != 0
    assert b"head_dim %d unsupported" % d in lib.qpam_last_error()
    g = _lib.PrologueBwdArgs()
    g.fwd = ctypes.pointer(a)
    assert lib.qpam_prologue_bwd(ctypes.byref(g), None) != 0
    assert b"head_dim %d unsupported" % d in lib.qpam_last_error()


def test_cpu_tensors_are_refused():
    from qllm2_amd import decode, pam_scan
    s = torch.zeros(1, 1, 1, 4, 4, 2)
    q = torch.zeros(1, 1, 4, 2)
    with pytest.raises(ValueError, match="GPU"):
        decode.decode_step(s, q, q, q, torch.zeros(1, 1, 1))
    x = torch.zeros(1, 1, 8, 64)
    with pytest.raises(ValueError, match="GPU"):
        pam_scan.pam_scan_planar(x, x, x, x, x, x, torch.ones(1, 1, 1, 8), q_scale=0.125)


@pytest.mark.parametrize("M,B,H,T,chunk,bf16", [(3, 8, 12, 2048, 64, True), (1, 2, 3, 200, 64, False),
                                                 (2, 1, 5, 70, 16, True), (1, 1, 1, 7, 32, False),
                                                 (4, 3, 1, 129, 64, True)])
def test_scan_workspace_size_matches_python_mirror(M, B, H, T, chunk, bf16):
    """The fake (meta) kernel of qpam::scan_fwd sizes the workspace output with
    the Python mirror of qpam_scan_workspace_size; both must agree."""
    from qllm2_amd import pam_scan
    a = _lib.ScanArgs()
    a.B, a.H, a.T, a.d, a.M, a.C = B, H, T, 64, M, chunk
    a.dtype = 1 if bf16 else 0
    assert _lib.lib().qpam_scan_workspace_size(ctypes.byref(a)) == pam_scan.fwd_workspace_bytes(M, B, H, T, chunk,
                                                                                                 bf16)
