"""ctypes binding of the qpam C ABI (include/qpam.h).

The library is loaded lazily, after torch (so the HIP runtime that torch
bundles is the one the library binds to: both resolve the soname
libamdhip64.so.7).  There is no fallback: if the library is missing or was
built for another ABI version every entry point raises.
"""

import ctypes
import os

import torch  # noqa: F401  (must be loaded before the HIP library)

LIB_NAME = "libqpam.so"
ABI_VERSION = 14
_HERE = os.path.dirname(os.path.abspath(__file__))

QPAM_F32 = 0
QPAM_BF16 = 1
QPAM_OK = 0
QPAM_ERR_ARG = 1
QPAM_ERR_WORKSPACE = 4
QPAM_SCAN_FWD_NOALLOC_MAX_BYTES = 64 << 20

c_i32 = ctypes.c_int32
c_i64 = ctypes.c_int64
c_ptr = ctypes.c_void_p
c_f32 = ctypes.c_float


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("n_slots", c_i32), ("n_active", c_i32), ("active", c_ptr), ("n_groups", c_i32),
        ("n_states", c_i32), ("d", c_i32), ("q_scale", c_f32),
        ("state", c_ptr), ("st_slot", c_i64), ("st_group", c_i64), ("st_state", c_i64),
        ("q", c_ptr), ("k", c_ptr), ("v", c_ptr),
        ("sq_slot", c_i64), ("sq_group", c_i64), ("sk_slot", c_i64), ("sk_group", c_i64),
        ("sv_slot", c_i64), ("sv_group", c_i64),
        ("gamma", c_ptr), ("sg_slot", c_i64), ("sg_group", c_i64), ("sg_state", c_i64),
        ("rot", c_ptr), ("sr_slot", c_i64), ("sr_group", c_i64), ("sr_state", c_i64),
        ("y", c_ptr), ("sy_slot", c_i64), ("sy_group", c_i64),
        ("rope", c_ptr), ("pos", c_ptr), ("rope_len", c_i32), ("vec_by_rank", c_i32),
        ("q_im", c_ptr), ("k_im", c_ptr), ("v_im", c_ptr), ("rot_im", c_ptr), ("gamma_per_channel", c_i32), ("y_dtype", c_i32),
        ("proj", c_ptr), ("proj_dtype", c_i32), ("qk_norm", c_i32), ("proj_ld", c_i64),
        ("gate", c_ptr), ("gate_ld", c_i64), ("protect_col", c_i32), ("phase_col", c_i32),
        ("dt_bias", c_ptr), ("state_offset", c_ptr), ("gamma_floor", c_f32),
    ]


class CView(ctypes.Structure):
    _fields_ = [("re", c_ptr), ("im", c_ptr), ("s0", c_i64), ("s1", c_i64), ("s2", c_i64)]


class MView(ctypes.Structure):
    _fields_ = [("re", c_ptr), ("im", c_ptr), ("s0", c_i64), ("s1", c_i64), ("s2", c_i64)]


class ScanArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_i32), ("H", c_i32), ("T", c_i32), ("d", c_i32), ("C", c_i32), ("M", c_i32),
        ("dtype", c_i32), ("q_scale", c_f32), ("y_dtype", c_i32), ("reserved0", c_i32),
        ("q", CView), ("k", CView), ("v", CView),
        ("gamma", c_ptr), ("sg_m", c_i64), ("sg_b", c_i64), ("sg_h", c_i64), ("sg_t", c_i64),
        ("rot_re", c_ptr), ("rot_im", c_ptr), ("sr_m", c_i64), ("sr_b", c_i64), ("sr_h", c_i64), ("sr_t", c_i64),
        ("s0_re", c_ptr), ("s0_im", c_ptr),
        ("y", MView),
        ("s_re", c_ptr), ("s_im", c_ptr),
        ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
        ("prof_ev", c_ptr * 2),
    ]


class ScanBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", ctypes.POINTER(ScanArgs)),
        ("dy", CView), ("dy_dtype", c_i32), ("reserved0", c_i32),
        ("ds_re", c_ptr), ("ds_im", c_ptr),
        ("dq", MView), ("dk", MView), ("dv", MView),
        ("dgamma", c_ptr),
        ("drot_re", c_ptr), ("drot_im", c_ptr),
        ("ds0_re", c_ptr), ("ds0_im", c_ptr),
        ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
    ]


class CeFwdArgs(ctypes.Structure):
    _fields_ = [
        ("N", c_i32), ("V", c_i32), ("D", c_i32), ("dtype", c_i32),
        ("h", c_ptr), ("ldh", c_i64), ("w", c_ptr), ("ldw", c_i64),
        ("targets", c_ptr), ("mask", c_ptr), ("ignore_index", c_i64),
        ("lse", c_ptr), ("loss", c_ptr), ("correct", c_ptr), ("loss_sum", c_ptr),
        ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
    ]


class CeBwdArgs(ctypes.Structure):
    _fields_ = [
        ("N", c_i32), ("V", c_i32), ("D", c_i32), ("dtype", c_i32),
        ("h", c_ptr), ("ldh", c_i64), ("w", c_ptr), ("ldw", c_i64),
        ("targets", c_ptr), ("mask", c_ptr), ("ignore_index", c_i64),
        ("lse", c_ptr), ("grad_scale", c_ptr),
        ("dh", c_ptr), ("lddh", c_i64), ("dw", c_ptr), ("lddw", c_i64),
        ("chunk", c_i32),
        ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
        ("dw_out", c_i32),
    ]


QPAM_CPLX_NORM, QPAM_CPLX_MOD_SWISH, QPAM_CPLX_MOD_RELU, QPAM_CPLX_CGU_GATE = 0, 1, 2, 3


class CplxArgs(ctypes.Structure):
    _fields_ = [
        ("op", c_i32), ("dtype", c_i32), ("rows", c_i64), ("dim", c_i32), ("eps", c_f32),
        ("z", c_ptr), ("up", c_ptr), ("p0", c_ptr), ("p1", c_ptr), ("out", c_ptr),
        ("gout", c_ptr), ("gz", c_ptr), ("gup", c_ptr), ("gp0", c_ptr), ("gp1", c_ptr),
        ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
    ]


# symbol -> (restype, argtypes); every symbol include/qpam.h declares
class DeltaArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_i32), ("H", c_i32), ("T", c_i32), ("d", c_i32), ("q_scale", c_f32), ("gamma_eps", c_f32),
        ("chunk", c_i32), ("exact_write", c_i32),
        ("q", CView), ("k", CView), ("v", CView),
        ("gamma", c_ptr), ("beta", c_ptr), ("sg_b", c_i64), ("sg_h", c_i64), ("sg_t", c_i64),
        ("s0_re", c_ptr), ("s0_im", c_ptr), ("y", MView), ("s_re", c_ptr), ("s_im", c_ptr),
        ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
        ("scratch", c_ptr), ("scratch_bytes", ctypes.c_size_t),
    ]


class DeltaBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", ctypes.POINTER(DeltaArgs)), ("dy", CView), ("ds_re", c_ptr), ("ds_im", c_ptr),
        ("dq", MView), ("dk", MView), ("dv", MView), ("dgamma", c_ptr), ("dbeta", c_ptr),
        ("ds0_re", c_ptr), ("ds0_im", c_ptr), ("workspace", c_ptr), ("workspace_bytes", ctypes.c_size_t),
    ]


class PrologueArgs(ctypes.Structure):
    _fields_ = [
        ("B", c_i32), ("T", c_i32), ("H", c_i32), ("d", c_i32), ("M", c_i32),
        ("in_dtype", c_i32), ("out_dtype", c_i32), ("qk_norm", c_i32), ("gamma_floor", c_f32),
        ("rope_offset", c_i32), ("rope_len", c_i32), ("rope", c_ptr),
        ("q_re", c_ptr), ("q_im", c_ptr), ("k_re", c_ptr), ("k_im", c_ptr), ("v_re", c_ptr), ("v_im", c_ptr),
        ("sx_b", c_i64), ("sx_t", c_i64), ("sx_h", c_i64),
        ("dt", c_ptr), ("sd_b", c_i64), ("sd_t", c_i64), ("sd_h", c_i64),
        ("dt_bias", c_ptr), ("state_offset", c_ptr),
        ("protect", c_ptr), ("sp_b", c_i64), ("sp_t", c_i64), ("sp_h", c_i64),
        ("phase", c_ptr), ("routing", c_ptr), ("sr_b", c_i64), ("sr_t", c_i64), ("sr_h", c_i64), ("sr_m", c_i64),
        ("oq_re", c_ptr), ("oq_im", c_ptr), ("ok_re", c_ptr), ("ok_im", c_ptr), ("ov_re", c_ptr), ("ov_im", c_ptr),
        ("gamma", c_ptr), ("rot_re", c_ptr), ("rot_im", c_ptr), ("param_dtype", c_i32), ("dt_bias2", c_ptr),
    ]


class PrologueBwdArgs(ctypes.Structure):
    _fields_ = [
        ("fwd", ctypes.POINTER(PrologueArgs)),
        ("gq_re", c_ptr), ("gq_im", c_ptr), ("gk_re", c_ptr), ("gk_im", c_ptr), ("gv_re", c_ptr), ("gv_im", c_ptr),
        ("ggamma", c_ptr), ("grot_re", c_ptr), ("grot_im", c_ptr),
        ("dq_re", c_ptr), ("dq_im", c_ptr), ("dk_re", c_ptr), ("dk_im", c_ptr), ("dv_re", c_ptr), ("dv_im", c_ptr),
        ("sg_b", c_i64), ("sg_t", c_i64), ("sg_h", c_i64),
        ("dpre", c_ptr), ("ddt", c_ptr), ("sdd_b", c_i64), ("sdd_t", c_i64), ("sdd_h", c_i64),
        ("dprotect", c_ptr), ("dphase", c_ptr), ("drouting", c_ptr), ("dlogit_dtype", c_i32), ("ddt_pad", c_i32),
        ("sdp_b", c_i64), ("sdp_t", c_i64), ("sdp_h", c_i64),
        ("sdq_b", c_i64), ("sdq_t", c_i64), ("sdq_h", c_i64), ("sdq_m", c_i64),
        ("dbias", c_ptr), ("doffset", c_ptr),
    ]


class DecodeBwdArgs(ctypes.Structure):
    _fields_ = [
        ("n", c_i64), ("d", c_i32), ("gamma_per_channel", c_i32),
        ("state", c_ptr), ("gamma", c_ptr), ("q", c_ptr), ("k", c_ptr), ("v", c_ptr), ("dy", c_ptr),
        ("dstate_new", c_ptr),
        ("dstate", c_ptr), ("dgamma", c_ptr), ("dq", c_ptr), ("dk", c_ptr), ("dv", c_ptr),
    ]


class PcFoldArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_i32), ("g_dtype", c_i32), ("B", c_i64), ("H", c_i64), ("T", c_i64), ("d", c_i64),
        ("chunk", c_i32), ("q_scale", c_f32),
        ("q", c_ptr), ("k", c_ptr), ("q_sb", c_i64), ("q_sh", c_i64), ("q_st", c_i64),
        ("k_sb", c_i64), ("k_sh", c_i64), ("k_st", c_i64),
        ("gamma", c_ptr), ("g_sb", c_i64), ("g_sh", c_i64), ("g_st", c_i64),
        ("qf", c_ptr), ("kf", c_ptr), ("wf", c_ptr), ("atot", c_ptr),
        ("dqf", c_ptr), ("dkf", c_ptr), ("dwf", c_ptr), ("datot", c_ptr),
        ("dq", c_ptr), ("dk", c_ptr), ("dgamma", c_ptr),
    ]


class PcScanArgs(ctypes.Structure):
    _fields_ = [
        ("N", c_i64), ("n", c_i64), ("d", c_i64), ("x", c_ptr), ("a", c_ptr), ("out", c_ptr),
        ("init", c_ptr), ("fin", c_ptr), ("reverse", c_i32),
    ]


class CWeightArgs(ctypes.Structure):
    _fields_ = [
        ("dtype", c_i32), ("layout", c_i32), ("R", c_i64), ("C", c_i64), ("wr", c_ptr), ("wi", c_ptr),
        ("tail", c_ptr), ("tail_rows", c_i64), ("zero_rows", c_i64), ("w", c_ptr), ("ldw", c_i64),
        ("g", c_ptr), ("g_dtype", c_i32), ("slices", c_i32), ("slice_stride", c_i64),
        ("g_wr", c_ptr), ("g_wi", c_ptr), ("g_tail", c_ptr),
    ]


QPAM_CW_IN, QPAM_CW_OUT = 0, 1


class ResidNormArgs(ctypes.Structure):
    _fields_ = [
        ("rows", c_i64), ("dim", c_i32), ("eps", c_f32), ("x", c_ptr), ("ldx", c_i64), ("y", c_ptr),
        ("y_dtype", c_i32), ("ldy", c_i64), ("y_scale", c_ptr), ("norm_scale", c_ptr), ("out", c_ptr),
        ("out_dtype", c_i32), ("ldo", c_i64),
    ]


class CguMixArgs(ctypes.Structure):
    _fields_ = [
        ("rows", c_i64), ("hid", c_i32), ("gu", c_ptr), ("gu_dtype", c_i32), ("ldg", c_i64), ("bias", c_ptr),
        ("beta", c_ptr), ("phase_alpha", c_ptr), ("phase_beta", c_ptr), ("out", c_ptr), ("out_dtype", c_i32),
        ("ldo", c_i64),
    ]

SIGNATURES = {
    "qpam_version": (ctypes.c_int, []),
    "qpam_last_error": (ctypes.c_char_p, []),
    "qpam_event_create": (ctypes.c_int, [ctypes.POINTER(c_ptr)]),
    "qpam_event_destroy": (ctypes.c_int, [c_ptr]),
    "qpam_event_elapsed_ms": (ctypes.c_int, [c_ptr, c_ptr, ctypes.POINTER(c_f32)]),
    "qpam_decode_step": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), c_ptr]),
    "qpam_decode_step_bwd": (ctypes.c_int, [ctypes.POINTER(DecodeBwdArgs), c_ptr]),
    "qpam_scan_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(ScanArgs)]),
    "qpam_scan_fwd": (ctypes.c_int, [ctypes.POINTER(ScanArgs), c_ptr]),
    "qpam_scan_fwd_noalloc": (ctypes.c_int, [ctypes.POINTER(ScanArgs), c_ptr]),
    "qpam_scan_bwd_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(ScanBwdArgs)]),
    "qpam_scan_bwd": (ctypes.c_int, [ctypes.POINTER(ScanBwdArgs), c_ptr]),
    "qpam_decay_matrix": (ctypes.c_int, [c_i32, c_i32, c_ptr, c_i64, c_ptr, c_ptr]),
    "qpam_ce_fwd_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(CeFwdArgs)]),
    "qpam_ce_fwd": (ctypes.c_int, [ctypes.POINTER(CeFwdArgs), c_ptr]),
    "qpam_ce_bwd_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(CeBwdArgs)]),
    "qpam_ce_bwd": (ctypes.c_int, [ctypes.POINTER(CeBwdArgs), c_ptr]),
    "qpam_cplx_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(CplxArgs)]),
    "qpam_cplx_fwd": (ctypes.c_int, [ctypes.POINTER(CplxArgs), c_ptr]),
    "qpam_cplx_bwd": (ctypes.c_int, [ctypes.POINTER(CplxArgs), c_ptr]),
    "qpam_resid_norm": (ctypes.c_int, [ctypes.POINTER(ResidNormArgs), c_ptr]),
    "qpam_cgu_mix": (ctypes.c_int, [ctypes.POINTER(CguMixArgs), c_ptr]),
    "qpam_prologue_fwd": (ctypes.c_int, [ctypes.POINTER(PrologueArgs), c_ptr]),
    "qpam_prologue_bwd": (ctypes.c_int, [ctypes.POINTER(PrologueBwdArgs), c_ptr]),
    "qpam_cabs_fwd": (ctypes.c_int, [c_i32, c_i64, c_ptr, c_ptr, c_ptr]),
    "qpam_delta_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(DeltaArgs)]),
    "qpam_delta_scratch_size": (ctypes.c_size_t, [ctypes.POINTER(DeltaArgs)]),
    "qpam_delta_fwd": (ctypes.c_int, [ctypes.POINTER(DeltaArgs), c_ptr]),
    "qpam_delta_bwd_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(DeltaBwdArgs)]),
    "qpam_delta_bwd": (ctypes.c_int, [ctypes.POINTER(DeltaBwdArgs), c_ptr]),
    "qpam_cabs_bwd": (ctypes.c_int, [c_i32, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "qpam_mag_linear": (ctypes.c_int, [c_i32, c_i32, c_i64, c_i32, c_i32, c_ptr, c_ptr, c_ptr, c_ptr, c_i64, c_ptr]),
    "qpam_pc_fold_fwd": (ctypes.c_int, [ctypes.POINTER(PcFoldArgs), c_ptr]),
    "qpam_pc_fold_bwd": (ctypes.c_int, [ctypes.POINTER(PcFoldArgs), c_ptr]),
    "qpam_pc_scan": (ctypes.c_int, [ctypes.POINTER(PcScanArgs), c_ptr]),
    "qpam_cweight_pack": (ctypes.c_int, [ctypes.POINTER(CWeightArgs), c_ptr]),
    "qpam_cweight_unpack": (ctypes.c_int, [ctypes.POINTER(CWeightArgs), c_ptr]),
    "qpam_cabs_bwd_acc": (ctypes.c_int, [c_i32, c_i64, c_ptr, c_ptr, c_ptr, c_ptr, c_ptr]),
    "qpam_slice_sum": (ctypes.c_int, [c_i32, c_i32, c_i32, c_i64, c_i64, c_ptr, c_ptr, c_ptr]),
}

_LIB = None


class QpamError(RuntimeError):
    pass


def lib_path():
    return os.path.join(_HERE, LIB_NAME)


def lib():
    """Load (once) and return the ctypes library.  Raises if it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = lib_path()
    if not os.path.exists(path):
        raise QpamError(f"{path} is not built; run __graft_entry__.build() (hipcc --offload-arch=gfx950)")
    handle = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    ver = handle.qpam_version()
    if ver != ABI_VERSION:
        raise QpamError(f"{path}: ABI version {ver}, expected {ABI_VERSION}; rebuild")
    _LIB = handle
    return _LIB


def check(status, what):
    if status != 0:
        msg = lib().qpam_last_error().decode(errors="replace")
        raise QpamError(f"{what} failed (status {status}): {msg}")


def stream_ptr(device=None):
    """Raw hipStream_t of torch's current stream on `device`."""
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


class EventPair:
    """Two HIP timing events created by the library (for the prof_ev fields)."""

    def __init__(self):
        L = lib()
        self.ev = [c_ptr(), c_ptr()]
        for e in self.ev:
            check(L.qpam_event_create(ctypes.byref(e)), "qpam_event_create")

    def elapsed_ms(self):
        ms = c_f32()
        check(lib().qpam_event_elapsed_ms(self.ev[0], self.ev[1], ctypes.byref(ms)), "qpam_event_elapsed_ms")
        return ms.value

    def __del__(self):
        try:
            for e in self.ev:
                lib().qpam_event_destroy(e)
        except Exception:
            pass
