"""ctypes binding of libqhtp.so (the C ABI declared in include/qhtp.h).

The library is loaded from the package directory only; there is no fallback.  If it is
missing, ``lib()`` raises with the build command, so no GPU path can silently degrade.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libqhtp.so"

QH_STATUS_OK = 0
QH_STATUS_INVALID_ARGUMENT = 1
QH_STATUS_UNSUPPORTED = 2
QH_STATUS_RUNTIME_ERROR = 3
QH_STATUS_SHAPE_UNSUPPORTED = 4

QH_WEIGHT_I8 = 0
QH_WEIGHT_I4 = 1
QH_WEIGHT_I4_LPBQ = 2
QH_WEIGHT_I4_GROUP = 3
QH_WEIGHT_I16 = 4

# Integer output contracts (qh_contract).
QH_CONTRACT_CLIP_I32 = 0
QH_CONTRACT_CLIP_I64 = 1
QH_CONTRACT_DIV_RINT = 2
QH_CONTRACT_FLOOR256_DIV_RINT = 3
QH_CONTRACT_ROUND_DIV = 4
QH_CONTRACT_U8_DRAIN = 5
QH_CONTRACT_NONE = 0xFFFFFFFF

# Packed weight carriers (qh_weight_carrier) and their flags.
CARRIERS = {
    "i8_kn": 0,
    "w8_kmajor": 1,
    "w8_kmajor_split128": 2,
    "w4_kmajor_n64": 3,
    "w4_kpair": 4,
    "w4_nmajor_kpair": 5,
    "w4_nmajor_k4": 6,
    "w4_kblock32_nmajor_k4": 7,
    "w4_npair_nmajor": 8,
    "w4_npair_tile32_nmajor": 9,
    "w4_full_codes": 10,
}
QH_CARRIER_XOR80 = 1
QH_CARRIER_HILO = 2
QH_CARRIER_BIASED = 4

QH_GDN_FP32 = 0
QH_GDN_BF16 = 1
QH_GDN_OP_MODEL = 2

QH_GDN_W_DECAY = 1
QH_GDN_OUT_F32 = 2
QH_GDN_WU_F32 = 4

# Every symbol include/qhtp.h declares (checked by the CPU test-suite).
EXPORTED = (
    "qh_status_string",
    "qh_last_error",
    "qh_version",
    "qh_qmm_prepare",
    "qh_qmm_run",
    "qh_qmm_run_path",
    "qh_qmm_accumulate",
    "qh_qmm_run_contract",
    "qh_qmm_run_chain",
    "qh_qmm_run_chain_noalloc",
    "qh_qmm_query",
    "qh_qmm_release",
    "qh_weight_unpack",
    "qh_w4_lpbq_expand_to_i8",
    "qh_gdn_solve_f32",
    "qh_gdn_solve_u16",
    "qh_gdn_chunk_uw",
    "qh_gdn_chunk_uw_ex",
    "qh_gdn_chunk_state",
)


class QhtpError(RuntimeError):
    """A libqhtp entry point returned a non-OK status."""

    def __init__(self, status: int, where: str, detail: str):
        self.status = status
        super().__init__(f"{where}: {status_name(status)}: {detail}")


class QmmDesc(C.Structure):
    _fields_ = [
        ("k", C.c_uint32),
        ("n", C.c_uint32),
        ("act_bits", C.c_uint32),
        ("out_bits", C.c_uint32),
        ("weight_format", C.c_uint32),
        ("lpbq_block", C.c_uint32),
        ("act_zp", C.c_int32),
        ("out_zp", C.c_int32),
        ("act_scale", C.c_double),
        ("out_scale", C.c_double),
        ("weight_nk", C.c_void_p),
        ("lpbq_block_scale", C.c_void_p),
        ("weight_scale", C.c_void_p),
        ("bias_q", C.c_void_p),
        ("group_scale", C.c_void_p),
        ("group_size", C.c_uint32),
        ("bias_float", C.c_void_p),
        ("weight16_nk", C.c_void_p),
    ]


class QmmInfo(C.Structure):
    _fields_ = [
        ("k", C.c_uint32),
        ("n", C.c_uint32),
        ("act_bits", C.c_uint32),
        ("out_bits", C.c_uint32),
        ("weight_format", C.c_uint32),
        ("lpbq_block", C.c_uint32),
        ("device_bytes", C.c_uint64),
        ("gemm_weight_bytes", C.c_uint64),
        ("gemv_weight_bytes", C.c_uint64),
    ]


_lock = threading.Lock()
_lib: C.CDLL | None = None


def _declare(L: C.CDLL) -> None:
    st = C.c_int
    vp = C.c_void_p
    u32 = C.c_uint32
    i32 = C.c_int32
    f32 = C.c_float
    L.qh_status_string.argtypes = [st]
    L.qh_status_string.restype = C.c_char_p
    L.qh_last_error.argtypes = []
    L.qh_last_error.restype = C.c_char_p
    L.qh_version.argtypes = []
    L.qh_version.restype = u32
    L.qh_qmm_prepare.argtypes = [C.POINTER(QmmDesc), C.POINTER(vp)]
    L.qh_qmm_prepare.restype = st
    L.qh_qmm_run.argtypes = [vp, u32, vp, vp, vp]
    L.qh_qmm_run.restype = st
    L.qh_qmm_run_path.argtypes = [vp, u32, vp, vp, u32, vp]
    L.qh_qmm_run_path.restype = st
    L.qh_qmm_accumulate.argtypes = [vp, u32, vp, vp, vp]
    L.qh_qmm_accumulate.restype = st
    L.qh_qmm_run_contract.argtypes = [vp, u32, vp, vp, u32, u32, vp]
    L.qh_qmm_run_contract.restype = st
    L.qh_qmm_run_chain.argtypes = [vp, u32, u32, vp, vp, vp, u32, u32, vp]
    L.qh_qmm_run_chain.restype = st
    L.qh_qmm_run_chain_noalloc.argtypes = [vp, u32, u32, vp, vp, u32, u32, vp]
    L.qh_qmm_run_chain_noalloc.restype = st
    L.qh_qmm_query.argtypes = [vp, C.POINTER(QmmInfo)]
    L.qh_qmm_query.restype = st
    L.qh_qmm_release.argtypes = [vp]
    L.qh_qmm_release.restype = st
    L.qh_weight_unpack.argtypes = [u32, u32, vp, C.c_size_t, u32, u32, vp]
    L.qh_weight_unpack.restype = st
    L.qh_w4_lpbq_expand_to_i8.argtypes = [vp, vp, vp, u32, u32, vp]
    L.qh_w4_lpbq_expand_to_i8.restype = st
    L.qh_gdn_solve_f32.argtypes = [vp, vp, u32, u32, u32, vp]
    L.qh_gdn_solve_f32.restype = st
    L.qh_gdn_solve_u16.argtypes = [vp, vp, u32, u32, i32, i32, f32, f32, u32, vp]
    L.qh_gdn_solve_u16.restype = st
    L.qh_gdn_chunk_uw.argtypes = [vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, vp]
    L.qh_gdn_chunk_uw.restype = st
    L.qh_gdn_chunk_uw_ex.argtypes = [vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, vp]
    L.qh_gdn_chunk_uw_ex.restype = st
    L.qh_gdn_chunk_state.argtypes = [vp, vp, vp, vp, vp, vp, vp, vp, u32, u32, u32, u32, u32, u32, u32, vp]
    L.qh_gdn_chunk_state.restype = st


def lib() -> C.CDLL:
    """The loaded libqhtp (raises if it has not been built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with `python -m qcom_htp_amd.build` "
                    "(there is no fallback path)"
                )
            L = C.CDLL(str(LIB_PATH))
            _declare(L)
            _lib = L
        return _lib


def status_name(status: int) -> str:
    try:
        return lib().qh_status_string(status).decode()
    except Exception:  # pragma: no cover - only when the library itself is unavailable
        return str(status)


def check(status: int, where: str) -> None:
    if status != QH_STATUS_OK:
        raise QhtpError(status, where, lib().qh_last_error().decode())
