"""CPU tests of the C ABI: the library loads, exports every declared symbol, and rejects
invalid arguments with a status (no GPU is touched on these paths)."""

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from qcom_htp_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "qhtp.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(qh_[a-z0-9_]+)\s*\(", text)))


def test_header_declarations_match_binding():
    assert declared_functions() == sorted(_lib.EXPORTED)


def test_library_exports_every_declared_symbol(qhtp_lib):
    for name in declared_functions():
        assert hasattr(qhtp_lib, name), name


def test_status_strings(qhtp_lib):
    names = [qhtp_lib.qh_status_string(i).decode() for i in range(5)]
    assert names == ["ok", "invalid_argument", "unsupported", "runtime_error", "shape_unsupported"]
    assert qhtp_lib.qh_status_string(99).decode() == "unknown"
    assert qhtp_lib.qh_version() >= 0x000100


def _desc(**kw):
    w = kw.pop("w", np.zeros((32, 64), np.int8))
    s = kw.pop("s", np.full(32, 0.01, np.float32))
    d = _lib.QmmDesc(k=w.shape[1], n=w.shape[0], act_bits=8, out_bits=8, weight_format=0, lpbq_block=0,
                     act_zp=128, out_zp=0, act_scale=0.02, out_scale=0.05,
                     weight_nk=w.ctypes.data, lpbq_block_scale=None, weight_scale=s.ctypes.data, bias_q=None)
    for k, v in kw.items():
        setattr(d, k, v)
    return d, (w, s)


@pytest.mark.parametrize(
    "field,value,status",
    [
        ("act_bits", 12, _lib.QH_STATUS_UNSUPPORTED),
        ("out_bits", 4, _lib.QH_STATUS_UNSUPPORTED),
        ("weight_format", 7, _lib.QH_STATUS_UNSUPPORTED),
        ("k", 48, _lib.QH_STATUS_SHAPE_UNSUPPORTED),
        ("n", 0, _lib.QH_STATUS_SHAPE_UNSUPPORTED),
        ("act_zp", 300, _lib.QH_STATUS_INVALID_ARGUMENT),
        ("out_scale", 0.0, _lib.QH_STATUS_INVALID_ARGUMENT),
        ("act_scale", float("nan"), _lib.QH_STATUS_INVALID_ARGUMENT),
        ("weight_nk", None, _lib.QH_STATUS_INVALID_ARGUMENT),
    ],
)
def test_prepare_rejects_invalid_descriptors(qhtp_lib, field, value, status):
    d, keep = _desc(**{field: value})
    h = C.c_void_p()
    assert qhtp_lib.qh_qmm_prepare(C.byref(d), C.byref(h)) == status
    assert h.value is None
    assert qhtp_lib.qh_last_error().decode() != ""


def test_prepare_rejects_out_of_range_codes(qhtp_lib):
    w = np.zeros((32, 64), np.int8)
    w[3, 5] = -128
    d, keep = _desc(w=w)
    h = C.c_void_p()
    assert qhtp_lib.qh_qmm_prepare(C.byref(d), C.byref(h)) == _lib.QH_STATUS_INVALID_ARGUMENT
    assert "outside" in qhtp_lib.qh_last_error().decode()
    w = np.full((32, 64), 8, np.int8)  # int4 codes must be within [-7, 7]
    d, keep = _desc(w=w, weight_format=_lib.QH_WEIGHT_I4)
    assert qhtp_lib.qh_qmm_prepare(C.byref(d), C.byref(h)) == _lib.QH_STATUS_INVALID_ARGUMENT


def test_prepare_rejects_bad_lpbq(qhtp_lib):
    w = np.zeros((32, 128), np.int8)
    blk = np.zeros((32, 4), np.uint8)  # factor 0 is outside [1, 16]
    d, keep = _desc(w=w, weight_format=_lib.QH_WEIGHT_I4_LPBQ, lpbq_block=32, lpbq_block_scale=blk.ctypes.data)
    h = C.c_void_p()
    assert qhtp_lib.qh_qmm_prepare(C.byref(d), C.byref(h)) == _lib.QH_STATUS_INVALID_ARGUMENT
    d, keep = _desc(w=w, weight_format=_lib.QH_WEIGHT_I4_LPBQ, lpbq_block=48, lpbq_block_scale=blk.ctypes.data)
    assert qhtp_lib.qh_qmm_prepare(C.byref(d), C.byref(h)) == _lib.QH_STATUS_UNSUPPORTED


def test_run_rejects_null_and_bad_shapes(qhtp_lib):
    L = qhtp_lib
    assert L.qh_qmm_run(None, 4, 16, 16, None) == _lib.QH_STATUS_INVALID_ARGUMENT
    assert L.qh_qmm_accumulate(None, 4, 16, 16, None) == _lib.QH_STATUS_INVALID_ARGUMENT
    assert L.qh_qmm_query(None, None) == _lib.QH_STATUS_INVALID_ARGUMENT
    assert L.qh_qmm_release(None) == _lib.QH_STATUS_OK
    # GDN: C not a multiple of 16 / too large / zero heads / NULL
    assert L.qh_gdn_solve_f32(16, 16, 1, 40, 0, None) == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert L.qh_gdn_solve_f32(16, 16, 1, 512, 0, None) == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert L.qh_gdn_solve_f32(16, 16, 0, 64, 0, None) == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert L.qh_gdn_solve_f32(None, 16, 1, 64, 0, None) == _lib.QH_STATUS_INVALID_ARGUMENT
    assert L.qh_gdn_solve_f32(16, 16, 1, 64, 5, None) == _lib.QH_STATUS_UNSUPPORTED
    assert L.qh_gdn_solve_u16(16, 16, 1, 64, 70000, 0, 1.0, 1.0, 0, None) == _lib.QH_STATUS_INVALID_ARGUMENT
    assert L.qh_gdn_solve_u16(16, 16, 1, 64, 0, 0, 0.0, 1.0, 0, None) == _lib.QH_STATUS_INVALID_ARGUMENT
    assert L.qh_gdn_solve_u16(8, 16, 1, 64, 0, 0, 1.0, 1.0, 0, None) == _lib.QH_STATUS_INVALID_ARGUMENT


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libqhtp.so")
    monkeypatch.setattr(_lib, "_lib", None)
    with pytest.raises(RuntimeError, match="no fallback"):
        _lib.lib()
