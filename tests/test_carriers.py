"""qh_weight_unpack (host code of libqhtp) against the carrier oracle.

Bit-exact: every carrier x flag combination the generator can emit decodes back to the
logical codes the oracle packed.  No GPU is touched: the decode is prepare-time host work.
"""

import numpy as np
import pytest

from oracle import layouts as L
from qcom_htp_amd import _lib
from qcom_htp_amd.ops import carrier_shape, unpack_weight

RNG = np.random.default_rng(7)
W8 = [c for c, (_, bits) in L.PACKERS.items() if bits == 8]
W4 = [c for c, (_, bits) in L.PACKERS.items() if bits == 4]


def encode(carrier, w_kn, flags):
    pack, bits = L.PACKERS[carrier]
    kw = {}
    if bits == 4:
        kw = {"order": "hilo" if flags & _lib.QH_CARRIER_HILO else "lohi",
              "encoding": "biased" if flags & _lib.QH_CARRIER_BIASED else "twos"}
    s = pack(w_kn, **kw)
    if flags & _lib.QH_CARRIER_XOR80:
        s = L.carrier_xor80(s)
    k, n = w_kn.shape
    return np.ascontiguousarray(s).reshape(carrier_shape(carrier, k, n))


@pytest.mark.parametrize("k,n", [(64, 128), (96, 256)])
@pytest.mark.parametrize("flags", [0, _lib.QH_CARRIER_XOR80])
@pytest.mark.parametrize("carrier", W8)
def test_w8_carriers_round_trip(qhtp_lib, carrier, flags, k, n):
    w = RNG.integers(-128, 128, size=(k, n)).astype(np.int8)
    got = unpack_weight(encode(carrier, w, flags), carrier, flags)
    assert np.array_equal(got, w.T)


W4_FLAGS = [0, _lib.QH_CARRIER_XOR80, _lib.QH_CARRIER_HILO, _lib.QH_CARRIER_BIASED,
            _lib.QH_CARRIER_XOR80 | _lib.QH_CARRIER_HILO | _lib.QH_CARRIER_BIASED]


# the full-code carrier has one code per byte, hence no nibble order
W4_CASES = [(c, f) for c in W4 for f in W4_FLAGS if not (c == "w4_full_codes" and f & _lib.QH_CARRIER_HILO)]


@pytest.mark.parametrize("k,n", [(64, 128), (96, 256)])
@pytest.mark.parametrize("carrier,flags", W4_CASES)
def test_w4_carriers_round_trip(qhtp_lib, carrier, flags, k, n):
    w = RNG.integers(-8, 8, size=(k, n)).astype(np.int8)
    got = unpack_weight(encode(carrier, w, flags), carrier, flags)
    assert np.array_equal(got, w.T)


def test_reference_op_readers_agree_with_product_decode(qhtp_lib):
    # the op packages' own per-element readers, restated, on the same bytes
    k, n = 128, 192
    w = RNG.integers(-8, 8, size=(k, n)).astype(np.int8)
    s = L.pack_w4_kmajor_n64(w)
    assert np.array_equal(unpack_weight(s, "w4_kmajor_n64"), L.read_w4_kmajor_n64(s, k, n).T)
    s = L.pack_w4_kblock32_nmajor_k4(w)
    assert np.array_equal(unpack_weight(s, "w4_kblock32_nmajor_k4"), L.read_w4_kblock32_nmajor_k4(s, k, n).T)


def _call(lib, carrier, flags, buf, k, n):
    out = np.empty((n, k), np.int8)
    return lib.qh_weight_unpack(carrier, flags, buf.ctypes.data, buf.size, k, n, out.ctypes.data)


def test_unpack_rejects_bad_arguments(qhtp_lib):
    buf = np.zeros(64 * 128, np.uint8)
    c = _lib.CARRIERS
    assert _call(qhtp_lib, 99, 0, buf, 64, 128) == _lib.QH_STATUS_UNSUPPORTED
    assert _call(qhtp_lib, c["w8_kmajor"], 8, buf, 64, 128) == _lib.QH_STATUS_UNSUPPORTED
    assert _call(qhtp_lib, c["w8_kmajor"], _lib.QH_CARRIER_HILO, buf, 64, 128) == _lib.QH_STATUS_INVALID_ARGUMENT
    assert _call(qhtp_lib, c["w8_kmajor"], 0, buf, 48, 128) == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert _call(qhtp_lib, c["w8_kmajor_split128"], 0, buf[: 64 * 64], 64, 64) == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert _call(qhtp_lib, c["w4_kmajor_n64"], 0, buf[: 64 * 48], 64, 96) == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert _call(qhtp_lib, c["w4_kpair"], 0, buf, 64, 128) == _lib.QH_STATUS_INVALID_ARGUMENT  # 2x too many bytes
    assert "bytes" in qhtp_lib.qh_last_error().decode()
    assert _call(qhtp_lib, c["w4_kpair"], 0, buf[: 64 * 64], 64, 128) == _lib.QH_STATUS_OK
    bad = np.zeros(32 * 32, np.uint8)
    bad[5] = 0x10
    assert _call(qhtp_lib, c["w4_full_codes"], 0, bad, 32, 32) == _lib.QH_STATUS_INVALID_ARGUMENT
    out = np.empty((32, 32), np.int8)
    assert qhtp_lib.qh_weight_unpack(c["i8_kn"], 0, None, 0, 32, 32, out.ctypes.data) == _lib.QH_STATUS_INVALID_ARGUMENT


def test_carrier_shapes_follow_the_generator():
    k, n = 128, 256
    for carrier, (pack, bits) in L.PACKERS.items():
        w = np.zeros((k, n), np.int8)
        assert np.asarray(pack(w)).size == int(np.prod(carrier_shape(carrier, k, n))), carrier
