"""Pins the carrier oracle (oracle/layouts.py) against the reference's own statements.

* Generator writers vs op-package readers: ``read(pack(w)) == w`` for the three W4 streams
  the reference's C++ ops decode (two independent statements of one layout each).
* The generator's W8 K-major packer of the logical LPBQ expansion vs the C++ expand op's
  own tile writer, byte for byte (with saturating scales).
* Hand-derived positions: one nonzero code per carrier, located by working the reference's
  loops by hand; the test checks the only nonzero byte and its nibble.
* Structural identities the generator states (K32-block K4 = N-major K4 with the outer grid
  transposed; split128 = K-major at N = 128; N-major K-pair = transposed K-pair).
"""

import numpy as np
import pytest

from oracle import layouts as L

RNG = np.random.default_rng(20240611)


def w4(k, n):
    return RNG.integers(-8, 8, size=(k, n)).astype(np.int8)


@pytest.mark.parametrize("k,n", [(32, 64), (64, 128), (128, 192)])
def test_w4_matmul_stream_writer_matches_op_reader(k, n):
    w = w4(k, n)
    s = L.pack_w4_kmajor_n64(w)
    assert s.shape == (k, n // 2)
    assert np.array_equal(L.read_w4_kmajor_n64(s, k, n), w)


@pytest.mark.parametrize("k,n", [(32, 32), (64, 96), (128, 64)])
def test_w4_kblock32_k4_writer_matches_op_reader(k, n):
    w = w4(k, n)
    s = L.pack_w4_kblock32_nmajor_k4(w)
    assert s.shape == (k // 2, n)
    assert np.array_equal(L.read_w4_kblock32_nmajor_k4(s, k, n), w)


@pytest.mark.parametrize("k,n", [(2, 3), (32, 32), (96, 64)])
def test_w4_kpair_writer_matches_expand_reader(k, n):
    w = w4(k, n)
    s = L.pack_w4_kpair(w)
    assert np.array_equal(L.read_w4_kpair(s, k, n), w)


def test_reader_rejects_a_swapped_nibble_order():
    # the "hilo" byte order is a different stream: the op reader must not decode it as w
    w = w4(64, 128)
    assert not np.array_equal(L.read_w4_kmajor_n64(L.pack_w4_kmajor_n64(w, order="hilo"), 64, 128), w)


@pytest.mark.parametrize("k,n,hi", [(32, 32, 16), (64, 96, 16), (128, 64, 255)])
def test_expand_op_matches_generator_pack_of_logical_expansion(k, n, hi):
    codes = w4(k, n)
    scales = RNG.integers(0 if hi > 16 else 1, hi + 1, size=(n, k // 32)).astype(np.uint8)
    op = L.lpbq_expand_to_i8(L.pack_w4_kpair(codes), scales.reshape(-1), k, n)
    gen = L.pack_w8_kmajor(L.expand_lpbq_logical_kn(codes, scales, 32))
    assert np.array_equal(op, gen)
    if hi > 16:  # saturation is exercised
        lg = L.expand_lpbq_logical_kn(codes, scales, 32)
        assert (lg == 127).any() and (lg == -128).any()


def one_hot(k, n, kk, nn, v):
    w = np.zeros((k, n), np.int8)
    w[kk, nn] = v
    return w


def only_nonzero(stream):
    s = np.asarray(stream, dtype=np.uint8).reshape(-1)
    nz = np.flatnonzero(s)
    assert nz.size == 1, nz
    return int(nz[0]), int(s[nz[0]])


# (packer, K, N, k, n, byte, value) -- byte offsets worked out by hand from the reference loops
HAND = [
    ("w4_kmajor_n64", 64, 128, 5, 33, 133, 0x30),       # kt 0, kg 1, kr 1, nb 0, n%32 1, high nibble
    ("w4_kmajor_n64", 64, 128, 37, 70, 1024 * 3 + 128 + 24 + 1, 0x03),  # kt 1 nb 1 -> tile 3; n%64 = 6 low
    ("w8_kmajor", 64, 96, 37, 70, 5 * 1024 + 128 + 24 + 1, 0x03),       # tile (1, 2) = 5, r 5, c 6
    ("w8_kmajor_split128", 32, 256, 2, 130, 32 * 128 + 2 * 4 + 2, 0x03),  # slice 1, r 2, c 2
    ("w4_kpair", 64, 32, 3, 5, 32 + 5, 0x30),            # row k/2 = 1, odd k -> high
    ("w4_nmajor_kpair", 64, 32, 3, 5, 5 * 32 + 1, 0x30),  # memory [N][K/2]
    ("w4_nmajor_k4", 64, 64, 13, 40, ((1 * 8 + 1) * 32 + 8) * 4 + 1, 0x30),  # nt 1, kg 1, c 8, k%8 = 5
    ("w4_kblock32_nmajor_k4", 64, 64, 45, 40, (((1 * 2 + 1) * 4 + 1) * 32 + 8) * 4 + 1, 0x30),
    ("w4_npair_nmajor", 64, 32, 10, 7, 3 * 64 + 10, 0x30),   # pair row 3, odd channel -> high
    ("w4_npair_tile32_nmajor", 64, 128, 10, 100, (32 + 4) * 64 + 10, 0x30),  # nb 1, nc 36 -> high
    ("w4_full_codes", 32, 32, 7, 9, 7 * 32 + 9, 0x03),
    ("i8_kn", 32, 32, 7, 9, 7 * 32 + 9, 0x03),
]


@pytest.mark.parametrize("name,K,N,k,n,byte,value", HAND)
def test_hand_derived_positions(name, K, N, k, n, byte, value):
    pack, _ = L.PACKERS[name]
    got = only_nonzero(pack(one_hot(K, N, k, n, 3)))
    assert got == (byte, value)


def test_kblock32_order_is_nmajor_k4_with_outer_grid_transposed():
    k, n = 96, 64
    w = w4(k, n)
    a = L.pack_w4_nmajor_k4(w).reshape(n // 32, k // 32, 512)
    b = L.pack_w4_kblock32_nmajor_k4(w).reshape(k // 32, n // 32, 512)
    assert np.array_equal(a.transpose(1, 0, 2), b)


def test_split128_and_nmajor_kpair_identities():
    w8 = RNG.integers(-128, 128, size=(64, 128)).astype(np.int8)
    assert np.array_equal(L.pack_w8_kmajor_split128(w8), L.pack_w8_kmajor(w8))
    w = w4(64, 96)
    assert np.array_equal(L.pack_w4_nmajor_kpair(w).reshape(96, 32), L.pack_w4_kpair(w).T)


def test_encodings_and_carrier_toggle():
    w = np.arange(-8, 8, dtype=np.int8).reshape(1, 16)
    assert np.array_equal(L.int4_twos(L.nibbles(w)), w)
    assert np.array_equal(L.nibbles(w, "biased").astype(np.int16) - 8, w)
    s = np.arange(256, dtype=np.uint8)
    assert np.array_equal(L.carrier_xor80(L.carrier_xor80(s)), s)
    assert L.carrier_xor80(np.array([0x00, 0x7F, 0x80], np.uint8)).tolist() == [0x80, 0xFF, 0x00]
