"""Oracle for the reference's packed weight carriers -- TEST INFRASTRUCTURE ONLY.

Restates, on the CPU with numpy, how the reference lays int8 / int4 weight codes out in
the byte streams its graph generator writes and its op packages read.  Only tests,
``smoke()`` and bench's ``cpu_baseline`` leg use it; the product decodes carriers in
``qh_weight_unpack`` (C++) and expands LPBQ weights in a HIP kernel.

Every array here is a logical weight ``w_kn[K, N]`` (K rows, N output channels, the
generator's ``w_raw_kn``) or a flat uint8 byte stream.

Functions and the reference lines they follow
---------------------------------------------
Writers (example/qnn_hmx_matmul_common/gen_quant_chain.py):

* ``nibbles``                  -- twos / biased nibble encodings, :622-625, :686-689.
* ``pack_w8_kmajor``           -- 32x32 K-major HMX W8 tiles, :285-303.
* ``pack_w8_kmajor_split128``  -- one K-major stream per 128 output channels, :306-314.
* ``pack_w4_kmajor_n64``       -- native W4 MatMul stream: 32x64 tiles of 1024 B, one byte
                                  holds channels n and n+32 of one k, :680-714.
* ``pack_w4_kpair``            -- native K-pair W4 [K/2, N], :369-382.
* ``pack_w4_nmajor_kpair``     -- the same bytes in N-major memory order, :385-398.
* ``pack_w4_nmajor_k4``        -- N32-tiled, K8-grouped k / k+4 pairs, :401-422.
* ``pack_w4_kblock32_nmajor_k4`` -- K32-block-major, then N32 tiles of k / k+4 pairs, :425-452.
* ``pack_w4_npair_nmajor``     -- adjacent output-channel pairs, [N/2, K], :455-468.
* ``pack_w4_npair_tile32_nmajor`` -- channel pairs n / n+32 per 64-column tile, [N/2, K], :471-489.
* ``pack_w4_full_codes``       -- one nibble code per byte, [K, N], :619-627.
* ``carrier_xor80``            -- the sign-bit toggle of the stored carrier, :645, :676, :716, :738.
* ``expand_lpbq_logical_kn``   -- sat_i8(code x block scale) on logical arrays, :333-350.

Readers (the op packages):

* ``read_w4_kmajor_n64``       -- example/qnn_hmx_matmul_w4a8/src/HmxU8I4ToU8MatMulOp.cpp:178-201.
* ``read_w4_kblock32_nmajor_k4`` -- example/qnn_hmx_matmul_w4a16/src/HmxU16I4ToU16MatMulOp.cpp:514-543.
* ``read_w4_kpair``            -- example/qnn_hmx_matmul_common/HmxW4LpbqExpandToI8Op.cpp:26-41.
* ``lpbq_expand_to_i8``        -- the HmxW4LpbqExpandToI8 kernel, HmxW4LpbqExpandToI8Op.cpp:47-104:
                                  K-pair int4 x per-block scale [N * K/32] -> saturated int8
                                  in the K-major W8 tile stream.

Pinning
-------
* ``pack_w4_kmajor_n64``, ``pack_w4_kpair``, ``pack_w4_kblock32_nmajor_k4`` are pinned
  against the op packages' own readers (writer from the generator, reader from the C++ op:
  two independent statements of one layout; a transposed index or a swapped nibble in
  either breaks ``read(pack(w)) == w``).
* ``pack_w8_kmajor`` and ``expand_lpbq_logical_kn`` are pinned against
  ``lpbq_expand_to_i8`` (the C++ op writes the K-major tile itself): the generator's
  ``pack_w8_kmajor(expand_lpbq_logical_kn(...))`` must equal the op's output byte for byte.
* Hand-derived positions (tests/test_oracle_layouts.py) fix single elements of every
  carrier, e.g. (k=5, n=33) of the W4 MatMul stream sits in byte 133, high nibble.
* ``pack_w4_nmajor_k4`` is pinned by the generator's own statement that the K32-block
  order holds the same 512-byte tile payloads with the outer grid transposed
  (gen_quant_chain.py:428-431); ``pack_w8_kmajor_split128`` equals ``pack_w8_kmajor`` at
  N = 128; ``pack_w4_nmajor_kpair`` is the transpose of ``pack_w4_kpair``.
* ``pack_w4_npair_nmajor``, ``pack_w4_npair_tile32_nmajor`` and ``pack_w4_full_codes``
  have no reader in the reference: they are pinned by the hand-derived positions only.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "nibbles",
    "int4_twos",
    "carrier_xor80",
    "pack_w8_kmajor",
    "pack_w8_kmajor_split128",
    "pack_w4_kmajor_n64",
    "pack_w4_kpair",
    "pack_w4_nmajor_kpair",
    "pack_w4_nmajor_k4",
    "pack_w4_kblock32_nmajor_k4",
    "pack_w4_npair_nmajor",
    "pack_w4_npair_tile32_nmajor",
    "pack_w4_full_codes",
    "expand_lpbq_logical_kn",
    "read_w4_kmajor_n64",
    "read_w4_kblock32_nmajor_k4",
    "read_w4_kpair",
    "lpbq_expand_to_i8",
    "PACKERS",
]


# ----------------------------------------------------------------------------- encodings
def nibbles(w_kn: np.ndarray, encoding: str = "twos") -> np.ndarray:
    """4-bit codes of int4 weights (gen_quant_chain.py:622-625): twos = w & 0xF, biased = (w+8) & 0xF."""
    w = np.asarray(w_kn)
    if encoding == "biased":
        return ((w.astype(np.int32) + 8) & 0x0F).astype(np.uint8)
    if encoding == "twos":
        return (w.astype(np.int8) & 0x0F).astype(np.uint8)
    raise ValueError(encoding)


def int4_twos(nib) -> np.ndarray:
    """Signed value of a twos-complement nibble (HmxU8I4ToU8MatMulOp.cpp:178-182)."""
    v = np.asarray(nib).astype(np.int16) & 0x0F
    return np.where(v < 8, v, v - 16).astype(np.int8)


def _byte(lo: np.ndarray, hi: np.ndarray, order: str) -> np.ndarray:
    if order == "lohi":
        return (lo | (hi << 4)).astype(np.uint8)
    if order == "hilo":
        return ((lo << 4) | hi).astype(np.uint8)
    raise ValueError(order)


def carrier_xor80(stream: np.ndarray) -> np.ndarray:
    """The stored carrier toggles every byte's sign bit (gen_quant_chain.py:716)."""
    return np.bitwise_xor(np.asarray(stream, dtype=np.uint8), np.uint8(0x80))


# ----------------------------------------------------------------------------- W8 writers
def pack_w8_kmajor(w_kn: np.ndarray) -> np.ndarray:
    """gen_quant_chain.py:285-303.  Tiles of 32 k x 32 n in (kt, nt) order; inside a tile,
    element (r, c) goes to byte (r // 4) * 128 + c * 4 + r % 4."""
    k, n = w_kn.shape
    if k % 32 or n % 32:
        raise ValueError("W8 K-major pack needs K and N multiples of 32")
    t = np.asarray(w_kn, dtype=np.int8).reshape(k // 32, 8, 4, n // 32, 32)  # kt, r/4, r%4, nt, c
    t = t.transpose(0, 3, 1, 4, 2)  # kt, nt, r/4, c, r%4
    return np.ascontiguousarray(t).reshape(-1).view(np.uint8)


def pack_w8_kmajor_split128(w_kn: np.ndarray) -> np.ndarray:
    """gen_quant_chain.py:306-314: the K-major stream of each 128-channel slice, concatenated."""
    k, n = w_kn.shape
    if n % 128:
        raise ValueError("split128 needs N multiple of 128")
    return np.concatenate([pack_w8_kmajor(w_kn[:, b:b + 128]) for b in range(0, n, 128)])


# ----------------------------------------------------------------------------- W4 writers
def pack_w4_kmajor_n64(w_kn: np.ndarray, order: str = "lohi", encoding: str = "twos") -> np.ndarray:
    """gen_quant_chain.py:680-714.  Per (kt, nb) a 1024-byte tile; byte kg*128 + nc*4 + kr
    holds k = 32 kt + 4 kg + kr for channels n = 64 nb + nc (low) and n + 32 (high).
    Returned as the runtime byte stream [K, N/2] (before the carrier toggle)."""
    k, n = w_kn.shape
    if k % 32 or n % 64:
        raise ValueError("W4 MatMul pack needs K multiple of 32 and N multiple of 64")
    nib = nibbles(w_kn, encoding).reshape(k // 32, 8, 4, n // 64, 2, 32)  # kt, kg, kr, nb, half, nc
    b = _byte(nib[:, :, :, :, 0, :], nib[:, :, :, :, 1, :], order)  # kt, kg, kr, nb, nc
    b = b.transpose(0, 3, 1, 4, 2)  # kt, nb, kg, nc, kr
    return np.ascontiguousarray(b).reshape(k, n // 2)


def pack_w4_kpair(w_kn: np.ndarray, order: str = "lohi", encoding: str = "twos") -> np.ndarray:
    """gen_quant_chain.py:369-382: byte (k/2, n) = nibble(k even) | nibble(k odd) << 4 for lohi."""
    k, n = w_kn.shape
    if k % 2:
        raise ValueError("K-pair pack needs even K")
    nib = nibbles(w_kn, encoding)
    return _byte(nib[0::2, :], nib[1::2, :], order)


def pack_w4_nmajor_kpair(w_kn: np.ndarray, order: str = "lohi", encoding: str = "twos") -> np.ndarray:
    """gen_quant_chain.py:385-398: the K-pair bytes in N-major memory order (shape [K/2, N],
    memory [N][K/2])."""
    k, n = w_kn.shape
    kp = pack_w4_kpair(w_kn, order, encoding)
    return np.ascontiguousarray(kp.T).reshape(k // 2, n)


def pack_w4_nmajor_k4(w_kn: np.ndarray, order: str = "lohi", encoding: str = "twos") -> np.ndarray:
    """gen_quant_chain.py:401-422: for each 32-channel tile, for each group of 8 k, for each
    channel, 4 bytes: k+kr (low) with k+kr+4 (high), kr = 0..3."""
    k, n = w_kn.shape
    if k % 8 or n % 32:
        raise ValueError("N-major K4 pack needs K multiple of 8 and N multiple of 32")
    nib = nibbles(w_kn, encoding).reshape(k // 8, 2, 4, n // 32, 32)  # kg, half, kr, nt, c
    b = _byte(nib[:, 0], nib[:, 1], order)  # kg, kr, nt, c
    b = b.transpose(2, 0, 3, 1)  # nt, kg, c, kr
    return np.ascontiguousarray(b).reshape(k // 2, n)


def pack_w4_kblock32_nmajor_k4(w_kn: np.ndarray, order: str = "lohi", encoding: str = "twos") -> np.ndarray:
    """gen_quant_chain.py:425-452: for each 32-k block, for each 32-channel tile, 512 bytes:
    4 groups of 8 k, 32 channels, 4 bytes (k+kr low, k+kr+4 high)."""
    k, n = w_kn.shape
    if k % 32 or n % 32:
        raise ValueError("K32-block K4 pack needs K and N multiples of 32")
    nib = nibbles(w_kn, encoding).reshape(k // 32, 4, 2, 4, n // 32, 32)  # kb, kg, half, kr, nt, c
    b = _byte(nib[:, :, 0], nib[:, :, 1], order)  # kb, kg, kr, nt, c
    b = b.transpose(0, 3, 1, 4, 2)  # kb, nt, kg, c, kr
    return np.ascontiguousarray(b).reshape(k // 2, n)


def pack_w4_npair_nmajor(w_kn: np.ndarray, order: str = "lohi", encoding: str = "twos") -> np.ndarray:
    """gen_quant_chain.py:455-468: byte (n/2, k) pairs channels n (even, low) and n+1 (high)."""
    k, n = w_kn.shape
    if n % 2:
        raise ValueError("N-pair pack needs even N")
    nib = nibbles(w_kn, encoding)
    return np.ascontiguousarray(_byte(nib[:, 0::2], nib[:, 1::2], order).T)


def pack_w4_npair_tile32_nmajor(w_kn: np.ndarray, order: str = "lohi", encoding: str = "twos") -> np.ndarray:
    """gen_quant_chain.py:471-489: row 32 nb + nc of [N/2, K] pairs channels 64 nb + nc (low)
    and 64 nb + nc + 32 (high)."""
    k, n = w_kn.shape
    if n % 64:
        raise ValueError("tile32 N-pair pack needs N multiple of 64")
    nib = nibbles(w_kn, encoding).reshape(k, n // 64, 2, 32)
    b = _byte(nib[:, :, 0, :], nib[:, :, 1, :], order)  # k, nb, nc
    return np.ascontiguousarray(b.reshape(k, n // 2).T)


def pack_w4_full_codes(w_kn: np.ndarray, encoding: str = "twos") -> np.ndarray:
    """gen_quant_chain.py:619-627: one 4-bit code per byte, logical [K, N]."""
    return nibbles(w_kn, encoding)


def expand_lpbq_logical_kn(codes_kn: np.ndarray, per_block_nb: np.ndarray, block: int) -> np.ndarray:
    """gen_quant_chain.py:333-350: sat_i8(code * scale[n, k // block]) on logical arrays."""
    k, n = codes_kn.shape
    if per_block_nb.shape != (n, k // block):
        raise ValueError("per-block scale shape mismatch")
    s = np.repeat(per_block_nb.astype(np.int16).T, block, axis=0)  # [K, N]
    return np.clip(codes_kn.astype(np.int16) * s, -128, 127).astype(np.int8)


# ----------------------------------------------------------------------------- readers
def read_w4_kmajor_n64(stream: np.ndarray, k: int, n: int) -> np.ndarray:
    """HmxU8I4ToU8MatMulOp.cpp:184-201 for every (k, n): byte
    (kt * N/64 + nb) * 1024 + kg * 128 + (n % 32) * 4 + kr, low nibble for n % 64 < 32."""
    s = np.asarray(stream, dtype=np.uint8).reshape(-1)
    kk, nn = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    kt, kin = kk // 32, kk & 31
    kg, kr = kin // 4, kin & 3
    nb, nin = nn // 64, nn & 63
    idx = (kt * (n // 64) + nb) * 1024 + kg * 128 + (nin & 31) * 4 + kr
    byte = s[idx]
    return int4_twos(np.where(nin < 32, byte, byte >> 4))


def read_w4_kblock32_nmajor_k4(stream: np.ndarray, k: int, n: int) -> np.ndarray:
    """HmxU16I4ToU16MatMulOp.cpp:526-543 for every (k, n): byte
    (((kb * N/32 + nt) * 4 + kg) * 32 + n % 32) * 4 + kr % 4, low nibble for kr < 4 (kr = k % 8)."""
    s = np.asarray(stream, dtype=np.uint8).reshape(-1)
    kk, nn = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    kb, kin = kk // 32, kk & 31
    kg, kr = kin // 8, kin & 7
    nt, nin = nn // 32, nn & 31
    idx = (((kb * (n // 32) + nt) * 4 + kg) * 32 + nin) * 4 + (kr & 3)
    byte = s[idx]
    return int4_twos(np.where(kr < 4, byte, byte >> 4))


def read_w4_kpair(stream: np.ndarray, k: int, n: int) -> np.ndarray:
    """HmxW4LpbqExpandToI8Op.cpp:35-41: byte (k >> 1) * N + n, low nibble for even k."""
    s = np.asarray(stream, dtype=np.uint8).reshape(-1)
    kk, nn = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    byte = s[(kk >> 1) * n + nn]
    return int4_twos(np.where((kk & 1) == 0, byte, byte >> 4))


def lpbq_expand_to_i8(compressed: np.ndarray, block_scale: np.ndarray, k: int, n: int) -> np.ndarray:
    """HmxW4LpbqExpandToI8Op.cpp:47-104: for every 32x32 tile (kt, nt) and element (r, c),
    q8 = sat_i8(q4(k, n) * scale[n * K/32 + kt]) written to byte
    (kt * N/32 + nt) * 1024 + (r / 4) * 128 + c * 4 + r % 4.  Returns the [K * N] byte stream."""
    if k % 32 or n % 32:
        raise ValueError("LPBQ expand needs K and N multiples of 32")
    q4 = read_w4_kpair(compressed, k, n).astype(np.int32)  # [K, N]
    sc = np.asarray(block_scale, dtype=np.uint8).reshape(-1)
    kk, nn = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    q8 = np.clip(q4 * sc[nn * (k // 32) + kk // 32].astype(np.int32), -128, 127).astype(np.int8)
    r, c = kk & 31, nn & 31
    dst = ((kk // 32) * (n // 32) + nn // 32) * 1024 + (r // 4) * 128 + c * 4 + (r & 3)
    out = np.empty(k * n, dtype=np.uint8)
    out[dst.reshape(-1)] = q8.reshape(-1).view(np.uint8)
    return out


#: carrier name -> (packer, weight bits); the names follow the generator's pack-order flags.
PACKERS = {
    "i8_kn": (lambda w, **_: np.asarray(w, dtype=np.int8).view(np.uint8).copy(), 8),
    "w8_kmajor": (lambda w, **_: pack_w8_kmajor(w), 8),
    "w8_kmajor_split128": (lambda w, **_: pack_w8_kmajor_split128(w), 8),
    "w4_kmajor_n64": (pack_w4_kmajor_n64, 4),
    "w4_kpair": (pack_w4_kpair, 4),
    "w4_nmajor_kpair": (pack_w4_nmajor_kpair, 4),
    "w4_nmajor_k4": (pack_w4_nmajor_k4, 4),
    "w4_kblock32_nmajor_k4": (pack_w4_kblock32_nmajor_k4, 4),
    "w4_npair_nmajor": (pack_w4_npair_nmajor, 4),
    "w4_npair_tile32_nmajor": (pack_w4_npair_tile32_nmajor, 4),
    "w4_full_codes": (lambda w, order="lohi", encoding="twos": pack_w4_full_codes(w, encoding), 4),
}
