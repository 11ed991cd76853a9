"""The reference's op packages, by name, on MI355X.

Each class mirrors one QNN op package of the reference, with the same name, operand order
and weight carriers:

========================  ==========================================================  ========
op                        reference                                                   family
========================  ==========================================================  ========
``HmxU8I8ToU8MatMul``     example/qnn_hmx_matmul_u8i8/src/HmxU8I8ToU8MatMulOp.cpp      u8i8, W4A8 LPBQ
``HmxU8I4ToU8MatMul``     example/qnn_hmx_matmul_w4a8/src/HmxU8I4ToU8MatMulOp.cpp      W4A8
``HmxU16I8ToU16MatMul``   example/qnn_hmx_matmul_w8a16/src/HmxU16I8ToU16MatMulOp.cpp   W8A16, W4A16 LPBQ
``HmxU16I4ToU16MatMul``   example/qnn_hmx_matmul_w4a16/src/HmxU16I4ToU16MatMulOp.cpp   W4A16
``HmxW4LpbqExpandToI8``   example/qnn_hmx_matmul_common/HmxW4LpbqExpandToI8Op.cpp      LPBQ pre-op
``GdnSolve``              example/gdn_native/solve_op/src/GdnSolveOp.cpp               GDN
========================  ==========================================================  ========

The reference ops take ``bias[0], weight[1], activation[2], scratch[3] -> output[0]``, with
the quantisation parameters carried by the tensors' encodings, and do their precompute once
at graph prepare (HmxU8I8ToU8MatMulOp.cpp:162-193).  Here the op object is that prepared
state: it is built from the constant operands (``bias``, ``weight``) and the encodings, and
called on the activation.  ``weight`` is the reference's carrier (default: the stream the
reference op reads; any carrier of ``qh_weight_unpack`` via ``carrier=``), ``bias`` is the
int32 bias code per output channel, ``activation`` is ``[1, M/32, 32, K]`` (or ``[M, K]``)
and the output has the matching ``[1, M/32, 32, N]`` (or ``[M, N]``) shape.  The scratch
operand has no counterpart: the kernels allocate nothing per call.

The W4A8 / W4A16 LPBQ chains of the reference are
``HmxW4LpbqExpandToI8(weight_lpbq, scales) -> HmxU8I8ToU8MatMul / HmxU16I8ToU16MatMul``
(example/qnn_hmx_matmul_common/gen_quant_chain.py:1235-1260); the same two calls work here.
"""

from __future__ import annotations

import ctypes as C
from typing import Optional

import numpy as np
import torch

from . import _lib
from .gdn import GdnSolve
from .qmm import PATH_AUTO, QuantMatmul, _stream_ptr

__all__ = [
    "HmxU8I8ToU8MatMul",
    "HmxU8I4ToU8MatMul",
    "HmxU16I8ToU16MatMul",
    "HmxU16I4ToU16MatMul",
    "HmxW4LpbqExpandToI8",
    "GdnSolve",
    "unpack_weight",
    "carrier_shape",
]


def carrier_shape(carrier: str, k: int, n: int) -> tuple:
    """Trailing [R, C] shape of a carrier tensor for a K x N weight."""
    if carrier in ("i8_kn", "w8_kmajor", "w8_kmajor_split128", "w4_full_codes"):
        return (k, n)
    if carrier == "w4_kmajor_n64":
        return (k, n // 2)
    if carrier in ("w4_kpair", "w4_nmajor_kpair", "w4_nmajor_k4", "w4_kblock32_nmajor_k4"):
        return (k // 2, n)
    if carrier in ("w4_npair_nmajor", "w4_npair_tile32_nmajor"):
        return (n // 2, k)
    raise ValueError(f"unknown carrier {carrier!r}")


def _kn_from_shape(carrier: str, shape) -> tuple:
    if len(shape) < 2:
        raise ValueError(f"weight carrier needs at least 2 dims, got {tuple(shape)}")
    r, c = int(shape[-2]), int(shape[-1])
    if any(int(d) != 1 for d in shape[:-2]):
        raise ValueError(f"weight carrier leading dims must be 1, got {tuple(shape)}")
    if carrier in ("i8_kn", "w8_kmajor", "w8_kmajor_split128", "w4_full_codes"):
        return r, c
    if carrier == "w4_kmajor_n64":
        return r, 2 * c
    if carrier in ("w4_kpair", "w4_nmajor_kpair", "w4_nmajor_k4", "w4_kblock32_nmajor_k4"):
        return 2 * r, c
    if carrier in ("w4_npair_nmajor", "w4_npair_tile32_nmajor"):
        return c, 2 * r
    raise ValueError(f"unknown carrier {carrier!r}")


def _host_bytes(x) -> np.ndarray:
    if isinstance(x, torch.Tensor):
        x = x.detach().cpu().numpy()
    a = np.ascontiguousarray(x)
    return a.reshape(-1).view(np.uint8) if a.dtype.itemsize == 1 else None


def unpack_weight(weight, carrier: str, flags: int = 0) -> np.ndarray:
    """Logical int8 codes [N, K] of a carrier tensor (``qh_weight_unpack``; host work)."""
    if carrier not in _lib.CARRIERS:
        raise ValueError(f"unknown carrier {carrier!r}")
    shape = tuple(weight.shape)
    k, n = _kn_from_shape(carrier, shape)
    raw = _host_bytes(weight)
    if raw is None:
        raise TypeError("weight carrier must have a 1-byte dtype (uint8 / int8)")
    out = np.empty((n, k), dtype=np.int8)
    st = _lib.lib().qh_weight_unpack(_lib.CARRIERS[carrier], int(flags), raw.ctypes.data, raw.size, k, n,
                                     out.ctypes.data)
    _lib.check(st, "qh_weight_unpack")
    return out


def HmxW4LpbqExpandToI8(weight_lpbq: torch.Tensor, per_block_int_scale: torch.Tensor,
                        out: Optional[torch.Tensor] = None,
                        stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """[1, 1, K/2, N] K-pair int4 bytes x [1, 1, 1, N*K/32] uint8 scales -> [1, 1, K, N] uint8
    (int8 values in the 32x32 K-major tile stream), on the device."""
    for name, x in (("weight_lpbq", weight_lpbq), ("per_block_int_scale", per_block_int_scale)):
        if not isinstance(x, torch.Tensor) or x.device.type != "cuda" or x.dtype != torch.uint8 or not x.is_contiguous():
            raise TypeError(f"{name} must be a contiguous uint8 CUDA tensor")
    k2, n = int(weight_lpbq.shape[-2]), int(weight_lpbq.shape[-1])
    k = 2 * k2
    if k % 32 or n % 32:
        raise ValueError(f"LPBQ expand needs K and N multiples of 32, got K={k} N={n}")
    if per_block_int_scale.numel() != n * (k // 32):
        raise ValueError(f"per_block_int_scale has {per_block_int_scale.numel()} entries, want N*K/32 = {n * (k // 32)}")
    if out is None:
        out = torch.empty((1, 1, k, n), dtype=torch.uint8, device=weight_lpbq.device)
    elif out.dtype != torch.uint8 or out.numel() != k * n or not out.is_contiguous():
        raise ValueError("bad output tensor")
    st = _lib.lib().qh_w4_lpbq_expand_to_i8(weight_lpbq.data_ptr(), per_block_int_scale.data_ptr(), out.data_ptr(),
                                            k, n, _stream_ptr(stream))
    _lib.check(st, "qh_w4_lpbq_expand_to_i8")
    return out


class _HmxMatMul:
    act_bits = 8
    out_bits = 8
    weight_bits = 8
    default_carrier = "w8_kmajor"

    def __init__(self, bias, weight, *, weight_scale, act_scale: float, act_zp: int, out_scale: float, out_zp: int,
                 carrier: Optional[str] = None, carrier_flags: int = 0, device=None):
        carrier = carrier or self.default_carrier
        if _lib.CARRIERS.get(carrier) is None:
            raise ValueError(f"unknown carrier {carrier!r}")
        is_w4 = carrier.startswith("w4_")
        if is_w4 != (self.weight_bits == 4):
            raise ValueError(f"{type(self).__name__} takes {self.weight_bits}-bit weights; carrier {carrier!r} is not")
        w_nk = unpack_weight(weight, carrier, carrier_flags)
        n, k = w_nk.shape
        s32 = np.asarray(weight_scale.detach().cpu().numpy() if isinstance(weight_scale, torch.Tensor) else weight_scale,
                         dtype=np.float32).reshape(-1)
        if s32.size == 1:
            s32 = np.full(n, s32[0], dtype=np.float32)
        b = None
        if bias is not None:
            b = np.asarray(bias.detach().cpu().numpy() if isinstance(bias, torch.Tensor) else bias).reshape(-1)
            if b.size != n:
                raise ValueError(f"bias has {b.size} entries, want N={n}")
            b = b.astype(np.int32)
        self.k, self.n, self.carrier = k, n, carrier
        self._op = QuantMatmul(
            w_nk, s32, b, act_bits=self.act_bits, out_bits=self.out_bits, act_scale=act_scale, out_scale=out_scale,
            act_zp=act_zp, out_zp=out_zp,
            weight_format=_lib.QH_WEIGHT_I4 if self.weight_bits == 4 else _lib.QH_WEIGHT_I8, device=device)

    def __call__(self, activation: torch.Tensor, out: Optional[torch.Tensor] = None, path: int = PATH_AUTO,
                 stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        if not isinstance(activation, torch.Tensor):
            raise TypeError("activation must be a CUDA (HIP) tensor")
        if activation.dim() == 4:
            if activation.shape[0] != 1 or activation.shape[2] != 32 or activation.shape[3] != self.k:
                raise ValueError(f"activation must be [1, M/32, 32, {self.k}], got {tuple(activation.shape)}")
            rows = activation.shape[1] * 32
            out_shape = (1, activation.shape[1], 32, self.n)
        elif activation.dim() == 2:
            rows = activation.shape[0]
            out_shape = (rows, self.n)
        else:
            raise ValueError(f"activation must be [1, M/32, 32, K] or [M, K], got {tuple(activation.shape)}")
        flat_out = None
        if out is not None:
            if tuple(out.shape) != out_shape:
                raise ValueError(f"output must be {out_shape}, got {tuple(out.shape)}")
            flat_out = out.view(rows, self.n)
        res = self._op(activation.view(rows, self.k), out=flat_out, path=path, stream=stream)
        return res.view(out_shape)

    def close(self) -> None:
        self._op.close()


class HmxU8I8ToU8MatMul(_HmxMatMul):
    """uint8 activations x int8 weights -> uint8 (also the W4A8 LPBQ chain's matmul)."""


class HmxU8I4ToU8MatMul(_HmxMatMul):
    """uint8 activations x int4 weights -> uint8; default carrier: the W4 MatMul stream."""

    weight_bits = 4
    default_carrier = "w4_kmajor_n64"


class HmxU16I8ToU16MatMul(_HmxMatMul):
    """uint16 activations x int8 weights -> uint16 (also the W4A16 LPBQ chain's matmul)."""

    act_bits = 16
    out_bits = 16


class HmxU16I4ToU16MatMul(_HmxMatMul):
    """uint16 activations x int4 weights -> uint16; default carrier: the K32-block K4 stream."""

    act_bits = 16
    out_bits = 16
    weight_bits = 4
    default_carrier = "w4_kblock32_nmajor_k4"
