"""GDN / KDA chunk triangular solve T = (I - A)^-1 on MI355X.

Mirrors the reference's solve entry points:
* ``gdn_solve`` -- float32 A [..., C, C] -> T (the fp64 recurrence of
  scripts/gdn_ref_kernel.py:84-87, computed on the GPU in fp32 / bf16-MFMA);
* ``GdnSolve`` -- the quantized op contract of example/gdn_native/solve_op/src/GdnSolveOp.cpp
  (uint16 codes with zero point and scale on input and output), also the ``gdnbm_solve``
  I/O of example/gdn_native/baremetal/inc/gdnbm.idl:7-13.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _lib

FP32 = _lib.QH_GDN_FP32
BF16 = _lib.QH_GDN_BF16

__all__ = ["gdn_solve", "GdnSolve", "FP32", "BF16"]


def _stream(stream):
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def gdn_solve(A: torch.Tensor, precision: int = FP32, out: Optional[torch.Tensor] = None,
              stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """T = (I - A)^-1 for float32 A [..., C, C] (strictly lower triangle used)."""
    if A.device.type != "cuda" or A.dtype != torch.float32 or not A.is_contiguous():
        raise TypeError("A must be a contiguous float32 CUDA tensor")
    C = A.shape[-1]
    if A.shape[-2] != C:
        raise ValueError("A must be square in its last two dims")
    heads = A.numel() // (C * C)
    if out is None:
        out = torch.empty_like(A)
    st = _lib.lib().qh_gdn_solve_f32(A.data_ptr(), out.data_ptr(), heads, C, precision, _stream(stream))
    _lib.check(st, "qh_gdn_solve_f32")
    return out


def GdnSolve(A_codes: torch.Tensor, zpA: int, sA: float, zpT: int, sT: float, precision: int = FP32,
             out: Optional[torch.Tensor] = None, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """uint16 codes A [B, H, C, C] -> uint16 codes T (the GdnSolve op contract)."""
    if A_codes.device.type != "cuda" or A_codes.dtype != torch.uint16 or not A_codes.is_contiguous():
        raise TypeError("A_codes must be a contiguous uint16 CUDA tensor")
    C = A_codes.shape[-1]
    heads = A_codes.numel() // (C * C)
    if out is None:
        out = torch.empty_like(A_codes)
    st = _lib.lib().qh_gdn_solve_u16(A_codes.data_ptr(), out.data_ptr(), heads, C, int(zpA), int(zpT), float(sA),
                                     float(sT), precision, _stream(stream))
    _lib.check(st, "qh_gdn_solve_u16")
    return out
