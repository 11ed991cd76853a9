"""GDN / KDA chunk triangular solve T = (I - A)^-1 on MI355X.

Mirrors the reference's solve entry points:
* ``gdn_solve`` -- float32 A [..., C, C] -> T (the fp64 recurrence of
  scripts/gdn_ref_kernel.py:84-87, computed on the GPU in fp32 / bf16-MFMA);
* ``gdn_chunk_uw`` -- the fused intra-chunk products U = T (beta V), W = T (beta K^) [e^g] of
  scripts/gdn_ref_kernel.py:71-89 from bf16 keys / values, per-token log decays and betas;
* ``gdn_chunk_state`` -- the inter-chunk half (stage B: P, v_new, o and the state recurrence)
  of scripts/gdn_ref_kernel.py:91-101 over every chunk of a sequence;
* ``gdn_prefill`` -- both halves, the reference's ``gdn_kernel`` (scripts/gdn_ref_kernel.py:104-131);
* ``GdnSolve`` -- the quantized op contract of example/gdn_native/solve_op/src/GdnSolveOp.cpp
  (uint16 codes with zero point and scale on input and output), also the ``gdnbm_solve``
  I/O of example/gdn_native/baremetal/inc/gdnbm.idl:7-13.
"""

from __future__ import annotations

import contextlib
from typing import Optional

import torch

from . import _lib

FP32 = _lib.QH_GDN_FP32
BF16 = _lib.QH_GDN_BF16
OP_MODEL = _lib.QH_GDN_OP_MODEL  # GdnSolve only: the reference op's own codes (C <= 64)

W_DECAY = _lib.QH_GDN_W_DECAY

__all__ = ["gdn_solve", "gdn_chunk_uw", "gdn_chunk_state", "gdn_prefill", "GdnSolve", "FP32", "BF16", "OP_MODEL",
           "W_DECAY"]


def _stream(stream):
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _on(stream):
    """Context in which tensors are allocated (and torch work is queued) on the launch stream, so
    the caching allocator never hands a temporary to other streams' work while kernels on
    ``stream`` still read it."""
    return torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext()


def _same_device(device: torch.device, **tensors) -> None:
    for name, x in tensors.items():
        if x is not None and x.device != device:
            raise TypeError(f"{name} must be on {device}, got {x.device}")


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
        with _on(stream):
            out = torch.empty_like(A)
    st = _lib.lib().qh_gdn_solve_f32(A.data_ptr(), out.data_ptr(), heads, C, precision, _stream(stream))
    _lib.check(st, "qh_gdn_solve_f32")
    return out


def GdnSolve(A_codes: torch.Tensor, zpA: int, sA: float, zpT: int, sT: float, precision: int = FP32,
             out: Optional[torch.Tensor] = None, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
    """uint16 codes A [B, H, C, C] -> uint16 codes T (the GdnSolve op contract).  ``OP_MODEL``
    (C <= 64) returns the op's own codes exactly (gdn_solve_core.h:28-83)."""
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


def gdn_chunk_uw(k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor, chunk: int,
                 decay_w: bool = False, out_dtype: torch.dtype = torch.bfloat16,
                 stream: Optional[torch.cuda.Stream] = None, max_workgroups: int = 0):
    """(W, U) [B, T, H, 128] from k, v bf16 [B, T, H, 128] and g (per-token log decay), beta
    float32 [B, T, H]: U = T (beta v), W = T (beta l2norm(k)) [times e^g when decay_w], with
    T = (I - A)^-1 of each chunk of ``chunk`` tokens.  ``max_workgroups`` caps the persistent
    grid (0: every workgroup the device holds at once)."""
    for name, x, dt in (("k", k, torch.bfloat16), ("v", v, torch.bfloat16), ("g", g, torch.float32),
                        ("beta", beta, torch.float32)):
        if x.device.type != "cuda" or x.dtype != dt or not x.is_contiguous():
            raise TypeError(f"{name} must be a contiguous {dt} CUDA tensor")
    if k.dim() != 4 or v.shape != k.shape or g.shape != k.shape[:3] or beta.shape != k.shape[:3]:
        raise ValueError("k, v: [B, T, H, D]; g, beta: [B, T, H]")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("out_dtype must be bfloat16 or float32")
    _same_device(k.device, v=v, g=g, beta=beta)
    B, T, H, D = k.shape
    with _on(stream):
        w = torch.empty((B, T, H, D), dtype=out_dtype, device=k.device)
        u = torch.empty_like(w)
    flags = (W_DECAY if decay_w else 0) | (_lib.QH_GDN_OUT_F32 if out_dtype == torch.float32 else 0)
    st = _lib.lib().qh_gdn_chunk_uw_ex(k.data_ptr(), v.data_ptr(), g.data_ptr(), beta.data_ptr(), w.data_ptr(),
                                       u.data_ptr(), B, T, H, D, chunk, flags, int(max_workgroups), _stream(stream))
    _lib.check(st, "qh_gdn_chunk_uw")
    return w, u


STATE_CHUNK = 64  # the chunk of qh_gdn_chunk_state (the reference kernel unit, gdn_ref_kernel.py:24)


def gdn_chunk_state(q: torch.Tensor, k: torch.Tensor, g: torch.Tensor, w: torch.Tensor, u: torch.Tensor,
                    initial_state: Optional[torch.Tensor] = None, precision: int = FP32,
                    out_dtype: torch.dtype = torch.bfloat16, stream: Optional[torch.cuda.Stream] = None):
    """(o [B, T, H, 128], S [B, H, 128, 128] float32): the chunk recurrence over chunks of 64
    tokens from q, k bf16 [B, T, H, 128], the per-token log decays g float32 [B, T, H] and the
    stage-A outputs w, u [B, T, H, 128] (bf16 or float32; ``gdn_chunk_uw(..., 64, decay_w=True)``),
    starting from ``initial_state`` (float32 [B, H, 128, 128]; None = zero)."""
    for name, x in (("q", q), ("k", k)):
        if x.device.type != "cuda" or x.dtype != torch.bfloat16 or not x.is_contiguous():
            raise TypeError(f"{name} must be a contiguous bfloat16 CUDA tensor")
    if g.device.type != "cuda" or g.dtype != torch.float32 or not g.is_contiguous():
        raise TypeError("g must be a contiguous float32 CUDA tensor")
    if w.dtype != u.dtype or w.dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("w and u must both be bfloat16 or both float32")
    if not (w.is_contiguous() and u.is_contiguous()) or w.device.type != "cuda" or u.device.type != "cuda":
        raise TypeError("w and u must be contiguous CUDA tensors")
    if out_dtype not in (torch.bfloat16, torch.float32):
        raise TypeError("out_dtype must be bfloat16 or float32")
    if q.dim() != 4 or k.shape != q.shape or w.shape != q.shape or u.shape != q.shape or g.shape != q.shape[:3]:
        raise ValueError("q, k, w, u: [B, T, H, D]; g: [B, T, H]")
    B, T, H, D = q.shape
    if initial_state is not None:
        if (not isinstance(initial_state, torch.Tensor) or initial_state.dtype != torch.float32
                or not initial_state.is_contiguous() or tuple(initial_state.shape) != (B, H, D, D)):
            raise TypeError("initial_state must be a contiguous float32 [B, H, D, D] tensor")
    # every operand on q's device: a host tensor's address would be dereferenced by the kernel
    _same_device(q.device, k=k, g=g, w=w, u=u, initial_state=initial_state)
    with _on(stream):
        o = torch.empty((B, T, H, D), dtype=out_dtype, device=q.device)
        s_out = torch.empty((B, H, D, D), dtype=torch.float32, device=q.device)
    flags = (_lib.QH_GDN_WU_F32 if w.dtype == torch.float32 else 0) | (
        _lib.QH_GDN_OUT_F32 if out_dtype == torch.float32 else 0)
    st = _lib.lib().qh_gdn_chunk_state(q.data_ptr(), k.data_ptr(), g.data_ptr(), w.data_ptr(), u.data_ptr(),
                                       0 if initial_state is None else initial_state.data_ptr(), s_out.data_ptr(),
                                       o.data_ptr(), B, T, H, D, STATE_CHUNK, flags, precision, _stream(stream))
    _lib.check(st, "qh_gdn_chunk_state")
    return o, s_out


def gdn_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                initial_state: Optional[torch.Tensor] = None, precision: int = FP32,
                out_dtype: torch.dtype = torch.bfloat16, stream: Optional[torch.cuda.Stream] = None):
    """The chunked gated-delta-rule prefill, the reference's ``gdn_kernel``
    (scripts/gdn_ref_kernel.py:104-131): q, k, v bf16 [B, T, H, 128], g (per-token log decay) and
    beta float32 [B, T, H] -> (o [B, T, H, 128], S [B, H, 128, 128] float32).  T is zero-padded
    to whole chunks of 64, which leaves o and S unchanged.  Stage A runs with float32 W, U for
    ``FP32`` and bf16 for ``BF16``."""
    B, T, H, D = q.shape
    _same_device(q.device, k=k, v=v, g=g, beta=beta, initial_state=initial_state)
    # the padded inputs and the stage-A outputs are temporaries: allocated (and padded) on the
    # launch stream, so they stay reserved until the kernels queued there have read them
    with _on(stream):
        pad = (-T) % STATE_CHUNK
        if pad:
            F = torch.nn.functional
            q, k, v = (F.pad(x, (0, 0, 0, 0, 0, pad)).contiguous() for x in (q, k, v))
            g, beta = (F.pad(x, (0, 0, 0, pad)).contiguous() for x in (g, beta))
        wu_dtype = torch.float32 if precision == FP32 else torch.bfloat16
        w, u = gdn_chunk_uw(k, v, g, beta, STATE_CHUNK, decay_w=True, out_dtype=wu_dtype, stream=stream)
        o, s = gdn_chunk_state(q, k, g, w, u, initial_state, precision, out_dtype, stream)
        return (o[:, :T].contiguous() if pad else o), s
