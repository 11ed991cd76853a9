"""QNN-semantics quantized matmul on MI355X.

``QuantMatmul`` is the prepared op: construct it once from the weight codes and quantisation
parameters (the reference's graph-prepare / QHPI precompute), then call it on device
activations (the reference's hot op callback).  All arithmetic runs in libqhtp's HIP kernels;
this module only marshals arguments.

Family naming follows the reference (scripts/generate_qnn_matmul_python_cases.py:74-125):
u8i8, w4a8_per_channel, w4a8_lpbq, w8a16, w4a16_per_channel, w4a16_lpbq.
"""

from __future__ import annotations

import contextlib
import ctypes as C
from typing import Optional

import numpy as np
import torch

from . import _lib
from .cases import FAMILIES, Family, GraphCase, QmmCase

PATH_AUTO, PATH_GEMM, PATH_GEMV = 0, 1, 2

__all__ = ["QuantMatmul", "PATH_AUTO", "PATH_GEMM", "PATH_GEMV", "CONTRACTS", "weight_format_of", "graph_contract"]


def weight_format_of(family: Family) -> int:
    if family.weight_schema == "lpbq_blockwise_expansion":
        return _lib.QH_WEIGHT_I4_LPBQ
    if family.weight_schema == "per_group":
        return _lib.QH_WEIGHT_I4_GROUP
    if family.weight_schema != "per_output_channel":
        raise ValueError(f"{family.name}: weight schema {family.weight_schema!r} is not supported")
    return _lib.QH_WEIGHT_I8 if family.weight_bits == 8 else _lib.QH_WEIGHT_I4


# Integer output contracts of qh_qmm_run_contract (see include/qhtp.h).
CONTRACTS = {
    "clip_i32": _lib.QH_CONTRACT_CLIP_I32,
    "clip_i64": _lib.QH_CONTRACT_CLIP_I64,
    "div_rint": _lib.QH_CONTRACT_DIV_RINT,
    "floor256_div_rint": _lib.QH_CONTRACT_FLOOR256_DIV_RINT,
    "round_div": _lib.QH_CONTRACT_ROUND_DIV,
    "u8_drain": _lib.QH_CONTRACT_U8_DRAIN,
}


def graph_contract(gc: GraphCase) -> tuple:
    """(contract name, divisor) of qh_qmm_run_contract that is a graph's reference step
    (gen_quant_chain.py:971-996): legacy -> int32 clip with the bias; native W4A16 -> the
    accumulator floored to a multiple of 256, then rint(acc / 7 + 32768); other native A16 ->
    rint(acc / qmax + 32768) with qmax = 2^(weight bits - 1) - 1 (127 for W8A16, 32767 for W16A16)."""
    if gc.contract == "legacy":
        return "clip_i32", 1
    qmax = (1 << (gc.weight_bits - 1)) - 1
    if gc.kernel_family == "w4a16":
        return "floor256_div_rint", qmax
    return "div_rint", qmax


def _stream_ptr(stream: Optional[torch.cuda.Stream]) -> int:
    s = stream if stream is not None else torch.cuda.current_stream()
    return int(s.cuda_stream)


def _overlaps(a: Optional[torch.Tensor], b: Optional[torch.Tensor]) -> bool:
    """True if the byte ranges of two contiguous tensors overlap."""
    if a is None or b is None:
        return False
    pa, pb = a.data_ptr(), b.data_ptr()
    na, nb = a.numel() * a.element_size(), b.numel() * b.element_size()
    return pa < pb + nb and pb < pa + na


class QuantMatmul:
    """out[M,N] = clip(rint(((act - act_zp) sA) @ fl32(w_int s32).T + bias_deq) / sO + out_zp)).

    Parameters mirror the reference case (``case.json`` qparams): ``weight_q_nk`` int codes
    [N,K] (int16 for ``QH_WEIGHT_I16``); ``weight_scale`` float32 [N], or [N, K/group] group
    scales for the per-group schema; ``bias_q`` int32 [N] (``bias_float`` float32 [N] for the
    per-group schema); ``lpbq_block_scale`` uint8 [N, K/block] for LPBQ; activation/output bit
    widths, scales and zero points.
    """

    def __init__(
        self,
        weight_q_nk: np.ndarray,
        weight_scale: np.ndarray,
        bias_q: Optional[np.ndarray],
        *,
        act_bits: int,
        out_bits: int,
        act_scale: float,
        out_scale: float,
        act_zp: int,
        out_zp: int,
        weight_format: int,
        lpbq_block_scale: Optional[np.ndarray] = None,
        lpbq_block: int = 0,
        bias_float: Optional[np.ndarray] = None,
        device: Optional[torch.device] = None,
    ):
        i16 = weight_format == _lib.QH_WEIGHT_I16
        group = weight_format == _lib.QH_WEIGHT_I4_GROUP
        w = np.ascontiguousarray(weight_q_nk, dtype=np.int16 if i16 else np.int8)
        n, k = w.shape
        if group:
            gs = np.ascontiguousarray(weight_scale, dtype=np.float32)
            if gs.ndim != 2 or gs.shape[0] != n or k % gs.shape[1]:
                raise ValueError("per-group weight_scale must be [N, K / group_size]")
            s32 = None
        else:
            gs = None
            s32 = None if weight_scale is None else np.ascontiguousarray(weight_scale, dtype=np.float32).reshape(n)
        b = None if bias_q is None else np.ascontiguousarray(bias_q, dtype=np.int32).reshape(n)
        bf = None if bias_float is None else np.ascontiguousarray(bias_float, dtype=np.float32).reshape(n)
        blk = None
        if weight_format == _lib.QH_WEIGHT_I4_LPBQ:
            if lpbq_block_scale is None or lpbq_block not in (32, 64):
                raise ValueError("LPBQ needs lpbq_block_scale and lpbq_block in {32, 64}")
            blk = np.ascontiguousarray(lpbq_block_scale, dtype=np.uint8).reshape(n, k // lpbq_block)
        self.n, self.k = n, k
        self.act_bits, self.out_bits = act_bits, out_bits
        self.act_dtype = torch.uint16 if act_bits == 16 else torch.uint8
        self.out_dtype = torch.uint16 if out_bits == 16 else torch.uint8
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        desc = _lib.QmmDesc(
            k=k,
            n=n,
            act_bits=act_bits,
            out_bits=out_bits,
            weight_format=weight_format,
            lpbq_block=lpbq_block if blk is not None else 0,
            act_zp=int(act_zp),
            out_zp=int(out_zp),
            act_scale=float(act_scale),
            out_scale=float(out_scale),
            weight_nk=None if i16 else w.ctypes.data,
            lpbq_block_scale=blk.ctypes.data if blk is not None else None,
            weight_scale=s32.ctypes.data if s32 is not None else None,
            bias_q=b.ctypes.data if b is not None else None,
            group_scale=gs.ctypes.data if gs is not None else None,
            group_size=k // gs.shape[1] if gs is not None else 0,
            bias_float=bf.ctypes.data if bf is not None else None,
            weight16_nk=w.ctypes.data if i16 else None,
        )
        handle = C.c_void_p()
        L = _lib.lib()
        with torch.cuda.device(self.device):
            _lib.check(L.qh_qmm_prepare(C.byref(desc), C.byref(handle)), "qh_qmm_prepare")
        self._h = handle
        info = _lib.QmmInfo()
        _lib.check(L.qh_qmm_query(self._h, C.byref(info)), "qh_qmm_query")
        self.info = {f: getattr(info, f) for f, _ in _lib.QmmInfo._fields_}

    # ------------------------------------------------------------------ construction helpers
    @classmethod
    def from_case(cls, case: QmmCase, device=None) -> "QuantMatmul":
        fam = case.family
        fmt = weight_format_of(fam)
        return cls(
            case.weight_q_nk,
            case.weight_scale,
            case.bias_q,
            act_bits=fam.act_bits,
            out_bits=fam.out_bits,
            act_scale=case.act_scale,
            out_scale=case.out_scale,
            act_zp=fam.act_zp,
            out_zp=fam.out_zp,
            weight_format=fmt,
            lpbq_block_scale=case.lpbq_block_int_scale,
            lpbq_block=fam.lpbq_block_size if fmt == _lib.QH_WEIGHT_I4_LPBQ else 0,
            bias_float=getattr(case, "bias_float", None),
            device=device,
        )

    @classmethod
    def from_graph_case(cls, gc: GraphCase, device=None) -> "QuantMatmul":
        """The prepared op of one of the reference's CHAIN graphs (integer operands; the scales are
        unused by the integer contracts its outputs follow, so they are 1)."""
        n = gc.weight_kn.shape[1]
        if gc.weight_bits == 16:
            fmt = _lib.QH_WEIGHT_I16
        elif gc.lpbq_block_scale is not None:
            fmt = _lib.QH_WEIGHT_I4_LPBQ
        else:
            fmt = _lib.QH_WEIGHT_I8 if gc.weight_bits == 8 or gc.name == "u8i8" else _lib.QH_WEIGHT_I4
        return cls(
            np.ascontiguousarray(gc.weight_kn.T),
            np.ones(n, np.float32),
            gc.bias_q,
            act_bits=gc.act_bits,
            out_bits=gc.out_bits,
            act_scale=1.0,
            out_scale=1.0,
            act_zp=gc.act_zp,
            out_zp=gc.out_zp,
            weight_format=fmt,
            lpbq_block_scale=gc.lpbq_block_scale,
            lpbq_block=gc.lpbq_block,
            device=device,
        )

    # ------------------------------------------------------------------ execution
    def _check_act(self, act: torch.Tensor) -> int:
        if not isinstance(act, torch.Tensor) or act.device.type != "cuda":
            raise TypeError("activation must be a CUDA (HIP) tensor")
        if act.dtype != self.act_dtype:
            raise TypeError(f"activation dtype must be {self.act_dtype}, got {act.dtype}")
        if act.dim() != 2 or act.shape[1] != self.k or not act.is_contiguous():
            raise ValueError(f"activation must be contiguous [M, {self.k}], got {tuple(act.shape)}")
        return act.shape[0]

    def _check_out(self, out: torch.Tensor, m: int, device: torch.device, what: str) -> None:
        """A caller-supplied output (or chain scratch) buffer: [m, N] of the output dtype,
        contiguous, on the activation's device."""
        if not isinstance(out, torch.Tensor) or out.device != device:
            raise TypeError(f"{what} must be a tensor on {device}")
        if tuple(out.shape) != (m, self.n) or out.dtype != self.out_dtype or not out.is_contiguous():
            raise ValueError(f"{what} must be contiguous [{m}, {self.n}] {self.out_dtype}, got "
                             f"{tuple(out.shape)} {out.dtype}")

    def __call__(self, act: torch.Tensor, out: Optional[torch.Tensor] = None, path: int = PATH_AUTO,
                 stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        m = self._check_act(act)
        if out is None:
            out = torch.empty((m, self.n), dtype=self.out_dtype, device=act.device)
        else:
            self._check_out(out, m, act.device, "output")
            if _overlaps(act, out):
                raise ValueError("the activation must not overlap the output")
        st = _lib.lib().qh_qmm_run_path(self._h, m, act.data_ptr(), out.data_ptr(), path, _stream_ptr(stream))
        _lib.check(st, "qh_qmm_run")
        return out

    def accumulate(self, act: torch.Tensor, stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        """Exact int64 accumulators sum_k (act - act_zp) * w_int, [M, N]."""
        m = self._check_act(act)
        acc = torch.empty((m, self.n), dtype=torch.int64, device=act.device)
        st = _lib.lib().qh_qmm_accumulate(self._h, m, act.data_ptr(), acc.data_ptr(), _stream_ptr(stream))
        _lib.check(st, "qh_qmm_accumulate")
        return acc

    def run_contract(self, act: torch.Tensor, contract, divisor: int = 1, out: Optional[torch.Tensor] = None,
                     stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        """One of the reference's integer output contracts (``CONTRACTS`` name or id) applied to
        the exact integer dot product sum_k (act - act_zp) * w_int."""
        m = self._check_act(act)
        cid = CONTRACTS[contract] if isinstance(contract, str) else int(contract)
        if out is None:
            out = torch.empty((m, self.n), dtype=self.out_dtype, device=act.device)
        else:
            self._check_out(out, m, act.device, "output")
            if _overlaps(act, out):
                raise ValueError("the activation must not overlap the output")
        st = _lib.lib().qh_qmm_run_contract(self._h, m, act.data_ptr(), out.data_ptr(), cid, int(divisor),
                                            _stream_ptr(stream))
        _lib.check(st, "qh_qmm_run_contract")
        return out

    def chain(self, act: torch.Tensor, chain: int, contract=None, divisor: int = 1,
              out: Optional[torch.Tensor] = None, scratch: Optional[torch.Tensor] = None,
              stream: Optional[torch.cuda.Stream] = None) -> torch.Tensor:
        """``chain`` identical matmuls, each output the next activation (the reference's CHAIN
        graphs), with the float requantisation (``contract=None``) or an integer contract."""
        m = self._check_act(act)
        cid = _lib.QH_CONTRACT_NONE if contract is None else (CONTRACTS[contract] if isinstance(contract, str)
                                                               else int(contract))
        if int(chain) < 1:
            raise ValueError(f"chain must be >= 1, got {chain}")
        if out is None:
            out = torch.empty((m, self.n), dtype=self.out_dtype, device=act.device)
        else:
            self._check_out(out, m, act.device, "output")
        if scratch is None and chain > 1:
            # allocated on the launch stream, so the caching allocator cannot hand it to other
            # work on the current stream while the chain still uses it
            with torch.cuda.stream(stream) if stream is not None else contextlib.nullcontext():
                scratch = torch.empty_like(out)
        elif scratch is not None:
            self._check_out(scratch, m, act.device, "scratch")
        if chain > 1 and _overlaps(out, scratch):
            raise ValueError("out and scratch must not overlap")
        if _overlaps(act, out) or (chain > 1 and _overlaps(act, scratch)):
            raise ValueError("the activation must not overlap out or scratch")
        st = _lib.lib().qh_qmm_run_chain(self._h, m, int(chain), act.data_ptr(), out.data_ptr(),
                                         scratch.data_ptr() if scratch is not None else None, cid, int(divisor),
                                         _stream_ptr(stream))
        _lib.check(st, "qh_qmm_run_chain")
        return out

    def close(self) -> None:
        if getattr(self, "_h", None) and self._h.value:
            _lib.lib().qh_qmm_release(self._h)
            self._h = C.c_void_p()

    def __del__(self):  # pragma: no cover - best effort
        try:
            self.close()
        except Exception:
            pass


def family(name: str) -> Family:
    return FAMILIES[name]
