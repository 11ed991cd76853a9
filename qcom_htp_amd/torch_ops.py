"""``torch.ops.qhtp.*``: the hot paths as PyTorch custom operators.

The reference puts its kernels into graphs as QNN custom ops in the ``hmx`` domain, built by
its ONNX graph generator (example/qnn_hmx_matmul_common/gen_quant_chain.py:1234-1430) and
prepared once at graph finalize.  Here the same operations are registered with
``torch.library`` so that they can sit in a traced / compiled PyTorch program or a captured
HIP graph, each with a fake (meta) implementation for shape propagation:

=================================  ==================================================================
``qhtp::qmm(act, handle, path)``   one prepared quantized matmul (``QuantMatmul.__call__``)
``qhtp::qmm_contract``             the same with one of the reference's integer output contracts
``qhtp::qmm_chain``                ``chain`` identical matmuls, each output the next activation
``qhtp::qmm_accumulate``           the exact int64 accumulators
``qhtp::lpbq_expand_to_i8``        ``HmxW4LpbqExpandToI8`` (HmxW4LpbqExpandToI8Op.cpp:47-104)
``qhtp::gdn_solve``                T = (I - A)^-1 (fp32 / bf16-merge precision)
``qhtp::gdn_solve_u16``            the ``GdnSolve`` op's u16 code contract (GdnSolveOp.cpp:185-254)
``qhtp::gdn_chunk_uw``             the fused intra-chunk W, U products
``qhtp::gdn_chunk_state``          the chunk recurrence (stage B): o and the final state
``qhtp::gdn_prefill``              both stages, the reference's chunked ``gdn_kernel``
=================================  ==================================================================

A prepared matmul enters a graph as an integer handle (``register``): the weight re-layout is
prepare-time work, as in the reference, and the handle keeps the prepared state alive until
``unregister``.
"""

from __future__ import annotations

import itertools
import threading
from typing import Optional

import torch
from torch.library import custom_op

from .qmm import QuantMatmul

__all__ = ["register", "unregister", "prepared"]

_lock = threading.Lock()
_ids = itertools.count(1)
_registry: dict[int, QuantMatmul] = {}


def register(op: QuantMatmul) -> int:
    """Handle of a prepared matmul for the ``qhtp::qmm*`` operators."""
    with _lock:
        h = next(_ids)
        _registry[h] = op
    return h


def unregister(handle: int) -> None:
    with _lock:
        _registry.pop(handle, None)


def prepared(handle: int) -> QuantMatmul:
    try:
        return _registry[handle]
    except KeyError:
        raise KeyError(f"qhtp: no prepared matmul with handle {handle}") from None


# ------------------------------------------------------------------------------ quantized matmul


@custom_op("qhtp::qmm", mutates_args=())
def qmm(act: torch.Tensor, handle: int, path: int = 0) -> torch.Tensor:
    return prepared(handle)(act, path=path)


@qmm.register_fake
def _(act, handle, path=0):
    op = prepared(handle)
    return act.new_empty((act.shape[0], op.n), dtype=op.out_dtype)


@custom_op("qhtp::qmm_contract", mutates_args=())
def qmm_contract(act: torch.Tensor, handle: int, contract: int, divisor: int = 1) -> torch.Tensor:
    return prepared(handle).run_contract(act, contract, divisor)


@qmm_contract.register_fake
def _(act, handle, contract, divisor=1):
    op = prepared(handle)
    return act.new_empty((act.shape[0], op.n), dtype=op.out_dtype)


@custom_op("qhtp::qmm_chain", mutates_args=())
def qmm_chain(act: torch.Tensor, handle: int, chain: int, contract: int = -1, divisor: int = 1) -> torch.Tensor:
    return prepared(handle).chain(act, chain, None if contract < 0 else contract, divisor)


@qmm_chain.register_fake
def _(act, handle, chain, contract=-1, divisor=1):
    op = prepared(handle)
    return act.new_empty((act.shape[0], op.n), dtype=op.out_dtype)


@custom_op("qhtp::qmm_accumulate", mutates_args=())
def qmm_accumulate(act: torch.Tensor, handle: int) -> torch.Tensor:
    return prepared(handle).accumulate(act)


@qmm_accumulate.register_fake
def _(act, handle):
    return act.new_empty((act.shape[0], prepared(handle).n), dtype=torch.int64)


@custom_op("qhtp::lpbq_expand_to_i8", mutates_args=())
def lpbq_expand_to_i8(weight_lpbq: torch.Tensor, per_block_int_scale: torch.Tensor) -> torch.Tensor:
    from .ops import HmxW4LpbqExpandToI8

    return HmxW4LpbqExpandToI8(weight_lpbq, per_block_int_scale)


@lpbq_expand_to_i8.register_fake
def _(weight_lpbq, per_block_int_scale):
    return weight_lpbq.new_empty((1, 1, 2 * weight_lpbq.shape[-2], weight_lpbq.shape[-1]), dtype=torch.uint8)


# ------------------------------------------------------------------------------------------ GDN


@custom_op("qhtp::gdn_solve", mutates_args=())
def gdn_solve(A: torch.Tensor, precision: int = 0) -> torch.Tensor:
    from .gdn import gdn_solve as _solve

    return _solve(A, precision=precision)


@gdn_solve.register_fake
def _(A, precision=0):
    return torch.empty_like(A)


@custom_op("qhtp::gdn_solve_u16", mutates_args=())
def gdn_solve_u16(A_codes: torch.Tensor, zpA: int, sA: float, zpT: int, sT: float, precision: int = 0) -> torch.Tensor:
    from .gdn import GdnSolve

    return GdnSolve(A_codes, zpA, sA, zpT, sT, precision=precision)


@gdn_solve_u16.register_fake
def _(A_codes, zpA, sA, zpT, sT, precision=0):
    return torch.empty_like(A_codes)


@custom_op("qhtp::gdn_chunk_uw", mutates_args=())
def gdn_chunk_uw(k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor, chunk: int,
                 decay_w: bool = False, out_f32: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    from .gdn import gdn_chunk_uw as _uw

    return _uw(k, v, g, beta, chunk, decay_w=decay_w, out_dtype=torch.float32 if out_f32 else torch.bfloat16)


@gdn_chunk_uw.register_fake
def _(k, v, g, beta, chunk, decay_w=False, out_f32=False):
    dt = torch.float32 if out_f32 else torch.bfloat16
    return k.new_empty(k.shape, dtype=dt), k.new_empty(k.shape, dtype=dt)


@custom_op("qhtp::gdn_chunk_state", mutates_args=())
def gdn_chunk_state(q: torch.Tensor, k: torch.Tensor, g: torch.Tensor, w: torch.Tensor, u: torch.Tensor,
                    initial_state: Optional[torch.Tensor] = None, precision: int = 0,
                    out_f32: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    from .gdn import gdn_chunk_state as _state

    return _state(q, k, g, w, u, initial_state, precision, torch.float32 if out_f32 else torch.bfloat16)


@gdn_chunk_state.register_fake
def _(q, k, g, w, u, initial_state=None, precision=0, out_f32=False):
    B, T, H, D = q.shape
    return (q.new_empty(q.shape, dtype=torch.float32 if out_f32 else torch.bfloat16),
            q.new_empty((B, H, D, D), dtype=torch.float32))


@custom_op("qhtp::gdn_prefill", mutates_args=())
def gdn_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor, beta: torch.Tensor,
                initial_state: Optional[torch.Tensor] = None, precision: int = 0,
                out_f32: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    from .gdn import gdn_prefill as _prefill

    return _prefill(q, k, v, g, beta, initial_state, precision, torch.float32 if out_f32 else torch.bfloat16)


@gdn_prefill.register_fake
def _(q, k, v, g, beta, initial_state=None, precision=0, out_f32=False):
    B, T, H, D = q.shape
    return (q.new_empty(q.shape, dtype=torch.float32 if out_f32 else torch.bfloat16),
            q.new_empty((B, H, D, D), dtype=torch.float32))
