"""Oracle for the QNN-semantics quantized matmul family -- TEST INFRASTRUCTURE ONLY.

Restates, on the CPU with numpy, what the reference computes for one quantized
matmul.  Only tests, ``smoke()`` and bench's ``cpu_baseline`` leg use it.

Functions and the reference lines they follow
---------------------------------------------
* ``expected_output``  -- ``quantize_case`` output half,
  scripts/generate_qnn_matmul_python_cases.py:446-481:
  ``output_ref_q = clip(rint((x_deq @ w_deq.T + bias_deq) / out_scale + out_zp))``
  with ``x_deq = (x_q - zp) * sA`` (float64), ``w_deq = fl32(w_int * s32)`` and
  ``bias_deq = bias_q * fl64(sA * s32)``.
* ``int_accumulator``  -- the integer accumulator contract
  ``acc = sum_k (a - zp) * w`` (scripts/reconstruct_hmx_u8_drain.py:10-16,
  example/qnn_hmx_matmul_w4a8/src/HmxU8I4ToU8MatMulOp.cpp:203-233).
* ``reference_step``   -- ``_make_reference_step`` legacy / native contracts,
  example/qnn_hmx_matmul_common/gen_quant_chain.py:971-996.
* ``w4a8_lpbq_scalar`` -- HmxU8I4ToU8MatMulOp.cpp:210-233 on logical arrays.
* ``w4a16_lpbq_scalar_native`` / ``round_div7`` -- HmxU16I4ToU16MatMulOp.cpp:514-568.

Pinning
-------
* ``expected_output``: pinned bit-for-bit against golden vectors written by the
  reference generator itself (tests/golden/qmm_small.npz, all 8 families x 7 cases at
  32x128x32, and the sha256 of ``output_q`` for every family x case at 256^3).
* ``int_accumulator``: pinned by brute-force int64 loops on small shapes and by the
  float64-exactness identity (|partial sums| < 2^53).
* ``reference_step``, ``w4a8_lpbq_scalar``, ``w4a16_lpbq_scalar_native``: pinned by
  closed-form special cases (zero activations at the zero point give the bias /
  the output zero point; single-k impulses give rank-1 products; round_div7 on
  +-(7q+3), +-(7q+4) ties) in tests/test_oracle_qmm.py.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "dequantized_output",
    "expected_output",
    "expected_output_case",
    "int_accumulator",
    "reference_step",
    "w4a8_lpbq_scalar",
    "round_div7",
    "w4a16_lpbq_scalar_native",
]


def _weight_deq(w_int_nk: np.ndarray, w_scale: np.ndarray) -> np.ndarray:
    """fl32(w_int * s32): the float32 product the reference stores as ``w_deq``."""
    return w_int_nk.astype(np.float32) * np.asarray(w_scale, dtype=np.float32)[:, None]


def dequantized_output(x_q, w_int_nk, w_scale, bias_q, act_scale, act_zp):
    """float64 ``quant_real = x_deq @ w_deq.T + bias_deq`` (generate_qnn_matmul_python_cases.py:447-473)."""
    bias_scale = act_scale * np.asarray(w_scale, dtype=np.float32).astype(np.float64)
    bias_deq = np.asarray(bias_q).astype(np.float64) * bias_scale
    x_deq = (np.asarray(x_q).astype(np.float64) + (-act_zp)) * act_scale
    w_deq = _weight_deq(np.asarray(w_int_nk), w_scale)
    return x_deq @ w_deq.astype(np.float64).T + bias_deq


def expected_output(x_q, w_int_nk, w_scale, bias_q, act_scale, out_scale, act_zp, out_zp, out_bits):
    """``output_ref_q`` of the reference (generate_qnn_matmul_python_cases.py:474-481)."""
    qr = dequantized_output(x_q, w_int_nk, w_scale, bias_q, act_scale, act_zp)
    qmax = (1 << out_bits) - 1
    q = np.rint(qr / out_scale - (-out_zp))
    dtype = np.dtype("<u2") if out_bits == 16 else np.dtype("uint8")
    return np.clip(q, 0, qmax).astype(dtype)


def _w_int(case):
    if getattr(case, "lpbq_expanded_q_nk", None) is not None:
        return case.lpbq_expanded_q_nk
    return case.weight_q_nk


def expected_output_case(case):
    """``expected_output`` for any object carrying the case attributes of ``QmmCase``."""
    fam = case.family
    return expected_output(
        case.activation_q,
        _w_int(case),
        case.weight_scale,
        case.bias_q,
        case.act_scale,
        case.out_scale,
        fam.act_zp,
        fam.out_zp,
        fam.out_bits,
    )


def int_accumulator(x_q, w_int_nk, act_zp) -> np.ndarray:
    """Exact int64 ``acc[m, n] = sum_k (x_q[m,k] - zp) * w[n,k]``.

    Evaluated as a float64 GEMM on integer-valued arrays: every partial sum is an
    integer below 2^53 in magnitude for K <= 2^20 (|a - zp| <= 2^15, |w| <= 2^7), so
    the float64 result is exact.
    """
    a = np.asarray(x_q).astype(np.float64) - act_zp
    w = np.asarray(w_int_nk).astype(np.float64)
    k = a.shape[1]
    bound = k * float(np.abs(a).max(initial=0)) * float(np.abs(w).max(initial=0))
    if bound >= 2.0 ** 53:
        raise ValueError("int_accumulator: float64 exactness bound exceeded")
    return (a @ w.T).astype(np.int64)


def reference_step(act_bits, weight_bits, out_bits, cur, w_raw_kn, bias_q, contract="legacy", family_name=""):
    """Integer reference contracts of gen_quant_chain._make_reference_step (:971-996).

    legacy : clip((cur - act_zp) @ w + bias, 0, qmax)
    native : A16 families only; W4A16 floors the accumulator to a multiple of 256
             before ``rint(acc / wqmax + 32768)``; W8A16 uses ``rint(acc / 127 + 32768)``.
    """
    max_out = (1 << out_bits) - 1
    out_dtype = np.dtype("<u2") if out_bits == 16 else np.dtype("uint8")
    if contract == "native":
        if act_bits != 16:
            raise ValueError("native reference contract is only valid for A16/U16 families")
        qmax = (1 << (weight_bits - 1)) - 1
        if family_name == "w4a16":
            acc = (cur.astype(np.int64) - 32768) @ w_raw_kn.astype(np.int64)
            acc = np.floor_divide(acc, 256) * 256
            y = acc.astype(np.float64) / float(qmax)
        else:
            y = ((cur.astype(np.float64) - 32768.0) @ w_raw_kn.astype(np.float64)) / float(qmax)
        return np.clip(np.rint(y + 32768.0), 0, max_out).astype(out_dtype)
    zp = 1 << (act_bits - 1)
    acc = (cur.astype(np.int64) - zp) @ w_raw_kn.astype(np.int64) + np.asarray(bias_q, dtype=np.int64)
    return np.clip(acc, 0, max_out).astype(out_dtype)


def w4a8_lpbq_scalar(effective_bias, w_kn, act_u8) -> np.ndarray:
    """Unit-scale W4A8 model: clamp(effective[n] + sum_k a_u8 * w[k, n], 0, 255).

    Follows hmx_w4a8_lpbq_scalar (HmxU8I4ToU8MatMulOp.cpp:210-233) on logical arrays;
    ``effective`` already folds ``-zp * sum_k w`` as the sidecar record does.
    """
    acc = act_u8.astype(np.int64) @ w_kn.astype(np.int64) + np.asarray(effective_bias, np.int64)[None, :]
    return np.clip(acc, 0, 255).astype(np.uint8)


def round_div7(v):
    """Integer division by 7 rounding half away from zero (HmxU16I4ToU16MatMulOp.cpp:520-524)."""
    v = np.asarray(v, dtype=np.int64)
    pos = (v + 3) // 7
    neg = -((-v + 3) // 7)
    return np.where(v >= 0, pos, neg)


def w4a16_lpbq_scalar_native(act_u16, w_kn) -> np.ndarray:
    """clip(round_div7(sum_k (a - 32768) * w) + 32768, 0, 65535) (:545-568)."""
    acc = (act_u16.astype(np.int64) - 32768) @ w_kn.astype(np.int64)
    return np.clip(round_div7(acc) + 32768, 0, 65535).astype(np.uint16)
