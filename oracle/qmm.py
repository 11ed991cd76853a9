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
* ``contract_output``  -- the integer output contracts above on an exact accumulator, one
  function (legacy clip in int32 arithmetic, int64 clip, native ``rint(acc / qmax + zp)``
  with and without the floor-256 step, round-half-away division).
* ``split_int16`` / ``w16a16_accumulator`` -- the W16A16 = two W8A16 passes identity,
  scripts/verify_w16a16_two_w8a16.py:21-57 (q16 = 256 hi + lo, hi signed, lo unsigned).

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
  +-(7q+3), +-(7q+4) ties) in tests/test_oracle_qmm.py, and by exact-rational rounding
  (``fractions.Fraction``) and Python-integer brute force on small random inputs.
* ``contract_output``: pinned against ``reference_step`` / ``w4a8_lpbq_scalar`` /
  ``w4a16_lpbq_scalar_native`` on the same accumulators, against exact-rational rounding
  (odd divisors leave no ties) and against Python-integer loops with explicit int32 wrap.
* ``w16a16_accumulator``: pinned by Python-integer brute force and the byte-split identity.
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
    "contract_output",
    "round_div",
    "split_int16",
    "w16a16_accumulator",
    "CONTRACT_NAMES",
]


def _weight_deq(w_int_nk: np.ndarray, w_scale: np.ndarray) -> np.ndarray:
    """fl32(w_int * s32): the float32 product the reference stores as ``w_deq``.  ``w_scale``
    is per output channel [N], or per (channel, K-group) [N, G] for the per-group schema
    (generate_qnn_matmul_python_cases.py:406-410)."""
    s = np.asarray(w_scale, dtype=np.float32)
    if s.ndim == 2:
        k = w_int_nk.shape[1]
        return w_int_nk.astype(np.float32) * np.repeat(s, k // s.shape[1], axis=1)
    return w_int_nk.astype(np.float32) * s[:, None]


def dequantized_output(x_q, w_int_nk, w_scale, bias_q, act_scale, act_zp, bias_float=None):
    """float64 ``quant_real = x_deq @ w_deq.T + bias_deq`` (generate_qnn_matmul_python_cases.py:447-473).
    Per-channel scales: ``bias_deq = bias_q * fl64(sA * s32)``; per-group scales: ``bias_deq``
    is the float bias (:460-470)."""
    s = np.asarray(w_scale, dtype=np.float32)
    if s.ndim == 2:
        n = s.shape[0]
        bias_deq = (np.zeros(n) if bias_float is None else np.asarray(bias_float, dtype=np.float32).astype(np.float64))
    else:
        bias_scale = act_scale * s.astype(np.float64)
        bias_deq = np.asarray(bias_q).astype(np.float64) * bias_scale
    x_deq = (np.asarray(x_q).astype(np.float64) + (-act_zp)) * act_scale
    w_deq = _weight_deq(np.asarray(w_int_nk), w_scale)
    return x_deq @ w_deq.astype(np.float64).T + bias_deq


def expected_output(x_q, w_int_nk, w_scale, bias_q, act_scale, out_scale, act_zp, out_zp, out_bits, bias_float=None):
    """``output_ref_q`` of the reference (generate_qnn_matmul_python_cases.py:474-481)."""
    qr = dequantized_output(x_q, w_int_nk, w_scale, bias_q, act_scale, act_zp, bias_float)
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
        getattr(case, "bias_float", None),
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


CONTRACT_NAMES = ("clip_i32", "clip_i64", "div_rint", "floor256_div_rint", "round_div", "u8_drain")


def round_div(v, d: int):
    """Integer division rounding half away from zero: (|v| + d // 2) // d with v's sign (the
    round_div7 rule of HmxU16I4ToU16MatMulOp.cpp:520-524 for any divisor d)."""
    v = np.asarray(v, dtype=np.int64)
    h = d // 2
    return np.where(v >= 0, (v + h) // d, -((-v + h) // d))


def contract_output(acc, contract: str, divisor: int = 1, bias_q=None, out_zp: int = 0, out_bits: int = 8):
    """One of the reference's integer output contracts on an exact accumulator acc [M, N]
    (sum_k (a - zp) w_int):

    * clip_i32          -- clip((acc + bias) in int32 arithmetic, 0, qmax): numpy's int32 matmul
                           and add wrap modulo 2^32 (gen_quant_chain.py:991-995, legacy);
    * clip_i64          -- clip(acc + bias, 0, qmax) in int64 (hmx_w4a8_lpbq_scalar,
                           HmxU8I4ToU8MatMulOp.cpp:210-233, bias = its "effective" bias);
    * div_rint          -- clip(rint(float64(acc) / d + out_zp)) (gen_quant_chain.py:986-987);
    * floor256_div_rint -- the same after acc = floor(acc / 256) * 256 (:981-985);
    * round_div         -- clip(round_half_away(acc / d) + out_zp) (HmxU16I4ToU16MatMulOp.cpp:545-568);
    * u8_drain          -- clip(trunc(float64(acc + bias) * s / 512) + (b >> 7)), the closed-form A8
                           drain of scripts/reconstruct_hmx_u8_drain.py:10-16,153-156 (``_drain_to_u8``)
                           with acc taken at act_zp = 128; d packs s as IEEE half bits (low 16)
                           and the u16 baseline b (high 16).
    """
    acc = np.asarray(acc, dtype=np.int64)
    qmax = (1 << out_bits) - 1
    dtype = np.dtype("<u2") if out_bits == 16 else np.dtype("uint8")
    b = np.zeros(acc.shape[-1], np.int64) if bias_q is None else np.asarray(bias_q, dtype=np.int64)
    if contract == "clip_i32":
        v = (acc + b[None, :]).astype(np.int32)  # modulo 2^32, as numpy's int32 arithmetic
        return np.clip(v, 0, qmax).astype(dtype)
    if contract == "clip_i64":
        return np.clip(acc + b[None, :], 0, qmax).astype(dtype)
    if contract in ("div_rint", "floor256_div_rint"):
        if contract == "floor256_div_rint":
            acc = np.floor_divide(acc, 256) * 256
        y = acc.astype(np.float64) / float(divisor)
        return np.clip(np.rint(y + float(out_zp)), 0, qmax).astype(dtype)
    if contract == "round_div":
        return np.clip(round_div(acc, divisor) + out_zp, 0, qmax).astype(dtype)
    if contract == "u8_drain":
        scale = float(np.array([divisor & 0xFFFF], np.uint16).view(np.float16)[0])
        baseline = (divisor >> 16) & 0xFFFF
        scaled = np.trunc((acc + b[None, :]).astype(np.float64) * scale / 512.0).astype(np.int64)
        return np.clip(scaled + (baseline >> 7), 0, qmax).astype(dtype)
    raise ValueError(f"unknown contract {contract!r}")


def split_int16(q16):
    """q16 = 256 hi + lo with hi = q16 >> 8 (int8) and lo = q16 & 0xff (uint8)
    (scripts/verify_w16a16_two_w8a16.py:21-28)."""
    q = np.asarray(q16, dtype=np.int64)
    return q >> 8, q & 0xFF


def w16a16_accumulator(x_q, w16_nk, act_zp) -> np.ndarray:
    """Exact int64 sum_k (x - zp) q16 as the two 8-bit-weight passes, combined with x 256:
    (x - zp) @ hi * 256 + (x - zp) @ lo (scripts/verify_w16a16_two_w8a16.py:44-47)."""
    hi, lo = split_int16(w16_nk)
    a = np.asarray(x_q, dtype=np.int64) - act_zp
    return (a @ hi.T) * 256 + a @ lo.T
