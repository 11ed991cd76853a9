"""Seeded case generators for the QNN-semantics quantized matmul family.

This module is the host-side *input* half of the reference's case generator
(``scripts/generate_qnn_matmul_python_cases.py``): it builds the float source
tensors of the seven named cases, derives the affine/symmetric quantisation
parameters, and quantises activations, weights and bias exactly the way the
reference does.  It does not compute expected outputs; the GPU kernels produce
outputs and the oracle under ``oracle/`` checks them.

Reference correspondence (file:line in the reference repository):

* ``Family`` / ``FAMILIES`` / ``CASES``  -> generate_qnn_matmul_python_cases.py:27-136
* ``affine_scale_from_minmax``           -> :174-182
* ``symmetric_scale_from_minmax``        -> :185-186
* ``lpbq_factorize_group_scales``        -> :189-200
* ``quantize_affine``                    -> :203-218 (``quantize_affine_aimet_qnn``)
* ``seed_for`` / ``make_float_case``     -> :225-285
* ``quantize_weight``                    -> :288-423 (vectorised over channels here)
* ``make_case``                          -> :426-481 (everything except the output GEMM)

The RNG draw order of ``make_float_case`` and the float32/float64 rounding steps of
the quantisers are part of the case definition, so they follow the reference
step for step; the loops over channels and blocks are vectorised.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Optional

import numpy as np

__all__ = [
    "Family",
    "FAMILIES",
    "CASES",
    "QmmCase",
    "seed_for",
    "make_float_case",
    "affine_scale_from_minmax",
    "symmetric_scale_from_minmax",
    "lpbq_factorize_group_scales",
    "quantize_affine",
    "quantize_weight",
    "make_case",
    "synthetic_case",
    "uniform_u8i8_case",
    "GraphCase",
    "GRAPH_FAMILIES",
    "W4A16_PRECISION_SUITE",
    "graph_activation",
    "graph_weight_kn",
    "graph_lpbq_block_scales",
    "graph_case",
]


@dataclass(frozen=True)
class Family:
    """Bit widths and weight schema of one matmul family."""

    name: str
    act_bits: int
    weight_bits: int
    out_bits: int
    weight_schema: str = "per_output_channel"
    kernel_family: Optional[str] = None
    lpbq_block_size: int = 32

    @property
    def act_zp(self) -> int:
        return 1 << (self.act_bits - 1)

    @property
    def out_zp(self) -> int:
        return 32768 if self.out_bits == 16 else 0

    @property
    def act_qmax(self) -> int:
        return (1 << self.act_bits) - 1

    @property
    def out_qmax(self) -> int:
        return (1 << self.out_bits) - 1

    @property
    def weight_qmax(self) -> int:
        return (1 << (self.weight_bits - 1)) - 1

    @property
    def weight_group_size(self) -> Optional[int]:
        return 64 if self.weight_schema == "per_group" else None

    @property
    def kernel_name(self) -> str:
        return self.kernel_family or self.name

    @property
    def is_lpbq(self) -> bool:
        return self.weight_schema == "lpbq_blockwise_expansion"

    @property
    def act_dtype(self) -> np.dtype:
        return np.dtype("<u2") if self.act_bits == 16 else np.dtype("uint8")

    @property
    def out_dtype(self) -> np.dtype:
        return np.dtype("<u2") if self.out_bits == 16 else np.dtype("uint8")


def _fam(name, a, w, o, schema="per_output_channel", kernel=None):
    return Family(name, act_bits=a, weight_bits=w, out_bits=o, weight_schema=schema, kernel_family=kernel)


FAMILIES = {
    "u8i8": _fam("u8i8", 8, 8, 8),
    "w4a8_per_channel": _fam("w4a8_per_channel", 8, 4, 8, "per_output_channel", "w4a8"),
    "w4a8_per_group": _fam("w4a8_per_group", 8, 4, 8, "per_group", "w4a8"),
    "w4a8_lpbq": _fam("w4a8_lpbq", 8, 4, 8, "lpbq_blockwise_expansion", "w4a8"),
    "w8a16": _fam("w8a16", 16, 8, 16),
    "w4a16_per_channel": _fam("w4a16_per_channel", 16, 4, 16, "per_output_channel", "w4a16"),
    "w4a16_per_group": _fam("w4a16_per_group", 16, 4, 16, "per_group", "w4a16"),
    "w4a16_lpbq": _fam("w4a16_lpbq", 16, 4, 16, "lpbq_blockwise_expansion", "w4a16"),
}

# The families of the reference's promoted gates (per-channel and LPBQ).  The per-group
# schema (K64 group scales, float bias: its bias contract is "not modelled" in the
# reference, generate_qnn_matmul_python_cases.py:460-470) is implemented too but is not part
# of that gated set.
PER_GROUP_FAMILIES = ("w4a8_per_group", "w4a16_per_group")
GATED_FAMILIES = (
    "u8i8",
    "w4a8_per_channel",
    "w4a8_lpbq",
    "w8a16",
    "w4a16_per_channel",
    "w4a16_lpbq",
)

CASES = (
    "normal_random",
    "zp_neutral",
    "positive_boundary",
    "negative_boundary",
    "single_k_impulse",
    "bias_only",
    "scale_only",
)


def seed_for(family: str, case: str) -> int:
    """Deterministic 32-bit seed per (family, case): a base-131 rolling hash of
    ``"family:case"`` started at 0x5EED (generate_qnn_matmul_python_cases.py:225-229)."""
    seed = 0x5EED
    for ch in f"{family}:{case}":
        seed = (seed * 131 + ord(ch)) & 0xFFFFFFFF
    return seed


def make_float_case(family: Family, case: str, m: int, k: int, n: int):
    """Float32 x[M,K], w[N,K], bias[N] of one named case.

    The draw sequence per case is fixed by the reference (:236-285): uniform draws of
    x, then w, then bias from ``default_rng(seed_for(...))``.
    """
    rng = np.random.default_rng(seed_for(family.name, case))
    ww = 1.0 if family.weight_bits == 8 else 0.75
    aw = 1.0 if family.act_bits == 16 else 0.85
    f32 = np.float32

    def uni(lo, hi, size):
        return rng.uniform(lo, hi, size=size).astype(f32)

    if case == "normal_random":
        return uni(-aw, aw, (m, k)), uni(-ww, ww, (n, k)), uni(-0.05, 0.05, n)
    if case == "zp_neutral":
        x = np.zeros((m, k), f32)
        return x, uni(-ww, ww, (n, k)), np.zeros(n, f32)
    if case == "positive_boundary":
        return uni(0.75 * aw, aw, (m, k)), uni(0.75 * ww, ww, (n, k)), uni(0.05, 0.15, n)
    if case == "negative_boundary":
        return uni(0.75 * aw, aw, (m, k)), uni(-ww, -0.75 * ww, (n, k)), uni(-0.15, -0.05, n)
    if case == "single_k_impulse":
        x = np.zeros((m, k), f32)
        x[:, 1 % k] = 0.25 * aw
        w = np.zeros((n, k), f32)
        w[:, 1 % k] = uni(-ww, ww, n)
        return x, w, np.zeros(n, f32)
    if case == "bias_only":
        return uni(-0.1 * aw, 0.1 * aw, (m, k)), uni(-0.1 * ww, 0.1 * ww, (n, k)), uni(-0.75, 0.75, n)
    if case == "scale_only":
        return uni(-3.0 * aw, 3.0 * aw, (m, k)), uni(-2.5 * ww, 2.5 * ww, (n, k)), np.zeros(n, f32)
    raise ValueError(f"unknown case: {case}")


def affine_scale_from_minmax(min_v: float, max_v: float, qmin: int, qmax: int, zp: int) -> float:
    """Scale of a fixed-zero-point affine grid covering [min_v, max_v]; floor 1e-12."""
    best = 1.0e-12
    if min_v < 0 and zp > qmin:
        best = max(best, (-min_v) / float(zp - qmin))
    if max_v > 0 and qmax > zp:
        best = max(best, max_v / float(qmax - zp))
    return best


def symmetric_scale_from_minmax(min_v, max_v, qmax: int):
    """max(|min|, |max|, 1e-12) / qmax; works elementwise on float64 arrays too."""
    return np.maximum(np.maximum(np.abs(min_v), np.abs(max_v)), 1.0e-12) / float(qmax)


def lpbq_factorize_group_scales(group_scales: np.ndarray, max_int_scale: int = 16):
    """Factor per-group scales (rows = channels) into base scale x integer factors.

    base = max(min_scale, max_scale / max_int_scale) per channel (float64);
    factor = clip(ceil(group/base - 1e-9), 1, max_int_scale) as uint8.
    Accepts [blocks] or [channels, blocks]; returns (base, factors) of matching rank.
    """
    if max_int_scale <= 0:
        raise ValueError(f"invalid LPBQ max_int_scale={max_int_scale}")
    gs = np.asarray(group_scales)
    squeeze = gs.ndim == 1
    gs2 = gs.reshape(1, -1) if squeeze else gs
    gmax = np.maximum(gs2.max(axis=1).astype(np.float64), 1.0e-12)
    gmin = np.maximum(gs2.min(axis=1).astype(np.float64), 1.0e-12)
    base = np.maximum(gmin, gmax / float(max_int_scale))
    factors = np.ceil(gs2.astype(np.float64) / base[:, None] - 1.0e-9)
    factors = np.clip(factors, 1, max_int_scale).astype(np.uint8)
    if squeeze:
        return float(base[0]), factors[0]
    return base, factors


def quantize_affine(values: np.ndarray, scale: float, qnn_offset: int, qmin: int, qmax: int, dtype) -> np.ndarray:
    """AIMET/QNN affine quantiser: clip(rint(x/scale - offset)), offset = -zero_point."""
    q = np.rint(values.astype(np.float64) / scale - qnn_offset)
    return np.clip(q, qmin, qmax).astype(dtype)


def _block_absmax_scale(w: np.ndarray, block: int, qmax: int) -> np.ndarray:
    """Symmetric scale of each K-block of each row, float64 [N, K/block]."""
    n, k = w.shape
    wb = w.reshape(n, k // block, block)
    return symmetric_scale_from_minmax(wb.min(axis=2).astype(np.float64), wb.max(axis=2).astype(np.float64), qmax)


def quantize_weight(family: Family, w: np.ndarray) -> dict[str, Any]:
    """Quantise float32 weight[N,K] under the family's weight schema.

    Returns a dict with ``q`` (int codes [N,K]), ``scale`` (float32 per channel, or
    [N, groups] for per-group), ``deq`` (float32 dequantised weight = fl32(q_eff * s32))
    and, for LPBQ, ``block_int_scale`` (uint8 [N, K/block]), ``expanded`` (int16
    q * factor) and ``pre_group_scale`` (float32 [N, K/block]).
    """
    n, k = w.shape
    qmax = family.weight_qmax
    q_dtype = np.int8 if qmax <= 127 else np.int16
    w64 = w.astype(np.float64)

    if family.weight_schema == "per_output_channel":
        scale = symmetric_scale_from_minmax(w.min(axis=1).astype(np.float64), w.max(axis=1).astype(np.float64), qmax)
        q = np.clip(np.rint(w64 / scale[:, None]), -qmax, qmax).astype(q_dtype)
        s32 = scale.astype(np.float32)
        deq = q.astype(np.float32) * s32[:, None]
        return {"q": q, "scale": s32, "deq": deq}

    if family.weight_schema == "lpbq_blockwise_expansion":
        bs = family.lpbq_block_size
        if k <= bs or k % bs:
            raise ValueError(f"{family.name}: LPBQ K={k} must be > {bs} and divisible by {bs}")
        nb = k // bs
        group = _block_absmax_scale(w, bs, qmax).astype(np.float32)
        base, factors = lpbq_factorize_group_scales(group)
        eff = base[:, None] * factors.astype(np.float64)  # float64 per (channel, block)
        eff_k = np.repeat(eff, bs, axis=1)
        q = np.clip(np.rint(w64 / eff_k), -qmax, qmax).astype(q_dtype)
        expanded = q.astype(np.int16) * np.repeat(factors, bs, axis=1).astype(np.int16)
        s32 = base.astype(np.float32)
        deq = expanded.astype(np.float32) * s32[:, None]
        return {
            "q": q,
            "scale": s32,
            "deq": deq,
            "block_int_scale": factors,
            "expanded": expanded,
            "pre_group_scale": group,
        }

    gsz = family.weight_group_size
    if gsz is None:
        raise ValueError(f"{family.name}: missing W4 group size")
    if k <= gsz or k % gsz:
        raise ValueError(f"{family.name}: W4 K={k} must be > {gsz} and divisible by {gsz}")
    scale = _block_absmax_scale(w, gsz, qmax)
    sk = np.repeat(scale, gsz, axis=1)
    q = np.clip(np.rint(w64 / sk), -qmax, qmax).astype(q_dtype)
    s32 = scale.astype(np.float32)
    deq = q.astype(np.float32) * np.repeat(s32, gsz, axis=1)
    return {"q": q, "scale": s32, "deq": deq}


@dataclass
class QmmCase:
    """Quantised operands and quantisation parameters of one matmul case.

    Mirrors the ``case.json`` + ``.npy`` set the reference generator writes
    (generate_qnn_matmul_python_cases.py:537-606) minus the expected output.
    """

    family: Family
    case: str
    m: int
    k: int
    n: int
    activation_q: np.ndarray  # [M,K] uint8 / uint16
    weight_q_nk: np.ndarray  # [N,K] int8 codes (int4 values for W4)
    weight_scale: np.ndarray  # float32 [N]
    bias_q: np.ndarray  # int32 [N]
    act_scale: float
    out_scale: float
    weight_deq: np.ndarray  # float32 [N,K] = fl32(q_eff * s32)
    lpbq_block_int_scale: Optional[np.ndarray] = None  # uint8 [N, K/block]
    lpbq_expanded_q_nk: Optional[np.ndarray] = None  # int16 [N,K]
    lpbq_pre_group_scale: Optional[np.ndarray] = None
    bias_float: Optional[np.ndarray] = None  # float32 [N]: the per-group schema's float bias
    seed: Optional[int] = None
    extra: dict = field(default_factory=dict)

    @property
    def act_zp(self) -> int:
        return self.family.act_zp

    @property
    def out_zp(self) -> int:
        return self.family.out_zp

    @property
    def weight_int_nk(self) -> np.ndarray:
        """Integer weight that multiplies the per-channel scale (expanded for LPBQ)."""
        if self.lpbq_expanded_q_nk is not None:
            return self.lpbq_expanded_q_nk
        return self.weight_q_nk


def make_case(family: Family | str, case: str, m: int, k: int, n: int) -> QmmCase:
    """Build one seeded case: float sources -> derived scales -> quantised operands.

    Follows ``quantize_case`` (generate_qnn_matmul_python_cases.py:426-481) up to but
    excluding the dequantised output GEMM.  The output scale is derived from the
    float64 product ``x @ w.T + bias`` of the float sources, as in the reference.
    """
    fam = FAMILIES[family] if isinstance(family, str) else family
    x, w, bias = make_float_case(fam, case, m, k, n)
    out_float = x.astype(np.float64) @ w.astype(np.float64).T + bias.astype(np.float64)
    act_scale = affine_scale_from_minmax(float(x.min()), float(x.max()), 0, fam.act_qmax, fam.act_zp)
    out_scale = affine_scale_from_minmax(float(out_float.min()), float(out_float.max()), 0, fam.out_qmax, fam.out_zp)
    x_q = quantize_affine(x, act_scale, -fam.act_zp, 0, fam.act_qmax, fam.act_dtype)
    wq = quantize_weight(fam, w)
    bias_float = None
    if wq["scale"].ndim == 1:
        bias_scale = act_scale * wq["scale"].astype(np.float64)
        bias_q = np.clip(np.rint(bias.astype(np.float64) / bias_scale), -(1 << 31), (1 << 31) - 1).astype(np.int32)
    else:
        # per-group scales: bias_q is all zeros and the float bias is added as it is (:460-470)
        bias_q = np.zeros(n, np.int32)
        bias_float = bias.astype(np.float32)
    return QmmCase(
        family=fam,
        case=case,
        m=m,
        k=k,
        n=n,
        activation_q=x_q,
        weight_q_nk=wq["q"],
        weight_scale=wq["scale"],
        bias_q=bias_q,
        act_scale=act_scale,
        out_scale=out_scale,
        weight_deq=wq["deq"],
        lpbq_block_int_scale=wq.get("block_int_scale"),
        lpbq_expanded_q_nk=wq.get("expanded"),
        lpbq_pre_group_scale=wq.get("pre_group_scale"),
        bias_float=bias_float,
        seed=seed_for(fam.name, case),
    )


def synthetic_case(
    family: Family | str,
    m: int,
    k: int,
    n: int,
    seed: int = 2,
    lpbq_block: int = 64,
    lpbq_max_scale: int = 15,
    out_scale: Optional[float] = None,
    calib_rows: int = 16,
) -> QmmCase:
    """Integer-domain synthetic operands for throughput runs at large shapes.

    * activations: uint8 ~ clip(rint(N(128, 40))), or uint16 ~ clip(rint(N(32768, 10000)));
      per-tensor scale 0.02 (A8) / 1e-4 (A16) with the family's fixed zero point;
    * weights: symmetric int4 in [-7, 7] (int8 in [-127, 127] for W8); LPBQ weights are
      int4 with ``lpbq_block``-wide K blocks carrying integer scales in [1, lpbq_max_scale];
    * per-output-channel float32 scales ~ U(1e-3, 1e-2); int32 bias ~ U(-2^15, 2^15);
    * per-group families: float32 scales ~ U(1e-3, 1e-2) per (channel, 64-k group) and a
      float32 bias ~ U(-0.5, 0.5) (the per-group schema's bias is the float bias itself).

    The output scale, unless given, is fitted (as the reference fits it from the float
    output range) to the exact dequantised output of the first ``calib_rows`` rows.
    """
    fam = FAMILIES[family] if isinstance(family, str) else family
    rng = np.random.default_rng(seed)
    if fam.act_bits == 8:
        x_q = np.clip(np.rint(rng.normal(128.0, 40.0, size=(m, k))), 0, 255).astype(np.uint8)
        act_scale = 0.02
    else:
        x_q = np.clip(np.rint(rng.normal(32768.0, 10000.0, size=(m, k))), 0, 65535).astype(np.uint16)
        act_scale = 1.0e-4
    qmax = fam.weight_qmax
    q = rng.integers(-qmax, qmax + 1, size=(n, k), dtype=np.int8)
    s32 = rng.uniform(1.0e-3, 1.0e-2, size=n).astype(np.float32)
    bias_q = rng.integers(-(1 << 15), (1 << 15) + 1, size=n).astype(np.int32)
    block_scale = None
    expanded = None
    bias_float = None
    w_int = q.astype(np.int16)
    if fam.weight_schema == "per_group":
        # per-(channel, 64-k group) float32 scales ~ U(1e-3, 1e-2); float bias ~ U(-0.5, 0.5)
        gsz = fam.weight_group_size
        if k % gsz:
            raise ValueError(f"K={k} must be a multiple of the group size {gsz}")
        s32 = rng.uniform(1.0e-3, 1.0e-2, size=(n, k // gsz)).astype(np.float32)
        bias_q = np.zeros(n, np.int32)
        bias_float = rng.uniform(-0.5, 0.5, size=n).astype(np.float32)
        deq = q.astype(np.float32) * np.repeat(s32, gsz, axis=1)
        if out_scale is None:
            rows = min(calib_rows, m)
            xd = (x_q[:rows].astype(np.float64) - fam.act_zp) * act_scale
            qr = xd @ deq.astype(np.float64).T + bias_float.astype(np.float64)
            out_scale = affine_scale_from_minmax(float(qr.min()), float(qr.max()), 0, fam.out_qmax, fam.out_zp)
        return QmmCase(family=fam, case="synthetic", m=m, k=k, n=n, activation_q=x_q, weight_q_nk=q,
                       weight_scale=s32, bias_q=bias_q, act_scale=float(act_scale), out_scale=float(out_scale),
                       weight_deq=deq, bias_float=bias_float, seed=seed)
    if fam.is_lpbq:
        if k % lpbq_block:
            raise ValueError(f"K={k} must be a multiple of the LPBQ block {lpbq_block}")
        block_scale = rng.integers(1, lpbq_max_scale + 1, size=(n, k // lpbq_block)).astype(np.uint8)
        expanded = q.astype(np.int16) * np.repeat(block_scale, lpbq_block, axis=1).astype(np.int16)
        w_int = expanded
    deq = w_int.astype(np.float32) * s32[:, None]
    if out_scale is None:
        rows = min(calib_rows, m)
        bias_scale = act_scale * s32.astype(np.float64)
        bias_deq = bias_q.astype(np.float64) * bias_scale
        xd = (x_q[:rows].astype(np.float64) - fam.act_zp) * act_scale
        qr = xd @ deq.astype(np.float64).T + bias_deq
        out_scale = affine_scale_from_minmax(float(qr.min()), float(qr.max()), 0, fam.out_qmax, fam.out_zp)
    fam_used = fam
    if fam.is_lpbq and lpbq_block != fam.lpbq_block_size:
        fam_used = Family(
            fam.name,
            fam.act_bits,
            fam.weight_bits,
            fam.out_bits,
            fam.weight_schema,
            fam.kernel_family,
            lpbq_block,
        )
    return QmmCase(
        family=fam_used,
        case="synthetic",
        m=m,
        k=k,
        n=n,
        activation_q=x_q,
        weight_q_nk=q,
        weight_scale=s32,
        bias_q=bias_q,
        act_scale=float(act_scale),
        out_scale=float(out_scale),
        weight_deq=deq,
        lpbq_block_int_scale=block_scale,
        lpbq_expanded_q_nk=expanded,
        seed=seed,
    )


def uniform_u8i8_case(m: int = 256, k: int = 256, n: int = 256, seed: int = 1) -> QmmCase:
    """The u8i8 matmul described with fixed per-tensor parameters instead of min/max-derived ones:

    * activations uint8 ~ U[0, 255], scale 0.02, offset -128 (zero point 128);
    * weights int8 ~ U[-127, 127], one scale 0.01 for every output channel;
    * int32 bias ~ U[-2^15, 2^15] at the bias scale 0.02 * 0.01;
    * output uint8, scale 0.05, offset 0.

    The seven seeded cases of ``make_case`` derive their scales from each case's float ranges;
    this one keeps the stated constants, so most outputs land on the clip rails.
    """
    fam = FAMILIES["u8i8"]
    rng = np.random.default_rng(seed)
    x_q = rng.integers(0, 256, size=(m, k)).astype(np.uint8)
    q = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    s32 = np.full(n, 0.01, dtype=np.float32)
    bias_q = rng.integers(-(1 << 15), (1 << 15) + 1, size=n).astype(np.int32)
    deq = q.astype(np.float32) * s32[:, None]
    return QmmCase(family=fam, case="uniform_fixed_scales", m=m, k=k, n=n, activation_q=x_q, weight_q_nk=q,
                   weight_scale=s32, bias_q=bias_q, act_scale=0.02, out_scale=0.05, weight_deq=deq, seed=seed)


# ---------------------------------------------------------------------------- graph operands
# The reference's CHAIN graphs (its op-package perf and CI flows) do not use the seeded float
# cases above: their operands are closed-form integer patterns, and their expected outputs are
# integer contracts applied chain times (gen_quant_chain.py:1525-1560).  The restatements below
# produce the same operands; the contracts run through qh_qmm_run_contract.

GRAPH_SEED_STRIDE = 374761393  # activation seed = (index + 1) * this (gen_quant_chain.py:271)


def graph_activation(act_bits: int, m: int, k: int, index: int = 0, mode: str = "default",
                     impulse_k: int = 0) -> np.ndarray:
    """[M, K] activation codes of graph input ``index`` (gen_quant_chain.py:253-274;
    gen_u8i8_chain.py:68-73 for u8i8):

    * ``default``: element i (row-major) = (37 i + seed) mod 2^act_bits, seed = (index + 1) * 374761393;
    * ``zp``: every element the zero point 2^(act_bits - 1);
    * ``k_impulse``: the zero point, except column ``impulse_k mod K`` = zero point + 1.
    """
    dt = np.dtype("<u2") if act_bits == 16 else np.dtype("uint8")
    mask = (1 << act_bits) - 1
    zp = 1 << (act_bits - 1)
    if mode == "zp":
        return np.full((m, k), zp, dtype=dt)
    if mode == "k_impulse":
        a = np.full((m, k), zp, dtype=dt)
        a[:, impulse_k % k] = zp + 1
        return a
    if mode != "default":
        raise ValueError(f"unknown activation mode {mode!r}")
    seed = (index + 1) * GRAPH_SEED_STRIDE
    i = np.arange(m * k, dtype=np.int64)
    return ((i * 37 + seed) & mask).astype(dt).reshape(m, k)


def graph_weight_kn(weight_bits: int, k: int, n: int, limit: Optional[int] = None) -> np.ndarray:
    """[K, N] integer weight codes ((31 k + 13 n) mod (2 q + 1)) - q, q = 2^(weight_bits - 1) - 1
    (or min(q, limit)) (gen_quant_chain.py:277-282; u8i8 uses the q = 7 pattern,
    gen_u8i8_chain.py:173-174)."""
    q = (1 << (weight_bits - 1)) - 1
    if limit is not None:
        q = max(1, min(q, int(limit)))
    kk = np.arange(k, dtype=np.int64)[:, None]
    nn = np.arange(n, dtype=np.int64)[None, :]
    return (((kk * 31 + nn * 13) % (2 * q + 1)) - q).astype(np.int32)


def graph_lpbq_block_scales(kernel_family: str, k: int, n: int, block: int) -> np.ndarray:
    """[N, K / block] LPBQ integer block scales in {1, 2, 3} (gen_quant_chain.py:316-329):
    w4a8: 1 + ((3 p + 5 b) mod 3) with p = 32 (n // 64) + n mod 32; w4a16: 1 + ((3 n + 5 (b // 2)) mod 3)."""
    if k % block:
        raise ValueError(f"LPBQ K={k} must be divisible by block size {block}")
    nn = np.arange(n, dtype=np.int64)[:, None]
    bb = np.arange(k // block, dtype=np.int64)[None, :]
    if kernel_family == "w4a8":
        pair = (nn // 64) * 32 + nn % 32
        f = 1 + (pair * 3 + bb * 5) % 3
    else:
        f = 1 + (nn * 3 + (bb // 2) * 5) % 3
    return f.astype(np.uint8)


@dataclass
class GraphCase:
    """Operands and expected-output contract of one of the reference's CHAIN graphs."""

    name: str
    act_bits: int
    weight_bits: int
    out_bits: int
    activation: np.ndarray         # [M, K] codes
    weight_kn: np.ndarray          # [K, N] integer codes (LPBQ: before the block scales)
    weight_compute_kn: np.ndarray  # [K, N] the integer weight the contract multiplies
    bias_q: np.ndarray             # [N] int32 (the legacy contract adds it; native ignores it)
    contract: str                  # "legacy" or "native"
    chain: int                     # the reference's CI chain length for this family
    lpbq_block_scale: Optional[np.ndarray] = None  # [N, K / block] uint8
    lpbq_block: int = 0
    kernel_family: str = ""

    @property
    def act_zp(self) -> int:
        return 1 << (self.act_bits - 1)

    @property
    def out_zp(self) -> int:
        return 32768 if self.out_bits == 16 else 0


# name: (act bits, weight bits, out bits, kernel family, LPBQ, contract, CI chain) -- the families of
# run_qnn_kernel_e2e_ci.sh:108-330 with their run-script defaults: the A8 flows use the legacy
# contract with bias 1..N (bias layout "legacy", gen_quant_chain.py:869-873), the A16 flows the
# native contract (run_w8a16_chain.sh / run_w4a16_chain.sh: --reference-contract native, a native
# A16 bias layout whose bias_q is zero); W4A16 per-channel gates CHAIN=1 (its precision suite),
# the others CHAIN=8; LPBQ blocks are 32 deep (--w4-lpbq-block-size default).
GRAPH_FAMILIES = {
    "u8i8": (8, 8, 8, "u8i8", False, "legacy", 8),
    "w4a8_per_channel": (8, 4, 8, "w4a8", False, "legacy", 8),
    "w4a8_lpbq": (8, 4, 8, "w4a8", True, "legacy", 8),
    "w8a16": (16, 8, 16, "w8a16", False, "native", 8),
    "w4a16_per_channel": (16, 4, 16, "w4a16", False, "native", 1),
    "w4a16_lpbq": (16, 4, 16, "w4a16", True, "native", 8),
    "w16a16": (16, 16, 16, "w16a16", False, "native", 8),
}

# The W4A16 precision suite of run_qnn_kernel_e2e_ci.sh:429-455: (activation mode, impulse column).
W4A16_PRECISION_SUITE = {
    "default": ("default", 0),
    "zp": ("zp", 0),
    "k_impulse0": ("k_impulse", 0),
    "k_impulse1": ("k_impulse", 1),
    "k_impulse7": ("k_impulse", 7),
}


def graph_case(name: str, m: int = 256, k: int = 256, n: int = 256, mode: str = "default", impulse_k: int = 0,
               lpbq_block: int = 32) -> GraphCase:
    """The operands of the reference's ``name`` CHAIN graph at M x K x N (gen_quant_chain.py:1078-1098,
    gen_u8i8_chain.py:170-213)."""
    a_bits, w_bits, o_bits, kfam, lpbq, contract, chain = GRAPH_FAMILIES[name]
    # u8i8 carries int8 storage but its graph weights are the q = 7 pattern
    w = graph_weight_kn(4 if name == "u8i8" else w_bits, k, n)
    scales = None
    wc = w
    if lpbq:
        scales = graph_lpbq_block_scales(kfam, k, n, lpbq_block)
        wc = w * np.repeat(scales.T.astype(np.int32), lpbq_block, axis=0)
    bias = np.arange(1, n + 1, dtype=np.int32) if contract == "legacy" else np.zeros(n, np.int32)
    return GraphCase(name=name, act_bits=a_bits, weight_bits=w_bits, out_bits=o_bits,
                     activation=graph_activation(a_bits, m, k, 0, mode, impulse_k), weight_kn=w,
                     weight_compute_kn=wc.astype(np.int32), bias_q=bias, contract=contract, chain=chain,
                     lpbq_block_scale=scales, lpbq_block=lpbq_block if lpbq else 0, kernel_family=kfam)
