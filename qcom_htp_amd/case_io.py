"""``case.json`` case directories of the reference's case generator, read and written.

The reference writes one directory per (family, case) with a ``case.json`` (schema
``qnn_hmx_matmul_python_case.v2``) and every array as ``<name>.npy`` plus ``<name>.raw``
(scripts/generate_qnn_matmul_python_cases.py:162-171 ``write_array``, :537-606
``generate_case``).  ``read_case`` turns such a directory into the ``QmmCase`` the prepared op
takes (and the expected ``output_ref_q`` when present); ``write_case`` writes a case -- with the
output the GPU computed -- in the same layout, so the reference's own consumers
(``run_qnn_python_case_native.py``, ``gen_quant_chain.py --case-dir``) can read it.

Arrays are loaded with ``numpy.load(allow_pickle=False)``; nothing in a case directory is
executed.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path
from typing import Any, Optional

import numpy as np

from .cases import FAMILIES, Family, QmmCase

__all__ = ["SCHEMA", "read_case", "write_case"]

SCHEMA = "qnn_hmx_matmul_python_case.v2"


def _stats(arr: np.ndarray) -> dict[str, Any]:
    """Per-array summary recorded beside each file (the fields of the reference's ``stats``)."""
    flt = arr.dtype.kind == "f"
    conv = float if flt else int
    return {
        "shape": list(arr.shape),
        "dtype": str(arr.dtype),
        "min": conv(arr.min()),
        "max": conv(arr.max()),
        "unique_count": int(np.unique(arr).size),
        "first8": [conv(v) for v in arr.reshape(-1)[:8]],
    }


def _write_array(path: Path, arr: np.ndarray) -> dict[str, Any]:
    arr = np.ascontiguousarray(arr)
    np.save(path.with_suffix(".npy"), arr)
    raw = path.with_suffix(".raw")
    arr.reshape(-1).tofile(raw)
    return {
        "npy": path.with_suffix(".npy").name,
        "raw": raw.name,
        "raw_sha256": hashlib.sha256(raw.read_bytes()).hexdigest(),
        **_stats(arr),
    }


def _load(case_dir: Path, files: dict, name: str) -> Optional[np.ndarray]:
    entry = files.get(name)
    if entry is None:
        return None
    return np.load(case_dir / entry["npy"], allow_pickle=False)


def read_case(case_dir) -> tuple[QmmCase, Optional[np.ndarray]]:
    """(QmmCase, output_ref_q or None) of a reference case directory."""
    case_dir = Path(case_dir)
    payload = json.loads((case_dir / "case.json").read_text(encoding="utf-8"))
    if not str(payload.get("schema", "")).startswith("qnn_hmx_matmul_python_case"):
        raise ValueError(f"{case_dir}: not a quantized-matmul case (schema {payload.get('schema')!r})")
    fam = FAMILIES[payload["family"]]
    qp = payload["qparams"]
    wq = qp["weight"]
    if fam.is_lpbq and int(wq.get("block_size", fam.lpbq_block_size)) != fam.lpbq_block_size:
        fam = Family(fam.name, fam.act_bits, fam.weight_bits, fam.out_bits, fam.weight_schema, fam.kernel_family,
                     int(wq["block_size"]))
    files = payload["files"]
    m, k, n = (int(v) for v in payload["shape_mkn"])
    bias_float = None
    if fam.weight_schema == "per_group":
        bias_float = _load(case_dir, files, "bias_float")
    case = QmmCase(
        family=fam,
        case=payload["case"],
        m=m,
        k=k,
        n=n,
        activation_q=_load(case_dir, files, "activation_q").astype(fam.act_dtype),
        weight_q_nk=_load(case_dir, files, "weight_q_nk"),
        weight_scale=_load(case_dir, files, "weight_scale").astype(np.float32),
        bias_q=_load(case_dir, files, "bias_q_int32").astype(np.int32),
        act_scale=float(qp["activation"]["scale"]),
        out_scale=float(qp["output"]["scale"]),
        weight_deq=None,
        lpbq_block_int_scale=_load(case_dir, files, "weight_lpbq_per_block_int_scale"),
        lpbq_expanded_q_nk=_load(case_dir, files, "weight_lpbq_expanded_q_nk"),
        lpbq_pre_group_scale=_load(case_dir, files, "weight_lpbq_pre_group_scale"),
        bias_float=None if bias_float is None else bias_float.astype(np.float32),
        seed=payload.get("seed"),
        extra={"case_json": payload},
    )
    return case, _load(case_dir, files, "output_ref_q")


def _weight_qparams(case: QmmCase) -> dict[str, Any]:
    fam = case.family
    qmax = fam.weight_qmax
    if fam.weight_schema == "per_group":
        return {"schema": "signed_symmetric_per_group", "axis": "K_group",
                "scale_storage_axes": ["output_row", "k_group"], "group_size": fam.weight_group_size,
                "bitwidth": fam.weight_bits, "scale_shape": list(case.weight_scale.shape), "zero_point": 0,
                "signed_range": [-qmax, qmax]}
    if fam.is_lpbq:
        blk = case.lpbq_block_int_scale
        return {"schema": "signed_symmetric_lpbq_from_per_group", "axis": "N", "block_axis": "K",
                "block_size": fam.lpbq_block_size, "bitwidth": 8, "compressed_bitwidth": fam.weight_bits,
                "scale_shape": list(case.weight_scale.shape), "pre_lpbq_group_size": fam.lpbq_block_size,
                "per_block_int_scale_shape": list(blk.shape),
                "per_block_int_scale_range": [int(blk.min()), int(blk.max())], "zero_point": 0, "offset": -128,
                "signed_range": [-qmax, qmax],
                "expanded_signed_range": [int(case.lpbq_expanded_q_nk.min()), int(case.lpbq_expanded_q_nk.max())]}
    return {"schema": "signed_symmetric_per_output_channel", "axis": "N", "bitwidth": fam.weight_bits,
            "scale_shape": list(case.weight_scale.shape), "zero_point": 0, "signed_range": [-qmax, qmax]}


def _affine_qparams(bits: int, scale: float, zp: int) -> dict[str, Any]:
    return {"schema": "aimet_qnn_affine_fixed_offset", "bitwidth": bits, "scale": float(scale), "zero_point": zp,
            "qnn_offset": -zp, "quantize_formula": "round(x / scale) - qnn_offset, then clamp",
            "dequantize_formula": "(q + qnn_offset) * scale"}


def write_case(case: QmmCase, root, output_q: Optional[np.ndarray] = None) -> Path:
    """Write ``case`` (and the computed ``output_q`` as ``output_ref_q``) as
    ``<root>/<family>/<case>/`` in the reference's case-directory layout.  Float source arrays
    that the case does not carry are left out of ``files``."""
    fam = case.family
    out_dir = Path(root) / fam.name / case.case
    out_dir.mkdir(parents=True, exist_ok=True)
    files = {
        "activation_q": _write_array(out_dir / "activation_q", case.activation_q),
        "weight_q_nk": _write_array(out_dir / "weight_q_nk", case.weight_q_nk),
        "weight_q_kn": _write_array(out_dir / "weight_q_kn", np.ascontiguousarray(case.weight_q_nk.T)),
        "weight_scale": _write_array(out_dir / "weight_scale", case.weight_scale),
        "bias_q_int32": _write_array(out_dir / "bias_q_int32", case.bias_q),
    }
    if case.bias_float is not None:
        files["bias_float"] = _write_array(out_dir / "bias_float", case.bias_float)
    if fam.is_lpbq:
        files["weight_lpbq_per_block_int_scale"] = _write_array(out_dir / "weight_lpbq_per_block_int_scale",
                                                                case.lpbq_block_int_scale)
        files["weight_lpbq_expanded_q_nk"] = _write_array(out_dir / "weight_lpbq_expanded_q_nk",
                                                          case.lpbq_expanded_q_nk)
        if case.lpbq_pre_group_scale is not None:
            files["weight_lpbq_pre_group_scale"] = _write_array(out_dir / "weight_lpbq_pre_group_scale",
                                                                case.lpbq_pre_group_scale)
    if output_q is not None:
        files["output_ref_q"] = _write_array(out_dir / "output_ref_q", output_q)
    bias_qp = ({"schema": "float32_per_group_bias_not_modeled"} if fam.weight_schema == "per_group" else
               {"schema": "float_source_quantized_to_int32", "bitwidth": 32,
                "scale_shape": list(case.weight_scale.shape),
                "scale": (case.act_scale * case.weight_scale.astype(np.float64)).tolist(), "zero_point": 0})
    payload = {
        "schema": SCHEMA,
        "family": fam.name,
        "kernel_family": fam.kernel_name,
        "weight_schema_variant": fam.weight_schema,
        "case": case.case,
        "seed": case.seed,
        "shape_mkn": [case.m, case.k, case.n],
        "qparams": {
            "activation": _affine_qparams(fam.act_bits, case.act_scale, fam.act_zp),
            "weight": _weight_qparams(case),
            "bias": bias_qp,
            "output": _affine_qparams(fam.out_bits, case.out_scale, fam.out_zp),
        },
        "files": files,
    }
    if output_q is not None:
        payload["output_counts"] = {"zero": int((output_q == 0).sum()), "max": int((output_q == fam.out_qmax).sum()),
                                    "zp": int((output_q == fam.out_zp).sum()), "total": int(output_q.size)}
    (out_dir / "case.json").write_text(json.dumps(payload, indent=2, sort_keys=True) + "\n", encoding="utf-8")
    return out_dir
