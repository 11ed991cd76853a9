#!/usr/bin/env python3
"""Write golden vectors for the quantized-matmul case generator and oracle.

Imports the reference generator ``scripts/generate_qnn_matmul_python_cases.py`` from
/root/reference (read-only; bytecode writing is disabled so nothing is written there)
and records, for every family x case:

* at the generator's default shape M=32, K=128, N=32: the full quantised operands,
  the per-channel / LPBQ scales, bias codes, the float32 image of the dequantised
  output and ``output_ref_q``  -> ``qmm_small.npz`` + ``qmm_small.json``;
* at the gate shape 256^3: scalar quant params, output counts and the sha256 of
  every array the reference writes                       -> ``qmm_256.json``.

Run once in the development container (the reference does not exist on GPU hosts):
    python tests/golden/make_qmm_golden.py
"""

from __future__ import annotations

import hashlib
import importlib.util
import json
import sys
from pathlib import Path

import numpy as np

sys.dont_write_bytecode = True
REF = Path("/root/reference/scripts/generate_qnn_matmul_python_cases.py")
HERE = Path(__file__).resolve().parent

SMALL = (32, 128, 32)
GATE = (256, 256, 256)

ARRAYS = (
    "activation_q",
    "weight_q_nk",
    "weight_scale",
    "bias_q_int32",
    "output_q",
    "output_quantized_path_float",
    "output_float",
    "weight_lpbq_per_block_int_scale",
    "weight_lpbq_expanded_q_nk",
    "weight_lpbq_pre_group_scale",
)


def load_reference():
    spec = importlib.util.spec_from_file_location("ref_qmm_cases", REF)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod
    spec.loader.exec_module(mod)
    return mod


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a).reshape(-1).tobytes()).hexdigest()


def run_case(ref, fam, case, shape):
    m, k, n = shape
    x, w, b = ref.make_float_case(fam, case, m, k, n)
    q = ref.quantize_case(fam, x, w, b)
    return q


def main() -> int:
    ref = load_reference()
    small_arrays: dict[str, np.ndarray] = {}
    small_meta: dict[str, dict] = {}
    gate_meta: dict[str, dict] = {}
    for fam_name, fam in ref.FAMILIES.items():
        for case in ref.CASES:
            key = f"{fam_name}/{case}"
            q = run_case(ref, fam, case, SMALL)
            qp = q["qparams"]
            small_meta[key] = {
                "seed": ref.seed_for(fam_name, case),
                "shape_mkn": list(SMALL),
                "act_scale": float(qp["activation"]["scale"]).hex(),
                "out_scale": float(qp["output"]["scale"]).hex(),
            }
            for name in ARRAYS:
                arr = q.get(name)
                if arr is not None:
                    small_arrays[f"{key}/{name}"] = np.asarray(arr)

            q = run_case(ref, fam, case, GATE)
            qp = q["qparams"]
            entry = {
                "seed": ref.seed_for(fam_name, case),
                "shape_mkn": list(GATE),
                "act_scale": float(qp["activation"]["scale"]).hex(),
                "out_scale": float(qp["output"]["scale"]).hex(),
                "output_counts": ref.output_counts(q["output_q"], fam),
                "sha256": {},
            }
            for name in ARRAYS:
                arr = q.get(name)
                if arr is not None:
                    entry["sha256"][name] = sha(np.asarray(arr))
            gate_meta[key] = entry
            print(f"{key}: sA={float(qp['activation']['scale']):.6g} sO={float(qp['output']['scale']):.6g}")

    np.savez_compressed(HERE / "qmm_small.npz", **small_arrays)
    (HERE / "qmm_small.json").write_text(json.dumps(small_meta, indent=1, sort_keys=True) + "\n")
    (HERE / "qmm_256.json").write_text(json.dumps(gate_meta, indent=1, sort_keys=True) + "\n")
    print(f"wrote {len(small_meta)} small cases and {len(gate_meta)} gate-shape digests")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
