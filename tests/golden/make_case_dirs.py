#!/usr/bin/env python3
"""Write reference-generated ``case.json`` directories as fixtures for the case I/O tests.

Imports the reference generator ``scripts/generate_qnn_matmul_python_cases.py`` from
/root/reference (read-only; bytecode writing is disabled so nothing is written there) and calls
its ``generate_case`` for a few (family, case) pairs at the generator's default shape
M=32, K=128, N=32, into ``tests/golden/case_dirs/<family>/<case>/`` (``case.json`` plus the
``.npy`` / ``.raw`` arrays it writes).  These directories are the reference's own output: the
reader must load them unchanged and the GPU must reproduce their ``output_ref_q``.

Run once in the development container (the reference does not exist on GPU hosts):
    python tests/golden/make_case_dirs.py
"""

from __future__ import annotations

import importlib.util
import shutil
import sys
from pathlib import Path

sys.dont_write_bytecode = True
REF = Path("/root/reference/scripts/generate_qnn_matmul_python_cases.py")
OUT = Path(__file__).resolve().parent / "case_dirs"
PAIRS = (("u8i8", "normal_random"), ("w4a16_lpbq", "positive_boundary"), ("w4a8_per_group", "bias_only"))


def main() -> int:
    spec = importlib.util.spec_from_file_location("ref_qmm_cases", REF)
    mod = importlib.util.module_from_spec(spec)
    sys.modules[spec.name] = mod
    spec.loader.exec_module(mod)
    if OUT.exists():
        shutil.rmtree(OUT)
    for fam, case in PAIRS:
        mod.generate_case(OUT, mod.FAMILIES[fam], case, 32, 128, 32)
        print(f"wrote {OUT / fam / case}")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
