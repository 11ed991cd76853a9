"""Build libqhtp.so (gfx950) in-tree with hipcc.

    python -m qcom_htp_amd.build          # compiles qcom_htp_amd/libqhtp.so

Every HIP source is compiled with ``--offload-arch=gfx950`` and packed-fp32 code generation
disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``); objects are compiled in
parallel and linked into one shared library next to this file.
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
OBJDIR = PKG / "_build"
LIB = PKG / "libqhtp.so"

ARCH = "gfx950"
COMMON = [
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]
HIP_FLAGS = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found (ROCm toolchain required to build libqhtp)")
    return exe


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(CSRC.glob("*.cpp"))


# Sources whose device assembly is kept and checked (qcom_htp_amd.isa_check): the GEMM's k loop
# counts its own memory waits.
ISA_CHECKED = ("qmm_gemm.hip",)


def _compile(src: Path) -> Path:
    obj = OBJDIR / (src.name + ".o")
    cmd = [_hipcc(), *COMMON]
    if src.suffix == ".hip":
        cmd += ["-x", "hip", *HIP_FLAGS]
        if src.name in ISA_CHECKED:
            cmd += ["-save-temps=obj"]
    else:
        cmd += ["-D__HIP_PLATFORM_AMD__"]
    cmd += ["-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (res.stderr or "").splitlines() if noise not in l)
    if res.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)
    if src.name in ISA_CHECKED:
        from .isa_check import check_file

        asm = device_asm(src)
        names, errs = check_file(str(asm))
        if not names or errs:
            raise RuntimeError(f"{src.name}: memory-wait check of {asm.name} failed "
                               f"({len(names)} kernels):\n" + "\n".join(errs[:20]))
    return obj


def device_asm(src: Path) -> Path:
    """The gfx950 assembly that -save-temps=obj left for ``src`` in the build folder."""
    return OBJDIR / f"{src.stem}-hip-amdgcn-amd-amdhsa-{ARCH}.s"


def build(verbose: bool = True) -> Path:
    """Compile every source under csrc/ and link qcom_htp_amd/libqhtp.so."""
    OBJDIR.mkdir(exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), max(1, min(16, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        objs = list(ex.map(_compile, srcs))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(srcs)} sources")
    return LIB


if __name__ == "__main__":
    build()
