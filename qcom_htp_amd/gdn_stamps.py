"""Per-phase cycle stamps of the GDN solve kernel, and its matrix-core utilisation in the strips.

    python -m qcom_htp_amd.gdn_stamps [--heads 32] [--C 256] [--json out.json]

A profiling tool, not a product path: it writes a timing copy of ``csrc/gdn_solve.hip`` in which
thread 0 of every workgroup records ``s_memtime`` (shader clock) at the phase boundaries of
``gdn_fs_kernel`` -- A reads issued and the diagonal blocks staged, level 0, the strictly lower
blocks staged, the strip steps of wave 0 (the workgroup's longest strip, each storing its tile) --
compiles it into ``_build/stamps/`` and runs it on the C x heads solve workload (both
precisions).  It prints the median cycles of each phase over the workgroups and the strip window
(strips start to the end of wave 0's steps).

With the executed MFMA operations of the same launch (``SQ_INSTS_VALU_MFMA_MOPS_BF16`` x 512 from
``rocprofv3 --pmc``, passed as ``--exec-bf16-ops``/``--exec-fp32-ops``), it also prints the
per-active-CU utilisation inside the strip window: operations per workgroup / (window cycles x
4096 bf16 flop per CU cycle, MI355X's 2.5 PFLOP/s at 2.4 GHz over 256 CUs).  The algorithmic
count is the C^3 / 3 flop of the unit lower-triangular inverse (C^3 / 6 multiply-adds) minus level
0's diagonal blocks, spread over the head's workgroups.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import subprocess
import sys
from pathlib import Path

from . import build as B

OUT = B.OBJDIR / "stamps"
PHASES = ["A reads and diagonal staging", "level 0", "lower blocks staged", "strip steps (stores issued as they go)", "strip end"]
BF16_FLOP_PER_CU_CYCLE = 2.5e15 / (256 * 2.4e9)

_ANCHORS = [
    ("  // ---- A reads", 0),
    ("  fs_level0<SPLIT>(Td, dstage, NB, t);\n", 1),
    ("#pragma unroll\n  for (int u = 0; u < kLowLoads; ++u) {\n    const int s = t + kRdThreads * u, blk = s >> 6;\n    if (blk < nlow) {", 2),
    ("  // ---- the wave's strip", 3),
    ("#pragma unroll\n  for (int v = 0; v < kFsMaxNB; ++v)\n    if (v <= steps) asm volatile", 4),
]


def stamped_source() -> str:
    """The solve source with the stamps inserted (raises if the kernel's structure changed)."""
    src = (B.CSRC / "gdn_solve.hip").read_text()
    cut = src.index("// G = 2 workgroups per head for more than 8 strips, one otherwise.\nGdnArgs make_args")
    src = src[:cut] + "}  // namespace\n}  // namespace qh\n"
    src = src.replace(
        "namespace qh {\nnamespace {",
        "namespace qh {\ninline namespace stampsns {\n__device__ unsigned long long *g_st;\n"
        "__shared__ unsigned long long s_ts[16];\n"
        "#define STAMP(k) do { if (threadIdx.x == 0) s_ts[(k)] = __builtin_readcyclecounter(); } while (0)\n", 1)
    for anchor, k in _ANCHORS:
        if src.count(anchor) != 1:
            raise RuntimeError(f"gdn_solve.hip changed: anchor not found once: {anchor!r}")
        src = src.replace(anchor, f"  STAMP({k});\n" + anchor, 1)
    call = "  if (j >= 0) fs_strip_solve<U16, SPLIT>(g, hbase, Al, Td, dstage, NB, j, lane);\n"
    if src.count(call) != 1:
        raise RuntimeError("gdn_solve.hip changed: strip call not found")
    src = src.replace(call, call + "  STAMP(5);\n"
                      "  if (threadIdx.x == 0) for (int k = 0; k < 6; ++k) g_st[(head * g.groups + part) * 16 + k] = s_ts[k];\n", 1)
    src += """
extern "C" int stamps_set(unsigned long long *stamps) {
  return (int)hipMemcpyToSymbol(HIP_SYMBOL(qh::g_st), &stamps, sizeof(stamps));
}
extern "C" int stamps_solve(const void *A, void *T, int heads, int C, int split, void *stream) {
  qh::GdnArgs g{A, T, C, C / 16 > 8 ? 2 : 1, heads, 0, 0, 1.0f, 1.0f, 1.0f};
  const dim3 grid((heads + 7) / 8 * 8 * g.groups);
  if (split) hipLaunchKernelGGL((qh::gdn_fs_kernel<false, true>), grid, dim3(512), 0, (hipStream_t)stream, g);
  else hipLaunchKernelGGL((qh::gdn_fs_kernel<false, false>), grid, dim3(512), 0, (hipStream_t)stream, g);
  return (int)hipGetLastError();
}
"""
    return src


def build_stamped() -> Path:
    OUT.mkdir(parents=True, exist_ok=True)
    src = OUT / "gdn_solve_stamps.hip"
    lib = OUT / "libgdn_solve_stamps.so"
    src.write_text(stamped_source())
    cmd = [B._hipcc(), *B.COMMON, *B.HIP_FLAGS, "-shared", "-x", "hip", str(src), "-o", str(lib)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"stamped build failed:\n{r.stderr[-3000:]}")
    return lib


def config4_A(heads: int, C: int, D: int = 128, seed: int = 4):
    """A [heads, C, C] (float32) of the solve workload: A_ij = -beta_i (k^_i . k^_j) e^{g_i - g_j}
    for i > j, k^ the l2-normalised N(0, 1) keys of dimension D, beta = sigmoid(N(0, 1)), g the
    cumulative sum of logsigmoid(N(0, 1) + 3)."""
    import numpy as np

    rng = np.random.default_rng(seed)
    k = rng.standard_normal((heads, C, D))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((heads, C))))
    g = np.cumsum(-np.logaddexp(0.0, -(rng.standard_normal((heads, C)) + 3.0)), axis=-1)
    kn = k / np.linalg.norm(k, axis=-1, keepdims=True)
    lower = np.tril(np.ones((C, C), dtype=bool), -1)
    decay = np.exp(np.where(lower, g[..., :, None] - g[..., None, :], 0.0)) * lower
    return (-(beta[..., :, None] * (kn @ np.swapaxes(kn, -1, -2))) * decay).astype(np.float32)


def run(heads: int, C: int, exec_ops: dict) -> dict:
    import numpy as np
    import torch

    lib = ctypes.CDLL(str(build_stamped()))
    lib.stamps_solve.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    lib.stamps_set.argtypes = [ctypes.c_void_p]
    G = 2 if C // 16 > 8 else 1
    A = torch.from_numpy(config4_A(heads, C)).cuda()
    T = torch.empty_like(A)
    st = torch.zeros(((heads + 7) // 8 * 8) * G * 16, dtype=torch.int64, device="cuda")
    if lib.stamps_set(st.data_ptr()) != 0:
        raise RuntimeError("stamps_set failed")
    alg_wg = (C ** 3 / 3.0 - (C // 16) * 16 ** 3 / 3.0) / G
    res = {}
    for split, name in ((0, "bf16"), (1, "fp32")):
        for _ in range(5):
            if lib.stamps_solve(A.data_ptr(), T.data_ptr(), heads, C, split, torch.cuda.current_stream().cuda_stream) != 0:
                raise RuntimeError("stamps_solve failed")
        torch.cuda.synchronize()
        s = st.view(-1, 16).cpu().numpy().astype(np.int64)[: heads * G, :6]
        d = np.diff(s, axis=1)
        window = s[:, 4] - s[:, 3]
        r = {"phase_cycles_median": {PHASES[i]: float(np.median(d[:, i])) for i in range(5)},
             "strip_window_cycles_median": float(np.median(window)), "strip_window_cycles_mean": float(window.mean()),
             "workgroup_cycles_median": float(np.median(s[:, 5] - s[:, 0])), "workgroups": int(len(s)),
             "algorithmic_flop_per_workgroup": alg_wg,
             "algorithmic_strip_utilisation": alg_wg / (window.mean() * BF16_FLOP_PER_CU_CYCLE)}
        if exec_ops.get(name):
            ops_wg = exec_ops[name] / (heads * G)
            r["executed_ops_per_workgroup"] = ops_wg
            r["executed_strip_utilisation"] = ops_wg / (window.mean() * BF16_FLOP_PER_CU_CYCLE)
        res[name] = r
        print(f"{name}: " + ", ".join(f"{p} {v:.0f}" for p, v in r["phase_cycles_median"].items()) +
              f"; strip window {r['strip_window_cycles_median']:.0f} cycles (median of {len(s)} workgroups); "
              f"algorithmic strip utilisation {100 * r['algorithmic_strip_utilisation']:.2f}%" +
              (f", executed {100 * r['executed_strip_utilisation']:.2f}%" if "executed_strip_utilisation" in r else ""),
              flush=True)
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--heads", type=int, default=32)
    ap.add_argument("--C", type=int, default=256)
    ap.add_argument("--exec-bf16-ops", type=float, default=0.0, help="executed MFMA ops per launch, bf16 products")
    ap.add_argument("--exec-fp32-ops", type=float, default=0.0, help="executed MFMA ops per launch, fp32 (hi/lo) products")
    ap.add_argument("--json", default="")
    a = ap.parse_args()
    sys.path.insert(0, str(B.ROOT))
    res = run(a.heads, a.C, {"bf16": a.exec_bf16_ops, "fp32": a.exec_fp32_ops})
    if a.json:
        Path(a.json).write_text(json.dumps(res, indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
