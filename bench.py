#!/usr/bin/env python3
"""Benchmark of the qcom_htp hot paths on one MI355X.

Primary line (the driver contract): the W4A8 per-channel quantized GEMM at M=K=N=4096
(uint8 activations ~ N(128, 40), int4 weights, per-channel fp32 scales, int32 bias, uint8
output), one step = one full requantised GEMM.  ``value`` is TOPS (2*M*K*N per step).
Extra figures in the same JSON line: W8A16 and u8i8 GEMMs at 4096^3, LPBQ GEMMs at
4096x4096x14336, the M=1 / M=16 LPBQ GEMV in GB/s (weights rotated over > 256 MB so the
MALL cannot serve them), and the GDN (I - A)^-1 solve at C=256 x 32 heads in heads/s.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--quick]
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path


def _cpu_threads() -> int:
    """Host threads for the CPU baseline: the job's CPU share (OMP_NUM_THREADS when the
    environment sets it, else the CPUs this process may run on)."""
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        return int(env)
    return len(os.sched_getaffinity(0))


# BLAS / OpenMP thread counts are read when numpy is first imported: pin them before that.
CPU_THREADS = _cpu_threads()
for _var in ("OMP_NUM_THREADS", "OPENBLAS_NUM_THREADS", "MKL_NUM_THREADS"):
    os.environ[_var] = str(CPU_THREADS)

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

I8_PEAK_TOPS = 5000.0  # MI355X dense int8 MFMA (5.0 POPS)
BF16_PEAK_TFLOPS = 2500.0
FP32_PEAK_TFLOPS = 157.3
HBM_PEAK_GBS = 8000.0


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_kernel(fn, steps: int, warmup: int):
    """(ms per step, from host wall clock with syncs; ms per step from stream events)."""
    import torch

    for _ in range(warmup):
        fn(0)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        fn(i)
    stop.record()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3 / steps
    ev = start.elapsed_time(stop) / steps
    return wall, ev


def time_graph(launch, steps: int, warmup: int):
    """(ms per step, wall clock; ms per step, stream events) of one replay of a HIP graph that holds
    `steps` launches, captured after `warmup` eager launches: the GPU runs the kernels back to back,
    without the gaps of launches issued one by one from Python.  (Capturing runs nothing.)"""
    import torch

    for _ in range(warmup):
        launch(0)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            launch(i)
    wall, ev = time_kernel(lambda i: graph.replay(), 1, 0)
    return wall / steps, ev / steps


def parity_check(case, got) -> dict:
    """Every output of the timed launches against the oracle (after the timed region)."""
    import numpy as np

    from oracle import qmm as oq  # the checker, never the thing measured

    want = oq.expected_output_case(case)
    bad = int((got.astype(np.int64) != want.astype(np.int64)).sum())
    if bad:
        raise RuntimeError(f"{case.family.name} {case.m}x{case.k}x{case.n}: {bad} outputs differ from the oracle")
    return {"parity_outputs_checked": int(got.size), "parity_mismatches": bad}


def gemm_workload(family: str, m: int, k: int, n: int, steps: int, warmup: int, lpbq_block: int = 64):
    import torch

    from qcom_htp_amd import cases
    from qcom_htp_amd.qmm import PATH_GEMM, QuantMatmul

    dev = torch.device("cuda", 0)
    case = cases.synthetic_case(family, m, k, n, seed=2, lpbq_block=lpbq_block)
    op = QuantMatmul.from_case(case, device=dev)
    act = torch.from_numpy(case.activation_q).to(dev)
    out = torch.empty((m, n), dtype=op.out_dtype, device=dev)
    launch = lambda i: op(act, out=out, path=PATH_GEMM)
    wall, ev = time_graph(launch, steps, warmup)
    wall_e, ev_e = time_kernel(launch, steps, 0)  # the same launches issued from Python, after the timed ones
    ops = 2.0 * m * k * n
    res = {"family": family, "m": m, "k": k, "n": n, "ms": ev, "wall_ms": wall, "tops": ops / (ev * 1e-3) / 1e12,
           "eager_ms": ev_e, "eager_tops": ops / (ev_e * 1e-3) / 1e12,
           "timing": f"one replay of a HIP graph holding the {steps} timed launches (stream events); eager_ms: the same launches issued from Python"}
    res.update(parity_check(case, out.cpu().numpy()))
    op.close()
    return res, case


def gemm_rotated_workload(family: str, m: int, k: int, n: int, steps: int, warmup: int, copies: int):
    """The GEMM over `copies` prepared weight sets and activation buffers in turn (more bytes
    than the 256 MB MALL holds), so every launch reads its operands from HBM; every copy's
    output is checked against the oracle after the timed region."""
    import torch

    from qcom_htp_amd import cases
    from qcom_htp_amd.qmm import PATH_GEMM, QuantMatmul

    dev = torch.device("cuda", 0)
    case = cases.synthetic_case(family, m, k, n, seed=2)
    ops = [QuantMatmul.from_case(case, device=dev) for _ in range(copies)]
    act0 = torch.from_numpy(case.activation_q).to(dev)
    acts = [act0.clone() for _ in range(copies)]
    outs = [torch.empty((m, n), dtype=ops[0].out_dtype, device=dev) for _ in range(copies)]
    launch = lambda i: ops[i % copies](acts[i % copies], out=outs[i % copies], path=PATH_GEMM)
    wall, ev = time_graph(launch, steps, warmup)
    wall_e, ev_e = time_kernel(launch, steps, 0)
    torch.cuda.synchronize()
    res = {"family": family, "m": m, "k": k, "n": n, "ms": ev, "wall_ms": wall, "tops": 2.0 * m * k * n / (ev * 1e-3) / 1e12,
           "eager_ms": ev_e, "eager_tops": 2.0 * m * k * n / (ev_e * 1e-3) / 1e12,
           "copies": copies, "rotated_mb": copies * (k * n + m * k) / 1e6}  # int8 weight tiles + activations
    res.update(parity_check(case, outs[0].cpu().numpy()))
    same = all(torch.equal(outs[0], o) for o in outs[1:])
    if not same:
        raise RuntimeError("rotated GEMM copies disagree")
    for op in ops:
        op.close()
    return res


def gemv_workload(family: str, m: int, k: int, n: int, steps: int, warmup: int, copies: int, lpbq_block: int = 64):
    import torch

    from qcom_htp_amd import cases
    from qcom_htp_amd.qmm import PATH_GEMV, QuantMatmul

    dev = torch.device("cuda", 0)
    case = cases.synthetic_case(family, m, k, n, seed=3, lpbq_block=lpbq_block)
    ops = [QuantMatmul.from_case(case, device=dev) for _ in range(copies)]
    act = torch.from_numpy(case.activation_q).to(dev)
    out = torch.empty((m, n), dtype=ops[0].out_dtype, device=dev)
    # A decode step is a few microseconds of GPU work, less than the host needs to issue it from
    # Python: the timed launches are captured in a HIP graph and replayed, so the events measure
    # the kernels back to back (the eager result is checked against the replayed one).
    want = ops[0](act, path=PATH_GEMV).clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            ops[i % copies](act, out=out, path=PATH_GEMV)
    wall, ev = time_kernel(lambda i: graph.replay(), 3, 1)
    ev /= steps
    wall /= steps
    if not torch.equal(out, want):
        raise RuntimeError(f"{family} GEMV: graph replay differs from the eager launch")
    check = parity_check(case, out.cpu().numpy())
    info = ops[0].info
    act_b = m * k * (2 if family.endswith("a16") or "a16" in family else 1)
    out_b = m * n * (2 if "a16" in family else 1)
    per_ch = n * (4 + 4)  # fp32 scale + int32 bias (the reference's per-channel operands)
    nbytes = info["gemv_weight_bytes"] + per_ch + act_b + out_b
    res = {"family": family, "m": m, "k": k, "n": n, "ms": ev, "wall_ms": wall, "bytes": nbytes,
           "gbs": nbytes / (ev * 1e-3) / 1e9, "weight_copies": copies,
           "rotated_mb": copies * info["gemv_weight_bytes"] / 1e6,
           # device memory the prepared weight state holds (GEMM tiles, GEMV stream, residue plane,
           # per-channel constants), as qh_qmm_query reports it
           "prepared_state_mb": info["device_bytes"] / 1e6, **check}
    for o in ops:
        o.close()
    return res


def stream_copy_workload(nbytes: int, steps: int, copies: int):
    """Context, not a product path: the vendor's elementwise copy (torch copy_, nbytes / 2 read and
    nbytes / 2 written: the GEMV's byte count in total), timed like the GEMV (a replayed graph of
    back-to-back launches over rotated sources): what a kernel that moves this many bytes once
    costs on this GPU, launch gaps included."""
    import torch

    n = nbytes // 8  # int32 elements per direction
    srcs = [torch.randint(0, 1 << 20, (n,), dtype=torch.int32, device="cuda") for _ in range(copies)]
    dst = torch.empty((n,), dtype=torch.int32, device="cuda")
    dst.copy_(srcs[0])
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(steps):
            dst.copy_(srcs[i % copies])
    wall, ev = time_kernel(lambda i: graph.replay(), 3, 1)
    ev /= steps
    return {"bytes": 8 * n, "ms": ev, "wall_ms": wall / steps, "gbs": 8 * n / (ev * 1e-3) / 1e9, "copies": copies,
            "what": "torch copy_ of int32 (half the bytes read, half written), graph-replayed over rotated sources"}


def gdn_workload(heads: int, C: int, steps: int, warmup: int, precision: int):
    import numpy as np
    import torch

    from qcom_htp_amd.gdn import gdn_solve

    rng = np.random.default_rng(4)
    k = rng.standard_normal((heads, C, 128))
    k /= np.sqrt((k * k).sum(-1, keepdims=True) + 1e-6)
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((heads, C))))
    g = np.cumsum(-np.logaddexp(0.0, -(rng.standard_normal((heads, C)) + 3.0)), axis=-1)
    low = np.tril(np.ones((C, C), bool), -1)
    A = np.where(low, -(beta[:, :, None] * (k @ k.transpose(0, 2, 1))) * np.exp(g[:, :, None] - g[:, None, :]), 0.0)
    dev = torch.device("cuda", 0)
    a = torch.from_numpy(A.astype(np.float32)).to(dev)
    out = torch.empty_like(a)
    launch = lambda i: gdn_solve(a, precision=precision, out=out)
    wall, ev = time_graph(launch, steps, warmup)  # a solve is about as short as its launch from Python
    wall_e, ev_e = time_kernel(launch, steps, 0)
    # the inverse of a unit lower-triangular C x C matrix: sum_j sum_{i>j} (i - j) multiply-adds
    # = C^3 / 6, i.e. C^3 / 3 flop
    flops = C ** 3 / 3.0 * heads
    from oracle import gdn as og  # the checker

    err = og.oc(out.cpu().numpy(), og.inverse_fp64(A))
    tol = og.GATE_FP32 if precision == 0 else og.GATE_BF16
    if not err <= tol:
        raise RuntimeError(f"GDN solve C={C} precision={precision}: oc {err:.3e} > {tol:.1e}")
    return {"heads": heads, "C": C, "precision": "fp32" if precision == 0 else "bf16", "ms": ev, "wall_ms": wall,
            "heads_per_s": heads / (ev * 1e-3), "tflops_alg": flops / (ev * 1e-3) / 1e12, "oc_vs_fp64": err,
            "eager_ms": ev_e, "timing": "graph replay of the timed launches; eager_ms: issued one by one"}, A


def gdn_chunk_workload(B: int, T: int, H: int, C: int, steps: int, warmup: int):
    """Fused chunk products W, U (bf16 out) from bf16 K, V at [B, T, H, 128]."""
    import torch

    from qcom_htp_amd.gdn import gdn_chunk_uw

    D = 128
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(5)
    k = torch.randn((B, T, H, D), generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn((B, T, H, D), generator=gen, device=dev).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn((B, T, H), generator=gen, device=dev))
    gc = torch.nn.functional.logsigmoid(torch.randn((B, T, H), generator=gen, device=dev) + 3.0)
    wall, ev = time_kernel(lambda i: gdn_chunk_uw(k, v, gc, beta, C), steps, warmup)
    chunk_heads = B * (T // C) * H
    # dense algorithmic work per chunk-head: A = K K^T (2 C^2 D), inverse (C^3 / 3), W and U (2 C^2 D each)
    flops = chunk_heads * (3 * 2.0 * C * C * D + C ** 3 / 3.0)
    nbytes = B * T * H * (4 * D * 2 + 2 * 4)  # K, V in + W, U out (bf16) + beta, g (fp32)
    # after the timed region: the outputs of a sample of (batch, chunk, head) items, first and
    # last included, against the float64 solve
    import numpy as np

    from oracle import gdn as og  # the checker

    w, u = gdn_chunk_uw(k, v, gc, beta, C)
    nch = T // C
    worst = 0.0
    for it in np.linspace(0, chunk_heads - 1, 8).astype(int).tolist():
        h, c, b = it % H, (it // H) % nch, it // (H * nch)
        sl = slice(c * C, (c + 1) * C)
        kc, vc = (x[b, sl, h].double().cpu().numpy() for x in (k, v))
        bc, gcc = beta[b, sl, h].double().cpu().numpy(), gc[b, sl, h].double().cpu().numpy()
        U, W = og.chunk_uw(og.inverse_fp64(og.build_A(kc, bc, gcc)), kc, vc, bc, gcc)
        worst = max(worst, og.oc(u[b, sl, h].double().cpu().numpy(), U), og.oc(w[b, sl, h].double().cpu().numpy(), W))
    if not worst <= og.GATE_BF16:
        raise RuntimeError(f"GDN chunk C={C}: oc {worst:.3e} > {og.GATE_BF16}")
    return {"B": B, "T": T, "H": H, "C": C, "ms": ev, "wall_ms": wall, "chunk_heads_per_s": chunk_heads / (ev * 1e-3),
            "tflops_alg": flops / (ev * 1e-3) / 1e12, "bytes": nbytes, "gbs": nbytes / (ev * 1e-3) / 1e9,
            "oc_vs_fp64_worst_of_8_items": worst}


def gdn_prefill_workload(B: int, T: int, H: int, steps: int, warmup: int, precision: int):
    """The chunked prefill at chunk 64: stage A (W, U; float32 for FP32, bf16 for BF16) then the
    chunk recurrence (stage B, o bf16 and the final state), timed as one step and per kernel."""
    import torch

    from qcom_htp_amd.gdn import FP32, gdn_chunk_state, gdn_chunk_uw, gdn_prefill

    D = 128
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(6)
    q, k, v = (torch.randn((B, T, H, D), generator=gen, device=dev).to(torch.bfloat16) for _ in range(3))
    beta = torch.sigmoid(torch.randn((B, T, H), generator=gen, device=dev))
    gc = torch.nn.functional.logsigmoid(torch.randn((B, T, H), generator=gen, device=dev) + 3.0)
    wu_dtype = torch.float32 if precision == FP32 else torch.bfloat16
    wall, ev = time_kernel(lambda i: gdn_prefill(q, k, v, gc, beta, precision=precision), steps, warmup)
    w, u = gdn_chunk_uw(k, v, gc, beta, 64, decay_w=True, out_dtype=wu_dtype)
    wall_b, ev_b = time_kernel(lambda i: gdn_chunk_state(q, k, gc, w, u, precision=precision), steps, warmup)
    # stage B bytes: q, k (bf16), W, U, o (bf16), gc, the final state
    wu_b = 4 if precision == FP32 else 2
    nbytes_b = B * T * H * (D * (2 + 2 + 2 * wu_b + 2) + 4) + B * H * D * D * 4
    # stage B flops per chunk-head: q k^T, W S, q S, P v_new, k^T v_new
    flops_b = B * H * (T // 64) * 2.0 * (64 * 64 * D * 2 + 3 * 64 * D * D)
    # after the timed region: two whole sequences against the float64 oracle
    import numpy as np

    from oracle import gdn as og  # the checker

    o, S = gdn_prefill(q, k, v, gc, beta, precision=precision)
    worst = 0.0
    for b, h in ((0, 0), (B - 1, H - 1)):
        seq = lambda x: x[b, :, h].double().cpu().numpy()[None]
        o_ref, S_ref = og.gdn_prefill_torch(seq(q), seq(k), seq(v), seq(gc), seq(beta), 64)
        worst = max(worst, og.oc(o[b, :, h].double().cpu().numpy(), o_ref.numpy()[0]),
                    og.oc(S[b, h].double().cpu().numpy(), S_ref.numpy()[0]))
    if not worst <= og.GATE_BF16:
        raise RuntimeError(f"GDN prefill: oc {worst:.3e} > {og.GATE_BF16}")
    return {"B": B, "T": T, "H": H, "chunk": 64, "precision": "fp32" if precision == FP32 else "bf16", "ms": ev,
            "wall_ms": wall, "tokens_per_s": B * T / (ev * 1e-3), "stage_b_ms": ev_b, "stage_b_wall_ms": wall_b,
            "stage_b_bytes": nbytes_b, "stage_b_gbs": nbytes_b / (ev_b * 1e-3) / 1e9,
            "stage_b_tflops_alg": flops_b / (ev_b * 1e-3) / 1e12, "oc_vs_fp64_worst_of_2_sequences": worst}


# The reference's custom-op CHAIN=8 graphs at 256^3 on the Hexagon v75 HTP: (kernel "main" cycles,
# graph timeline cycles) per graph run, example/qnn_matmul_profile/alignment_e2e_256_report.md:43-46,
# at the 1.594 GHz TURBO clock of example/gdn_native/baremetal/src/gdnbm_test.c:84.
REFERENCE_CHAIN8_CYCLES = {"u8i8": (10891, 36342), "w4a8_per_channel": (10025, 38644),
                           "w8a16": (30871, 80217), "w4a16_per_channel": (31419, 77854)}
REFERENCE_CLOCK_GHZ = 1.594


def graph_chain_workload(name: str, reps: int, chain: int = 8):
    """The reference's own CHAIN graph of family `name` at M = K = N = 256: its closed-form
    operands and integer contract (qcom_htp_amd.cases.graph_case; gen_quant_chain.py:253-329,
    971-996), `chain` dependent matmuls per graph run.  `reps` graph runs are captured in one HIP
    graph and replayed; after the timed region the output is checked against the reference step
    applied `chain` times."""
    import numpy as np
    import torch

    from oracle import qmm as oq  # the checker
    from qcom_htp_amd import cases
    from qcom_htp_amd.qmm import QuantMatmul, graph_contract

    dev = torch.device("cuda", 0)
    gc = cases.graph_case(name)
    op = QuantMatmul.from_graph_case(gc, device=dev)
    contract, d = graph_contract(gc)
    act = torch.from_numpy(gc.activation).to(dev)
    out = torch.empty((256, 256), dtype=op.out_dtype, device=dev)
    scr = torch.empty_like(out)
    op.chain(act, chain, contract, d, out=out, scratch=scr)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(reps):
            op.chain(act, chain, contract, d, out=out, scratch=scr)
    wall, ev = time_kernel(lambda i: graph.replay(), 3, 1)
    cur = gc.activation
    for _ in range(chain):
        cur = oq.reference_step(gc.act_bits, gc.weight_bits, gc.out_bits, cur, gc.weight_compute_kn, gc.bias_q,
                                contract=gc.contract, family_name=gc.kernel_family)
    bad = int((out.cpu().numpy().astype(np.int64) != cur.astype(np.int64)).sum())
    if bad:
        raise RuntimeError(f"graph chain {name}: {bad} outputs differ from the reference step applied {chain} times")
    op.close()
    us = ev * 1e3 / reps
    ref = {}
    if name in REFERENCE_CHAIN8_CYCLES and chain == 8:
        main, timeline = REFERENCE_CHAIN8_CYCLES[name]
        ref = {"reference_main_us": main / REFERENCE_CLOCK_GHZ / 1e3,
               "reference_timeline_us": timeline / REFERENCE_CLOCK_GHZ / 1e3,
               "speedup_vs_reference_timeline": timeline / REFERENCE_CLOCK_GHZ / 1e3 / us}
    return {"family": name, "m": 256, "k": 256, "n": 256, "chain": chain, "contract": f"{contract}/{d}",
            **ref, "us_per_chain": us, "us_per_matmul": us / chain, "wall_us_per_chain": wall * 1e3 / reps,
            "parity_outputs_checked": int(out.numel()), "parity_mismatches": bad,
            "what": "the reference's CHAIN graph operands and contract, graph-replayed"}


def gdn_u16_workload(heads: int, C: int, steps: int, warmup: int, precision: int):
    """The GdnSolve op's u16 I/O contract at C x heads: A quantised with the reference gate's
    parameters (sA = max|A| / 32767, zero points 32768, sT = 2 / 32767,
    scripts/gdn_solve_br_probe.py:59-60), T returned as u16 codes; oc of the dequantised T against
    the float64 inverse of the dequantised A (scripts/gdn_solve_oc_check.py:28-31)."""
    import numpy as np
    import torch

    from oracle import gdn as og  # the checker
    from qcom_htp_amd.gdn import GdnSolve

    k, beta, gc = og.config4_inputs(heads=heads, C=C, seed=4)
    A = og.build_A(k, beta, gc)
    sA = float(np.float32(max(np.abs(A).max() / 32767.0, 1e-12)))
    sT = float(np.float32(2.0 / 32767.0))
    codes = np.clip(np.rint(A / sA) + 32768, 0, 65535).astype(np.uint16)
    dev = torch.device("cuda", 0)
    a = torch.from_numpy(codes.view(np.int16)).to(dev).view(torch.uint16)
    out = torch.empty_like(a)
    launch = lambda i: GdnSolve(a, 32768, sA, 32768, sT, precision=precision, out=out)
    wall, ev = time_graph(launch, steps, warmup)
    wall_e, ev_e = time_kernel(launch, steps, 0)
    Ad = (codes.astype(np.int64) - 32768) * sA
    Td = (out.cpu().view(torch.int16).numpy().view(np.uint16).astype(np.int64) - 32768) * sT
    err = og.oc(Td, og.inverse_fp64(Ad))
    if not err <= og.GATE_BF16:
        raise RuntimeError(f"GDN u16 C={C}: oc {err:.3e} > {og.GATE_BF16}")
    flops = C ** 3 / 3.0 * heads  # the inverse's C^3 / 3 flop per head
    return {"heads": heads, "C": C, "precision": "fp32" if precision == 0 else "bf16", "ms": ev, "wall_ms": wall,
            "heads_per_s": heads / (ev * 1e-3), "tflops_alg": flops / (ev * 1e-3) / 1e12, "oc_vs_fp64": err,
            "eager_ms": ev_e, "sA": sA, "sT": sT, "zp": 32768}


def cpu_baseline(case, gdn_A):
    """The oracle (numpy/LAPACK/torch restatement of the reference's CPU path) on the host cores
    of this job: one warm-up, then the median of 5 runs per shape (3 for the slowest)."""
    import numpy as np
    import torch

    from oracle import gdn as og
    from oracle import qmm as oq
    from qcom_htp_amd import cases

    torch.set_num_threads(CPU_THREADS)
    try:
        from threadpoolctl import threadpool_info

        blas = max((p.get("num_threads", 1) for p in threadpool_info() if p.get("user_api") == "blas"), default=1)
    except Exception:  # pragma: no cover
        blas = CPU_THREADS

    def med(fn, reps=5):
        fn()
        ts = []
        for _ in range(reps):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts))

    def rows_of(c, r):
        return cases.QmmCase(**{**c.__dict__, "activation_q": c.activation_q[:r], "m": r})

    shapes = {}
    # primary: W4A8 per-channel at 4096^3, sampled to 1024 of the 4096 rows
    rows = 1024
    sub = rows_of(case, rows)
    t = med(lambda: oq.expected_output_case(sub))
    value = 2.0 * rows * case.k * case.n / t / 1e12
    # 256^3, the seven seeded u8i8 cases
    c1 = [cases.make_case("u8i8", cn, 256, 256, 256) for cn in cases.CASES]
    t = med(lambda: [oq.expected_output_case(c) for c in c1])
    shapes["u8i8_256^3_7_cases"] = {"s": t, "tops": 7 * 2.0 * 256 ** 3 / t / 1e12}
    # LPBQ at K=4096, N=14336: 512 prefill rows, and the decode shapes M=16 and M=1
    for fam in ("w4a8_lpbq", "w4a16_lpbq"):
        c = cases.synthetic_case(fam, 512, 4096, 14336, seed=2, lpbq_block=64)
        for m in (512, 16, 1):
            sc = rows_of(c, m)
            t = med(lambda: oq.expected_output_case(sc), reps=5 if m == 512 else 3)
            shapes[f"{fam}_{m}x4096x14336"] = {"s": t, "tops": 2.0 * m * 4096 * 14336 / t / 1e12}
    # GDN solve at C=256 x 32 heads: LAPACK inverse per head, and the reference's float64 row
    # recurrence in torch
    t = med(lambda: og.inverse_fp64(gdn_A))
    shapes["gdn_inverse_c256_h32_lapack"] = {"s": t, "heads_per_s": gdn_A.shape[0] / t}
    At = torch.from_numpy(np.ascontiguousarray(gdn_A))
    t = med(lambda: og.forward_subst_torch(At), reps=3)
    shapes["gdn_forward_subst_c256_h32_torch"] = {"s": t, "heads_per_s": gdn_A.shape[0] / t}
    # the intra-chunk half of the chunked GDN (A-build, row recurrence, U and W) in torch
    # float64, on a sample of chunk-heads
    rng = np.random.default_rng(8)
    for C, n in ((64, 256), (256, 32)):
        kk = torch.from_numpy(rng.standard_normal((n, C, 128)))
        vv = torch.from_numpy(rng.standard_normal((n, C, 128)))
        bb = torch.sigmoid(torch.from_numpy(rng.standard_normal((n, C))))
        gg = torch.nn.functional.logsigmoid(torch.from_numpy(rng.standard_normal((n, C))) + 3.0)
        t = med(lambda: og.chunk_stage_a_torch(kk, vv, gg, bb), reps=3)
        shapes[f"gdn_chunk_uw_c{C}_torch"] = {"s": t, "chunk_heads": n, "chunk_heads_per_s": n / t}
    # the whole chunked prefill (stage A + the chunk recurrence, scripts/gdn_ref_kernel.py:104-131)
    # in torch float64 on 8 of the 256 (batch, head) sequences of B=8, T=4096, H=32
    ns, T = 8, 4096
    qq, kk, vv = (torch.from_numpy(rng.standard_normal((ns, T, 128))) for _ in range(3))
    gg = torch.nn.functional.logsigmoid(torch.from_numpy(rng.standard_normal((ns, T))) + 3.0)
    bb = torch.sigmoid(torch.from_numpy(rng.standard_normal((ns, T))))
    t = med(lambda: og.gdn_prefill_torch(qq, kk, vv, gg, bb, 64), reps=3)
    shapes["gdn_prefill_c64_torch"] = {"s": t, "sequences": ns, "tokens": ns * T, "tokens_per_s": ns * T / t}
    return {
        "value": value,
        "unit": "TOPS",
        "cores": int(CPU_THREADS),
        "kind": "port",
        "sample": f"oracle output_ref_q (float64 dgemm + requant) on {rows} of {case.m} rows of the "
                  f"{case.k}x{case.n} W4A8 case; one warm-up, median of 5",
        "blas_threads": int(blas),
        "affinity_cpus": len(os.sched_getaffinity(0)),
        "shapes": shapes,
    }


def copy_calibration() -> int:
    """A plain streaming kernel of known HBM traffic: bitwise_not over 1 GiB of int32
    (reads 1 GiB, writes 1 GiB), five launches.  The FETCH_SIZE / WRITE_SIZE counters of
    these launches give the factor that converts the counters' units into bytes."""
    import torch

    n = 1 << 28
    a = torch.ones(n, dtype=torch.int32, device="cuda")
    b = torch.empty_like(a)
    for _ in range(5):
        torch.bitwise_not(a, out=b)
    torch.cuda.synchronize()
    print(json.dumps({"copy_kernel": "bitwise_not int32", "read_bytes": 4 * n, "write_bytes": 4 * n}), flush=True)
    return 0


def measured_traffic(kernel_key: str):
    """HBM bytes per launch of a kernel from the committed counter summary (profiles/traffic.json:
    FETCH_SIZE + WRITE_SIZE per dispatch, each scaled by the copy-kernel factor), or None."""
    p = ROOT / "profiles" / "traffic.json"
    try:
        d = json.loads(p.read_text())
        return d["kernels"][kernel_key]["traffic_bytes"]
    except Exception:
        return None


def vendor_int8_gemm_workload(M: int, K: int, N: int, steps: int, warmup: int):
    """Context, not a product path: the vendor library's plain int8 GEMM (torch._int_mm, i8 x i8
    -> i32, no requantisation) at the primary shape on the same GPU, for comparison with the
    requantising kernel above."""
    import torch

    g = torch.Generator(device="cuda").manual_seed(5)
    a = torch.randint(-128, 128, (M, K), dtype=torch.int8, device="cuda", generator=g)
    b = torch.randint(-128, 128, (N, K), dtype=torch.int8, device="cuda", generator=g)
    bt = b.t()
    try:  # timed like the GEMM lines: one replay of a graph of the timed launches
        wall, ev = time_graph(lambda i: torch._int_mm(a, bt), steps, warmup)
        how = "graph replay"
    except Exception as e:  # the library may refuse capture: eager only
        log(f"vendor GEMM graph capture failed ({e}); eager timing")
        torch.cuda.synchronize()
        wall, ev, how = *time_kernel(lambda i: torch._int_mm(a, bt), steps, warmup), "eager"
    wall_e, ev_e = time_kernel(lambda i: torch._int_mm(a, bt), steps, 0)
    return {"m": M, "k": K, "n": N, "ms": ev, "wall_ms": wall, "tops": 2.0 * M * K * N / (ev * 1e-3) / 1e12,
            "eager_ms": ev_e, "timing": how, "what": "torch._int_mm (i8 x i8 -> i32, no requantisation)"}


def lpbq_expand_workload(k: int, n: int, steps: int, warmup: int):
    """HmxW4LpbqExpandToI8 on the device: [K/2, N] int4 K-pair codes + [N * K/32] scales -> [K, N]
    int8 K-major tiles.  Byte work: K*N/2 + N*K/32 bytes in, K*N bytes out."""
    import torch

    from qcom_htp_amd.ops import HmxW4LpbqExpandToI8

    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(6)
    codes = torch.randint(0, 256, (1, 1, k // 2, n), dtype=torch.uint8, device=dev, generator=gen)
    scales = torch.randint(1, 16, (1, 1, 1, n * (k // 32)), dtype=torch.uint8, device=dev, generator=gen)
    out = torch.empty((1, 1, k, n), dtype=torch.uint8, device=dev)
    wall, ev = time_kernel(lambda i: HmxW4LpbqExpandToI8(codes, scales, out=out), steps, warmup)
    nbytes = k * n // 2 + n * (k // 32) + k * n
    return {"k": k, "n": n, "ms": ev, "wall_ms": wall, "bytes": nbytes, "gbs": nbytes / (ev * 1e-3) / 1e9}


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--quick", action="store_true", help="primary line only (no extras, no CPU baseline)")
    ap.add_argument("--only", default="", help="regex: run only the extra workloads whose key matches")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a plain streaming kernel of known size (for scaling HBM counters)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build measures one GPU only (no multi-GPU path); run with --gpus 1", file=sys.stderr)
        return 2

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 2
    torch.cuda.init()
    if args.copy_calibration:
        return copy_calibration()

    M = K = N = 4096
    log("primary: w4a8_per_channel GEMM 4096^3")
    prim, case = gemm_workload("w4a8_per_channel", M, K, N, args.steps, args.warmup)
    extra = {"w4a8_gemm_4096": prim}
    gdn_A = None
    if not args.quick:
        import re

        jobs = []
        for fam in ("w8a16", "u8i8", "w4a16_per_channel"):
            jobs.append((f"{fam}_gemm_4096", lambda fam=fam: gemm_workload(fam, M, K, N, max(5, args.steps // 2), 2)[0]))
        jobs.append(("w4a8_gemm_4096_rotated", lambda: gemm_rotated_workload("w4a8_per_channel", M, K, N, 20, 10, copies=10)))
        for fam in ("w4a8_lpbq", "w4a16_lpbq"):
            jobs.append((f"{fam}_gemm_4096x14336", lambda fam=fam: gemm_workload(fam, 4096, 4096, 14336, 5, 2)[0]))
        for fam in ("w4a8_lpbq", "w4a16_lpbq"):
            for m in (1, 16):
                jobs.append((f"{fam}_gemv_m{m}", lambda fam=fam, m=m: gemv_workload(fam, m, 4096, 14336, 200, 20, copies=10)))
        for prec in (0, 1):
            jobs.append((f"gdn_c256_h32_{'fp32' if prec == 0 else 'bf16'}", lambda prec=prec: gdn_workload(32, 256, 50, 5, prec)))
        for C in (64, 256):
            jobs.append((f"gdn_chunk_uw_c{C}", lambda C=C: gdn_chunk_workload(8, 4096, 32, C, 10, 2)))
        for prec in (0, 1):
            jobs.append((f"gdn_prefill_c64_{'fp32' if prec == 0 else 'bf16'}",
                         lambda prec=prec: gdn_prefill_workload(8, 4096, 32, 10, 2, prec)))
        for prec in (0, 1):
            jobs.append((f"gdn_u16_c256_h32_{'fp32' if prec == 0 else 'bf16'}", lambda prec=prec: gdn_u16_workload(32, 256, 50, 5, prec)))
        for name in ("u8i8", "w4a8_per_channel", "w4a8_lpbq", "w8a16", "w4a16_per_channel", "w4a16_lpbq", "w16a16"):
            jobs.append((f"graph_chain8_256_{name}", lambda name=name: graph_chain_workload(name, 50)))
        jobs.append(("lpbq_expand_4096x14336", lambda: lpbq_expand_workload(4096, 14336, 20, 3)))
        jobs.append(("vendor_int8_gemm_4096", lambda: vendor_int8_gemm_workload(M, K, N, 20, 5)))
        jobs.append(("vendor_copy_gemv_bytes", lambda: stream_copy_workload(30_410_000, 200, 10)))
        for key, job in jobs:
            if args.only and not re.search(args.only, key):
                continue
            log(key)
            r = job()
            if key.startswith("gdn_c256"):
                r, gdn_A = r
            extra[key] = r
    torch.cuda.synchronize()

    tops = prim["tops"]
    line = {
        "metric": "W4A8/W8A16 GEMM TOPS (% i8 MFMA peak) @4096³; GDN (I−A)⁻¹ heads/s @C=256",
        "value": round(tops, 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(prim["wall_ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {"workload": "w4a8_per_channel quantized GEMM, u8 act x int4 weight -> u8, M=K=N=4096",
                   "m": M, "k": K, "n": N, "family": "w4a8_per_channel"},
        "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": I8_PEAK_TOPS, "unit": "TOPS",
                     "frac": round(tops / I8_PEAK_TOPS, 4), "traffic": measured_traffic("w4a8_gemm_4096"),
                     "kernel": "qmm_gemm_kernel<A8> (int8 weight tiles)",
                     "measured": "stream events over one replay of a HIP graph of the timed steps"},
        "extra": extra,
    }
    if not args.quick and not args.only:
        log(f"cpu baseline (oracle on {CPU_THREADS} host threads)")
        line["cpu_baseline"] = cpu_baseline(case, gdn_A)
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
