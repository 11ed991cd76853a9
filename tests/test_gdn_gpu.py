"""GPU parity of the GDN triangular solve vs the fp64 inverse.

Tolerances (relative Frobenius error, scripts/gdn_solve_oc_check.py:31):
  fp32 path  <= 1e-4
  bf16 path  <= 1.05e-2 (tests/qnn_kernel_e2e/correctness/test_gdn_solve_e2e.sh:18)
"""

import numpy as np
import pytest

from oracle import gdn as og

pytestmark = pytest.mark.gpu

FP32_TOL = 1.0e-4
BF16_TOL = 1.05e-2


def solve(A, gpu, precision):
    import torch

    from qcom_htp_amd.gdn import gdn_solve

    t = torch.from_numpy(np.ascontiguousarray(A, dtype=np.float32)).to(gpu)
    T = gdn_solve(t, precision=precision)
    torch.cuda.synchronize()
    return T.cpu().numpy().astype(np.float64)


@pytest.mark.parametrize("C", [16, 32, 48, 64, 128, 256])
@pytest.mark.parametrize("precision", [0, 1], ids=["fp32", "bf16"])
def test_gdn_solve_config4_inputs(gpu, C, precision):
    heads = 8 if C == 256 else 6
    k, beta, gc = og.config4_inputs(heads=heads, C=C, seed=C)
    A = og.build_A(k, beta, gc).astype(np.float32)
    print(f"[gdn] C={C} heads={heads} precision={precision}", flush=True)
    T = solve(A, gpu, precision)
    Tref = og.inverse_fp64(A.astype(np.float64))
    err = og.oc(T, Tref)
    tol = FP32_TOL if precision == 0 else BF16_TOL
    print(f"[gdn] C={C} precision={precision} oc={err:.3e}", flush=True)
    assert err <= tol, f"oc={err:.3e} > {tol:.1e}"
    # exact structure: zeros above the diagonal, unit diagonal
    iu = np.triu_indices(C, 1)
    assert np.all(T[:, iu[0], iu[1]] == 0.0)
    if precision == 0:
        np.testing.assert_allclose(np.diagonal(T, axis1=1, axis2=2), 1.0, atol=1e-6)


def test_gdn_solve_full_config4(gpu):
    k, beta, gc = og.config4_inputs(heads=32, C=256, seed=4)
    A = og.build_A(k, beta, gc).astype(np.float32)
    Tref = og.inverse_fp64(A.astype(np.float64))
    for precision, tol in ((0, FP32_TOL), (1, BF16_TOL)):
        print(f"[gdn] config4 32x256 precision={precision}", flush=True)
        err = og.oc(solve(A, gpu, precision), Tref)
        print(f"[gdn] config4 32x256 precision={precision} oc={err:.3e}", flush=True)
        assert err <= tol, f"precision {precision}: oc={err:.3e}"


def test_gdn_zero_and_identity_cases(gpu):
    A = np.zeros((2, 64, 64), np.float32)
    T = solve(A, gpu, 0)
    np.testing.assert_array_equal(T, np.broadcast_to(np.eye(64), T.shape))
    # a single sub-diagonal: T is the closed-form nilpotent series sum_k A^k
    A = np.zeros((1, 32, 32), np.float32)
    idx = np.arange(31)
    A[0, idx + 1, idx] = 0.5
    T = solve(A, gpu, 0)[0]
    want = np.tril(0.5 ** (np.arange(32)[:, None] - np.arange(32)[None, :]).astype(np.float64))
    np.testing.assert_allclose(T, want, rtol=1e-6, atol=1e-7)


def test_gdn_upper_triangle_is_ignored(gpu):
    k, beta, gc = og.config4_inputs(heads=2, C=64, seed=9)
    A = og.build_A(k, beta, gc).astype(np.float32)
    A_dirty = A + np.triu(np.full((64, 64), 7.0, np.float32))
    np.testing.assert_array_equal(solve(A, gpu, 0), solve(A_dirty, gpu, 0))


@pytest.mark.parametrize("precision", [0, 1], ids=["fp32", "bf16"])
def test_gdn_u16_code_contract(gpu, precision):
    import torch

    from qcom_htp_amd.gdn import GdnSolve

    heads, C = 8, 256
    k, beta, gc = og.config4_inputs(heads=heads, C=C, seed=21)
    A = og.build_A(k, beta, gc)
    sA, sT = og.SA_REF, og.ST_REF
    Aq = og.quantize_u16(A, sA)
    Adeq = og.dequantize_u16(Aq, sA)
    print(f"[gdn] u16 contract precision={precision}", flush=True)
    Tq = GdnSolve(torch.from_numpy(Aq.view(np.uint16)).to(gpu), 32768, sA, 32768, sT, precision=precision)
    torch.cuda.synchronize()
    T = og.dequantize_u16(Tq.cpu().numpy(), sT)
    err = og.oc(T, og.inverse_fp64(Adeq))
    # u16 output quantisation at sT adds ~sT/sqrt(12) per element on top of the solve error
    tol = 5e-4 if precision == 0 else BF16_TOL
    assert err <= tol, f"oc={err:.3e}"
    assert np.all(Tq.cpu().numpy()[:, np.triu_indices(C, 1)[0], np.triu_indices(C, 1)[1]] == 32768)


def chunk_inputs(B, T, H, seed):
    """Config-5 style inputs: k, v ~ N(0,1) rounded to bf16, beta = sigmoid(N(0,1)),
    gc = logsigmoid(N(0,1) + 3), in the reference kernel's [B, T, H, (D)] layout."""
    rng = np.random.default_rng(seed)

    def bf16(x):  # float32 -> bf16 bit patterns, round to nearest even
        u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
        return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)

    kb = bf16(rng.standard_normal((B, T, H, 128)))
    vb = bf16(rng.standard_normal((B, T, H, 128)))
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H))))).astype(np.float32)
    gc = (-np.logaddexp(0.0, -(rng.standard_normal((B, T, H)) + 3.0))).astype(np.float32)
    return kb, vb, beta, gc


def bf16_to_f64(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


@pytest.mark.parametrize("C", [64, 128, 256])
@pytest.mark.parametrize("decay_w", [False, True], ids=["W_beta_k", "W_beta_k_eg"])
@pytest.mark.parametrize("out", ["bf16", "f32"])
def test_gdn_chunk_uw_matches_fp64(gpu, C, decay_w, out):
    """U = T (beta V), W = T (beta K^) [e^g] per chunk and head, against float64 (A built
    from the same bf16 inputs, T by LAPACK); bound 1.05e-2 relative Frobenius per chunk-head."""
    import torch

    from qcom_htp_amd.gdn import gdn_chunk_uw

    B, H, nch = 2, 3, 2
    T = nch * C
    kb, vb, beta, gc = chunk_inputs(B, T, H, seed=C + 7 * decay_w)
    print(f"[gdn] chunk_uw C={C} decay_w={decay_w} out={out}", flush=True)
    dev = gpu
    kt = torch.from_numpy(kb.view(np.int16)).to(dev).view(torch.bfloat16)
    vt = torch.from_numpy(vb.view(np.int16)).to(dev).view(torch.bfloat16)
    w, u = gdn_chunk_uw(kt, vt, torch.from_numpy(gc).to(dev), torch.from_numpy(beta).to(dev), C, decay_w=decay_w,
                        out_dtype=torch.bfloat16 if out == "bf16" else torch.float32)
    torch.cuda.synchronize()
    w = w.float().cpu().numpy().astype(np.float64)
    u = u.float().cpu().numpy().astype(np.float64)
    k64, v64 = bf16_to_f64(kb), bf16_to_f64(vb)
    worst = 0.0
    for b in range(B):
        for c in range(nch):
            sl = slice(c * C, (c + 1) * C)
            for h in range(H):
                kc, vc = k64[b, sl, h], v64[b, sl, h]
                bc, gcc = beta[b, sl, h].astype(np.float64), gc[b, sl, h].astype(np.float64)
                Tm = og.inverse_fp64(og.build_A(kc, bc, gcc))
                U, W = og.chunk_uw(Tm, kc, vc, bc, gcc, decay_w=decay_w)
                eu, ew = og.oc(u[b, sl, h], U), og.oc(w[b, sl, h], W)
                worst = max(worst, eu, ew)
                assert eu <= BF16_TOL and ew <= BF16_TOL, f"b={b} chunk={c} h={h}: oc(U)={eu:.3e} oc(W)={ew:.3e}"
    print(f"[gdn] chunk_uw C={C} worst oc {worst:.3e}", flush=True)


def test_gdn_chunk_uw_rejects_bad_shapes(gpu):
    import torch

    from qcom_htp_amd import _lib
    from qcom_htp_amd.gdn import gdn_chunk_uw

    k = torch.zeros((1, 96, 2, 128), dtype=torch.bfloat16, device=gpu)
    g = torch.zeros((1, 96, 2), dtype=torch.float32, device=gpu)
    with pytest.raises(_lib.QhtpError):
        gdn_chunk_uw(k, k, g, g, 64)  # 96 tokens is not a multiple of the 64-token chunk
    with pytest.raises(_lib.QhtpError):
        gdn_chunk_uw(k, k, g, g, 32)  # unsupported chunk


def _op_codes(A, sA):
    return np.clip(np.rint(A / sA), -32767, 32767).astype(np.int64)


@pytest.mark.parametrize("C", [16, 32, 48, 64])
@pytest.mark.parametrize("case", ["config4", "zero", "full_range"])
def test_gdn_op_model_codes_exact(gpu, C, case):
    """QH_GDN_OP_MODEL returns the GdnSolve op's own uint16 codes (gdn_solve_core.h:28-83 via
    GdnSolveOp.cpp:201-208), compared code for code with oracle.gdn.gdn_solve_op_u16, which is
    pinned to the op core compiled from the reference."""
    import torch

    from qcom_htp_amd.gdn import OP_MODEL, GdnSolve

    heads, zpA, zpT = 6, 32768, 32768
    sT = float(np.float32(2.0 / 32767.0))
    if case == "config4":
        k, beta, gc = og.config4_inputs(heads=heads, C=C, seed=70 + C)
        A = og.build_A(k, beta, gc)
        sA = float(np.float32(np.abs(A).max() / 32767.0))
        codes = _op_codes(A, sA)
    elif case == "zero":
        sA = 1e-4
        codes = np.zeros((heads, C, C), np.int64)
    else:  # full-range strictly-lower codes: clipping and int32 wrap-around paths
        rng = np.random.default_rng(C)
        codes = np.tril(rng.integers(-32767, 32768, (heads, C, C)), -1)
        sA = 3e-5
    Au = (codes + zpA).astype(np.uint16)
    print(f"[gdn] op model C={C} case={case}", flush=True)
    dev = torch.from_numpy(Au.view(np.int16)).to(gpu).view(torch.uint16)
    T = GdnSolve(dev, zpA, sA, zpT, sT, precision=OP_MODEL)
    torch.cuda.synchronize()
    got = T.cpu().view(torch.int16).numpy().view(np.uint16)
    want = og.gdn_solve_op_u16(Au, zpA, sA, zpT, sT)
    diff = np.count_nonzero(got != want)
    assert diff == 0, f"{diff} codes differ"


def test_gdn_op_model_rejects_large_chunks(gpu):
    import torch

    from qcom_htp_amd import _lib

    A = torch.zeros((1, 128, 128), dtype=torch.uint16, device=gpu)
    st = _lib.lib().qh_gdn_solve_u16(A.data_ptr(), A.data_ptr(), 1, 128, 32768, 32768, 1e-4, 1e-4, 2,
                                    int(torch.cuda.current_stream().cuda_stream))
    assert st == _lib.QH_STATUS_SHAPE_UNSUPPORTED
