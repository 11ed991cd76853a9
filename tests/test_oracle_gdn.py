"""CPU tests pinning the GDN oracle: independent algorithms agree, closed forms hold, and the
int16 block model matches the reference's own C model compiled from its sources."""

import subprocess
from pathlib import Path

import numpy as np
import pytest

from oracle import gdn as og

REF_DIR = Path(__file__).resolve().parents[1] / "oracle" / "_ref"


def test_inverse_agrees_with_forward_substitution():
    k, beta, gc = og.config4_inputs(heads=4, C=64, seed=1)
    A = og.build_A(k, beta, gc)
    T1 = og.inverse_fp64(A)
    T2 = og.forward_subst(A)
    assert og.oc(T2, T1) < 1e-12
    eye = np.eye(64)
    for h in range(4):
        np.testing.assert_allclose(T1[h] @ (eye - A[h]), eye, atol=1e-10)


def test_neumann_closed_form_small():
    rng = np.random.default_rng(3)
    C = 12
    A = np.tril(rng.standard_normal((C, C)) * 0.3, -1)
    series = np.eye(C)
    P = np.eye(C)
    for _ in range(C):
        P = P @ A
        series = series + P
    np.testing.assert_allclose(og.inverse_fp64(A[None])[0], series, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(og.forward_subst(A), series, rtol=1e-10, atol=1e-12)


def test_build_A_special_cases():
    rng = np.random.default_rng(5)
    k = rng.standard_normal((1, 8, 16))
    gc = -np.abs(rng.standard_normal((1, 8)))
    assert np.all(og.build_A(k, np.zeros((1, 8)), gc) == 0.0)
    # orthogonal keys -> no interaction
    ko = np.eye(8)[None, :, :8]
    assert np.allclose(og.build_A(ko, np.ones((1, 8)), gc), 0.0)
    # two tokens: A[1,0] = -beta_1 * cos(k0, k1) * exp(gc_1)
    k2 = rng.standard_normal((2, 4))
    b = np.array([0.3, 0.7])
    g = np.array([-0.2, -0.5])
    A = og.build_A(k2[None], b[None], g[None])[0]
    cos = k2[0] @ k2[1] / np.sqrt((k2[0] @ k2[0] + 1e-6) * (k2[1] @ k2[1] + 1e-6))
    assert A[0, 0] == 0 and A[0, 1] == 0 and A[1, 1] == 0
    assert np.isclose(A[1, 0], -0.7 * cos * np.exp(-0.5))


def test_oc_definition():
    T = np.ones((2, 3, 3))
    assert og.oc(T, T) == 0.0
    assert np.isclose(og.oc(2 * T, T), 1.0)


def test_u16_codes_roundtrip():
    x = np.linspace(-1.5, 1.5, 101)
    q = og.quantize_u16(x, og.ST_REF)
    np.testing.assert_allclose(og.dequantize_u16(q, og.ST_REF), x, atol=og.ST_REF / 2 + 1e-15)


def _int16_codes(A):
    sA = float(np.abs(A).max() / 32767.0)
    return np.clip(np.rint(A / sA), -32767, 32767).astype(np.int16), sA


@pytest.mark.skipif(not (REF_DIR / "gdn_solve_ref").exists(), reason="oracle/_ref not built (needs /root/reference)")
def test_int16_block_model_matches_reference_c(tmp_path):
    k, beta, gc = og.config4_inputs(heads=3, C=64, seed=7)
    A = og.build_A(k, beta, gc)
    codes, sAs = [], []
    for h in range(3):
        q, s = _int16_codes(A[h])
        codes.append(q)
        sAs.append(s)
    sT = 2.0 / 32767.0
    np.array([3, 64], np.int32).tofile(tmp_path / "dims.i32")
    np.stack(codes).astype(np.int16).tofile(tmp_path / "A_codes.i16")
    np.array(sAs, np.float32).tofile(tmp_path / "sA.f32")
    np.array([sT], np.float32).tofile(tmp_path / "sT.f32")
    subprocess.run([str(REF_DIR / "gdn_solve_ref")], cwd=tmp_path, check=True, capture_output=True)
    T_ref = np.fromfile(tmp_path / "T_out.f64", np.float64).reshape(3, 64, 64)
    for h in range(3):
        # the C model reads sA as float32 and sT as float32
        T_py = og.solve_int16_blocks(codes[h], float(np.float32(sAs[h])), float(np.float32(sT)))
        np.testing.assert_allclose(T_py, T_ref[h], rtol=0, atol=1e-12)
        # and the model is a faithful inverse at its int16 precision
        assert og.oc(T_py, og.inverse_fp64(codes[h].astype(np.float64) * np.float32(sAs[h]))) < 5e-4


def test_chunk_uw_solves_the_triangular_system():
    """U and W from chunk_uw satisfy (I - A) U = beta V and (I - A) W = beta K^ (e^g)."""
    rng = np.random.default_rng(3)
    C = 32
    k = rng.standard_normal((C, 128))
    v = rng.standard_normal((C, 128))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal(C)))
    gc = -np.logaddexp(0.0, -(rng.standard_normal(C) + 3.0))
    A = og.build_A(k, beta, gc)
    T = og.inverse_fp64(A)
    ImA = np.eye(C) - A
    for decay_w in (False, True):
        U, W = og.chunk_uw(T, k, v, beta, gc, decay_w=decay_w)
        np.testing.assert_allclose(ImA @ U, beta[:, None] * v, rtol=0, atol=1e-10)
        kb = beta[:, None] * og.l2norm(k)
        if decay_w:
            kb = kb * np.exp(np.cumsum(gc))[:, None]
        np.testing.assert_allclose(ImA @ W, kb, rtol=0, atol=1e-10)


def test_torch_row_recurrence_matches_lapack():
    import torch

    k, beta, gc = og.config4_inputs(heads=3, C=96, seed=12)
    A = og.build_A(k, beta, gc)
    T = og.forward_subst_torch(torch.from_numpy(A)).numpy()
    assert og.oc(T, og.inverse_fp64(A)) < 1e-12


@pytest.mark.parametrize("decay_w", [False, True])
def test_torch_stage_a_matches_lapack_products(decay_w):
    import torch

    rng = np.random.default_rng(13)
    n, C = 3, 64
    k = rng.standard_normal((n, C, 128))
    v = rng.standard_normal((n, C, 128))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((n, C))))
    gc = -np.logaddexp(0.0, -(rng.standard_normal((n, C)) + 3.0))
    U, W = og.chunk_stage_a_torch(torch.from_numpy(k), torch.from_numpy(v), torch.from_numpy(gc),
                                  torch.from_numpy(beta), decay_w=decay_w)
    Uref, Wref = og.chunk_uw(og.inverse_fp64(og.build_A(k, beta, gc)), k, v, beta, gc, decay_w=decay_w)
    assert og.oc(U.numpy(), Uref) < 1e-12
    assert og.oc(W.numpy(), Wref) < 1e-12


@pytest.mark.parametrize("C", [16, 64, 256])
@pytest.mark.parametrize("decay_w", [False, True])
def test_stage_a_triangular_solve_form_matches_recurrence(decay_w, C):
    """chunk_stage_a_solve_torch (batched unit-lower solve, used for the full-size checks) equals the
    row recurrence of the reference kernel and the LAPACK inverse, and a wrong decay sign is caught."""
    import torch

    rng = np.random.default_rng(C + decay_w)
    n = 3
    k = rng.standard_normal((n, C, 128))
    v = rng.standard_normal((n, C, 128))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((n, C))))
    gc = -np.logaddexp(0.0, -(rng.standard_normal((n, C)) + 3.0))
    U, W = og.chunk_stage_a_solve_torch(k, v, gc, beta, decay_w=decay_w)
    U2, W2 = og.chunk_stage_a_torch(k, v, gc, beta, decay_w=decay_w)
    Uref, Wref = og.chunk_uw(og.inverse_fp64(og.build_A(k, beta, gc)), k, v, beta, gc, decay_w=decay_w)
    for X, R in ((U, U2), (W, W2), (U, Uref), (W, Wref)):
        assert og.oc(np.asarray(X), np.asarray(R)) < 1e-11
    Ubad, _ = og.chunk_stage_a_solve_torch(k, v, -gc, beta, decay_w=decay_w)
    assert og.oc(Ubad.numpy(), Uref) > 1e-3


def _seq_inputs(n=3, T=100, D=16, seed=0):
    rng = np.random.default_rng(seed)
    q, k, v = (rng.standard_normal((n, T, D)) for _ in range(3))
    gc = -np.logaddexp(0.0, -(rng.standard_normal((n, T)) + 3.0))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((n, T))))
    return q, k, v, gc, beta


@pytest.mark.parametrize("C", [16, 32, 64])
@pytest.mark.parametrize("with_state", [False, True])
def test_chunked_prefill_equals_token_recurrence(C, with_state):
    """The chunked stage A + stage B equals the gated delta rule applied token by token, for
    every chunk size, with zero padding of a ragged T and with an incoming state."""
    q, k, v, gc, beta = _seq_inputs()
    S0 = np.random.default_rng(1).standard_normal((3, 16, 16)) * 0.1 if with_state else None
    o_r, S_r = og.gdn_recurrent(q, k, v, gc, beta, S0)
    o_c, S_c = og.gdn_prefill_torch(q, k, v, gc, beta, C, S0)
    assert float((o_c - o_r).abs().max()) < 1e-12
    assert float((S_c - S_r).abs().max()) < 1e-12


@pytest.mark.parametrize("plant", ["state_decay", "transpose_S", "strict_causal", "q_decay", "k_decay", "w_form"])
def test_chunk_state_plausible_mistakes_are_caught(plant):
    """Each plausible mistake planted in the chunked oracle (a dropped decay of the state, of q or
    of k, a transposed state read, a causal mask without its diagonal, W without e^g) makes it
    differ from the token-by-token recurrence, with an incoming state and over several chunks."""
    q, k, v, gc, beta = _seq_inputs(T=96)
    S0 = np.random.default_rng(2).standard_normal((3, 16, 16)) * 0.3
    o_r, S_r = og.gdn_recurrent(q, k, v, gc, beta, S0)
    if plant == "w_form":
        U, W = og.chunk_stage_a_torch(k.reshape(-1, 32, 16), v.reshape(-1, 32, 16), gc.reshape(-1, 32),
                                      beta.reshape(-1, 32), decay_w=False)
        o_bad, S_bad = og.chunk_state_torch(q, k, gc, W.reshape(3, 96, 16), U.reshape(3, 96, 16), S0, 32)
    else:
        o_bad, S_bad = og.gdn_prefill_torch(q, k, v, gc, beta, 32, S0, _plant=plant)
    err = max(float((o_bad - o_r).abs().max()), float((S_bad - S_r).abs().max()))
    assert err > 1e-3, (plant, err)
    o_ok, S_ok = og.gdn_prefill_torch(q, k, v, gc, beta, 32, S0)
    assert float((o_ok - o_r).abs().max()) < 1e-12 and float((S_ok - S_r).abs().max()) < 1e-12


@pytest.mark.skipif(not (REF_DIR / "gdn_test_core").exists(), reason="oracle/_ref not built (needs /root/reference)")
@pytest.mark.parametrize("case", ["config4", "full_range"])
@pytest.mark.parametrize("C", [16, 32, 64])
def test_int16_op_model_matches_reference_core(tmp_path, C, case):
    """solve_int16_op reproduces the op core's int8 output codes (gdn_solve_core.h through its
    own host driver test_core.cpp, sTout = 1/127) code for code.  ``full_range``: strictly-lower
    codes uniform over [-32767, 32767] at a small scale, which drive the int16 clip and the
    int32 wrap-around of the diagonal solves (the GPU op-model test's full-range case)."""
    H = 3
    codes, sAs = [], []
    if case == "config4":
        k, beta, gc = og.config4_inputs(heads=H, C=C, seed=17 + C)
        A = og.build_A(k, beta, gc)
        for h in range(H):
            q, s = _int16_codes(A[h])
            codes.append(q)
            sAs.append(s)
    else:
        rng = np.random.default_rng(C)
        for h in range(H):
            codes.append(np.tril(rng.integers(-32767, 32768, (C, C)), -1).astype(np.int16))
            sAs.append(3e-5)
    np.array([H, C], np.int32).tofile(tmp_path / "dims.i32")
    np.stack(codes).astype(np.int16).tofile(tmp_path / "A_codes.i16")
    np.array(sAs, np.float32).tofile(tmp_path / "sA.f32")
    subprocess.run([str(REF_DIR / "gdn_test_core")], cwd=tmp_path, check=True, capture_output=True)
    T_ref = np.fromfile(tmp_path / "T_i8.f64", np.float64).reshape(H, C, C)
    sTout = np.float32(1.0) / np.float32(127.0)
    ref_codes = np.rint(T_ref / np.float64(sTout)).astype(np.int64)
    for h in range(H):
        got = og.solve_int16_op(codes[h], float(np.float32(sAs[h])), float(sTout), 127.0)
        assert np.array_equal(got, ref_codes[h]), f"head {h}: {np.count_nonzero(got != ref_codes[h])} codes differ"


def test_int16_op_model_tracks_float64_block_model():
    """The op's float32 model and the float64 block model are the same algorithm: their T agree
    to float32 rounding (int16 output codes within one unit)."""
    k, beta, gc = og.config4_inputs(heads=2, C=64, seed=23)
    A = og.build_A(k, beta, gc)
    sT = 2.0 / 32767.0
    for h in range(2):
        q, s = _int16_codes(A[h])
        s32 = float(np.float32(s))
        codes = og.solve_int16_op(q, s32, sT, 32767.0)
        T64 = og.solve_int16_blocks(q, s32, float(np.float32(sT)))
        assert np.abs(codes - np.clip(np.rint(T64 / sT), -32767, 32767)).max() <= 1
        assert np.all(np.triu(codes, 1) == 0)


def test_op_u16_contract_wraps_the_model():
    """gdn_solve_op_u16 = model(codes - zpA) + zpT, zero (= zpT) above the diagonal."""
    k, beta, gc = og.config4_inputs(heads=1, C=32, seed=29)
    A = og.build_A(k, beta, gc)[0]
    q, s = _int16_codes(A)
    Au = (q.astype(np.int64) + 32768).astype(np.uint16)
    out = og.gdn_solve_op_u16(Au[None], 32768, s, 32768, 2.0 / 32767.0)[0]
    assert np.array_equal(out.astype(np.int64) - 32768, og.solve_int16_op(q, s, 2.0 / 32767.0, 32767.0))
    assert np.all(out[np.triu_indices(32, 1)] == 32768)
