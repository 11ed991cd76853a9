"""GPU parity of the quantized matmul family: HIP kernels vs the reference's oracle.

Bar: bit-exact.  The 7 named cases x 6 gated families at 256^3 are compared against the
sha256 of the reference generator's own ``output_ref_q`` (tests/golden/qmm_256.json); the
32x128x32 cases against the full golden arrays; other shapes against the oracle restatement
(itself pinned to the golden vectors by tests/test_oracle_qmm.py).
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import qmm as oq
from qcom_htp_amd import cases as C

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
GATE_META = json.loads((GOLD / "qmm_256.json").read_text())
SMALL = np.load(GOLD / "qmm_small.npz")


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).reshape(-1).tobytes()).hexdigest()


def run(case, gpu, path=0, rows=None):
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    op = QuantMatmul.from_case(case, device=gpu)
    act = case.activation_q if rows is None else case.activation_q[:rows]
    a = torch.from_numpy(np.ascontiguousarray(act)).to(gpu)
    out = op(a, path=path)
    torch.cuda.synchronize()
    res = out.cpu().numpy()
    op.close()
    return res


def diff_msg(got, want):
    bad = np.argwhere(got.astype(np.int64) != want.astype(np.int64))
    if bad.size == 0:
        return "identical"
    i, j = bad[0]
    return f"{len(bad)} mismatches, first at {tuple(bad[0])}: got {got[i, j]} want {want[i, j]}"


@pytest.mark.parametrize("fam", C.GATED_FAMILIES)
@pytest.mark.parametrize("case", C.CASES)
def test_gemm_seven_cases_256_bit_exact(gpu, fam, case):
    c = C.make_case(fam, case, 256, 256, 256)
    print(f"[qmm] {fam}/{case} 256^3 gemm", flush=True)
    got = run(c, gpu, path=1)
    want_sha = GATE_META[f"{fam}/{case}"]["sha256"]["output_q"]
    if sha(got) != want_sha:
        pytest.fail(f"{fam}/{case}: {diff_msg(got, oq.expected_output_case(c))}")


@pytest.mark.parametrize("fam", C.GATED_FAMILIES)
@pytest.mark.parametrize("case", C.CASES)
def test_small_cases_match_golden_arrays(gpu, fam, case):
    c = C.make_case(fam, case, 32, 128, 32)
    want = SMALL[f"{fam}/{case}/output_q"]
    print(f"[qmm] {fam}/{case} 32x128x32 gemm", flush=True)
    got = run(c, gpu, path=1)
    assert got.dtype == want.dtype
    assert np.array_equal(got, want), f"gemm: {diff_msg(got, want)}"
    # the decode GEMV takes at most 16 rows per call: run both halves
    print(f"[qmm] {fam}/{case} 32x128x32 gemv", flush=True)
    for r0 in (0, 16):
        sub = C.QmmCase(**{**c.__dict__, "activation_q": c.activation_q[r0:r0 + 16], "m": 16})
        got = run(sub, gpu, path=2)
        assert np.array_equal(got, want[r0:r0 + 16]), f"gemv rows {r0}..: {diff_msg(got, want[r0:r0 + 16])}"


@pytest.mark.parametrize("fam", C.GATED_FAMILIES)
@pytest.mark.parametrize("rows", [1, 3, 7, 13, 16])
def test_gemv_decode_rows_bit_exact(gpu, fam, rows):
    c = C.make_case(fam, "normal_random", 256, 256, 256)
    print(f"[qmm] {fam} gemv rows={rows}", flush=True)
    got = run(c, gpu, path=2, rows=rows)
    want = oq.expected_output_case(c)[:rows]
    assert np.array_equal(got, want), diff_msg(got, want)


@pytest.mark.parametrize("fam", ["w4a8_lpbq", "w4a16_lpbq"])
@pytest.mark.parametrize("block", [32, 64])
@pytest.mark.parametrize("rows", [1, 4, 6, 16])
def test_gemv_lpbq_block_scale_16_bit_exact(gpu, fam, block, rows):
    """LPBQ block scales over the reference's whole range [1, 16]: the factorisation gives 16 to a
    column's largest group (generate_qnn_matmul_python_cases.py:189-200), which selects the last
    entry of the per-(column, scale) tables of the 16-bit-activation GEMV."""
    c = C.synthetic_case(fam, 16, 1024, 256, seed=41 + block, lpbq_block=block, lpbq_max_scale=16)
    assert int(np.asarray(c.lpbq_block_int_scale).max()) == 16
    print(f"[qmm] {fam} gemv block={block} scales<=16 rows={rows}", flush=True)
    got = run(c, gpu, path=2, rows=rows)
    want = oq.expected_output_case(c)[:rows]
    assert np.array_equal(got, want), diff_msg(got, want)


@pytest.mark.parametrize("fam", ["w4a8_lpbq", "w4a16_lpbq"])
@pytest.mark.parametrize("rows", [1, 4, 6, 16])
def test_gemv_block_scale_16_near_ties_bit_exact(gpu, fam, rows):
    """Every block scale 16 and every row a near-tie row: weights 16 x code make the dot
    product even, so an odd bias puts t half way between two outputs and the float32 rounding
    residues of the weights decide the rounding."""
    import dataclasses

    from stress_cases import near_tie_case

    c = near_tie_case(fam, 16, 512, 96, 13, tie_rows=list(range(16)))
    codes = c.weight_q_nk.astype(np.int16)
    c = dataclasses.replace(
        c,
        lpbq_block_int_scale=np.full_like(c.lpbq_block_int_scale, 16),
        lpbq_expanded_q_nk=16 * codes,
        weight_deq=(16 * codes).astype(np.float32) * np.asarray(c.weight_scale, np.float32)[:, None],
    )
    print(f"[qmm] {fam} gemv all block scales 16, near ties, rows={rows}", flush=True)
    got = run(c, gpu, path=2, rows=rows)
    want = oq.expected_output_case(c)[:rows]
    assert np.array_equal(got, want), diff_msg(got, want)


@pytest.mark.parametrize("rows", [1, 4, 6, 16])
def test_gemv_block_scale_16_rail_activations_bit_exact(gpu, rows):
    """16-bit activations on the rails (0 or 65535, so the high byte is +-128) with every block
    scale 16: the high-byte rounding-residue sum the kernel forms exactly moves t by up to
    0.005 output LSB, well beyond the low-byte margin, so a residue table read for the wrong
    block scale changes outputs (2, 5, 5 and 12 of them at 1, 4, 6 and 16 rows for this seed)."""
    import dataclasses

    c = C.synthetic_case("w4a16_lpbq", 16, 1024, 2048, seed=3, lpbq_block=64, lpbq_max_scale=16)
    codes = c.weight_q_nk.astype(np.int16)
    rng = np.random.default_rng(103)
    x = np.where(rng.random(c.activation_q.shape) < 0.5, 0, 65535).astype(np.uint16)
    c = dataclasses.replace(
        c,
        activation_q=x,
        lpbq_block_int_scale=np.full_like(c.lpbq_block_int_scale, 16),
        lpbq_expanded_q_nk=16 * codes,
        weight_deq=(16 * codes).astype(np.float32) * np.asarray(c.weight_scale, np.float32)[:, None],
    )
    print(f"[qmm] w4a16_lpbq gemv rail activations, block scales 16, rows={rows}", flush=True)
    got = run(c, gpu, path=2, rows=rows)
    want = oq.expected_output_case(c)[:rows]
    assert np.array_equal(got, want), diff_msg(got, want)


@pytest.mark.parametrize("fam", ["w4a8_lpbq", "w4a16_lpbq"])
@pytest.mark.parametrize("rows", [1, 16])
def test_gemv_single_k_impulse_bit_exact(gpu, fam, rows):
    """The reference's single_k_impulse case (block scales up to 16) on the decode path."""
    c = C.make_case(fam, "single_k_impulse", 256, 256, 256)
    print(f"[qmm] {fam} single_k_impulse gemv rows={rows}", flush=True)
    got = run(c, gpu, path=2, rows=rows)
    want = oq.expected_output_case(c)[:rows]
    assert np.array_equal(got, want), diff_msg(got, want)


@pytest.mark.parametrize("fam", C.GATED_FAMILIES)
def test_accumulators_exact(gpu, fam):
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    c = C.synthetic_case(fam, 96, 512, 160, seed=11, lpbq_block=32, lpbq_max_scale=16)
    print(f"[qmm] {fam} accumulate 96x512x160", flush=True)
    op = QuantMatmul.from_case(c, device=gpu)
    acc = op.accumulate(torch.from_numpy(c.activation_q).to(gpu))
    torch.cuda.synchronize()
    want = oq.int_accumulator(c.activation_q, c.weight_int_nk, c.family.act_zp)
    np.testing.assert_array_equal(acc.cpu().numpy(), want)
    op.close()


SHAPES = [(1, 256, 32), (17, 96, 64), (300, 1024, 480), (257, 512, 288), (64, 4096, 256), (1, 4128, 544),
          (16, 4096, 96), (4, 8192, 64)]


@pytest.mark.parametrize("fam", C.GATED_FAMILIES)
@pytest.mark.parametrize("mkn", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_synthetic_shapes_bit_exact(gpu, fam, mkn):
    m, k, n = mkn
    F = C.FAMILIES[fam]
    if F.is_lpbq and k <= 64:
        pytest.skip("LPBQ needs K > block size")
    c = C.synthetic_case(fam, m, k, n, seed=m + k + n, lpbq_block=64 if k % 64 == 0 else 32)
    want = oq.expected_output_case(c)
    for path in ((1, 2) if m <= 16 else (1,)):
        print(f"[qmm] {fam} synthetic {m}x{k}x{n} path={path}", flush=True)
        got = run(c, gpu, path=path)
        assert np.array_equal(got, want), f"path {path}: {diff_msg(got, want)}"


def test_invalid_arguments_report_status(gpu):
    import torch

    from qcom_htp_amd import _lib
    from qcom_htp_amd.qmm import QuantMatmul

    c = C.make_case("u8i8", "normal_random", 32, 128, 32)
    op = QuantMatmul.from_case(c, device=gpu)
    with pytest.raises(TypeError):
        op(torch.zeros((4, 128), dtype=torch.uint16, device=gpu))
    with pytest.raises(ValueError):
        op(torch.zeros((4, 64), dtype=torch.uint8, device=gpu))
    with pytest.raises(_lib.QhtpError):
        op(torch.zeros((32, 128), dtype=torch.uint8, device=gpu), path=2)  # M=32 > 16 on the GEMV
    op.close()


@pytest.mark.parametrize("fam", C.GATED_FAMILIES)
def test_near_tie_outputs_bit_exact(gpu, fam):
    """Outputs packed next to rounding boundaries: per-tile lists under and over capacity
    (8-bit activations), exact ties left to the float64 emulation, ragged column tile."""
    from stress_cases import near_tie_case, stress_layout

    m, k, n, tie, zero, rail = stress_layout()
    c = near_tie_case(fam, m, k, n, 5, tie, zero, rail)
    want = oq.expected_output_case(c)
    print(f"[qmm] {fam} near-tie {m}x{k}x{n} gemm", flush=True)
    got = run(c, gpu, path=1)
    assert np.array_equal(got, want), f"gemm: {diff_msg(got, want)}"
    print(f"[qmm] {fam} near-tie rows 0..15 gemv", flush=True)
    got = run(c, gpu, path=2, rows=16)
    assert np.array_equal(got, want[:16]), f"gemv: {diff_msg(got, want[:16])}"


@pytest.mark.parametrize("fam", ["u8i8", "w4a8_per_channel", "w4a8_lpbq"])
@pytest.mark.parametrize("k", [512, 8192])
@pytest.mark.parametrize("rows", [1, 6, 16])
def test_gemv_exact_ties_bit_exact(gpu, fam, k, rows):
    """Power-of-two scales make every weight product exact (zero rounding residues) and the
    output scale puts odd integer dot products exactly half way between two outputs: the exact
    integer completion of 8-bit-activation outputs cannot settle them, so they take the
    term-by-term float64 recomputation, which rounds them half to even as the oracle does."""
    import dataclasses

    c = C.synthetic_case(fam, 16, k, 96, seed=43)
    rng = np.random.default_rng(44)
    zp = c.family.act_zp
    x = np.full_like(c.activation_q, zp)
    for r in range(16):
        pos = rng.choice(k, size=5, replace=False)
        x[r, pos] = zp + rng.integers(-3, 4, size=5)
    sA, sg = 2.0 ** -7, 2.0 ** -8
    w_int = c.lpbq_expanded_q_nk if c.lpbq_expanded_q_nk is not None else c.weight_q_nk
    c = dataclasses.replace(c, activation_q=x, act_scale=sA, weight_scale=np.full(96, sg, np.float32),
                            out_scale=2.0 * sA * sg, bias_q=rng.integers(-8, 8, size=96).astype(np.int32),
                            weight_deq=w_int.astype(np.float32) * np.float32(sg))
    want = oq.expected_output_case(c)[:rows]
    print(f"[qmm] {fam} exact-tie gemv rows={rows} k={k}", flush=True)
    got = run(c, gpu, path=2, rows=rows)
    assert np.array_equal(got, want), f"gemv: {diff_msg(got, want)}"


@pytest.mark.parametrize("fam", C.GATED_FAMILIES)
@pytest.mark.parametrize("k", [512, 8192])
@pytest.mark.parametrize("rows", [1, 4, 6, 16])
def test_gemv_near_tie_decode_rows_bit_exact(gpu, fam, k, rows):
    """Decode GEMV (1 to 16 rows) on tie / zero / rail rows: K = 512 recomputes uncertain
    outputs from the weight words the workgroup holds in registers, K = 8192 (more than one
    batch of k-groups per lane) re-reads them; 6 and 16 rows take the matrix-core path."""
    from stress_cases import near_tie_case

    c = near_tie_case(fam, 16, k, 96, 7, tie_rows=[0, 2, 9], zero_rows=[3, 12], rail_rows=[1, 15])
    want = oq.expected_output_case(c)[:rows]
    print(f"[qmm] {fam} near-tie gemv rows={rows} k={k}", flush=True)
    if c.family.act_bits == 16 and 2 * rows * k > 140 * 1024:
        # the forced GEMV path stages every row in LDS: 16-bit rows this long do not fit and the
        # entry point says so (the automatic path takes the GEMM for them)
        from qcom_htp_amd import _lib

        with pytest.raises(_lib.QhtpError) as ei:
            run(c, gpu, path=2, rows=rows)
        assert ei.value.status == _lib.QH_STATUS_SHAPE_UNSUPPORTED
        assert np.array_equal(run(c, gpu, path=0, rows=rows), want)
        return
    got = run(c, gpu, path=2, rows=rows)
    assert np.array_equal(got, want), f"gemv: {diff_msg(got, want)}"


@pytest.mark.parametrize("path,rows", [(1, 256), (0, 256), (2, 1), (2, 16), (1, 100)],
                         ids=["gemm", "auto", "gemv_m1", "gemv_m16", "gemm_ragged"])
def test_uniform_fixed_scale_u8i8_bit_exact(gpu, path, rows):
    """The u8i8 matmul as stated with fixed per-tensor parameters (U[0,255] activations at 0.02 /
    zero point 128, U[-127,127] weights at 0.01, bias U(+-2^15), output 0.05 / 0): 256^3, every
    output (most on the clip rails) equal to the oracle's."""
    c = C.uniform_u8i8_case(256, 256, 256, seed=1)
    want = oq.expected_output_case(c)[:rows]
    print(f"[qmm] uniform u8i8 path={path} rows={rows}", flush=True)
    got = run(c, gpu, path=path, rows=rows)
    assert np.array_equal(got, want), diff_msg(got, want)
