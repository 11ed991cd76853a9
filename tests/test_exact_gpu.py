"""GPU parity of the exact integer GEMM: the per-group (K64) families, the reference's integer
output contracts and W16A16 (int16 weights as two byte planes).

Bar: bit-exact.  Per-group outputs at 256^3 are compared with the sha256 of the reference
generator's own ``output_ref_q`` (tests/golden/qmm_256.json), the 32x128x32 cases with the full
golden arrays, other shapes with the oracle; contracts and accumulators with the oracle's
restatements (pinned in tests/test_oracle_qmm.py).
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


def diff_msg(got, want):
    bad = np.argwhere(got.astype(np.int64) != want.astype(np.int64))
    if bad.size == 0:
        return "identical"
    i, j = bad[0]
    return f"{len(bad)} mismatches, first at {tuple(bad[0])}: got {got[i, j]} want {want[i, j]}"


def run(case, gpu, path=0):
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    op = QuantMatmul.from_case(case, device=gpu)
    out = op(torch.from_numpy(np.ascontiguousarray(case.activation_q)).to(gpu), path=path)
    torch.cuda.synchronize()
    res = out.cpu().numpy()
    op.close()
    return res


# ---------------------------------------------------------------------------------- per-group


@pytest.mark.parametrize("fam", C.PER_GROUP_FAMILIES)
@pytest.mark.parametrize("case", C.CASES)
def test_per_group_seven_cases_256_bit_exact(gpu, fam, case):
    c = C.make_case(fam, case, 256, 256, 256)
    print(f"[exact] {fam}/{case} 256^3", flush=True)
    got = run(c, gpu)
    if sha(got) != GATE_META[f"{fam}/{case}"]["sha256"]["output_q"]:
        pytest.fail(f"{fam}/{case}: {diff_msg(got, oq.expected_output_case(c))}")


@pytest.mark.parametrize("fam", C.PER_GROUP_FAMILIES)
@pytest.mark.parametrize("case", C.CASES)
def test_per_group_small_cases_match_golden_arrays(gpu, fam, case):
    c = C.make_case(fam, case, 32, 128, 32)
    want = SMALL[f"{fam}/{case}/output_q"]
    print(f"[exact] {fam}/{case} 32x128x32", flush=True)
    for path in (0, 2):  # every path runs the exact GEMM for per-group weights
        got = run(c, gpu, path=path)
        assert got.dtype == want.dtype
        assert np.array_equal(got, want), f"path {path}: {diff_msg(got, want)}"


PG_SHAPES = [(1, 256, 32), (17, 192, 64), (300, 1024, 480), (64, 4096, 256), (5, 8192, 96), (130, 512, 4128)]


@pytest.mark.parametrize("fam", C.PER_GROUP_FAMILIES)
@pytest.mark.parametrize("mkn", PG_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_per_group_synthetic_shapes_bit_exact(gpu, fam, mkn):
    m, k, n = mkn
    c = C.synthetic_case(fam, m, k, n, seed=m + k + n)
    want = oq.expected_output_case(c)
    print(f"[exact] {fam} synthetic {m}x{k}x{n}", flush=True)
    got = run(c, gpu)
    assert np.array_equal(got, want), diff_msg(got, want)


@pytest.mark.parametrize("fam", C.PER_GROUP_FAMILIES)
def test_per_group_full_size_4096_bit_exact(gpu, fam):
    c = C.synthetic_case(fam, 4096, 4096, 4096, seed=2)
    print(f"[exact] {fam} 4096^3: oracle", flush=True)
    want = oq.expected_output_case(c)
    print(f"[exact] {fam} 4096^3: gpu", flush=True)
    got = run(c, gpu)
    assert np.array_equal(got, want), diff_msg(got, want)


@pytest.mark.parametrize("fam", C.PER_GROUP_FAMILIES)
@pytest.mark.parametrize("tie_rows", [8, 64], ids=["listed", "over_capacity"])
def test_per_group_exact_ties(gpu, fam, tie_rows):
    """Power-of-two scales make every product exact, and the output scale makes odd integer
    dot products land exactly on half-integers: those outputs go through the float64
    emulation (listed; with 64 tie rows a 64 x 64 tile holds ~2000 of them, beyond the list)."""
    import dataclasses

    m, k, n = 128, 256, 128
    c = C.synthetic_case(fam, m, k, n, seed=41)
    rng = np.random.default_rng(42)
    zp = c.family.act_zp
    x = c.activation_q.copy()
    for r in range(tie_rows):
        x[r] = zp
        pos = rng.choice(k, size=5, replace=False)
        x[r, pos] = zp + rng.integers(-3, 4, size=5)
    sA, sg = 2.0 ** -7, 2.0 ** -8
    scales = np.full(c.weight_scale.shape, sg, np.float32)
    c = dataclasses.replace(c, activation_q=x, act_scale=sA, weight_scale=scales, out_scale=2.0 * sA * sg,
                            bias_float=(rng.integers(-8, 8, size=n) * (sA * sg)).astype(np.float32),
                            weight_deq=c.weight_q_nk.astype(np.float32) * sg)
    want = oq.expected_output_case(c)
    print(f"[exact] {fam} exact ties rows={tie_rows}", flush=True)
    got = run(c, gpu)
    assert np.array_equal(got, want), diff_msg(got, want)


@pytest.mark.parametrize("fam", C.PER_GROUP_FAMILIES)
def test_per_group_accumulate_is_raw_code_product(gpu, fam):
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    c = C.synthetic_case(fam, 70, 1024, 160, seed=9)
    op = QuantMatmul.from_case(c, device=gpu)
    acc = op.accumulate(torch.from_numpy(c.activation_q).to(gpu))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(acc.cpu().numpy(), oq.int_accumulator(c.activation_q, c.weight_q_nk, c.family.act_zp))
    op.close()


# ---------------------------------------------------------------------------- integer contracts


CONTRACT_CASES = [("clip_i32", 1), ("clip_i64", 1), ("div_rint", 127), ("div_rint", 7), ("floor256_div_rint", 7),
                  ("round_div", 7), ("round_div", 127)]


@pytest.mark.parametrize("fam", C.GATED_FAMILIES + C.PER_GROUP_FAMILIES)
def test_contracts_match_oracle(gpu, fam):
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    c = C.synthetic_case(fam, 45, 320, 96, seed=17)
    op = QuantMatmul.from_case(c, device=gpu)
    act = torch.from_numpy(c.activation_q).to(gpu)
    acc = oq.int_accumulator(c.activation_q, c.weight_int_nk, c.family.act_zp)
    for name, d in CONTRACT_CASES:
        print(f"[exact] {fam} contract {name} d={d}", flush=True)
        got = op.run_contract(act, name, d).cpu().numpy()
        want = oq.contract_output(acc, name, d, c.bias_q, c.family.out_zp, c.family.out_bits)
        assert np.array_equal(got, want), f"{name}/{d}: {diff_msg(got, want)}"
    op.close()


DRAIN_PARAMS = [(512.0, 0), (1.0, 32768), (2.0 ** -8, 16384), (-2.0, 0), (0.3, 0x1280), (2.0 ** -24, 65535)]


@pytest.mark.parametrize("fam", ["u8i8", "w4a8_per_channel"])
def test_u8_drain_contract_matches_oracle(gpu, fam):
    """QH_CONTRACT_U8_DRAIN (the closed-form A8 drain, act_zp 128) against the oracle, several
    half scales (normal, negative, subnormal) and baselines."""
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    c = C.synthetic_case(fam, 37, 256, 64, seed=23)
    assert c.family.act_zp == 128
    op = QuantMatmul.from_case(c, device=gpu)
    act = torch.from_numpy(c.activation_q).to(gpu)
    acc = oq.int_accumulator(c.activation_q, c.weight_int_nk, c.family.act_zp)
    for scale, baseline in DRAIN_PARAMS:
        d = int(np.array([scale], np.float16).view(np.uint16)[0]) | (baseline << 16)
        print(f"[exact] {fam} u8 drain s={scale} b={baseline}", flush=True)
        got = op.run_contract(act, "u8_drain", d).cpu().numpy()
        want = oq.contract_output(acc, "u8_drain", d, c.bias_q, c.family.out_zp, c.family.out_bits)
        assert np.array_equal(got, want), f"s={scale} b={baseline}: {diff_msg(got, want)}"
    op.close()


def test_contract_reference_models(gpu):
    """The reference's own integer models through the contracts: the legacy and native chain
    steps (gen_quant_chain.py:971-996), hmx_w4a16_lpbq_scalar_native (round_div7 on raw int4
    codes) and hmx_w4a8_lpbq_scalar (unit scale, act_zp 0, the effective bias)."""
    import torch

    from qcom_htp_amd import _lib
    from qcom_htp_amd.qmm import QuantMatmul

    rng = np.random.default_rng(5)
    m, k, n = 64, 512, 96

    def prep(w_nk, act_bits, out_bits, act_zp, out_zp, fmt, bias=None):
        return QuantMatmul(w_nk, np.ones(n, np.float32), bias, act_bits=act_bits, out_bits=out_bits, act_scale=1.0,
                           out_scale=1.0, act_zp=act_zp, out_zp=out_zp, weight_format=fmt, device=gpu)

    x16 = rng.integers(0, 65536, size=(m, k)).astype(np.uint16)
    x8 = rng.integers(0, 256, size=(m, k)).astype(np.uint8)
    w8 = rng.integers(-127, 128, size=(n, k)).astype(np.int8)
    w4 = rng.integers(-7, 8, size=(n, k)).astype(np.int8)
    bias = rng.integers(-(1 << 20), 1 << 20, size=n).astype(np.int32)
    a16 = torch.from_numpy(x16).to(gpu)
    a8 = torch.from_numpy(x8).to(gpu)
    checks = []
    op = prep(w8, 16, 16, 32768, 32768, _lib.QH_WEIGHT_I8, bias)
    checks.append(("legacy w8a16", op.run_contract(a16, "clip_i32"),
                   oq.reference_step(16, 8, 16, x16, w8.T, bias, contract="legacy")))
    checks.append(("native w8a16", op.run_contract(a16, "div_rint", 127),
                   oq.reference_step(16, 8, 16, x16, w8.T, None, contract="native", family_name="w8a16")))
    op.close()
    op = prep(w4, 16, 16, 32768, 32768, _lib.QH_WEIGHT_I4)
    checks.append(("native w4a16", op.run_contract(a16, "floor256_div_rint", 7),
                   oq.reference_step(16, 4, 16, x16, w4.T, None, contract="native", family_name="w4a16")))
    checks.append(("w4a16 lpbq scalar native", op.run_contract(a16, "round_div", 7),
                   oq.w4a16_lpbq_scalar_native(x16, w4.T)))
    op.close()
    eff = (-128 * w4.astype(np.int64).sum(1) + bias).astype(np.int32)
    op = prep(w4, 8, 8, 0, 0, _lib.QH_WEIGHT_I4, eff)
    checks.append(("w4a8 lpbq scalar", op.run_contract(a8, "clip_i64"), oq.w4a8_lpbq_scalar(eff, w4.T, x8)))
    op.close()
    op = prep(w8, 8, 8, 128, 0, _lib.QH_WEIGHT_I8, bias)
    checks.append(("legacy u8i8", op.run_contract(a8, "clip_i32"),
                   oq.reference_step(8, 8, 8, x8, w8.T, bias, contract="legacy")))
    op.close()
    torch.cuda.synchronize()
    for name, got, want in checks:
        got = got.cpu().numpy()
        assert np.array_equal(got, want), f"{name}: {diff_msg(got, want)}"


# ------------------------------------------------------------------------------------- W16A16


@pytest.mark.parametrize("mkn", [(1, 256, 64), (70, 512, 96), (130, 4096, 160)], ids=lambda s: "x".join(map(str, s)))
def test_w16a16_two_byte_planes_exact(gpu, mkn):
    import torch

    from qcom_htp_amd import _lib
    from qcom_htp_amd.qmm import QuantMatmul

    m, k, n = mkn
    rng = np.random.default_rng(m + k)
    x = rng.integers(0, 65536, size=(m, k)).astype(np.uint16)
    q16 = rng.integers(-32768, 32768, size=(n, k)).astype(np.int16)
    q16[:, 0] = 32767  # the ends of the int16 range (symmetric quantisation reaches +-32767)
    q16[:, 1] = -32768
    op = QuantMatmul(q16, None, None, act_bits=16, out_bits=16, act_scale=1.0, out_scale=1.0, act_zp=32768,
                     out_zp=32768, weight_format=_lib.QH_WEIGHT_I16, device=gpu)
    act = torch.from_numpy(x).to(gpu)
    print(f"[exact] w16a16 {m}x{k}x{n}", flush=True)
    acc = op.accumulate(act).cpu().numpy()
    want = oq.w16a16_accumulator(x, q16, 32768)
    np.testing.assert_array_equal(acc, want)
    out = op.run_contract(act, "div_rint", 32767).cpu().numpy()
    w_out = oq.contract_output(want, "div_rint", 32767, None, 32768, 16)
    assert np.array_equal(out, w_out), diff_msg(out, w_out)
    with pytest.raises(_lib.QhtpError) as ei:
        op(act)  # no float requantisation for int16 weights
    assert ei.value.status == _lib.QH_STATUS_UNSUPPORTED
    op.close()
