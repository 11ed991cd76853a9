"""GPU tests of the graph-level surface: reference case directories run on the GPU, CHAIN runs
(the reference's CHAIN=8 perf graphs), the torch.ops operators, and a captured HIP graph of
them replayed several times."""

from pathlib import Path

import numpy as np
import pytest

from oracle import qmm as oq
from qcom_htp_amd import cases as C

pytestmark = pytest.mark.gpu

DIRS = Path(__file__).resolve().parent / "golden" / "case_dirs"


def diff_msg(got, want):
    bad = np.argwhere(got.astype(np.int64) != want.astype(np.int64))
    return "identical" if bad.size == 0 else f"{len(bad)} mismatches, first at {tuple(bad[0])}"


@pytest.mark.parametrize("fam,case", [("u8i8", "normal_random"), ("w4a16_lpbq", "positive_boundary"),
                                      ("w4a8_per_group", "bias_only")])
def test_reference_case_directory_runs_bit_exact(gpu, fam, case):
    import torch

    from qcom_htp_amd.case_io import read_case
    from qcom_htp_amd.qmm import QuantMatmul

    c, out_ref = read_case(DIRS / fam / case)
    op = QuantMatmul.from_case(c, device=gpu)
    got = op(torch.from_numpy(c.activation_q).to(gpu)).cpu().numpy()
    op.close()
    assert np.array_equal(got, out_ref), diff_msg(got, out_ref)


def oracle_chain(c, steps, contract=None, divisor=1):
    F = c.family
    cur = c.activation_q
    for _ in range(steps):
        if contract is None:
            cur = oq.expected_output(cur, c.weight_int_nk, c.weight_scale, c.bias_q, c.act_scale, c.out_scale,
                                     F.act_zp, F.out_zp, F.out_bits, c.bias_float)
        else:
            acc = oq.int_accumulator(cur, c.weight_int_nk, F.act_zp)
            cur = oq.contract_output(acc, contract, divisor, c.bias_q, F.out_zp, F.out_bits)
    return cur


@pytest.mark.parametrize("fam", ["u8i8", "w8a16", "w4a8_lpbq", "w4a16_per_group"])
@pytest.mark.parametrize("chain", [1, 2, 8])
def test_chain_requant_matches_oracle(gpu, fam, chain):
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    c = C.make_case(fam, "normal_random", 256, 256, 256)
    op = QuantMatmul.from_case(c, device=gpu)
    print(f"[graph] {fam} chain={chain}", flush=True)
    got = op.chain(torch.from_numpy(c.activation_q).to(gpu), chain).cpu().numpy()
    op.close()
    want = oracle_chain(c, chain)
    assert np.array_equal(got, want), diff_msg(got, want)


def test_chain_legacy_contract_is_the_generators_reference(gpu):
    """gen_quant_chain's CHAIN reference: _make_reference_step applied chain times (:1542-1544)."""
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    c = C.make_case("u8i8", "normal_random", 128, 128, 128)
    op = QuantMatmul.from_case(c, device=gpu)
    got = op.chain(torch.from_numpy(c.activation_q).to(gpu), 8, "clip_i32").cpu().numpy()
    op.close()
    cur = c.activation_q
    for _ in range(8):
        cur = oq.reference_step(8, 8, 8, cur, c.weight_q_nk.T, c.bias_q, contract="legacy")
    assert np.array_equal(got, cur), diff_msg(got, cur)


def test_torch_ops_and_graph_replays(gpu):
    import torch

    from qcom_htp_amd import torch_ops
    from qcom_htp_amd.qmm import QuantMatmul

    c = C.make_case("w4a16_lpbq", "normal_random", 256, 256, 256)
    op = QuantMatmul.from_case(c, device=gpu)
    h = torch_ops.register(op)
    try:
        act = torch.from_numpy(c.activation_q).to(gpu)
        direct = op(act).cpu().numpy()
        assert np.array_equal(torch.ops.qhtp.qmm(act, h, 0).cpu().numpy(), direct)
        eager = torch.ops.qhtp.qmm_chain(act, h, 4, -1, 1)
        np.testing.assert_array_equal(eager.cpu().numpy(), oracle_chain(c, 4))
        k = torch.randn((1, 128, 2, 128), device=gpu).to(torch.bfloat16)
        g = torch.nn.functional.logsigmoid(torch.randn((1, 128, 2), device=gpu) + 3.0)
        b = torch.sigmoid(torch.randn((1, 128, 2), device=gpu))
        w0, u0 = torch.ops.qhtp.gdn_chunk_uw(k, k, g, b, 64, False, False)
        torch.cuda.synchronize()
        # a captured HIP graph of the operators, replayed with eager work in between
        static_act = act.clone()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out_g = torch.ops.qhtp.qmm_chain(static_act, h, 4, -1, 1)
            w_g, u_g = torch.ops.qhtp.gdn_chunk_uw(k, k, g, b, 64, False, False)
        for rep in range(3):
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out_g, eager), f"replay {rep}: chain differs"
            assert torch.equal(w_g, w0) and torch.equal(u_g, u0), f"replay {rep}: gdn differs"
            _ = op(act)  # eager work between replays
            torch.cuda.synchronize()
    finally:
        torch_ops.unregister(h)
        op.close()


def test_chain_rejects_bad_out_and_scratch(gpu):
    """Caller buffers of QuantMatmul.chain are checked like __call__'s (shape, dtype, device,
    contiguity) and must not overlap; the C entry point rejects overlapping ranges itself."""
    import torch

    from qcom_htp_amd import _lib
    from qcom_htp_amd.qmm import QuantMatmul

    c = C.make_case("u8i8", "normal_random", 64, 256, 256)
    op = QuantMatmul.from_case(c, device=gpu)
    try:
        act = torch.from_numpy(c.activation_q).to(gpu)
        m = act.shape[0]
        good = torch.empty((m, 256), dtype=torch.uint8, device=gpu)
        with pytest.raises(ValueError):
            op.chain(act, 2, out=torch.empty((m, 128), dtype=torch.uint8, device=gpu))
        with pytest.raises(ValueError):
            op.chain(act, 2, out=good, scratch=torch.empty((m - 1, 256), dtype=torch.uint8, device=gpu))
        with pytest.raises(ValueError):
            op.chain(act, 2, out=good, scratch=torch.empty((m, 256), dtype=torch.uint16, device=gpu))
        with pytest.raises(TypeError):
            op.chain(act, 2, out=torch.empty((m, 256), dtype=torch.uint8))
        big = torch.empty((2 * m, 256), dtype=torch.uint8, device=gpu)
        with pytest.raises(ValueError, match="overlap"):
            op.chain(act, 2, out=big[:m], scratch=big[m // 2: m // 2 + m])
        with pytest.raises(ValueError):
            op(act, out=torch.empty((m, 256), dtype=torch.uint8, device=gpu).t())
        # the C ABI: overlapping out / scratch ranges (not only equal pointers) are refused
        L = _lib.lib()
        st = L.qh_qmm_run_chain(op._h, m, 2, act.data_ptr(), big.data_ptr(), big.data_ptr() + 64, 0xFFFFFFFF, 1,
                                torch.cuda.current_stream().cuda_stream)
        assert st == _lib.QH_STATUS_INVALID_ARGUMENT and b"overlap" in L.qh_last_error()
        # a well-formed call still runs
        np.testing.assert_array_equal(op.chain(act, 2, out=good, scratch=big[m:]).cpu().numpy(), oracle_chain(c, 2))
    finally:
        op.close()


def oracle_graph_chain(gc, steps):
    """gen_quant_chain's CHAIN reference: _make_reference_step applied ``steps`` times (:1540-1544)."""
    cur = gc.activation
    for _ in range(steps):
        cur = oq.reference_step(gc.act_bits, gc.weight_bits, gc.out_bits, cur, gc.weight_compute_kn, gc.bias_q,
                                contract=gc.contract, family_name=gc.kernel_family)
    return cur


@pytest.mark.parametrize("name", list(C.GRAPH_FAMILIES))
def test_reference_graph_chains_256(gpu, name):
    """The reference's own CHAIN graphs at 256^3 (closed-form operands of gen_quant_chain.py:253-329,
    its per-family contract and bias): CHAIN = 1 and 8 against the reference step applied that many
    times, through qh_qmm_run_chain and the allocation-free chain."""
    import torch

    from qcom_htp_amd import _lib
    from qcom_htp_amd.qmm import CONTRACTS, QuantMatmul, graph_contract

    gc = C.graph_case(name)
    op = QuantMatmul.from_graph_case(gc, device=gpu)
    try:
        contract, d = graph_contract(gc)
        act = torch.from_numpy(gc.activation).to(gpu)
        for chain in (1, 8):
            print(f"[graph] reference graph {name} chain={chain} contract={contract}/{d}", flush=True)
            want = oracle_graph_chain(gc, chain)
            got = op.chain(act, chain, contract, d).cpu().numpy()
            assert np.array_equal(got, want), f"chain {chain}: {diff_msg(got, want)}"
        out = torch.empty((256, 256), dtype=op.out_dtype, device=gpu)
        _lib.check(_lib.lib().qh_qmm_run_chain_noalloc(op._h, 256, 8, act.data_ptr(), out.data_ptr(),
                                                       CONTRACTS[contract], d,
                                                       torch.cuda.current_stream().cuda_stream), "noalloc")
        torch.cuda.synchronize()
        assert np.array_equal(out.cpu().numpy(), want)
        if name == "u8i8":
            # gen_u8i8_chain's drain reference with the default record (scale 512.0 as half 0x6000,
            # baseline 0) is the same step: the closed-form drain contract gives the same chain
            got = op.chain(act, 8, "u8_drain", 0x6000).cpu().numpy()
            assert np.array_equal(got, want), f"u8 drain: {diff_msg(got, want)}"
    finally:
        op.close()


@pytest.mark.parametrize("case", list(C.W4A16_PRECISION_SUITE))
def test_w4a16_precision_suite(gpu, case):
    """The W4A16 precision case suite of run_qnn_kernel_e2e_ci.sh:429-455 (default, zp, k_impulse0/1/7)
    at 256^3 CHAIN=1 through the native floor-256 contract, and the same graphs at CHAIN=8."""
    import torch

    from qcom_htp_amd.qmm import QuantMatmul, graph_contract

    mode, kimp = C.W4A16_PRECISION_SUITE[case]
    gc = C.graph_case("w4a16_per_channel", mode=mode, impulse_k=kimp)
    op = QuantMatmul.from_graph_case(gc, device=gpu)
    try:
        contract, d = graph_contract(gc)
        assert (contract, d) == ("floor256_div_rint", 7)
        act = torch.from_numpy(gc.activation).to(gpu)
        for chain in (1, 8):
            print(f"[graph] w4a16 precision suite {case} chain={chain}", flush=True)
            want = oracle_graph_chain(gc, chain)
            got = op.run_contract(act, contract, d).cpu().numpy() if chain == 1 else \
                op.chain(act, chain, contract, d).cpu().numpy()
            assert np.array_equal(got, want), f"chain {chain}: {diff_msg(got, want)}"
    finally:
        op.close()


# ------------------------------------------------------- fused integer-contract chains (one launch)


def _mid_divisors(acc, out_bits):
    """Divisors that keep a contract's outputs spread over the output range, so that later steps
    of a chain see unsaturated activations: (name, divisor) for every contract."""
    qmax = (1 << out_bits) - 1
    d = max(1, int(round(float(np.std(acc)) / ((qmax + 1) / 6.0))))
    half = int(np.array([512.0 / d], np.float16).view(np.uint16)[0])
    out = [("clip_i32", 1), ("clip_i64", 1), ("div_rint", d), ("div_rint", 127), ("floor256_div_rint", d),
           ("round_div", d), ("round_div", 7)]
    if out_bits == 8:
        out.append(("u8_drain", half | ((128 << 7) << 16)))  # baseline 16384: + 128
    return out


@pytest.mark.parametrize("fam", ["u8i8", "w4a8_per_channel", "w4a8_lpbq", "w8a16", "w4a16_lpbq", "w4a8_per_group",
                                 "w4a16_per_group"])
@pytest.mark.parametrize("mk", [(1, 64), (45, 192), (256, 256), (33, 320)], ids=lambda s: f"m{s[0]}_k{s[1]}")
def test_contract_chain_matches_oracle_and_single_steps(gpu, fam, mk):
    """An integer-contract chain with K == N <= 256 runs every step in one launch (intermediate
    activations on chip); K = N = 320 takes one launch per step.  Either way, 5 steps equal the
    oracle's contract applied 5 times and 5 single-step contract launches, for every contract."""
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    m, k = mk
    c = C.synthetic_case(fam, m, k, k, seed=m + k)
    F = c.family
    op = QuantMatmul.from_case(c, device=gpu)
    act = torch.from_numpy(c.activation_q).to(gpu)
    acc1 = oq.int_accumulator(c.activation_q, c.weight_int_nk, F.act_zp)
    try:
        for name, d in _mid_divisors(acc1, F.out_bits):
            print(f"[graph] fused chain {fam} m={m} k=n={k} {name}/{d}", flush=True)
            want = oracle_chain(c, 5, name, d)
            got = op.chain(act, 5, name, d).cpu().numpy()
            assert np.array_equal(got, want), f"{name}/{d}: {diff_msg(got, want)}"
            cur = act
            for _ in range(5):
                cur = op.run_contract(cur, name, d)
            assert np.array_equal(cur.cpu().numpy(), want), f"single steps {name}/{d}"
    finally:
        op.close()


@pytest.mark.parametrize("mk", [(1, 32), (70, 256), (256, 256)], ids=lambda s: f"m{s[0]}_k{s[1]}")
def test_w16a16_contract_chain_matches_oracle(gpu, mk):
    """int16 weights (two byte planes and the all-ones plane) through the one-launch chain:
    5 steps of the W16A16 requantisation contract against the oracle's int16 accumulator."""
    import torch

    from qcom_htp_amd import _lib
    from qcom_htp_amd.qmm import QuantMatmul

    m, k = mk
    rng = np.random.default_rng(m * 7 + k)
    x = rng.integers(0, 65536, size=(m, k)).astype(np.uint16)
    q16 = rng.integers(-32768, 32768, size=(k, k)).astype(np.int16)
    q16[:, 0] = 32767
    q16[:, 1] = -32768
    op = QuantMatmul(q16, None, None, act_bits=16, out_bits=16, act_scale=1.0, out_scale=1.0, act_zp=32768,
                     out_zp=32768, weight_format=_lib.QH_WEIGHT_I16, device=gpu)
    try:
        acc1 = oq.w16a16_accumulator(x, q16, 32768)
        d = max(1, int(round(float(np.std(acc1)) / (65536 / 6.0))))
        for name, dd in (("div_rint", 32767), ("div_rint", d), ("round_div", d)):
            print(f"[graph] fused w16a16 chain m={m} k=n={k} {name}/{dd}", flush=True)
            cur = x
            for _ in range(5):
                cur = oq.contract_output(oq.w16a16_accumulator(cur, q16, 32768), name, dd, None, 32768, 16)
            got = op.chain(torch.from_numpy(x).to(gpu), 5, name, dd).cpu().numpy()
            assert np.array_equal(got, cur), f"{name}/{dd}: {diff_msg(got, cur)}"
    finally:
        op.close()


def test_contract_chain_graph_replays(gpu):
    """The one-launch contract chain captured in a HIP graph: every replay equals the eager chain
    (the kernel allocates nothing and clears nothing with memset)."""
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    c = C.synthetic_case("w4a8_lpbq", 256, 256, 256, seed=5)
    op = QuantMatmul.from_case(c, device=gpu)
    try:
        act = torch.from_numpy(c.activation_q).to(gpu)
        eager = op.chain(act, 8, "div_rint", 300).clone()
        out = torch.empty_like(eager)
        scratch = torch.empty_like(eager)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            op.chain(act, 8, "div_rint", 300, out=out, scratch=scratch)
        for rep in range(3):
            out.zero_()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {rep}"
        np.testing.assert_array_equal(eager.cpu().numpy(), oracle_chain(c, 8, "div_rint", 300))
    finally:
        op.close()
