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
