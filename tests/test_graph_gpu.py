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
