"""GPU test of qh_qmm_run_chain_noalloc (the chain entry point whose intermediate results live
in a static per-device array): through the C ABI, bit-exact against qh_qmm_run_chain with a
caller scratch buffer, on two calls in a row, the second with a smaller input; and the size
limit reported as a status."""

import ctypes as C

import numpy as np
import pytest

from qcom_htp_amd import cases

pytestmark = pytest.mark.gpu


def _run_both(op, act, m, chain, contract, divisor):
    import torch

    from qcom_htp_amd import _lib

    L = _lib.lib()
    stream = torch.cuda.current_stream().cuda_stream
    ref = torch.empty((m, op.n), dtype=op.out_dtype, device=act.device)
    scr = torch.empty_like(ref)
    _lib.check(L.qh_qmm_run_chain(op._h, m, chain, act.data_ptr(), ref.data_ptr(), scr.data_ptr(), contract, divisor,
                                  stream), "qh_qmm_run_chain")
    out = torch.full((m, op.n), 7, dtype=op.out_dtype, device=act.device)
    _lib.check(L.qh_qmm_run_chain_noalloc(op._h, m, chain, act.data_ptr(), out.data_ptr(), contract, divisor, stream),
               "qh_qmm_run_chain_noalloc")
    torch.cuda.synchronize()
    return out.cpu().numpy(), ref.cpu().numpy()


@pytest.mark.parametrize("fam,contract,divisor", [("u8i8", 0xFFFFFFFF, 1), ("w8a16", 0xFFFFFFFF, 1),
                                                  ("w4a16_lpbq", 2, 127)])
def test_chain_noalloc_matches_chain_with_scratch(gpu, fam, contract, divisor):
    import torch

    from qcom_htp_amd.qmm import QuantMatmul

    c = cases.make_case(fam, "normal_random", 256, 256, 256)
    op = QuantMatmul.from_case(c, device=gpu)
    act = torch.from_numpy(c.activation_q).to(gpu)
    for m, chain in ((256, 8), (40, 3)):  # the second call is smaller
        print(f"[noalloc] {fam} m={m} chain={chain}", flush=True)
        got, want = _run_both(op, act[:m].contiguous(), m, chain, contract, divisor)
        assert np.array_equal(got, want), f"m={m} chain={chain}: {int((got != want).sum())} mismatches"
    op.close()


def test_chain_noalloc_rejects_outputs_beyond_the_static_scratch(gpu):
    import torch

    from qcom_htp_amd import _lib
    from qcom_htp_amd.qmm import QuantMatmul

    c = cases.synthetic_case("w8a16", 32, 2048, 2048, seed=3)
    op = QuantMatmul.from_case(c, device=gpu)
    m = 4096  # 4096 x 2048 u16 outputs = 16 MiB > 8 MiB
    act = torch.zeros((m, 2048), dtype=torch.uint16, device=gpu)
    out = torch.empty((m, 2048), dtype=torch.uint16, device=gpu)
    st = _lib.lib().qh_qmm_run_chain_noalloc(op._h, m, 2, act.data_ptr(), out.data_ptr(), 0xFFFFFFFF, 1,
                                             torch.cuda.current_stream().cuda_stream)
    assert st == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert b"static scratch" in _lib.lib().qh_last_error()
    op.close()


def test_chain_noalloc_under_graph_capture(gpu):
    """The use the entry point exists for: captured into a HIP graph (no allocation is possible
    during capture), replayed several times with eager work in between, every replay equal to
    the chain with a caller scratch buffer run eagerly."""
    import torch

    from qcom_htp_amd import _lib
    from qcom_htp_amd.qmm import QuantMatmul

    L = _lib.lib()
    c = cases.make_case("w4a8_lpbq", "normal_random", 256, 256, 256)
    op = QuantMatmul.from_case(c, device=gpu)
    act = torch.from_numpy(c.activation_q).to(gpu)
    m, chain = 256, 4
    print(f"[noalloc graph] w4a8_lpbq m={m} chain={chain}", flush=True)
    want = torch.empty((m, op.n), dtype=op.out_dtype, device=gpu)
    scr = torch.empty_like(want)
    _lib.check(L.qh_qmm_run_chain(op._h, m, chain, act.data_ptr(), want.data_ptr(), scr.data_ptr(), 0xFFFFFFFF, 1,
                                  torch.cuda.current_stream().cuda_stream), "qh_qmm_run_chain")
    out = torch.zeros_like(want)
    other_act = act.flip(0).contiguous()
    other_out = torch.empty_like(want)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _lib.check(L.qh_qmm_run_chain_noalloc(op._h, m, chain, act.data_ptr(), out.data_ptr(), 0xFFFFFFFF, 1,
                                              torch.cuda.current_stream().cuda_stream), "noalloc (capture)")
    for rep in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {rep}: {int((out != want).sum())} mismatches"
        # eager work between replays, which also overwrites the shared static array
        _lib.check(L.qh_qmm_run_chain_noalloc(op._h, m, chain, other_act.data_ptr(), other_out.data_ptr(), 0xFFFFFFFF,
                                              1, torch.cuda.current_stream().cuda_stream), "noalloc (eager)")
        torch.cuda.synchronize()
    op.close()
