"""CPU tests of the case-directory reader / writer against directories the reference
generator wrote itself (tests/golden/case_dirs, made by tests/golden/make_case_dirs.py), and of
the torch.ops registration (shape propagation only; no kernel runs)."""

import json
from pathlib import Path

import numpy as np
import pytest

from oracle import qmm as oq
from qcom_htp_amd import cases as C
from qcom_htp_amd.case_io import read_case, write_case

DIRS = Path(__file__).resolve().parent / "golden" / "case_dirs"
PAIRS = [("u8i8", "normal_random"), ("w4a16_lpbq", "positive_boundary"), ("w4a8_per_group", "bias_only")]


@pytest.mark.parametrize("fam,case", PAIRS)
def test_reader_loads_reference_directory(fam, case):
    c, out_ref = read_case(DIRS / fam / case)
    g = C.make_case(fam, case, 32, 128, 32)
    assert c.family.name == fam and (c.m, c.k, c.n) == (32, 128, 32)
    assert c.act_scale == g.act_scale and c.out_scale == g.out_scale
    for name in ("activation_q", "weight_q_nk", "weight_scale", "bias_q"):
        np.testing.assert_array_equal(getattr(c, name), getattr(g, name), err_msg=name)
    if c.family.is_lpbq:
        np.testing.assert_array_equal(c.lpbq_block_int_scale, g.lpbq_block_int_scale)
        np.testing.assert_array_equal(c.lpbq_expanded_q_nk, g.lpbq_expanded_q_nk)
    if c.family.weight_schema == "per_group":
        np.testing.assert_array_equal(c.bias_float, g.bias_float)
    # the oracle on the loaded case reproduces the reference's own output_ref_q
    np.testing.assert_array_equal(oq.expected_output_case(c), out_ref)


@pytest.mark.parametrize("fam,case", PAIRS)
def test_writer_round_trip_and_schema(tmp_path, fam, case):
    c, out_ref = read_case(DIRS / fam / case)
    d = write_case(c, tmp_path, out_ref)
    c2, out2 = read_case(d)
    np.testing.assert_array_equal(out2, out_ref)
    for name in ("activation_q", "weight_q_nk", "weight_scale", "bias_q"):
        a, b = getattr(c, name), getattr(c2, name)
        assert a.dtype == b.dtype, name
        np.testing.assert_array_equal(a, b, err_msg=name)
    ours = json.loads((d / "case.json").read_text())
    ref = json.loads((DIRS / fam / case / "case.json").read_text())
    assert ours["schema"] == ref["schema"]
    for key in ("family", "kernel_family", "weight_schema_variant", "case", "seed", "shape_mkn"):
        assert ours[key] == ref[key], key
    for part in ("activation", "weight", "bias", "output"):
        for key, val in ours["qparams"][part].items():
            assert key in ref["qparams"][part], (part, key)
            assert val == ref["qparams"][part][key], (part, key)
    for name, entry in ours["files"].items():
        r = ref["files"][name]
        for key in ("npy", "raw", "raw_sha256", "shape", "dtype", "min", "max", "unique_count", "first8"):
            assert entry[key] == r[key], (name, key)
    assert ours["output_counts"] == ref["output_counts"]


def test_torch_ops_registered_with_fake_shapes():
    import torch
    from torch._subclasses.fake_tensor import FakeTensorMode

    from qcom_htp_amd import torch_ops

    for name in ("qmm", "qmm_contract", "qmm_chain", "qmm_accumulate", "lpbq_expand_to_i8", "gdn_solve",
                 "gdn_solve_u16", "gdn_chunk_uw"):
        assert hasattr(torch.ops.qhtp, name), name

    class Stub:  # shape-only stand-in for a prepared matmul
        n = 96
        out_dtype = torch.uint16

    h = torch_ops.register(Stub())
    try:
        with FakeTensorMode():
            act = torch.empty((5, 64), dtype=torch.uint16)
            assert torch.ops.qhtp.qmm(act, h, 0).shape == (5, 96)
            assert torch.ops.qhtp.qmm_chain(act, h, 4, -1, 1).dtype == torch.uint16
            assert torch.ops.qhtp.qmm_accumulate(act, h).dtype == torch.int64
            k = torch.empty((2, 128, 3, 128), dtype=torch.bfloat16)
            g = torch.empty((2, 128, 3), dtype=torch.float32)
            w, u = torch.ops.qhtp.gdn_chunk_uw(k, k, g, g, 64, False, True)
            assert w.shape == k.shape and w.dtype == torch.float32
            assert torch.ops.qhtp.lpbq_expand_to_i8(torch.empty((1, 1, 64, 32), dtype=torch.uint8),
                                                    torch.empty((1, 1, 1, 128), dtype=torch.uint8)).shape == (1, 1, 128, 32)
    finally:
        torch_ops.unregister(h)
