"""GPU parity of the op-level mirror: the reference's carriers and op names end to end.

* ``qh_w4_lpbq_expand_to_i8`` (the HmxW4LpbqExpandToI8 op) against the oracle's restatement
  of the C++ op, byte for byte, including saturating scales, and at the 4096 x 14336 LPBQ
  weight of the decode benchmark against the generator's logical expansion + K-major pack.
* Every gated family at 256^3 built from the carrier the reference op reads (or the DLC
  carrier with the sign toggle), called with a ``[1, M/32, 32, K]`` activation: the output
  must hash to the reference generator's own ``output_ref_q`` (tests/golden/qmm_256.json).
  The LPBQ families run the reference's two-op chain (expand, then the W8 matmul).
"""

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from oracle import layouts as L
from qcom_htp_amd import _lib
from qcom_htp_amd import cases as C

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
GATE_META = json.loads((GOLD / "qmm_256.json").read_text())


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).reshape(-1).tobytes()).hexdigest()


def expand_on_gpu(gpu, packed_kpair, scales_flat, k, n):
    import torch

    from qcom_htp_amd.ops import HmxW4LpbqExpandToI8

    wl = torch.from_numpy(np.ascontiguousarray(packed_kpair).reshape(1, 1, k // 2, n)).to(gpu)
    sc = torch.from_numpy(np.ascontiguousarray(scales_flat).reshape(1, 1, 1, -1)).to(gpu)
    out = HmxW4LpbqExpandToI8(wl, sc)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (1, 1, k, n)
    return out


@pytest.mark.parametrize("k,n,hi", [(32, 32, 16), (64, 96, 255), (256, 512, 16), (4096, 4096, 255)])
def test_expand_matches_op_restatement(gpu, k, n, hi):
    rng = np.random.default_rng(k * 7 + n)
    codes = rng.integers(-8, 8, size=(k, n)).astype(np.int8)
    scales = rng.integers(0, hi + 1, size=(n, k // 32)).astype(np.uint8)
    packed = L.pack_w4_kpair(codes)
    print(f"[carriers] expand K={k} N={n} scale<= {hi}", flush=True)
    got = expand_on_gpu(gpu, packed, scales.reshape(-1), k, n).cpu().numpy().reshape(-1)
    if k * n <= 1 << 20:
        want = L.lpbq_expand_to_i8(packed, scales.reshape(-1), k, n)
    else:
        want = L.pack_w8_kmajor(L.expand_lpbq_logical_kn(codes, scales, 32))
    assert np.array_equal(got, want)


def test_expand_decode_benchmark_weight(gpu):
    k, n = 4096, 14336
    rng = np.random.default_rng(14336)
    codes = rng.integers(-7, 8, size=(k, n)).astype(np.int8)
    scales = rng.integers(1, 17, size=(n, k // 32)).astype(np.uint8)
    print(f"[carriers] expand K={k} N={n}", flush=True)
    got = expand_on_gpu(gpu, L.pack_w4_kpair(codes), scales.reshape(-1), k, n).cpu().numpy().reshape(-1)
    assert np.array_equal(got, L.pack_w8_kmajor(L.expand_lpbq_logical_kn(codes, scales, 32)))


def test_expand_rejects_bad_shapes(gpu):
    import torch

    L_ = _lib.lib()
    buf = torch.zeros(64 * 64, dtype=torch.uint8, device=gpu)
    assert L_.qh_w4_lpbq_expand_to_i8(buf.data_ptr(), buf.data_ptr(), buf.data_ptr(), 48, 64, None) \
        == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert L_.qh_w4_lpbq_expand_to_i8(buf.data_ptr() + 1, buf.data_ptr(), buf.data_ptr(), 32, 32, None) \
        == _lib.QH_STATUS_INVALID_ARGUMENT


# family -> (op class name, carrier, flags) as the reference's graph hands the op its weight
OPS = {
    "u8i8": ("HmxU8I8ToU8MatMul", "i8_kn", _lib.QH_CARRIER_XOR80),
    "w4a8_per_channel": ("HmxU8I4ToU8MatMul", "w4_kmajor_n64", _lib.QH_CARRIER_XOR80),
    "w8a16": ("HmxU16I8ToU16MatMul", "w8_kmajor", 0),
    "w4a16_per_channel": ("HmxU16I4ToU16MatMul", "w4_kblock32_nmajor_k4", 0),
    "w4a8_lpbq": ("HmxU8I8ToU8MatMul", "w8_kmajor", 0),
    "w4a16_lpbq": ("HmxU16I8ToU16MatMul", "w8_kmajor", 0),
}


@pytest.mark.parametrize("case", C.CASES)
@pytest.mark.parametrize("fam", C.GATED_FAMILIES)
def test_ops_from_reference_carriers_match_generator_outputs(gpu, fam, case):
    import torch

    from qcom_htp_amd import ops

    c = C.make_case(fam, case, 256, 256, 256)
    name, carrier, flags = OPS[fam]
    w_kn = c.weight_q_nk.T.copy()
    print(f"[carriers] {fam}/{case} via {name}({carrier})", flush=True)
    if c.family.is_lpbq:
        weight = expand_on_gpu(gpu, L.pack_w4_kpair(w_kn), c.lpbq_block_int_scale.reshape(-1), c.k, c.n)
    else:
        pack, bits = L.PACKERS[carrier]
        s = pack(w_kn)
        if flags & _lib.QH_CARRIER_XOR80:
            s = L.carrier_xor80(s)
        weight = np.ascontiguousarray(s).reshape((1, 1) + ops.carrier_shape(carrier, c.k, c.n))
    op = getattr(ops, name)(c.bias_q, weight, weight_scale=c.weight_scale, act_scale=c.act_scale, act_zp=c.act_zp,
                            out_scale=c.out_scale, out_zp=c.out_zp, carrier=carrier, carrier_flags=flags, device=gpu)
    act = torch.from_numpy(np.ascontiguousarray(c.activation_q)).to(gpu).view(1, c.m // 32, 32, c.k)
    out = op(act)
    torch.cuda.synchronize()
    assert tuple(out.shape) == (1, c.m // 32, 32, c.n)
    got = out.cpu().numpy().reshape(c.m, c.n)
    op.close()
    assert sha(got) == GATE_META[f"{fam}/{case}"]["sha256"]["output_q"]
