"""CPU tests of the graph-generator operands (qcom_htp_amd.cases.graph_*), the closed forms of the
reference's CHAIN graphs (gen_quant_chain.py:253-329, gen_u8i8_chain.py:68-73,170-213).  No
reference-written output exists for these graphs, so each closed form is pinned by values derived
by hand from its formula (hex arithmetic on the seed, residues mod 2q + 1) and by the
periodicities the formulas imply."""

import numpy as np
import pytest

from oracle import qmm as oq
from qcom_htp_amd import cases as C


def test_default_activation_hand_values():
    # seed = 374761393 = 0x165667B1: low byte 0xB1 = 177, low 16 bits 0x67B1 = 26545; then +37 per element
    a8 = C.graph_activation(8, 2, 256)
    assert a8.dtype == np.uint8 and a8.shape == (2, 256)
    assert a8[0, :4].tolist() == [177, 214, 251, 32]  # 288 mod 256 = 32
    assert a8[1, 0] == (177 + 37 * 256) % 256 == 177
    a16 = C.graph_activation(16, 1, 4)
    assert a16.dtype == np.dtype("<u2") and a16[0].tolist() == [26545, 26582, 26619, 26656]
    # input 1: seed 2 * 0x165667B1 = 0x2CACCF62 -> low byte 0x62 = 98
    assert C.graph_activation(8, 1, 1, index=1)[0, 0] == 98


def test_zp_and_impulse_activations():
    zp = C.graph_activation(16, 4, 32, mode="zp")
    assert np.all(zp == 32768)
    imp = C.graph_activation(8, 4, 32, mode="k_impulse", impulse_k=7)
    assert np.all(imp[:, 7] == 129) and np.all(np.delete(imp, 7, axis=1) == 128)
    assert np.all(C.graph_activation(8, 2, 32, mode="k_impulse", impulse_k=33)[:, 1] == 129)  # k mod K
    with pytest.raises(ValueError):
        C.graph_activation(8, 2, 32, mode="bogus")


@pytest.mark.parametrize("bits,q", [(4, 7), (8, 127), (16, 32767)])
def test_weight_pattern_hand_values_and_period(bits, q):
    w = C.graph_weight_kn(bits, 64, 64)
    assert w.shape == (64, 64) and w.min() >= -q and w.max() <= q
    assert w[0, 0] == -q and w[0, 1] == 13 - q
    assert w[1, 0] == (31 % (2 * q + 1)) - q  # q = 7: 31 mod 15 = 1 -> -6
    if q == 7:
        assert w[1, 0] == -6 and np.array_equal(w[15:30], w[0:15])  # 31 * 15 = 0 mod 15
    assert C.graph_weight_kn(8, 8, 8, limit=3).max() == 3


def test_lpbq_block_scale_patterns():
    # w4a8: 3p = 0 mod 3, so the factor is 1 + (5b mod 3) = 1 + (2b mod 3) for every channel
    s = C.graph_lpbq_block_scales("w4a8", 256, 128, 32)
    assert s.shape == (128, 8) and s.dtype == np.uint8
    assert np.all(s == np.array([1, 3, 2, 1, 3, 2, 1, 3], np.uint8)[None, :])
    # w4a16: 1 + (5 (b // 2) mod 3): blocks 0,1 -> 1; 2,3 -> 3; 4,5 -> 2; 6,7 -> 1
    s = C.graph_lpbq_block_scales("w4a16", 256, 64, 32)
    assert np.all(s == np.array([1, 1, 3, 3, 2, 2, 1, 1], np.uint8)[None, :])


@pytest.mark.parametrize("name", list(C.GRAPH_FAMILIES))
def test_graph_case_assembly(name):
    g = C.graph_case(name, 64, 64, 64)
    assert g.activation.shape == (64, 64) and g.weight_compute_kn.shape == (64, 64)
    if g.lpbq_block_scale is not None:
        f = np.repeat(g.lpbq_block_scale.T.astype(np.int32), g.lpbq_block, axis=0)
        assert np.array_equal(g.weight_compute_kn, g.weight_kn * f) and np.abs(g.weight_compute_kn).max() <= 21
    else:
        assert np.array_equal(g.weight_compute_kn, g.weight_kn)
    if g.contract == "legacy":
        assert g.bias_q.tolist() == list(range(1, 65))
    else:
        assert not g.bias_q.any() and g.act_bits == 16
    assert g.chain == (1 if name == "w4a16_per_channel" else 8)


def test_graph_contract_mapping_and_oracle_step():
    from qcom_htp_amd.qmm import graph_contract  # noqa: F401  (ctypes binding loads lazily)

    assert graph_contract(C.graph_case("u8i8", 32, 32, 32)) == ("clip_i32", 1)
    assert graph_contract(C.graph_case("w8a16", 32, 32, 32)) == ("div_rint", 127)
    assert graph_contract(C.graph_case("w4a16_lpbq", 32, 32, 32)) == ("floor256_div_rint", 7)
    assert graph_contract(C.graph_case("w16a16", 32, 32, 32)) == ("div_rint", 32767)
    # the contract, applied to the exact accumulator, is the generator's reference step
    for name in ("u8i8", "w4a8_lpbq", "w8a16", "w4a16_per_channel", "w16a16"):
        g = C.graph_case(name, 64, 64, 64)
        step = oq.reference_step(g.act_bits, g.weight_bits, g.out_bits, g.activation, g.weight_compute_kn, g.bias_q,
                                 contract=g.contract, family_name=g.kernel_family)
        cname, d = graph_contract(g)
        acc = oq.int_accumulator(g.activation, g.weight_compute_kn.T, g.act_zp)
        via = oq.contract_output(acc, cname, d, g.bias_q, g.out_zp, g.out_bits)
        assert np.array_equal(step, via), name
