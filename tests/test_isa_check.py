"""CPU tests of qcom_htp_amd.isa_check, the static check of the GEMM's hand-counted memory waits:
synthetic kernels with a correct and a planted too-loose wait (a register read before its load
is covered, a register reused while a load is pending, a loop-carried load), and the built
assembly of qmm_gemm.hip when the build folder holds it."""

from pathlib import Path

import pytest

from qcom_htp_amd import isa_check

KERNEL = """_Z15qmm_gemm_kernelv:
\tglobal_load_dwordx4 v[10:13], v1, s[0:1]
\tglobal_load_dwordx4 v[14:17], v1, s[0:1] offset:1024
\tglobal_load_lds_dwordx4 v2, s[2:3]
.LBB0_1:
\ts_waitcnt vmcnt({w1})
\tv_mfma_i32_32x32x32_i8 v[20:35], v[4:7], v[10:13], v[20:35]
\tglobal_load_dwordx4 v[10:13], v1, s[0:1] offset:2048
\ts_waitcnt vmcnt({w2})
\tv_mfma_i32_32x32x32_i8 v[20:35], v[4:7], v[14:17], v[20:35]
\tglobal_load_dwordx4 v[14:17], v1, s[0:1] offset:3072
\ts_cbranch_scc1 .LBB0_1
\ts_waitcnt vmcnt(0)
\tv_mov_b32 v10, 0
\ts_endpgm
"""


def check(text):
    names, errs = [], []
    lines = text.splitlines()
    for n in [l.split(":")[0] for l in lines if l.startswith("_Z")]:
        names.append(n)
        errs += isa_check.check_kernel(lines, n)
    return names, errs


def test_exact_waits_pass():
    # in the loop each fragment is followed by exactly one later request (the other fragment's
    # reload) -> vmcnt(1) before each MFMA; on entry the DMA follows as well (stricter still)
    names, errs = check(KERNEL.format(w1=1, w2=1))
    assert names and not errs, errs


@pytest.mark.parametrize("w1,w2", [(2, 1), (1, 2)])
def test_too_loose_wait_is_reported(w1, w2):
    _, errs = check(KERNEL.format(w1=w1, w2=w2))
    assert errs and "pending" in errs[0]


def test_register_reuse_while_pending_is_reported():
    bad = KERNEL.format(w1=1, w2=1).replace("\tv_mov_b32 v10, 0\n", "").replace(
        "\ts_cbranch_scc1 .LBB0_1\n", "\ts_cbranch_scc1 .LBB0_1\n\tv_mov_b32 v15, 0\n")
    _, errs = check(bad)
    assert any("v[15]" in e for e in errs)


def test_lds_dma_has_no_register_destination():
    # the DMA's first operand is its address, not a destination: reading v2 is not a violation
    ok = KERNEL.format(w1=1, w2=1).replace(".LBB0_1:\n", "\tv_mov_b32 v2, 0\n.LBB0_1:\n")
    _, errs = check(ok)
    assert not errs


ASM = Path(__file__).resolve().parents[1] / "qcom_htp_amd" / "_build" / "qmm_gemm-hip-amdgcn-amd-amdhsa-gfx950.s"


@pytest.mark.skipif(not ASM.exists(), reason="qcom_htp_amd/_build has no GEMM assembly (build first)")
def test_built_gemm_assembly_passes():
    names, errs = isa_check.check_file(str(ASM))
    assert len(names) >= 8 and not errs, errs[:5]
