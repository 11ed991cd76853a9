"""GPU parity at the full benchmark sizes.

* Quantized GEMM at M = K = N = 4096 (u8i8, W4A8 / W8A16 / W4A16 per-channel) and the LPBQ GEMM
  at M = 4096, K = 4096, N = 14336 (64-wide K blocks, block scales in [1, 15]): every output is
  compared with the float64 oracle, bit for bit.
* The decode GEMV at M = 1 and M = 16 on the same LPBQ weights (N = 14336: 896 column groups,
  so the 16-row launch walks several groups per workgroup), and on per-channel weights with
  N = 8704 at 6 and 16 rows.
* The fused GDN chunk products at B = 8, T = 4096, H = 32, C in {64, 256}: a sample of
  (batch, chunk, head) items spread over the whole range -- most of them past the first wave
  of the persistent grid, so they run on a workgroup's second or later trip round its item loop
  -- against the float64 solve, bound 1.05e-2 relative Frobenius; and small inputs whose grid is
  capped at 1, 2 and 3 workgroups, compared with the float64 solve item by item and with the
  uncapped launch bit for bit.
"""

import numpy as np
import pytest

from oracle import gdn as og
from oracle import qmm as oq
from qcom_htp_amd import cases as C

pytestmark = pytest.mark.gpu

BF16_TOL = 1.05e-2


def diff_msg(got, want):
    bad = np.argwhere(got.astype(np.int64) != want.astype(np.int64))
    if bad.size == 0:
        return "identical"
    i, j = bad[0]
    return f"{len(bad)} mismatches, first at {tuple(bad[0])}: got {got[i, j]} want {want[i, j]}"


def run_rows(op, act_dev, rows, path):
    import torch

    out = op(act_dev[:rows].contiguous(), path=path)
    torch.cuda.synchronize()
    return out.cpu().numpy()


GEMM_FULL = [
    ("w4a8_per_channel", 4096, 4096, 4096),
    ("w8a16", 4096, 4096, 4096),
    ("u8i8", 4096, 4096, 4096),
    ("w4a16_per_channel", 4096, 4096, 4096),
    ("w4a8_lpbq", 4096, 4096, 14336),
    ("w4a16_lpbq", 4096, 4096, 14336),
]


@pytest.mark.parametrize("fam,m,k,n", GEMM_FULL, ids=[f"{f}_{m}x{k}x{n}" for f, m, k, n in GEMM_FULL])
def test_full_size_gemm_and_gemv_bit_exact(gpu, fam, m, k, n):
    import torch

    from qcom_htp_amd.qmm import PATH_GEMM, PATH_GEMV, QuantMatmul

    print(f"[full] {fam} {m}x{k}x{n}: case", flush=True)
    c = C.synthetic_case(fam, m, k, n, seed=2, lpbq_block=64, lpbq_max_scale=15)
    print(f"[full] {fam}: oracle", flush=True)
    want = oq.expected_output_case(c)
    print(f"[full] {fam}: prepare", flush=True)
    op = QuantMatmul.from_case(c, device=gpu)
    act = torch.from_numpy(c.activation_q).to(gpu)
    print(f"[full] {fam}: gemm", flush=True)
    got = run_rows(op, act, m, PATH_GEMM)
    assert np.array_equal(got, want), f"gemm: {diff_msg(got, want)}"
    if c.family.is_lpbq:
        for rows in (1, 16):
            print(f"[full] {fam}: gemv rows={rows}", flush=True)
            got = run_rows(op, act, rows, PATH_GEMV)
            assert np.array_equal(got, want[:rows]), f"gemv rows={rows}: {diff_msg(got, want[:rows])}"
    op.close()


@pytest.mark.parametrize("fam", C.GATED_FAMILIES)
def test_gemv_many_groups_per_workgroup_bit_exact(gpu, fam):
    """N = 8704 (544 column groups): launches with 5..16 rows cap the grid at 512 workgroups,
    so some workgroups take a second group (next-group prefetch, reused reduction buffers,
    near-tie recomputation from re-read weights)."""
    import torch

    from qcom_htp_amd.qmm import PATH_GEMV, QuantMatmul

    c = C.synthetic_case(fam, 16, 4096, 8704, seed=31, lpbq_block=64, lpbq_max_scale=15)
    want = oq.expected_output_case(c)
    op = QuantMatmul.from_case(c, device=gpu)
    act = torch.from_numpy(c.activation_q).to(gpu)
    for rows in (6, 16):
        print(f"[full] {fam} gemv 16x4096x8704 rows={rows}", flush=True)
        got = run_rows(op, act, rows, PATH_GEMV)
        assert np.array_equal(got, want[:rows]), f"rows={rows}: {diff_msg(got, want[:rows])}"
    op.close()


# ---------------------------------------------------------------------------- GDN chunk products


def chunk_inputs_dev(B, T, H, seed, dev):
    """k, v ~ N(0,1) as bf16, beta = sigmoid(N(0,1)), gc = logsigmoid(N(0,1) + 3), generated on
    the device ([B, T, H, 128] / [B, T, H])."""
    import torch

    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    k = torch.randn((B, T, H, 128), generator=gen, device=dev).to(torch.bfloat16)
    v = torch.randn((B, T, H, 128), generator=gen, device=dev).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn((B, T, H), generator=gen, device=dev))
    gc = torch.nn.functional.logsigmoid(torch.randn((B, T, H), generator=gen, device=dev) + 3.0)
    return k, v, beta, gc


def item_error(k, v, beta, gc, w, u, b, c, h, C_, decay_w):
    """Worst relative Frobenius error of W and U of item (b, chunk c, head h) vs float64."""
    sl = slice(c * C_, (c + 1) * C_)
    kc = k[b, sl, h].float().cpu().numpy().astype(np.float64)
    vc = v[b, sl, h].float().cpu().numpy().astype(np.float64)
    bc = beta[b, sl, h].cpu().numpy().astype(np.float64)
    gcc = gc[b, sl, h].cpu().numpy().astype(np.float64)
    Tm = og.inverse_fp64(og.build_A(kc, bc, gcc))
    U, W = og.chunk_uw(Tm, kc, vc, bc, gcc, decay_w=decay_w)
    eu = og.oc(u[b, sl, h].float().cpu().numpy(), U)
    ew = og.oc(w[b, sl, h].float().cpu().numpy(), W)
    return max(eu, ew)


def _items(x, C_):
    """[T, H, ...] of one batch -> [chunks * H, C_, ...] (one row per (chunk, head) item)."""
    T, H = x.shape[0], x.shape[1]
    y = x.reshape(T // C_, C_, H, -1).permute(0, 2, 1, 3).reshape((T // C_) * H, C_, -1)
    return y if x.dim() == 3 else y[..., 0]


def _rel_fro(x, ref):
    """Per-item relative Frobenius error (the oc of scripts/gdn_solve_oc_check.py:31) over [n, ...]."""
    import torch

    d = (x - ref).flatten(1).norm(dim=1)
    return d / ref.flatten(1).norm(dim=1).clamp_min(torch.finfo(torch.float64).tiny)


@pytest.mark.parametrize("C_", [64, 256])
def test_gdn_chunk_uw_full_config5(gpu, C_):
    """Config 5 at full size (B=8, T=4096, H=32): every (batch, chunk, head) item of W and U against
    a batched float64 triangular solve (oracle.gdn.chunk_stage_a_solve_torch, pinned to the row
    recurrence), batch by batch on the host."""
    import torch

    from qcom_htp_amd.gdn import gdn_chunk_uw

    B, T, H = 8, 4096, 32
    print(f"[full] gdn chunk B={B} T={T} H={H} C={C_}: inputs", flush=True)
    k, v, beta, gc = chunk_inputs_dev(B, T, H, seed=50 + C_, dev=gpu)
    print(f"[full] gdn chunk C={C_}: kernel", flush=True)
    w, u = gdn_chunk_uw(k, v, gc, beta, C_)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(w.float()).all()) and bool(torch.isfinite(u.float()).all())
    worst, n = 0.0, 0
    for b in range(B):
        f64 = lambda x: x[b].to(torch.float64).cpu()
        U, W = og.chunk_stage_a_solve_torch(_items(f64(k), C_), _items(f64(v), C_), _items(f64(gc), C_),
                                            _items(f64(beta), C_), decay_w=False)
        e = torch.maximum(_rel_fro(_items(f64(u), C_), U), _rel_fro(_items(f64(w), C_), W))
        worst = max(worst, float(e.max()))
        n += e.numel()
        bad = int((e > BF16_TOL).sum())
        assert bad == 0, f"batch {b}: {bad} items above {BF16_TOL}, worst oc {float(e.max()):.3e}"
        print(f"[full] gdn chunk C={C_} batch {b}: worst oc {float(e.max()):.3e}", flush=True)
    print(f"[full] gdn chunk C={C_}: all {n} items, worst oc {worst:.3e}", flush=True)


@pytest.mark.parametrize("C_", [64, 256])
def test_gdn_chunk_uw_capped_grid(gpu, C_):
    """Small inputs on 1, 2 and 3 workgroups: every workgroup walks 8 to 24 items (next-item key
    prefetch, the next item's phase 1 at the end of the current one, LDS reuse across items)."""
    import torch

    from qcom_htp_amd.gdn import gdn_chunk_uw

    B, H, nch = 2, 3, 4
    T = nch * C_
    k, v, beta, gc = chunk_inputs_dev(B, T, H, seed=70 + C_, dev=gpu)
    for decay_w in (False, True):
        w0, u0 = gdn_chunk_uw(k, v, gc, beta, C_, decay_w=decay_w)
        torch.cuda.synchronize()
        for cap in (1, 2, 3):
            print(f"[full] gdn chunk C={C_} decay_w={decay_w} max_workgroups={cap}", flush=True)
            w, u = gdn_chunk_uw(k, v, gc, beta, C_, decay_w=decay_w, max_workgroups=cap)
            torch.cuda.synchronize()
            assert torch.equal(w, w0) and torch.equal(u, u0), f"cap {cap}: results differ from the full grid"
        worst = 0.0
        for b in range(B):
            for c in range(nch):
                for h in range(H):
                    e = item_error(k, v, beta, gc, w, u, b, c, h, C_, decay_w)
                    worst = max(worst, e)
                    assert e <= BF16_TOL, f"b={b} chunk={c} h={h}: oc={e:.3e}"
        print(f"[full] gdn chunk C={C_} decay_w={decay_w}: worst oc {worst:.3e}", flush=True)
