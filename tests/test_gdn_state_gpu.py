"""GPU parity of the GDN chunk recurrence (stage B) and of the whole chunked prefill against the
float64 oracle (oracle.gdn.chunk_state_torch / gdn_prefill_torch, themselves pinned to the
token-by-token gated delta rule).

Error measure: relative Frobenius error per (batch, head) sequence, the oc of
scripts/gdn_solve_oc_check.py:31 applied to o [T, D] and to the final state S [D, D].
Bounds:
  stage B alone, W and U exact (float64 -> float32):
    QH_GDN_FP32  <= 1e-4   (hi/lo split products; the solve's fp32 bound)
    QH_GDN_BF16  <= 1.05e-2 (the bf16 bound of tests/qnn_kernel_e2e/correctness/test_gdn_solve_e2e.sh:18)
  prefill (stage A + B): stage A is bf16-MFMA (qh_gdn_chunk_uw, bound 1.05e-2), so the whole
  path is held to 1.05e-2.
"""

import numpy as np
import pytest

from oracle import gdn as og

pytestmark = pytest.mark.gpu

FP32_TOL = 1.0e-4
BF16_TOL = 1.05e-2


def bf16_bits(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def bits_f64(b):
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def seq_inputs(B, T, H, seed):
    """q, k, v ~ N(0,1) as bf16 bits, beta = sigmoid(N(0,1)), gc = logsigmoid(N(0,1) + 3),
    [B, T, H, (D)] as the reference kernel takes them."""
    rng = np.random.default_rng(seed)
    qb, kb, vb = (bf16_bits(rng.standard_normal((B, T, H, 128))) for _ in range(3))
    beta = (1.0 / (1.0 + np.exp(-rng.standard_normal((B, T, H))))).astype(np.float32)
    gc = (-np.logaddexp(0.0, -(rng.standard_normal((B, T, H)) + 3.0))).astype(np.float32)
    return qb, kb, vb, beta, gc


def to_dev(x, gpu):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(x))
    if x.dtype == np.uint16:
        t = t.view(torch.int16).view(torch.bfloat16)
    return t.to(gpu)


def per_seq(a):  # [B, T, H, D] -> [B*H, T, D]
    B, T, H, D = a.shape
    return np.ascontiguousarray(a.transpose(0, 2, 1, 3).reshape(B * H, T, D))


def worst_oc(x, ref, B, H):
    x = x.reshape(B * H, -1)
    ref = ref.reshape(B * H, -1)
    return max(og.oc(x[i], ref[i]) for i in range(B * H))


def stage_a_exact(kb, vb, beta, gc):
    """W (e^g form), U per 64-token chunk in float64 ([B, T, H, D])."""
    k64, v64 = bits_f64(kb), bits_f64(vb)
    B, T, H, D = k64.shape
    n = B * H * (T // 64)
    resh = lambda a: per_seq(a).reshape(n, 64, D)
    reshs = lambda a: np.ascontiguousarray(a.transpose(0, 2, 1).reshape(n, 64)).astype(np.float64)
    U, W = og.chunk_stage_a_torch(resh(k64), resh(v64), reshs(gc), reshs(beta), decay_w=True)
    back = lambda X: X.numpy().reshape(B, H, T, D).transpose(0, 2, 1, 3)
    return back(W), back(U)


@pytest.mark.parametrize("wu", ["f32", "bf16"], ids=["wu_f32", "wu_bf16"])
@pytest.mark.parametrize("precision", [0, 1], ids=["fp32", "bf16"])
@pytest.mark.parametrize("with_state", [False, True], ids=["zero_state", "incoming_state"])
@pytest.mark.parametrize("T", [192, 64], ids=["three_chunks", "one_chunk"])
def test_chunk_state_matches_fp64(gpu, precision, with_state, T, wu):
    """Stage B against the float64 recurrence; one chunk runs only the first (peeled) chunk, whose
    next-chunk prefetch reloads itself.  W and U go in as float32 or as bf16 (the instantiation
    gdn_prefill uses for BF16); the oracle gets the same rounded values."""
    import torch

    from qcom_htp_amd.gdn import gdn_chunk_state

    B, H = 2, 3
    qb, kb, vb, beta, gc = seq_inputs(B, T, H, seed=21 + with_state)
    W, U = stage_a_exact(kb, vb, beta, gc)
    if wu == "f32":
        Wd, Ud = W.astype(np.float32), U.astype(np.float32)
        W_in, U_in = Wd.astype(np.float64), Ud.astype(np.float64)
    else:
        Wd, Ud = bf16_bits(W), bf16_bits(U)
        W_in, U_in = bits_f64(Wd), bits_f64(Ud)
    S0 = (np.random.default_rng(5).standard_normal((B, H, 128, 128)) * 0.05).astype(np.float32) if with_state else None
    print(f"[gdn-state] stage B T={T} precision={precision} state={with_state} wu={wu}", flush=True)
    o, S = gdn_chunk_state(to_dev(qb, gpu), to_dev(kb, gpu), to_dev(gc, gpu), to_dev(Wd, gpu),
                           to_dev(Ud, gpu), None if S0 is None else to_dev(S0, gpu),
                           precision=precision, out_dtype=torch.float32)
    torch.cuda.synchronize()
    o_ref, S_ref = og.chunk_state_torch(per_seq(bits_f64(qb)), per_seq(bits_f64(kb)),
                                        np.ascontiguousarray(gc.transpose(0, 2, 1).reshape(B * H, T)),
                                        per_seq(W_in), per_seq(U_in),
                                        None if S0 is None else S0.reshape(B * H, 128, 128), 64)
    eo = worst_oc(per_seq(o.cpu().numpy().astype(np.float64)), o_ref.numpy(), B, H)
    es = worst_oc(S.cpu().numpy().astype(np.float64).reshape(B * H, 128, 128), S_ref.numpy(), B, H)
    tol = FP32_TOL if precision == 0 else BF16_TOL
    print(f"[gdn-state] precision={precision} state={with_state} wu={wu}: worst oc(o)={eo:.3e} oc(S)={es:.3e}",
          flush=True)
    assert eo <= tol and es <= tol


@pytest.mark.parametrize("precision", [0, 1], ids=["fp32", "bf16"])
@pytest.mark.parametrize("T", [256, 100], ids=["whole_chunks", "ragged"])
def test_prefill_matches_fp64(gpu, T, precision):
    """The whole prefill; BF16 runs stage A with bf16 W, U and stage B on its bf16-W/U kernel."""
    import torch

    from qcom_htp_amd.gdn import gdn_prefill

    B, H = 2, 3
    qb, kb, vb, beta, gc = seq_inputs(B, T, H, seed=31 + T)
    print(f"[gdn-state] prefill T={T} precision={precision}", flush=True)
    o, S = gdn_prefill(to_dev(qb, gpu), to_dev(kb, gpu), to_dev(vb, gpu), to_dev(gc, gpu), to_dev(beta, gpu),
                       precision=precision, out_dtype=torch.float32)
    torch.cuda.synchronize()
    gcs = np.ascontiguousarray(gc.transpose(0, 2, 1).reshape(B * H, T))
    bts = np.ascontiguousarray(beta.transpose(0, 2, 1).reshape(B * H, T))
    o_ref, S_ref = og.gdn_prefill_torch(per_seq(bits_f64(qb)), per_seq(bits_f64(kb)), per_seq(bits_f64(vb)), gcs,
                                        bts, 64)
    assert o.shape == (B, T, H, 128)
    eo = worst_oc(per_seq(o.cpu().numpy().astype(np.float64)), o_ref.numpy(), B, H)
    es = worst_oc(S.cpu().numpy().astype(np.float64).reshape(B * H, 128, 128), S_ref.numpy(), B, H)
    print(f"[gdn-state] prefill T={T}: worst oc(o)={eo:.3e} oc(S)={es:.3e}", flush=True)
    assert eo <= BF16_TOL and es <= BF16_TOL


def test_state_handoff_equals_one_pass(gpu):
    """Two calls, the second starting from the first's final state, give the one-pass result
    (same chunks, same arithmetic: equal to float32 rounding of the state hand-off)."""
    import torch

    from qcom_htp_amd.gdn import gdn_chunk_state, gdn_chunk_uw

    B, T, H = 1, 256, 4
    qb, kb, vb, beta, gc = seq_inputs(B, T, H, seed=41)
    q, k, v, g, bt = (to_dev(x, gpu) for x in (qb, kb, vb, gc, beta))
    w, u = gdn_chunk_uw(k, v, g, bt, 64, decay_w=True, out_dtype=torch.float32)
    o_all, S_all = gdn_chunk_state(q, k, g, w, u, out_dtype=torch.float32)
    h = T // 2
    cut = lambda x: (x[:, :h].contiguous(), x[:, h:].contiguous())
    (q1, q2), (k1, k2), (g1, g2), (w1, w2), (u1, u2) = (cut(x) for x in (q, k, g, w, u))
    o1, S1 = gdn_chunk_state(q1, k1, g1, w1, u1, out_dtype=torch.float32)
    o2, S2 = gdn_chunk_state(q2, k2, g2, w2, u2, S1, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(o1, o_all[:, :h])
    assert torch.equal(o2, o_all[:, h:])
    assert torch.equal(S2, S_all)


@pytest.mark.parametrize("precision", [0, 1], ids=["fp32", "bf16"])
def test_chunk_state_bf16_output_is_rounded_fp32_output(gpu, precision):
    """The bfloat16 output path (4 rows x 4 columns of each lane quad exchanged so that every lane
    stores 4 adjacent outputs of one row) gives the float32 output rounded to nearest even, element
    for element: the two kernels differ only in how o is stored."""
    import torch

    from qcom_htp_amd.gdn import gdn_chunk_state, gdn_chunk_uw

    B, T, H = 2, 192, 3
    qb, kb, vb, beta, gc = seq_inputs(B, T, H, seed=43)
    q, k, v, g, bt = (to_dev(x, gpu) for x in (qb, kb, vb, gc, beta))
    w, u = gdn_chunk_uw(k, v, g, bt, 64, decay_w=True, out_dtype=torch.float32)
    print(f"[gdn-state] bf16 output, precision={precision}", flush=True)
    o32, S32 = gdn_chunk_state(q, k, g, w, u, precision=precision, out_dtype=torch.float32)
    o16, S16 = gdn_chunk_state(q, k, g, w, u, precision=precision, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    assert o16.dtype == torch.bfloat16 and o16.shape == o32.shape
    assert torch.equal(o16, o32.to(torch.bfloat16))
    assert torch.equal(S16, S32)


def test_chunk_state_rejects_bad_arguments(gpu):
    import torch

    from qcom_htp_amd import _lib

    B, T, H = 1, 64, 1
    x = torch.zeros((B, T, H, 128), dtype=torch.bfloat16, device=gpu)
    g = torch.zeros((B, T, H), dtype=torch.float32, device=gpu)
    s = torch.zeros((B, H, 128, 128), dtype=torch.float32, device=gpu)
    o = torch.zeros_like(x)
    L = _lib.lib()
    args = lambda tok, chunk, hd, sin: (x.data_ptr(), x.data_ptr(), g.data_ptr(), x.data_ptr(), x.data_ptr(), sin,
                                        s.data_ptr(), o.data_ptr(), B, tok, H, hd, chunk, 0, 0, 0)
    assert L.qh_gdn_chunk_state(*args(T, 128, 128, 0)) == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert L.qh_gdn_chunk_state(*args(T, 64, 64, 0)) == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert L.qh_gdn_chunk_state(*args(100, 64, 128, 0)) == _lib.QH_STATUS_SHAPE_UNSUPPORTED
    assert L.qh_gdn_chunk_state(*args(T, 64, 128, s.data_ptr())) == _lib.QH_STATUS_INVALID_ARGUMENT  # alias


def test_prefill_full_config5_every_sequence(gpu):
    """Config 5 at full size (B=8, T=4096, H=32, D=128; 64 chunks per sequence): the GPU prefill
    against the float64 oracle on all 256 (batch, head) sequences, o and the final state, one
    batch of 32 sequences at a time on the host."""
    import torch

    from qcom_htp_amd.gdn import gdn_prefill

    B, T, H = 8, 4096, 32
    qb, kb, vb, beta, gc = seq_inputs(B, T, H, seed=55)
    print("[gdn-state] prefill config 5 B=8 T=4096 H=32", flush=True)
    o, S = gdn_prefill(to_dev(qb, gpu), to_dev(kb, gpu), to_dev(vb, gpu), to_dev(gc, gpu), to_dev(beta, gpu),
                       out_dtype=torch.float32)
    torch.cuda.synchronize()
    o = o.cpu().numpy()
    S = S.cpu().numpy()
    worst_o = worst_s = 0.0
    for b in range(B):
        sl = lambda a: a[b:b + 1]
        q1, k1, v1 = (per_seq(bits_f64(sl(x))) for x in (qb, kb, vb))
        o_ref, S_ref = og.gdn_prefill_torch(q1, k1, v1, np.ascontiguousarray(gc[b].T).astype(np.float64),
                                            np.ascontiguousarray(beta[b].T).astype(np.float64), 64)
        o_ref, S_ref = o_ref.numpy(), S_ref.numpy()
        ob = per_seq(o[b:b + 1].astype(np.float64))
        eo = max(og.oc(ob[h], o_ref[h]) for h in range(H))
        es = max(og.oc(S[b, h].astype(np.float64), S_ref[h]) for h in range(H))
        worst_o, worst_s = max(worst_o, eo), max(worst_s, es)
        print(f"[gdn-state] config 5 batch {b}: worst oc(o)={eo:.3e} oc(S)={es:.3e}", flush=True)
        assert eo <= BF16_TOL and es <= BF16_TOL, f"batch {b}"
    print(f"[gdn-state] config 5, all 256 sequences: worst oc(o)={worst_o:.3e} oc(S)={worst_s:.3e}", flush=True)


def test_torch_ops_prefill_matches_direct(gpu):
    import torch

    from qcom_htp_amd import torch_ops  # noqa: F401 (registers torch.ops.qhtp)
    from qcom_htp_amd.gdn import gdn_prefill

    B, T, H = 1, 128, 2
    qb, kb, vb, beta, gc = seq_inputs(B, T, H, seed=61)
    args = [to_dev(x, gpu) for x in (qb, kb, vb, gc, beta)]
    o_op, S_op = torch.ops.qhtp.gdn_prefill(*args, None, 0, True)
    o_d, S_d = gdn_prefill(*args, out_dtype=torch.float32)
    torch.cuda.synchronize()
    assert torch.equal(o_op, o_d) and torch.equal(S_op, S_d)


def test_python_surface_rejects_host_or_foreign_tensors(gpu):
    """A host initial_state (its address would be dereferenced on the device) and inputs on another
    device are refused before any launch."""
    import torch

    from qcom_htp_amd.gdn import gdn_chunk_state, gdn_prefill

    B, T, H = 1, 64, 1
    x = torch.zeros((B, T, H, 128), dtype=torch.bfloat16, device=gpu)
    g = torch.zeros((B, T, H), dtype=torch.float32, device=gpu)
    s_host = torch.zeros((B, H, 128, 128), dtype=torch.float32)
    with pytest.raises(TypeError, match="initial_state"):
        gdn_chunk_state(x, x, g, x, x, s_host)
    with pytest.raises(TypeError, match="initial_state"):
        gdn_prefill(x, x, x, g, g, s_host)
    with pytest.raises(TypeError):
        gdn_chunk_state(x, x, g, x, x, [0.0])


def test_prefill_on_a_side_stream_matches_current_stream(gpu):
    """gdn_prefill with a side stream (its temporaries allocated on that stream) gives the
    current-stream result."""
    import torch

    from qcom_htp_amd.gdn import gdn_prefill

    B, T, H = 1, 100, 2
    qb, kb, vb, beta, gc = seq_inputs(B, T, H, seed=77)
    q, k, v, g, bt = (to_dev(x, gpu) for x in (qb, kb, vb, gc, beta))
    o0, s0 = gdn_prefill(q, k, v, g, bt)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    o1, s1 = gdn_prefill(q, k, v, g, bt, stream=side)
    torch.cuda.current_stream().wait_stream(side)
    _ = torch.empty((1 << 20,), device=gpu).fill_(1.0)  # reuse pressure on the current stream
    torch.cuda.synchronize()
    assert torch.equal(o0, o1) and torch.equal(s0, s1)
