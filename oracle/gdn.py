"""Oracle for the GDN / KDA triangular solve -- TEST INFRASTRUCTURE ONLY.

Functions and the reference lines they follow
---------------------------------------------
* ``l2norm``          -- scripts/gdn_ref_kernel.py:31-32 (x / sqrt(sum x^2 + 1e-6)).
* ``build_A``         -- the strictly-lower A of a chunk, scripts/gdn_ref_kernel.py:71-83:
                         A_ij = -beta_i (k_i . k_j) exp(g_i - g_j) for i > j, g = cumsum(gc).
* ``config4_inputs``  -- the synthetic inputs of the C=256 x 32-head solve: k ~ N(0,1) of
                         dimension 128, beta = sigmoid(N(0,1)), gc = logsigmoid(N(0,1) + 3).
* ``inverse_fp64``    -- np.linalg.inv(I - A) per head, scripts/gdn_solve_oc_check.py:30.
* ``forward_subst``   -- the row recurrence T[i,:i] += T[i,:i] @ T[:i,:i], then + I,
                         scripts/gdn_ref_kernel.py:84-87.
* ``oc``              -- ||T - Tref||_F / (||Tref||_F + 1e-12), scripts/gdn_solve_oc_check.py:31.
* ``quantize_u16`` / ``dequantize_u16`` -- the u16 code contract (zp 32768) of
                         scripts/gdn_solve_oc_check.py:27-29 and GdnSolveOp.cpp:185-254.
* ``solve_int16_blocks`` -- the reference's int16 block model (BL=16 diagonal forward
                         substitution on int16 codes at sT = 2/32767 with int32 accumulation,
                         fp64 block merges): scripts/gdn_solve_int16_model.py:25-56 and
                         example/gdn_native/solve_op/gdn_solve_ref.c:19-69.
* ``solve_int16_op``  -- the GdnSolve op's own scalar model (example/gdn_native/solve_op/src/
                         gdn_solve_core.h:28-83, driven by GdnSolveOp.cpp:201-208): diagonal blocks
                         by forward substitution on int16 codes at the fixed internal scale
                         2/32767 with int32 accumulation and float32 requant (lroundf, clip
                         +-32767), block merges in float32 in the op's loop order, output codes
                         lroundf(T / sTout) clipped to +-maxc.  Every float32 operation is
                         rounded separately (no fused multiply-add), in the op's order.
* ``gdn_solve_op_u16`` -- the op's uint16 contract around it: A = code - zpA, T code + zpT.
* ``chunk_uw``        -- U = T (beta * V), W = T (beta * K) [or T (beta * K * e^g)],
                         scripts/gdn_ref_kernel.py:88-89.
* ``forward_subst_torch`` / ``chunk_stage_a_torch`` -- the same row recurrence and the whole
                         intra-chunk stage (l2norm, A-build, recurrence, U, W) in torch float64,
                         batched over heads as the reference runs them
                         (scripts/gdn_ref_kernel.py:71-89); the CPU baseline times these.
* ``chunk_state_torch`` -- the inter-chunk stage B over a whole sequence of chunks, from the
                         stage-A outputs W (e^g form) and U: P = (q^ k^T) decay (causal),
                         v_new = U - W S, o = (q^ e^g) S + P v_new, S <- S e^{g_last} +
                         (k^ e^{g_last - g})^T v_new, with q^ = l2norm(q) / sqrt(D)
                         (scripts/gdn_ref_kernel.py:66-69,91-101 and the chunk loop :104-131).
* ``gdn_prefill_torch`` -- stage A then stage B per chunk: the reference's ``gdn_kernel``
                         (scripts/gdn_ref_kernel.py:54-131), zero-padding T to whole chunks.
* ``gdn_recurrent``   -- the gated delta rule token by token (decay, delta-rule write,
                         read-out): S <- S e^{g_t}; S <- S + beta_t k^_t (v_t - S^T k^_t)^T;
                         o_t = S^T q^_t.  An independent statement of what the chunked form
                         computes, used to pin it.

Pinning
-------
* ``inverse_fp64`` is LAPACK; it is cross-checked against ``forward_subst`` (independent
  algorithm), against the identity T (I - A) = I, and against the closed form of the
  nilpotent Neumann series on small C.
* ``solve_int16_blocks`` is pinned against the reference's own C model compiled from
  /root/reference (oracle/_ref/gdn_solve_ref, built by oracle/Makefile) on the same codes.
* ``solve_int16_op`` is pinned code for code against the op's core compiled from
  /root/reference (oracle/_ref/gdn_test_core: int8 output at sTout = 1/127), and its float T
  against ``solve_int16_blocks`` (same algorithm in float64).
* ``build_A`` is pinned by closed-form special cases (beta = 0 -> A = 0; orthogonal keys ->
  A = 0; a rank-one check on two tokens).
* ``forward_subst_torch`` and ``chunk_stage_a_torch`` are pinned against LAPACK's inverse
  (``inverse_fp64``) with ``build_A`` / ``chunk_uw``.
* ``gdn_prefill_torch`` (and with it ``chunk_state_torch``) is pinned against
  ``gdn_recurrent``, a token-by-token derivation that shares no code with it, at several chunk
  sizes (the chunked result does not depend on the chunk size), with and without an incoming
  state, and with a ragged T (zero padding must not change the result).
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "l2norm",
    "build_A",
    "config4_inputs",
    "inverse_fp64",
    "forward_subst",
    "oc",
    "quantize_u16",
    "dequantize_u16",
    "solve_int16_blocks",
    "solve_int16_op",
    "gdn_solve_op_u16",
    "chunk_uw",
    "forward_subst_torch",
    "chunk_stage_a_torch",
    "chunk_state_torch",
    "gdn_prefill_torch",
    "gdn_recurrent",
    "GATE_BF16",
    "GATE_FP32",
    "SA_REF",
    "ST_REF",
]

GATE_BF16 = 1.05e-2  # tests/qnn_kernel_e2e/correctness/test_gdn_solve_e2e.sh:18
GATE_FP32 = 1.0e-4
SA_REF = 2.770166930875267e-05  # test_gdn_solve_e2e.sh:19
ST_REF = 6.103701895199438e-05


def l2norm(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    return x / np.sqrt((x * x).sum(axis=-1, keepdims=True) + eps)


def build_A(k: np.ndarray, beta: np.ndarray, gc: np.ndarray) -> np.ndarray:
    """A [..., C, C] (float64) from keys k [..., C, D], beta [..., C], per-token log decay gc [..., C]."""
    kn = l2norm(k.astype(np.float64))
    b = beta.astype(np.float64)
    g = np.cumsum(gc.astype(np.float64), axis=-1)
    C = k.shape[-2]
    diff = g[..., :, None] - g[..., None, :]
    lower = np.tril(np.ones((C, C), dtype=bool), -1)
    decay = np.exp(np.where(lower, diff, 0.0)) * lower
    kk = kn @ np.swapaxes(kn, -1, -2)
    return -(b[..., :, None] * kk) * decay


def config4_inputs(heads: int = 32, C: int = 256, D: int = 128, seed: int = 4):
    rng = np.random.default_rng(seed)
    k = rng.standard_normal((heads, C, D))
    beta = 1.0 / (1.0 + np.exp(-rng.standard_normal((heads, C))))
    z = rng.standard_normal((heads, C)) + 3.0
    gc = -np.logaddexp(0.0, -z)  # logsigmoid(z)
    return k, beta, gc


def inverse_fp64(A: np.ndarray) -> np.ndarray:
    A = np.asarray(A, dtype=np.float64)
    C = A.shape[-1]
    eye = np.eye(C)
    flat = A.reshape(-1, C, C)
    out = np.stack([np.linalg.inv(eye - a) for a in flat])
    return out.reshape(A.shape)


def forward_subst(A: np.ndarray) -> np.ndarray:
    """(I - A)^-1 by the reference's row recurrence on strictly-lower A (float64)."""
    A = np.asarray(A, dtype=np.float64)
    C = A.shape[-1]
    T = np.tril(A, -1).copy()
    for i in range(1, C):
        row = T[..., i, :i].copy()
        T[..., i, :i] = row + np.einsum("...j,...jk->...k", row, T[..., :i, :i])
    return T + np.eye(C)


def oc(T: np.ndarray, Tref: np.ndarray) -> float:
    T = np.asarray(T, dtype=np.float64)
    Tref = np.asarray(Tref, dtype=np.float64)
    return float(np.linalg.norm(T - Tref) / (np.linalg.norm(Tref) + 1e-12))


def quantize_u16(x: np.ndarray, scale: float, zp: int = 32768) -> np.ndarray:
    return np.clip(np.rint(np.asarray(x, np.float64) / scale) + zp, 0, 65535).astype(np.uint16)


def dequantize_u16(codes: np.ndarray, scale: float, zp: int = 32768) -> np.ndarray:
    return (codes.astype(np.int64) - zp) * scale


def solve_int16_blocks(Aq: np.ndarray, sA: float, sT: float, BL: int = 16) -> np.ndarray:
    """Reference int16 block model on int16 codes Aq [C, C] at scale sA; returns T (float64)."""
    Aq = np.asarray(Aq, dtype=np.int64)
    C = Aq.shape[0]
    nb = C // BL
    Ti = np.zeros((nb, BL, BL), np.int64)
    for b in range(nb):
        d = Aq[b * BL:(b + 1) * BL, b * BL:(b + 1) * BL]
        Tb = np.zeros((BL, BL), np.int64)
        for i in range(BL):
            acc = (d[i, :i][:, None] * Tb[:i, :]).sum(0) if i else np.zeros(BL, np.int64)
            e = np.zeros(BL)
            e[i] = 1.0 / sT
            v = e + acc.astype(np.float64) * sA
            v = np.clip(v, -32767.0, 32767.0)
            # llround: half away from zero
            Tb[i, :] = (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int64)
        Ti[b] = Tb
    blk = {(b, b): Ti[b].astype(np.float64) * sT for b in range(nb)}
    for i in range(nb):
        for j in range(i - 1, -1, -1):
            acc = np.zeros((BL, BL))
            for k in range(j, i):
                Aik = Aq[i * BL:(i + 1) * BL, k * BL:(k + 1) * BL].astype(np.float64) * sA
                acc += Aik @ blk[(k, j)]
            blk[(i, j)] = blk[(i, i)] @ acc
    T = np.zeros((C, C))
    for i in range(nb):
        for j in range(i + 1):
            T[i * BL:(i + 1) * BL, j * BL:(j + 1) * BL] = blk[(i, j)]
    return T


def _lroundf(v: np.ndarray) -> np.ndarray:
    """C lroundf on float32 values: round half away from zero (evaluated in float64, where
    |v| + 0.5 is exact)."""
    v = np.asarray(v, np.float32).astype(np.float64)
    return (np.sign(v) * np.floor(np.abs(v) + 0.5)).astype(np.int64)


def solve_int16_op(Aq: np.ndarray, sA: float, sTout: float, maxc: float) -> np.ndarray:
    """The GdnSolve op's scalar model on one head (gdn_solve_core.h:28-83): int16 codes Aq
    [C, C] (C % 16 == 0, C <= 64) at scale sA -> output codes [C, C] (int64) at sTout, clipped to
    +-maxc, zero above the diagonal.  float32 arithmetic, one rounding per operation."""
    f32 = np.float32
    A = np.asarray(Aq, np.int64)
    C = A.shape[0]
    BL, nb = 16, C // 16
    sA, sTout, maxc = f32(sA), f32(sTout), f32(maxc)
    sTi = f32(2.0) / f32(32767.0)
    inv_sTi = f32(1.0) / sTi
    inv_sTout = f32(1.0) / sTout
    Tf = np.zeros((C, C), f32)
    for b in range(nb):
        Tb = np.zeros((BL, BL), np.int64)
        d = A[b * BL:(b + 1) * BL, b * BL:(b + 1) * BL]
        for i in range(BL):
            acc = (d[i, :i][:, None] * Tb[:i, :]).sum(0) if i else np.zeros(BL, np.int64)
            acc = (acc + 2 ** 31) % 2 ** 32 - 2 ** 31  # the core's int32 accumulator (two's complement)
            ei = np.where(np.arange(BL) == i, inv_sTi, f32(0.0)).astype(f32)
            v = (ei + (acc.astype(f32) * sA)).astype(f32)
            Tb[i] = np.clip(_lroundf(v), -32767, 32767)
        Tf[b * BL:(b + 1) * BL, b * BL:(b + 1) * BL] = (Tb.astype(f32) * sTi).astype(f32)
    Af = A.astype(f32)
    for j in range(nb):
        for i in range(j + 1, nb):
            acc = np.zeros((BL, BL), f32)
            for k in range(j, i):
                s = np.zeros((BL, BL), f32)
                for m in range(BL):  # s += (A * sA) * Tf, left to right, one rounding each
                    a = (Af[i * BL:(i + 1) * BL, k * BL + m] * sA).astype(f32)
                    s = (s + (a[:, None] * Tf[k * BL + m, j * BL:(j + 1) * BL][None, :]).astype(f32)).astype(f32)
                acc = (acc + s).astype(f32)
            s = np.zeros((BL, BL), f32)
            for m in range(BL):
                s = (s + (Tf[i * BL:(i + 1) * BL, i * BL + m][:, None] * acc[m][None, :]).astype(f32)).astype(f32)
            Tf[i * BL:(i + 1) * BL, j * BL:(j + 1) * BL] = s
    q = np.clip(_lroundf((Tf * inv_sTout).astype(f32)), -int(maxc), int(maxc))
    return np.tril(q)


def gdn_solve_op_u16(Au: np.ndarray, zpA: int, sA: float, zpT: int, sT: float) -> np.ndarray:
    """The op's uint16 contract per head (GdnSolveOp.cpp:201-208): A codes - zpA as int16, the
    model with output scale sT and clip 32767, + zpT.  Au [..., C, C] uint16 -> uint16."""
    Au = np.asarray(Au)
    C = Au.shape[-1]
    flat = Au.reshape(-1, C, C)
    out = np.empty(flat.shape, np.uint16)
    for h in range(flat.shape[0]):
        As = (flat[h].astype(np.int64) - zpA).astype(np.int16)
        out[h] = (solve_int16_op(As, sA, sT, 32767.0) + zpT).astype(np.uint16)
    return out.reshape(Au.shape)


def chunk_uw(T: np.ndarray, k: np.ndarray, v: np.ndarray, beta: np.ndarray, gc: np.ndarray, decay_w: bool = False):
    """U = T (beta * v), W = T (beta * l2norm(k)) [times e^g when decay_w] (float64)."""
    kn = l2norm(k.astype(np.float64))
    b = beta.astype(np.float64)[..., None]
    U = T @ (b * v.astype(np.float64))
    kb = b * kn
    if decay_w:
        kb = kb * np.exp(np.cumsum(gc.astype(np.float64), axis=-1))[..., None]
    return U, T @ kb


def forward_subst_torch(A):
    """(I - A)^-1 of strictly-lower A [..., C, C] by the reference's row recurrence, in torch
    float64 (scripts/gdn_ref_kernel.py:84-87)."""
    import torch

    A = torch.as_tensor(A, dtype=torch.float64)
    C = A.shape[-1]
    T = torch.tril(A, -1).clone()
    for i in range(1, C):
        row = T[..., i, :i].clone()
        T[..., i, :i] = row + torch.einsum("...j,...jk->...k", row, T[..., :i, :i])
    return T + torch.eye(C, dtype=torch.float64)


def chunk_stage_a_torch(k, v, gc, beta, decay_w: bool = True):
    """The intra-chunk stage of the reference GDN kernel on [n, C, D] keys / values and [n, C]
    per-token log decays / betas, torch float64 (scripts/gdn_ref_kernel.py:71-89): l2norm,
    k_beta / v_beta, g = cumsum, A = -(k_beta k^T) decay below the diagonal, the row recurrence,
    U = T v_beta, W = T (k_beta [e^g]).  Returns (U, W)."""
    import torch

    k = torch.as_tensor(k, dtype=torch.float64)
    v = torch.as_tensor(v, dtype=torch.float64)
    gc = torch.as_tensor(gc, dtype=torch.float64)
    beta = torch.as_tensor(beta, dtype=torch.float64)
    C = k.shape[-2]
    kn = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    v_beta = v * beta.unsqueeze(-1)
    k_beta = kn * beta.unsqueeze(-1)
    g = torch.cumsum(gc, dim=-1)
    lower = torch.tril(torch.ones(C, C, dtype=torch.bool), -1)
    decay = torch.exp(torch.where(lower, g.unsqueeze(-1) - g.unsqueeze(-2), torch.zeros((), dtype=torch.float64)))
    A = -(k_beta @ kn.transpose(-1, -2)) * decay * lower
    T = forward_subst_torch(A)
    U = T @ v_beta
    W = T @ (k_beta * torch.exp(g).unsqueeze(-1) if decay_w else k_beta)
    return U, W


def chunk_stage_a_solve_torch(k, v, gc, beta, decay_w: bool = True):
    """The outputs (U, W) of ``chunk_stage_a_torch`` by a batched float64 triangular solve
    (I - A) [U | W] = [v_beta | k_beta (e^g)] in place of the row recurrence (LAPACK's unit-lower
    solve; T is never formed).  Same definitions as scripts/gdn_ref_kernel.py:71-89; this form
    checks every item of a full-size launch in seconds."""
    import torch

    k = torch.as_tensor(k, dtype=torch.float64)
    v = torch.as_tensor(v, dtype=torch.float64)
    gc = torch.as_tensor(gc, dtype=torch.float64)
    beta = torch.as_tensor(beta, dtype=torch.float64)
    C = k.shape[-2]
    kn = k / torch.sqrt((k * k).sum(-1, keepdim=True) + 1e-6)
    v_beta = v * beta.unsqueeze(-1)
    k_beta = kn * beta.unsqueeze(-1)
    g = torch.cumsum(gc, dim=-1)
    lower = torch.tril(torch.ones(C, C, dtype=torch.bool), -1)
    decay = torch.exp(torch.where(lower, g.unsqueeze(-1) - g.unsqueeze(-2), torch.zeros((), dtype=torch.float64)))
    A = -(k_beta @ kn.transpose(-1, -2)) * decay * lower
    M = torch.eye(C, dtype=torch.float64) - A
    rhs = torch.cat([v_beta, k_beta * torch.exp(g).unsqueeze(-1) if decay_w else k_beta], dim=-1)
    X = torch.linalg.solve_triangular(M, rhs, upper=False, unitriangular=True)
    return X[..., : v.shape[-1]], X[..., v.shape[-1]:]


def _l2n(x):
    import torch

    return x / torch.sqrt((x * x).sum(-1, keepdim=True) + 1e-6)


def chunk_state_torch(q, k, gc, W, U, S_in=None, C: int = 64, _plant: str = ""):
    """Stage B over whole sequences, torch float64 (scripts/gdn_ref_kernel.py:66-69,91-101).

    q, k [n, T, D] (raw; l2norm and 1/sqrt(D) applied here), gc [n, T] per-token log decays,
    W, U [n, T, D] the stage-A outputs of the same chunking (W in the T (beta k^ e^g) form),
    S_in [n, D, D] or None.  Returns (o [n, T, D], S_out [n, D, D]).

    ``_plant`` (tests only) plants one plausible mistake, to show that the comparison against
    the token recurrence catches it: "state_decay" (S not decayed by e^{g_last}), "transpose_S"
    (S read transposed), "strict_causal" (P without its diagonal), "q_decay" (o's first term
    without e^g), "k_decay" (the S update without e^{g_last - g})."""
    import torch

    f64 = torch.float64
    q, k, gc, W, U = (torch.as_tensor(x, dtype=f64) for x in (q, k, gc, W, U))
    n, T, D = q.shape
    assert T % C == 0
    qn = _l2n(q) * (1.0 / D ** 0.5)
    kn = _l2n(k)
    S = torch.zeros(n, D, D, dtype=f64) if S_in is None else torch.as_tensor(S_in, dtype=f64).clone()
    o = torch.zeros(n, T, D, dtype=f64)
    assert _plant in ("", "state_decay", "transpose_S", "strict_causal", "q_decay", "k_decay")
    causal = torch.tril(torch.ones(C, C, dtype=torch.bool), diagonal=-1 if _plant == "strict_causal" else 0)
    for c0 in range(0, T, C):
        sl = slice(c0, c0 + C)
        g = torch.cumsum(gc[:, sl], dim=-1)
        decay = torch.exp(torch.where(causal, g.unsqueeze(-1) - g.unsqueeze(-2), torch.zeros((), dtype=f64))) * causal
        P = (qn[:, sl] @ kn[:, sl].transpose(-1, -2)) * decay
        Sr = S.transpose(-1, -2) if _plant == "transpose_S" else S
        v_new = U[:, sl] - W[:, sl] @ Sr
        qe = qn[:, sl] if _plant == "q_decay" else qn[:, sl] * torch.exp(g).unsqueeze(-1)
        o[:, sl] = qe @ Sr + P @ v_new
        g_last = g[:, -1]
        dec = torch.exp(g_last.unsqueeze(-1) - g).unsqueeze(-1)
        if _plant == "k_decay":
            dec = torch.ones_like(dec)
        keep = torch.ones_like(g_last) if _plant == "state_decay" else torch.exp(g_last)
        S = S * keep[:, None, None] + (kn[:, sl] * dec).transpose(-1, -2) @ v_new
    return o, S


def gdn_prefill_torch(q, k, v, gc, beta, C: int = 64, S_in=None, _plant: str = ""):
    """The reference's chunked prefill (scripts/gdn_ref_kernel.py:54-131) in torch float64 on
    [n, T, D] / [n, T] inputs: zero-pad T to whole chunks, stage A per chunk
    (``chunk_stage_a_torch``, W in the e^g form), then stage B.  Returns (o [n, T, D], S).
    ``_plant``: passed to ``chunk_state_torch`` (tests only)."""
    import torch

    f64 = torch.float64
    q, k, v, gc, beta = (torch.as_tensor(x, dtype=f64) for x in (q, k, v, gc, beta))
    n, T, D = q.shape
    pad = (-T) % C
    if pad:
        F = torch.nn.functional
        q, k, v = (F.pad(x, (0, 0, 0, pad)) for x in (q, k, v))
        gc, beta = F.pad(gc, (0, pad)), F.pad(beta, (0, pad))
    Tp = T + pad
    U, W = chunk_stage_a_torch(k.reshape(n * Tp // C, C, D), v.reshape(n * Tp // C, C, D),
                               gc.reshape(n * Tp // C, C), beta.reshape(n * Tp // C, C), decay_w=True)
    o, S = chunk_state_torch(q, k, gc, W.reshape(n, Tp, D), U.reshape(n, Tp, D), S_in, C, _plant)
    return o[:, :T], S


def gdn_recurrent(q, k, v, gc, beta, S_in=None):
    """The gated delta rule one token at a time, torch float64 on [n, T, D] / [n, T] inputs:
    S <- S e^{gc_t};  S <- S + beta_t k^_t (v_t - S^T k^_t)^T;  o_t = S^T q^_t, with
    k^ = l2norm(k), q^ = l2norm(q) / sqrt(D).  Returns (o, S)."""
    import torch

    f64 = torch.float64
    q, k, v, gc, beta = (torch.as_tensor(x, dtype=f64) for x in (q, k, v, gc, beta))
    n, T, D = q.shape
    qn = _l2n(q) * (1.0 / D ** 0.5)
    kn = _l2n(k)
    S = torch.zeros(n, D, D, dtype=f64) if S_in is None else torch.as_tensor(S_in, dtype=f64).clone()
    o = torch.zeros(n, T, D, dtype=f64)
    for t in range(T):
        S = S * torch.exp(gc[:, t])[:, None, None]
        kt = kn[:, t]
        delta = (v[:, t] - torch.einsum("nkv,nk->nv", S, kt)) * beta[:, t, None]
        S = S + kt[:, :, None] * delta[:, None, :]
        o[:, t] = torch.einsum("nkv,nk->nv", S, qn[:, t])
    return o, S
