"""Adversarial quantized-matmul inputs that put many outputs next to a rounding boundary.

The kernels round ``t = S * alpha + beta`` directly when t is farther than a per-channel margin
from a half-integer; closer outputs go to the exact recomputation (the integer residue pass for
8-bit activations, the float64 emulation of the oracle's dot product for the rest).  Ordinary
data flags about 1e-4 of the outputs.  The cases here flag far more:

* one weight scale s for every channel and the output scale 2 * sA * s * (1 + 1e-9), so each
  unit of the integer dot product moves t by almost exactly half an output LSB;
* "tie rows": activations equal to the zero point except at 6 random positions, so t sits
  within ~1e-6 LSB of a half-integer for about half of the outputs -- decided only by the
  float32 rounding residues of the dequantised weights;
* "zero rows": activations equal to the zero point everywhere, so t = bias / 2 + out_zp
  (times 1 - 1e-9), which the integer pass leaves to the float64 emulation;
* "rail rows": activations 0 or 255 at random, so most of their outputs saturate.

A row tile with a few tie rows stays under the per-tile list capacity; a tile of tie rows
overflows it and takes the whole-tile path.
"""

import dataclasses

import numpy as np

from qcom_htp_amd import cases as C


def near_tie_case(fam, m, k, n, seed, tie_rows, zero_rows=(), rail_rows=()):
    c = C.synthetic_case(fam, m, k, n, seed=seed)
    rng = np.random.default_rng(seed + 1)
    # odd float32 mantissa: the products w * s need more than 24 bits, so residues are nonzero
    s = np.array([rng.uniform(1e-3, 1e-2)], dtype=np.float32)
    s = (s.view(np.uint32) | np.uint32(1)).view(np.float32)[0]
    zp = c.family.act_zp
    x = c.activation_q.copy()
    for r in tie_rows:
        x[r] = zp
        pos = rng.choice(k, size=6, replace=False)
        x[r, pos] = zp + rng.integers(-3, 4, size=6)
    for r in zero_rows:
        x[r] = zp
    for r in rail_rows:
        x[r] = rng.choice(np.array([0, c.family.act_qmax], x.dtype), size=k)
    w_int = c.lpbq_expanded_q_nk if c.lpbq_expanded_q_nk is not None else c.weight_q_nk
    return dataclasses.replace(
        c,
        activation_q=x,
        weight_scale=np.full(n, s, np.float32),
        bias_q=rng.integers(-200, 200, size=n).astype(np.int32),
        out_scale=2.0 * c.act_scale * float(s) * (1.0 + 1e-9),
        weight_deq=w_int.astype(np.float32) * s,
    )


def flagged_per_tile(c, dequantized, tile=256):
    """Outputs per 256 x 256 tile whose rounding an 8-bit-activation kernel cannot certify
    from the int32 accumulator alone (|t - rint t| > 0.5 - margin), from the float64 t."""
    fam = c.family
    w = (c.lpbq_expanded_q_nk if c.lpbq_expanded_q_nk is not None else c.weight_q_nk).astype(np.int64)
    s = np.asarray(c.weight_scale, np.float32)
    fr, e = np.frexp(s.astype(np.float64))
    mant = np.ldexp(fr, 24).astype(np.int64)
    ex = e - 24
    wp = np.ldexp((w.astype(np.float32) * s[:, None]).astype(np.float64), -ex[:, None]).astype(np.int64)
    resid = wp - w * mant[:, None]
    amax = max(fam.act_zp, fam.act_qmax - fam.act_zp)
    margin = c.act_scale * np.ldexp(1.0, ex) / c.out_scale * amax * np.abs(resid).sum(1)
    t = dequantized / c.out_scale + fam.out_zp
    fl = (np.abs(t - np.rint(t)) > 0.5 - margin[None, :]) & (t > -1) & (t < fam.out_qmax + 1)
    m, n = fl.shape
    return np.array([[fl[i:i + tile, j:j + tile].sum() for j in range(0, n, tile)] for i in range(0, m, tile)])


def stress_layout(k=512):
    """(m, k, n, tie_rows, zero_rows, rail_rows): row tile 0 has 5 tie rows, a zero row and rail
    rows, row tile 1 is all tie rows; n = 288 leaves a ragged second column tile."""
    tie = list(range(0, 256, 52)) + list(range(256, 512))
    zero = [3]
    rail = [r for r in range(256) if r not in tie and r not in zero]
    return 512, k, 288, tie, zero, rail
