"""The one-launch contract chain computes the dividing contracts in float64 without a division
(a reciprocal product; only quotients near a half-integer take the exact integer remainder that
picks the rounding neighbour).  This
restates that algorithm with numpy and checks it against the oracle's contracts over random
accumulators, exact ties, near-ties and the extremes of the divisor range (CPU only).  numpy has
no fused multiply-add: the reciprocal product and the sum round separately here, which the error
bound of the kernel's comment covers as well."""

import numpy as np
import pytest

from oracle import qmm as oq


def chain_div_rint(D, d, zp, qmax, floor256=False):
    Dd = D.astype(np.float64)
    if floor256:
        Dd = np.floor(Dd * 2.0 ** -8) * 256.0
    rcp = 1.0 / float(d)
    y = Dd * rcp + zp
    c = np.rint(y)
    near = (np.abs(y - c) > 0.5 - 2.0 ** -20) & (c >= -1.0) & (c <= qmax + 1.0)
    near = np.broadcast_to(near.any(), near.shape)  # the kernel corrects every lane of such a wave
    r2 = 2.0 * ((zp - c) * d + Dd)
    h = c * 0.5
    odd = h != np.floor(h)
    up = near & ((r2 > d) | ((r2 == d) & odd))
    down = near & ((r2 < -d) | ((r2 == -d) & odd))
    c = np.where(up, c + 1.0, np.where(down, c - 1.0, c))
    return np.clip(c, 0.0, qmax).astype(np.int64)


def chain_round_div(D, d, zp, qmax):
    Dd = D.astype(np.float64)
    rcp = 1.0 / float(d)
    n = np.abs(Dd) + float(d // 2)
    q = np.floor(n * rcp)
    r = n - q * d
    q = np.where(r < 0, q - 1.0, np.where(r >= d, q + 1.0, q))
    return np.clip(np.where(Dd >= 0, q, -q) + zp, 0.0, qmax).astype(np.int64)


def accumulators(d, rng):
    """Random |D| < 2^40, exact ties (D = (2n + 1) d / 2), their integer neighbours, and values
    that divide to just inside and outside the output range."""
    base = rng.integers(-(1 << 40), 1 << 40, size=4000, dtype=np.int64)
    mid = rng.integers(-(1 << 20), 1 << 20, size=4000, dtype=np.int64) * d + rng.integers(-d, d + 1, size=4000)
    ties = []
    if d % 2 == 0:
        n = rng.integers(-(1 << 17), 1 << 17, size=2000, dtype=np.int64)
        t = (2 * n + 1) * (d // 2)
        ties = [t, t - 1, t + 1]
    edge = np.arange(-3 * d, 3 * d + 1, max(1, d // 7), dtype=np.int64)
    edge2 = edge + 65535 * d
    return np.concatenate([base, mid, edge, edge2] + ties)


@pytest.mark.parametrize("d", [1, 2, 7, 127, 256, 1000, 32767, 65536, (1 << 30) - 1, 1 << 30])
@pytest.mark.parametrize("zp,bits", [(0, 8), (128, 8), (32768, 16), (0, 16)])
def test_f64_dividing_contracts_match_oracle(d, zp, bits):
    rng = np.random.default_rng(d + zp + bits)
    D = accumulators(d, rng)[None, :]
    qmax = (1 << bits) - 1
    for name, floor256 in (("div_rint", False), ("floor256_div_rint", True)):
        want = oq.contract_output(D, name, d, None, zp, bits).astype(np.int64)
        got = chain_div_rint(D, d, zp, qmax, floor256)
        assert np.array_equal(got, want), f"{name} d={d}: {int((got != want).sum())} differ"
    want = oq.contract_output(D, "round_div", d, None, zp, bits).astype(np.int64)
    assert np.array_equal(chain_round_div(D, d, zp, qmax), want)


def test_f64_contract_mistake_is_caught():
    """A remainder test without the ties-to-even rule (a plausible slip) fails on exact ties."""
    d, zp, qmax = 2, 0, 255
    D = np.arange(-20, 600, dtype=np.int64)[None, :]
    want = oq.contract_output(D, "div_rint", d, None, zp, 8).astype(np.int64)
    Dd = D.astype(np.float64)
    c = np.rint(Dd / d + zp)
    r2 = 2.0 * ((zp - c) * d + Dd)
    wrong = np.clip(np.where(r2 >= d, c + 1, np.where(r2 < -d, c - 1, c)), 0, qmax)
    assert not np.array_equal(wrong, want)
