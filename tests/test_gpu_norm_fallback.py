"""RmsNorm's sequential fallback (src/CpuRef.cs:186-188: the double sum of x_i^2 in index order, then
(float)(sum / n)), which the kernels take when the bound on their parallel sum cannot certify the float
mean.

What is pinned:
- the wave routine that replays the sequential sum (seq_sum_sq_wave, selftest op 10), bit for bit against
  the sequential float64 sum on rows that keep it in one binade, cross powers of two at chunk edges, add
  exact halves of the sum's last place (round to even against the sum's parity), start with zeros or
  with one huge term, hold inf or NaN, and on every length class (the term-by-term path below 512
  elements, chunk counts that do not divide the row);
- the layer paths that call it: token rows planted with a mean of squares on a float rounding boundary
  (within 1e-13 of the midpoint, far inside the bound) send the prologue's and the many-token router's
  means to the fallback (counted); ids and lists stay bit-exact and the expert inputs too (gate, up and
  down products), two tied experts send most tokens through the exact chains, which scale by the
  router's fallback mean, and with the exact-chain router (which scales by the prologue's) logits,
  weights and outputs equal the oracle's bit for bit."""
import math
import sys
from fractions import Fraction

import numpy as np
import pytest

from test_gpu_parity import check_layer

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def seq_sq(row):
    """The reference's sum: float64 squares added in index order (np.add.accumulate is sequential)."""
    sq = row.astype(np.float64) ** 2
    return np.add.accumulate(sq)[-1] if len(sq) else 0.0


def dev_seq(ctx, rows):
    m = rows.shape[1]
    b = np.zeros(rows.size, np.float32)
    b[0] = m
    out = ctx.selftest(10, rows.ravel(), b)
    bits = out.view(np.uint32)[: 2 * rows.shape[0]].reshape(-1, 2).astype(np.uint64)
    return (bits[:, 0] | (bits[:, 1] << np.uint64(32))).view(np.float64)


def rows_of(kind, m, rng, nrows=6):
    if kind == "normal":
        return rng.standard_normal((nrows, m)).astype(np.float32)
    if kind == "wide":
        return (rng.standard_normal((nrows, m)) * np.exp2(rng.integers(-30, 30, (nrows, m)))).astype(np.float32)
    if kind == "halves":  # the sum reaches [512, 1024), then terms whose last bit is half its last place
        r = np.ones((nrows, m), np.float32)
        for i in range(nrows):
            r[i, int(m * (0.15 + 0.13 * i)):] = np.float32(1 + 2.0 ** -22)
            r[i, rng.integers(0, m, 7)] = np.float32(1 + 2.0 ** -23)
        return r
    if kind == "steps":  # exact sums that land on powers of two at chunk edges
        r = np.ones((nrows, m), np.float32)
        r[:, ::3] = np.float32(2.0)
        return r
    if kind == "leading_zeros":
        r = rng.standard_normal((nrows, m)).astype(np.float32)
        for i in range(nrows):
            r[i, : int(m * 0.1 * (i + 1))] = 0.0
        return r
    if kind == "huge_first":
        r = (rng.standard_normal((nrows, m)) * 1e-3).astype(np.float32)
        r[:, 0] = np.float32(3e4)
        return r
    if kind == "nonfinite":
        r = rng.standard_normal((nrows, m)).astype(np.float32)
        r[0, m // 3] = np.inf
        r[1, m // 2] = np.nan
        r[2, -1] = -np.inf
        r[3, 0] = np.float32(3e38)  # its square is finite in double
        return r
    raise ValueError(kind)


@pytest.mark.parametrize("m", [2, 63, 511, 512, 513, 704, 1000, 2816, 4096, 5000, 16384])
def test_seq_sum_sq_wave(ctx, m):
    say(f"seq_sum_sq_wave m={m}")
    rng = np.random.default_rng(m)
    for kind in ["normal", "wide", "halves", "steps", "leading_zeros", "huge_first", "nonfinite"]:
        rows = rows_of(kind, m, rng)
        got = dev_seq(ctx, rows)
        ref = np.array([seq_sq(r) for r in rows])
        same = (got.view(np.uint64) == ref.view(np.uint64)) | (np.isnan(got) & np.isnan(ref))
        assert same.all(), f"m={m} {kind}: {[(g, r) for g, r, o in zip(got, ref, same) if not o][:3]}"


def plant_boundary(row):
    """A copy of the row whose sequential mean of squares lies within 1e-13 (relative) of the midpoint
    between two floats, far inside any certifying bound: elements 0 and 1 are set so that the exact sum
    hits d times the midpoint (element 1 a small value whose square takes up the remainder)."""
    r = row.astype(np.float32).copy()
    d = len(r)
    r[0] = r[1] = 0.0
    rest = sum(Fraction(float(v) * float(v)) for v in r)  # exact
    m = np.float32(float(rest) / d + 1.0)
    mid = (Fraction(float(m)) + Fraction(float(np.nextafter(m, np.float32(np.inf))))) / 2
    need = mid * d - rest  # x0^2 + x1^2
    x0 = np.float32(math.sqrt(float(need)))
    while Fraction(float(x0)) ** 2 > need:
        x0 = np.nextafter(x0, np.float32(0))
    r[0] = x0
    r[1] = np.float32(math.sqrt(float(need - Fraction(float(x0)) ** 2)))
    S = seq_sq(r)
    assert abs(S / d - float(mid)) <= 1e-13 * float(mid)
    B = (d + 64.0) * 2.0 ** -52 * S  # the kernels' bound: its float ends straddle the midpoint
    assert np.float32((S - B) / d) != np.float32((S + B) / d)
    return r


CASES = {
    # (layer config, tokens): T * E > 8192 in each, so the matrix-core router forms the rows' scales
    "d512_E32_T300": dict(idx=74, T=300, d=512, E=32, k=4, nf=256, gu=2, dn=2),
    "c3_T300": "c3_prefill",
    "c4_T300": "c4_kquant",
}


@pytest.mark.parametrize("case", list(CASES))
def test_layer_planted_mean_boundary(ctx, pkg, orc, case):
    cfg = CASES[case]
    T = 300
    say(f"planted mean boundary {case}")
    L = dict(pkg.synth.make_layer(cfg))
    x = pkg.synth.make_input(cfg, T=T).copy()
    # two tied experts along the tokens' mean: tokens that rank both take the exact chains
    W = L["gate_inp"].copy()
    xbar = x.mean(0)
    W[2] = (0.5 * xbar / np.linalg.norm(xbar)).astype(np.float32)
    W[5] = W[2]
    L["gate_inp"] = W
    planted = [0, 7, 150, 151, T - 1]
    for t in planted:
        x[t] = plant_boundary(x[t])
    ctx.upload(0, L)
    for exact in (False, True):
        before = ctx.fallback_counts()
        check_layer(ctx, orc, L, x, tag=f"planted {case} exact={exact}", exact=exact)
        after = ctx.fallback_counts()
        nfb = after[0] - before[0]
        say(f"  exact router {exact}: norm fallbacks {nfb}, exact-chain tokens {after[1] - before[1]}")
        # each planted row's mean in the prologue, and with the matrix-core router in the router too (the
        # combine's norms may add more)
        assert nfb >= (1 if exact else 2) * len(planted)
        if not exact:
            assert after[1] - before[1] >= T // 3
