"""The certified router for many tokens (T * E above the workgroup-per-pair router's 8192 pairs): logits
as fp32 matrix-core sums with an error bound, the top-k certified from the bounds, the exact float chains
of the reference (src/GemmaCpu.cs:389-405) for the tokens whose order the bounds leave open.

What is pinned:
- the matrix-core arithmetic the bound assumes (every rounding inside a 4-deep fp32 product to nearest:
  |D - exact| <= 5 u (|C| + sum |a b|)), on random and crafted inputs;
- ids and expert lists bit-exact against the oracle on partial tiles in both tile shapes, odd row
  widths (chunk counts not a multiple of the eight waves), E not a multiple of 16, the CPUREF weight
  rule; logits within 1e-5, weights and outputs within the tolerance;
- the fallback: planted exact ties are resolved to the lower index through the exact chains, and a NaN
  router weight sends every token of the call through them."""
import math
import sys

import numpy as np
import pytest

from test_gpu_parity import check_layer, layer

pytestmark = pytest.mark.gpu

U = 2.0 ** -24


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _mfma_ref(a, b, c):
    """Exact D[4 (l / 16)][l % 16] of each 64-lane group (A[i][k] = a[i + 16 k], B[k][j] = b[j + 16 k]),
    with sum |C| + |a b| beside it."""
    a = a.reshape(-1, 4, 16).astype(np.float64)  # [group][k][i]
    b = b.reshape(-1, 4, 16).astype(np.float64)  # [group][k][j]
    exact = np.empty((a.shape[0], 64))
    mag = np.empty_like(exact)
    for gi in range(a.shape[0]):
        for l in range(64):
            i, j = 4 * (l // 16), l % 16
            terms = [c] + [a[gi, k, i] * b[gi, k, j] for k in range(4)]  # products exact in float64
            exact[gi, l] = math.fsum(terms)
            mag[gi, l] = sum(abs(t) for t in terms)
    return exact.reshape(-1), mag.reshape(-1)


@pytest.mark.parametrize("op,c", [(8, 0.0), (9, 1.0)])
def test_mfma_f32_rounding(ctx, op, c):
    """v_mfma_f32_16x16x4_f32 within 5 u (|C| + sum |a b|) of the exact sum on random operands of mixed
    magnitudes and signs (the bound's premise), and rounding to nearest where truncation would differ."""
    say(f"mfma f32 numerics op={op}")
    rng = np.random.default_rng(31 + op)
    n = 64 * 512
    a = (rng.standard_normal(n) * np.exp2(rng.integers(-8, 8, n))).astype(np.float32)
    b = (rng.standard_normal(n) * np.exp2(rng.integers(-8, 8, n))).astype(np.float32)
    got = ctx.selftest(op, a, b).astype(np.float64)
    exact, mag = _mfma_ref(a, b, c)
    err = np.abs(got - exact)
    assert np.all(err <= 5 * U * mag + 1e-38), f"worst {np.max(err / (U * mag + 1e-38)):.2f} u"
    say(f"  worst error {np.max(err / (U * mag + 1e-38)):.3f} u of sum |terms| (bound 5)")
    if op == 9:
        # C = 1 plus one product of 1.5 u: to nearest 1 + 2 u, truncated 1
        a = np.zeros(64, np.float32)
        b = np.zeros(64, np.float32)
        a[0], b[0] = np.float32(1.5 * U), np.float32(1.0)
        assert ctx.selftest(9, a, b)[0] == np.float32(1.0 + 2 * U)
        # C = 1 plus two products of 0.75 u each: exact sum then one rounding gives 1 + 2 u, a rounding per
        # addition 1 (either lies within the bound; reported)
        a[0], a[16], b[16] = np.float32(0.75 * U), np.float32(0.75 * U), np.float32(1.0)
        r = float(ctx.selftest(9, a, b)[0])
        say(f"  1 + 0.75 u + 0.75 u -> 1 + {(r - 1.0) / U:.0f} u")


def _layer(pkg, cfg):
    return layer(pkg, cfg) if isinstance(cfg, str) else pkg.synth.make_layer(cfg)


CASES = {
    # (layer, T): T * E > 8192 in each
    "c3_T600_small_tiles": ("c3_prefill", 600),
    # E = 72 (not a multiple of 16), d = 1056 (66 chunks of 16: two of the eight waves take nine)
    "odd_E72_d1056_T200": (dict(idx=71, T=200, d=1056, E=72, k=6, nf=256, gu=2, dn=2), 200),
    # 35 x 8 tiles of 32 x 32 (at least 256: the large tiles), the last token tile partial
    "E256_T1100_large_tiles": (dict(idx=72, T=1100, d=512, E=256, k=8, nf=128, gu=2, dn=2), 1100),
    "c4_kquant_T300": ("c4_kquant", 300),
}


@pytest.mark.parametrize("case", list(CASES))
def test_router_mm_layers(ctx, pkg, orc, case):
    cfg, T = CASES[case]
    say(f"router_mm {case}")
    L = _layer(pkg, cfg)
    x = pkg.synth.make_input(cfg, T=T)
    assert T * L["n_expert"] > 8192
    before = ctx.fallback_counts()[1]
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"router_mm {case}")
    say(f"  {ctx.fallback_counts()[1] - before} of {T} tokens through the exact chains")


def test_router_mm_cpuref_weights(ctx, pkg, orc):
    say("router_mm CPUREF weights c3 T=300")
    L = layer(pkg, "c3_prefill", weight_rule=1)
    x = pkg.synth.make_input("c3_prefill", T=300)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag="router_mm cpuref")


def test_router_mm_tie_fallback(ctx, pkg, orc):
    """Identical router rows for experts 2 and 5 along the tokens' mean: both rank in most tokens' top-k
    with equal logits, which no bound separates; the exact chains take the lower index first."""
    cfg = dict(idx=73, T=300, d=512, E=32, k=4, nf=256, gu=2, dn=2)
    L = dict(_layer(pkg, cfg))
    x = pkg.synth.make_input(cfg, T=300)
    W = L["gate_inp"].copy()
    xbar = x.mean(0)
    W[2] = (0.5 * xbar / np.linalg.norm(xbar)).astype(np.float32)
    W[5] = W[2]
    L["gate_inp"] = W
    before = ctx.fallback_counts()[1]
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag="router_mm tie")
    ids = ctx.routing()[0]
    both = [list(r) for r in ids if 2 in r and 5 in r]
    assert len(both) >= 150 and all(r.index(2) < r.index(5) for r in both)
    fb = ctx.fallback_counts()[1] - before
    say(f"  tokens with both tied experts {len(both)}, through the exact chains {fb}")
    assert fb >= len(both)


def test_router_mm_nan_row(ctx, pkg, orc):
    """A NaN router weight: no token's order is certified, every token takes the exact chains for every
    expert, and the NaN expert ranks as the reference's scan ranks it."""
    L = dict(layer(pkg, "c2_decode"))
    W = L["gate_inp"].copy()
    W[11, 5] = np.nan
    L["gate_inp"] = W
    T = 80
    x = pkg.synth.make_input("c2_decode", T=T)
    before = ctx.fallback_counts()[1]
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"router_mm NaN row T={T}")
    ids, _, _, _, logits = ctx.routing()
    assert np.isnan(logits[:, 11]).all() and not (ids == 11).any()
    assert ctx.fallback_counts()[1] - before == T
