"""BASELINE.json's configurations at their full sizes on the GPU against the CPU oracle.

configs[2] (C3): prefill, T = 2048 with Zipf(1.1) routing, on the matrix-core path; configs[3] (C4):
K-quants at T = 512 with the Q6_K down padded 1408 -> 1536; configs[4] (C5): the 30-layer batched
decode stack at T = 32 with one hot expert, captured as one HIP graph.  T > 16 runs the general path;
under PHX_FLAG_EXACT_ROUTER its router replays the reference's float chains, so logits, ids, lists,
weights and outputs are all compared bit for bit.  Without the flag the routers are the certified ones
(C3 and C4: the matrix-core sums with bounds; a C5 layer: the workgroup-per-pair sums): ids, lists and
the expert products bit-exact, logits within 1e-5, weights and outputs within the tolerance.
"""
import sys
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _check_layer_exact(ctx, orc, L, x, tag):
    """Both routers on the same layer and input against one oracle pass: the exact router bit for bit in
    every stage; the default (certified) router with bit-exact ids, lists and products."""
    T = x.shape[0]
    k = L["n_used"]
    t0 = time.time()
    out = ctx.ffn(0, x, exact_router=True, keep_intermediates=True)
    ids, w, off, perm, logits = ctx.routing()
    g, u, yd = ctx.intermediates()
    fb0 = ctx.fallback_counts()[1]
    cout = ctx.ffn(0, x, keep_intermediates=True)
    cids, cw, coff, cperm, clog = ctx.routing()
    cg, cu, cyd = ctx.intermediates()
    fb = ctx.fallback_counts()[1] - fb0
    say(f"{tag}: GPU done ({time.time() - t0:.1f} s); oracle on {T} tokens ...")
    t0 = time.time()
    worst = 0.0
    for t in range(T):
        rout, rids, rw, rg, ru, ryd = orc.moe_token(L, x[t], None)
        rlog = orc.router(L, x[t])[0]
        np.testing.assert_array_equal(ids[t], rids, err_msg=f"{tag} t={t} ids")
        np.testing.assert_array_equal(logits[t], rlog, err_msg=f"{tag} t={t} logits")
        np.testing.assert_array_equal(w[t], rw, err_msg=f"{tag} t={t} weights")
        np.testing.assert_array_equal(g[t * k:(t + 1) * k], rg, err_msg=f"{tag} t={t} gate")
        np.testing.assert_array_equal(u[t * k:(t + 1) * k], ru, err_msg=f"{tag} t={t} up")
        np.testing.assert_array_equal(yd[t * k:(t + 1) * k], ryd, err_msg=f"{tag} t={t} down")
        np.testing.assert_array_equal(out[t], rout, err_msg=f"{tag} t={t} output")
        # the certified router: the same ids (so the same products), logits and weights within bounds
        np.testing.assert_array_equal(cids[t], rids, err_msg=f"{tag} certified t={t} ids")
        assert np.abs(clog[t].astype(np.float64) - rlog).max() <= 1e-5, f"{tag} certified t={t} logits"
        np.testing.assert_allclose(cw[t], rw, rtol=1e-4, atol=1e-7, err_msg=f"{tag} certified t={t} weights")
        np.testing.assert_array_equal(cg[t * k:(t + 1) * k], rg, err_msg=f"{tag} certified t={t} gate")
        np.testing.assert_array_equal(cyd[t * k:(t + 1) * k], ryd, err_msg=f"{tag} certified t={t} down")
        err = np.abs(cout[t].astype(np.float64) - rout)
        assert np.all(err <= np.maximum(2e-3 * np.abs(rout), 1e-4)), f"{tag} certified t={t} output"
        worst = max(worst, float(err.max()))
        if t % 256 == 255:
            say(f"  {t + 1} tokens checked ({time.time() - t0:.1f} s)")
    roff, rperm = orc.bucket(ids, L["n_expert"])
    for o, pm, m in ((off, perm, "exact"), (coff, cperm, "certified")):
        np.testing.assert_array_equal(o, roff, err_msg=f"{tag} {m} offsets")
        np.testing.assert_array_equal(pm, rperm, err_msg=f"{tag} {m} lists")
    say(f"{tag}: certified router: {fb} of {T} tokens through the exact chains, outputs max abs err {worst:.3g}")
    return ids


def test_c3_prefill_full(ctx, pkg, orc):
    """configs[2] at T = 2048: 16,384 assignments on the MFMA grouped kernels, uneven experts (some
    empty, the hottest above 400 assignments, as the committed Zipf histogram fixture records)."""
    say("c3_prefill T=2048: generating ...")
    L = pkg.synth.make_layer("c3_prefill")
    x = pkg.synth.make_input("c3_prefill")
    assert x.shape[0] == 2048
    ctx.upload(0, L)
    ids = _check_layer_exact(ctx, orc, L, x, "c3 T=2048")
    cnt = np.bincount(ids.ravel(), minlength=L["n_expert"])
    say(f"c3 T=2048: exact router bit-exact in every stage; experts per count: max {cnt.max()}, "
        f"empty {(cnt == 0).sum()}")
    assert cnt.max() > 400


def test_c4_kquant_full(ctx, pkg, orc):
    """configs[3] at T = 512: Q4_K gate|up, Q6_K down over rows padded 1408 -> 1536, E = 64, top-4."""
    say("c4_kquant T=512: generating ...")
    L = pkg.synth.make_layer("c4_kquant")
    assert L["down_cols"] == 1536 and L["n_ff"] == 1408
    x = pkg.synth.make_input("c4_kquant")
    assert x.shape[0] == 512
    ctx.upload(0, L)
    _check_layer_exact(ctx, orc, L, x, "c4 T=512")
    say("c4 T=512: exact router bit-exact in every stage")


def test_c5_stack_30_layers(ctx, pkg, orc):
    """30 Q8_0 layers with RMSNorm and residual, T = 32, one hot expert taking about 40% of
    the tokens entering the stack, captured as one HIP graph and replayed twice.  Three distinct seeded
    layers fill the 30 slots in turn (generating 30 distinct 0.8 GB layers would take minutes); the
    oracle applies the same sequence layer by layer, and the replayed stack's result equals it bit for
    bit."""
    cfg = pkg.synth.CONFIGS["c5_stack"]
    n, T = cfg["layers"], cfg["T"]
    assert (n, T) == (30, 32)
    x0 = pkg.synth.make_input("c5_stack")
    ref = x0.copy()
    hot = []
    distinct = []
    for j in range(3):
        say(f"c5: generating distinct layer {j} ...")
        distinct.append(pkg.synth.make_layer("c5_stack", layer=j))
    t0 = time.time()
    for i in range(n):
        L = distinct[i % 3]
        ctx.upload(i, L)
        out, ids, _ = orc.moe_block(L, ref)
        ref = orc.residual(L, ref, out)
        hot.append(np.bincount(ids.ravel(), minlength=L["n_expert"]).max() / T)
    say(f"c5: 30 slots uploaded, oracle stack done ({time.time() - t0:.1f} s); "
        f"hot expert share per layer {min(hot):.2f}..{max(hot):.2f}")
    # the bias channel x[t][d-1] carries the hot expert into layer 0; every residual add then moves it,
    # so later layers see the bias only partly
    assert hot[0] > 0.3
    ctx.stack_capture(0, n, T, exact_router=True)
    for rep in range(2):
        got = ctx.stack_run(x0)
        np.testing.assert_array_equal(got, ref, err_msg=f"replay {rep}: 30-layer stack differs from the oracle")
        say(f"c5 replay {rep}: 30 layers bit-exact")
    # the default routing (certified router): each distinct layer on the oracle's own input for it
    from test_gpu_parity import check_layer
    xin = x0.copy()
    for i in range(3):
        L = distinct[i]
        check_layer(ctx, orc, L, xin, tag=f"c5 certified layer {i}", layer=i)
        out, _, _ = orc.moe_block(L, xin)
        xin = orc.residual(L, xin, out)
    del distinct
