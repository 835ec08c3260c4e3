"""GPU parity: the HIP path through the C ABI against the CPU oracle on identical seeded inputs.

Bar: router ids and per-expert lists bit-exact; expert intermediates (gate/up/down products) and
outputs compared bit for bit, with the north star's tolerance (relative 2e-3, absolute 1e-4 near
zero) as the hard limit.
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

RTOL, ATOL = 2e-3, 1e-4


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


_LAYERS = {}


def layer(pkg, name, **kw):
    key = (name, tuple(sorted(kw.items())))
    if key not in _LAYERS:
        _LAYERS[key] = pkg.synth.make_layer(name, **kw)
    return _LAYERS[key]


def within(gpu, ref):
    """Tolerance check; a NaN matches only a NaN (a NaN logit selected by the scan makes every weight
    and output of its token NaN)."""
    gpu, ref = gpu.astype(np.float64), ref.astype(np.float64)
    both_nan = np.isnan(gpu) & np.isnan(ref)
    err = np.where(both_nan, 0.0, np.abs(gpu - ref))
    ok = both_nan | (err <= np.maximum(RTOL * np.abs(ref), ATOL))
    return bool(ok.all()), float(np.max(np.where(np.isnan(err), np.inf, err), initial=0.0))


def check_layer(ctx, orc, L, x, shared=None, tag="", exact=False, layer=0):
    """Run one layer on the GPU and compare every stage with the oracle.

    layer: the uploaded slot that holds L.  exact=True forces the router that replays the reference's
    float sums: then logits, weights and outputs are compared bit for bit too.  Otherwise (the decode path's certified router for T <= 16)
    ids and lists are bit-exact, logits agree within the router's error bound and weights/outputs
    within the tolerance; gate/up/down products are bit-exact on both paths."""
    T = x.shape[0]
    out = ctx.ffn(layer, x, shared, exact_router=exact, keep_intermediates=True)
    ids, w, off, perm, logits = ctx.routing()
    g, u, yd = ctx.intermediates()
    k = L["n_used"]
    bad_ids = 0
    exact_out = 0
    worst = 0.0
    for t in range(T):
        sh = None if shared is None else shared[t]
        if shared is None and L.get("n_ff_shared", 0) > 0:
            sh = orc.shared_ffn(L, x[t])
        rout, rids, rw, rg, ru, ryd = orc.moe_token(L, x[t], sh)
        rlog, _, _ = orc.router(L, x[t])
        if not np.array_equal(ids[t], rids):
            bad_ids += 1
            continue
        if exact:
            # NaN logits (a NaN router weight) compare equal to NaN
            np.testing.assert_array_equal(logits[t], rlog, err_msg=f"{tag} t={t}: router logits differ")
            np.testing.assert_array_equal(w[t], rw, err_msg=f"{tag} t={t} weights")
        else:
            fin = np.isfinite(rlog)
            np.testing.assert_array_equal(logits[t][~fin], rlog[~fin], err_msg=f"{tag} t={t}: nonfinite logits")
            err = np.abs(logits[t][fin].astype(np.float64) - rlog[fin])
            assert err.max(initial=0.0) <= 1e-5, f"{tag} t={t}: logits beyond bound"
            np.testing.assert_allclose(w[t], rw, rtol=1e-4, atol=1e-7, err_msg=f"{tag} t={t} weights")
        np.testing.assert_array_equal(g[t * k:(t + 1) * k], rg, err_msg=f"{tag} t={t} gate")
        np.testing.assert_array_equal(u[t * k:(t + 1) * k], ru, err_msg=f"{tag} t={t} up")
        np.testing.assert_array_equal(yd[t * k:(t + 1) * k], ryd, err_msg=f"{tag} t={t} down")
        ok, emax = within(out[t], rout)
        assert ok, f"{tag} t={t}: output beyond tolerance, max abs err {emax}"
        worst = max(worst, emax)
        same = bool(np.array_equal(out[t], rout, equal_nan=True))
        exact_out += int(same)
        if exact:
            assert same, f"{tag} t={t}: exact-router output not bit-exact (max abs err {emax})"
    assert bad_ids == 0, f"{tag}: {bad_ids} tokens routed differently"
    roff, rperm = orc.bucket(ids, L["n_expert"])
    np.testing.assert_array_equal(off, roff, err_msg=f"{tag} offsets")
    np.testing.assert_array_equal(perm, rperm, err_msg=f"{tag} lists")
    say(f"{tag}: T={T} ids/lists bit-exact, outputs bit-exact {exact_out}/{T} tokens, max abs err {worst:.3g}")
    return out


def test_selftest_arith(ctx, orc):
    say("selftest arith")
    rng = np.random.default_rng(7)
    a = (rng.standard_normal(1 << 16) * np.exp(rng.uniform(-20, 20, 1 << 16))).astype(np.float32)
    b = (rng.standard_normal(1 << 16) * np.exp(rng.uniform(-20, 20, 1 << 16))).astype(np.float32)
    # IEEE binary32 division
    np.testing.assert_array_equal(ctx.selftest(0, a, b), a / b)
    # (float)((double)a / (double)b)
    np.testing.assert_array_equal(ctx.selftest(2, a, b), (a.astype(np.float64) / b.astype(np.float64)).astype(np.float32))
    # rms scale 1f / (float)sqrt((double)(mean + eps)) for mean >= 0
    mean = np.abs(a)
    eps = np.full_like(a, 1e-6)
    ref = np.float32(1.0) / np.sqrt((mean + eps).astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(ctx.selftest(1, mean, eps), ref)
    # roundf: half away from zero; exact halves included
    r = np.concatenate([a[:1000] % 300, np.arange(-300, 300, dtype=np.float32) + 0.5]).astype(np.float32)
    rr = np.where(r >= 0, np.floor(r.astype(np.float64) + 0.5), np.ceil(r.astype(np.float64) - 0.5)).astype(np.float32)
    np.testing.assert_array_equal(ctx.selftest(3, r), rr)
    # fp16 bits (round to nearest even) against the oracle's Half.FromFloat
    np.testing.assert_array_equal(ctx.selftest(4, a).astype(np.uint32), orc.half_from_float(a).astype(np.uint32))
    # and its edge cases: NaNs of both signs and any payload, infinities, signed zeros, overflow and
    # the 65520 boundary, ties to even among normals and subnormals, the 2^-25 underflow boundary
    edge = np.array([0.0, -0.0, np.inf, -np.inf, 65504.0, 65519.996, 65520.0, -65520.0, 1e30,
                     1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 2.0 ** -14, 2.0 ** -14 * (1 - 2.0 ** -11),
                     2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -25, 2.0 ** -25 * (1 + 2.0 ** -20), 2.0 ** -26,
                     -2.0 ** -25, 3 * 2.0 ** -25, 5 * 2.0 ** -25, 2.0 ** -30], dtype=np.float32)
    nans = np.array([0x7FC00000, 0xFFC00000, 0x7F800001, 0xFF812345, 0x7FFFFFFF], dtype=np.uint32).view(np.float32)
    edge = np.concatenate([edge, nans])
    np.testing.assert_array_equal(ctx.selftest(4, edge).astype(np.uint32), orc.half_from_float(edge).astype(np.uint32))
    # nearest_int (1.5*2^23) on |x| < 2^22
    z = (rng.uniform(-4e6, 4e6, 4096)).astype(np.float32)
    z = np.concatenate([z, np.arange(-200, 200, dtype=np.float32) + 0.5])
    np.testing.assert_array_equal(ctx.selftest(5, z).astype(np.int64), np.array([orc.nearest_int(v) for v in z]))
    # GELU on every fp16 value and on random floats
    hv = orc.half_to_float(np.arange(65536, dtype=np.uint16))
    fin = np.isfinite(hv)
    np.testing.assert_array_equal(ctx.selftest(6, hv[fin]), orc.gelu(hv[fin]))
    gx = (rng.standard_normal(1 << 16) * 4).astype(np.float32)
    np.testing.assert_array_equal(ctx.selftest(6, gx), orc.gelu(gx))
    # fp16 -> float, all 65,536 patterns (NaN payloads compared as bits)
    h = np.arange(65536, dtype=np.float32)
    got = ctx.selftest(7, h)
    np.testing.assert_array_equal(got.view(np.uint32)[fin], hv[fin].view(np.uint32))


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("rule", [0, 1])
def test_c1_tiny(ctx, pkg, orc, rule, exact):
    say(f"c1_tiny rule={rule} exact={exact}")
    L = layer(pkg, "c1_tiny", weight_rule=rule)
    x = pkg.synth.make_input("c1_tiny")
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"c1 rule={rule} exact={exact}", exact=exact)


def test_c1_norms_and_shared_input(ctx, pkg, orc):
    say("c1_tiny noisy norms, shared input given")
    L = pkg.synth.make_layer("c1_tiny", norms="noisy")
    x = pkg.synth.make_input("c1_tiny")
    shared = pkg.synth.normal(1001, "shared", x.shape)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, shared, tag="c1 noisy+shared")


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("T", [1, 4, 8, 16])
def test_c2_decode(ctx, pkg, orc, T, exact):
    say(f"c2_decode T={T} exact={exact}")
    L = layer(pkg, "c2_decode")
    x = pkg.synth.make_input("c2_decode", T=T)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"c2 T={T} exact={exact}", exact=exact)


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("T", [1, 8])
def test_c2_decode_cpuref_weights(ctx, pkg, orc, T, exact):
    """The reference CPU's own weight rule (sel[0] replaced by 1 before the later terms read it,
    src/GemmaCpu.cs:406-407) on the decode path, certified and exact."""
    say(f"c2_decode CPUREF weights T={T} exact={exact}")
    L = layer(pkg, "c2_decode", weight_rule=1)
    x = pkg.synth.make_input("c2_decode", T=T)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"c2 cpuref T={T} exact={exact}", exact=exact)


@pytest.mark.parametrize("cfg,T", [("c3_prefill", 256), ("c4_kquant", 64), ("c5_stack", 32)])
def test_general_path_cpuref_weights(ctx, pkg, orc, cfg, T):
    """The CPUREF weight rule on the general path: the matrix-core products at C3, the K-quant
    products at C4, the certified many-token router at C5."""
    say(f"{cfg} CPUREF weights T={T}")
    L = layer(pkg, cfg, weight_rule=1)
    x = pkg.synth.make_input(cfg, T=T)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"{cfg} cpuref T={T}")


def test_router_tie_forces_fallback(ctx, pkg, orc):
    """Two experts with identical router rows tie exactly: the certified order cannot separate
    them, the exact fallback must pick the lower index first (src/GemmaCpu.cs:400-405)."""
    say("router tie: duplicate router rows in c1")
    L = dict(layer(pkg, "c1_tiny"))
    W = L["gate_inp"].copy()
    x = pkg.synth.make_input("c1_tiny")
    # experts 2 and 5: identical rows pointing along the tokens' mean, so both rank first for most tokens
    xbar = x.mean(0)
    W[2] = (0.5 * xbar / np.linalg.norm(xbar)).astype(np.float32)
    W[5] = W[2]
    L["gate_inp"] = W
    logits = np.stack([orc.router(L, xt)[0] for xt in x])
    assert (logits[:, 2] == logits[:, 5]).all()
    before = ctx.fallback_counts()[1]
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag="c1 tie")
    ids = ctx.routing()[0]
    both = [(t, list(r)) for t, r in enumerate(ids) if 2 in r and 5 in r]
    assert all(r.index(2) < r.index(5) for _, r in both)
    after = ctx.fallback_counts()[1]
    say(f"tokens with both tied experts: {len(both)}; router fallbacks {after - before}")
    assert len(both) >= x.shape[0] // 2, "the planted tie should reach the top-k of most tokens"
    assert after - before >= len(both)


@pytest.mark.parametrize("T", [1, 8])
def test_router_ties_decode(ctx, pkg, orc, T):
    """The exact fallback at the decode path's full width (d=2816, 128 experts): three planted pairs of
    identical router rows along the tokens' mean reach most tokens' top-k, so most tokens are ranked by
    the reference's float chains (ties to the lower index); one token alone and eight in one call."""
    say(f"router ties: duplicate router rows in c2 T={T}")
    L = dict(layer(pkg, "c2_decode"))
    W = L["gate_inp"].copy()
    x = pkg.synth.make_input("c2_decode", T=T)
    xbar = x.mean(0)
    for a, b, scale in [(3, 90, 0.9), (17, 40, 0.7), (64, 65, 0.5)]:
        W[a] = (scale * xbar / np.linalg.norm(xbar)).astype(np.float32)
        W[b] = W[a]
    L["gate_inp"] = W
    before = ctx.fallback_counts()[1]
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"c2 T={T} ties")
    ids = ctx.routing()[0]
    for a, b, _ in [(3, 90, 0), (17, 40, 0), (64, 65, 0)]:
        both = [list(r) for r in ids if a in r and b in r]
        assert all(r.index(a) < r.index(b) for r in both)
    fb = ctx.fallback_counts()[1] - before
    say(f"router fallbacks {fb}")
    assert fb >= (T + 1) // 2, "the planted ties should send most tokens to the exact fallback"


@pytest.mark.parametrize("T,exact", [(8, False), (8, True), (1, False)])
def test_router_nan_row_decode(ctx, pkg, orc, T, exact):
    """A NaN router weight makes one expert's logit NaN for every token: no order is certified, every
    expert of every token goes to the exact chains (two groups of 64 in the fallback), and NaN ranks
    below every number (the strict '>' scan of src/GemmaCpu.cs:400-405)."""
    say(f"router NaN row in c2 T={T} exact={exact}")
    L = dict(layer(pkg, "c2_decode"))
    W = L["gate_inp"].copy()
    W[11, 5] = np.nan
    L["gate_inp"] = W
    x = pkg.synth.make_input("c2_decode", T=T)
    before = ctx.fallback_counts()[1]
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"c2 T={T} NaN row exact={exact}", exact=exact)
    ids, _, _, _, logits = ctx.routing()
    assert np.isnan(logits[:, 11]).all() and not (ids == 11).any()
    if not exact:
        assert ctx.fallback_counts()[1] - before == T


# NaN router rows that the reference's scan does select (src/GemmaCpu.cs:400-405): a round starts at the
# lowest untaken expert and keeps it when its logit is NaN, so a NaN expert is taken as soon as every
# lower-index expert is.  (NaN expert, experts boosted to the top so that happens early.)
NAN_PICKS = {"nan0": (0, ()), "nan1_after0": (1, (0,)), "nan3_after012": (3, (0, 1, 2))}


@pytest.mark.parametrize("T,exact", [(1, False), (1, True), (8, False), (8, True), (40, False)])
@pytest.mark.parametrize("case", list(NAN_PICKS))
def test_router_nan_taken_by_scan(ctx, pkg, orc, case, T, exact):
    """Decode T=1 and T=8 (certified with the exact fallback, and the exact router), and the general
    path at T=40: ids, lists and logits match the oracle's scan; tokens that select the NaN expert have
    all-NaN weights and outputs, as the reference computes them."""
    nan_e, boost = NAN_PICKS[case]
    say(f"router NaN pick {case} T={T} exact={exact}")
    L = dict(layer(pkg, "c2_decode"))
    W = L["gate_inp"].copy()
    x = pkg.synth.make_input("c2_decode", T=T)
    xbar = x.mean(0)
    for j, e in enumerate(boost):
        W[e] = ((0.9 - 0.1 * j) * xbar / np.linalg.norm(xbar)).astype(np.float32)
    W[nan_e, 5] = np.nan
    L["gate_inp"] = W
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"NaN {case} T={T} exact={exact}", exact=exact)
    ids, w, _, _, logits = ctx.routing()
    assert np.isnan(logits[:, nan_e]).all()
    picked = (ids == nan_e).any(1)
    if not boost:
        assert (ids[:, 0] == nan_e).all()
    else:
        # the boosted experts rank first for most tokens, and then the NaN expert comes next
        top = [set(r[:len(boost)]) == set(boost) for r in ids]
        assert sum(top) >= T // 2
        assert all(r[len(boost)] == nan_e for r, tp in zip(ids, top) if tp)
    assert np.isnan(w[picked]).all()
    say(f"tokens taking the NaN expert: {int(picked.sum())}/{T}")


def test_router_nan_row0_c1(ctx, pkg, orc):
    """configs[0] with NaN in router row 0: every token takes expert 0 first (the reference's scan),
    then its best expert."""
    say("router NaN row 0 in c1")
    L = dict(layer(pkg, "c1_tiny"))
    W = L["gate_inp"].copy()
    W[0, 0] = np.nan
    L["gate_inp"] = W
    x = pkg.synth.make_input("c1_tiny")
    for exact in (False, True):
        ctx.upload(0, L)
        check_layer(ctx, orc, L, x, tag=f"c1 NaN row 0 exact={exact}", exact=exact)
        ids = ctx.routing()[0]
        assert (ids[:, 0] == 0).all()


def test_c3_prefill_reduced(ctx, pkg, orc):
    say("c3_prefill T=48 (zipf router)")
    L = pkg.synth.make_layer("c3_prefill")
    x = pkg.synth.make_input("c3_prefill", T=48)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag="c3 T=48")


def test_c3_prefill_wide_router(ctx, pkg, orc):
    """T = 1030 (past the size where the exact router switches to its many-token kernel, and not a
    multiple of its four-token workgroups): router logits bit-exact for every token through the exact
    router, ids and expert lists bit-exact, and the layer output of 40 sampled tokens bit-exact."""
    T = 1030
    say(f"c3_prefill T={T} (zipf router, exact)")
    L = pkg.synth.make_layer("c3_prefill")
    x = pkg.synth.make_input("c3_prefill", T=T)
    ctx.upload(0, L)
    out = ctx.ffn(0, x, exact_router=True)
    ids, w, off, perm, logits = ctx.routing()
    k = L["n_used"]
    for t in range(T):
        rlog, rids, rw = orc.router(L, x[t])
        np.testing.assert_array_equal(logits[t], rlog, err_msg=f"t={t} logits")
        np.testing.assert_array_equal(ids[t], rids, err_msg=f"t={t} ids")
    roff, rperm = orc.bucket(ids, L["n_expert"])
    np.testing.assert_array_equal(off, roff)
    np.testing.assert_array_equal(perm, rperm)
    rng = np.random.default_rng(5)
    sample = sorted(set([0, 1, T - 2, T - 1] + rng.choice(T, 36, replace=False).tolist()))
    for t in sample:
        rout = orc.moe_token(L, x[t], orc.shared_ffn(L, x[t]) if L.get("n_ff_shared", 0) > 0 else None)[0]
        np.testing.assert_array_equal(out[t], rout, err_msg=f"t={t} output")
    say(f"c3 T={T}: logits, ids, lists bit-exact; {len(sample)} sampled outputs bit-exact")


def test_c4_kquant_reduced(ctx, pkg, orc):
    say("c4_kquant T=12")
    L = pkg.synth.make_layer("c4_kquant")
    x = pkg.synth.make_input("c4_kquant", T=12)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag="c4 T=12")


def test_kquant_full_tiles(ctx, pkg, orc):
    """About 32 assignments per expert: the K-quant grouped kernel's full tiles (Q4_K gate|up, Q6_K
    down with its rows padded to whole super-blocks), bit-exact through the exact router."""
    say("k-quant T=64, E=4, k=2: full tiles")
    cfg = dict(idx=15, T=64, d=512, E=4, k=2, nf=384, gu=12, dn=14)
    L = pkg.synth.make_layer(cfg, norms="noisy")
    x = pkg.synth.make_input(cfg, T=64)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag="kquant full tiles", exact=True)


@pytest.mark.parametrize("exact", [False, True])
def test_c5_stack_graph(ctx, pkg, orc, exact):
    say(f"c5 stack: 3 layers, T=8, HIP graph replayed 3 times, exact={exact}")
    cfg = dict(pkg.synth.CONFIGS["c5_stack"])
    layers = [layer(pkg, "c5_stack", layer=i) for i in range(3)]
    for i, L in enumerate(layers):
        ctx.upload(i, L)
    x0 = pkg.synth.make_input(cfg, T=8)
    # oracle: x += rmsnorm(moe_block(x)) * post_ffw_norm, layer after layer
    ref = x0.copy()
    for L in layers:
        out, _, _ = orc.moe_block(L, ref)
        ref = orc.residual(L, ref, out)
    ctx.stack_capture(0, 3, 8, exact_router=exact)
    for rep in range(3):
        got = ctx.stack_run(x0)
        ok, emax = within(got, ref)
        assert ok, f"replay {rep}: max abs err {emax}"
        if exact:
            assert np.array_equal(got, ref), f"replay {rep}: exact stack not bit-exact"
        say(f"replay {rep}: bit-exact {int((got == ref).sum())}/{got.size}")
        # eager work between replays
        eager = ctx.ffn(1, x0)
        assert np.isfinite(eager).all()


@pytest.mark.parametrize("T", [1, 3, 8])
def test_decode_stack_folds_combines(ctx, pkg, orc, T):
    """A decode stack folds each layer's combine into the next layer's router while T * E <= 512
    (every router workgroup forms its token's x from the previous layer's outputs, the expert-0 one
    writes it; T = 8 keeps the standalone combines): the replayed graph equals the same layers called
    one by one with the residual, bit for bit, with the shared FFN in every layer (C2 layers), and
    stays within tolerance of the oracle."""
    n = 4
    say(f"c2 decode stack: {n} layers, T={T}, folded combines vs layer-by-layer calls")
    layers = [layer(pkg, "c2_decode", layer=i) for i in range(n)]
    for i, L in enumerate(layers):
        ctx.upload(i, L)
    x0 = pkg.synth.make_input("c2_decode", T=T)
    seq = x0.copy()
    for i in range(n):
        _, seq = ctx.ffn(i, seq, residual=True)
    ref = x0.copy()
    for L in layers:
        out, _, _ = orc.moe_block(L, ref)
        ref = orc.residual(L, ref, out)
    ctx.stack_capture(0, n, T)
    for rep in range(2):
        got = ctx.stack_run(x0)
        np.testing.assert_array_equal(got, seq, err_msg=f"replay {rep}: folded stack differs from the layer calls")
        ok, emax = within(got, ref)
        assert ok, f"replay {rep}: max abs err {emax}"
    say(f"stack == layer calls bit for bit; max abs err vs oracle {within(got, ref)[1]:.3g}")


def test_stack_profiled_replays(ctx, pkg, orc):
    """A stack captured while profiling carries timing nodes around its kernels: its replays still give
    the oracle's results, the router, gate|up and down kinds report one timed launch per layer and
    replay and the combine one per replay (the earlier layers' combines are folded into the next
    layer's router), and later calls run cleanly."""
    say("c5 stack: 2 layers, T=4, captured while profiling, replayed 3 times")
    cfg = dict(pkg.synth.CONFIGS["c5_stack"])
    layers = [layer(pkg, "c5_stack", layer=i) for i in range(2)]
    for i, L in enumerate(layers):
        ctx.upload(i, L)
    x0 = pkg.synth.make_input(cfg, T=4)
    ref = x0.copy()
    for L in layers:
        out, _, _ = orc.moe_block(L, ref)
        ref = orc.residual(L, ref, out)
    ctx.profile(True)
    ctx.stack_capture(0, 2, 4)
    for rep in range(3):
        got = ctx.stack_run(x0)
        ok, emax = within(got, ref)
        assert ok, f"replay {rep}: max abs err {emax}"
    prof = ctx.profile_read()
    ctx.profile(False)
    say({k: v for k, v in prof.items() if v[1]})
    for kind, launches in (("router", 6), ("gate_up", 6), ("down", 6), ("combine", 3)):
        ms, n = prof[kind]
        assert n == launches and ms > 0, (kind, ms, n)
    ctx.stack_capture(0, 2, 4)  # a plain capture again
    assert within(ctx.stack_run(x0), ref)[0]
    assert np.isfinite(ctx.ffn(1, x0)).all()


@pytest.mark.parametrize("exact", [False, True])
def test_nonfinite_inputs_route_safely(ctx, pkg, orc, exact):
    """A token with a NaN or an Inf activation has all-NaN router logits; the reference's strict '>'
    scan then takes experts 0..k-1 in order.  The GPU must do the same, never fault, and keep the
    other tokens exact (regression: NaN comparisons once stalled the parallel argmax)."""
    say(f"non-finite inputs exact={exact}")
    L = layer(pkg, "c2_decode")
    x = pkg.synth.make_input("c2_decode", T=4).copy()
    x[1, 5] = np.nan
    x[2, 7] = np.inf
    ctx.upload(0, L)
    out = ctx.ffn(0, x, exact_router=exact)
    ids, w, off, perm, logits = ctx.routing()
    k, E = L["n_used"], L["n_expert"]
    for t in range(4):
        _, rids, _ = orc.router(L, x[t])
        np.testing.assert_array_equal(ids[t], rids, err_msg=f"t={t}")
        assert len(set(ids[t].tolist())) == k and ids[t].min() >= 0 and ids[t].max() < E
    np.testing.assert_array_equal(ids[1], np.arange(k))
    roff, rperm = orc.bucket(ids, E)
    np.testing.assert_array_equal(off, roff)
    np.testing.assert_array_equal(perm, rperm)
    for t in (0, 3):
        rout, _, _, _, _, _ = orc.moe_token(L, x[t], orc.shared_ffn(L, x[t]))
        ok, emax = within(out[t], rout)
        assert ok, f"t={t}: {emax}"


# ---------------------------------------------------------------------------------------- fixtures
def _golden():
    from pathlib import Path
    gold = Path(__file__).resolve().parent / "golden"
    if str(gold) not in sys.path:
        sys.path.insert(0, str(gold))
    import make_golden
    return gold, make_golden


@pytest.mark.parametrize("exact", [False, True])
@pytest.mark.parametrize("rule", [0, 1])
def test_golden_c1_fixture(ctx, pkg, rule, exact):
    """configs[0] at full size against tests/golden/c1_tiny.npz (noisy norms, shared input given)."""
    say(f"golden c1 rule={rule} exact={exact}")
    gold, MG = _golden()
    f = np.load(gold / "c1_tiny.npz")
    L, x, shared = MG.c1_inputs(pkg.synth)
    assert MG.layer_digest(L) == str(f["layer_sha256"]), "synthetic generator drifted from the fixture"
    L["weight_rule"] = rule
    ctx.upload(0, L)
    out = ctx.ffn(0, f["x"], f["shared"], exact_router=exact)
    ids, w, off, perm, logits = ctx.routing()
    np.testing.assert_array_equal(ids, f[f"ids_r{rule}"])
    np.testing.assert_array_equal(off, f["offsets"])
    np.testing.assert_array_equal(perm, f["perm"])
    ok, emax = within(out, f[f"out_r{rule}"])
    assert ok, f"max abs err {emax}"
    if exact:
        np.testing.assert_array_equal(logits, f["logits"])
        np.testing.assert_array_equal(w, f[f"w_r{rule}"])
        np.testing.assert_array_equal(out, f[f"out_r{rule}"])
    say(f"golden c1: bit-exact {int((out == f[f'out_r{rule}']).sum())}/{out.size}, max abs err {emax:.3g}")


def test_golden_kquant_fixture(ctx, pkg):
    """Q4_K gate|up and a padded Q6_K down (288 -> 512) against tests/golden/kquant_tiny.npz."""
    say("golden kquant T=4")
    gold, MG = _golden()
    f = np.load(gold / "kquant_tiny.npz")
    L, x = MG.kq_inputs(pkg.synth)
    assert MG.layer_digest(L) == str(f["layer_sha256"])
    ctx.upload(0, L)
    out = ctx.ffn(0, f["x"], exact_router=True)
    ids = ctx.routing()[0]
    np.testing.assert_array_equal(ids, f["ids"])
    np.testing.assert_array_equal(out, f["out"])


# ---------------------------------------------------------------------------------------- matrix cores
MFMA_CASES = {
    # (layer config, T, shared input given): n = T * k >= 8 * E puts the experts on the MFMA kernel,
    # T >= 32 the shared FFN
    "c1_T64_q4_0": ("c1_tiny", 64, True),
    "q8_0_shared_T64": (dict(idx=12, T=64, d=512, E=8, k=2, nf=256, gu=8, dn=8, nff=256, sh=8), 64, False),
    "c2_T64_shared_only": ("c2_decode", 64, False),
    "c3_T128": ("c3_prefill", 128, False),
    # about 128 assignments per expert: full and partial 128-token tiles; 9 paired row groups (an odd
    # count leaves a workgroup with a spare wave pair), 608 down rows, odd block counts (19 and 9)
    "q4_0_T256_full_tiles": (dict(idx=13, T=256, d=608, E=4, k=2, nf=288, gu=2, dn=2), 256, False),
    "q8_0_T256_full_tiles": (dict(idx=14, T=256, d=512, E=4, k=2, nf=256, gu=8, dn=8), 256, False),
}


@pytest.mark.parametrize("case", list(MFMA_CASES))
def test_mfma_grouped_products_bit_exact(ctx, pkg, orc, case):
    """The MFMA grouped kernel keeps the reference's per-block float chain: gate/up/down rows and the
    outputs equal the CPU reference bit for bit (the general path's router is the exact one)."""
    cfg, T, with_shared = MFMA_CASES[case]
    say(f"mfma {case}: T={T}")
    L = pkg.synth.make_layer(cfg, norms="noisy")
    x = pkg.synth.make_input(cfg, T=T)
    shared = pkg.synth.normal(1234, "mfma.shared", x.shape) if with_shared else None
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, shared, tag=f"mfma {case}", exact=True)


# K-quants on the matrix cores: n = T * k >= 8 * E; tiles of up to 32 assignments (one or two 16-wide
# column tiles), Q4_K with its min term, Q6_K's split scales, either type on either product
KMMA_CASES = {
    "q4k_gu_q6k_dn_T96": (dict(idx=51, T=96, d=1024, E=8, k=2, nf=512, gu=12, dn=14), 96),
    "q6k_gu_q4k_dn_T64": (dict(idx=52, T=64, d=768, E=4, k=2, nf=256, gu=14, dn=12), 64),
    # nine paired row groups (a spare wave quartet) and down rows padded 288 -> 512
    "q4k_q6k_odd_rows_T80": (dict(idx=53, T=80, d=1280, E=4, k=2, nf=288, gu=12, dn=14), 80),
    "q4k_both_T40": (dict(idx=54, T=40, d=512, E=4, k=4, nf=512, gu=12, dn=12), 40),
}


@pytest.mark.parametrize("case", list(KMMA_CASES))
def test_kmma_grouped_products_bit_exact(ctx, pkg, orc, case):
    """The K-quant MFMA kernel keeps DotK's lane chains: gate/up/down rows and the outputs equal the CPU
    reference bit for bit (exact router)."""
    cfg, T = KMMA_CASES[case]
    say(f"kmma {case}: T={T}")
    L = pkg.synth.make_layer(cfg, norms="noisy")
    x = pkg.synth.make_input(cfg, T=T)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"kmma {case}", exact=True)


# Q5_K (the VALU row walk at any T: five-bit values with the min term) and Q3_K (held on the device as
# the Q6_K blocks of the same values, so the Q6_K kernels run it, on the matrix cores from 8 assignments
# per expert); either type on either product, a shared FFN in Q5_K, padded down rows
Q35_CASES = {
    "q5k_gu_q3k_dn_T8": (dict(idx=61, T=8, d=512, E=8, k=2, nf=512, gu=13, dn=11), 8),
    "q3k_gu_q5k_dn_T12_shared": (dict(idx=62, T=12, d=768, E=8, k=2, nf=512, gu=11, dn=13, nff=512, sh=13), 12),
    "q5k_both_T64_full_tiles": (dict(idx=63, T=64, d=512, E=4, k=2, nf=512, gu=13, dn=13), 64),
    "q3k_both_T96_kmma": (dict(idx=64, T=96, d=1024, E=8, k=2, nf=384, gu=11, dn=11), 96),
}


@pytest.mark.parametrize("case", list(Q35_CASES))
def test_q3k_q5k_layers_bit_exact(ctx, pkg, orc, case):
    """Q3_K and Q5_K experts (src/CpuRefKQuants.cs:92-147 through DotK :177-212): gate, up and down
    products and outputs equal the oracle bit for bit (exact router)."""
    cfg, T = Q35_CASES[case]
    say(f"q3k/q5k {case}: T={T}")
    L = pkg.synth.make_layer(cfg, norms="noisy")
    x = pkg.synth.make_input(cfg, T=T)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"q3k/q5k {case}", exact=True)


# ---------------------------------------------------------------------------------------- IQ formats
IQ_CASES = {
    # gate|up, down (and the shared FFN) in the IQ formats (CpuRefIQuants.cs); n_ff 384 pads the down rows
    # to 512 (zero activations in the tail), 512 does not
    "iq2xxs_gu_iq2s_dn": (dict(idx=41, T=12, d=512, E=8, k=2, nf=384, gu=16, dn=22), 12),
    "iq3s_both_shared": (dict(idx=42, T=12, d=768, E=8, k=2, nf=512, gu=21, dn=21, nff=512, sh=21), 12),
    "iq2s_gu_iq2xxs_dn_full_tiles": (dict(idx=43, T=64, d=512, E=4, k=2, nf=512, gu=22, dn=16), 64),
}


@pytest.mark.parametrize("case", list(IQ_CASES))
def test_iq_layers_bit_exact(ctx, pkg, orc, case):
    """IQ2_XXS / IQ2_S / IQ3_S experts on the VALU grouped kernel, codebooks in LDS: gate, up and down
    products and outputs equal the oracle's DotIQ chains bit for bit (exact router)."""
    cfg, T = IQ_CASES[case]
    say(f"iq {case}: T={T}")
    L = pkg.synth.make_layer(cfg, norms="noisy")
    x = pkg.synth.make_input(cfg, T=T)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"iq {case}", exact=True)


def test_host_buffer_calls_replay_graphs(ctx, pkg, orc):
    """phx_moe_ffn on host buffers replays one captured graph per (layer, T, flags, shared given): repeated
    calls equal the device-pointer call bit for bit (decode-sized calls end on the completion word, large
    ones on a stream wait); a layer uploaded again, another T, the residual and a given shared branch each
    take their own graph and the oracle's results."""
    S = pkg.synth
    La = layer(pkg, "c1_tiny")
    Lb = layer(pkg, "c1_tiny", norms="noisy")
    ctx.upload(0, La)
    d = La["d"]
    for T in (1, 3, 64, 1):
        x = S.make_input("c1_tiny", T=T)
        say(f"host graphs: T={T}")
        outs = [ctx.ffn(0, x) for _ in range(3)]
        xb, ob = ctx.alloc(x.nbytes), ctx.alloc(x.nbytes)
        xb.upload(x)
        ctx.ffn_device(0, T, xb.ptr, None, ob.ptr)
        ctx.sync()
        dev = ob.download((T, d))
        xb.free()
        ob.free()
        for o in outs:
            np.testing.assert_array_equal(o, dev)
        assert within(outs[0], orc.moe_block(La, x)[0])[0]
    # the same slot uploaded with other weights: a fresh capture
    x = S.make_input("c1_tiny", T=3)
    before = ctx.ffn(0, x)
    ctx.upload(0, Lb)
    after = ctx.ffn(0, x)
    assert within(after, orc.moe_block(Lb, x)[0])[0] and not np.array_equal(before, after)
    # residual (x updated in place through the pinned rows) and a given shared branch
    Lc = layer(pkg, "c5_stack", norms="noisy")
    ctx.upload(1, Lc)
    x = S.make_input("c5_stack", T=2)
    ro = orc.moe_block(Lc, x)[0]
    for _ in range(2):
        out, xn = ctx.ffn(1, x, residual=True)
        assert within(out, ro)[0]
        assert within(xn, orc.residual(Lc, x, ro))[0]
    sh = S.normal(99, "host.shared", (3, d))
    xs = S.make_input("c1_tiny", T=3)
    ctx.upload(0, La)
    o1 = ctx.ffn(0, xs, sh)
    o2 = ctx.ffn(0, xs, sh)
    np.testing.assert_array_equal(o1, o2)
    assert within(o1, orc.moe_block(La, xs, sh)[0])[0]
