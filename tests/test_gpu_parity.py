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
    err = np.abs(gpu.astype(np.float64) - ref.astype(np.float64))
    return bool((err <= np.maximum(RTOL * np.abs(ref), ATOL)).all()), float(err.max())


def check_layer(ctx, orc, L, x, shared=None, tag=""):
    T = x.shape[0]
    out = ctx.ffn(0, x, shared)
    ids, w, off, perm, logits = ctx.routing()
    g, u, yd = ctx.intermediates()
    k, nf, d = L["n_used"], L["n_ff"], L["d"]
    bad_ids = 0
    exact_out = 0
    for t in range(T):
        sh = None if shared is None else shared[t]
        if shared is None and L.get("n_ff_shared", 0) > 0:
            sh = orc.shared_ffn(L, x[t])
        rout, rids, rw, rg, ru, ryd = orc.moe_token(L, x[t], sh)
        rlog, _, _ = orc.router(L, x[t])
        assert np.array_equal(logits[t], rlog), f"{tag} t={t}: router logits differ"
        if not np.array_equal(ids[t], rids):
            bad_ids += 1
            continue
        np.testing.assert_array_equal(w[t], rw, err_msg=f"{tag} t={t} weights")
        np.testing.assert_array_equal(g[t * k:(t + 1) * k], rg, err_msg=f"{tag} t={t} gate")
        np.testing.assert_array_equal(u[t * k:(t + 1) * k], ru, err_msg=f"{tag} t={t} up")
        np.testing.assert_array_equal(yd[t * k:(t + 1) * k], ryd, err_msg=f"{tag} t={t} down")
        ok, emax = within(out[t], rout)
        assert ok, f"{tag} t={t}: output beyond tolerance, max abs err {emax}"
        exact_out += int(np.array_equal(out[t], rout))
    assert bad_ids == 0, f"{tag}: {bad_ids} tokens routed differently"
    roff, rperm = orc.bucket(ids, L["n_expert"])
    np.testing.assert_array_equal(off, roff, err_msg=f"{tag} offsets")
    np.testing.assert_array_equal(perm, rperm, err_msg=f"{tag} lists")
    say(f"{tag}: T={T} ids/lists bit-exact, outputs bit-exact {exact_out}/{T} tokens")
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


@pytest.mark.parametrize("rule", [0, 1])
def test_c1_tiny(ctx, pkg, orc, rule):
    say(f"c1_tiny rule={rule}")
    L = pkg.synth.make_layer("c1_tiny", weight_rule=rule)
    x = pkg.synth.make_input("c1_tiny")
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"c1 rule={rule}")


def test_c1_norms_and_shared_input(ctx, pkg, orc):
    say("c1_tiny noisy norms, shared input given")
    L = pkg.synth.make_layer("c1_tiny", norms="noisy")
    x = pkg.synth.make_input("c1_tiny")
    shared = pkg.synth.normal(1001, "shared", x.shape)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, shared, tag="c1 noisy+shared")


@pytest.mark.parametrize("T", [1, 4, 8])
def test_c2_decode(ctx, pkg, orc, T):
    say(f"c2_decode T={T}")
    L = layer(pkg, "c2_decode")
    x = pkg.synth.make_input("c2_decode", T=T)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag=f"c2 T={T}")


def test_c3_prefill_reduced(ctx, pkg, orc):
    say("c3_prefill T=48 (zipf router)")
    L = pkg.synth.make_layer("c3_prefill")
    x = pkg.synth.make_input("c3_prefill", T=48)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag="c3 T=48")


def test_c4_kquant_reduced(ctx, pkg, orc):
    say("c4_kquant T=12")
    L = pkg.synth.make_layer("c4_kquant")
    x = pkg.synth.make_input("c4_kquant", T=12)
    ctx.upload(0, L)
    check_layer(ctx, orc, L, x, tag="c4 T=12")


def test_c5_stack_graph(ctx, pkg, orc):
    say("c5 stack: 3 layers, T=8, HIP graph replayed 3 times")
    cfg = dict(pkg.synth.CONFIGS["c5_stack"])
    layers = [pkg.synth.make_layer(cfg, layer=i) for i in range(3)]
    for i, L in enumerate(layers):
        ctx.upload(i, L)
    x0 = pkg.synth.make_input(cfg, T=8)
    # oracle: x += rmsnorm(moe_block(x)) * post_ffw_norm, layer after layer
    ref = x0.copy()
    for L in layers:
        out, _, _ = orc.moe_block(L, ref)
        ref = orc.residual(L, ref, out)
    ctx.stack_capture(0, 3, 8)
    for rep in range(3):
        got = ctx.stack_run(x0)
        ok, emax = within(got, ref)
        assert ok, f"replay {rep}: max abs err {emax}"
        say(f"replay {rep}: bit-exact {int((got == ref).sum())}/{got.size}")
        # eager work between replays
        eager = ctx.ffn(1, x0)
        assert np.isfinite(eager).all()
