"""Pins of the oracle's layer functions (oracle/oracle.c: orc_router, orc_bucket, orc_moe_token,
orc_shared_ffn_token, orc_residual) against brute force on small expert counts, the invariants of
top-k routing (distinct ids, descending logits, ties to the lower index, weights summing to one),
the closed form of the reference's in-place weight quirk (GemmaCpu.cs:406-407), a stable sort for
the expert lists (KernelsMoe.cs:281-330), and the float64 textbook layer of tests/textbook.py.
CPU only."""
import numpy as np
import pytest

import textbook as TB


def _cfg(**kw):
    base = dict(idx=9, T=4, d=256, E=8, k=2, nf=128, gu=2, dn=2)
    base.update(kw)
    return base


@pytest.fixture(scope="module")
def synth(pkg):
    return pkg.synth


# ---------------------------------------------------------------------------------------- router
@pytest.mark.parametrize("norms", ["unit", "noisy"])
def test_router_brute_force(orc, synth, norms):
    L = synth.make_layer(_cfg(E=8, k=3), norms=norms)
    x = synth.normal(77, "x", (24, L["d"]))
    for t in range(x.shape[0]):
        logits, ids, w = orc.router(L, x[t])
        want = TB.router_logits(L, x[t])
        inp = x[t].astype(np.float64) / np.sqrt(np.mean(x[t].astype(np.float64) ** 2)) / 16.0
        bound = 4 * L["d"] * 2.0 ** -24 * (np.abs(L["gate_inp"]) @ np.abs(inp * L["gate_inp_scale"])) + 1e-12
        assert np.all(np.abs(logits - want) <= bound)
        # top-k by brute force over the oracle's own logits: descending, ties to the lower index
        assert list(ids) == list(TB.topk(logits, 3))
        sel = logits[ids].astype(np.float64)
        wr = w / L["down_scale"][ids]
        assert np.allclose(wr, TB.weights_softmax(sel), rtol=3e-7, atol=0)
        assert abs(wr.sum() - 1) < 1e-6


def test_router_ties_pick_lower_index(orc, synth):
    L = synth.make_layer(_cfg(E=8, k=2))
    W = L["gate_inp"]
    W[5] = W[3]
    W[6] = W[3]
    x = synth.normal(78, "x", (1, L["d"]))[0]
    # make expert 3's row the best one: align it with x
    W[3] = W[5] = W[6] = x * 0.05
    logits, ids, w = orc.router(L, x)
    assert logits[3] == logits[5] == logits[6]
    assert list(ids) == [3, 5]
    assert w[0] == w[1]
    # all rows equal: the first k experts, equal weights
    L["gate_inp"][:] = W[0]
    logits, ids, w = orc.router(L, x)
    assert list(ids) == [0, 1] and w[0] == w[1] == np.float32(0.5)


def _planted_logits_layer(synth, vals):
    """A layer whose router logits are exactly fl(vals[e] * m_0): W[e] is vals[e] at element 0 and zero
    elsewhere, so every other product is a zero and the reference's chain adds only zeros to it."""
    E = len(vals)
    L = synth.make_layer(_cfg(E=E, k=E))
    W = np.zeros_like(L["gate_inp"])
    W[:, 0] = np.asarray(vals, np.float32)
    L["gate_inp"] = W
    x = np.ones(L["d"], np.float32)  # m_0 = 1/sqrt(d) > 0, so the logits keep the order of vals
    return L, x


# Known answers of the reference's scan (GemmaCpu.cs:400-405) with NaN logits, derived by hand: a round
# starts at the lowest untaken expert and moves only to a strictly greater logit, so it stays on a NaN
# start and never moves to a NaN.
NAN_SCAN_CASES = [
    ([np.nan, 1.0, 2.0], [0, 2, 1]),
    ([1.0, np.nan, 2.0], [2, 0, 1]),
    ([3.0, np.nan, 5.0, 1.0, np.nan, np.nan, 7.0, 2.0], [6, 2, 0, 1, 7, 3, 4, 5]),
    ([np.nan] * 4, [0, 1, 2, 3]),
    ([2.0, 2.0, np.nan, -np.inf, np.nan, 2.0], [0, 1, 2, 5, 3, 4]),
    ([-np.inf, np.nan, -np.inf, 4.0], [3, 0, 1, 2]),
]


@pytest.mark.parametrize("case", range(len(NAN_SCAN_CASES)))
def test_router_nan_scan_known_answers(orc, synth, case):
    vals, want = NAN_SCAN_CASES[case]
    L, x = _planted_logits_layer(synth, vals)
    logits, ids, w = orc.router(L, x)
    assert np.array_equal(np.isnan(logits), np.isnan(np.asarray(vals)))
    assert list(ids) == want


def nan_scan_positions(logits):
    """The positions the decode path's exact fallback assigns in parallel (kernels_decode.hip,
    select_exact): a non-NaN expert at its rank r among the non-NaN ones plus the NaN experts whose P
    lies below r; a NaN expert at P + 1 + the NaN experts below it, P being the largest rank among the
    non-NaN experts below it (-1 if none).  Checked here against the oracle's sequential scan."""
    E = len(logits)
    isn = np.isnan(logits)
    r = np.zeros(E, np.int64)
    for e in range(E):
        if not isn[e]:
            r[e] = sum(1 for c in range(E) if not isn[c] and (logits[c] > logits[e] or (logits[c] == logits[e] and c < e)))
    P = np.full(E, np.iinfo(np.int64).max)
    pos = r.copy()
    for n in range(E):
        if isn[n]:
            P[n] = max([r[c] for c in range(n) if not isn[c]], default=-1)
            pos[n] = P[n] + 1 + int(isn[:n].sum())
    for e in range(E):
        if not isn[e]:
            pos[e] = r[e] + int((P < r[e]).sum())
    order = np.empty(E, np.int64)
    order[pos] = np.arange(E)
    return order


def test_router_nan_parallel_positions_equal_scan(orc, synth):
    rng = np.random.default_rng(11)
    for trial in range(300):
        E = int(rng.integers(2, 20))
        vals = rng.integers(-3, 4, E).astype(np.float64)  # small integers: many exact ties
        vals[rng.random(E) < rng.uniform(0, 0.7)] = np.nan
        if trial % 7 == 0:
            vals[rng.random(E) < 0.2] = -np.inf
        L, x = _planted_logits_layer(synth, vals)
        logits, ids, _ = orc.router(L, x)
        assert list(nan_scan_positions(logits)) == list(ids), (vals, list(ids))
    for c, (vals, want) in enumerate(NAN_SCAN_CASES):
        assert list(nan_scan_positions(np.asarray(vals, np.float32))) == want


def test_router_cpuref_weight_quirk(orc, synth):
    """weight_rule 1 keeps the reference CPU's in-place update: w_0 = 1/S, w_j = exp(l_j - 1)/S."""
    L = synth.make_layer(_cfg(E=8, k=4), weight_rule=1)
    x = synth.normal(79, "x", (8, L["d"]))
    for t in range(8):
        logits, ids, w = orc.router(L, x[t])
        sel = logits[ids].astype(np.float64)
        assert np.allclose(w, TB.weights_cpuref(sel), rtol=3e-7, atol=0)
        L0 = dict(L, weight_rule=0)
        _, ids0, w0 = orc.router(L0, x[t])
        assert list(ids0) == list(ids)
        assert not np.allclose(w0, w)  # the two rules differ whenever the top logit is not 1


# ---------------------------------------------------------------------------------------- lists
def test_bucket_is_stable_counting_sort(orc):
    rng = np.random.default_rng(3)
    for T, k, E in ((1, 8, 128), (37, 4, 16), (300, 8, 128), (64, 2, 8)):
        ids = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
        off, perm = orc.bucket(ids, E)
        flat = ids.reshape(-1)
        assert np.array_equal(off, np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))]))
        assert np.array_equal(perm, np.argsort(flat, kind="stable"))
        assert off[-1] == T * k


def test_bucket_edge_cases(orc):
    off, perm = orc.bucket(np.zeros((0, 4), np.int32), 16)
    assert not off.any() and perm.size == 0
    ids = np.tile(np.array([[7, 0, 3]], np.int32), (5, 1))  # one hot expert set
    off, perm = orc.bucket(ids, 8)
    assert list(off) == [0, 5, 5, 5, 10, 10, 10, 10, 15]
    assert list(perm[:5]) == [1, 4, 7, 10, 13] and list(perm[10:]) == [0, 3, 6, 9, 12]


# ---------------------------------------------------------------------------------------- layer
LAYERS = {
    "q4_0": _cfg(gu=2, dn=2),
    "q8_0_shared": _cfg(gu=8, dn=8, nff=256, sh=8),
    "q4_0_noisy": _cfg(gu=2, dn=8, E=16, k=4),
    "kquant": _cfg(d=512, nf=256, gu=12, dn=14, E=4, k=2),
    "kquant_padded": _cfg(d=512, nf=288, gu=12, dn=14, E=4, k=2),  # Q6_K down rows padded 288 -> 512
}


def _rms(a):
    return float(np.sqrt(np.mean(np.asarray(a, np.float64) ** 2)))


@pytest.mark.parametrize("name", list(LAYERS))
def test_layer_vs_textbook(orc, synth, name):
    cfg = LAYERS[name]
    L = synth.make_layer(cfg, norms="noisy" if "noisy" in name else "unit")
    x = synth.make_input(cfg, T=3)
    shared = None
    if L["n_ff_shared"]:
        shared = np.stack([orc.shared_ffn(L, x[t]) for t in range(3)])
        for t in range(3):
            sw = TB.shared_ffn(L, x[t])
            assert np.abs(shared[t] - sw).max() <= 2e-5 * _rms(sw)
    for t in range(3):
        out, ids, w, g, u, yd = orc.moe_token(L, x[t], None if shared is None else shared[t], nthreads=2)
        logits = TB.router_logits(L, x[t])
        top = TB.topk(logits, L["n_used"])
        margin = np.sort(logits)[::-1]
        if margin[L["n_used"] - 1] - margin[L["n_used"]] > 1e-5:
            assert list(ids) == list(top)
        tout, _, tw, tg, tu, tyd = TB.moe_token(L, x[t], None if shared is None else shared[t], ids=ids)
        assert np.allclose(w, tw, rtol=2e-6, atol=0)
        # gate/up: exact float64 dots of the same quantized activations, up to fp32 summation and the
        # rare 1-ulp differences of the fp32 vs float64 RMSNorm feeding the quantizer
        for a, b in ((g, tg), (u, tu)):
            assert np.abs(a - b).max() <= 1e-5 * _rms(b)
        for j in range(L["n_used"]):
            assert np.abs(yd[j] - tyd[j]).max() <= 2e-5 * _rms(tyd[j])
        assert np.abs(out - tout).max() <= 2e-5 * _rms(tout), np.abs(out - tout).max() / _rms(tout)


def test_layer_zero_shared_and_residual(orc, synth):
    cfg = LAYERS["q4_0"]
    L = synth.make_layer(cfg, norms="noisy")
    x = synth.make_input(cfg, T=2)
    out0, *_ = orc.moe_token(L, x[0], np.zeros(L["d"], np.float32))
    out1, *_ = orc.moe_token(L, x[0], None)
    assert np.array_equal(out0, out1)  # rmsnorm(0) is exactly 0 (GemmaCpu.cs:384 with _xb = 0)
    out, ids, w = orc.moe_block(L, x)
    xr = orc.residual(L, x, out)
    want = x.astype(np.float64) + np.stack([TB.rmsnorm(out[t], L["post_ffw_norm"], L["eps"]) for t in range(2)])
    assert np.all(np.abs(xr - want) <= 4 * 2.0 ** -24 * (np.abs(want) + np.abs(x)))


def test_layer_rows_independent_of_threads_and_batch(orc, synth):
    cfg = LAYERS["q8_0_shared"]
    L = synth.make_layer(cfg)
    x = synth.make_input(cfg, T=4)
    a, ia, wa = orc.moe_block(L, x, nthreads=1)
    b, ib, wb = orc.moe_block(L, x, nthreads=3)
    assert np.array_equal(a, b) and np.array_equal(ia, ib) and np.array_equal(wa, wb)
    c, ic, wc = orc.moe_block(L, x[2:3], nthreads=2)
    assert np.array_equal(a[2], c[0]) and np.array_equal(ia[2], ic[0])
