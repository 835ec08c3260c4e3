"""Known answers that pin the oracle's single-step roundings, where an error bound cannot tell two
readings of the reference apart:

- the router input m_i = ((x_i * rinv) * sc) * s_i, with rinv = 1f / (float)sqrt((float)(ss / d) + eps)
  (src/GemmaCpu.cs:387-389);
- RMSNorm's mean (float)(sum / n) and its product x * scale * w, left to right (src/CpuRef.cs:184-191);
- the combine, rank by rank from j = 0 (src/GemmaCpu.cs:410, 417-418);
- the combine weight (float)(p / sum) * down_scale: the cast comes before the multiply (:417);
- Q8_0's reciprocal id = 1f / d with d = amax / 127f, not 127 / amax (src/CpuRef.cs:56-60).

Each case is built so that the reference's reading gives bits fixed in closed form (a power of two, an
exact product, or one rounding of an exact value), and each test also checks that the plausible
misreadings give other bits at the same inputs, so the known answer discriminates.  C# evaluates
float expressions left to right in IEEE single precision and Math.Sqrt in double; numpy's float32 and
float64 operations are the same correctly rounded IEEE operations, used here only to show that the
misreadings land elsewhere.  CPU only."""
import numpy as np
import pytest

F32 = np.float32
D = 2816  # the configs' hidden size: 1 / sqrt(2816) is not a power of two


def f(v):
    return F32(v)


def _sqrt_f(v64):
    """(float)Math.Sqrt(v) for a double v."""
    return F32(np.sqrt(np.float64(v64)))


SC = f(1) / _sqrt_f(D)  # the router's 1f / (float)Math.Sqrt(d)


def _router_layer(pkg, E=16, k=2):
    L = pkg.synth.make_layer(dict(idx=9, T=1, d=D, E=E, k=k, nf=128, gu=2, dn=2), experts=False)
    L["gate_inp"] = np.zeros((E, D), F32)
    L["gate_inp_scale"] = np.ones(D, F32)
    L["eps"] = 0.0
    return L


# ---------------------------------------------------------------------------------------- RMSNorm
def _row_mean_above_boundary():
    """x = 2 + 5 * 2^-22 then seven 2s: the sum of squares is 32 + 5 * 2^-20 + 25 * 2^-44 exactly, so
    mean = 4 + 5 * 2^-23 + 25 * 2^-47.  (float)mean = 4 + 2^-21 (the nearest float: ulp(4) = 2^-21), whose
    square root 2 + 2^-23 - 2^-48 lies below the midpoint 2 + 2^-23 between the floats 2 and 2 + 2^-22 and
    rounds to 2: scale = 1f / 2 = 0.5.  The double mean's root, 2 + 2^-23 + 2^-25 - ..., lies above that
    midpoint and rounds to 2 + 2^-22, whose reciprocal rounds to 0.5 - 2^-24."""
    x = np.full(8, 2.0, F32)
    x[0] = 2 + 5 * 2.0 ** -22
    return x


def test_rms_scale_rounds_the_mean_to_float(orc):
    x = _row_mean_above_boundary()
    mean64 = sum(float(v) * float(v) for v in x) / x.size
    assert mean64 == 4 + 5 * 2.0 ** -23 + 25 * 2.0 ** -47
    assert f(mean64) == f(4 + 2.0 ** -21)
    assert orc.rms_scale(x, 0.0) == f(0.5)
    # the mean kept in double lands one float lower
    assert f(1) / _sqrt_f(mean64) == f(0.5 - 2.0 ** -24)
    w = np.ones(x.size, F32)
    assert np.array_equal(orc.rmsnorm(x, w, 0.0), x * f(0.5))


def test_rmsnorm_multiplies_x_by_scale_then_by_w(orc, pkg):
    """|x| = 3 everywhere, eps = 0: mean = 9 exactly, scale = 1f / 3f = (1 + 2^-25) / 3.  Then x * scale
    = +-(1 + 2^-25), which rounds to +-1 (below half an ulp of 1), so y = x * scale * w = +-w exactly, for
    any w.  Multiplying scale * w first (or x * w first) rounds a non-power-of-two product and lands
    elsewhere for many w."""
    n = 512
    x = np.full(n, 3.0, F32)
    x[1::3] = -3.0
    w = pkg.synth.normal(31, "w", (n,), 1.0, 0.1)
    scale = orc.rms_scale(x, 0.0)
    assert scale == f(1) / f(3)
    y = orc.rmsnorm(x, w, 0.0)
    assert np.array_equal(y, np.sign(x) * w)
    for name, alt in (("x * (scale * w)", x * (scale * w)), ("(x * w) * scale", (x * w) * scale)):
        assert np.count_nonzero(alt != y) > n // 8, f"{name} agrees with the known answer: nothing pinned"


# ---------------------------------------------------------------------------------------- router input
def test_router_rounds_the_mean_to_float(orc, pkg):
    """x = 2 except x_0 = 2 + 1760 * 2^-22 over d = 2816: ss = 11264 + 1760 * 2^-20 + 1760^2 * 2^-44 exactly,
    and ss / d = 4 + 5 * 2^-23 + 1100 * 2^-44 (rounded once in double).  As in the RMSNorm case, the float
    mean 4 + 2^-21 gives rinv = 0.5, so x_1 * rinv = 1 and a probe expert whose row is the unit vector e_1
    (s_1 = 1) has logit ((2 * 0.5) * sc) * 1 = sc exactly.  The double mean gives rinv = 0.5 - 2^-24 and
    the logit (1 - 2^-23) * sc, a different float."""
    L = _router_layer(pkg)
    L["gate_inp"][3, 1] = 1.0
    x = np.full(D, 2.0, F32)
    x[0] = 2 + 1760 * 2.0 ** -22
    ss = sum(float(v) * float(v) for v in x)
    assert ss == 11264 + 1760 * 2.0 ** -20 + 1760 ** 2 * 2.0 ** -44
    assert f(ss / D) == f(4 + 2.0 ** -21)
    logits, _, _ = orc.router(L, x)
    assert logits[3] == SC
    rinv_double_mean = f(1) / _sqrt_f(ss / D)
    assert rinv_double_mean == f(0.5 - 2.0 ** -24)
    assert (f(2) * rinv_double_mean) * SC != SC


# Eight values a / 16 whose squares sum to 8 * 9 exactly (56^2 + 76^2 + ... + 68^2 = 18432 = 8 * 9 * 256),
# with a router scale each; among them every misreading below changes at least two probes.
GROUP = [56, 76, 9, 31, 43, 18, 41, 68]
GROUP_S = [1.0, 1.1, 0.9, 1.25, 0.75, 1.2, 0.8, 1.05]


def test_router_input_is_x_times_rinv_times_sc_times_s(orc, pkg):
    """x = 3 except eight probe positions holding a / 16 with the same sum of squares, so ss = 9 * d
    exactly, the mean is 9 and rinv = 1f / 3f.  Probe expert e's row is the unit vector at probe position
    p_e, so its logit is m_p = ((x_p * rinv) * sc) * s_p itself (every other product is zero).  The
    groupings x * (rinv * sc) * s, x * rinv * (sc * s), (x * sc) * rinv * s, x * ((rinv * sc) * s) and
    (x * s) * rinv * sc each differ from it at two or more probes."""
    assert sum(a * a for a in GROUP) == 8 * 9 * 256
    L = _router_layer(pkg, E=len(GROUP) + 2)
    x = np.full(D, 3.0, F32)
    pos = [100 + 37 * i for i in range(len(GROUP))]
    for e, (p, a, s) in enumerate(zip(pos, GROUP, GROUP_S)):
        x[p] = a / 16
        L["gate_inp_scale"][p] = s
        L["gate_inp"][e, p] = 1.0
    assert sum(float(v) * float(v) for v in x) == 9.0 * D
    logits, _, _ = orc.router(L, x)
    r = f(1) / f(3)
    xs, ss = x[pos], L["gate_inp_scale"][pos]
    want = ((xs * r) * SC) * ss
    assert np.array_equal(logits[:len(GROUP)], want)
    alts = {
        "x * (rinv * sc) * s": (xs * (r * SC)) * ss,
        "x * rinv * (sc * s)": (xs * r) * (SC * ss),
        "(x * sc) * rinv * s": ((xs * SC) * r) * ss,
        "x * ((rinv * sc) * s)": xs * ((r * SC) * ss),
        "(x * s) * rinv * sc": ((xs * ss) * r) * SC,
    }
    for name, alt in alts.items():
        assert np.count_nonzero(alt != want) >= 2, f"{name} agrees with the known answer: nothing pinned"


# ---------------------------------------------------------------------------------------- weights, combine
def test_weight_is_cast_before_the_down_scale(orc, pkg):
    """Three experts with identical router rows tie for the top three: p_j = exp(0) = 1, sum = 3, and
    (float)(1.0 / 3.0) = (1 + 2^-25) / 3.  With down_scale 3 + 2^-21 the float product is
    (1 + 2^-25)(1 + 2^-21 / 3) = 1 + 1.583 ulp(1), which rounds to 1 + 2^-22.  Casting after the multiply
    rounds (1 / 3)(3 + 2^-21) = 1 + 1.333 ulp(1) once, to 1 + 2^-23."""
    L = _router_layer(pkg, E=8, k=3)
    x = pkg.synth.normal(32, "x", (D,))
    for e in range(3):
        L["gate_inp"][e] = x * 0.01
    L["gate_inp"][3:] = -x * 0.01
    ds = f(3 + 2.0 ** -21)
    assert float(ds) == 3 + 2.0 ** -21
    L["down_scale"] = np.full(8, ds, F32)
    logits, ids, w = orc.router(L, x)
    assert list(ids) == [0, 1, 2] and logits[0] == logits[1] == logits[2]
    assert np.all(w == f(1 + 2.0 ** -22))
    assert f((1.0 / 3.0) * float(ds)) == f(1 + 2.0 ** -23)


def test_combine_adds_ranks_in_order(orc):
    """Rank 0 puts 1000 on element 0 (weight 1) and ranks 1..7 put 600 * 2^-24 each (2400 * 2^-24 times
    the weight 2^-2, an exact product), each between half an ulp and an ulp of 1000
    (ulp(1000) = 2^-14 = 1024 * 2^-24).  Added rank by rank from j = 0, every small term rounds the sum
    up by one ulp: 1000 + 7 * 2^-14.  Any other order first adds small terms to each other."""
    k, d = 8, 4
    small = 600 * 2.0 ** -24
    yd = np.zeros((k, d), F32)
    w = np.zeros(k, F32)
    yd[0, 0], w[0] = 1000.0, 1.0
    for j in range(1, k):
        yd[j, 0], w[j] = small * 4, 0.25  # 2400 * 2^-24 * 2^-2: exact
    yd[:, 1] = 1.5  # a plain column: 1.5 * sum of weights
    acc = orc.combine(yd, w)
    ulp = float(np.spacing(F32(1000.0)))
    assert ulp / 2 < small < ulp
    assert acc[0] == f(1000.0 + 7 * ulp)
    assert acc[1] == f(1.5 + 7 * 0.375) and acc[2] == 0 and acc[3] == 0
    rev = F32(0)
    for j in reversed(range(k)):
        rev = F32(rev + yd[j, 0] * w[j])
    assert rev != acc[0]


def test_layer_output_is_the_rank_order_combine(orc, pkg):
    """The whole token (GemmaCpu.cs:376-422) equals its pinned parts composed: out = rmsnorm(shared) *
    post1 + rmsnorm(combine(yd, w)) * post2, bit for bit, on noisy norms and down scales; the combine
    summed from the last rank gives other bits."""
    L = pkg.synth.make_layer(dict(idx=9, T=1, d=256, E=8, k=4, nf=128, gu=2, dn=2), norms="noisy")
    x = pkg.synth.normal(33, "x", (3, 256))
    sh = pkg.synth.normal(34, "sh", (3, 256))
    differs = 0
    for t in range(3):
        out, ids, w, _, _, yd = orc.moe_token(L, x[t], sh[t])
        _, rids, rw = orc.router(L, x[t])
        assert np.array_equal(ids, rids) and np.array_equal(w, rw)
        acc = orc.combine(yd, w)
        want = orc.rmsnorm(sh[t], L["post_ffw_norm_1"], L["eps"]) + \
            orc.rmsnorm(acc, L["post_ffw_norm_2"], L["eps"])
        assert np.array_equal(out, want)
        rev = orc.combine(yd[::-1].copy(), w[::-1].copy())
        differs += np.count_nonzero(rev != acc)
    assert differs > 0


# ---------------------------------------------------------------------------------------- Q8_0
def test_q8_0_quantizes_with_the_reciprocal_of_d(orc):
    """amax = 1 + 2^-11: d = amax / 127f, id = 1f / d.  The element x (float bits 0x3d113468) has
    x * id = 4.5 exactly in float, which rounds half away from zero to 5.  With id = 127f / amax the
    product is 4.4999995 and rounds to 4."""
    amax = f(1 + 2.0 ** -11)
    xv = np.array([1024537704], np.uint32).view(F32)[0]
    d = amax / f(127)
    idv = f(1) / d
    assert xv * idv == f(4.5)
    assert xv * (f(127) / amax) == f(4.5 - 2.0 ** -21)
    blk = np.zeros(32, F32)
    blk[0], blk[5] = amax, xv
    _, q = orc.quantize_q8_0(blk)
    assert q[0] == 127 and q[5] == 5
