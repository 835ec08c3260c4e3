"""Pins of the oracle's element and row functions (oracle/oracle.c) against what the mathematics and
the file formats fix: numpy's IEEE fp16 conversion, closed forms of the two activation quantizers
(with the reference test's planted tie, nvidia/tests/KernelTests.cs:181), an independent decoder of
the GGUF block layouts (tests/gguf_spec.py), exact float64 dot products, and the textbook GELU and
RMSNorm.  CPU only."""
import numpy as np
import pytest

import gguf_spec as G
import textbook as TB

TYPES = [2, 8, 11, 12, 13, 14]


# ---------------------------------------------------------------------------------------- fp16
def test_half_to_float_exhaustive(orc):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    got = orc.half_to_float(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_half_round_trip_exhaustive(orc):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    f = orc.half_to_float(h)
    back = orc.half_from_float(f)
    ok = ~np.isnan(f)
    assert np.array_equal(back[ok], h[ok])
    assert np.all((back[~ok] & 0x7C00) == 0x7C00) and np.all((back[~ok] & 0x3FF) != 0)


def _float_patterns(rng):
    """float32 bit patterns over every exponent from below the fp16 subnormal range to above its
    overflow: random mantissas, and for every rounding position the exact halfway point +-1 ulp."""
    pats = []
    for sign in (0, 1):
        for e in range(90, 146):
            base = np.uint32((sign << 31) | (e << 23))
            pats.append(base | rng.integers(0, 1 << 23, 40000, dtype=np.uint32))
            for s in range(13, 24):
                hi = rng.integers(0, 1 << 23, 600, dtype=np.uint32) & ~np.uint32((1 << s) - 1)
                half = np.uint32(1 << (s - 1))
                for delta in (-1, 0, 1):
                    pats.append(base | ((hi | half) + np.uint32(delta & 0xFFFFFFFF)) & np.uint32(0x7FFFFF))
    pats.append(np.array([0x7F800000, 0xFF800000, 0x7FC00000, 0x7F800001, 0, 0x80000000,
                          0x477FEFFF, 0x477FF000, 0x477FF001, 0x33000000, 0x33000001, 0x387FE000],
                         np.uint32))
    return np.concatenate(pats)


def test_half_from_float_rne_vs_numpy(orc):
    rng = np.random.default_rng(11)
    f = _float_patterns(rng).view(np.float32)
    got = orc.half_from_float(f)
    with np.errstate(over="ignore"):
        want = f.astype(np.float16).view(np.uint16)
    nan = np.isnan(f)
    assert np.array_equal(got[~nan], want[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all((got[nan] & 0x3FF) != 0)


# ---------------------------------------------------------------------------------------- Q8_0
def test_q8_0_closed_form_random(orc):
    rng = np.random.default_rng(12)
    for scale in (1e-6, 0.02, 1.0, 300.0):
        x = (rng.standard_normal(32 * 257) * scale).astype(np.float32)
        d, q = orc.quantize_q8_0(x)
        dd, qq = TB.q8_0(x)
        assert np.array_equal(orc.half_to_float(d), dd)
        assert np.array_equal(q.astype(np.int32), qq)


def test_q8_0_known_answers(orc):
    # amax 127 -> d = 1 exactly, id = 1: the q values are x rounded half away from zero
    x = np.zeros(64, np.float32)
    x[:8] = [127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.49999988, 126.5]
    d, q = orc.quantize_q8_0(x)
    assert orc.half_to_float(d)[0] == 1.0
    assert list(q[:8]) == [127, 3, -3, 1, -1, 2, -1, 127]
    # an all-zero block: d = 0, id = 0, q = 0 (CpuRef.cs:60-61)
    assert d[1] == 0 and not q[32:].any()


def test_q8_0_reference_test_shape(orc):
    """KernelTests.Quant (KernelTests.cs:151-173): 4096 values in [-4, 4); every scale and value must
    agree with the closed form (the reference tolerated GPU mismatches from floor(|t|+0.5))."""
    rng = np.random.default_rng(5)
    x = rng.uniform(-4, 4, 4096).astype(np.float32)
    d, q = orc.quantize_q8_0(x)
    dd, qq = TB.q8_0(x)
    assert np.array_equal(orc.half_to_float(d), dd) and np.array_equal(q.astype(np.int32), qq)


# ---------------------------------------------------------------------------------------- Q8_K
def test_nearest_int_is_round_half_even(orc):
    # the 1.5*2^23 trick holds for |f| < 2^22 (the quantizer only feeds it |f| <= 127.x)
    rng = np.random.default_rng(13)
    v = np.concatenate([rng.uniform(-4e6, 4e6, 20000), rng.integers(-1000, 1000, 2000) + 0.5,
                        [0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 0.49999997, -0.49999997, 4194302.5, -4194302.5]]).astype(np.float32)
    got = np.array([orc.nearest_int(f) for f in v])
    assert np.array_equal(got, np.rint(v).astype(np.int64))


def test_q8_k_closed_form_random(orc):
    rng = np.random.default_rng(14)
    for scale in (1e-5, 1.0, 50.0):
        x = (rng.standard_normal(256 * 9) * scale).astype(np.float32)
        d, q, bs = orc.quantize_q8_k(x)
        dd, qq, bb = TB.q8_k(x)
        assert np.array_equal(d, dd)
        assert np.array_equal(q.astype(np.int32), qq)
        assert np.array_equal(bs.astype(np.int32), bb)


def test_q8_k_planted_tie_first_index(orc):
    """KernelTests.QuantK (KernelTests.cs:176-181): x[300] = 5, x[301] = -5 in [-3, 3) noise; the
    first index sets the sign, so iscale = -127/5, q[300] = -127, q[301] = +127, d < 0."""
    rng = np.random.default_rng(6)
    x = rng.uniform(-3, 3, 4096).astype(np.float32)
    x[300], x[301] = 5.0, -5.0
    d, q, bs = orc.quantize_q8_k(x)
    assert q[300] == -127 and q[301] == 127
    assert d[1] == np.float32(1) / (np.float32(-127) / np.float32(5))
    assert d[1] < 0
    dd, qq, bb = TB.q8_k(x)
    assert np.array_equal(d, dd) and np.array_equal(q.astype(np.int32), qq) and np.array_equal(bs.astype(np.int32), bb)


def test_q8_k_zero_block(orc):
    x = np.zeros(512, np.float32)
    x[256:] = 1.0
    d, q, bs = orc.quantize_q8_k(x)
    assert d[0] == 0 and not q[:256].any() and not bs[:16].any()
    assert d[1] == np.float32(1) / np.float32(-127) and np.all(q[256:] == -127) and np.all(bs[16:] == -127 * 16)


# ---------------------------------------------------------------------------------------- layouts
@pytest.mark.parametrize("t", TYPES)
def test_dequantize_matches_independent_decoder(orc, t):
    rng = np.random.default_rng(20 + t)
    elems, size = G.BLOCK[t]
    cols = 1024 if elems == 256 else 256
    for _ in range(8):
        row = G.random_blocks(rng, t, cols // elems)
        got = orc.dequantize_row(t, row, cols)
        want = G.DEQUANT[t](row, cols)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert orc.row_bytes(t, cols) == cols // elems * size


# ---------------------------------------------------------------------------------------- dots
def _dot_bound(t, w64, xa):
    nb = len(xa) // G.BLOCK[t][0]
    return (nb + 10) * 2.0 ** -23 * (np.abs(w64) @ np.abs(xa)) + 1e-30


@pytest.mark.parametrize("t", TYPES)
def test_matvec_vs_exact_float64(orc, t):
    rng = np.random.default_rng(30 + t)
    elems, size = G.BLOCK[t]
    cols, rows = (1024, 12) if elems == 256 else (512, 12)
    w = G.random_blocks(rng, t, rows * cols // elems)
    x = rng.standard_normal(cols).astype(np.float32)
    y = orc.matvec(t, w, rows, cols, x, nthreads=2)
    W = TB.weights(t, w, rows, cols)
    xa = TB.act_dequant(t, x)
    want = W @ xa
    bound = np.array([_dot_bound(t, W[r], xa) for r in range(rows)])
    assert np.all(np.abs(y - want) <= bound), np.max(np.abs(y - want) / bound)


def _pow2_scales(blocks, t, exp2=-8):
    """Set every fp16 scale of the blocks to 2^exp2 (so each block term is exact in fp32)."""
    h = np.float16(2.0 ** exp2).view(np.uint16)
    size = G.BLOCK[t][1]
    b = blocks.reshape(-1, size)
    offs = {2: [0], 8: [0], 11: [108], 12: [0, 2], 13: [0, 2], 14: [208]}[t]
    for o in offs:
        b[:, o] = h & 0xFF
        b[:, o + 1] = h >> 8
    return b.reshape(-1)


@pytest.mark.parametrize("t", TYPES)
def test_dot_exact_identity(orc, t):
    """With power-of-two weight and activation scales and integer activations, every partial sum of the
    integer path is exact in fp32, so the oracle must equal sum(dequant(w) * x) exactly (this pins the
    nibble order, the -8/-32 offsets, the scale/min unpacking and the Q4_K min term)."""
    rng = np.random.default_rng(40 + t)
    elems, size = G.BLOCK[t]
    cols = 512
    rows = 16
    w = _pow2_scales(G.random_blocks(rng, t, rows * cols // elems), t)
    if t == 14:  # keep |scale| <= 32 so the 8 lane sums stay below 2^24 units
        b = w.reshape(-1, size)
        b[:, 192:208] = (rng.integers(-32, 33, (b.shape[0], 16))).astype(np.int8).view(np.uint8)
        w = b.reshape(-1)
    x = rng.integers(-10, 11, cols).astype(np.float32)
    x[::elems] = 127.0  # first max of every block: Q8_0 d = 1, Q8_K iscale = -1, d = -1
    y = orc.matvec(t, w, rows, cols, x, nthreads=1)
    W = TB.weights(t, w, rows, cols)
    xa = TB.act_dequant(t, x)
    assert np.array_equal(xa, x.astype(np.float64))  # the activation quantization is lossless here
    units = np.abs(W) @ np.abs(xa) / 2.0 ** -8  # every partial sum is a multiple of 2^-8
    assert np.all(units < 2.0 ** 24)
    assert np.array_equal(y.astype(np.float64), W @ xa)


def test_matvec_f32_double_sum(orc):
    rng = np.random.default_rng(50)
    rows, cols = 9, 777
    W = rng.standard_normal((rows, cols)).astype(np.float32)
    x = rng.standard_normal(cols).astype(np.float32)
    y = orc.matvec(0, W.view(np.uint8).reshape(-1), rows, cols, x)
    want = (W * x).astype(np.float32).astype(np.float64).sum(axis=1)  # float products, double sum
    assert np.array_equal(y, want.astype(np.float32))


# ---------------------------------------------------------------------------------------- GELU
def _ulp_key(v):
    """fp16 values -> integers that step by one per representable fp16 value (-0 and +0 both 0)"""
    b = np.asarray(v, np.float32).astype(np.float16).view(np.uint16).astype(np.int32)
    return np.where(b & 0x8000, -(b & 0x7FFF), b)


def test_gelu_exhaustive_fp16_inputs(orc):
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    x = h[np.isfinite(h)].astype(np.float32)
    got = orc.gelu(x)
    want = TB.gelu(x)
    # outputs are fp16 values (the reference's fp16 table)
    assert np.array_equal(TB.fp16(got), got)
    diff = got != want
    # Away from the negative tail the fp32 evaluation can only straddle an fp16 rounding boundary:
    # at most 1 fp16 ulp, rarely.
    core = x > -2.0
    assert np.all(np.abs(_ulp_key(got[diff & core]) - _ulp_key(want[diff & core])) <= 1)
    assert (diff & core).sum() <= 0.001 * core.sum(), (diff & core).sum()
    # In the tail, 1 + tanh(inner) cancels in fp32 (absolute error ~2^-24, times 0.5 h), which the fp16
    # subnormals resolve: bound |got - want| by that error plus one fp16 ulp.
    h = TB.fp16(x).astype(np.float64)
    ulp16 = np.maximum(np.abs(want.astype(np.float64)) * 2.0 ** -10, 2.0 ** -24)
    assert np.all(np.abs(got.astype(np.float64) - want) <= ulp16 + np.abs(h) * 2.0 ** -23)


def test_gelu_rounds_input_to_fp16_and_cutoffs(orc):
    rng = np.random.default_rng(60)
    x = (rng.standard_normal(20000) * 4).astype(np.float32)
    x = x[np.abs(x) < 9.99]  # the table range; outside it the value is 0 or x itself
    assert np.array_equal(orc.gelu(x), orc.gelu(TB.fp16(x)))
    edge = np.array([-1e30, -10.0, -9.99, 0.0, -0.0, 9.99, 10.0, 10.5, 1e30], np.float32)
    g = orc.gelu(edge)
    assert g[0] == 0 and g[1] == 0 and g[3] == 0 and g[6] == 10.0 and g[7] == 10.5 and g[8] == 1e30
    assert g[5] == TB.gelu(edge[5:6])[0]


# ---------------------------------------------------------------------------------------- SiLU
def test_silu_against_the_logistic_function(orc):
    """silu(x) = x * sigmoid(x) (scipy's expit in float64) to within the three float roundings of the
    reference expression, with the limits fixed exactly: 0 at 0, x where exp(-x) vanishes against 1,
    -0 where exp(-x) overflows float."""
    from scipy.special import expit
    rng = np.random.default_rng(75)
    x = np.concatenate([rng.standard_normal(20000) * 6, rng.uniform(-80, 80, 2000)]).astype(np.float32)
    y = orc.silu(x).astype(np.float64)
    want = x.astype(np.float64) * expit(x.astype(np.float64))
    assert np.all(np.abs(y - want) <= 4 * 2.0 ** -24 * np.abs(want) + 1e-38)
    edge = orc.silu(np.array([0.0, 40.0, 100.0, -100.0, -1.0], np.float32))
    assert edge[0] == 0 and edge[1] == 40.0 and edge[2] == 100.0
    assert edge[3] == 0 and np.signbit(edge[3])
    assert edge[4] == np.float32(-1.0) / (np.float32(1.0) + np.float32(np.e))


# ---------------------------------------------------------------------------------------- RMSNorm
def test_rmsnorm_closed_form(orc):
    rng = np.random.default_rng(70)
    for n, scale in ((512, 1.0), (2816, 30.0), (64, 1e-3)):
        x = (rng.standard_normal(n) * scale).astype(np.float32)
        w = rng.normal(1, 0.1, n).astype(np.float32)
        y = orc.rmsnorm(x, w, 1e-6)
        want = TB.rmsnorm(x, w, 1e-6)
        assert np.all(np.abs(y - want) <= 4 * 2.0 ** -24 * np.abs(want) + 1e-30)
        s = orc.rms_scale(x, 1e-6)
        assert abs(s - 1 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6)) <= 2 * 2.0 ** -24 * s


def test_rmsnorm_special_inputs(orc):
    w = np.ones(256, np.float32)
    assert not orc.rmsnorm(np.zeros(256, np.float32), w, 1e-6).any()
    y = orc.rmsnorm(np.full(256, -3.0, np.float32), w, 1e-6)
    assert np.allclose(y, -1.0, rtol=1e-6)
    tiny = np.full(256, 1e-20, np.float32)  # eps dominates: scale = 1/sqrt(1e-6) = 1000
    assert np.allclose(orc.rmsnorm(tiny, w, 1e-6), 1e-17, rtol=1e-5)
