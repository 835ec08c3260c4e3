"""Known answers that pin the ORDER of the oracle's sequential fp32 chains, which an error bound cannot:
the router logit (src/GemmaCpu.cs:392-395), the Q4_0 and Q8_0 block chains (src/CpuRefGemma.cs:27-36,
src/CpuRef.cs:106-115), and DotK's eight float lanes with their final fold (src/CpuRefKQuants.cs:200-211).

Each case plants one large term M (not a power of two) followed by small terms that each lie strictly
between half an ulp and one ulp of the running sum.  Added left to right, every small term rounds the
sum up by exactly one ulp, so the chain ends at M + n ulp(M) (the sum stays inside M's binade).  Any
other order (reversed, pairwise, a double accumulator, lanes merged into one chain, the min term moved)
first adds small terms to each other, exactly, and lands elsewhere; each test also checks that those
alternatives give different bits, so the known answer discriminates.  CPU only."""
import numpy as np
import pytest

import gguf_spec as G

F32 = np.float32
Q4_0, Q8_0, Q4_K, Q6_K = 2, 8, 12, 14


def ulp(v):
    return float(np.spacing(F32(abs(v))))


def _seq(terms):
    s = F32(0)
    for t in terms:
        s = F32(s + F32(t))
    return s


def _rev(terms):
    return _seq(list(terms)[::-1])


def _pairwise(terms):
    t = [F32(v) for v in terms]
    while len(t) > 1:
        t = [F32(t[i] + t[i + 1]) if i + 1 < len(t) else t[i] for i in range(0, len(t), 2)]
    return t[0]


def _double(terms):
    return F32(sum(float(v) for v in terms))


def _assert_discriminates(want, terms):
    for alt in (_rev, _pairwise, _double):
        assert alt(terms) != want, f"{alt.__name__} gives the known answer too: the case pins nothing"


# ---------------------------------------------------------------------------------------- router
def test_router_logit_chain_is_left_to_right(orc, pkg):
    """logit_e = sum_i W[e][i] * m_i as one float chain from i = 0.  W[2] = (1, 2^-24, ..., 2^-24, 0...):
    the first product is m_0 and each later one is m_1 * 2^-24, exactly (power-of-two scaling).  The
    router input scale 1.2 on elements 1.. puts m_1 mid-binade, so that product is about 0.6 ulp(m_0)."""
    n = 200
    L = pkg.synth.make_layer(dict(idx=9, T=1, d=256, E=8, k=2, nf=128, gu=2, dn=2))
    W = np.zeros_like(L["gate_inp"])
    W[0, 0] = 1.0  # probe: logit 0 = m_0
    W[1, 1] = 1.0  # probe: logit 1 = m_1
    W[2, 0] = 1.0
    W[2, 1:1 + n] = 2.0 ** -24
    L["gate_inp"] = W
    L["gate_inp_scale"] = np.full(L["d"], 1.2, F32)
    L["gate_inp_scale"][0] = 1.0
    x = np.ones(L["d"], F32)
    x[0] = 1.3  # m_0 inside its binade, the other m_i equal
    logits, _, _ = orc.router(L, x)
    m0, m1 = float(logits[0]), float(logits[1])
    p = m1 * 2.0 ** -24
    assert m0 != 2.0 ** np.floor(np.log2(m0)), "M must not be a power of two"
    assert ulp(m0) / 2 < p < ulp(m0), "each small product must lie between half an ulp and one ulp"
    want = F32(m0 + n * ulp(m0))
    assert np.floor(np.log2(float(want))) == np.floor(np.log2(m0)), "the sum must stay in M's binade"
    assert logits[2] == want, (float(logits[2]), float(want))
    _assert_discriminates(want, [m0] + [p] * n)


# ---------------------------------------------------------------------------------------- Q4_0 / Q8_0 chains
def _block_chain_case(t, nblk=64):
    """One row of nblk blocks and its input: block 0's term is 14224 (isum 889 or 14224 times d_w), each
    later block's is 8890 * 2^-24 (d_w = 2^-24, the smallest fp16 subnormal).  ulp(14224) = 2^-10 =
    16384 * 2^-24, so every later term is between half an ulp and an ulp."""
    x = np.zeros(32 * nblk, F32)
    x[0] = 127.0  # Q8_0 of the input: d_x = 127 / 127 = 1 exactly, q = x
    for b in range(1, nblk):
        x[32 * b:32 * b + 10] = 127.0
    if t == Q4_0:
        row = np.zeros((nblk, 18), np.uint8)
        row[:, 2:] = 0x88  # nibble 8: weight 0
        row[0, 0], row[0, 1] = G.h16_bits(16.0) & 0xFF, G.h16_bits(16.0) >> 8
        row[0, 2] = 0x8F  # element 0: nibble 15 -> 7; isum 889, term 889 * 16 = 14224
        row[1:, 0] = 0x01  # fp16 0x0001 = 2^-24
        row[1:, 2:12] = 0x8F  # elements 0..9: weight 7; isum 10 * 7 * 127 = 8890
    else:
        row = np.zeros((nblk, 34), np.uint8)
        row[0, 0], row[0, 1] = G.h16_bits(1.0) & 0xFF, G.h16_bits(1.0) >> 8
        row[0, 2] = 112  # isum 127 * 112 = 14224
        row[1:, 0] = 0x01
        row[1:, 2:12] = 7  # isum 8890
    return row.reshape(-1), x


@pytest.mark.parametrize("t", [Q4_0, Q8_0])
def test_block_chain_is_left_to_right(orc, t):
    nblk = 64
    row, x = _block_chain_case(t, nblk)
    got = orc.matvec(t, row, 1, 32 * nblk, x)[0]
    small = 8890 * 2.0 ** -24
    assert ulp(14224.0) / 2 < small < ulp(14224.0)
    want = F32(14224.0 + (nblk - 1) * ulp(14224.0))
    assert got == want, (float(got), float(want))
    _assert_discriminates(want, [14224.0] + [small] * (nblk - 1))


# ---------------------------------------------------------------------------------------- DotK
def _q8k_input(nsb, values):
    """An input of nsb super-blocks whose Q8_K quantization is exact: element 0 of every super-block is
    -127, the largest magnitude, so iscale = -127 / -127 = 1, q = x and d = 1.  values: {index: value}."""
    x = np.zeros(256 * nsb, F32)
    x[::256] = -127.0
    for i, v in values.items():
        x[i] = v
    return x


def _q6k_row(blocks):
    """blocks: list of (d_bits, {element: a}) with all 16 scales 1 and a = 0 elsewhere."""
    out = []
    for d_bits, a in blocks:
        q = np.zeros(256, np.int32)
        for e, v in a.items():
            q[e] = v
        out.append(G.pack_q6_k(d_bits, np.ones(16, np.int32), q))
    return np.concatenate(out)


D1, DTINY = G.h16_bits(1.0), 0x0001  # 1.0 and 2^-24
LANE_BIG, LANE_SMALL = 1000.0, 600 * 2.0 ** -24  # ulp(1000) = 2^-14 = 1024 * 2^-24


def test_dotk_lane_fold_is_left_to_right(orc):
    """Super-block 0 puts 1000 on lane 0 (element 8: q 100 times a 10, d = 1); super-block 1 puts
    600 * 2^-24 on each of lanes 1..7 (elements 1..7: q 100 times a 6, d = 2^-24).  The fold
    sumf += sums[l], l = 0..7, gains one ulp per lane: 1000 + 7 * 2^-14."""
    x = _q8k_input(2, {8: 100.0, **{256 + l: 100.0 for l in range(1, 8)}})
    row = _q6k_row([(D1, {8: 10}), (DTINY, {l: 6 for l in range(1, 8)})])
    got = orc.matvec(Q6_K, row, 1, 512, x)[0]
    assert ulp(LANE_BIG) / 2 < LANE_SMALL < ulp(LANE_BIG)
    want = F32(LANE_BIG + 7 * ulp(LANE_BIG))
    assert got == want, (float(got), float(want))
    _assert_discriminates(want, [LANE_BIG] + [LANE_SMALL] * 7)


def test_dotk_lanes_accumulate_across_superblocks(orc):
    """Lane 1 takes 600 * 2^-24 in each of super-blocks 1..4 and sums them exactly in its own float
    (2400 * 2^-24); the fold then adds that once to lane 0's 1000: 1000 + 2 * 2^-14 (2.34 ulps rounded).
    One chain over every block's terms (no lanes) would reach 1000 + 4 * 2^-14."""
    x = _q8k_input(5, {8: 100.0, **{256 * b + 1: 100.0 for b in range(1, 5)}})
    row = _q6k_row([(D1, {8: 10})] + [(DTINY, {1: 6})] * 4)
    got = orc.matvec(Q6_K, row, 1, 1280, x)[0]
    want = F32(LANE_BIG + 2 * ulp(LANE_BIG))
    assert got == want, (float(got), float(want))
    assert _seq([LANE_BIG] + [LANE_SMALL] * 4) != want  # the merged single chain


def test_dotk_min_term_precedes_the_fold(orc):
    """Q4_K with dmin = 1 and the sub-block-0 min 8 against q sums of 125 (elements 0..3: -127, 100,
    100, 52, all at nibble 0): sumf = -(1 * 1000) first.  d = 2^-24 and elements 32..39 (sub-block 1,
    scale 1, min 0: q 100 times nibble 6) put 600 * 2^-24 on every lane.  Folding the eight lanes onto
    -1000 gains one ulp each: -1000 + 8 * 2^-14.  With the min term last the lanes would sum first
    (4800 * 2^-24) and give -1000 + 5 * 2^-14."""
    x = _q8k_input(1, {1: 100.0, 2: 100.0, 3: 52.0, **{32 + l: 100.0 for l in range(8)}})
    q = np.zeros(256, np.int32)
    q[32:40] = 6
    sc = np.zeros(8, np.int32)
    sc[1] = 1
    m = np.zeros(8, np.int32)
    m[0] = 8
    row = G.pack_q4_k(DTINY, D1, sc, m, q)
    got = orc.matvec(Q4_K, row, 1, 256, x)[0]
    want = F32(-LANE_BIG + 8 * ulp(LANE_BIG))
    assert got == want, (float(got), float(want))
    terms = [-LANE_BIG] + [LANE_SMALL] * 8
    assert _seq(terms[1:] + terms[:1]) != want  # min term added after the lanes
    _assert_discriminates(want, terms)


def test_iq_superblock_chain_is_left_to_right(orc):
    """DotIQ2XXS's sumf += d * bsum over super-blocks (src/CpuRefIQuants.cs:51-75), then 0.125 * sumf.
    Every super-block uses grid entry 0 (all eights), no signs and scale 1, so bsum = 8 * (sum of its
    quants): 800 in super-block 0 (d = 1), 600 in super-blocks 1..7 (d = 2^-24: 600 * 2^-24 is between
    half an ulp and an ulp of 800).  The chain ends at 800 + 7 * 2^-14, scaled exactly by 0.125."""
    nsb = 8
    row = np.zeros((nsb, 66), np.uint8)
    row[0, 0], row[0, 1] = D1 & 0xFF, D1 >> 8
    row[1:, 0] = DTINY
    x = np.zeros(256 * nsb, F32)
    x[::256] = -127.0
    x[1::256] = 127.0
    x[2] = 100.0
    x[256 + 2::256] = 75.0
    got = orc.matvec(16, row.reshape(-1), 1, 256 * nsb, x)[0]
    small = 600 * 2.0 ** -24
    assert ulp(800.0) / 2 < small < ulp(800.0)
    want = F32(F32(800.0 + (nsb - 1) * ulp(800.0)) * F32(0.125))
    assert got == want, (float(got), float(want))
    for alt in (_rev, _pairwise, _double):
        assert F32(alt([800.0] + [small] * (nsb - 1)) * F32(0.125)) != want
