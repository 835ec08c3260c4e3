"""The certification rule of the kernels' means of squares (device_common.h mean_ends): a parallel double
sum S of n squares with error bound B certifies the reference's (float)(sum / n) (CpuRef.RmsNorm,
src/CpuRef.cs:186-188) when the float ends of (S -/+ B') * (1 / n), B' = B + S * 2^-49, agree.  Checked
here in float64 / float32 arithmetic (Python floats are IEEE doubles, as the device's) against the
true quotient of every sum the bound allows: the interval's ends and points inside, on random sums and
on sums planted next to a float rounding boundary of the mean."""
import numpy as np
import pytest


def ends(S, B, n):
    rn = 1.0 / n
    Bw = B + S * 2.0 ** -49
    return np.float32((S - Bw) * rn), np.float32((S + Bw) * rn)


def ref_mean(ss, n):
    return np.float32(ss / n)


@pytest.mark.parametrize("n", [512, 2112, 2816, 4096, 12288])
def test_certified_means_equal_the_reference(n):
    rng = np.random.default_rng(n)
    certified = 0
    for i in range(4000):
        S = float(np.exp(rng.uniform(-40, 40)))
        if i % 2:  # planted: S / n within a few double ulps of a float rounding boundary
            m = np.float32(S / n)
            up = np.nextafter(m, np.float32(np.inf))
            mid = (float(m) + float(up)) / 2.0
            S = mid * n * (1.0 + rng.integers(-8, 9) * 2.0 ** -52)
        B = (n + 64.0) * 2.0 ** -52 * S
        lo, hi = ends(S, B, n)
        if lo != hi:
            continue
        certified += 1
        for ss in (S - B, S + B, S, S - B * rng.random(), S + B * rng.random()):
            assert ref_mean(ss, n) == lo, (S, B, ss, n)
    assert certified > 1000


def test_widening_covers_the_reciprocal_rounding():
    # the widening S * 2^-49 exceeds the relative error of rn = 1/n and of the product S * rn (each
    # below 2^-53): a quotient computed as a product never leaves the widened ends
    rng = np.random.default_rng(7)
    for _ in range(20000):
        n = int(rng.integers(32, 1 << 15))
        S = float(np.exp(rng.uniform(-30, 30)))
        assert (S - S * 2.0 ** -49) * (1.0 / n) <= S / n <= (S + S * 2.0 ** -49) * (1.0 / n)
