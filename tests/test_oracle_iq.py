"""Pins of the oracle's IQ dots (oracle/oracle.c orc_dot_iq: DotIQ2XXS / DotIQ2S / DotIQ3S,
src/CpuRefIQuants.cs:45-146) and of the codebooks the library and the oracle share
(phoenix-lai_amd/csrc/iq_grids.h): the codebooks expand to the reference's IqTables (src/IqTables.cs,
read as text when present), the sign tables follow their rule, and on blocks with power-of-two scales and
small integer activations every float step is exact, so the oracle equals the exact dot of an
independent decoder (tests/gguf_spec.py) bit for bit.  CPU only."""
import re
from pathlib import Path

import numpy as np
import pytest

import gguf_spec as G

IQ = {"iq2_xxs": 16, "iq2_s": 22, "iq3_s": 21}
REF_TABLES = Path("/root/reference/src/IqTables.cs")


@pytest.mark.skipif(not REF_TABLES.exists(), reason="the reference's tables are not on this machine")
def test_codebooks_equal_the_reference_tables():
    src = REF_TABLES.read_text()

    def arr(name):
        body = re.search(name + r"\s*=\s*//[^\n]*\n\s*\{(.*?)\};", src, re.S).group(1)
        return [int(v.rstrip("UL"), 0) for v in re.findall(r"0x[0-9a-fA-F]+UL|0x[0-9a-fA-F]+|\d+", body)]

    books = G.iq_codebooks()
    for name, t, n in (("Iq2xxsGrid", 16, 8), ("Iq2sGrid", 22, 8), ("Iq3sGrid", 21, 4)):
        words = [sum(int(b) << (8 * j) for j, b in enumerate(row)) for row in books[t]]
        assert words == arr(name), name
    assert arr("KsignsIq2xs") == [G.ksigns(i) for i in range(128)]
    assert arr("KmaskIq2xs") == [1 << j for j in range(8)]


def _exact_case(rng, t, nsb):
    """nsb super-blocks of random IQ bytes with one power-of-two d, and an input whose Q8_K is exact
    (-127 leads every super-block, the rest small integers): every product and partial sum of the
    reference's chain is then a float without rounding."""
    bb = {16: 66, 22: 82, 21: 110}[t]
    row = rng.integers(0, 256, (nsb, bb), dtype=np.uint8)
    row[:, :2] = np.array([2.0 ** -6], np.float16).view(np.uint8)
    x = rng.integers(-10, 11, 256 * nsb).astype(np.float32)
    x[::256] = -127.0
    return row.reshape(-1), x


@pytest.mark.parametrize("t", list(IQ.values()), ids=list(IQ))
def test_iq_dot_exact_identity(orc, t):
    rng = np.random.default_rng(t)
    books = G.iq_codebooks()
    for trial in range(6):
        row, x = _exact_case(rng, t, 2)
        got = orc.matvec(t, row, 1, 512, x)[0]
        want = float(np.dot(G.dequant_iq(t, row, 512, books), x.astype(np.float64)))
        assert got == np.float32(want), (trial, float(got), want)


@pytest.mark.parametrize("t", list(IQ.values()), ids=list(IQ))
def test_iq_dot_vs_float64(orc, t):
    """Random blocks and inputs: within the fp32 error of the chain of the exact decoded dot."""
    rng = np.random.default_rng(100 + t)
    books = G.iq_codebooks()
    bb = {16: 66, 22: 82, 21: 110}[t]
    for trial in range(4):
        row = rng.integers(0, 256, (4, bb), dtype=np.uint8)
        row[:, :2] = (np.abs(rng.standard_normal(4)) * 1e-3).astype(np.float16).view(np.uint8).reshape(4, 2)
        x = rng.standard_normal(1024).astype(np.float32)
        got = float(orc.matvec(t, row.reshape(-1), 1, 1024, x)[0])
        kd, kq, _ = orc.quantize_q8_k(x)
        w = G.dequant_iq(t, row.reshape(-1), 1024, books)
        want = sum(float(kd[b]) * float(np.dot(w[256 * b:256 * b + 256], kq[256 * b:256 * b + 256])) for b in range(4))
        mag = sum(abs(float(kd[b])) * float(np.abs(w[256 * b:256 * b + 256]) @ np.abs(kq[256 * b:256 * b + 256]))
                  for b in range(4))
        assert abs(got - want) <= 8 * 2.0 ** -24 * mag + 1e-30, (trial, got, want)


def test_iq_rows_do_not_dequantize(orc):
    """The reference does not dequantize IQ rows (src/CpuRefKQuants.cs:151): neither does the oracle."""
    with pytest.raises(AssertionError):
        orc.dequantize_row(16, np.zeros(66, np.uint8), 256)
