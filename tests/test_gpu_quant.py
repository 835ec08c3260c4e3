"""GPU parity of the standalone activation quantizers (phx_quant_q8_0 / phx_quant_q8_k, the
KernelsQuant.Q80 / Q8K ops of src/KernelsQuant.cs:57-172) and of the residual norm-add with the next
norm's quantized input (phx_norm_add, KernelsGemma.NormAdd / NormAddQuant, src/KernelsGemma.cs:126-226)
through the C ABI: every mode's quantized integers, scales and block sums equal the oracle's
CpuRef.QuantizeQ8_0 / QuantizeQ8_K of the transformed input (CpuRef.RmsNorm, gelu(x) * u, silu(x) * u),
and the new residual rows the oracle's, bit for bit."""
import ctypes as C
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

EPS = 1e-6
MODES = {"plain": 0, "silu_mul": 1, "rms_norm": 2, "gelu_mul": 3}


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def transformed(orc, mode, x, aux):
    """The reference's input to the quantizer, row by row (float32 products as the C# code rounds them)."""
    if mode == "plain":
        return x
    if mode == "rms_norm":
        return np.stack([orc.rmsnorm(r, aux, EPS) for r in x])
    f = orc.gelu(x) if mode == "gelu_mul" else orc.silu(x)
    return (f * aux).astype(np.float32)


def inputs(rows, n, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, n)) * 3.0).astype(np.float32)
    u = rng.standard_normal((rows, n)).astype(np.float32)
    w = (1.0 + 0.2 * rng.standard_normal(n)).astype(np.float32)
    # edge rows: an all-zero row; ties of |x| of both signs (the first index wins in Q8_K) and
    # halfway products (Q8_0 rounds them away from zero, Q8_K to even)
    x[1] = 0.0
    x[2, :64] = np.tile(np.float32([127.0, -127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 126.5]), 8)
    if n >= 512:
        x[2, 256:264] = np.float32([-127.0, 127.0, 2.5, -2.5, 3.5, -3.5, 0.0, -0.0])
    return x, u, w


# n above 8192 (RmsNorm mode): several 2048-element workgroups per row, each forming the row mean, with a
# partial last chunk at 9216 and 8448
@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("n", [256, 2816, 4352, 9216, 12288])
def test_q8_0_matches_oracle(ctx, orc, mode, n):
    say(f"quant q8_0: mode={mode} rows=4 n={n}")
    x, u, w = inputs(4, n, seed=n + MODES[mode])
    aux = None if mode == "plain" else (w if mode == "rms_norm" else u)
    qs, d = ctx.Q80(MODES[mode], x, aux, EPS)
    v = transformed(orc, mode, x, aux)
    for r in range(4):
        rd, rq = orc.quantize_q8_0(v[r])
        np.testing.assert_array_equal(d[r], rd, err_msg=f"row {r}: fp16 scales")
        np.testing.assert_array_equal(qs[r], rq, err_msg=f"row {r}: quants")


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("n", [256, 3072, 4608, 8448, 12288])
def test_q8_k_matches_oracle(ctx, orc, mode, n):
    say(f"quant q8_k: mode={mode} rows=4 n={n}")
    x, u, w = inputs(4, n, seed=7 * n + MODES[mode])
    aux = None if mode == "plain" else (w if mode == "rms_norm" else u)
    qs, d, bs = ctx.Q8K(MODES[mode], x, aux, EPS)
    v = transformed(orc, mode, x, aux)
    for r in range(4):
        rd, rq, rb = orc.quantize_q8_k(v[r])
        np.testing.assert_array_equal(d[r].view(np.uint32), rd.view(np.uint32), err_msg=f"row {r}: scales")
        np.testing.assert_array_equal(qs[r], rq, err_msg=f"row {r}: quants")
        np.testing.assert_array_equal(bs[r], rb, err_msg=f"row {r}: block sums")


def test_quant_rejects_bad_arguments(ctx, pkg, orc):
    say("quant: argument checks")
    x = np.ones((2, 64), np.float32)
    with pytest.raises(pkg.moe.ArgumentError):
        ctx.Q80(7, x)  # no such mode
    with pytest.raises(pkg.moe.ArgumentError):
        ctx.Q80(0, np.ones((2, 48), np.float32))  # n not a multiple of 32
    with pytest.raises(pkg.moe.ArgumentError):
        ctx.Q8K(0, x)  # n not a multiple of 256
    with pytest.raises(pkg.moe.ArgumentError):
        ctx.Q80(3, x)  # gelu_mul without u
    qs, d = ctx.Q80(0, x)  # the context still works
    rd, rq = orc.quantize_q8_0(x[0])
    assert (qs == rq).all() and (d == rd).all()


# ---------------------------------------------------------------------------------------- norm + residual
def norm_add_ref(orc, x, y, w, s, w2):
    """GemmaCpu.PostAndFfn's residual (src/GemmaCpu.cs:353-356, 367) and the next layer's quantized
    RmsNorm input (src/CpuRef.cs:49-62, 183-191), row by row through the oracle."""
    xn = np.stack([(x[r] + orc.rmsnorm(y[r], w, EPS)).astype(np.float32) for r in range(x.shape[0])])
    if s != 1.0:
        xn = (xn * np.float32(s)).astype(np.float32)
    if w2 is None:
        return xn, None, None
    q = [orc.quantize_q8_0(orc.rmsnorm(xn[r], w2, EPS)) for r in range(x.shape[0])]
    return xn, np.stack([a[1] for a in q]), np.stack([a[0] for a in q])


@pytest.mark.parametrize("s", [1.0, 0.75])
@pytest.mark.parametrize("quant", [False, True])
@pytest.mark.parametrize("n", [2816, 16384])
def test_norm_add_matches_oracle(ctx, orc, s, quant, n):
    say(f"norm_add: rows=3 n={n} s={s} quant={quant}")
    rng = np.random.default_rng(n + int(4 * s) + quant)
    x = (rng.standard_normal((3, n)) * 4).astype(np.float32)
    y = (rng.standard_normal((3, n)) * 40).astype(np.float32)
    y[1] = 0.0  # rmsnorm of zeros adds zeros
    w = (1 + 0.3 * rng.standard_normal(n)).astype(np.float32)
    w2 = (1 + 0.3 * rng.standard_normal(n)).astype(np.float32) if quant else None
    got = ctx.NormAdd(x, y, w, EPS, s, w2)
    want = norm_add_ref(orc, x, y, w, s, w2)
    if not quant:
        np.testing.assert_array_equal(got, want[0])
        return
    np.testing.assert_array_equal(got[0], want[0], err_msg="new x")
    np.testing.assert_array_equal(got[1], want[1], err_msg="quants")
    np.testing.assert_array_equal(got[2], want[2], err_msg="fp16 scales")


def test_norm_add_rejects_bad_arguments(ctx, pkg):
    say("norm_add: argument checks")
    x = np.ones((2, 64), np.float32)
    with pytest.raises(pkg.moe.ArgumentError):
        ctx.NormAdd(np.ones((1, 16392), np.float32), np.ones((1, 16392), np.float32), np.ones(16392, np.float32))
    with pytest.raises(pkg.moe.ArgumentError):
        ctx.NormAdd(np.ones((1, 36), np.float32), np.ones((1, 36), np.float32), np.ones(36, np.float32),
                    w2=np.ones(36, np.float32))  # n not a multiple of 32 with the quantized output
    np.testing.assert_array_equal(ctx.NormAdd(x, np.zeros_like(x), np.ones(64, np.float32)), x)


# ---------------------------------------------------------------------------------------- dense matvec
def gguf_rows(rng, wtype, rows, cols):
    """Random GGUF rows of Q4_0 (18-byte blocks) or Q8_0 (34-byte): random quants, finite fp16 scales."""
    bb = 18 if wtype == 2 else 34
    blocks = rng.integers(0, 256, (rows * cols // 32, bb), dtype=np.uint8)
    d = (rng.standard_normal(rows * cols // 32) * 0.01).astype(np.float16)
    blocks[:, :2] = d.view(np.uint8).reshape(-1, 2)
    return blocks.reshape(-1)


@pytest.mark.parametrize("wtype", [2, 8])
@pytest.mark.parametrize("T,rows,cols", [(1, 2112, 2816), (3, 301, 2816), (2, 64, 12288)])
def test_matvec_matches_oracle(ctx, orc, wtype, T, rows, cols):
    """phx_quant_q8_0 then phx_matvec equals CpuRef.MatVec (the oracle's matvec: Q8_0 input, block terms
    added in order), bit for bit; rows not a multiple of the workgroup's four."""
    say(f"matvec: type={wtype} T={T} rows={rows} cols={cols}")
    rng = np.random.default_rng(rows + cols + wtype)
    w = gguf_rows(rng, wtype, rows, cols)
    x = rng.standard_normal((T, cols)).astype(np.float32)
    qs, d = ctx.Q80(0, x)
    y = ctx.MatVec(wtype, w, rows, cols, qs, d)
    for t in range(T):
        np.testing.assert_array_equal(y[t], orc.matvec(wtype, w, rows, cols, x[t]), err_msg=f"token {t}")


@pytest.mark.parametrize("wtype", [2, 8])
@pytest.mark.parametrize("T,rows,cols", [(1, 301, 512), (5, 2112, 2816), (31, 64, 12288), (32, 301, 2816),
                                         (200, 2112, 2816), (2048, 2816, 2112)])
def test_matmul_matches_oracle(ctx, orc, wtype, T, rows, cols):
    """phx_weight_upload + phx_matmul (KernelsPrefill.MatMulQ4Q8Tile as GemmaGpu.Mm records it) equal
    CpuRef.MatVec per token, bit for bit: the VALU row walk below 32 tokens, the matrix cores from 32 (one
    partial 128-token tile, several, and C3's 2048 prompt rows through the shared FFN's down shape); row
    counts not a multiple of the 64-row group."""
    say(f"matmul: type={wtype} T={T} rows={rows} cols={cols}")
    rng = np.random.default_rng(rows + cols + wtype + T)
    w = gguf_rows(rng, wtype, rows, cols)
    h = ctx.weight_upload(wtype, w, rows, cols)
    try:
        x = rng.standard_normal((T, cols)).astype(np.float32)
        qs, d = ctx.Q80(0, x)
        y = ctx.MatMul(h, rows, cols, qs, d)
    finally:
        ctx.weight_free(h)
    toks = range(T) if T <= 200 else sorted(set([0, 1, T - 1] + rng.choice(T, 45, replace=False).tolist()))
    for t in toks:
        np.testing.assert_array_equal(y[t], orc.matvec(wtype, w, rows, cols, x[t]), err_msg=f"token {t}")


def gguf_k_rows(rng, wtype, rows, cols):
    """Random GGUF rows of Q3_K (110-byte super-blocks), Q4_K (144), Q5_K (176) or Q6_K (210): every quant,
    high bit, 6-bit scale and min, and int8 sub-block scale value, with finite fp16 super-block scales."""
    bb = {11: 110, 12: 144, 13: 176, 14: 210}[wtype]
    n = rows * cols // 256
    blocks = rng.integers(0, 256, (n, bb), dtype=np.uint8)
    d = (rng.standard_normal(n) * 0.002).astype(np.float16)
    if wtype in (12, 13):
        blocks[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        dmin = (np.abs(rng.standard_normal(n)) * 0.001).astype(np.float16)
        blocks[:, 2:4] = dmin.view(np.uint8).reshape(-1, 2)
    else:
        off = 108 if wtype == 11 else 208
        blocks[:, off:off + 2] = d.view(np.uint8).reshape(-1, 2)
    return blocks.reshape(-1)


@pytest.mark.parametrize("wtype", [11, 12, 13, 14])
@pytest.mark.parametrize("T,rows,cols", [(1, 1408, 4096), (3, 301, 2816), (7, 64, 12288), (8, 301, 2816),
                                         (48, 4096, 1536), (200, 2112, 4096), (512, 4096, 1536)])
def test_matmul_k_matches_oracle(ctx, orc, wtype, T, rows, cols):
    """phx_quant_q8_k, phx_weight_upload and phx_matmul_k (KernelsK.MatVec as GemmaGpu.MatVec records it for
    Q4_K / Q6_K weights) equal CpuRefKQuants.MatVecK per token, bit for bit: the VALU row walk below 8
    tokens, the matrix cores from 8 (one partial tile, whole tiles, and C4's 512 rows through its down
    shape); row counts not a multiple of the 64-row group."""
    say(f"matmul_k: type={wtype} T={T} rows={rows} cols={cols}")
    rng = np.random.default_rng(rows + cols + wtype + T)
    w = gguf_k_rows(rng, wtype, rows, cols)
    h = ctx.weight_upload(wtype, w, rows, cols)
    try:
        x = rng.standard_normal((T, cols)).astype(np.float32)
        x[0, :256] = 0.0  # an all-zero super-block (d = 0)
        qs, d, _ = ctx.Q8K(0, x)
        y = ctx.MatMulK(h, rows, cols, qs, d)
    finally:
        ctx.weight_free(h)
    toks = range(T) if T <= 64 else sorted(set([0, 1, T - 1] + rng.choice(T, 45, replace=False).tolist()))
    for t in toks:
        np.testing.assert_array_equal(y[t], orc.matvec(wtype, w, rows, cols, x[t]), err_msg=f"token {t}")


def test_matmul_rejects_bad_arguments(ctx, pkg):
    say("matmul: argument checks")
    with pytest.raises(pkg.moe.NotSupportedError):  # IQ2_XXS: no dense upload
        ctx._check(ctx.lib.phx_weight_upload(ctx.h, 16, 1, 256, np.zeros(66, np.uint8).ctypes.data,
                                             C.byref(C.c_void_p())))
    with pytest.raises(pkg.moe.ArgumentError):
        ctx.weight_upload(12, np.zeros(144, np.uint8), 1, 128)  # K-quant cols not a multiple of 256
    hk = ctx.weight_upload(12, np.zeros(144, np.uint8), 1, 256)
    h0 = ctx.weight_upload(2, np.zeros(18 * 8, np.uint8), 1, 256)
    try:
        q, dk, d0 = np.zeros((1, 256), np.int8), np.zeros((1, 1), np.float32), np.zeros((1, 8), np.uint16)
        with pytest.raises(pkg.moe.NotSupportedError):  # a K-quant weight takes Q8_K input
            ctx.MatMul(hk, 1, 256, q, d0)
        with pytest.raises(pkg.moe.NotSupportedError):  # and a Q4_0 weight Q8_0 input
            ctx.MatMulK(h0, 1, 256, q, dk)
        np.testing.assert_array_equal(ctx.MatMulK(hk, 1, 256, q, dk), np.zeros((1, 1), np.float32))
    finally:
        ctx.weight_free(hk)
        ctx.weight_free(h0)
    with pytest.raises(pkg.moe.ArgumentError):
        ctx.weight_upload(2, np.zeros(17, np.uint8), 1, 32)  # short rows
    with pytest.raises(pkg.moe.ArgumentError):
        ctx.weight_upload(2, np.zeros(18 * 2, np.uint8), 1, 48)  # cols not a multiple of 32


def test_matvec_rejects_other_types(ctx, pkg):
    say("matvec: argument checks")
    q, d = np.zeros(64, np.int8), np.zeros(2, np.uint16)
    with pytest.raises(pkg.moe.NotSupportedError):
        ctx.MatVec(12, np.zeros(144, np.uint8), 1, 64, q, d)  # Q4_K
    with pytest.raises(pkg.moe.ArgumentError):
        ctx.MatVec(2, np.zeros(18, np.uint8), 1, 48, np.zeros(48, np.int8), np.zeros(1, np.uint16))
