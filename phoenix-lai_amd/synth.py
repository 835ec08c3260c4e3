"""Seeded synthetic MoE layers for the benchmark configurations (libphxsynth.so).

Config i uses base seed 1000 + i; every tensor has its own stream keyed by its GGUF name, so a
tensor's values do not depend on which other tensors are generated.  Expert weights are N(0, 0.02)
quantized by this project's GGUF block encoders (the reference has no weight-side quantizer).
Router popularity bias (Zipf, or one hot expert) is carried by one input channel: x[t][d-1] = 4
and W[e][d-1] = b_e / m, with b calibrated so the top-k selection shares follow the target
(the reference router has no bias term).
"""
from __future__ import annotations

import ctypes as C
from functools import lru_cache
from pathlib import Path

import numpy as np

from .moe import PHX

_HERE = Path(__file__).resolve().parent

CONFIGS = {
    # tiny CPU-runnable layer
    "c1_tiny": dict(idx=1, T=16, d=512, E=8, k=2, nf=1024, gu=PHX.Q4_0, dn=PHX.Q4_0),
    # decode (the bench workload), plus the dense shared FFN
    "c2_decode": dict(idx=2, T=1, d=2816, E=128, k=8, nf=704, gu=PHX.Q4_0, dn=PHX.Q4_0, nff=2112, sh=PHX.Q4_0),
    # prefill with Zipf(1.1) expert popularity
    "c3_prefill": dict(idx=3, T=2048, d=2816, E=128, k=8, nf=704, gu=PHX.Q4_0, dn=PHX.Q4_0, zipf=1.1),
    # K-quants, Q6_K down padded 1408 -> 1536
    "c4_kquant": dict(idx=4, T=512, d=4096, E=64, k=4, nf=1408, gu=PHX.Q4_K, dn=PHX.Q6_K),
    # 30-layer batched decode stack, Q8_0, ~40% of tokens to one hot expert
    "c5_stack": dict(idx=5, T=32, d=2816, E=128, k=8, nf=704, gu=PHX.Q8_0, dn=PHX.Q8_0, layers=30, hot=0.40),
}

BIAS_X = 4.0  # value of the bias channel x[t][d-1]


def _lib():
    lib = C.CDLL(str(_HERE / "libphxsynth.so"))
    u64, i64, f32, i32, vp = C.c_uint64, C.c_int64, C.c_float, C.c_int, C.c_void_p
    lib.phx_synth_normal.argtypes = [u64, C.c_char_p, f32, f32, vp, i64, i64]
    lib.phx_synth_bytes.argtypes = [u64, C.c_char_p, vp, i64]
    lib.phx_synth_quantize.argtypes = [i32, vp, i64, i32, vp]
    lib.phx_synth_quantize.restype = i32
    lib.phx_synth_quantized_normal.argtypes = [u64, C.c_char_p, f32, f32, i32, i64, i32, i32, vp]
    lib.phx_synth_quantized_normal.restype = i32
    lib.phx_synth_row_bytes.argtypes = [i32, i32]
    lib.phx_synth_row_bytes.restype = i64
    lib.phx_synth_calibrate_bias.argtypes = [u64, i32, i32, vp, C.c_double, i32, i32, vp]
    return lib


_L = None


def lib():
    global _L
    if _L is None:
        _L = _lib()
    return _L


_IQ_BYTES = {PHX.IQ2_XXS: 66, PHX.IQ2_S: 82, PHX.IQ3_S: 110}


def row_bytes(t: int, cols: int) -> int:
    if t in _IQ_BYTES:
        return cols // 256 * _IQ_BYTES[t]
    return int(lib().phx_synth_row_bytes(t, cols))


def block_elems(t: int) -> int:
    return 256 if t in (PHX.Q3_K, PHX.Q4_K, PHX.Q5_K, PHX.Q6_K) or t in _IQ_BYTES else (1 if t == PHX.F32 else 32)


def normal(seed: int, name: str, shape, mean=0.0, std=1.0, offset=0) -> np.ndarray:
    out = np.empty(shape, np.float32)
    lib().phx_synth_normal(seed, name.encode(), mean, std, out.ctypes.data, out.size, offset)
    return out


def random_bytes(seed: int, name: str, n: int) -> np.ndarray:
    out = np.empty(n, np.uint8)
    lib().phx_synth_bytes(seed, name.encode(), out.ctypes.data, n)
    return out


def quantize(t: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    out = np.empty(rows * row_bytes(t, cols), np.uint8)
    rc = lib().phx_synth_quantize(t, x.ctypes.data, rows, cols, out.ctypes.data)
    if rc:
        raise ValueError(f"quantize type {t} cols {cols}: {rc}")
    return out


IQ_TYPES = (PHX.IQ2_XXS, PHX.IQ2_S, PHX.IQ3_S)


def iq_blocks(seed: int, name: str, t: int, rows: int, cols: int, std=0.02) -> np.ndarray:
    """Seeded IQ2_XXS / IQ2_S / IQ3_S rows.  Every bit pattern of an IQ super-block is a valid encoding
    (grid indices, signs and scales all decode), so the payload is seeded random bytes and only the fp16
    d is chosen: |N(0, 1)| * std over the format's typical |grid * scale| (about 50 for the IQ2 types with
    their 1/8, 128 for IQ3_S), so the decoded weights have roughly the given spread."""
    bb = row_bytes(t, 256)
    blocks = random_bytes(seed, name, rows * (cols // 256) * bb).reshape(-1, bb)
    d = np.abs(normal(seed, name + ".d", (blocks.shape[0],))) * (std / (128.0 if t == PHX.IQ3_S else 50.0))
    blocks[:, :2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    return blocks.reshape(-1)


def quantized_normal(seed: int, name: str, t: int, rows: int, logical_cols: int, cols: int, std=0.02) -> np.ndarray:
    if t in IQ_TYPES:
        return iq_blocks(seed, name, t, rows, cols, std)
    out = np.empty(rows * row_bytes(t, cols), np.uint8)
    rc = lib().phx_synth_quantized_normal(seed, name.encode(), 0.0, std, t, rows, logical_cols, cols, out.ctypes.data)
    if rc:
        raise ValueError(f"quantized_normal {name}: {rc}")
    return out


def round_up(v: int, m: int) -> int:
    return (v + m - 1) // m * m


@lru_cache(maxsize=None)
def calibrated_bias(seed: int, E: int, k: int, kind: str, param: float) -> np.ndarray:
    """Router bias b[E] (logit units) whose top-k shares follow the target: 'zipf' (exponent param,
    over a seeded expert permutation) or 'hot' (expert 0 takes share param of the tokens)."""
    if kind == "zipf":
        rng = np.random.default_rng(seed)
        order = rng.permutation(E)
        w = 1.0 / np.arange(1, E + 1) ** param
        share = np.empty(E)
        share[order] = w / w.sum() * k
        # an expert serves a token at most once: cap shares at 0.95 and spread the excess
        for _ in range(64):
            over = share > 0.95
            if not over.any():
                break
            excess = (share[over] - 0.95).sum()
            share[over] = 0.95
            free = ~over
            share[free] += excess * share[free] / share[free].sum()
    elif kind == "hot":
        share = np.full(E, (k - param) / (E - 1))
        share[0] = param
    else:
        raise ValueError(kind)
    target = np.ascontiguousarray(share, np.float64)
    bias = np.zeros(E, np.float64)
    lib().phx_synth_calibrate_bias(seed, E, k, target.ctypes.data, 0.02, 4096, 60, bias.ctypes.data)
    return bias.astype(np.float32)


def make_layer(cfg: dict | str, layer: int = 0, weight_rule: int = 0, norms: str = "unit", seed: int | None = None,
               with_post: bool = True, experts: bool = True) -> dict:
    """One MoE layer (numpy arrays in GGUF byte layout) of a configuration.  experts=False leaves out
    the expert and shared-FFN weights (router-only uses); every other tensor is unchanged."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    seed = 1000 + cfg["idx"] if seed is None else seed
    d, E, k, nf = cfg["d"], cfg["E"], cfg["k"], cfg["nf"]
    gu, dn = cfg["gu"], cfg["dn"]
    dc = round_up(nf, block_elems(dn))
    p = f"blk.{layer}."
    L = dict(d=d, n_expert=E, n_used=k, n_ff=nf, down_cols=dc, eps=np.float32(1e-6).item(), gate_up_type=gu,
             down_type=dn, weight_rule=weight_rule, n_ff_shared=0, shared_type=0, seed=seed, layer=layer)
    L["gate_inp"] = normal(seed, p + "ffn_gate_inp.weight", (E, d), 0.0, 0.02)

    def vec(name, n):
        if norms == "unit":
            return np.ones(n, np.float32)
        return normal(seed, p + name, (n,), 1.0, 0.1)

    L["gate_inp_scale"] = vec("ffn_gate_inp.scale", d)
    L["down_scale"] = vec("ffn_down_exps.scale", E)
    L["pre_ffw_norm_2"] = vec("pre_ffw_norm_2.weight", d)
    L["post_ffw_norm_1"] = vec("post_ffw_norm_1.weight", d)
    L["post_ffw_norm_2"] = vec("post_ffw_norm_2.weight", d)
    if with_post:
        L["post_ffw_norm"] = vec("post_ffw_norm.weight", d)
    if experts:
        L["gate_up_exps"] = quantized_normal(seed, p + "ffn_gate_up_exps.weight", gu, E * 2 * nf, d, d)
        L["down_exps"] = quantized_normal(seed, p + "ffn_down_exps.weight", dn, E * d, nf, dc)
    if cfg.get("nff") and experts:
        nff, st = cfg["nff"], cfg["sh"]
        L["n_ff_shared"], L["shared_type"] = nff, st
        L["ffn_norm"] = vec("ffn_norm.weight", d)
        L["ffn_gate"] = quantized_normal(seed, p + "ffn_gate.weight", st, nff, d, d)
        L["ffn_up"] = quantized_normal(seed, p + "ffn_up.weight", st, nff, d, d)
        L["ffn_down"] = quantized_normal(seed, p + "ffn_down.weight", st, d, nff, round_up(nff, block_elems(st)))
    bias = None
    if cfg.get("zipf"):
        bias = calibrated_bias(seed, E, k, "zipf", cfg["zipf"])
    elif cfg.get("hot"):
        bias = calibrated_bias(seed, E, k, "hot", cfg["hot"])
    if bias is not None:
        m = BIAS_X / np.sqrt(d)  # the bias channel's router input, m = x * rinv / sqrt(d) with rinv ~ 1
        L["gate_inp"][:, d - 1] = bias / m
    L["biased"] = bias is not None
    return L


def make_stack(cfg: dict | str, n_layers: int | None = None) -> list[dict]:
    """The layers of a decode stack: layer i has its own router, router scale, norms and down
    scales (the blk.i. tensors, hot-expert bias included); the expert weights are generated once and
    shared in value by every layer.  Each upload still places its own copy in device memory, so one step
    through the stack reads n_layers distinct weight sets from HBM."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    n_layers = n_layers or cfg.get("layers", 1)
    base = make_layer(cfg, layer=0)
    layers = [base]
    for i in range(1, n_layers):
        L = make_layer(cfg, layer=i, experts=False)
        for key in ("gate_up_exps", "down_exps", "n_ff_shared", "shared_type", "ffn_norm", "ffn_gate", "ffn_up",
                    "ffn_down"):
            if key in base:
                L[key] = base[key]
        layers.append(L)
    return layers


def make_input(cfg: dict | str, T: int | None = None, seed: int | None = None, name: str = "x", biased=None) -> np.ndarray:
    """Activations x[T][d] ~ N(0, 1); with a biased router the last channel carries BIAS_X."""
    if isinstance(cfg, str):
        cfg = CONFIGS[cfg]
    seed = 1000 + cfg["idx"] if seed is None else seed
    T = cfg["T"] if T is None else T
    x = normal(seed, name, (T, cfg["d"]))
    if biased if biased is not None else (cfg.get("zipf") or cfg.get("hot")):
        x[:, -1] = BIAS_X
    return x
