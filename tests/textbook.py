"""float64 "textbook" MoE FFN layer in numpy, the second reading of the algorithm the oracle is
checked against.  Weights are decoded by gguf_spec (not the oracle), dot products are exact float64
sums, and only the parts that define the reference's numbers are kept:

- activation quantization before every quantized matvec, written from the closed forms of
  CpuRef.QuantizeQ8_0 (CpuRef.cs:49-67: d = amax/127, q = round half away from zero of x/d, d stored
  as fp16) and CpuRef.QuantizeQ8_K (CpuRefKQuants.cs:53-86: the signed value of largest |x|, first
  index on ties, sets iscale = -127/max, q = round half even, d = 1/iscale), with numpy's own fp16;
- GELU as the tanh approximation (Hendrycks & Gimpel) evaluated in float64 on fp16(x) and rounded to
  fp16 (the table semantics of CpuRefGemma.cs:83-92), identity above 10 and zero below -10;
- RMSNorm, router softmax and top-k as textbook formulas (GemmaCpu.cs:376-422).
"""
import numpy as np

import gguf_spec as G

F16 = np.float16


def fp16(x):
    return np.asarray(x, np.float32).astype(F16).astype(np.float32)


def round_half_away(v: np.ndarray) -> np.ndarray:
    v = np.asarray(v, np.float32)
    t = np.trunc(v)
    frac = np.abs(v - t)  # exact for |v| < 2^23
    return (t + np.sign(v) * (frac >= 0.5)).astype(np.int32)


def q8_0(x: np.ndarray):
    """(d fp16 as float32 [nb], q int32 [n]) of x (float32)."""
    xb = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        idv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, np.float32(1)), np.float32(0)).astype(np.float32)
    q = round_half_away((xb * idv[:, None]).astype(np.float32))
    return fp16(d), q.reshape(-1)


def q8_k(x: np.ndarray):
    """(d float32 [nb], q int32 [n], bsums int32 [n/16]) of x (float32)."""
    xb = np.asarray(x, np.float32).reshape(-1, 256)
    nb = xb.shape[0]
    d = np.zeros(nb, np.float32)
    q = np.zeros((nb, 256), np.int32)
    for b in range(nb):
        i = int(np.argmax(np.abs(xb[b])))  # first index of the largest |x|
        mx = xb[b, i]
        if mx == 0:
            continue
        iscale = np.float32(-127) / mx
        q[b] = np.minimum(127, np.rint((iscale * xb[b]).astype(np.float32))).astype(np.int32)
        d[b] = np.float32(1) / iscale
    return d, q.reshape(-1), q.reshape(-1, 16).sum(axis=1)


def act_dequant(t: int, x: np.ndarray) -> np.ndarray:
    """The activation values the reference's matvec of weight type t actually multiplies (float64)."""
    x = np.asarray(x, np.float32)
    if t == 0:
        return x.astype(np.float64)
    if t in (2, 8):
        d, q = q8_0(x)
        return (q.reshape(-1, 32) * d[:, None].astype(np.float64)).reshape(-1)
    d, q, _ = q8_k(x)
    return (q.reshape(-1, 256) * d[:, None].astype(np.float64)).reshape(-1)


def weights(t: int, w: np.ndarray, rows: int, cols: int) -> np.ndarray:
    if t == 0:
        return np.asarray(w).view(np.float32).reshape(rows, cols).astype(np.float64)
    rb = len(w) // rows
    w = np.asarray(w, np.uint8).reshape(rows, rb)
    return np.stack([G.DEQUANT[t](w[r], cols) for r in range(rows)]).astype(np.float64)


def matvec(t: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray) -> np.ndarray:
    return weights(t, w, rows, cols) @ act_dequant(t, x)


def gelu(x: np.ndarray) -> np.ndarray:
    x = np.asarray(x, np.float32)
    h = fp16(x).astype(np.float64)
    g = 0.5 * h * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (h + 0.044715 * h ** 3)))
    out = fp16(g.astype(np.float32))
    out = np.where(x >= 10, x, out)
    return np.where(x <= -10, np.float32(0), out).astype(np.float32)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + eps) * np.asarray(w, np.float64)


def router_logits(L: dict, x: np.ndarray) -> np.ndarray:
    d = L["d"]
    x = np.asarray(x, np.float64)
    inp = x / np.sqrt(np.mean(x * x) + L["eps"]) / np.sqrt(d) * L["gate_inp_scale"].astype(np.float64)
    return L["gate_inp"].astype(np.float64) @ inp


def topk(logits: np.ndarray, k: int) -> np.ndarray:
    """k largest, ties to the lower index."""
    order = np.lexsort((np.arange(len(logits)), -np.asarray(logits, np.float64)))
    return order[:k].astype(np.int32)


def weights_softmax(sel: np.ndarray) -> np.ndarray:
    e = np.exp(sel - sel[0])
    return e / e.sum()


def weights_cpuref(sel: np.ndarray) -> np.ndarray:
    """GemmaCpu.cs:406-407 as written: sel[0] becomes exp(0) = 1 in place, so every later term
    subtracts 1 instead of the top logit."""
    e = np.concatenate([[1.0], np.exp(sel[1:] - 1.0)])
    return e / e.sum()


def moe_token(L: dict, x: np.ndarray, shared=None, ids=None):
    """(out, ids, w, g, u, yd) of GemmaCpu.MoeFfn for one token, in float64.  With ids given, the
    experts are taken from there (so near-ties between fp32 and fp64 logits cannot flip the choice)."""
    d, nf, k, dc = L["d"], L["n_ff"], L["n_used"], L["down_cols"]
    eps = L["eps"]
    logits = router_logits(L, x)
    if ids is None:
        ids = topk(logits, k)
    sel = logits[ids]
    wr = weights_cpuref(sel) if L.get("weight_rule", 0) == 1 else weights_softmax(sel)
    w = wr * L["down_scale"][ids].astype(np.float64)
    moe_in = rmsnorm(x, L["pre_ffw_norm_2"], eps).astype(np.float32)
    gu_rb = len(L["gate_up_exps"]) // L["n_expert"]
    dn_rb = len(L["down_exps"]) // L["n_expert"]
    acc = np.zeros(d)
    g_all, u_all, yd_all = [], [], []
    for j, e in enumerate(ids):
        gu = matvec(L["gate_up_type"], L["gate_up_exps"][e * gu_rb:(e + 1) * gu_rb], 2 * nf, d, moe_in)
        g, u = gu[:nf], gu[nf:]
        eg = np.zeros(dc, np.float32)
        eg[:nf] = (gelu(g.astype(np.float32)).astype(np.float64) * u).astype(np.float32)
        yd = matvec(L["down_type"], L["down_exps"][e * dn_rb:(e + 1) * dn_rb], d, dc, eg)
        acc += yd * np.float64(np.float32(w[j]))
        g_all.append(g), u_all.append(u), yd_all.append(yd)
    out = rmsnorm(acc, L["post_ffw_norm_2"], eps)
    if shared is not None:
        out = out + rmsnorm(shared, L["post_ffw_norm_1"], eps)
    return out, np.asarray(ids), w, np.array(g_all), np.array(u_all), np.array(yd_all)


def shared_ffn(L: dict, x: np.ndarray) -> np.ndarray:
    d, nff, t = L["d"], L["n_ff_shared"], L["shared_type"]
    n = rmsnorm(x, L["ffn_norm"], L["eps"]).astype(np.float32)
    g = matvec(t, L["ffn_gate"], nff, d, n)
    u = matvec(t, L["ffn_up"], nff, d, n)
    eg = (gelu(g.astype(np.float32)).astype(np.float64) * u).astype(np.float32)
    dcs = len(L["ffn_down"]) // d * G.BLOCK[t][0] // G.BLOCK[t][1] if t else nff
    if dcs > nff:
        eg = np.concatenate([eg, np.zeros(dcs - nff, np.float32)])
    return matvec(t, L["ffn_down"], d, dcs, eg)
