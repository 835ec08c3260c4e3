"""ctypes binding of the CPU oracle (oracle/_build/liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg, as the checker (or the timed CPU baseline).  The product never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
# PHX_ORACLE_LIB names another build of oracle.c (tests/mutation_check.py loads planted-mistake copies)
LIB = Path(os.environ.get("PHX_ORACLE_LIB", HERE / "_build" / "liboracle.so"))


def build():
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)


class OrcLayer(C.Structure):
    _fields_ = [
        ("d", C.c_int), ("n_expert", C.c_int), ("n_used", C.c_int), ("n_ff", C.c_int), ("down_cols", C.c_int),
        ("eps", C.c_float), ("gate_up_type", C.c_int), ("down_type", C.c_int), ("weight_rule", C.c_int),
        ("gate_inp", C.c_void_p), ("gate_inp_scale", C.c_void_p), ("down_scale", C.c_void_p),
        ("pre_ffw_norm_2", C.c_void_p), ("post_ffw_norm_1", C.c_void_p), ("post_ffw_norm_2", C.c_void_p),
        ("gate_up_exps", C.c_void_p), ("down_exps", C.c_void_p),
        ("n_ff_shared", C.c_int), ("shared_type", C.c_int),
        ("ffn_norm", C.c_void_p), ("ffn_gate", C.c_void_p), ("ffn_up", C.c_void_p), ("ffn_down", C.c_void_p),
        ("post_ffw_norm", C.c_void_p),
    ]


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = C.CDLL(str(LIB))
        vp, i32, f32, i64 = C.c_void_p, C.c_int, C.c_float, C.c_int64
        L.orc_half_from_float.argtypes = [f32]
        L.orc_half_from_float.restype = C.c_uint16
        L.orc_half_to_float.argtypes = [C.c_uint16]
        L.orc_half_to_float.restype = f32
        L.orc_half_round.argtypes = [f32]
        L.orc_half_round.restype = f32
        L.orc_half_from_float_n.argtypes = [vp, vp, i64]
        L.orc_half_to_float_n.argtypes = [vp, vp, i64]
        L.orc_quantize_q8_0.argtypes = [vp, i32, vp, vp]
        L.orc_nearest_int.argtypes = [f32]
        L.orc_nearest_int.restype = i32
        L.orc_quantize_q8_k.argtypes = [vp, i32, vp, vp, vp]
        L.orc_row_bytes.argtypes = [i32, i32]
        L.orc_row_bytes.restype = i64
        L.orc_dequantize_row.argtypes = [i32, vp, i32, vp]
        L.orc_dequantize_row.restype = i32
        L.orc_dot_q4_0.argtypes = [vp, i32, vp, vp]
        L.orc_dot_q4_0.restype = f32
        L.orc_dot_q8_0.argtypes = [vp, i32, vp, vp]
        L.orc_dot_q8_0.restype = f32
        L.orc_dot_k.argtypes = [i32, vp, i32, vp, vp, vp]
        L.orc_dot_k.restype = f32
        L.orc_dot_iq.argtypes = [i32, vp, i32, vp, vp]
        L.orc_dot_iq.restype = f32
        L.orc_matvec.argtypes = [i32, vp, i32, i32, vp, vp, i32]
        L.orc_matvec.restype = i32
        L.orc_gelu.argtypes = [f32]
        L.orc_gelu.restype = f32
        L.orc_gelu_n.argtypes = [vp, vp, i64]
        L.orc_silu.argtypes = [f32]
        L.orc_silu.restype = f32
        L.orc_silu_n.argtypes = [vp, vp, i64]
        L.orc_rmsnorm.argtypes = [vp, i32, vp, f32, vp]
        L.orc_rms_scale.argtypes = [vp, i32, f32]
        L.orc_rms_scale.restype = f32
        L.orc_router.argtypes = [C.POINTER(OrcLayer), vp, vp, vp, vp]
        L.orc_combine.argtypes = [i32, i32, vp, vp, vp]
        L.orc_moe_token.argtypes = [C.POINTER(OrcLayer), vp, vp, vp, vp, vp, vp, vp, vp, i32]
        L.orc_shared_ffn_token.argtypes = [C.POINTER(OrcLayer), vp, vp, i32]
        L.orc_moe_block.argtypes = [C.POINTER(OrcLayer), i32, vp, vp, vp, vp, vp, i32]
        L.orc_residual.argtypes = [C.POINTER(OrcLayer), i32, vp, vp]
        L.orc_bucket.argtypes = [vp, i32, i32, i32, vp, vp]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def f32(a):
    return np.ascontiguousarray(a, np.float32)


def layer_struct(Ld: dict) -> OrcLayer:
    s = OrcLayer()
    for f in ("d", "n_expert", "n_used", "n_ff", "down_cols", "gate_up_type", "down_type"):
        setattr(s, f, int(Ld[f]))
    s.eps = Ld["eps"]
    s.weight_rule = int(Ld.get("weight_rule", 0))
    s.n_ff_shared = int(Ld.get("n_ff_shared", 0))
    s.shared_type = int(Ld.get("shared_type", 0))
    for f in ("gate_inp", "gate_inp_scale", "down_scale", "pre_ffw_norm_2", "post_ffw_norm_1", "post_ffw_norm_2",
              "gate_up_exps", "down_exps", "ffn_norm", "ffn_gate", "ffn_up", "ffn_down", "post_ffw_norm"):
        setattr(s, f, _p(Ld.get(f)))
    return s


# ---------------------------------------------------------------- element / row functions
def half_from_float(x):
    x = f32(x)
    h = np.empty(x.shape, np.uint16)
    lib().orc_half_from_float_n(x.ctypes.data, h.ctypes.data, x.size)
    return h


def half_to_float(h):
    h = np.ascontiguousarray(h, np.uint16)
    x = np.empty(h.shape, np.float32)
    lib().orc_half_to_float_n(h.ctypes.data, x.ctypes.data, h.size)
    return x


def quantize_q8_0(x):
    x = f32(x)
    n = x.size
    d = np.empty(n // 32, np.uint16)
    q = np.empty(n, np.int8)
    lib().orc_quantize_q8_0(x.ctypes.data, n, d.ctypes.data, q.ctypes.data)
    return d, q


def quantize_q8_k(x):
    x = f32(x)
    n = x.size
    d = np.empty(n // 256, np.float32)
    q = np.empty(n, np.int8)
    bs = np.empty(n // 16, np.int16)
    lib().orc_quantize_q8_k(x.ctypes.data, n, d.ctypes.data, q.ctypes.data, bs.ctypes.data)
    return d, q, bs


def nearest_int(f):
    return lib().orc_nearest_int(float(np.float32(f)))


def row_bytes(t, cols):
    return int(lib().orc_row_bytes(t, cols))


def dequantize_row(t, row, cols):
    row = np.ascontiguousarray(row, np.uint8)
    out = np.empty(cols, np.float32)
    rc = lib().orc_dequantize_row(t, row.ctypes.data, cols, out.ctypes.data)
    assert rc == 0
    return out


def matvec(t, w, rows, cols, x, nthreads=0):
    w = np.ascontiguousarray(w, np.uint8)
    x = f32(x)
    y = np.empty(rows, np.float32)
    rc = lib().orc_matvec(t, w.ctypes.data, rows, cols, x.ctypes.data, y.ctypes.data, nthreads)
    assert rc == 0, rc
    return y


def gelu(x):
    x = f32(x)
    y = np.empty_like(x)
    lib().orc_gelu_n(x.ctypes.data, y.ctypes.data, x.size)
    return y


def silu(x):
    x = f32(x)
    y = np.empty_like(x)
    lib().orc_silu_n(x.ctypes.data, y.ctypes.data, x.size)
    return y


def rmsnorm(x, w, eps):
    x, w = f32(x), f32(w)
    y = np.empty_like(x)
    lib().orc_rmsnorm(x.ctypes.data, x.size, w.ctypes.data, eps, y.ctypes.data)
    return y


def rms_scale(x, eps):
    x = f32(x)
    return lib().orc_rms_scale(x.ctypes.data, x.size, eps)


# ---------------------------------------------------------------- layer functions
def router(Ld, x):
    s = layer_struct(Ld)
    x = f32(x)
    logits = np.empty(Ld["n_expert"], np.float32)
    ids = np.empty(Ld["n_used"], np.int32)
    w = np.empty(Ld["n_used"], np.float32)
    lib().orc_router(C.byref(s), x.ctypes.data, logits.ctypes.data, ids.ctypes.data, w.ctypes.data)
    return logits, ids, w


def combine(yd, w):
    """acc[d] = sum over ranks j = 0..k-1, in order, of yd[j] * w[j] (GemmaCpu.cs:417-418)."""
    yd, w = f32(yd), f32(w)
    k, d = yd.shape
    acc = np.empty(d, np.float32)
    lib().orc_combine(k, d, yd.ctypes.data, w.ctypes.data, acc.ctypes.data)
    return acc


def moe_token(Ld, x, shared=None, nthreads=0):
    """out[d], ids[k], w[k], g[k][nf], u[k][nf], yd[k][d] of one token (GemmaCpu.MoeFfn)."""
    s = layer_struct(Ld)
    d, k, nf = Ld["d"], Ld["n_used"], Ld["n_ff"]
    x = f32(x)
    sh = None if shared is None else f32(shared)
    out = np.empty(d, np.float32)
    ids = np.empty(k, np.int32)
    w = np.empty(k, np.float32)
    g = np.empty((k, nf), np.float32)
    u = np.empty((k, nf), np.float32)
    yd = np.empty((k, d), np.float32)
    lib().orc_moe_token(C.byref(s), x.ctypes.data, _p(sh), out.ctypes.data, ids.ctypes.data, w.ctypes.data,
                        g.ctypes.data, u.ctypes.data, yd.ctypes.data, nthreads)
    return out, ids, w, g, u, yd


def shared_ffn(Ld, x, nthreads=0):
    s = layer_struct(Ld)
    x = f32(x)
    out = np.empty(Ld["d"], np.float32)
    lib().orc_shared_ffn_token(C.byref(s), x.ctypes.data, out.ctypes.data, nthreads)
    return out


def moe_block(Ld, x, shared=None, nthreads=0):
    s = layer_struct(Ld)
    x = f32(x)
    T = x.shape[0]
    sh = None if shared is None else f32(shared)
    out = np.empty_like(x)
    ids = np.empty((T, Ld["n_used"]), np.int32)
    w = np.empty((T, Ld["n_used"]), np.float32)
    lib().orc_moe_block(C.byref(s), T, x.ctypes.data, _p(sh), out.ctypes.data, ids.ctypes.data, w.ctypes.data,
                        nthreads)
    return out, ids, w


def residual(Ld, x, out):
    s = layer_struct(Ld)
    x = f32(x).copy()
    out = f32(out)
    lib().orc_residual(C.byref(s), x.shape[0], x.ctypes.data, out.ctypes.data)
    return x


def bucket(ids, E):
    ids = np.ascontiguousarray(ids, np.int32)
    T, k = ids.shape
    off = np.empty(E + 1, np.int32)
    perm = np.empty(T * k, np.int32)
    lib().orc_bucket(ids.ctypes.data, T, k, E, off.ctypes.data, perm.ctypes.data)
    return off, perm
