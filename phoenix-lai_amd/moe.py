"""ctypes binding of libphxmoe.so (include/phx_moe.h).

Error behaviour follows the reference host: a nonzero status raises the exception the C# side
maps it to (src/Vulkan.cs:194-208 device lost, src/Gpu.cs:851-852 bad arguments,
src/GemmaGpu.cs:189-190 unsupported layouts).
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent


class PHX:
    OK, ERR_ARG, ERR_OOM, ERR_UNSUPPORTED, ERR_DEVICE_LOST, ERR_HIP, ERR_FORMAT = 0, -1, -2, -3, -4, -5, -6
    F32, Q4_0, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K, IQ2_XXS, IQ3_S, IQ2_S = 0, 2, 8, 11, 12, 13, 14, 16, 21, 22
    WEIGHTS_SOFTMAX, WEIGHTS_CPUREF = 0, 1
    FLAG_DEVICE_PTRS, FLAG_ASYNC, FLAG_RESIDUAL, FLAG_EXACT_ROUTER, FLAG_FAST_MATH = 1, 2, 4, 8, 16
    FLAG_KEEP_INTERMEDIATES = 32
    KINDS = ["prologue", "router", "topk", "dispatch", "gate_up", "requant", "down", "combine", "shared"]
    MAX_EXPERTS, MAX_USED = 256, 16
    # activation quantizer modes (KernelsQuant.Mode, src/KernelsQuant.cs:13)
    QUANT_PLAIN, QUANT_SILU_MUL, QUANT_RMS_NORM, QUANT_GELU_MUL = 0, 1, 2, 3


class MoeError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"phx_moe error {code}: {msg}")
        self.code = code


class ArgumentError(MoeError, ValueError):
    pass


class NotSupportedError(MoeError):
    pass


class GpuDeviceLostError(MoeError):
    pass


class OutOfDeviceMemoryError(MoeError, MemoryError):
    """PHX_ERR_OOM: a device allocation failed (the context stays usable)."""


class InvalidDataError(MoeError, ValueError):
    """A malformed GGUF file (InvalidDataException in the reference, src/Gguf.cs:116-210)."""


def _raise(code: int, msg: str):
    if code == PHX.ERR_ARG:
        raise ArgumentError(code, msg)
    if code == PHX.ERR_UNSUPPORTED:
        raise NotSupportedError(code, msg)
    if code == PHX.ERR_DEVICE_LOST:
        raise GpuDeviceLostError(code, msg)
    if code == PHX.ERR_OOM:
        raise OutOfDeviceMemoryError(code, msg)
    if code == PHX.ERR_FORMAT:
        raise InvalidDataError(code, msg)
    raise MoeError(code, msg)


class LayerDesc(C.Structure):
    """phx_moe_layer_desc (include/phx_moe.h)."""

    _fields_ = [
        ("d", C.c_int32), ("n_expert", C.c_int32), ("n_used", C.c_int32), ("n_ff", C.c_int32),
        ("down_cols", C.c_int32), ("eps", C.c_float), ("gate_up_type", C.c_int32), ("down_type", C.c_int32),
        ("weight_rule", C.c_int32), ("n_ff_shared", C.c_int32), ("shared_type", C.c_int32), ("reserved", C.c_int32),
        ("gate_inp", C.c_void_p), ("gate_inp_scale", C.c_void_p), ("down_scale", C.c_void_p),
        ("pre_ffw_norm_2", C.c_void_p), ("post_ffw_norm_1", C.c_void_p), ("post_ffw_norm_2", C.c_void_p),
        ("gate_up_exps", C.c_void_p), ("down_exps", C.c_void_p), ("ffn_norm", C.c_void_p),
        ("ffn_gate", C.c_void_p), ("ffn_up", C.c_void_p), ("ffn_down", C.c_void_p), ("post_ffw_norm", C.c_void_p),
    ]

    @classmethod
    def from_layer(cls, L: dict) -> "LayerDesc":
        """Descriptor over the numpy arrays of a layer dict (see synth.make_layer); the dict must
        outlive every call that uses the descriptor."""
        def p(name):
            a = L.get(name)
            return None if a is None else a.ctypes.data
        d = cls()
        d.d, d.n_expert, d.n_used, d.n_ff = L["d"], L["n_expert"], L["n_used"], L["n_ff"]
        d.down_cols, d.eps = L["down_cols"], L["eps"]
        d.gate_up_type, d.down_type, d.weight_rule = L["gate_up_type"], L["down_type"], L.get("weight_rule", 0)
        d.n_ff_shared, d.shared_type = L.get("n_ff_shared", 0), L.get("shared_type", 0)
        for f in ("gate_inp", "gate_inp_scale", "down_scale", "pre_ffw_norm_2", "post_ffw_norm_1", "post_ffw_norm_2",
                  "gate_up_exps", "down_exps", "ffn_norm", "ffn_gate", "ffn_up", "ffn_down", "post_ffw_norm"):
            setattr(d, f, p(f))
        return d


def lib_path() -> Path:
    """libphxmoe.so in the package directory, or the file PHX_MOE_LIB names (an instrumented build)."""
    return Path(os.environ["PHX_MOE_LIB"]) if os.environ.get("PHX_MOE_LIB") else _HERE / "libphxmoe.so"


_LIB = None


def load_lib():
    """Load libphxmoe.so (built by __graft_entry__.build()); raise if it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    path = lib_path()
    if not path.exists():
        raise FileNotFoundError(f"{path} is not built: run __graft_entry__.build() (hipcc, gfx950)")
    lib = C.CDLL(str(path))
    vp, i32, u32, f32p, i32p = C.c_void_p, C.c_int, C.c_uint, C.POINTER(C.c_float), C.POINTER(C.c_int32)
    sig = {
        "phx_moe_create": (i32, [i32, C.POINTER(vp)]),
        "phx_moe_destroy": (None, [vp]),
        "phx_moe_last_error": (C.c_char_p, [vp]),
        "phx_moe_check_desc": (i32, [C.POINTER(LayerDesc)]),
        "phx_moe_layer_upload": (i32, [vp, i32, C.POINTER(LayerDesc)]),
        "phx_moe_ffn": (i32, [vp, i32, i32, vp, vp, vp, u32]),
        "phx_moe_ffn_noalloc": (i32, [vp, i32, i32, vp, vp, vp, u32]),
        "phx_moe_get_routing": (i32, [vp, vp, vp, vp, vp, vp]),
        "phx_moe_get_intermediates": (i32, [vp, vp, vp, vp]),
        "phx_moe_stack_capture": (i32, [vp, i32, i32, i32]),
        "phx_moe_stack_capture2": (i32, [vp, i32, i32, i32, u32]),
        "phx_moe_stack_run": (i32, [vp, vp, i32, u32]),
        "phx_moe_sync": (i32, [vp]),
        "phx_moe_graph_stats": (i32, [vp, C.POINTER(C.c_int64), C.POINTER(C.c_int64)]),
        "phx_moe_dev_alloc": (i32, [vp, C.c_uint64, C.POINTER(vp)]),
        "phx_moe_dev_free": (i32, [vp, vp]),
        "phx_moe_memcpy_h2d": (i32, [vp, vp, vp, C.c_uint64]),
        "phx_moe_memcpy_d2h": (i32, [vp, vp, vp, C.c_uint64]),
        "phx_moe_profile": (i32, [vp, i32]),
        "phx_moe_profile_read": (i32, [vp, C.POINTER(C.c_double), C.POINTER(C.c_int64)]),
        "phx_moe_selftest": (i32, [vp, i32, i32, f32p, f32p, f32p]),
        "phx_moe_fallback_count": (i32, [vp, i32p]),
        "phx_moe_stream_read": (i32, [vp, vp, C.c_uint64, i32, C.POINTER(C.c_double)]),
        "phx_moe_stream_copy": (i32, [vp, vp, vp, C.c_uint64, i32, C.POINTER(C.c_double)]),
        "phx_quant_q8_0": (i32, [vp, i32, vp, vp, i32, i32, C.c_float, vp, vp]),
        "phx_quant_q8_k": (i32, [vp, i32, vp, vp, i32, i32, C.c_float, vp, vp, vp]),
        "phx_norm_add": (i32, [vp, vp, vp, vp, i32, i32, C.c_float, C.c_float, vp, vp, vp]),
        "phx_matvec": (i32, [vp, i32, vp, i32, i32, i32, vp, vp, vp]),
        "phx_weight_upload": (i32, [vp, i32, i32, i32, vp, C.POINTER(vp)]),
        "phx_weight_free": (None, [vp, vp]),
        "phx_matmul": (i32, [vp, vp, i32, vp, vp, vp]),
        "phx_matmul_k": (i32, [vp, vp, i32, vp, vp, vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


class DeviceBuffer:
    def __init__(self, ctx: "MoeContext", nbytes: int):
        self.ctx, self.nbytes = ctx, nbytes
        p = C.c_void_p()
        ctx._check(ctx.lib.phx_moe_dev_alloc(ctx.h, nbytes, C.byref(p)))
        self.ptr = p.value

    def upload(self, arr: np.ndarray):
        arr = np.ascontiguousarray(arr)
        if arr.nbytes > self.nbytes:
            raise ArgumentError(PHX.ERR_ARG, f"upload of {arr.nbytes} bytes into a {self.nbytes}-byte buffer")
        self.ctx._check(self.ctx.lib.phx_moe_memcpy_h2d(self.ctx.h, self.ptr, arr.ctypes.data, arr.nbytes))

    def download(self, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        if out.nbytes > self.nbytes:
            raise ArgumentError(PHX.ERR_ARG, f"download of {out.nbytes} bytes from a {self.nbytes}-byte buffer")
        self.ctx._check(self.ctx.lib.phx_moe_memcpy_d2h(self.ctx.h, out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self):
        if self.ptr:
            self.ctx._check(self.ctx.lib.phx_moe_dev_free(self.ctx.h, self.ptr))
            self.ptr = None


class MoeContext:
    """A libphxmoe context on one HIP device (GpuDevice + the MoE parts of GemmaGpu)."""

    def __init__(self, device: int = 0):
        self.lib = load_lib()
        h = C.c_void_p()
        rc = self.lib.phx_moe_create(device, C.byref(h))
        if rc:
            _raise(rc, f"phx_moe_create({device}) failed")
        self.h = h.value
        self.layers: dict[int, dict] = {}

    def close(self):
        if self.h:
            self.lib.phx_moe_destroy(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc: int):
        if rc:
            msg = self.lib.phx_moe_last_error(self.h).decode(errors="replace") if self.h else ""
            _raise(rc, msg)

    # ------------------------------------------------------------------ layers
    def upload(self, layer: int, L: dict):
        desc = LayerDesc.from_layer(L)
        self._check(self.lib.phx_moe_layer_upload(self.h, layer, C.byref(desc)))
        self.layers[layer] = {k: L[k] for k in ("d", "n_expert", "n_used", "n_ff")}

    def ffn(self, layer: int, x: np.ndarray, shared: np.ndarray | None = None, residual: bool = False,
            exact_router: bool = False, fast_math: bool = False, keep_intermediates: bool = False) -> np.ndarray:
        """out[T][d] of one MoE FFN block on host arrays; with residual, returns (out, x + rmsnorm(out) * post).
        fast_math: the tolerance mode of the prefill-sized expert products (PHX_FLAG_FAST_MATH).
        keep_intermediates: store g and u for intermediates() (PHX_FLAG_KEEP_INTERMEDIATES; the
        prefill-sized Q4_0 / Q8_0 products skip those stores without it)."""
        x = _f32(x)
        if residual:
            x = x.copy()
        T, d = x.shape
        out = np.empty_like(x)
        sh = None if shared is None else _f32(shared)
        flags = (PHX.FLAG_RESIDUAL if residual else 0) | (PHX.FLAG_EXACT_ROUTER if exact_router else 0) | \
            (PHX.FLAG_FAST_MATH if fast_math else 0) | (PHX.FLAG_KEEP_INTERMEDIATES if keep_intermediates else 0)
        self._last_layer, self._last_T = layer, T
        self._check(self.lib.phx_moe_ffn(self.h, layer, T, x.ctypes.data, None if sh is None else sh.ctypes.data,
                                         out.ctypes.data, flags))
        return (out, x) if residual else out

    def ffn_device(self, layer: int, T: int, x_ptr: int, shared_ptr, out_ptr: int, flags: int = 0):
        self._last_layer, self._last_T = layer, T
        self._check(self.lib.phx_moe_ffn(self.h, layer, T, x_ptr, shared_ptr, out_ptr, flags | PHX.FLAG_DEVICE_PTRS))

    def ffn_noalloc_device(self, layer: int, T: int, x_ptr: int, shared_ptr, out_ptr: int, flags: int = 0):
        """phx_moe_ffn_noalloc: ffn_device with the workspace in the library's fixed scratch array."""
        self._last_layer, self._last_T = layer, T
        self._check(self.lib.phx_moe_ffn_noalloc(self.h, layer, T, x_ptr, shared_ptr, out_ptr, flags))

    # the reference's three call sites
    def RecordMoe(self, layer: int, x: np.ndarray, shared: np.ndarray) -> np.ndarray:
        """src/GemmaGpu.cs:656-669: one decode token, the shared MLP's output given."""
        return self.ffn(layer, np.reshape(x, (1, -1)), np.reshape(shared, (1, -1)))[0]

    def RecordFfnMoe(self, layer: int, x: np.ndarray) -> np.ndarray:
        """src/GemmaGpu.cs:683-704: one decode token, the layer's dense shared FFN computed too."""
        return self.ffn(layer, np.reshape(x, (1, -1)))[0]

    def RecordMoeRows(self, layer: int, x: np.ndarray, shared: np.ndarray | None) -> np.ndarray:
        """src/GemmaGpu.cs:850-882: T prompt rows (shared: the shared MLP's down outputs)."""
        return self.ffn(layer, x, shared)

    def routing(self):
        """(ids [T][k], weights [T][k], offsets [E+1], perm [T*k], logits [T][E]) of the last call."""
        lay = self._last_dims()
        T, k, E = self._last_T, lay["n_used"], lay["n_expert"]
        ids = np.empty((T, k), np.int32)
        w = np.empty((T, k), np.float32)
        off = np.empty(E + 1, np.int32)
        perm = np.empty(T * k, np.int32)
        logits = np.empty((T, E), np.float32)
        self._check(self.lib.phx_moe_get_routing(self.h, ids.ctypes.data, w.ctypes.data, off.ctypes.data,
                                                 perm.ctypes.data, logits.ctypes.data))
        return ids, w, off, perm, logits

    def intermediates(self):
        lay = self._last_dims()
        n = self._last_T * lay["n_used"]
        g = np.empty((n, lay["n_ff"]), np.float32)
        u = np.empty_like(g)
        yd = np.empty((n, lay["d"]), np.float32)
        self._check(self.lib.phx_moe_get_intermediates(self.h, g.ctypes.data, u.ctypes.data, yd.ctypes.data))
        return g, u, yd

    def _last_dims(self):
        return self.layers[self._last_layer]

    # the last call, for routing()/intermediates()
    _last_T = 0
    _last_layer = 0

    # ------------------------------------------------------------------ stack (HIP graph)
    def stack_capture(self, first: int, n_layers: int, T: int, exact_router: bool = False):
        self._check(self.lib.phx_moe_stack_capture2(self.h, first, n_layers, T,
                                                    PHX.FLAG_EXACT_ROUTER if exact_router else 0))
        self._stack_last = first + n_layers - 1

    def stack_run(self, x: np.ndarray) -> np.ndarray:
        x = _f32(x).copy()
        self._last_layer, self._last_T = self._stack_last, x.shape[0]
        self._check(self.lib.phx_moe_stack_run(self.h, x.ctypes.data, x.shape[0], 0))
        return x

    # ------------------------------------------------------------------ misc
    def sync(self):
        self._check(self.lib.phx_moe_sync(self.h))

    def alloc(self, nbytes: int) -> DeviceBuffer:
        return DeviceBuffer(self, nbytes)

    def profile(self, enable: bool):
        self._check(self.lib.phx_moe_profile(self.h, 1 if enable else 0))

    def profile_read(self) -> dict:
        ms = (C.c_double * len(PHX.KINDS))()
        n = (C.c_int64 * len(PHX.KINDS))()
        self._check(self.lib.phx_moe_profile_read(self.h, ms, n))
        return {k: (ms[i], n[i]) for i, k in enumerate(PHX.KINDS)}

    def selftest(self, op: int, a: np.ndarray, b: np.ndarray | None = None) -> np.ndarray:
        a = _f32(a).ravel()
        b = np.zeros_like(a) if b is None else _f32(b).ravel()
        out = np.empty_like(a)
        fp = C.POINTER(C.c_float)
        self._check(self.lib.phx_moe_selftest(self.h, op, a.size, a.ctypes.data_as(fp), b.ctypes.data_as(fp),
                                              out.ctypes.data_as(fp)))
        return out

    def stream_read_ms(self, buf: "DeviceBuffer", iters: int = 20) -> float:
        ms = C.c_double()
        self._check(self.lib.phx_moe_stream_read(self.h, buf.ptr, buf.nbytes, iters, C.byref(ms)))
        return ms.value

    def stream_copy_ms(self, dst: "DeviceBuffer", src: "DeviceBuffer", nbytes: int, iters: int = 2) -> float:
        ms = C.c_double()
        self._check(self.lib.phx_moe_stream_copy(self.h, dst.ptr, src.ptr, nbytes, iters, C.byref(ms)))
        return ms.value

    def quant_device(self, k_quant: bool, mode: int, x_ptr: int, aux_ptr, rows: int, n: int, eps: float,
                     qs_ptr: int, d_ptr: int, bsums_ptr=None):
        """Enqueue phx_quant_q8_0 (k_quant False) or phx_quant_q8_k on device buffers (sync() waits)."""
        if k_quant:
            rc = self.lib.phx_quant_q8_k(self.h, mode, x_ptr, aux_ptr, rows, n, eps, qs_ptr, d_ptr, bsums_ptr)
        else:
            rc = self.lib.phx_quant_q8_0(self.h, mode, x_ptr, aux_ptr, rows, n, eps, qs_ptr, d_ptr)
        self._check(rc)

    def _quant(self, k_quant: bool, mode: int, x: np.ndarray, aux, eps: float):
        x = _f32(x)
        x2 = x.reshape(1, -1) if x.ndim == 1 else x
        rows, n = x2.shape
        bufs = [self.alloc(max(x2.nbytes, 16))]
        bufs[0].upload(x2)
        aux_ptr = None
        if aux is not None:
            a = _f32(aux)
            bufs.append(self.alloc(max(a.nbytes, 16)))
            bufs[-1].upload(a)
            aux_ptr = bufs[-1].ptr
        nd = rows * n // (256 if k_quant else 32)
        qs, d = self.alloc(rows * n), self.alloc(nd * (4 if k_quant else 2))
        bs = self.alloc(rows * n // 16 * 2) if k_quant else None
        bufs += [qs, d] + ([bs] if bs else [])
        try:
            self.quant_device(k_quant, mode, bufs[0].ptr, aux_ptr, rows, n, eps, qs.ptr, d.ptr, bs.ptr if bs else None)
            self.sync()
            out = [qs.download((rows, n), np.int8),
                   d.download((rows, n // (256 if k_quant else 32)), np.float32 if k_quant else np.uint16)]
            if k_quant:
                out.append(bs.download((rows, n // 16), np.int16))
        finally:
            for b in bufs:
                b.free()
        if x.ndim == 1:
            out = [o[0] for o in out]
        return tuple(out)

    def Q80(self, mode: int, x: np.ndarray, aux: np.ndarray | None = None, eps: float = 1e-6):
        """KernelsQuant.Q80 (src/KernelsQuant.cs:133-170) on host arrays: (qs int8, d fp16 bits) per row."""
        return self._quant(False, mode, x, aux, eps)

    def Q8K(self, mode: int, x: np.ndarray, aux: np.ndarray | None = None, eps: float = 1e-6):
        """KernelsQuant.Q8K (src/KernelsQuant.cs:60-128) on host arrays: (qs int8, d f32, bsums int16) per row."""
        return self._quant(True, mode, x, aux, eps)

    def NormAdd(self, x: np.ndarray, y: np.ndarray, w: np.ndarray, eps: float = 1e-6, s: float = 1.0,
                w2: np.ndarray | None = None):
        """KernelsGemma.NormAdd / NormAddQuant (src/KernelsGemma.cs:126-226) on host arrays: returns the new
        x, and with w2 also (qs int8, d fp16 bits) of rmsnorm(x_new, w2)."""
        x = _f32(x)
        x2 = x.reshape(1, -1) if x.ndim == 1 else x
        rows, n = x2.shape
        y, w = _f32(y), _f32(w)
        if y.size != x2.size or w.size != n or (w2 is not None and _f32(w2).size != n):
            raise ArgumentError(PHX.ERR_ARG, f"norm_add: y has {y.size}, w {w.size} values for {rows} rows of {n}")
        bufs = [self.alloc(x2.nbytes), self.alloc(x2.nbytes), self.alloc(n * 4)]
        for b, a in zip(bufs, (x2, y, w)):
            b.upload(a)
        if w2 is not None:
            bufs += [self.alloc(n * 4), self.alloc(rows * n), self.alloc(rows * n // 32 * 2)]
            bufs[3].upload(_f32(w2))
        try:
            self._check(self.lib.phx_norm_add(self.h, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, rows, n, eps, s,
                                              bufs[3].ptr if w2 is not None else None,
                                              bufs[4].ptr if w2 is not None else None,
                                              bufs[5].ptr if w2 is not None else None))
            self.sync()
            out = [bufs[0].download((rows, n))]
            if w2 is not None:
                out += [bufs[4].download((rows, n), np.int8), bufs[5].download((rows, n // 32), np.uint16)]
        finally:
            for b in bufs:
                b.free()
        if x.ndim == 1:
            out = [o[0] for o in out]
        return out[0] if w2 is None else tuple(out)

    def MatVec(self, wtype: int, w: np.ndarray, rows: int, cols: int, xq: np.ndarray, xd: np.ndarray) -> np.ndarray:
        """GemmaGpu.MatVec for Q4_0 / Q8_0 weights (src/GemmaGpu.cs:463-476) on host arrays: w the GGUF rows
        (bytes), xq / xd the Q8_0 input rows as Q80 returns them; y [T][rows] f32."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        bb = {PHX.Q4_0: 18, PHX.Q8_0: 34}.get(wtype)
        if bb is not None and (cols % 32 or w.size != rows * (cols // 32) * bb):
            raise ArgumentError(PHX.ERR_ARG, f"weight bytes {w.size} != {rows} rows x {cols // 32} blocks x {bb}")
        xq = np.ascontiguousarray(xq, dtype=np.int8)
        xd = np.ascontiguousarray(xd, dtype=np.uint16)
        if cols <= 0 or xq.size % cols or xd.size * 32 != xq.size:
            raise ArgumentError(PHX.ERR_ARG, f"input of {xq.size} quants and {xd.size} scales for {cols} columns")
        xq = xq.reshape(-1, cols)
        xd = xd.reshape(xq.shape[0], cols // 32)
        T = xq.shape[0]
        bufs = [self.alloc(w.nbytes), self.alloc(xq.nbytes), self.alloc(xd.nbytes), self.alloc(T * rows * 4)]
        for b, a in zip(bufs, (w, xq, xd)):
            b.upload(a)
        try:
            self._check(self.lib.phx_matvec(self.h, wtype, bufs[0].ptr, rows, cols, T, bufs[1].ptr, bufs[2].ptr,
                                            bufs[3].ptr))
            self.sync()
            return bufs[3].download((T, rows))
        finally:
            for b in bufs:
                b.free()

    def weight_upload(self, wtype: int, w: np.ndarray, rows: int, cols: int) -> int:
        """phx_weight_upload (GemmaGpu.UploadW): GGUF rows from host memory, repacked on the device once;
        returns the handle for matmul_device / weight_free."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        be, bb = {PHX.Q4_0: (32, 18), PHX.Q8_0: (32, 34), PHX.Q3_K: (256, 110), PHX.Q4_K: (256, 144), PHX.Q5_K: (256, 176),
                  PHX.Q6_K: (256, 210)}.get(wtype, (32, 0))
        if cols <= 0 or cols % be or w.size != rows * (cols // be) * bb:
            raise ArgumentError(PHX.ERR_ARG, f"weight bytes {w.size} != {rows} rows x {cols // be} blocks x {bb}")
        h = C.c_void_p()
        self._check(self.lib.phx_weight_upload(self.h, wtype, rows, cols, w.ctypes.data, C.byref(h)))
        return h.value

    def weight_free(self, handle: int):
        self.lib.phx_weight_free(self.h, handle)

    def matmul_device(self, handle: int, T: int, xq_ptr: int, xd_ptr: int, y_ptr: int):
        """phx_matmul (KernelsPrefill.MatMulQ4Q8Tile as GemmaGpu.Mm records it), asynchronous."""
        self._check(self.lib.phx_matmul(self.h, handle, T, xq_ptr, xd_ptr, y_ptr))

    def MatMul(self, handle: int, rows: int, cols: int, xq: np.ndarray, xd: np.ndarray) -> np.ndarray:
        """GemmaGpu.Mm on host arrays: y [T][rows] f32 from T Q8_0 rows (as Q80 returns them)."""
        xq = np.ascontiguousarray(xq, dtype=np.int8).reshape(-1, cols)
        xd = np.ascontiguousarray(xd, dtype=np.uint16).reshape(xq.shape[0], cols // 32)
        T = xq.shape[0]
        bufs = [self.alloc(xq.nbytes), self.alloc(xd.nbytes), self.alloc(T * rows * 4)]
        try:
            bufs[0].upload(xq)
            bufs[1].upload(xd)
            self.matmul_device(handle, T, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr)
            self.sync()
            return bufs[2].download((T, rows))
        finally:
            for b in bufs:
                b.free()

    def matmul_k_device(self, handle: int, T: int, xq_ptr: int, xd_ptr: int, y_ptr: int):
        """phx_matmul_k (KernelsK.MatVec as GemmaGpu.MatVec records it for K-quant weights), asynchronous."""
        self._check(self.lib.phx_matmul_k(self.h, handle, T, xq_ptr, xd_ptr, y_ptr))

    def MatMulK(self, handle: int, rows: int, cols: int, xq: np.ndarray, xd: np.ndarray) -> np.ndarray:
        """GemmaGpu.MatVec for a Q4_K / Q6_K weight on host arrays: y [T][rows] f32 from T Q8_K rows (qs and
        d as Q8K returns them; the block sums are formed on the device)."""
        if cols <= 0 or cols % 256:
            raise ArgumentError(PHX.ERR_ARG, f"cols {cols} is not a multiple of 256")
        xq = np.ascontiguousarray(xq, dtype=np.int8)
        xd = np.ascontiguousarray(xd, dtype=np.float32)
        if xq.size % cols or xd.size * 256 != xq.size:
            raise ArgumentError(PHX.ERR_ARG, f"input of {xq.size} quants and {xd.size} scales for {cols} columns")
        xq = xq.reshape(-1, cols)
        T = xq.shape[0]
        bufs = [self.alloc(xq.nbytes), self.alloc(xd.nbytes), self.alloc(T * rows * 4)]
        try:
            bufs[0].upload(xq)
            bufs[1].upload(xd)
            self.matmul_k_device(handle, T, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr)
            self.sync()
            return bufs[2].download((T, rows))
        finally:
            for b in bufs:
                b.free()

    def stack_run_device(self, x_ptr: int, T: int):
        """Replay the captured stack on a device-resident x (async; sync() waits)."""
        self._check(self.lib.phx_moe_stack_run(self.h, x_ptr, T, PHX.FLAG_DEVICE_PTRS | PHX.FLAG_ASYNC))

    def graph_stats(self) -> tuple[int, int]:
        """(host-buffer calls that replayed a cached graph, calls that captured one)"""
        h, m = C.c_int64(), C.c_int64()
        self._check(self.lib.phx_moe_graph_stats(self.h, C.byref(h), C.byref(m)))
        return h.value, m.value

    def fallback_counts(self) -> tuple[int, int]:
        """(norm sums re-summed sequentially, decode tokens routed through the exact router)"""
        c = (C.c_int32 * 2)()
        self._check(self.lib.phx_moe_fallback_count(self.h, c))
        return c[0], c[1]
