"""GGUF ingestion through libphxmoe.so's reader (include/phx_gguf.h), shaped like the reference's GgufFile
(src/Gguf.cs:92-239) and the MoE part of GemmaConfig.FromGguf (src/GemmaCpu.cs:66-74): Open, Version,
Alignment, DataOffset, Keys, Tensors, TensorsByName, Has, GetString, GetInt, GetFloat, GetArray.
Errors raise the classes of moe.py (InvalidDataError for a malformed file, as GgufFile.Load throws
InvalidDataException).  Host-only: no GPU is needed to read a file."""
from __future__ import annotations

import ctypes as C

import numpy as np

from .moe import PHX, LayerDesc, _raise, load_lib

_SIGS = False


class TensorInfo(C.Structure):
    _fields_ = [("name", C.c_char_p), ("n_dims", C.c_int32), ("dims", C.c_int64 * 4), ("type", C.c_int32),
                ("offset", C.c_int64), ("size_bytes", C.c_int64), ("data", C.c_void_p)]


class ModelConfig(C.Structure):
    _fields_ = [("arch", C.c_char * 32), ("n_embd", C.c_int32), ("n_layer", C.c_int32), ("n_expert", C.c_int32),
                ("n_expert_used", C.c_int32), ("n_ff_exp", C.c_int32), ("eps", C.c_float)]


def _lib():
    global _SIGS
    lib = load_lib()
    if not _SIGS:
        vp, i32, i64, u32 = C.c_void_p, C.c_int, C.c_int64, C.c_uint32
        sig = {
            "phx_gguf_open": (i32, [C.c_char_p, C.POINTER(vp), C.c_char_p, C.c_size_t]),
            "phx_gguf_close": (None, [vp]),
            "phx_gguf_last_error": (C.c_char_p, [vp]),
            "phx_gguf_version": (u32, [vp]),
            "phx_gguf_n_tensors": (i64, [vp]),
            "phx_gguf_n_kv": (i64, [vp]),
            "phx_gguf_data_offset": (i64, [vp]),
            "phx_gguf_alignment": (C.c_int32, [vp]),
            "phx_gguf_key_at": (C.c_char_p, [vp, i64]),
            "phx_gguf_value_type": (i32, [vp, C.c_char_p, C.POINTER(C.c_int32), C.POINTER(i64)]),
            "phx_gguf_get_int": (i32, [vp, C.c_char_p, C.POINTER(i64)]),
            "phx_gguf_get_float": (i32, [vp, C.c_char_p, C.POINTER(C.c_float)]),
            "phx_gguf_get_string": (i32, [vp, C.c_char_p, C.POINTER(C.c_void_p), C.POINTER(C.c_uint64)]),
            "phx_gguf_get_array_int": (i32, [vp, C.c_char_p, i64, C.POINTER(i64)]),
            "phx_gguf_get_array_float": (i32, [vp, C.c_char_p, i64, C.POINTER(C.c_double)]),
            "phx_gguf_tensor_at": (i32, [vp, i64, C.POINTER(TensorInfo)]),
            "phx_gguf_find_tensor": (i32, [vp, C.c_char_p, C.POINTER(TensorInfo)]),
            "phx_gguf_moe_config": (i32, [vp, C.POINTER(ModelConfig)]),
            "phx_gguf_layer_desc": (i32, [vp, i32, i32, i32, C.POINTER(LayerDesc)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        _SIGS = True
    return lib


class GgufTensor:
    """GgufTensor (src/Gguf.cs:77-90): Dims with ne[0] first, Type (GgmlType), Offset, SizeBytes, Data (address)."""

    def __init__(self, info: TensorInfo, owner: "GgufFile"):
        self.Name = info.name.decode()
        self.Dims = [int(info.dims[i]) for i in range(info.n_dims)]
        self.Type = int(info.type)
        self.Offset = int(info.offset)
        self.SizeBytes = int(info.size_bytes)
        self.Data = int(info.data)
        self._owner = owner

    @property
    def ElementCount(self) -> int:
        return int(np.prod(self.Dims))

    def bytes(self) -> np.ndarray:
        """The tensor's bytes as a read-only uint8 view of the mapping (valid while the file is open)."""
        buf = (C.c_uint8 * self.SizeBytes).from_address(self.Data)
        a = np.frombuffer(buf, np.uint8)
        a.flags.writeable = False
        return a


class GgufFile:
    def __init__(self, path: str):
        self.lib = _lib()
        h = C.c_void_p()
        err = C.create_string_buffer(512)
        rc = self.lib.phx_gguf_open(str(path).encode(), C.byref(h), err, 512)
        if rc:
            _raise(rc, err.value.decode(errors="replace"))
        self.h = h.value
        self.Path = str(path)
        self.Version = int(self.lib.phx_gguf_version(self.h))
        self.Alignment = int(self.lib.phx_gguf_alignment(self.h))
        self.DataOffset = int(self.lib.phx_gguf_data_offset(self.h))
        self.Keys = [self.lib.phx_gguf_key_at(self.h, i).decode() for i in range(self.lib.phx_gguf_n_kv(self.h))]
        self.Tensors = []
        for i in range(self.lib.phx_gguf_n_tensors(self.h)):
            info = TensorInfo()
            self._check(self.lib.phx_gguf_tensor_at(self.h, i, C.byref(info)))
            self.Tensors.append(GgufTensor(info, self))
        self.TensorsByName = {t.Name: t for t in self.Tensors}

    @staticmethod
    def Open(path: str) -> "GgufFile":
        return GgufFile(path)

    def _check(self, rc: int):
        if rc:
            _raise(rc, self.lib.phx_gguf_last_error(self.h).decode(errors="replace"))

    def Dispose(self):
        if getattr(self, "h", None):
            self.lib.phx_gguf_close(self.h)
            self.h = None

    close = Dispose

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.Dispose()

    # typed metadata helpers (src/Gguf.cs:218-239)
    def Has(self, key: str) -> bool:
        return self.lib.phx_gguf_value_type(self.h, key.encode(), None, None) >= 0

    def ValueType(self, key: str):
        at, n = C.c_int32(), C.c_int64()
        t = self.lib.phx_gguf_value_type(self.h, key.encode(), C.byref(at), C.byref(n))
        return t, at.value, n.value

    def GetInt(self, key: str) -> int:
        v = C.c_int64()
        self._check(self.lib.phx_gguf_get_int(self.h, key.encode(), C.byref(v)))
        return v.value

    def GetFloat(self, key: str) -> float:
        v = C.c_float()
        self._check(self.lib.phx_gguf_get_float(self.h, key.encode(), C.byref(v)))
        return v.value

    def GetString(self, key: str) -> str:
        p, n = C.c_void_p(), C.c_uint64()
        self._check(self.lib.phx_gguf_get_string(self.h, key.encode(), C.byref(p), C.byref(n)))
        return C.string_at(p.value, n.value).decode()

    def GetArray(self, key: str, as_float: bool = False) -> list:
        t, at, n = self.ValueType(key)
        out = []
        for i in range(n):
            if as_float:
                v = C.c_double()
                self._check(self.lib.phx_gguf_get_array_float(self.h, key.encode(), i, C.byref(v)))
            else:
                v = C.c_int64()
                self._check(self.lib.phx_gguf_get_array_int(self.h, key.encode(), i, C.byref(v)))
            out.append(v.value)
        return out

    # mixture-of-experts ingestion
    def moe_config(self) -> dict:
        """GemmaConfig.FromGguf's MoE part (src/GemmaCpu.cs:26-31, 66-74)."""
        c = ModelConfig()
        self._check(self.lib.phx_gguf_moe_config(self.h, C.byref(c)))
        return {"arch": c.arch.decode(), "n_embd": c.n_embd, "n_layer": c.n_layer, "n_expert": c.n_expert,
                "n_expert_used": c.n_expert_used, "n_ff_exp": c.n_ff_exp, "eps": c.eps}

    def layer_desc(self, layer: int, without_shared: bool = False, weight_rule: int = PHX.WEIGHTS_SOFTMAX) -> LayerDesc:
        """The layer's MoE tensors (and its dense FFN as the shared FFN) as a descriptor into the mapping."""
        d = LayerDesc()
        self._check(self.lib.phx_gguf_layer_desc(self.h, layer, 1 if without_shared else 0, weight_rule, C.byref(d)))
        return d


def upload_layer(ctx, g: GgufFile, layer: int, slot: int | None = None, without_shared: bool = False,
                 weight_rule: int = PHX.WEIGHTS_SOFTMAX):
    """Upload one GGUF layer into a MoeContext slot (default: its own index), the role of GemmaGpu's
    UploadW / UploadF32 calls for the MoE tensors (src/GemmaGpu.cs:180-188)."""
    d = g.layer_desc(layer, without_shared, weight_rule)
    slot = layer if slot is None else slot
    ctx._check(ctx.lib.phx_moe_layer_upload(ctx.h, slot, C.byref(d)))
    ctx.layers[slot] = {"d": d.d, "n_expert": d.n_expert, "n_used": d.n_used, "n_ff": d.n_ff}
