"""A GGUF writer for tests, from the format (little-endian; GGUF v3): magic "GGUF", version u32,
tensor count and key/value count (u64 each), the key/value pairs (key as a u64-length string, value
type u32, value; arrays carry their element type u32 and length u64), the tensor infos (name, dims
count u32, dims u64 each with ne[0] first, GgmlType u32, data offset u64), padding to the alignment,
then the tensor data, each tensor at an aligned offset.  It also writes deliberately broken files for
the reader's validation tests.  Test infrastructure only."""
from __future__ import annotations

import struct

import numpy as np

UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)
_FMT = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f", BOOL: "<B",
        UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}
_NP = {UINT8: np.uint8, INT8: np.int8, UINT16: np.uint16, INT16: np.int16, UINT32: np.uint32, INT32: np.int32,
       FLOAT32: np.float32, BOOL: np.uint8, UINT64: np.uint64, INT64: np.int64, FLOAT64: np.float64}


def _str(s: str | bytes) -> bytes:
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


class Writer:
    """kv: list of (key, type, value) with value a scalar, a string, or for ARRAY a tuple
    (element type, list of values); tensors: list of (name, dims ne[0] first, ggml type, raw bytes)."""

    def __init__(self, alignment: int = 32, version: int = 3):
        self.kv: list = []
        self.tensors: list = []
        self.alignment = alignment
        self.version = version

    def add(self, key, vtype, value):
        self.kv.append((key, vtype, value))
        return self

    def tensor(self, name, dims, gtype, data: bytes | np.ndarray):
        raw = data.tobytes() if isinstance(data, np.ndarray) else bytes(data)
        self.tensors.append((name, list(dims), gtype, raw))
        return self

    @staticmethod
    def value(vtype, v) -> bytes:
        if vtype == STRING:
            return _str(v)
        if vtype == ARRAY:
            et, vals = v
            out = struct.pack("<IQ", et, len(vals))
            if et == STRING:
                return out + b"".join(_str(s) for s in vals)
            return out + np.asarray(vals, _NP[et]).tobytes()
        return struct.pack(_FMT[vtype], v)

    def header(self, offsets=None) -> bytes:
        out = bytearray(b"GGUF" + struct.pack("<IQQ", self.version, len(self.tensors), len(self.kv)))
        for k, t, v in self.kv:
            out += _str(k) + struct.pack("<I", t) + self.value(t, v)
        off = 0
        self._offsets = []
        for i, (name, dims, gt, raw) in enumerate(self.tensors):
            o = offsets[i] if offsets else off
            self._offsets.append(o)
            out += _str(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<q", d) for d in dims)
            out += struct.pack("<IQ", gt, o)
            off = (o + len(raw) + self.alignment - 1) // self.alignment * self.alignment
        return bytes(out)

    def bytes(self, offsets=None, truncate: int = 0) -> bytes:
        h = self.header(offsets)
        data_off = (len(h) + self.alignment - 1) // self.alignment * self.alignment
        buf = bytearray(h + b"\0" * (data_off - len(h)))
        end = data_off + max([o + len(raw) for o, (_, _, _, raw) in zip(self._offsets, self.tensors)], default=0)
        buf += b"\0" * (end - len(buf))
        for o, (_, _, _, raw) in zip(self._offsets, self.tensors):
            buf[data_off + o:data_off + o + len(raw)] = raw
        return bytes(buf[:len(buf) - truncate] if truncate else buf)

    def write(self, path, **kw):
        with open(path, "wb") as f:
            f.write(self.bytes(**kw))
        return path


def moe_model(layers: list[dict], arch: str = "gemma4", extra_kv=(), dense_type=None) -> Writer:
    """A Gemma-4-style MoE model file from layer dicts as the synthetic generator makes them (every layer
    with the same d, E, k, n_ff and types): the MoE keys GemmaConfig reads and, per layer, the MoE tensors
    plus the dense FFN (ffn_norm, ffn_gate, ffn_up, ffn_down) taken from the layer's shared FFN."""
    L0 = layers[0]
    d, E, k, nf = L0["d"], L0["n_expert"], L0["n_used"], L0["n_ff"]
    w = Writer()
    w.add("general.architecture", STRING, arch)
    w.add("general.alignment", UINT32, 32)
    w.add(f"{arch}.block_count", UINT32, len(layers))
    w.add(f"{arch}.embedding_length", UINT32, d)
    w.add(f"{arch}.attention.layer_norm_rms_epsilon", FLOAT32, float(L0["eps"]))
    w.add(f"{arch}.expert_count", UINT32, E)
    w.add(f"{arch}.expert_used_count", UINT32, k)
    w.add(f"{arch}.expert_feed_forward_length", UINT32, nf)
    w.add(f"{arch}.feed_forward_length", ARRAY, (INT32, [int(L.get("n_ff_shared", 0)) for L in layers]))
    for kv in extra_kv:
        w.add(*kv)
    for i, L in enumerate(layers):
        p = f"blk.{i}."
        w.tensor(p + "ffn_gate_inp.weight", [d, E], 0, L["gate_inp"])
        w.tensor(p + "ffn_gate_inp.scale", [d], 0, L["gate_inp_scale"])
        w.tensor(p + "ffn_down_exps.scale", [E], 0, L["down_scale"])
        for n in ("pre_ffw_norm_2", "post_ffw_norm_1", "post_ffw_norm_2", "post_ffw_norm"):
            w.tensor(p + n + ".weight", [d], 0, L[n])
        w.tensor(p + "ffn_gate_up_exps.weight", [d, 2 * nf, E], L["gate_up_type"], L["gate_up_exps"])
        assert L["down_cols"] == nf, "a GGUF row is whole blocks: the down rows cannot be padded"
        w.tensor(p + "ffn_down_exps.weight", [nf, d, E], L["down_type"], L["down_exps"])
        if L.get("n_ff_shared"):
            nff, st = L["n_ff_shared"], L["shared_type"]
            w.tensor(p + "ffn_norm.weight", [d], 0, L["ffn_norm"])
            w.tensor(p + "ffn_gate.weight", [d, nff], st, L["ffn_gate"])
            w.tensor(p + "ffn_up.weight", [d, nff], st, L["ffn_up"])
            w.tensor(p + "ffn_down.weight", [nff, d], st, L["ffn_down"])
    return w
