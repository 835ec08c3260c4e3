"""The GGUF reader of libphxmoe.so (include/phx_gguf.h) on files the tests write (tests/gguf_writer.py):
the parse against the arrays written, the typed metadata helpers, every validation rule of the
reference's GgufFile.Load (src/Gguf.cs:116-210) with its outcome, the MoE part of GemmaConfig.FromGguf
(src/GemmaCpu.cs:26-31, 66-74) and the per-layer descriptor over the mapping.  Host-only: CPU."""
import ctypes as C
import struct

import numpy as np
import pytest

import gguf_writer as GW


def _layers(pkg, cfg, n, **kw):
    return [pkg.synth.make_layer(cfg, layer=i, norms="noisy", **kw) for i in range(n)]


SMALL = dict(idx=21, T=4, d=512, E=8, k=2, nf=256, gu=2, dn=2, nff=384, sh=2)
SMALL_Q8 = dict(idx=22, T=4, d=512, E=8, k=2, nf=256, gu=8, dn=8, nff=256, sh=8)
SMALL_K = dict(idx=23, T=4, d=512, E=4, k=2, nf=512, gu=12, dn=14)  # K-quant rows: nf a multiple of 256
SMALL_K35 = dict(idx=24, T=4, d=512, E=4, k=2, nf=512, gu=13, dn=11, nff=512, sh=13)  # Q5_K and Q3_K (types 13, 11)


@pytest.fixture(scope="module")
def small_file(pkg, tmp_path_factory):
    layers = _layers(pkg, SMALL, 2)
    path = tmp_path_factory.mktemp("gguf") / "small.gguf"
    GW.moe_model(layers).write(path)
    return path, layers


def _desc_bytes(ptr, n):
    return np.frombuffer(C.string_at(ptr, n), np.uint8)


def _arr_bytes(a):
    return np.frombuffer(np.ascontiguousarray(a).tobytes(), np.uint8)


def test_parse_round_trip(pkg, small_file):
    path, layers = small_file
    with pkg.gguf.GgufFile.Open(str(path)) as g:
        assert g.Version == 3 and g.Alignment == 32 and g.DataOffset % 32 == 0
        assert g.Keys[:3] == ["general.architecture", "general.alignment", "gemma4.block_count"]
        assert g.GetString("general.architecture") == "gemma4"
        assert g.GetInt("gemma4.block_count") == 2 and g.GetInt("gemma4.embedding_length") == 512
        assert g.GetFloat("gemma4.attention.layer_norm_rms_epsilon") == np.float32(1e-6)
        assert g.GetArray("gemma4.feed_forward_length") == [384, 384]
        assert len(g.Tensors) == 2 * 13
        t = g.TensorsByName["blk.1.ffn_gate_up_exps.weight"]
        assert t.Dims == [512, 512, 8] and t.Type == 2 and t.Offset % 32 == 0
        assert t.SizeBytes == 512 // 32 * 18 * 512 * 8 == layers[1]["gate_up_exps"].nbytes
        assert np.array_equal(t.bytes(), _arr_bytes(layers[1]["gate_up_exps"]))
        r = g.TensorsByName["blk.0.ffn_gate_inp.weight"]
        assert r.Dims == [512, 8] and r.Type == 0
        assert np.array_equal(np.frombuffer(r.bytes().tobytes(), np.float32).reshape(8, 512), layers[0]["gate_inp"])
        assert g.moe_config() == {"arch": "gemma4", "n_embd": 512, "n_layer": 2, "n_expert": 8, "n_expert_used": 2,
                                  "n_ff_exp": 256, "eps": np.float32(1e-6)}


@pytest.mark.parametrize("cfg", [SMALL, SMALL_Q8, SMALL_K, SMALL_K35])
def test_layer_descriptor_points_at_the_tensors(pkg, tmp_path, cfg):
    layers = _layers(pkg, cfg, 2)
    path = GW.moe_model(layers).write(tmp_path / "m.gguf")
    with pkg.gguf.GgufFile.Open(str(path)) as g:
        for i, L in enumerate(layers):
            if not L.get("n_ff_shared"):  # every Gemma layer has a dense FFN (src/GemmaCpu.cs:167-169)
                with pytest.raises(pkg.ArgumentError, match="ffn_gate.weight not found"):
                    g.layer_desc(i)
            d = g.layer_desc(i, without_shared=not L.get("n_ff_shared"))
            assert (d.d, d.n_expert, d.n_used, d.n_ff, d.down_cols) == (L["d"], L["n_expert"], L["n_used"], L["n_ff"],
                                                                        L["n_ff"])
            assert (d.gate_up_type, d.down_type, d.weight_rule) == (L["gate_up_type"], L["down_type"], 0)
            assert d.eps == np.float32(L["eps"])
            for f in ("gate_inp", "gate_inp_scale", "down_scale", "pre_ffw_norm_2", "post_ffw_norm_1",
                      "post_ffw_norm_2", "post_ffw_norm", "gate_up_exps", "down_exps"):
                assert np.array_equal(_desc_bytes(getattr(d, f), L[f].nbytes), _arr_bytes(L[f])), f
            if L.get("n_ff_shared"):
                assert (d.n_ff_shared, d.shared_type) == (L["n_ff_shared"], L["shared_type"])
                for f in ("ffn_norm", "ffn_gate", "ffn_up", "ffn_down"):
                    assert np.array_equal(_desc_bytes(getattr(d, f), L[f].nbytes), _arr_bytes(L[f])), f
            else:
                assert d.n_ff_shared == 0
            d2 = g.layer_desc(i, without_shared=True, weight_rule=1)
            assert d2.n_ff_shared == 0 and not d2.ffn_gate and d2.weight_rule == 1


def test_metadata_conversions(pkg, tmp_path):
    w = GW.Writer()
    for key, t, v in [("u8", GW.UINT8, 200), ("i8", GW.INT8, -7), ("u16", GW.UINT16, 60000), ("i16", GW.INT16, -30000),
                      ("u32", GW.UINT32, 4000000000), ("i32", GW.INT32, -2000000000), ("u64", GW.UINT64, 2 ** 63 + 5),
                      ("i64", GW.INT64, -2 ** 62), ("f32", GW.FLOAT32, 2.5), ("f64", GW.FLOAT64, 3.5),
                      ("b", GW.BOOL, 1), ("s", GW.STRING, "héllo"), ("nan", GW.FLOAT64, float("nan")),
                      ("af", GW.ARRAY, (GW.FLOAT32, [0.5, -1.25])), ("as", GW.ARRAY, (GW.STRING, ["a", "bc"])),
                      ("ai", GW.ARRAY, (GW.INT16, [1, -2, 3]))]:
        w.add(key, t, v)
    path = w.write(tmp_path / "kv.gguf")
    with pkg.gguf.GgufFile.Open(str(path)) as g:
        assert [g.GetInt(k) for k in ("u8", "i8", "u16", "i16", "u32", "i32", "i64", "b")] == \
            [200, -7, 60000, -30000, 4000000000, -2000000000, -2 ** 62, 1]
        assert g.GetInt("f32") == 2 and g.GetInt("f64") == 4  # Convert.ToInt64 rounds half to even
        assert g.GetFloat("f32") == 2.5 and g.GetFloat("i16") == -30000.0
        assert g.GetString("s") == "héllo"
        assert g.GetArray("af", as_float=True) == [0.5, -1.25] and g.GetArray("ai") == [1, -2, 3]
        assert g.ValueType("as") == (GW.ARRAY, GW.STRING, 2)
        for bad in ("u64", "nan", "s"):
            with pytest.raises(pkg.ArgumentError):
                g.GetInt(bad)
        with pytest.raises(pkg.ArgumentError, match="not found"):
            g.GetInt("missing")
        with pytest.raises(pkg.ArgumentError):
            g.GetArray("as")
        assert not g.Has("missing") and g.Has("u8")


def _kv_file(kv):
    w = GW.Writer()
    for k in kv:
        w.add(*k)
    return w


def _tensor_file(dims=(64, 2), gtype=0, nbytes=None, alignment=32, offsets=None):
    w = GW.Writer(alignment=alignment)
    if alignment != 32:
        w.add("general.alignment", GW.UINT32, alignment)
    n = int(np.prod(dims))
    size = nbytes if nbytes is not None else (n * 4 if gtype == 0 else n // 32 * 18)
    w.tensor("t", list(dims), gtype, b"\x01" * size)
    return w


def _raw(version=3, n_t=0, n_kv=0, body=b""):
    return b"GGUF" + struct.pack("<Iqq", version, n_t, n_kv) + body


# (description, file bytes, the reference's message)
def _bad_files():
    kv1 = GW.Writer().add("a", GW.UINT8, 1)
    big_str = _raw(n_kv=1, body=struct.pack("<Q", 2 ** 31) + b"x" * 8)
    dup_key = GW.Writer().add("a", GW.UINT8, 1).add("a", GW.UINT8, 2).bytes()
    bad_vt = _raw(n_kv=1, body=GW._str("k") + struct.pack("<I", 13) + b"\0" * 8)
    arr_arr = _raw(n_kv=1, body=GW._str("k") + struct.pack("<IIQ", GW.ARRAY, GW.ARRAY, 1) + b"\0" * 16)
    neg_arr = _raw(n_kv=1, body=GW._str("k") + struct.pack("<IIq", GW.ARRAY, GW.UINT8, -1) + b"\0" * 8)
    t_dims0 = _raw(n_t=1, body=GW._str("t") + struct.pack("<I", 0) + struct.pack("<IQ", 0, 0) + b"\0" * 64)
    t_dims5 = _raw(n_t=1, body=GW._str("t") + struct.pack("<I", 5) + struct.pack("<5q", 1, 1, 1, 1, 1)
                   + struct.pack("<IQ", 0, 0) + b"\0" * 64)
    t_neg = _raw(n_t=1, body=GW._str("t") + struct.pack("<Iq", 1, -4) + struct.pack("<IQ", 0, 0) + b"\0" * 64)
    dup_t = GW.Writer().tensor("t", [8], 0, b"\0" * 32).tensor("t", [8], 0, b"\0" * 32).bytes()
    return [
        ("too small", b"GGUF" + b"\0" * 10, "File too small to be GGUF."),
        ("bad magic", b"GGML" + kv1.bytes()[4:], "Not a GGUF file (bad magic)."),
        ("version 1", _raw(version=1), "Unsupported GGUF version 1."),
        ("version 4", _raw(version=4), "Unsupported GGUF version 4."),
        ("negative counts", _raw(n_t=-1), "Negative tensor or KV count."),
        ("truncated key/value", kv1.header()[:-1], "Unexpected end of GGUF header."),
        ("string too long", big_str, "String too long."),
        ("duplicate key", dup_key, "Duplicate key a."),
        ("unknown value type", bad_vt, "Unknown GGUF value type 13."),
        ("array of arrays", arr_arr, "Unsupported GGUF array type 9."),
        ("negative array length", neg_arr, "Bad array length."),
        ("alignment 48", _tensor_file(alignment=48).bytes(), "general.alignment must be a power of two."),
        ("alignment 0", _kv_file([("general.alignment", GW.UINT32, 0)]).bytes(), "general.alignment must be a power of two."),
        ("zero dims", t_dims0, "Tensor t has 0 dims."),
        ("five dims", t_dims5, "Tensor t has 5 dims."),
        ("non-positive dim", t_neg, "Tensor t has a non-positive dim."),
        ("duplicate tensor", dup_t, "Duplicate tensor t."),
        ("unsupported type", _tensor_file(gtype=4).bytes(), "Tensor t uses unsupported type 4."),
        ("partial block row", _tensor_file(dims=(48, 2), gtype=2, nbytes=54).bytes(),
         "Tensor t row is not a multiple of the block size."),
        ("unaligned offset", _tensor_file().bytes(offsets=[16]), "Tensor t offset is not aligned."),
        ("past end of file", _tensor_file().bytes(truncate=4), "Tensor t extends past end of file."),
    ]


@pytest.mark.parametrize("case", [c[0] for c in _bad_files()])
def test_validation_rules(pkg, tmp_path, case):
    data, msg = {c[0]: c[1:] for c in _bad_files()}[case]
    p = tmp_path / "bad.gguf"
    p.write_bytes(data)
    with pytest.raises(pkg.InvalidDataError) as e:
        pkg.gguf.GgufFile.Open(str(p))
    assert msg in str(e.value)


def test_open_missing_file(pkg, tmp_path):
    with pytest.raises(pkg.ArgumentError, match="cannot open"):
        pkg.gguf.GgufFile.Open(str(tmp_path / "none.gguf"))


def test_valid_edge_files(pkg, tmp_path):
    # version 2, no tensors and no keys; a 64-byte alignment; a tensor ending exactly at the end of the file
    p = tmp_path / "v2.gguf"
    p.write_bytes(_raw(version=2) + b"\0" * 8)
    with pkg.gguf.GgufFile.Open(str(p)) as g:
        assert g.Version == 2 and g.Tensors == [] and g.Keys == []
    p2 = _tensor_file(alignment=64).write(tmp_path / "a64.gguf")
    with pkg.gguf.GgufFile.Open(str(p2)) as g:
        assert g.Alignment == 64 and g.DataOffset % 64 == 0
        assert g.DataOffset + g.Tensors[0].SizeBytes == p2.stat().st_size


def _model_with(pkg, tmp_path, arch="gemma4", drop=(), set_kv=(), layers=None, mutate=None):
    layers = layers or _layers(pkg, SMALL, 1)
    w = GW.moe_model(layers, arch=arch)
    w.kv = [kv for kv in w.kv if kv[0] not in drop]
    for k, t, v in set_kv:
        w.kv = [kv for kv in w.kv if kv[0] != k] + [(k, t, v)]
    if mutate:
        mutate(w)
    return w.write(tmp_path / "m.gguf")


def test_moe_detection_and_limits(pkg, tmp_path):
    G = pkg.gguf.GgufFile
    with G.Open(str(_model_with(pkg, tmp_path, arch="llama"))) as g:
        with pytest.raises(pkg.NotSupportedError, match="Not a Gemma model: llama"):
            g.moe_config()
    with G.Open(str(_model_with(pkg, tmp_path, mutate=lambda w: w.tensors.pop(0)))) as g:
        with pytest.raises(pkg.NotSupportedError, match="not a mixture-of-experts model"):
            g.moe_config()
    for key, val in (("gemma4.expert_count", 300), ("gemma4.expert_used_count", 17),
                     ("gemma4.expert_feed_forward_length", 100)):
        with G.Open(str(_model_with(pkg, tmp_path, set_kv=[(key, GW.UINT32, val)]))) as g:
            with pytest.raises(pkg.NotSupportedError, match="Unexpected mixture-of-experts layout"):
                g.moe_config()
    with G.Open(str(_model_with(pkg, tmp_path, drop=("gemma4.expert_used_count",)))) as g:
        with pytest.raises(pkg.ArgumentError, match="not found"):
            g.moe_config()


def test_layer_descriptor_rejects_wrong_tensors(pkg, tmp_path):
    G = pkg.gguf.GgufFile

    def wrong_router(w):
        name, dims, t, raw = w.tensors[0]
        w.tensors[0] = (name, [dims[0] // 2, dims[1] * 2], t, raw)

    def f16_norm(w):
        i = [n for n, *_ in w.tensors].index("blk.0.pre_ffw_norm_2.weight")
        name, dims, t, raw = w.tensors[i]
        w.tensors[i] = (name, dims, 1, raw[:len(raw) // 2])

    with G.Open(str(_model_with(pkg, tmp_path, mutate=wrong_router))) as g:
        with pytest.raises(pkg.NotSupportedError, match="unexpected dims"):
            g.layer_desc(0)
    with G.Open(str(_model_with(pkg, tmp_path, mutate=f16_norm))) as g:
        with pytest.raises(pkg.NotSupportedError, match="must be f32"):
            g.layer_desc(0)
    with G.Open(str(_model_with(pkg, tmp_path))) as g:
        with pytest.raises(pkg.ArgumentError, match="out of range"):
            g.layer_desc(1)
