"""The C ABI of libphxmoe.so (include/phx_moe.h), checked without a GPU: every declared function is
exported (and nothing else under the phx_ prefix), the header compiles as C and C++, the layer
descriptor layout and constants agree between C and the Python mirror, the descriptor validation
(phx_moe_check_desc, pure host code) returns the reference host's error classes, and a context on a
machine without a HIP device fails with PHX_ERR_DEVICE_LOST instead of falling back to the CPU."""
import ctypes as C
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "phx_moe.h"
HEADERS = sorted((ROOT / "include").glob("*.h"))


def _strip_comments(src: str) -> str:
    src = re.sub(r"/\*.*?\*/", " ", src, flags=re.S)
    return re.sub(r"//[^\n]*", " ", src)


def declared_functions() -> list[str]:
    names = set()
    for h in HEADERS:
        names |= set(re.findall(r"\b(phx_\w+)\s*\(", _strip_comments(h.read_text())))
    return sorted(names)


def header_defines() -> dict[str, int]:
    out = {}
    for h in HEADERS:
        for name, val in re.findall(r"#define\s+(PHX_\w+)\s+\(?(-?\d+)u?\)?", h.read_text()):
            out[name] = int(val)
    return out


def test_every_declared_function_is_exported(pkg):
    lib = pkg.moe.load_lib()
    names = declared_functions()
    assert len(names) >= 20
    for n in names:
        assert hasattr(lib, n), n
    nm = subprocess.run(["nm", "-D", "--defined-only", str(pkg.moe.lib_path())], capture_output=True, text=True,
                        check=True).stdout
    exported = sorted(set(re.findall(r"\bT (phx_\w+)", nm)))
    assert exported == names


def test_python_binding_covers_the_header(pkg):
    import inspect
    src = inspect.getsource(pkg.moe.load_lib) + inspect.getsource(pkg.gguf._lib)
    for n in declared_functions():
        assert f'"{n}"' in src, f"{n} has no ctypes signature in moe.load_lib or gguf._lib"


@pytest.mark.parametrize("header", [h.name for h in HEADERS])
@pytest.mark.parametrize("compiler,std", [("gcc", "-std=c99"), ("g++", "-std=c++11")])
def test_header_compiles_standalone(tmp_path, compiler, std, header):
    src = tmp_path / ("t.c" if compiler == "gcc" else "t.cc")
    src.write_text(f'#include "{header}"\nint main(void) {{ return PHX_OK; }}\n')
    subprocess.run([compiler, std, "-Wall", "-Werror", "-pedantic", "-fsyntax-only", f"-I{HEADER.parent}", str(src)],
                   check=True)


@pytest.mark.parametrize("struct,cname", [("TensorInfo", "phx_gguf_tensor"), ("ModelConfig", "phx_moe_model_config")])
def test_gguf_struct_layouts_match_c(tmp_path, pkg, struct, cname):
    S = getattr(pkg.gguf, struct)
    fields = [f for f, _ in S._fields_]
    prog = ['#include <stdio.h>', '#include <stddef.h>', '#include "phx_gguf.h"', "int main(void) {",
            f'  printf("%zu\\n", sizeof({cname}));']
    prog += [f'  printf("%zu\\n", offsetof({cname}, {f}));' for f in fields]
    prog += ["  return 0;", "}"]
    (tmp_path / "g.c").write_text("\n".join(prog))
    exe = tmp_path / "g"
    subprocess.run(["gcc", "-std=c99", f"-I{HEADER.parent}", "-o", str(exe), str(tmp_path / "g.c")], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == C.sizeof(S)
    assert vals[1:] == [getattr(S, f).offset for f in fields]


def test_descriptor_layout_matches_c(tmp_path, pkg):
    D = pkg.moe.LayerDesc
    fields = [f for f, _ in D._fields_]
    prog = ['#include <stdio.h>', '#include <stddef.h>', '#include "phx_moe.h"', "int main(void) {",
            '  printf("%zu\\n", sizeof(phx_moe_layer_desc));']
    prog += [f'  printf("%zu\\n", offsetof(phx_moe_layer_desc, {f}));' for f in fields]
    prog += ["  return 0;", "}"]
    (tmp_path / "l.c").write_text("\n".join(prog))
    exe = tmp_path / "l"
    subprocess.run(["gcc", "-std=c99", f"-I{HEADER.parent}", "-o", str(exe), str(tmp_path / "l.c")], check=True)
    vals = [int(v) for v in subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout.split()]
    assert vals[0] == C.sizeof(D)
    assert vals[1:] == [getattr(D, f).offset for f in fields]


def test_constants_match_python_mirror(pkg):
    P = pkg.PHX
    d = header_defines()
    assert (d["PHX_OK"], d["PHX_ERR_ARG"], d["PHX_ERR_OOM"], d["PHX_ERR_UNSUPPORTED"], d["PHX_ERR_DEVICE_LOST"],
            d["PHX_ERR_HIP"], d["PHX_ERR_FORMAT"]) == (P.OK, P.ERR_ARG, P.ERR_OOM, P.ERR_UNSUPPORTED, P.ERR_DEVICE_LOST,
                                                   P.ERR_HIP, P.ERR_FORMAT)
    assert (d["PHX_F32"], d["PHX_Q4_0"], d["PHX_Q8_0"], d["PHX_Q3_K"], d["PHX_Q4_K"], d["PHX_Q5_K"], d["PHX_Q6_K"]) == (
        P.F32, P.Q4_0, P.Q8_0, P.Q3_K, P.Q4_K, P.Q5_K, P.Q6_K)
    assert (d["PHX_MAX_EXPERTS"], d["PHX_MAX_USED"]) == (P.MAX_EXPERTS, P.MAX_USED)
    assert (d["PHX_WEIGHTS_SOFTMAX"], d["PHX_WEIGHTS_CPUREF"]) == (P.WEIGHTS_SOFTMAX, P.WEIGHTS_CPUREF)
    assert (d["PHX_FLAG_DEVICE_PTRS"], d["PHX_FLAG_ASYNC"], d["PHX_FLAG_RESIDUAL"], d["PHX_FLAG_EXACT_ROUTER"],
            d["PHX_FLAG_FAST_MATH"], d["PHX_FLAG_KEEP_INTERMEDIATES"]) == (
        P.FLAG_DEVICE_PTRS, P.FLAG_ASYNC, P.FLAG_RESIDUAL, P.FLAG_EXACT_ROUTER, P.FLAG_FAST_MATH,
        P.FLAG_KEEP_INTERMEDIATES)
    assert (d["PHX_QUANT_PLAIN"], d["PHX_QUANT_SILU_MUL"], d["PHX_QUANT_RMS_NORM"], d["PHX_QUANT_GELU_MUL"]) == (
        P.QUANT_PLAIN, P.QUANT_SILU_MUL, P.QUANT_RMS_NORM, P.QUANT_GELU_MUL)


# ---------------------------------------------------------------------------------------- check_desc
@pytest.fixture(scope="module")
def tiny_layer(pkg):
    cfg = dict(idx=9, T=2, d=256, E=8, k=2, nf=128, gu=2, dn=2, nff=256, sh=8)
    return pkg.synth.make_layer(cfg)


def _check(pkg, L, **over):
    D = pkg.moe.LayerDesc.from_layer(L)
    for k, v in over.items():
        setattr(D, k, v)
    return pkg.moe.load_lib().phx_moe_check_desc(C.byref(D))


def test_check_desc_accepts_valid_layers(pkg, tiny_layer):
    P = pkg.PHX
    assert _check(pkg, tiny_layer) == P.OK
    L4 = pkg.synth.make_layer(dict(idx=9, T=1, d=512, E=4, k=2, nf=288, gu=P.Q4_K, dn=P.Q6_K))
    assert L4["down_cols"] == 512 and _check(pkg, L4) == P.OK


@pytest.mark.parametrize("over,code", [
    (dict(d=0), "ERR_ARG"), (dict(n_used=0), "ERR_ARG"), (dict(n_ff=-32), "ERR_ARG"),
    (dict(n_expert=257), "ERR_UNSUPPORTED"), (dict(n_used=17), "ERR_UNSUPPORTED"), (dict(n_used=9), "ERR_UNSUPPORTED"),
    (dict(n_ff=100), "ERR_UNSUPPORTED"), (dict(d=250), "ERR_UNSUPPORTED"),
    (dict(gate_up_type=3), "ERR_UNSUPPORTED"), (dict(down_type=0), "ERR_UNSUPPORTED"),
    (dict(down_cols=160), "ERR_ARG"), (dict(weight_rule=2), "ERR_ARG"), (dict(eps=float("nan")), "ERR_ARG"),
    (dict(eps=-1.0), "ERR_ARG"), (dict(gate_inp=None), "ERR_ARG"), (dict(down_exps=None), "ERR_ARG"),
    (dict(n_ff_shared=-1), "ERR_ARG"), (dict(shared_type=5), "ERR_UNSUPPORTED"), (dict(ffn_up=None), "ERR_ARG"),
    (dict(n_ff_shared=100), "ERR_UNSUPPORTED"),
])
def test_check_desc_rejects(pkg, tiny_layer, over, code):
    assert _check(pkg, tiny_layer, **over) == getattr(pkg.PHX, code)


def test_check_desc_k_quant_alignment(pkg, tiny_layer):
    P = pkg.PHX
    # Q4_K rows need whole 256-element super-blocks of d; the down K-dimension is padded to down_cols
    assert _check(pkg, tiny_layer, gate_up_type=P.Q4_K) == P.OK
    assert _check(pkg, tiny_layer, gate_up_type=P.Q4_K, d=288) == P.ERR_UNSUPPORTED
    assert _check(pkg, tiny_layer, down_type=P.Q6_K) == P.ERR_ARG  # down_cols 128 is not 256-aligned
    assert _check(pkg, tiny_layer, down_type=P.Q6_K, down_cols=256) == P.OK
    # Q3_K and Q5_K (GGUF types 11 and 13) on either product
    assert _check(pkg, tiny_layer, gate_up_type=P.Q5_K, down_type=P.Q3_K, down_cols=256) == P.OK
    assert _check(pkg, tiny_layer, gate_up_type=P.Q3_K, d=288) == P.ERR_UNSUPPORTED


def test_check_desc_null(pkg):
    assert pkg.moe.load_lib().phx_moe_check_desc(None) == pkg.PHX.ERR_ARG


# ---------------------------------------------------------------------------------------- no device
def test_context_without_device_fails_loudly(pkg):
    lib = pkg.moe.load_lib()
    h = C.c_void_p()
    rc = lib.phx_moe_create(0, C.byref(h))
    if rc == 0:
        lib.phx_moe_destroy(h)
        pytest.skip("a HIP device is present")
    assert rc == pkg.PHX.ERR_DEVICE_LOST and not h.value
    with pytest.raises(pkg.moe.GpuDeviceLostError):
        pkg.MoeContext(0)
    assert lib.phx_moe_create(0, None) == pkg.PHX.ERR_ARG
    assert lib.phx_moe_last_error(None) == b"null context"
    lib.phx_moe_destroy(None)


def test_missing_library_raises(pkg, monkeypatch, tmp_path):
    monkeypatch.setattr(pkg.moe, "_LIB", None)
    monkeypatch.setattr(pkg.moe, "lib_path", lambda: tmp_path / "libphxmoe.so")
    with pytest.raises(FileNotFoundError):
        pkg.moe.load_lib()


def test_error_classes(pkg):
    m = pkg.moe
    for code, cls in ((-1, m.ArgumentError), (-3, m.NotSupportedError), (-4, m.GpuDeviceLostError), (-5, m.MoeError),
                      (-2, m.MoeError)):
        with pytest.raises(cls) as e:
            m._raise(code, "x")
        assert e.value.code == code
    assert issubclass(m.ArgumentError, ValueError)
