"""phx_moe_ffn_noalloc, the entry point that allocates nothing (its workspace is the library's fixed
per-device scratch array), against phx_moe_ffn on the same device buffers: outputs, the residual
update, routing (ids, weights, logits, offsets, lists) and the expert intermediates are identical bit
for bit, over consecutive noalloc calls whose sizes go down and up (the array keeps the previous call's
bytes, so a stale value would show), on the decode path, the general path and K-quant weights; a call
whose workspace does not fit is refused with ArgumentError and leaves the context usable."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _call(ctx, fn, layer, x, shared, flags):
    T, d = x.shape
    xb, ob = ctx.alloc(x.nbytes), ctx.alloc(x.nbytes)
    sb = ctx.alloc(shared.nbytes) if shared is not None else None
    try:
        xb.upload(x)
        if sb:
            sb.upload(shared)
        fn(layer, T, xb.ptr, sb.ptr if sb else None, ob.ptr, flags | 32)  # | PHX_FLAG_KEEP_INTERMEDIATES: g, u compared
        ctx.sync()
        res = {"out": ob.download((T, d)), "x": xb.download((T, d))}
    finally:
        for b in (xb, ob, sb):
            if b:
                b.free()
    res["routing"] = ctx.routing()
    res["inter"] = ctx.intermediates()
    return res


def _same(a, b, what):
    assert a.dtype == b.dtype and a.shape == b.shape, what
    assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"{what} differs"


CASES = {
    # (layer config, [T of consecutive calls], shared input given, flags)
    "c2_decode_general": ("c2_decode", [40, 8, 33, 1], False, 0),
    "c2_residual_exact": ("c2_decode", [6, 2], False, 4 | 8),
    "c1_shared_given": ("c1_tiny", [16, 5], True, 0),
    "c4_kquant": ("c4_kquant", [12, 5], False, 0),
}


@pytest.mark.parametrize("case", list(CASES))
def test_noalloc_matches_ffn(ctx, pkg, case):
    cfg, Ts, with_shared, flags = CASES[case]
    say(f"noalloc {case}: T = {Ts}, flags {flags}")
    L = pkg.synth.make_layer(cfg, norms="noisy")
    ctx.upload(0, L)
    inputs = []
    for i, T in enumerate(Ts):
        x = pkg.synth.normal(500 + i, f"noalloc.x.{case}", (T, L["d"]))
        sh = pkg.synth.normal(600 + i, f"noalloc.sh.{case}", (T, L["d"])) if with_shared else None
        inputs.append((x, sh))
    refs = [_call(ctx, ctx.ffn_device, 0, x, sh, flags) for x, sh in inputs]
    for T, (x, sh), ref in zip(Ts, inputs, refs):  # consecutive noalloc calls
        got = _call(ctx, ctx.ffn_noalloc_device, 0, x, sh, flags)
        _same(got["out"], ref["out"], f"T={T} out")
        _same(got["x"], ref["x"], f"T={T} x (residual)")
        for name, a, b in zip(("ids", "weights", "offsets", "perm", "logits"), got["routing"], ref["routing"]):
            _same(a, b, f"T={T} {name}")
        for name, a, b in zip(("g", "u", "yd"), got["inter"], ref["inter"]):
            _same(a, b, f"T={T} {name}")
        say(f"  T={T}: identical to phx_moe_ffn")


def test_noalloc_refuses_what_does_not_fit(ctx, pkg):
    say("noalloc: C3 at T=2048 exceeds the scratch array")
    L = pkg.synth.make_layer("c3_prefill")
    ctx.upload(0, L)
    T = 2048
    x = pkg.synth.make_input("c3_prefill", T=T)
    xb, ob = ctx.alloc(x.nbytes), ctx.alloc(x.nbytes)
    try:
        xb.upload(x)
        with pytest.raises(pkg.moe.ArgumentError, match="scratch"):
            ctx.ffn_noalloc_device(0, T, xb.ptr, None, ob.ptr)
        # the context still works: a fitting noalloc call, then the allocating entry point
        ctx.ffn_noalloc_device(0, 16, xb.ptr, None, ob.ptr)
        ctx.sync()
        a = ob.download((16, L["d"]))
        ctx.ffn_device(0, 16, xb.ptr, None, ob.ptr)
        ctx.sync()
        _same(ob.download((16, L["d"])), a, "T=16 after the refusal")
    finally:
        xb.free()
        ob.free()
