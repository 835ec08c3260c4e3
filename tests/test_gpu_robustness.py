"""GPU checks of the library's guards: the certified general-path router only where its workgroups
cover every input block (small expert counts with wide rows take the exact router), a captured stack
refused once a layer is uploaded again or the workspace grows (the graph would name freed memory),
device-pointer calls refused on pageable host memory, the host-buffer call graph cache's counts, and
gate/up intermediates refused after a call that skipped their stores."""
import sys

import numpy as np
import pytest

from test_gpu_parity import check_layer

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


# (E, k, d, T): E = 2 at d = 4096 has 128 input blocks against 32 E = 64 covered by the 256-thread router
# workgroups, so it must take the exact router; E = 4 covers exactly 128 and stays certified (a workgroup
# per (token, expert): the four-expert workgroups would cover 32 E / 4); E = 8 likewise; E = 16 covers
# exactly 128 with four experts per workgroup
@pytest.mark.parametrize("E,k,d,T", [(2, 1, 4096, 600), (4, 2, 4096, 300), (2, 2, 2048, 1100), (8, 2, 4096, 300),
                                     (16, 2, 4096, 300)])
def test_general_router_covers_every_input_block(ctx, pkg, orc, E, k, d, T):
    say(f"general path, E={E} k={k} d={d} T={T}: vs oracle")
    cfg = dict(idx=31, T=T, d=d, E=E, k=k, nf=128, gu=2, dn=2)
    L = pkg.synth.make_layer(cfg, norms="noisy")
    ctx.upload(0, L)
    x = pkg.synth.normal(900 + E, "robust.x", (T, d))
    check_layer(ctx, orc, L, x, tag=f"E{E} d{d} T{T}")


def test_stack_refuses_a_stale_capture(pkg):
    """A context of its own, so the workspace starts at the stack's size (T = 4) and the larger call
    (T = 1024) regrows it."""
    say("stack: capture at T=4, then a larger call and a new upload make it stale")
    L0 = pkg.synth.make_layer("c1_tiny", layer=0, norms="noisy")
    L1 = pkg.synth.make_layer("c1_tiny", layer=1, norms="noisy")
    with pkg.MoeContext(0) as ctx:
        ctx.upload(0, L0)
        ctx.upload(1, L1)
        x = pkg.synth.normal(910, "robust.stack", (4, L0["d"]))
        ctx.stack_capture(0, 2, 4)
        ref = ctx.stack_run(x.copy())
        # a call with more tokens regrows the workspace the graph was captured over
        ctx.ffn(0, pkg.synth.normal(911, "robust.big", (1024, L0["d"])))
        with pytest.raises(pkg.moe.ArgumentError, match="stale"):
            ctx.stack_run(x.copy())
        ctx.stack_capture(0, 2, 4)
        np.testing.assert_array_equal(ctx.stack_run(x.copy()), ref)
        # uploading a layer of the stack again frees the weights the graph names
        ctx.upload(1, L1)
        with pytest.raises(pkg.moe.ArgumentError, match="stale"):
            ctx.stack_run(x.copy())
        ctx.stack_capture(0, 2, 4)
        np.testing.assert_array_equal(ctx.stack_run(x.copy()), ref)
    say("  refused twice, equal after each recapture")


def test_device_pointer_calls_refuse_pageable_host_memory(ctx, pkg):
    say("device-pointer calls on pageable host memory: ArgumentError, no launch")
    L = pkg.synth.make_layer("c1_tiny")
    ctx.upload(0, L)
    T, d = 4, L["d"]
    x = pkg.synth.normal(912, "robust.host", (T, d))
    out = np.zeros_like(x)
    ob = ctx.alloc(x.nbytes)
    try:
        for fn in (ctx.ffn_noalloc_device, ctx.ffn_device):
            with pytest.raises(pkg.moe.ArgumentError, match="device-accessible"):
                fn(0, T, x.ctypes.data, None, ob.ptr)
            with pytest.raises(pkg.moe.ArgumentError, match="device-accessible"):
                fn(0, T, ob.ptr, None, out.ctypes.data)
        # the context still runs a proper call
        xb = ctx.alloc(x.nbytes)
        try:
            xb.upload(x)
            ctx.ffn_noalloc_device(0, T, xb.ptr, None, ob.ptr)
            ctx.sync()
            np.testing.assert_array_equal(ob.download((T, d)), ctx.ffn(0, x))
        finally:
            xb.free()
    finally:
        ob.free()


def test_host_call_graphs_are_counted(ctx, pkg):
    say("host-buffer calls: one capture per shape, replays after")
    L = pkg.synth.make_layer("c1_tiny")
    ctx.upload(0, L)
    h0, m0 = ctx.graph_stats()
    x1 = pkg.synth.normal(913, "robust.g1", (1, L["d"]))
    x3 = pkg.synth.normal(914, "robust.g3", (3, L["d"]))
    a = ctx.ffn(0, x1)
    b = ctx.ffn(0, x3)
    np.testing.assert_array_equal(ctx.ffn(0, x1), a)
    np.testing.assert_array_equal(ctx.ffn(0, x3), b)
    h1, m1 = ctx.graph_stats()
    assert (h1 - h0, m1 - m0) == (2, 2)


@pytest.mark.parametrize("fast", [False, True])
def test_skipped_gate_up_stores_are_refused(ctx, pkg, orc, fast):
    """A prefill-sized Q4_0 call skips the g and u stores unless PHX_FLAG_KEEP_INTERMEDIATES is given:
    asking for them afterwards is an error (not the previous call's rows), yd stays available, the output
    is the same with and without the stores, and the kept g and u are the oracle's (exact mode)."""
    say(f"skipped g/u stores (fast={fast}): refused without the flag, kept with it")
    L = pkg.synth.make_layer("c3_prefill")
    ctx.upload(0, L)
    T = 256  # T * k = 2048 >= 8 E: the matrix-core path
    x = pkg.synth.make_input("c3_prefill", T=T)
    out0 = ctx.ffn(0, x, fast_math=fast)
    with pytest.raises(Exception, match="KEEP_INTERMEDIATES"):
        ctx.intermediates()
    n, d = T * L["n_used"], L["d"]
    yd = np.empty((n, d), np.float32)
    assert ctx.lib.phx_moe_get_intermediates(ctx.h, None, None, yd.ctypes.data) == 0
    out1 = ctx.ffn(0, x, fast_math=fast, keep_intermediates=True)
    np.testing.assert_array_equal(out0, out1)
    g, u, yd1 = ctx.intermediates()
    np.testing.assert_array_equal(yd, yd1)
    if not fast:
        for t in (0, T - 1):
            _, _, _, rg, ru, _ = orc.moe_token(L, x[t], None)
            np.testing.assert_array_equal(g[t * L["n_used"]:(t + 1) * L["n_used"]], rg)
            np.testing.assert_array_equal(u[t * L["n_used"]:(t + 1) * L["n_used"]], ru)
