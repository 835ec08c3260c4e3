"""Error paths on the GPU through the library's fault injector (PHX_FAULT, read when a context is
created): a failed device allocation surfaces as PHX_ERR_OOM (OutOfDeviceMemoryError) from whichever
call made it, a failed launch as PHX_ERR_DEVICE_LOST (GpuDeviceLostError, the host's
GpuDeviceLostException, src/Vulkan.cs:194-208).  No fault reaches the device: the allocation is not
made, the launch and every later one of the call are skipped.  After the fault the context stays
usable, and the repeated call gives the fault-free result bit for bit."""
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make_ctx(pkg, spec):
    os.environ["PHX_FAULT"] = spec
    try:
        return pkg.MoeContext(0)
    finally:
        del os.environ["PHX_FAULT"]


CASES = {
    # decode path (T=4: four launches per call) and general path (T=64: the grouped kernels)
    "decode": ("c1_tiny", 4),
    "general": ("c1_tiny", 64),
}


@pytest.mark.parametrize("case", list(CASES))
def test_allocation_faults(pkg, case):
    cfg, T = CASES[case]
    L = pkg.synth.make_layer(cfg)
    x = pkg.synth.make_input(cfg, T=T)
    with pkg.MoeContext(0) as c0:
        c0.upload(0, L)
        ref = c0.ffn(0, x)
    stages = set()
    for n in (1, 2, 3, 4, 6, 9, 12, 16, 20, 25, 30, 40, 50):
        say(f"{case}: PHX_FAULT=malloc:{n}")
        try:
            ctx = make_ctx(pkg, f"malloc:{n}")
        except pkg.OutOfDeviceMemoryError:
            stages.add("create")
            continue
        with ctx:
            try:
                ctx.upload(0, L)
            except pkg.OutOfDeviceMemoryError as e:
                assert "hipErrorOutOfMemory" in str(e) or "OOM" in str(e) or "memory" in str(e).lower()
                stages.add("upload")
                ctx.upload(0, L)
            try:
                out = ctx.ffn(0, x)
            except pkg.OutOfDeviceMemoryError:
                stages.add("ffn")
                out = ctx.ffn(0, x)
            np.testing.assert_array_equal(out, ref, err_msg=f"malloc:{n}")
    say(f"{case}: allocation faults surfaced at {sorted(stages)}")
    assert {"create", "upload", "ffn"} <= stages


@pytest.mark.parametrize("case", list(CASES))
def test_launch_faults(pkg, case):
    cfg, T = CASES[case]
    L = pkg.synth.make_layer(cfg)
    x = pkg.synth.make_input(cfg, T=T)
    with pkg.MoeContext(0) as c0:
        c0.upload(0, L)
        ref = c0.ffn(0, x)
        n_launch = 4 if T <= 16 else 6
    for n in range(1, n_launch + 1):
        say(f"{case}: PHX_FAULT=launch:{n}")
        with make_ctx(pkg, f"launch:{n}") as ctx:
            ctx.upload(0, L)
            with pytest.raises(pkg.GpuDeviceLostError):
                ctx.ffn(0, x)
            np.testing.assert_array_equal(ctx.ffn(0, x), ref, err_msg=f"launch:{n}")


def test_launch_fault_in_stack_capture(pkg):
    """A launch that fails while a stack is captured fails the capture; capturing again works."""
    cfg = dict(pkg.synth.CONFIGS["c5_stack"])
    L = pkg.synth.make_layer(cfg, norms="noisy")
    T = 4
    x = pkg.synth.make_input(cfg, T=T)
    with pkg.MoeContext(0) as c0:
        for i in range(2):
            c0.upload(i, L)
        c0.stack_capture(0, 2, T)
        ref = c0.stack_run(x)
    say("stack: PHX_FAULT=launch:3")
    with make_ctx(pkg, "launch:3") as ctx:
        for i in range(2):
            ctx.upload(i, L)
        with pytest.raises(pkg.GpuDeviceLostError):
            ctx.stack_capture(0, 2, T)
        ctx.stack_capture(0, 2, T)
        np.testing.assert_array_equal(ctx.stack_run(x), ref)
