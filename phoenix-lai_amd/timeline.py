"""Kernel-phase timelines from the instrumented library (libphxmoe_tl.so, `make -C csrc timeline`):
the kernels stamp the 100 MHz wall clock at their phases (TL_STAMP), per workgroup, and this tool runs a
layer and prints, per phase, the earliest / median / latest workgroup stamp.

  python3 phoenix-lai_amd/timeline.py decode [CONFIG [T [noshared]]]   a captured decode stack: per
      layer the router (0: start, 1: x staged, 2: RMS, 4: logit sums and bounds, 5: input blocks
      stored, 3: end), gate|up (0: start, 1: shared unit done, 10: the selection's inputs landed (the
      instrumented build waits for them there), 8: the wave's token ranked, 9: every
      token ranked, 2: selection done, 6: weight loads issued, 7: input in LDS, 3: after the barrier,
      4: chain done, 5: end, 11: the compute unit of each workgroup), down (0: start, 1: input in LDS, 2: chain done, 3: end) and the folded
      combine's phases
      (comb 4: loads in, 5: branch norms, 6: residual norm), µs from the layer's first router workgroup
  python3 phoenix-lai_amd/timeline.py prologue [CONFIG]   the general path's prologue phases (0: start,
      1: mean of squares, 2: router input and normed row in LDS, 3: quantized, 4: end)
  python3 phoenix-lai_amd/timeline.py mfma [CONFIG [fast]]   start and end of every workgroup of the
      prefill matrix-core products (fast: the tolerance mode's), by the tile's active 32-token columns,
      and the count running over time
"""
from __future__ import annotations

import ctypes as C
import os
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
TL_SEQ, TL_KIND, TL_SLOT, TL_WG = 64, 4, 12, 512
N = TL_SEQ * TL_KIND * TL_SLOT * TL_WG


def _package():
    os.environ["PHX_MOE_LIB"] = str(HERE / "libphxmoe_tl.so")
    sys.path.insert(0, str(HERE.parent))
    import __graft_entry__ as ge
    return ge.load_package()


def _reader(lib, name):
    f = getattr(lib, name)
    f.restype = C.c_int
    f.argtypes = [C.c_void_p, C.c_size_t, C.c_int]
    return f


HWID = 1 << 62  # entries holding a workgroup's compute unit (TL_HWID) instead of a time


def _phases(tab, base, kinds, names):
    for k in kinds:
        for sl in range(TL_SLOT):
            v = tab[k, sl]
            if (v & HWID).any():
                _units(tab, k, sl, names[k])
                continue
            v = v[v > 0]
            if v.size:
                v = (v - base) / 100.0
                print(f"   {names[k]:5s} slot {sl}: n={v.size:3d} min {v.min():7.2f} med {np.median(v):7.2f} "
                      f"max {v.max():7.2f}")


def _units(tab, k, sl, name):
    """Workgroups per compute unit from a TL_HWID slot, and the end stamps (slot 5) of those sharing one."""
    ids = tab[k, sl]
    wgs = np.nonzero(ids & HWID)[0]
    cu = ids[wgs] & 0xFFFFF
    uniq, cnt = np.unique(cu, return_counts=True)
    shared = uniq[cnt > 1]
    print(f"   {name:5s} units: {wgs.size} workgroups on {uniq.size} compute units, {shared.size} units with more "
          f"than one")
    for u in shared[:8]:
        w = wgs[cu == u]
        print(f"      unit {int(u):#07x}: workgroups {w.tolist()}")


def decode(cfg="c2_decode", T=1, noshared=False, layers=8):
    pkg = _package()
    S = pkg.synth
    L = S.make_layer(cfg)
    if noshared:
        L["n_ff_shared"] = 0
        for k in ("ffn_norm", "ffn_gate", "ffn_up", "ffn_down"):
            L.pop(k, None)
    ctx = pkg.MoeContext(0)
    for i in range(layers):
        ctx.upload(i, L)
    d = L["d"]
    xs = S.normal(7000, "bench.x", (4, T, d))
    if L.get("biased"):
        xs[:, :, -1] = S.BIAS_X
    xb = ctx.alloc(xs.nbytes)
    xb.upload(xs)
    ctx.stack_capture(0, layers, T)
    rd = _reader(ctx.lib, "phxdbg_timeline")
    buf = np.zeros(N, np.uint64)
    for r in range(20):
        ctx.stack_run_device(xb.ptr + (r % 4) * T * d * 4, T)
    ctx.sync()
    rd(None, 0, 1)
    ctx.stack_run_device(xb.ptr, T)
    ctx.sync()
    rd(buf.ctypes.data, N, 0)
    tl = buf.reshape(TL_SEQ, TL_KIND, TL_SLOT, TL_WG).astype(np.int64)
    print(f"{cfg} T={T}{' without the shared FFN' if noshared else ''}: µs from each layer's first router stamp")
    for seq in range(1, layers - 1):
        base = tl[seq, 0, 0][tl[seq, 0, 0] > 0].min()
        nxt = tl[seq + 1, 0, 0][tl[seq + 1, 0, 0] > 0].min()
        print(f"layer {seq}: the next layer's router starts at {(nxt - base) / 100:.2f}")
        _phases(tl[seq], base, range(4), {0: "route", 1: "gu", 2: "down", 3: "comb"})
    ctx.close()


def prologue(cfg="c3_prefill"):
    pkg = _package()
    S = pkg.synth
    L = S.make_layer(cfg)
    ctx = pkg.MoeContext(0)
    ctx.upload(0, L)
    x = S.make_input(cfg, T=S.CONFIGS[cfg]["T"])
    rd = _reader(ctx.lib, "phxdbg_timeline_general")
    buf = np.zeros(N, np.uint64)
    for _ in range(3):
        ctx.ffn(0, x)
    rd(None, 0, 1)
    ctx.ffn(0, x)
    rd(buf.ctypes.data, N, 0)
    tl = buf.reshape(TL_SEQ, TL_KIND, TL_SLOT, TL_WG).astype(np.int64)
    base = tl[0, 0, 0][tl[0, 0, 0] > 0].min()
    print(f"{cfg}: prologue phases, µs from the first workgroup's start (workgroups below {TL_WG})")
    _phases(tl[0], base, [0], {0: "pro"})
    ctx.close()


def mfma(cfg="c3_prefill", fast=False):
    pkg = _package()
    S = pkg.synth
    L = S.make_layer(cfg)
    ctx = pkg.MoeContext(0)
    ctx.upload(0, L)
    x = S.make_input(cfg, T=S.CONFIGS[cfg]["T"])
    rd = _reader(ctx.lib, "phxdbg_timeline_prefill")
    buf = np.zeros(N, np.uint64)
    for _ in range(3):
        ctx.ffn(0, x, fast_math=fast)
    rd(None, 0, 1)
    ctx.ffn(0, x, fast_math=fast)
    rd(buf.ctypes.data, N, 0)
    _, _, off, _, _ = ctx.routing()
    A = 128
    full, parts = [], {1: [], 2: [], 3: [], 4: []}  # the dispatch's order: full tiles, then partial by size
    for c in np.diff(off).tolist():
        full += [A] * (c // A)
        if c % A:
            parts[min(4, (4 * (c % A) + A - 1) // A)].append(c % A)
    tiles = full + parts[4] + parts[3] + parts[2] + parts[1]
    per = 4 if fast else 2  # row groups per workgroup
    for name, base, gx in (("gate_up", 0, (L["n_ff"] // 32 + per - 1) // per), ("down", 16384, (L["d"] // 64 + per - 1) // per)):
        st = buf[base:base + 16384].astype(np.int64).reshape(-1, 2)
        ok = np.nonzero(st[:, 0] > 0)[0]
        s0, s1 = st[ok, 0], st[ok, 1]
        t0 = s0.min()
        dur = (s1 - s0) / 100.0
        nj = np.array([(tiles[i // gx] + 31) // 32 for i in ok])
        print(f"{name}: {ok.size} workgroups, span {(s1.max() - t0) / 100:.1f} µs")
        for j in range(1, 5):
            m = nj == j
            if m.any():
                print(f"   NJ={j}: {m.sum():4d} workgroups, duration median {np.median(dur[m]):6.1f} µs, "
                      f"min {dur[m].min():6.1f}, max {dur[m].max():6.1f}")
        r0, r1 = (s0 - t0) / 100.0, (s1 - t0) / 100.0
        edges = np.linspace(0.0, r1.max(), 21)
        run = [int(((r0 <= (a + b) / 2) & (r1 > (a + b) / 2)).sum()) for a, b in zip(edges[:-1], edges[1:])]
        print("   workgroups running over twenty time bins:", run)
    ctx.close()


if __name__ == "__main__":
    a = sys.argv[1:] or ["decode"]
    if a[0] == "decode":
        decode(a[1] if len(a) > 1 else "c2_decode", int(a[2]) if len(a) > 2 else 1, len(a) > 3 and a[3] == "noshared")
    elif a[0] == "prologue":
        prologue(*a[1:2])
    elif a[0] == "mfma":
        mfma(a[1] if len(a) > 1 else "c3_prefill", len(a) > 2 and a[2] == "fast")
    else:
        sys.exit(__doc__)
