#!/usr/bin/env python3
"""Benchmark of the MoE FFN layer on one MI355X (libphxmoe.so through its C ABI).

Default workload: decode, T=1 token, d=2816, E=128 experts, top-8,
expert ffn 704, Q4_0 experts plus the dense shared FFN (ffn 2112, Q4_0), synthetic N(0,0.02)
weights.  One step = one MoE FFN layer applied to the T tokens.  The layer is placed in up to 32
distinct layer slots (as many as divide --steps, so exactly --steps layer steps are timed) and the
slots are captured as one HIP graph (the reference replays one recorded command buffer per decode
pass, src/GemmaGpu.cs:544-554); every replay starts from a different input, so the experts touched
change from replay to replay and the 256 MB MALL cannot serve them.

Prints one JSON line: value = tokens/s through the layer (inputs resident in HBM), a roofline
object for the dominant kernel (the grouped gate|up product: algorithmic bytes per launch over its
average duration, each launch's execution interval stamped by HIP events on the library's stream,
the interval a kernel-trace profiler reports), the CPU baseline (the C restatement of the reference
CPU path timed on this host's cores over a bounded sample), and three objects measured in the same
run: `prefill` for configs[2] (T=2048, Zipf routing: tokens/s and the matrix-core utilisation of the
grouped gate|up and down products), `kquant` for configs[3] (T=512, Q4_K gate|up and Q6_K down:
tokens/s, weight GB/s and matrix-core rates) and `stack` for configs[4] (30 Q8_0 layers at T=32 with a
hot expert, captured as one HIP graph: the step's latency and GB/s over the distinct experts read).

Kernel durations come from a fixed sample of eager layer calls (--prof-steps, 200 by default, after 20
unprofiled calls), independent of --steps, each launch's execution interval stamped by HIP events.

`--config quant` measures the ops either side of the layer instead (the activation quantizers, the
residual norm-add with the quantized next input and the dense matvec): one JSON line of the same form
whose value is the GELU-gated Q8_0 quantizer's GB/s at C3's down-input shape, with every other mode
and op under "modes_2048_rows".
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0  # dense fp16 / bf16 MFMA, MI355X

METRIC = "MoE layer tokens/s; decode HBM GB/s vs peak; prefill MFMA util"

# HBM bytes per launch of the roofline kernel, from two rocprofv3 counter runs (FETCH_SIZE, then
# WRITE_SIZE) of this file with --calibrate, each scaled by what the counter reads for the library's
# streaming read and copy kernels of known size (fetch factor 2.000, write factor 1.000).  Keyed by
# (config, T, kernel); re-measured whenever that kernel changes.
PMC_TRAFFIC = {
    # FETCH_SIZE 12,377.4 KiB x 2.000 + WRITE_SIZE 86.6 KiB x 1.000 per launch of phx::k_dec_gu<2>
    ("c2_decode", 1, "gate_up"): (25_432_268, "rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, 392 launches each"),
}


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def expert_bytes(L) -> tuple[int, int]:
    """(gate|up bytes, down bytes) of one expert in GGUF block sizes."""
    from phoenix_lai_amd import synth as S  # noqa
    gu = 2 * L["n_ff"] * S.row_bytes(L["gate_up_type"], L["d"])
    dn = L["d"] * S.row_bytes(L["down_type"], L["n_ff"] if L["down_cols"] == L["n_ff"] else L["down_cols"])
    if L["down_cols"] != L["n_ff"]:
        # algorithmic bytes count the unpadded K (the padding is a layout extension)
        dn = int(dn * L["n_ff"] / L["down_cols"])
    return gu, dn


def host_cpu():
    """(threads to use, description): every core this process may run on, capped by OMP_NUM_THREADS when
    the environment sets it (the GPU boxes give a job a fixed share of the host)."""
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = os.cpu_count() or 1
    omp = os.environ.get("OMP_NUM_THREADS")
    threads = min(affinity, int(omp)) if omp and omp.isdigit() and int(omp) > 0 else affinity
    model = "unknown"
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return threads, {"nproc": os.cpu_count(), "affinity_cores": affinity, "omp_num_threads": omp, "cpu_model": model}


def cpu_baseline(pkg, L, cfg_name, budget_s=12.0):
    """The oracle (C restatement of GemmaCpu.MoeFfn, row-parallel like Parallel.For) on this host, one token
    at a time as the reference's CPU path runs (GemmaCpu.Prefill), over a bounded sample of the workload."""
    from oracle import oracle as orc
    threads, host = host_cpu()
    S = pkg.synth
    pool = 1024  # distinct tokens; the sample cycles through them until the time budget is spent
    x = S.make_input(cfg_name, T=pool, seed=4242, name="cpu.x")
    orc.moe_block(L, x[:1], nthreads=threads)  # warm-up
    n, t0 = 0, time.perf_counter()
    while time.perf_counter() - t0 < budget_s:
        orc.moe_block(L, x[n % pool:n % pool + 1], nthreads=threads)
        n += 1
    dt = time.perf_counter() - t0
    return {"value": round(n / dt, 3), "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"{n} tokens of {cfg_name} one at a time (as GemmaCpu.Prefill does)"
                      + (", shared FFN included" if L.get("n_ff_shared") else "")
                      + f", {dt:.1f} s, OpenMP over rows with {threads} threads", **host}


def graph_slots(steps: int, max_slots: int) -> int:
    """Layer slots of the replayed graph: the largest count <= max_slots that divides steps, so the timed
    region is exactly `steps` layer steps of whole replays; if that is below 4, max_slots (the remainder
    then runs as eager layer calls inside the timed region)."""
    best = max(s for s in range(1, max_slots + 1) if steps % s == 0)
    return best if best >= 4 else max_slots


def decode_roofline(pkg, L, cfg_name, T, avg_experts, gu_ms):
    S = pkg.synth
    gu_b, _ = expert_bytes(L)
    sh_gu_b = 2 * L["n_ff_shared"] * S.row_bytes(L["shared_type"], L["d"]) if L.get("n_ff_shared") else 0
    gu_bytes = avg_experts * gu_b + sh_gu_b
    achieved = gu_bytes / (gu_ms * 1e-3) / 1e9
    tr = PMC_TRAFFIC.get((cfg_name, T, "gate_up"), (None, None))
    return {
        "bound": "hbm",
        "kernel": "phx::k_dec_gu (grouped Q4_0 x Q8_0 gate|up row products, decode)" if L["gate_up_type"] == 2
        else "phx::k_dec_gu (decode gate|up)",
        "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": tr[0], "traffic_source": tr[1],
        "bytes_per_launch": int(gu_bytes), "avg_launch_us": round(gu_ms * 1e3, 3),
        "per_unit": f"{gu_b} B of gate|up weights per touched expert x {avg_experts:.2f} experts per launch"
                    + (f" + {sh_gu_b} B of shared-FFN gate and up weights" if sh_gu_b else ""),
    }


def mfma_rates(L, T, gu_ms, dn_ms):
    """Matrix-core rates of the grouped products: 2 flops per multiply-add of the routed experts' gate|up
    (2 nf x d per assignment) and down (d x nf) products, against the dense fp16 peak (the operands are
    exact integers in fp16)."""
    n = T * L["n_used"]
    gu_ops = 2.0 * n * 2 * L["n_ff"] * L["d"]
    dn_ops = 2.0 * n * L["d"] * L["n_ff"]
    gu_t, dn_t = gu_ops / (gu_ms * 1e-3) / 1e12, dn_ops / (dn_ms * 1e-3) / 1e12
    return {"gate_up_tflops": round(gu_t, 2), "gate_up_frac_fp16_peak": round(gu_t / FP16_PEAK_TFLOPS, 4),
            "gate_up_avg_us": round(gu_ms * 1e3, 2), "gate_up_flops_per_launch": int(gu_ops),
            "down_tflops": round(dn_t, 2), "down_frac_fp16_peak": round(dn_t / FP16_PEAK_TFLOPS, 4),
            "down_avg_us": round(dn_ms * 1e3, 2), "down_flops_per_launch": int(dn_ops)}


def kernel_times(ctx, calls):
    """Run `calls` (eager layer calls) with profiling on: every kernel's own execution interval, summed
    per kind; returns {kind: (avg ms per launch, launches)}."""
    ctx.profile(True)
    calls()
    ctx.sync()
    prof = ctx.profile_read()
    ctx.profile(False)
    return {k: (v[0] / v[1], v[1]) for k, v in prof.items() if v[1]}


def side_objects(args, pkg):
    """The other configurations' objects of the default run (C3, C4, C5), each with its own context."""
    out = {}
    if not args.no_prefill:
        log("[bench] prefill (configs[2], T=2048) ...")
        out["prefill"] = run_prefill(args, pkg)
    if not args.no_kquant:
        log("[bench] K-quant layer (configs[3], T=512) ...")
        out["kquant"] = run_prefill(args, pkg, "c4_kquant", args.kquant_steps)
    if not args.no_stack:
        log("[bench] 30-layer stack (configs[4], T=32) ...")
        out["stack"] = run_stack(args, pkg)
    return out


def run_layer(args, pkg):
    S = pkg.synth
    cfg_name = args.config
    cfg = S.CONFIGS[cfg_name]
    T = args.T or cfg["T"]
    steps = args.steps
    n_slots = args.layers or graph_slots(steps, cfg.get("layers", 32))
    # the default run measures the other configurations first: the decode line is then timed on a GPU
    # already running at its working clocks, as a serving loop would be, whatever --steps is
    side = side_objects(args, pkg) if cfg_name == "c2_decode" else {}
    log(f"[bench] generating {cfg_name} layer ...")
    L = S.make_layer(cfg_name)
    ctx = pkg.MoeContext(0)
    log(f"[bench] uploading {n_slots} layer slots ...")
    for i in range(n_slots):
        ctx.upload(i, L)
    d, E, k = L["d"], L["n_expert"], L["n_used"]
    NX = int(min(64, max(4, (512 << 20) // (T * d * 4))))  # distinct inputs, cycled through the replays
    xs = S.normal(cfg["idx"] + 7000, "bench.x", (NX, T, d))
    if L.get("biased"):
        xs[:, :, -1] = S.BIAS_X
    xbuf = ctx.alloc(xs.nbytes)
    xbuf.upload(xs)
    obuf = ctx.alloc(T * d * 4)
    xstride = T * d * 4
    RES_ASYNC = pkg.PHX.FLAG_RESIDUAL | pkg.PHX.FLAG_ASYNC

    # ---- timed region: exactly `steps` layer steps: whole replays of the n_slots-layer graph, then any
    # remainder as eager layer calls (each with the residual update the graph's layers apply)
    ctx.stack_capture(0, n_slots, T)
    reps, rem = divmod(steps, n_slots)
    wreps = max(1, (args.warmup + n_slots - 1) // n_slots)
    for r in range(wreps):
        ctx.stack_run_device(xbuf.ptr + (r % NX) * xstride, T)
    ctx.sync()
    fb0 = ctx.fallback_counts()
    t0 = time.perf_counter()
    for r in range(reps):
        ctx.stack_run_device(xbuf.ptr + (r % NX) * xstride, T)
    for s in range(rem):
        ctx.ffn_device(s, T, xbuf.ptr + ((reps + s) % NX) * xstride, None, obuf.ptr, RES_ASYNC)
    ctx.sync()
    dt = time.perf_counter() - t0
    # tokens whose routing the certified router could not certify (their ambiguous experts' exact chains
    # ran) in the timed steps
    fb_tokens = ctx.fallback_counts()[1] - fb0[1]
    ms_per_step = dt * 1e3 / steps
    tokens_s = T * steps / dt

    # ---- per-kernel durations: eager layer calls over the slots and inputs, every launch stamped with
    # its own execution interval (hipExtLaunchKernel events on the library's stream); a fixed sample after
    # unprofiled warm-up calls, whatever --steps is
    prof_steps = max(1, args.prof_steps)
    for s in range(20):
        ctx.ffn_device(s % n_slots, T, xbuf.ptr + (s % NX) * xstride, None, obuf.ptr, RES_ASYNC)

    def prof_calls():
        for s in range(prof_steps):
            ctx.ffn_device(s % n_slots, T, xbuf.ptr + (s % NX) * xstride, None, obuf.ptr, RES_ASYNC)

    prof = kernel_times(ctx, prof_calls)
    # experts touched per step (the routing of each step read back)
    distinct = 0
    n_route = min(prof_steps, 64)
    for s in range(n_route):
        ctx.ffn_device(s % n_slots, T, xbuf.ptr + (s % NX) * xstride, None, obuf.ptr, pkg.PHX.FLAG_ASYNC)
        distinct += len(np.unique(ctx.routing()[0]))
    avg_experts = distinct / n_route
    gu_ms, dn_ms = prof["gate_up"][0], prof["down"][0]
    decode = "dispatch" not in prof  # the decode path has no separate dispatch launch
    mfma = (not decode and L["gate_up_type"] in (pkg.PHX.Q4_0, pkg.PHX.Q8_0)
            and L["down_type"] in (pkg.PHX.Q4_0, pkg.PHX.Q8_0) and T * k >= 8 * E)
    kmma = (not decode and L["gate_up_type"] in (pkg.PHX.Q4_K, pkg.PHX.Q6_K)
            and L["down_type"] in (pkg.PHX.Q4_K, pkg.PHX.Q6_K) and T * k >= 8 * E)
    gu_b, dn_b = expert_bytes(L)
    sh_bytes = 0
    if L.get("n_ff_shared"):
        sh_bytes = 3 * L["n_ff_shared"] * S.row_bytes(L["shared_type"], d)
    layer_expert_bytes = avg_experts * (gu_b + dn_b)
    router_bytes = E * d * 4
    if mfma:
        rates = mfma_rates(L, T, gu_ms, dn_ms)
        roofline = {"bound": "mfma", "kernel": "phx::k_grouped_mfma gate|up (fp16 MFMA on exact integer operands: "
                                               "block sums, scale products, reference float chain)",
                    "achieved": rates["gate_up_tflops"], "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": rates["gate_up_frac_fp16_peak"], "traffic": None,
                    "ops_per_launch": rates["gate_up_flops_per_launch"], "avg_launch_us": rates["gate_up_avg_us"],
                    "per_unit": f"2 x {2 * L['n_ff']} x {d} flops per assignment x {T * k} assignments per launch"}
        down_rate = {"down_tflops": rates["down_tflops"]}
    elif kmma:
        rates = mfma_rates(L, T, gu_ms, dn_ms)
        gu_gbs = avg_experts * gu_b / (gu_ms * 1e-3) / 1e9
        roofline = {"bound": "mfma", "kernel": "phx::k_grouped_kmma gate|up (K-quant integer lanes on fp16 MFMA, "
                                               "DotK's float lane chains on VALU)",
                    "achieved": rates["gate_up_tflops"], "peak": FP16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": rates["gate_up_frac_fp16_peak"], "traffic": None,
                    "ops_per_launch": rates["gate_up_flops_per_launch"], "avg_launch_us": rates["gate_up_avg_us"],
                    "per_unit": f"2 x {2 * L['n_ff']} x {d} flops per assignment x {T * k} assignments per launch",
                    "hbm": {"achieved_gbs": round(gu_gbs, 1), "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                            "bytes_per_launch": int(avg_experts * gu_b)},
                    "note": "the reference's per-lane float chain (2 rounded VALU operations per row, assignment, "
                            "lane and super-block) bounds this kernel, not the matrix cores"}
        down_rate = {"down_tflops": rates["down_tflops"]}
    else:
        roofline = decode_roofline(pkg, L, cfg_name, T, avg_experts, gu_ms) if decode else {
            "bound": "hbm", "kernel": f"gate_up (grouped {qname(L['gate_up_type'])} row products, VALU)",
            "achieved": round(avg_experts * gu_b / (gu_ms * 1e-3) / 1e9, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(avg_experts * gu_b / (gu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
            "bytes_per_launch": int(avg_experts * gu_b), "avg_launch_us": round(gu_ms * 1e3, 3),
            "per_unit": f"{gu_b} B of gate|up weights per touched expert x {avg_experts:.2f} experts per launch"}
        dn_bytes = avg_experts * dn_b + (L["d"] * S.row_bytes(L["shared_type"], L["n_ff_shared"])
                                         if decode and L.get("n_ff_shared") else 0)
        down_rate = {"down_gbs": round(dn_bytes / (dn_ms * 1e-3) / 1e9, 1)}

    # ---- the same layer called with host buffers (the C# host's boundary: x and the output cross PCIe
    # inside every call, which also waits for completion); a side figure, never `value`
    n_host = max(5, min(200, int(0.5 / max(ms_per_step * 1e-3, 1e-6))))
    for s in range(n_slots):  # the first call of each (layer, T) captures its graph: outside the timing
        ctx.ffn(s, xs[s % NX])
    th = time.perf_counter()
    for s in range(n_host):
        ctx.ffn(s % n_slots, xs[s % NX])
    host_dt = time.perf_counter() - th
    pcie = {"tokens_s": round(T * n_host / host_dt, 1), "us_per_call": round(host_dt / n_host * 1e6, 2),
            "note": "phx_moe_ffn on host x/out through Python (pinned staging, the layer call replayed as a graph, "
                    "one wait per call)"}

    # ---- measured streaming-read rate of this box (2 GiB, coalesced 128-bit loads)
    sbuf = ctx.alloc(2 << 30)
    sread_ms = ctx.stream_read_ms(sbuf, 10)
    stream_gbs = (2 << 30) / (sread_ms * 1e-3) / 1e9
    sbuf.free()

    kernels = {k_: {"avg_us": round(v[0] * 1e3, 2), "launches": v[1]} for k_, v in prof.items()}
    line = {
        "metric": METRIC,
        "value": round(tokens_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": wreps * n_slots,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16" if mfma or kmma else "int8",  # the products' arithmetic: fp16 MFMA, or int8 dot4 on VALU
        "data": "synthetic",
        "config": {
            "workload": f"{cfg_name}: MoE FFN layer, T={T}, d={d}, E={E}, top-{k}, "
                        f"expert ffn {L['n_ff']}, {qname(L['gate_up_type'])}/{qname(L['down_type'])} experts"
                        + (f", shared FFN {L['n_ff_shared']} {qname(L['shared_type'])}" if sh_bytes else "")
                        + (", Zipf(1.1) router bias" if cfg.get("zipf") else "")
                        + (f", hot expert {cfg['hot']:.0%} of tokens" if cfg.get("hot") else "")
                        + f"; {n_slots} layer slots replayed as one HIP graph ({reps} replays"
                        + (f" + {rem} eager layer calls" if rem else "") + "), x varied per replay",
            "global_batch": T,
            "parallelism": "none (1 GPU)",
            "path": "decode" if decode else ("mfma" if mfma or kmma else "valu"),
        },
        "roofline": roofline,
        "layer": {
            "expert_bytes_per_step": int(layer_expert_bytes),
            "expert_gbs": round(layer_expert_bytes / (ms_per_step * 1e-3) / 1e9, 1),
            "all_bytes_gbs": round((layer_expert_bytes + sh_bytes + router_bytes) / (ms_per_step * 1e-3) / 1e9, 1),
            "expert_gbs_frac_of_peak": round(layer_expert_bytes / (ms_per_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "distinct_experts_per_step": round(avg_experts, 2),
            "down_avg_us": round(dn_ms * 1e3, 3),
            **down_rate,
            "kernels": kernels,
            "kernel_timing": f"{prof_steps} eager layer calls after 20 unprofiled ones, each kernel's execution "
                             f"interval",
            "router_fallback_token_frac": round(fb_tokens / (T * steps), 4),
            "stream_read_gbs_measured": round(stream_gbs, 1),
            "pcie_inclusive": pcie,
        },
    }
    if args.calibrate:
        line["calibration"] = calibration_kernels(ctx)
    ctx.close()
    if not args.no_cpu:
        log("[bench] CPU baseline ...")
        line["cpu_baseline"] = cpu_baseline(pkg, L, cfg_name, args.cpu_seconds)
    del L
    line.update(side)
    return line


def run_prefill(args, pkg, cfg_name="c3_prefill", steps=None):
    """A many-token config in the same run, one eager layer call per step (inputs resident in HBM), the
    grouped products on the matrix cores: configs[2] (T = 2048 tokens with Zipf(1.1) expert popularity,
    Q4_0) or configs[3] (T = 512, Q4_K gate|up and Q6_K down, uniform router)."""
    S = pkg.synth
    cfg = S.CONFIGS[cfg_name]
    T = cfg["T"]
    L = S.make_layer(cfg_name)
    ctx = pkg.MoeContext(0)
    ctx.upload(0, L)
    NX = 4
    xs = S.normal(cfg["idx"] + 7000, "bench.x", (NX, T, L["d"]))
    if L.get("biased"):
        xs[:, :, -1] = S.BIAS_X
    xbuf = ctx.alloc(xs.nbytes)
    xbuf.upload(xs)
    obuf = ctx.alloc(T * L["d"] * 4)
    xstride = T * L["d"] * 4
    steps = steps or args.prefill_steps
    for s in range(3):
        ctx.ffn_device(0, T, xbuf.ptr + (s % NX) * xstride, None, obuf.ptr, pkg.PHX.FLAG_ASYNC)
    ctx.sync()
    fb0 = ctx.fallback_counts()[1]
    t0 = time.perf_counter()
    for s in range(steps):
        ctx.ffn_device(0, T, xbuf.ptr + (s % NX) * xstride, None, obuf.ptr, pkg.PHX.FLAG_ASYNC)
    ctx.sync()
    dt = time.perf_counter() - t0
    fb_tokens = ctx.fallback_counts()[1] - fb0

    def calls():
        for s in range(steps):
            ctx.ffn_device(0, T, xbuf.ptr + (s % NX) * xstride, None, obuf.ptr, pkg.PHX.FLAG_ASYNC)

    prof = kernel_times(ctx, calls)
    ids = ctx.routing()[0]
    cnt = np.bincount(ids.ravel(), minlength=L["n_expert"])
    fast, fast_sample = None, None
    if L["gate_up_type"] in (pkg.PHX.Q4_0, pkg.PHX.Q8_0, pkg.PHX.Q4_K, pkg.PHX.Q6_K) and not args.no_fast_math:
        fast, fast_sample = fast_math_object(args, pkg, ctx, L, xbuf, obuf, xs, steps)
    ctx.close()
    gu_b, dn_b = expert_bytes(L)
    touched = int((cnt > 0).sum())
    gu_ms, dn_ms = prof["gate_up"][0], prof["down"][0]
    layer_s = dt / steps
    out = {"workload": f"{cfg_name}: T={T}, d={L['d']}, E={L['n_expert']}, top-{L['n_used']}, expert ffn {L['n_ff']}, "
                       f"{qname(L['gate_up_type'])}/{qname(L['down_type'])}"
                       + (", Zipf(1.1) router bias" if cfg.get("zipf") else ", uniform router")
                       + (f" (down K padded {L['n_ff']} -> {L['down_cols']})" if L["down_cols"] != L["n_ff"] else "")
                       + f"; {steps} eager layer calls, inputs in HBM",
           "tokens_s": round(T * steps / dt, 1), "ms_per_step": round(dt * 1e3 / steps, 4), "steps": steps,
           **mfma_rates(L, T, gu_ms, dn_ms),
           "hbm": {"expert_bytes_per_step": touched * (gu_b + dn_b),
                   "layer_gbs": round(touched * (gu_b + dn_b) / layer_s / 1e9, 1),
                   "gate_up_gbs": round(touched * gu_b / (gu_ms * 1e-3) / 1e9, 1),
                   "gate_up_frac": round(touched * gu_b / (gu_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                   "down_gbs": round(touched * dn_b / (dn_ms * 1e-3) / 1e9, 1),
                   "floor_us": round(touched * (gu_b + dn_b) / (HBM_PEAK_GBS * 1e9) * 1e6, 1),
                   "note": "unpadded GGUF bytes of the experts with at least one assignment"},
           "kernels": {k_: {"avg_us": round(v[0] * 1e3, 2), "launches": v[1]} for k_, v in prof.items()},
           "kernel_timing": f"{steps} eager layer calls, each kernel's execution interval; 'router' is the "
                            f"certified router's matrix-core sums, 'topk' its selection (exact chains for the "
                            f"tokens the bounds leave open); the prologue runs on a side stream beside them, so "
                            f"its interval overlaps theirs",
           "router_fallback_token_frac": round(fb_tokens / (T * steps), 4),
           "assignments_per_expert": {"max": int(cnt.max()), "empty_experts": int((cnt == 0).sum())}}
    if fast:
        out["fast_math"] = fast
    if not args.no_cpu:
        log(f"[bench] {cfg_name} CPU baseline ...")
        out["cpu_baseline"] = cpu_baseline(pkg, L, cfg_name, min(args.cpu_seconds, 6.0 if cfg_name == "c3_prefill" else 3.0))
        if fast:
            fast["error_vs_cpu_reference"] = fast_math_error(L, fast_sample)
    return out


def fast_math_object(args, pkg, ctx, L, xbuf, obuf, xs, steps):
    """The same layer in the tolerance mode (PHX_FLAG_FAST_MATH: block scales folded into fp16 operands,
    rows accumulated on the matrix cores), timed the same way; returns the object and a token sample of
    its outputs (inputs, outputs), which the CPU leg compares with the CPU reference."""
    T, d = xs.shape[1], L["d"]
    xstride = T * d * 4
    FM = pkg.PHX.FLAG_FAST_MATH | pkg.PHX.FLAG_ASYNC
    for s in range(3):
        ctx.ffn_device(0, T, xbuf.ptr + (s % len(xs)) * xstride, None, obuf.ptr, FM)
    ctx.sync()
    t0 = time.perf_counter()
    for s in range(steps):
        ctx.ffn_device(0, T, xbuf.ptr + (s % len(xs)) * xstride, None, obuf.ptr, FM)
    ctx.sync()
    dt = time.perf_counter() - t0

    def calls():
        for s in range(steps):
            ctx.ffn_device(0, T, xbuf.ptr + (s % len(xs)) * xstride, None, obuf.ptr, FM)

    prof = kernel_times(ctx, calls)
    out = {"tokens_s": round(T * steps / dt, 1), "ms_per_step": round(dt * 1e3 / steps, 4),
           **mfma_rates(L, T, prof["gate_up"][0], prof["down"][0]),
           "kernels": {k_: {"avg_us": round(v[0] * 1e3, 2), "launches": v[1]} for k_, v in prof.items()}}
    # one more call on the first input (the calls leave their inputs unchanged): a token sample of its
    # outputs, compared with the CPU reference in the CPU leg (fast_math_error)
    ctx.ffn_device(0, T, xbuf.ptr, None, obuf.ptr, FM)
    ctx.sync()
    toks = np.arange(0, T, max(1, T // 32))
    return out, (xs[0][toks], obuf.download((T, d))[toks])


def fast_math_error(L, sample):
    """The CPU leg's check of the tolerance mode: the oracle's outputs for the sampled tokens against the
    GPU's (the mode is not bit-exact; routing still is)."""
    from oracle import oracle as orc
    x, got = sample
    threads, _ = host_cpu()
    ref, _, _ = orc.moe_block(L, x, nthreads=threads)
    err = np.abs(got.astype(np.float64) - ref)
    rms = float(np.sqrt(np.mean(ref.astype(np.float64) ** 2)))
    return {"tokens": int(len(x)), "max_abs": round(float(err.max()), 6),
            "rms": round(float(np.sqrt(np.mean(err ** 2))), 6), "output_rms": round(rms, 4),
            "within_2e-3_bar_frac": round(float((err <= np.maximum(2e-3 * np.abs(ref), 1e-4)).mean()), 4)}


def run_stack(args, pkg, cfg_name="c5_stack"):
    """configs[4] in the same run: 30 consecutive Q8_0 MoE layers, each with its RmsNorm and residual
    (GemmaCpu.cs:355-356), over T = 32 independent tokens with one hot expert, captured as ONE HIP graph
    of the 30-layer step and replayed (inputs resident in HBM, x varied per replay).  Layers have their own
    routers and norms; the expert weights are one generated set uploaded into 30 distinct device copies
    (synth.make_stack), so every step reads 30 layers' experts from HBM."""
    S = pkg.synth
    cfg = S.CONFIGS[cfg_name]
    T, n_layers = cfg["T"], cfg["layers"]
    layers = S.make_stack(cfg_name, n_layers)
    ctx = pkg.MoeContext(0)
    for i, L in enumerate(layers):
        ctx.upload(i, L)
    L0 = layers[0]
    d = L0["d"]
    NX = 8
    xs = S.normal(cfg["idx"] + 7000, "bench.x", (NX, T, d))
    xs[:, :, -1] = S.BIAS_X
    xbuf = ctx.alloc(xs.nbytes)
    xbuf.upload(xs)
    xstride = T * d * 4
    ctx.stack_capture(0, n_layers, T)
    for r in range(3):
        ctx.stack_run_device(xbuf.ptr + (r % NX) * xstride, T)
    ctx.sync()
    xbuf.upload(xs)
    steps = args.stack_steps
    fb0 = ctx.fallback_counts()
    t0 = time.perf_counter()
    for r in range(steps):
        ctx.stack_run_device(xbuf.ptr + (r % NX) * xstride, T)
    ctx.sync()
    dt = time.perf_counter() - t0
    fb_tokens = ctx.fallback_counts()[1] - fb0[1]
    # one step replayed layer by layer (the same calls the graph holds) for the experts each layer touches
    # and the per-kernel durations
    xbuf.upload(xs)
    obuf = ctx.alloc(T * d * 4)
    res = pkg.PHX.FLAG_RESIDUAL | pkg.PHX.FLAG_ASYNC
    touched = []
    for i in range(n_layers):
        ctx.ffn_device(i, T, xbuf.ptr, None, obuf.ptr, res)
        touched.append(len(np.unique(ctx.routing()[0])))

    def calls():
        for r in range(2):
            for i in range(n_layers):
                ctx.ffn_device(i, T, xbuf.ptr + (r % NX) * xstride, None, obuf.ptr, res)

    prof = kernel_times(ctx, calls)
    ctx.close()
    gu_b, dn_b = expert_bytes(L0)
    step_bytes = sum(touched) * (gu_b + dn_b)
    step_s = dt / steps
    out = {"workload": f"{cfg_name}: {n_layers} MoE layers (RmsNorm + residual each), T={T}, d={d}, "
                       f"E={L0['n_expert']}, top-{L0['n_used']}, expert ffn {L0['n_ff']}, "
                       f"{qname(L0['gate_up_type'])}, hot expert {cfg['hot']:.0%} of tokens; the {n_layers}-layer "
                       f"step captured as one HIP graph, {steps} replays, x varied per replay",
           "ms_per_step": round(step_s * 1e3, 4), "tokens_s": round(T / step_s, 1),
           "layer_us": round(step_s * 1e6 / n_layers, 2), "steps": steps,
           "distinct_experts_per_layer": round(sum(touched) / n_layers, 2),
           "expert_bytes_per_step": step_bytes,
           "expert_gbs": round(step_bytes / step_s / 1e9, 1),
           "expert_gbs_frac_of_peak": round(step_bytes / step_s / 1e9 / HBM_PEAK_GBS, 4),
           "hbm_floor_ms": round(step_bytes / (HBM_PEAK_GBS * 1e9) * 1e3, 3),
           "router_fallback_token_frac": round(fb_tokens / (T * n_layers * steps), 4),
           "kernels": {k_: {"avg_us": round(v[0] * 1e3, 2), "launches": v[1]} for k_, v in prof.items()},
           "kernel_timing": f"{2 * n_layers} eager layer calls, each kernel's execution interval"}
    if not args.no_cpu:
        log("[bench] stack CPU baseline ...")
        cb = cpu_baseline(pkg, L0, cfg_name, min(args.cpu_seconds, 3.0))
        cb["note"] = "tokens/s through one layer; a 30-layer step is 30 such layer-tokens per token"
        out["cpu_baseline"] = cb
    return out


QUANT_MODES = {"plain": 0, "silu_mul": 1, "rms_norm": 2, "gelu_mul": 3}


def run_quant(args, pkg):
    """The standalone activation quantizers (phx_quant_q8_0 / phx_quant_q8_k, KernelsQuant.Q80 / Q8K)
    at the C3 prefill shapes: gelu(g) * u of 2048 x 8 assignment rows of 704 into Q8_0 (the
    down input; the line's value), and every mode and format over 2048 token rows of 2816 (Q8_K:
    3072).  HBM-bound: algorithmic bytes = the float inputs read once + the quants, scales and block
    sums written, per launch; the time of a launch is the wall clock over `iters` back-to-back
    launches on the library's stream, inputs resident in HBM."""
    ctx = pkg.MoeContext(0)
    rng = np.random.default_rng(11)
    iters = max(20, args.steps // 20)

    def one(k_quant, mode, rows, n):
        x = (rng.standard_normal((rows, n)) * 2).astype(np.float32)
        aux = rng.standard_normal(n if mode == 2 else (rows, n)).astype(np.float32) if mode else None
        nd = rows * n // (256 if k_quant else 32)
        bufs = [ctx.alloc(x.nbytes), ctx.alloc(rows * n), ctx.alloc(nd * (4 if k_quant else 2))]
        bufs[0].upload(x)
        aux_ptr = bs_ptr = None
        if aux is not None:
            bufs.append(ctx.alloc(aux.nbytes))
            bufs[-1].upload(aux)
            aux_ptr = bufs[-1].ptr
        if k_quant:
            bufs.append(ctx.alloc(rows * n // 16 * 2))
            bs_ptr = bufs[-1].ptr
        run = lambda: ctx.quant_device(k_quant, mode, bufs[0].ptr, aux_ptr, rows, n, 1e-6, bufs[1].ptr, bufs[2].ptr,
                                       bs_ptr)
        for _ in range(max(3, args.warmup // 100)):
            run()
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(iters):
            run()
        ctx.sync()
        us = (time.perf_counter() - t0) / iters * 1e6
        nbytes = x.nbytes + (aux.nbytes if aux is not None and mode != 2 else 0) + rows * n + nd * (4 if k_quant else 2)
        nbytes += rows * n // 16 * 2 if k_quant else 0
        for b in bufs:
            b.free()
        return us, nbytes

    us, nbytes = one(False, 3, 2048 * 8, 704)
    gbs = nbytes / us / 1e3
    modes = {}
    for name, m in QUANT_MODES.items():
        for k_quant, n in ((False, 2816), (True, 3072)):
            u, b = one(k_quant, m, 2048, n)
            modes[f"{'q8_k' if k_quant else 'q8_0'}_{name}"] = {"us": round(u, 2), "gbs": round(b / u / 1e3, 1)}
    for rows in (1, 2048):  # NormAddQuant: the decode step's single row, and a prefill batch
        n = 2816
        x = ctx.alloc(rows * n * 4)
        y = ctx.alloc(rows * n * 4)
        w = ctx.alloc(n * 4)
        w2 = ctx.alloc(n * 4)
        qs, dq = ctx.alloc(rows * n), ctx.alloc(rows * n // 16)
        x.upload((rng.standard_normal((rows, n))).astype(np.float32))
        y.upload((rng.standard_normal((rows, n))).astype(np.float32))
        w.upload(np.ones(n, np.float32))
        w2.upload(np.ones(n, np.float32))
        run = lambda: ctx._check(ctx.lib.phx_norm_add(ctx.h, x.ptr, y.ptr, w.ptr, rows, n, 1e-6, 1.0, w2.ptr, qs.ptr,
                                                      dq.ptr))
        for _ in range(3):
            run()
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(iters):
            run()
        ctx.sync()
        u = (time.perf_counter() - t0) / iters * 1e6
        b = rows * n * (4 + 4 + 4 + 1) + rows * n // 16 + 2 * n * 4
        modes[f"norm_add_quant_{rows}_rows"] = {"us": round(u, 2), "gbs": round(b / u / 1e3, 1)}
        for buf in (x, y, w, w2, qs, dq):
            buf.free()
    for wtype, rows, cols in ((2, 2112, 2816), (2, 2816, 2112), (8, 2112, 2816)):  # the shared FFN's matvecs
        bb = 18 if wtype == 2 else 34
        wb = ctx.alloc(rows * cols // 32 * bb)
        blocks = rng.integers(0, 256, (rows * cols // 32, bb), dtype=np.uint8)
        blocks[:, :2] = (rng.standard_normal(rows * cols // 32) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
        wb.upload(blocks)
        xq, xd, y = ctx.alloc(cols), ctx.alloc(cols // 16), ctx.alloc(rows * 4)
        xq.upload(np.ones(cols, np.int8))
        xd.upload(np.full(cols // 32, 0x3C00, np.uint16))
        run = lambda: ctx._check(ctx.lib.phx_matvec(ctx.h, wtype, wb.ptr, rows, cols, 1, xq.ptr, xd.ptr, y.ptr))
        for _ in range(3):
            run()
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(iters):
            run()
        ctx.sync()
        u = (time.perf_counter() - t0) / iters * 1e6
        modes[f"matvec_{qname(wtype)}_{rows}x{cols}"] = {"us": round(u, 2), "gbs": round(wb.nbytes / u / 1e3, 1)}
        for buf in (wb, xq, xd, y):
            buf.free()
    for wtype, rows, cols in ((2, 2112, 2816), (2, 2816, 2112), (8, 2112, 2816)):  # prefill dense matmul, T = 2048
        T = 2048
        bb = 18 if wtype == 2 else 34
        blocks = rng.integers(0, 256, (rows * cols // 32, bb), dtype=np.uint8)
        blocks[:, :2] = (rng.standard_normal(rows * cols // 32) * 0.01).astype(np.float16).view(np.uint8).reshape(-1, 2)
        h = ctx.weight_upload(wtype, blocks.reshape(-1), rows, cols)
        xq, xd, y = ctx.alloc(T * cols), ctx.alloc(T * cols // 16), ctx.alloc(T * rows * 4)
        xq.upload(rng.integers(-127, 128, T * cols, dtype=np.int8))
        xd.upload(np.full(T * cols // 32, 0x2C00, np.uint16))
        run = lambda: ctx.matmul_device(h, T, xq.ptr, xd.ptr, y.ptr)
        for _ in range(3):
            run()
        ctx.sync()
        t0 = time.perf_counter()
        for _ in range(max(10, iters // 4)):
            run()
        ctx.sync()
        u = (time.perf_counter() - t0) / max(10, iters // 4) * 1e6
        tflops = 2.0 * T * rows * cols / (u * 1e-6) / 1e12
        modes[f"matmul_{qname(wtype)}_{rows}x{cols}_T{T}"] = {
            "us": round(u, 2), "tflops": round(tflops, 1), "frac_fp16_peak": round(tflops / FP16_PEAK_TFLOPS, 4)}
        for buf in (xq, xd, y):
            buf.free()
        ctx.weight_free(h)
    line = {"metric": "activation quantizer GB/s (algorithmic bytes) vs HBM peak", "value": round(gbs, 1),
            "unit": "GB/s", "n_gpus": 1, "steps": iters, "warmup": max(3, args.warmup // 100),
            "ms_per_step": round(us / 1e3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f32->int8", "data": "synthetic",
            "config": {"workload": "quant: phx_quant_q8_0 GELU_MUL, 16384 rows x 704 (C3's 2048 tokens x top-8 "
                                   "down inputs)", "parallelism": "none (1 GPU)"},
            "roofline": {"bound": "hbm", "kernel": "k_quant<GELU_MUL, Q8_0>", "achieved": round(gbs, 1),
                         "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": None,
                         "bytes_per_launch": nbytes, "avg_launch_us": round(us, 3),
                         "per_unit": "704 x (4 B g + 4 B u read, 1 B quant + 2/32 B fp16 scale written) per row"},
            "modes_2048_rows": modes}
    ctx.close()
    if not args.no_cpu:
        from oracle import oracle as orc
        g = (rng.standard_normal((256, 704)) * 2).astype(np.float32)
        u = rng.standard_normal((256, 704)).astype(np.float32)
        n, t0 = 0, time.perf_counter()
        while time.perf_counter() - t0 < min(args.cpu_seconds, 5.0):
            r = n % 256
            orc.quantize_q8_0((orc.gelu(g[r]) * u[r]).astype(np.float32))
            n += 1
        dt = time.perf_counter() - t0
        line["cpu_baseline"] = {"value": round(n * 704 * 9.0625 / dt / 1e9, 4), "unit": "GB/s", "cores": 1,
                                "kind": "port", "sample": f"{n} rows of 704 through the oracle's gelu and "
                                                         f"quantize_q8_0, one at a time, {dt:.1f} s"}
    return line


def calibration_kernels(ctx, mib=1024):
    """Kernels of known traffic for scaling the PMC byte counters (FETCH_SIZE, WRITE_SIZE): streaming
    reads of `mib` MiB (phx::k_stream_read) and streaming copies of `mib` MiB (phx::k_stream_copy:
    `mib` MiB read and `mib` MiB written), 3 launches each."""
    n = mib << 20
    src, dst = ctx.alloc(n), ctx.alloc(n)
    ctx.stream_read_ms(src, 2)
    ctx.stream_copy_ms(dst, src, n, 2)
    src.free()
    dst.free()
    return {"stream_read_bytes": n, "copy_read_bytes": n, "copy_write_bytes": n,
            "kernels": ["phx::k_stream_read", "phx::k_stream_copy"]}


def qname(t):
    return {0: "F32", 2: "Q4_0", 8: "Q8_0", 12: "Q4_K", 14: "Q6_K"}.get(t, str(t))


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=4000, help="layer steps timed (exactly this many)")
    ap.add_argument("--warmup", type=int, default=400)
    ap.add_argument("--config", default="c2_decode")
    ap.add_argument("--T", type=int, default=0)
    ap.add_argument("--layers", type=int, default=0,
                    help="layer slots in the replayed graph (default: the largest count <= 32, or <= the "
                         "config's stack depth, that divides --steps)")
    ap.add_argument("--prof-steps", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--calibrate", action="store_true", help="also run the PMC calibration kernels")
    ap.add_argument("--no-prefill", action="store_true", help="leave out the prefill object of the default run")
    ap.add_argument("--prefill-steps", type=int, default=40, help="timed C3 layer calls of the prefill object")
    ap.add_argument("--no-fast-math", action="store_true", help="leave out the prefill object's tolerance-mode figures")
    ap.add_argument("--no-kquant", action="store_true", help="leave out the K-quant object of the default run")
    ap.add_argument("--kquant-steps", type=int, default=40, help="timed C4 layer calls of the kquant object")
    ap.add_argument("--no-stack", action="store_true", help="leave out the 30-layer stack object of the default run")
    ap.add_argument("--stack-steps", type=int, default=20, help="timed replays of the 30-layer C5 step")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(f"bench.py: this build runs on one GPU only (the MoE path shards by experts across GPUs by design, "
              f"see DESIGN.md); --gpus {args.gpus} is not supported", file=sys.stderr)
        sys.exit(2)
    import __graft_entry__ as ge
    if not ge._built():
        ge.build()
    pkg = ge.load_package()
    line = run_quant(args, pkg) if args.config == "quant" else run_layer(args, pkg)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
