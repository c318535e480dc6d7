#!/usr/bin/env python3
"""bench.py - Qwen3-MoE expert-FFN layer throughput on one MI355X (libqmsg, gfx950).

A step is one call of the MoE layer (router -> dispatch -> int8 quantise -> gate/up + SwiGLU
-> down -> weighted combine) on one batch of T tokens. Weights (all 128 experts of each
layer, GGUF Q4_0 bytes) and inputs are resident in HBM before timing. Consecutive steps use
different resident layers and different tokens, so each step streams experts that are not in
the 256 MB last-level cache.

Prints one JSON line: tokens/s, ms per step, a roofline object for the dominant kernel
(algorithmic bytes / its HIP-event-timed average duration, against 8 TB/s), and the
reference's own CPU layer (its C sources built by oracle/Makefile, weights resident in host
RAM) timed on this host's cores on a bounded sample of the same workload.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))


def physical_cores() -> int:
    try:
        out = subprocess.run(["lscpu", "-p=CORE,SOCKET"], capture_output=True, text=True, check=True).stdout
        cores = {ln for ln in out.splitlines() if ln and not ln.startswith("#")}
        return max(1, len(cores))
    except Exception:
        return os.cpu_count() or 1


def cpu_model() -> str:
    try:
        for ln in subprocess.run(["lscpu"], capture_output=True, text=True, check=True).stdout.splitlines():
            if ln.startswith("Model name"):
                return ln.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


# OpenMP reads its environment when libgomp loads: pin the CPU baseline to the physical
# cores before anything that links it is imported.
os.environ.setdefault("OMP_NUM_THREADS", str(physical_cores()))
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")
sys.path.insert(0, ROOT)

import numpy as np  # noqa: E402

from large_model_amd import qmsg  # noqa: E402
from large_model_amd.workloads import HBM_PEAK_GBS, INT8_PEAK_TOPS, WORKLOADS, zipf_bias  # noqa: E402

METRIC = "MoE-layer tokens/s + achieved HBM GB/s (decode), int8 MFMA util (prefill), 1 GPU"
# every launch name the library's per-dispatch events report (QLAUNCH names in csrc)
KERNEL_NAMES = ("fill", "rmsnorm", "route", "select", "dispatch", "mxin", "layer", "gateup", "swiglu", "actq",
                "down", "combine", "add", "dquant", "dense")


# What int8_tops / int8_frac_of_peak measure: the layer's algorithmic int8 multiply-adds (the
# reference's int8 dots) per second against 5 POPS of dense int8 MFMA. The kernels do not issue
# int8 MFMAs: the prefill's lane sums come from f16 MFMAs on exact integer codes.
INT8_BASIS = ("algorithmic int8 multiply-adds of the reference's dots per second / 5 POPS dense int8; "
              "the kernels issue f16 MFMAs (block-diagonal, exact integer codes), not int8 ones")


def kernel_times(ctx):
    """Launch count and average duration per kernel name from the per-dispatch events."""
    kern = {}
    for name in KERNEL_NAMES:
        n, ms = ctx.profile_read(name)
        if n:
            kern[name] = {"launches": n, "avg_us": round(1e3 * ms / n, 3)}
    return kern


def log(msg: str):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def read_traffic(workload: str):
    """HBM bytes per dominant-kernel launch measured by rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE),
    as recorded in profiles/traffic_<kernel>_<workload>.txt; None when not measured."""
    path = os.path.join(ROOT, "profiles", f"traffic_gateup_{workload}.txt")
    if not os.path.exists(path):
        return None
    vals = {}
    with open(path) as f:
        for ln in f:
            if "=" in ln and not ln.lstrip().startswith("#"):
                k, v = ln.split("=", 1)
                vals[k.strip()] = v.strip()
    try:
        return float(vals["hbm_bytes_per_launch"])
    except (KeyError, ValueError):
        return None


def cpu_baseline(ctx, w, seconds: float):
    """The reference's moe() (oracle/_ref build of its own sources) on this host, else the
    oracle's restatement, over distinct seeded tokens of the same workload."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc  # checker only: times the CPU path beside the GPU

    R = orc.load_ref()
    kind = "reference" if R is not None else "port"
    host = orc.Layer(w.E, w.X, w.K, w.F, w.seed, layer=0, down_type=w.down_type, experts=[])
    router, gate, up, down = ctx.download(0)
    host.router[:] = router
    host.gate, host.up, host.down = gate, up, down
    host.have = set(range(w.X))
    xs = [orc.make_input(w.E, w.T, 10_000 + i, rmsnorm=w.rmsnorm) for i in range(64)]
    run = (lambda x: orc.ref_moe(R, host, x)) if R is not None else (lambda x: host.moe(x))
    for x in xs[:2]:
        run(x)
    n, t0 = 0, time.perf_counter()
    while True:
        run(xs[n % len(xs)])
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 5) or el >= 3 * seconds:
            break
    threads = R.qref_max_threads() if R is not None else int(os.environ.get("OMP_NUM_THREADS", "1"))
    isa = R.qref_isa().decode() if R is not None else "oracle restatement"
    return {
        "value": round(w.T * n / el, 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": kind,
        "sample": f"{n} calls of {'the reference moe() (its C sources, ' + isa + ' build)' if R else 'the oracle'}"
                  f" on one {w.name} layer, T={w.T}, {len(xs)} distinct seeded inputs cycled, all experts resident"
                  f" in host RAM; {el:.1f} s on {threads} OpenMP threads of {cpu_model()}",
        "ms_per_layer": round(1e3 * el / n, 4),
    }


def copy_calibration(nbytes: int, steps: int):
    """A plain device copy of nbytes, `steps` times: the known transfer against which
    rocprofv3's FETCH_SIZE / WRITE_SIZE readings are scaled."""
    nbytes -= nbytes % 16
    ctx = qmsg.Context(256, 16, 4, 128)
    src, dst = ctx.device_alloc(nbytes), ctx.device_alloc(nbytes)
    ctx.profile(True)
    for _ in range(steps):
        ctx.calibrate_copy(dst, src, nbytes)
    ctx.sync()
    n, ms = ctx.profile_read("copy")
    ctx.close()
    print(json.dumps({"copy_bytes": nbytes, "launches": n, "avg_us": round(1e3 * ms / n, 3),
                      "GBps_read_plus_write": round(2 * nbytes * n / (ms * 1e-3) / 1e9, 1)}), flush=True)


def cpu_baseline_stack(ctx, w, seconds: float, n_cpu_layers: int = 2):
    """The reference's moe() with its rmsnorm and residual add (src/model.c:1283-1285) chained
    over n_cpu_layers resident layers on the host, scaled to the full stack."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc  # checker only: times the CPU path beside the GPU

    R = orc.load_ref()
    if R is None:
        return None
    layers = []
    for l in range(n_cpu_layers):
        host = orc.Layer(w.E, w.X, w.K, w.F, w.seed + 1000 * l, layer=l, down_type=w.down_type, experts=[])
        router, gate, up, down = ctx.download(l)
        host.router[:] = router
        host.gate, host.up, host.down = gate, up, down
        host.have = set(range(w.X))
        layers.append(host)
    ones = np.ones(w.E, np.float32)
    xn = np.empty((w.T, w.E), np.float32)

    def chain(h):
        for host in layers:
            for t in range(w.T):
                R.qref_rmsnorm(xn[t].ctypes.data, h[t].ctypes.data, ones.ctypes.data, w.E, np.float32(1e-6))
            h += orc.ref_moe(R, host, xn)

    hs = [orc.make_input(w.E, w.T, 20_000 + i) for i in range(4)]
    chain(hs[0].copy())
    n, t0 = 0, time.perf_counter()
    while True:
        chain(hs[n % len(hs)].copy())
        n += 1
        el = time.perf_counter() - t0
        if (el >= seconds and n >= 2) or el >= 3 * seconds:
            break
    per_layer = el / (n * n_cpu_layers)
    threads = R.qref_max_threads()
    return {
        "value": round(w.T / (per_layer * w.layers), 3),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "reference",
        "sample": f"{n} passes of the reference rmsnorm + moe() + residual add over {n_cpu_layers} resident layers "
                  f"({R.qref_isa().decode()} build), T={w.T}; per-layer time x {w.layers} layers (the full "
                  f"{w.layers}-layer stack does not fit the host sample budget); {el:.1f} s on {threads} OpenMP "
                  f"threads of {cpu_model()}",
        "ms_per_layer": round(1e3 * per_layer, 4),
    }


def run_stack(args, w):
    """A step is the whole layer stack: h += moe(l, rmsnorm(h)) for every resident layer."""
    K_steps, W_steps, NL = args.steps, args.warmup, w.layers
    total = K_steps + W_steps
    log(f"workload {w.name}: E={w.E} X={w.X} K={w.K} F={w.F} T={w.T}, {NL}-layer stack")
    ctx = qmsg.Context(w.E, w.X, w.K, w.F, n_layer=NL, max_tokens=w.T)
    ctx.set_path({"auto": qmsg.PATH_AUTO, "exact": qmsg.PATH_EXACT, "mfma": qmsg.PATH_MFMA}[args.path])
    for l in range(NL):
        ctx.synth(l, w.seed + 1000 * l, down_type=w.down_type)
    ctx.sync()
    log("weights generated in HBM")
    row = w.T * w.E * 4
    d_h = ctx.device_alloc(total * row)
    for s in range(total):
        ctx.synth_input(w.seed + 7 + s, 0, w.T, d_h + s * row)
    ctx.sync()

    def step(s):
        ctx.moe_chain(0, NL, d_h + s * row, w.T)

    for s in range(W_steps):
        step(s)
    ctx.sync()
    t0 = time.perf_counter()
    for s in range(W_steps, total):
        step(s)
    ctx.sync()
    el = time.perf_counter() - t0
    ms_step = 1e3 * el / K_steps
    log(f"timed {K_steps} steps: {ms_step:.3f} ms/step ({1e3 * ms_step / NL:.1f} us/layer)")
    ctx.profile(True)
    for s in range(W_steps):                      # the warmup inputs again (unchanged by timing)
        step(s)
    ctx.sync()
    kern = kernel_times(ctx)
    ctx.profile(False)
    # distinct experts of the first layer on a fresh input (the routing is near uniform)
    x = ctx.d2h(d_h + W_steps * row, (w.T, w.E))
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc  # checker only: host rmsnorm of the sample input
    _, dbg = ctx.moe_debug(0, orc.rmsnorm(x))
    d_active = len(dbg["active"])
    step_bytes = NL * w.layer_bytes(d_active)
    g_us = kern.get("gateup", {}).get("avg_us")
    gate_up_bytes = d_active * 2 * w.gate_bytes
    achieved = gate_up_bytes / (g_us * 1e-6) / 1e9 if g_us else None
    result = {
        "metric": METRIC,
        "value": round(w.T * K_steps / el, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K_steps,
        "warmup": W_steps,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": f"{w.name}: {w.note}",
            "n_embd": w.E, "n_expert": w.X, "n_used": w.K, "n_ff_exp": w.F, "tokens_per_step": w.T,
            "layers": NL, "weights": "Q4_0 gate/up/" + ("Q6_K" if w.down_type == qmsg.QMSG_T_Q6_K else "Q4_0") +
            " down, F32 router", "path": args.path,
        },
        "roofline": {
            "kernel": "gateup (gate/up row dots + SwiGLU), per layer",
            "bound": "hbm",
            "achieved": round(achieved, 1) if achieved else None,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
            "traffic": None,
            "algorithmic_bytes_per_launch": int(gate_up_bytes),
        },
        "layer": {
            "algorithmic_bytes_per_step": int(step_bytes),
            "distinct_experts_per_layer": d_active,
            "achieved_GBps": round(step_bytes / (ms_step * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "us_per_layer": round(1e3 * ms_step / NL, 2),
        },
        "kernels": kern,
        "device": ctx.device_info(),
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        log("timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline_stack(ctx, w, args.cpu_seconds)
    ctx.close()
    print(json.dumps(result), flush=True)


def extra_prefill(steps: int = 10, warmup: int = 2, NL: int = 4):
    """The 512-token Zipf prefill of the 235B shape (the prefill half of the metric), bounded to
    a few seconds: ms per layer, distinct experts, int8 op/s against the MFMA peak, per-kernel
    times. Cycles NL resident layers."""
    w = WORKLOADS["q235b_prefill_t512"]
    ctx = qmsg.Context(w.E, w.X, w.K, w.F, n_layer=NL, max_tokens=w.T)
    bias = zipf_bias(w.X, w.K, w.T, w.E)
    for l in range(NL):
        ctx.synth(l, w.seed + 1000 * l, router_col0=bias)
    row = w.T * w.E * 4
    total = steps + warmup
    d_x = ctx.device_alloc(total * row)
    d_out = ctx.device_alloc(total * row)
    for s in range(total):
        ctx.synth_input(w.seed + 7 + s, 0, w.T, d_x + s * row, bias_col0=True)
    ctx.sync()
    for s in range(warmup):
        ctx.moe_device(s % NL, d_x + s * row, w.T, d_out + s * row)
    ctx.sync()
    t0 = time.perf_counter()
    for s in range(warmup, total):
        ctx.moe_device(s % NL, d_x + s * row, w.T, d_out + s * row)
    ctx.sync()
    el = time.perf_counter() - t0
    ms = 1e3 * el / steps
    ctx.profile(True)
    for s in range(warmup, total):
        ctx.moe_device(s % NL, d_x + s * row, w.T, d_out + s * row)
    ctx.sync()
    kern = kernel_times(ctx)
    ctx.profile(False)
    x = ctx.d2h(d_x + warmup * row, (w.T, w.E))
    _, dbg = ctx.moe_debug(warmup % NL, x)
    d_active = len(dbg["active"])
    ctx.close()
    ops = w.int8_ops()
    nbytes = w.layer_bytes(d_active)
    mfma_us = ops / (INT8_PEAK_TOPS * 1e12) * 1e6
    hbm_us = nbytes / (HBM_PEAK_GBS * 1e9) * 1e6
    return {
        "workload": f"{w.name}: {w.note}, {NL} resident layers cycled",
        "ms_per_layer": round(ms, 4), "tokens_per_s": round(w.T / (ms * 1e-3), 1),
        "distinct_experts": d_active, "int8_ops": ops,
        "int8_tops": round(ops / (ms * 1e-3) / 1e12, 3),
        "int8_frac_of_peak": round(ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 5),
        "int8_basis": INT8_BASIS,
        "algorithmic_bytes": nbytes, "achieved_GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
        "bound_us": {"mfma_at_peak": round(mfma_us, 1), "hbm_at_peak": round(hbm_us, 1)},
        "path": "auto (MFMA expert kernels at this batch)", "kernels": kern,
    }


def extra_stack_layer(steps: int = 4, warmup: int = 1, NL: int = 8):
    """Per-layer figures of the 94-layer stack shape (Q6_K down): h += moe(l, rmsnorm(h)) over NL
    resident layers (each layer's 1.57 GB exceeds the last-level cache, so NL distinct layers
    stream as the full stack does), at its 64-token batch and at batch 1 inside the chain."""
    w = WORKLOADS["q235b_stack_t64"]
    ctx = qmsg.Context(w.E, w.X, w.K, w.F, n_layer=NL, max_tokens=w.T)
    for l in range(NL):
        ctx.synth(l, w.seed + 1000 * l, down_type=w.down_type)
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as orc  # checker only: host rmsnorm of the sample input
    out = {"workload": f"{w.name}: {w.note}; {NL} resident layers chained, per-layer figures"}
    for T in (w.T, 1):
        row = T * w.E * 4
        total = steps + warmup
        d_h = ctx.device_alloc(total * row)
        for s in range(total):
            ctx.synth_input(w.seed + 7 + s, 0, T, d_h + s * row)
        ctx.sync()
        # the first timed step's input as generated: the chain overwrites it in place
        x0 = ctx.d2h(d_h + warmup * row, (T, w.E))
        for s in range(warmup):
            ctx.moe_chain(0, NL, d_h + s * row, T)
        ctx.sync()
        t0 = time.perf_counter()
        for s in range(warmup, total):
            ctx.moe_chain(0, NL, d_h + s * row, T)
        ctx.sync()
        el = time.perf_counter() - t0
        us_layer = 1e6 * el / (steps * NL)
        ctx.profile(True)
        ctx.moe_chain(0, NL, d_h, T)
        ctx.sync()
        kern = kernel_times(ctx)
        ctx.profile(False)
        # distinct experts of layer 0 on that untouched input (the byte count assumes every
        # layer touches as many; at T = 64 nearly all 128 are, at T = 1 exactly K)
        _, dbg = ctx.moe_debug(0, orc.rmsnorm(x0))
        d_active = len(dbg["active"])
        nbytes = 4 * w.X * w.E + d_active * w.expert_bytes + 8 * T * w.E
        out[f"t{T}"] = {
            "us_per_layer": round(us_layer, 2), "projected_94_layer_ms": round(us_layer * w.layers / 1e3, 3),
            "tokens_per_s_94_layers": round(T / (us_layer * w.layers * 1e-6), 2),
            "distinct_experts_per_layer": d_active, "distinct_experts_source": "layer 0 on the first timed input",
            "algorithmic_bytes_per_layer": nbytes,
            "achieved_GBps": round(nbytes / (us_layer * 1e-6) / 1e9, 1),
            "frac_of_hbm_peak": round(nbytes / (us_layer * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "kernels": kern,
        }
    ctx.close()
    return out


def extra_decode(name: str, steps: int = 200, warmup: int = 20, NL: int = 16):
    """A decode configuration beside the headline, bounded to a second or two: us per layer,
    tokens/s, distinct experts, the layer's algorithmic bytes against the HBM peak and per-kernel
    times. Cycles NL resident layers, different tokens per step, as the headline does."""
    w = WORKLOADS[name]
    ctx = qmsg.Context(w.E, w.X, w.K, w.F, n_layer=NL, max_tokens=w.T)
    for l in range(NL):
        ctx.synth(l, w.seed + 1000 * l, down_type=w.down_type)
    row = w.T * w.E * 4
    total = steps + warmup
    d_x = ctx.device_alloc(total * row)
    d_out = ctx.device_alloc(total * row)
    for s in range(total):
        ctx.synth_input(w.seed + 7 + s, 0, w.T, d_x + s * row, rmsnorm=w.rmsnorm)
    ctx.sync()
    for s in range(warmup):
        ctx.moe_device(s % NL, d_x + s * row, w.T, d_out + s * row)
    ctx.sync()
    t0 = time.perf_counter()
    for s in range(warmup, total):
        ctx.moe_device(s % NL, d_x + s * row, w.T, d_out + s * row)
    ctx.sync()
    el = time.perf_counter() - t0
    us = 1e6 * el / steps
    ctx.profile(True)
    for s in range(warmup, total):
        ctx.moe_device(s % NL, d_x + s * row, w.T, d_out + s * row)
    ctx.sync()
    kern = kernel_times(ctx)
    ctx.profile(False)
    ds = []
    for s in range(min(8, steps)):
        x = ctx.d2h(d_x + (warmup + s) * row, (w.T, w.E))
        _, dbg = ctx.moe_debug((warmup + s) % NL, x)
        ds.append(len(dbg["active"]))
    ctx.close()
    d_active = float(np.mean(ds))
    nbytes = w.layer_bytes(0) + d_active * w.expert_bytes
    return {
        "workload": f"{w.name}: {w.note}, {NL} resident layers cycled, {steps} timed steps",
        "n_embd": w.E, "n_expert": w.X, "n_used": w.K, "n_ff_exp": w.F, "tokens_per_step": w.T,
        "us_per_layer": round(us, 3), "tokens_per_s": round(w.T / (us * 1e-6), 1),
        "distinct_experts": d_active, "algorithmic_bytes": int(nbytes),
        "achieved_GBps": round(nbytes / (us * 1e-6) / 1e9, 1),
        "frac_of_hbm_peak": round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "kernels": kern,
    }


TRUNK_TYPES = {"f32": qmsg.QMSG_T_F32, "q4_0": qmsg.QMSG_T_Q4_0, "q4_1": qmsg.QMSG_T_Q4_1, "q6_k": qmsg.QMSG_T_Q6_K}


def run_trunk(args):
    """A step is the dense products of the 235B trunk for every resident layer (src/model.c:442,
    494): q/k/v in one qms_matmul_n call ([8192 | 512 | 512] x 4096, Q4_0), then attn_output
    (4096 x 8192), on T tokens, all in one type (Q4_0 unless --trunk-type says otherwise).
    Attention itself is not part of this library."""
    E, H, KV, NL, T = 4096, 8192, 512, args.trunk, args.tokens
    TT = TRUNK_TYPES[args.trunk_type]
    K_steps, W_steps = args.steps, args.warmup
    log(f"trunk q/k/v/o: {NL} resident layers, T={T}, {args.trunk_type}")
    ctx = qmsg.Context(256, 16, 4, 128, max_tokens=1)
    layers = []
    for l in range(NL):
        q = ctx.mat_synth(TT, H, E, 100 + 4 * l)
        k = ctx.mat_synth(TT, KV, E, 101 + 4 * l)
        v = ctx.mat_synth(TT, KV, E, 102 + 4 * l)
        o = ctx.mat_synth(TT, E, H, 103 + 4 * l)
        layers.append((q, k, v, o))
    d_x = ctx.device_alloc(T * E * 4)
    d_a = ctx.device_alloc(T * H * 4)
    ctx.synth_input(7, 0, T, d_x)
    d_y = [ctx.device_alloc(T * r * 4) for r in (H, KV, KV, E)]
    ctx.sync()

    def step():
        for q, k, v, o in layers:
            ctx.matmul_n_device([q, k, v], d_x, T, d_y[:3])
            ctx.matmul_n_device([o], d_a, T, d_y[3:])

    for _ in range(W_steps):
        step()
    ctx.sync()
    t0 = time.perf_counter()
    for _ in range(K_steps):
        step()
    ctx.sync()
    el = time.perf_counter() - t0
    ctx.profile(True)
    step()
    ctx.sync()
    kern = kernel_times(ctx)
    ctx.profile(False)
    rb = qmsg.row_bytes(TT, E)
    layer_bytes = (H + 2 * KV) * rb + E * qmsg.row_bytes(TT, H)
    us_layer = 1e6 * el / K_steps / NL
    # the layer's bytes over its dense launches' summed duration (q/k/v then o: two launches
    # for a quantised type, four for F32, whose matrices launch one by one)
    d_us_layer = kern["dense"]["avg_us"] * kern["dense"]["launches"] / NL
    achieved = layer_bytes / (d_us_layer * 1e-6) / 1e9
    result = {
        "metric": "trunk q/k/v/o dense products: us per layer + achieved HBM GB/s",
        "value": round(us_layer, 3), "unit": "us/layer", "higher_is_better": False, "n_gpus": 1,
        "steps": K_steps, "warmup": W_steps, "dtype": "f32" if TT == qmsg.QMSG_T_F32 else "int8",
        "data": "synthetic",
        "config": {"workload": f"Qwen3-235B-A22B trunk q/k/v/o shapes ({args.trunk_type}), {NL} resident layers",
                   "T": T},
        "layer_bytes": layer_bytes, "achieved_GBps_layer": round(layer_bytes / (us_layer * 1e-6) / 1e9, 1),
        "roofline": {"kernel": "dense (row dots over the layer's q/k/v and o launches)", "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None},
        "kernels": kern, "cpu_baseline": None,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline_trunk(T, args.cpu_seconds, TT)
    ctx.close()
    print(json.dumps(result), flush=True)


def cpu_baseline_trunk(T: int, seconds: float, TT: int):
    """The reference's own qms_matmul_n (src/quant.c:128-170) on one layer's q/k/v and o."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import ctypes

    import oracle as orc  # checker only: times the CPU path beside the GPU
    R = orc.load_ref()
    if R is None:
        return None

    class QmsMat(ctypes.Structure):   # src/quant.h:11-16
        _fields_ = [("type", ctypes.c_int), ("rows", ctypes.c_int64), ("cols", ctypes.c_int64),
                    ("row_bytes", ctypes.c_uint64), ("data", ctypes.c_void_p)]

    E, H, KV = 4096, 8192, 512
    bufs, mats = [], []
    for rows, cols, seed in ((H, E, 1), (KV, E, 2), (KV, E, 3), (E, H, 4)):
        w = orc.synth_mat(TT, rows, cols, seed)
        bufs.append(w)
        mats.append(QmsMat(TT, rows, cols, qmsg.row_bytes(TT, cols), w.ctypes.data))
    x = orc.make_input(E, T, 5)
    a = orc.make_input(H, T, 6)
    ys = [np.empty((T, m.rows), np.float32) for m in mats]
    P = ctypes.POINTER(QmsMat)
    qkv = (P * 3)(*[ctypes.pointer(m) for m in mats[:3]])
    yqkv = (ctypes.c_void_p * 3)(*[y.ctypes.data for y in ys[:3]])
    o = (P * 1)(ctypes.pointer(mats[3]))
    yo = (ctypes.c_void_p * 1)(ys[3].ctypes.data)
    R.qms_matmul_n.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    n, t0 = 0, time.perf_counter()
    while True:
        R.qms_matmul_n(qkv, 3, x.ctypes.data, T, yqkv)
        R.qms_matmul_n(o, 1, a.ctypes.data, T, yo)
        n += 1
        if time.perf_counter() - t0 > min(seconds, 10.0):
            break
    el = time.perf_counter() - t0
    return {"value": round(1e6 * el / n, 3), "unit": "us/layer", "cores": int(R.qref_max_threads()),
            "kind": "reference", "sample": f"{n} layers of q/k/v + o qms_matmul_n at T={T} on the host"}


def gguf_load(args):
    """File -> HBM rate of qmsg_gguf_upload for n layers of the 235B shape (Q4_0 gate/up; down
    Q4_0 and Q4_1 on alternate layers, as real files mix them), page cache warm: the file is
    written first, then loaded --steps times; prints one JSON line with the best rate."""
    import tempfile

    from large_model_amd import gguf_writer as gw
    E, X, K, F, NL = 4096, 128, 8, 1536, args.gguf_load
    tensors = []
    for l in range(NL):
        dt = qmsg.QMSG_T_Q4_1 if l % 2 else qmsg.QMSG_T_Q4_0
        b = f"blk.{l}."
        tensors += [
            (b + "ffn_norm.weight", qmsg.QMSG_T_F32, [E], np.ones(E, np.float32).tobytes()),
            (b + "ffn_gate_inp.weight", qmsg.QMSG_T_F32, [E, X], np.zeros((X, E), np.float32).tobytes()),
            (b + "ffn_gate_exps.weight", qmsg.QMSG_T_Q4_0, [E, F, X], qmsg.row_bytes(qmsg.QMSG_T_Q4_0, E) * F * X),
            (b + "ffn_up_exps.weight", qmsg.QMSG_T_Q4_0, [E, F, X], qmsg.row_bytes(qmsg.QMSG_T_Q4_0, E) * F * X),
            (b + "ffn_down_exps.weight", dt, [F, E, X], qmsg.row_bytes(dt, F) * E * X),
        ]
    nbytes = sum(t[3] if isinstance(t[3], int) else len(t[3]) for t in tensors)
    d = tempfile.mkdtemp(prefix="qmsg_gguf_")
    path = os.path.join(d, "moe.gguf")
    try:
        t0 = time.perf_counter()
        gw.write_gguf(path, gw.moe_header(E, X, K, F, NL), tensors)
        log(f"wrote {nbytes / 1e9:.2f} GB of MoE tensors ({NL} layers) in {time.perf_counter() - t0:.1f} s")
        runs = []
        with qmsg.Gguf(path) as g, qmsg.Context(E, X, K, F, n_layer=NL, max_tokens=1) as ctx:
            for r in range(args.steps):
                t0 = time.perf_counter()
                ctx.load_gguf(g, 0, NL)
                runs.append(time.perf_counter() - t0)
                log(f"load {r}: {runs[-1]:.3f} s, {nbytes / runs[-1] / 1e9:.2f} GB/s")
            dev = ctx.device_info()
    finally:
        if os.path.exists(path):
            os.remove(path)
        os.rmdir(d)
    best = min(runs)
    print(json.dumps({
        "metric": "GGUF MoE tensors file -> HBM (qmsg_gguf_upload), page cache warm",
        "value": round(nbytes / best / 1e9, 3), "unit": "GB/s", "higher_is_better": True, "n_gpus": 1,
        "steps": args.steps, "bytes_per_load": nbytes, "seconds": [round(t, 4) for t in runs],
        "config": {"workload": f"{NL} layers of the Qwen3-235B-A22B MoE shape (E=4096 X=128 F=1536)",
                   "staging": "2 x 64 MiB pinned buffers, 8 MiB pread pieces on parallel threads"},
        "host_cpu": cpu_model(), "device": dev,
    }), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=None, help="timed steps (default 500; 20 for a layer stack)")
    ap.add_argument("--warmup", type=int, default=None, help="untimed steps (default 50; 3 for a layer stack)")
    ap.add_argument("--workload", default="q235b_decode_t1", choices=sorted(WORKLOADS))
    ap.add_argument("--layers", type=int, default=16, help="distinct resident layers cycled by the steps")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extras", action="store_true",
                    help="skip the prefill and stack-layer figures the default decode run also reports")
    ap.add_argument("--path", choices=["auto", "exact", "mfma"], default="auto")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="instead of the layer, run the plain copy kernel on BYTES (reference transfer "
                         "for HBM byte counters) --steps times and exit")
    ap.add_argument("--trunk", type=int, default=0, metavar="LAYERS",
                    help="instead of the MoE layer, time the trunk's q/k/v/o dense products over LAYERS "
                         "resident layers and exit")
    ap.add_argument("--tokens", type=int, default=1, help="tokens per step of --trunk")
    ap.add_argument("--trunk-type", default="q4_0", choices=sorted(TRUNK_TYPES), help="matrix type of --trunk")
    ap.add_argument("--gguf-load", type=int, default=0, metavar="LAYERS",
                    help="instead of the layer, time loading LAYERS 235B-shape MoE layers from a GGUF file "
                         "into HBM (--steps loads, default 3) and exit")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (expert sharding is described in "
              "DESIGN.md, not built). Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.copy_calibration:
        copy_calibration(args.copy_calibration, args.steps)
        return
    if args.trunk:
        args.steps = args.steps or 200
        args.warmup = args.warmup if args.warmup is not None else 20
        run_trunk(args)
        return
    if args.gguf_load:
        args.steps = args.steps or 3
        gguf_load(args)
        return

    w = WORKLOADS[args.workload]
    stack = w.layers > 1
    if args.steps is None:
        args.steps = 20 if stack else 500
    if args.warmup is None:
        args.warmup = 3 if stack else 50
    if stack:
        run_stack(args, w)
        return
    K_steps, W_steps, NL = args.steps, args.warmup, max(1, args.layers)
    total = K_steps + W_steps
    log(f"workload {w.name}: E={w.E} X={w.X} K={w.K} F={w.F} T={w.T}, {NL} resident layers")
    ctx = qmsg.Context(w.E, w.X, w.K, w.F, n_layer=NL, max_tokens=w.T)
    ctx.set_path({"auto": qmsg.PATH_AUTO, "exact": qmsg.PATH_EXACT, "mfma": qmsg.PATH_MFMA}[args.path])
    bias = zipf_bias(w.X, w.K, w.T, w.E) if w.zipf else None
    for l in range(NL):
        ctx.synth(l, w.seed + 1000 * l, down_type=w.down_type, router_col0=bias)
    log("weights generated in HBM")
    row = w.T * w.E * 4
    d_x = ctx.device_alloc(total * row)
    d_out = ctx.device_alloc(total * row)
    for s in range(total):
        ctx.synth_input(w.seed + 7 + s, 0, w.T, d_x + s * row, rmsnorm=w.rmsnorm, bias_col0=w.zipf)
    ctx.sync()

    def step(s):
        ctx.moe_device(s % NL, d_x + s * row, w.T, d_out + s * row)

    for s in range(W_steps):
        step(s)
    ctx.sync()
    t0 = time.perf_counter()
    for s in range(W_steps, total):
        step(s)
    ctx.sync()
    el = time.perf_counter() - t0
    ms_step = 1e3 * el / K_steps
    log(f"timed {K_steps} steps: {ms_step * 1e3:.2f} us/step")

    # the same steps again, every dispatch stamping its own start/end into HIP events
    # (hipExtLaunchKernel on the library's stream)
    ctx.profile(True)
    t0 = time.perf_counter()
    for s in range(W_steps, total):
        step(s)
    ctx.sync()
    log(f"with per-dispatch events: {1e6 * (time.perf_counter() - t0) / K_steps:.2f} us/step")
    kern = kernel_times(ctx)
    ctx.profile(False)

    # distinct experts per call (8 at T=1); sampled through the debug entry for larger T
    if w.T == 1:
        d_active = w.K
    else:
        ds = []
        for s in range(min(8, K_steps)):
            x = ctx.d2h(d_x + (W_steps + s) * row, (w.T, w.E))
            _, dbg = ctx.moe_debug((W_steps + s) % NL, x)
            ds.append(len(dbg["active"]))
        d_active = float(np.mean(ds))
    gate_up_bytes = d_active * 2 * w.gate_bytes
    layer_bytes = w.layer_bytes(0) + d_active * w.expert_bytes
    g_us = kern.get("gateup", {}).get("avg_us")
    achieved = gate_up_bytes / (g_us * 1e-6) / 1e9 if g_us else None
    traffic = read_traffic(w.name)
    result = {
        "metric": METRIC,
        "value": round(w.T * K_steps / el, 3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K_steps,
        "warmup": W_steps,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic",
        "config": {
            "workload": f"{w.name}: {w.note}",
            "n_embd": w.E, "n_expert": w.X, "n_used": w.K, "n_ff_exp": w.F, "tokens_per_step": w.T,
            "weights": "Q4_0 gate/up/" + ("Q6_K" if w.down_type == qmsg.QMSG_T_Q6_K else "Q4_0") + " down, F32 router",
            "resident_layers_cycled": NL, "path": args.path,
        },
        "roofline": {
            "kernel": "gateup (routing of the token, gate/up Q4_0 row dots, SwiGLU)",
            "bound": "hbm",
            "achieved": round(achieved, 1) if achieved else None,
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4) if achieved else None,
            "traffic": traffic,
            "algorithmic_bytes_per_launch": int(gate_up_bytes),
        },
        "layer": {
            "algorithmic_bytes": int(layer_bytes),
            "distinct_experts": d_active,
            "achieved_GBps": round(layer_bytes / (ms_step * 1e-3) / 1e9, 1),
            "frac_of_hbm_peak": round(layer_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "int8_tops": round(w.int8_ops() / (ms_step * 1e-3) / 1e12, 3),
            "int8_frac_of_peak": round(w.int8_ops() / (ms_step * 1e-3) / 1e12 / INT8_PEAK_TOPS, 5),
            "int8_basis": INT8_BASIS,
        },
        "kernels": kern,
        "device": ctx.device_info(),
        "cpu_baseline": None,
    }
    if not args.no_cpu:
        log("timing the CPU baseline")
        result["cpu_baseline"] = cpu_baseline(ctx, w, args.cpu_seconds)
    ctx.close()
    if w.name == "q235b_decode_t1" and not args.no_extras:
        for key, name in (("tiny_t1", "tiny"), ("q30b_decode_t1", "q30b_decode_t1"),
                          ("q235b_decode_t4", "q235b_decode_t4"), ("q235b_decode_t16", "q235b_decode_t16")):
            log(f"decode extra: {name}")
            result[key] = extra_decode(name)
        log("prefill extra: 512-token Zipf prefill")
        result["prefill_t512"] = extra_prefill()
        log("stack extra: per-layer figure of the 94-layer stack shape")
        result["stack_t64_layer"] = extra_stack_layer()
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
