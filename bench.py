"""MoE-layer benchmark on one MI355X (BASELINE.json metric: MoE-layer tokens/s at
decode b=1 and prefill 512; % of HBM / MFMA roofline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--extra]

A step is one forward of the MoE layer (configs[4]: of the 48-layer stack) over
one batch of synthetic input already resident in HBM. Every configuration of
BASELINE.json is measured and reported under "configs", with the real
Qwen3-30B-A3B Q4_K_M format mix (Q4_K gate/up, Q6_K down) at the C0/C1 shapes,
the Qwen3.8 IQ2_XS checkpoint's mix (IQ2_S gate/up, IQ3_S down, IQ4_XS/Q2_0
shared expert) at the C2 shape, and the C1 layer at the reference's 4096-token
prefill block:

    configs[0]  decode b=1        (32 resident weight copies)
    configs[1]  prefill 512       (8 copies)  <- the headline `value`
    configs[2]  b=1 and b=4       (32 copies)
    configs[3]  64 tokens         (2 copies, 980 MB each)
    configs[4]  48 layers, b=1 and b=8
    Q4_K/Q6_K mix b=1 (32 copies) and prefill 512 (8 copies)
    IQ2_S/IQ3_S mix b=1 (32 copies) and prefill 512 (4 copies)
    configs[1] layer at prefill 4096 (2 copies)

Timing: W untimed warm-up steps in one HIP graph, then
exactly K timed steps as R graph launches of s = K / R steps each, each launch
between HIP events on the layer's stream. Step j of a launch runs on resident
copy j mod copies and R is the largest divisor of K up to 20 that leaves
s >= copies, so every timed launch reads every copy and the 256 MB Infinity
Cache cannot serve repeated weight reads. A step's time is the median over the
launches (the mean is reported too).

Each configuration carries a `roofline` object for its dominant kernel (the
gate/up or down stage with the larger time): that stage's launches are
graph-captured round-robin over the copies and timed with HIP events on the
stream it runs on, and achieved = its algorithmic bytes (decode: HBM-bound)
or FLOPs (prefill: MFMA-bound) per launch / its mean duration, priced against
MI355X's peak for what it issues (HBM 8 TB/s; dense fp16 MFMA 2.5 PFLOP/s for
the f16 GEMM, fp32 MFMA 157.3 TFLOP/s for the fp32 one). `traffic` is the
kernel's measured HBM bytes per launch from the committed rocprofv3 PMC summary
in profiles/ for the same kernel and workload (FETCH_SIZE and WRITE_SIZE
calibrated against a plain copy kernel), or null.

Decode configurations also carry a `floor`: the same bytes read by a plain
streaming kernel (ingot_device_read), timed the same way over the same number
of copies, once as one kernel per step and once as a chain of one dependent
kernel per stage reading that stage's bytes, plus an empty chain of as many
kernel nodes. The chain is the fastest a layer of this many dependent kernels
could run if every kernel only streamed its weights.

cpu_baseline (every configuration): the C++ CPU restatement of the layer
(oracle/liboracle.so, fp32 accumulation, one thread per available core up to
16) timed on a bounded sample of the same workload. The reference (Rust +
Metal) cannot run on Linux.
"""
from __future__ import annotations

import argparse
import glob
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F32_PEAK_TFLOPS = 157.3
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, the datatype the f16 grouped GEMM issues
PROFILES = os.path.join(ROOT, "profiles")
STAGE_ORDER = ("router", "route", "dispatch", "gate_up", "down", "combine")
from ingot_amd.profile_summary import WORKLOADS as PROFILE_WORKLOADS  # noqa: E402


def log(*a):
    print(*a, file=sys.stderr, flush=True)


# ------------------------------------------------------------------ timing
def plan_launches(steps, copies, max_launches=20):
    """(R, s): R launches of s = steps / R steps, R the largest divisor of steps
    up to max_launches with s >= min(copies, steps)."""
    need = min(copies, steps)
    R = max(d for d in range(1, min(steps, max_launches) + 1) if steps % d == 0 and steps // d >= need)
    return R, steps // R


def timed_launches(gpu, step, steps, warmup, copies):
    """step(c) enqueues one step on copy c. `warmup` untimed steps (one graph),
    then `steps` steps as R graph launches of s steps, each timed between HIP
    events; step j of a launch runs on copy j % copies. Returns ms per step
    (median and mean over the launches) and the launch plan."""
    step(0)
    gpu.synchronize()
    gpu.check_device_flags()
    R, s = plan_launches(steps, copies)
    gw = None
    if warmup:
        gpu.graph_begin()
        for j in range(warmup):
            step(j % copies)
        gw = gpu.graph_end()
    gpu.graph_begin()
    for j in range(s):
        step(j % copies)
    g = gpu.graph_end()
    if gw is not None:
        gw.launch()
    gpu.synchronize()
    per = np.array([g.time(1) / s for _ in range(R)])
    g.destroy()
    if gw is not None:
        gw.destroy()
    gpu.check_device_flags()
    return {"median_ms": float(np.median(per)), "mean_ms": float(per.mean()), "launches": R,
            "steps_per_launch": s, "steps": steps, "copies_per_launch": min(copies, s)}


def time_stages(layers, reps, repeat=3):
    """us per launch of every stage that ran in the layers' last forward: the
    median over `repeat` measurements of the mean of `reps` graph-captured
    replays round-robin over the layers (ingot_layers_time_stage, HIP events
    on the context stream)."""
    from ingot_amd.moe import (STAGE_COMBINE, STAGE_DISPATCH, STAGE_DOWN, STAGE_GATEUP, STAGE_ROUTE, STAGE_ROUTER,
                               time_stage)
    ids = {"router": STAGE_ROUTER, "route": STAGE_ROUTE, "dispatch": STAGE_DISPATCH, "gate_up": STAGE_GATEUP,
           "down": STAGE_DOWN, "combine": STAGE_COMBINE}
    out = {}
    for name in STAGE_ORDER:
        kernel = layers[0].stage_kernel(ids[name])
        if kernel:
            us = sorted(1e3 * time_stage(layers, ids[name], reps) for _ in range(repeat))
            out[name] = {"us": us[len(us) // 2], "kernel": kernel}
    layers[0].gpu.synchronize()
    return out


# -------------------------------------------------------------- algorithmic work
def work(spec, ids, T):
    """Algorithmic bytes (weights touched, router, vectors, inputs and outputs;
    intermediates excluded) and FLOPs of one forward and of its stages."""
    H, E, K, F = spec.hidden, spec.experts, spec.top_k, spec.ffn
    P = T * K
    touched = np.unique(ids)
    n = int(touched.size)
    gu = n * (spec.gate.rows * spec.gate.stride + spec.up.rows * spec.up.stride)
    dn = n * spec.down.rows * spec.down.stride
    SF, sgu, sdn = 0, 0, 0
    if spec.shared is not None:
        SF = spec.shared[0].rows
        sgu = sum(m.rows * m.stride for m in spec.shared[:2])
        sdn = spec.shared[2].rows * spec.shared[2].stride
    vec = 4 * H * ((spec.shared_gate_vec is not None) + (spec.norm_gain is not None)) + \
        4 * E * (spec.router_bias is not None)
    xb = 4 * T * H
    f_gu = 2.0 * (P * 2 * F + T * 2 * SF) * H
    f_dn = 2.0 * (P * F + T * SF) * H
    f_rt = 2.0 * T * E * H
    return {
        "touched": n,
        "router": {"bytes": 4 * E * H + vec + xb + 4 * T * E, "flops": f_rt},
        "route": {"bytes": 4 * T * E + 8 * P, "flops": 0.0},
        "gate_up": {"bytes": gu + sgu + xb, "flops": f_gu},
        "down": {"bytes": dn + sdn + 4 * (P * F + T * SF) + xb, "flops": f_dn},
        "layer": {"bytes": gu + dn + sgu + sdn + 4 * E * H + vec + 2 * xb, "flops": f_gu + f_dn + f_rt},
    }


def measured_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from a committed rocprofv3
    PMC summary in profiles/ (FETCH_SIZE + WRITE_SIZE, calibrated against the
    plain copy kernel; lines `traffic_bytes_per_launch[<kernel>] @ <workload>: N`
    written by ingot_amd.profile_summary), or (None, None)."""
    key = f"traffic_bytes_per_launch[{kernel}] @ {workload}:"
    for path in sorted(glob.glob(os.path.join(PROFILES, "*_pmc.md"))):
        for line in open(path):
            if line.startswith(key):
                return int(line[len(key):].strip()), os.path.relpath(path, ROOT)
    return None, None


def kernel_roofline(bound, stage, stages, w, workload):
    """Roofline object of one stage's kernel."""
    us = stages[stage]["us"]
    kernel = stages[stage]["kernel"]
    if bound == "hbm":
        achieved = w[stage]["bytes"] / (us * 1e-6) / 1e9
        peak, unit, algo = HBM_PEAK_GBS, "GB/s", {"algorithmic_bytes": w[stage]["bytes"]}
    else:
        achieved = w[stage]["flops"] / (us * 1e-6) / 1e12
        f16 = kernel.startswith("k_gemm_f16")
        peak = MFMA_F16_PEAK_TFLOPS if f16 else MFMA_F32_PEAK_TFLOPS
        unit, algo = "TFLOP/s", {"algorithmic_flops": w[stage]["flops"]}
    traffic, src = measured_traffic(kernel, workload)
    r = {"bound": bound, "kernel": kernel, "stage": stage, "achieved": achieved, "peak": peak, "unit": unit,
         "frac": achieved / peak, "traffic": traffic, "traffic_source": src,
         "traffic_over_algorithmic_bytes": traffic / w[stage]["bytes"] if traffic else None, "kernel_us": us, **algo}
    if bound == "mfma" and kernel.startswith("k_gemm_f16"):
        r["issued_f16_frac"] = 2.0 * achieved / MFMA_F16_PEAK_TFLOPS
        r["frac_vs_fp32_mfma_peak"] = achieved / MFMA_F32_PEAK_TFLOPS
        r["note"] = ("fp32-accurate products issued as two f16 MFMA products (A hi and lo) with fp32 "
                     "accumulation; peak = dense fp16 MFMA")
    if bound == "mfma":
        r["hbm_frac"] = w[stage]["bytes"] / (us * 1e-6) / 1e9 / HBM_PEAK_GBS
    return r


def record(name, desc, ids, T, t, copies, bound, stages, workload, w, layers_n=1):
    ms = t["median_ms"]
    r = {"config": desc, "tokens": T, "us_per_step": ms * 1e3, "us_per_step_mean": t["mean_ms"] * 1e3,
         "tokens_per_s": T / (ms * 1e-3), "timed_steps": t["steps"], "launches": t["launches"],
         "steps_per_launch": t["steps_per_launch"], "weight_copies": copies,
         "copies_per_launch": t["copies_per_launch"], "experts_touched": w["touched"],
         "bytes": w["layer"]["bytes"] * layers_n, "flops": w["layer"]["flops"] * layers_n, "bound": bound}
    r["hbm_frac"] = r["bytes"] / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9)
    r["frac_vs_fp32_mfma_peak"] = r["flops"] / (ms * 1e-3) / (MFMA_F32_PEAK_TFLOPS * 1e12)
    r["stages_us"] = {k: round(v["us"], 2) for k, v in stages.items()}
    r["stage_kernels"] = {k: v["kernel"] for k, v in stages.items()}
    dom = max(("gate_up", "down"), key=lambda k: stages[k]["us"])
    r["roofline"] = kernel_roofline("hbm" if bound == "hbm" else "mfma", dom, stages, w, workload)
    rf = r["roofline"]
    log(f"{name}: {ms * 1e3:.2f} us/step (mean {t['mean_ms'] * 1e3:.2f}; {t['launches']} launches of "
        f"{t['steps_per_launch']} steps over {t['copies_per_launch']} copies), {r['tokens_per_s']:.0f} tok/s, "
        f"HBM {100 * r['hbm_frac']:.1f} %; {rf['kernel']} {rf['achieved']:.1f} {rf['unit']} = "
        f"{100 * rf['frac']:.1f} % of peak")
    log("  stages (us): " + ", ".join(f"{k} {v['us']:.2f}" for k, v in stages.items()))
    return r


# -------------------------------------------------------------- decode floor
def decode_floor(gpu, nodes, copies, steps, warmup):
    """Streaming-read floor of one decode step. nodes: [(stage, bytes)] of the
    step's dependent kernels in launch order. Each copy gets its own span of
    the summed bytes; three graphs are timed like the layer itself (same
    steps, warm-up and copy rotation): `chain` one plain read kernel per stage
    over that stage's bytes, `one_kernel` one read of all of them, `empty` as
    many empty kernel nodes."""
    nb = [(b + 15) // 16 * 16 for _, b in nodes]
    total = sum(nb)
    offs = np.concatenate([[0], np.cumsum(nb)[:-1]]).astype(np.int64)
    buf = gpu.buffer(total * copies)
    sink = gpu.buffer(4 * (total // 16384 + 2))

    def chain(c):
        for b, o in zip(nb, offs):
            gpu.stream_read(buf, b, sink, c * total + int(o))

    def one(c):
        gpu.stream_read(buf, total, sink, c * total)

    def empty(c):
        for _ in nb:
            gpu.stream_read(buf, 0, sink)

    res = {"nodes": len(nb), "node_stages": sorted(set(s for s, _ in nodes), key=STAGE_ORDER.index),
           "bytes_per_step": total, "copies": copies}
    for key, fn in (("chain", chain), ("one_kernel", one), ("empty", empty)):
        t = timed_launches(gpu, fn, steps, warmup, copies)
        res[f"{key}_us"] = t["median_ms"] * 1e3
    res["chain_GBps"] = total / (res["chain_us"] * 1e-6) / 1e9
    res["one_kernel_GBps"] = total / (res["one_kernel_us"] * 1e-6) / 1e9
    buf.free()
    sink.free()
    return res


def attach_floor(r, floor):
    r["floor"] = floor
    r["step_over_chain_floor"] = r["us_per_step"] / floor["chain_us"]
    r["chain_floor_frac"] = floor["chain_us"] / r["us_per_step"]
    log(f"  floor: {floor['nodes']} nodes, {floor['bytes_per_step'] / 1e6:.2f} MB: chain {floor['chain_us']:.2f} us "
        f"({floor['chain_GBps']:.0f} GB/s), one kernel {floor['one_kernel_us']:.2f} us "
        f"({floor['one_kernel_GBps']:.0f} GB/s), empty chain {floor['empty_us']:.2f} us; "
        f"step = {r['step_over_chain_floor']:.2f} x the chain floor")


# -------------------------------------------------------------- CPU baseline
def cpu_baseline(specs, x, budget_s, label, total_layers=None):
    """The oracle's fp32 CPU layer (one thread per core up to 16) on x through
    `specs` in sequence (a sample of `total_layers` stacked layers, scaled to
    the whole stack), timed for about budget_s after one warm-up. Returns
    tokens/s from the median run."""
    from ingot_amd.configs import threads
    from oracle import pyoracle as O
    cores = threads()

    def run():
        h = x
        for s in specs:
            st, h, _, _ = O.moe_forward(s, h, O.F32, threads=cores)
            assert st == 0
        return h
    run()  # warm-up
    times = []
    t0 = time.perf_counter()
    while True:
        a = time.perf_counter()
        run()
        times.append(time.perf_counter() - a)
        el = time.perf_counter() - t0
        if (el >= budget_s and len(times) >= 3) or len(times) >= 200:
            break
    T = x.shape[0]
    med = float(np.median(times))
    scale = (total_layers or len(specs)) / len(specs)
    sample = f"{label}: {len(times)} run(s) of {T} token(s)"
    if total_layers:
        sample += f" through {len(specs)} of the {total_layers} layers (scaled to the stack)"
    sample += f", fp32 accumulation, {el:.1f} s"
    return {"value": T / (med * scale), "unit": "tokens/s", "cores": cores, "kind": "port", "sample": sample,
            "median_s_per_run": med}


# -------------------------------------------------------------- configurations
def run_layer_config(gpu, name, desc, spec, T, copies, x, steps, warmup, bound, workload, mode=None,
                     cpu_s=0.0, floor=False):
    from ingot_amd.moe import MoeLayer
    base = MoeLayer(gpu, spec)
    layers = [base] + [base.clone() for _ in range(copies - 1)]
    if mode is not None:
        for l in layers:
            l.set_gemm_mode(mode)
    dx = gpu.to_device(x)
    dout = gpu.buffer(4 * T * spec.hidden)
    dids = gpu.buffer(4 * T * spec.top_k)
    for l in layers:
        l.reserve(T)
    base.forward(dx, T, dout, dids)
    gpu.synchronize()
    gpu.check_device_flags()
    ids = dids.download(np.uint32, T * spec.top_k)

    def step(c):
        layers[c].forward(dx, T, dout)
    t = timed_launches(gpu, step, steps, warmup, copies)
    for l in layers:
        l.forward(dx, T, dout)
    stages = time_stages(layers, 40 if T > 8 else 256)
    w = work(spec, ids, T)
    r = record(name, desc, ids, T, t, copies, bound, stages, workload, w)
    for l in layers:
        l.destroy()
    del layers, base
    if floor:
        attach_floor(r, decode_floor(gpu, [(k, w[k]["bytes"]) for k in stages], copies, steps, warmup))
    if cpu_s > 0:
        r["cpu_baseline"] = cpu_baseline([spec], x, cpu_s, name)
        log(f"  cpu baseline: {r['cpu_baseline']['value']:.1f} tok/s on {r['cpu_baseline']['cores']} cores")
    return r


def run_c4(gpu, steps, warmup, cpu_s):
    """48 independent layers, h <- h + MoE_l(RMSNorm_l(h)); a step is the whole stack."""
    from ingot_amd import configs as CF
    from ingot_amd.moe import MoeLayer
    t0 = time.time()
    specs = [CF.c4_layer(l) for l in range(48)]
    layers = [MoeLayer(gpu, s) for s in specs]
    log(f"configs[4]: 48 layers synthesized and resident in {time.time() - t0:.1f} s")
    out = {}
    for T in (1, 8):
        x = CF.inputs(4, T, 2048)
        da = gpu.to_device(x)
        bufs = [gpu.buffer(4 * T * 2048), gpu.buffer(4 * T * 2048)]
        idb = [gpu.buffer(4 * T * 8) for _ in layers]
        for l in layers:
            l.reserve(T)
        src = da
        for j, (l, ib) in enumerate(zip(layers, idb)):
            l.forward(src, T, bufs[j & 1], ib)
            src = bufs[j & 1]
        gpu.synchronize()
        ids = [ib.download(np.uint32, T * 8) for ib in idb]

        def step(c):
            s_ = da
            for j, l in enumerate(layers):
                l.forward(s_, T, bufs[j & 1])
                s_ = bufs[j & 1]
        t = timed_launches(gpu, step, steps, warmup, 1)
        step(0)
        stages = time_stages(layers, 96)
        ws = [work(s, i, T) for s, i in zip(specs, ids)]
        w = {"touched": float(np.mean([x_["touched"] for x_ in ws]))}
        for k in ("router", "route", "gate_up", "down", "layer"):
            w[k] = {f: float(np.mean([x_[k][f] for x_ in ws])) for f in ("bytes", "flops")}
        key = f"configs[4] b={T}"
        r = record(key, f"configs[4]: 48 stacked Qwen3-30B-A3B-shaped Q4_K layers with RMSNorm and residual, "
                   f"decode batch {T} (per-layer stage times averaged over the 48 layers)", None, T, t, 1, "hbm",
                   stages, f"c4 b={T}", w, layers_n=48)
        r["layers"] = 48
        # the stack's floor: each layer's stages as dependent reads of its own bytes
        attach_floor(r, decode_floor(gpu, [(k, wl[k]["bytes"]) for wl in ws for k in stages], 1, steps, warmup))
        if cpu_s > 0:
            r["cpu_baseline"] = cpu_baseline(specs[:4], x, cpu_s, key, total_layers=48)
            log(f"  cpu baseline: {r['cpu_baseline']['value']:.2f} tok/s")
        out[key] = r
        del bufs, idb, da
    for l in layers:
        l.destroy()
    return out


def extra_configs(gpu, args):
    """More format mixes at the graded shapes (for the record): Q5_K_M-style,
    the Qwen3.8 mix on the fp32 GEMM, and configs[2]'s layer at prefill."""
    from ingot_amd import configs as CF
    from ingot_amd.moe import GEMM_FP32, Q5_K
    out = {}
    S = args.extra_steps
    spec5 = CF.make_layer(0, 0, 2048, 128, 8, 768, Q5_K, Q5_K, bias="zipf")
    out["Q5_K prefill 512"] = run_layer_config(gpu, "Q5_K prefill 512", "Q5_K gate/up and down, prefill 512",
                                               spec5, 512, 8, CF.inputs(0, 512, 2048), S, 10, "mfma", "q5k prefill512")
    del spec5
    specq = qwen38_mix(CF)
    out["IQ2_S/IQ3_S mix prefill 512, fp32 GEMM"] = run_layer_config(
        gpu, "IQ2_S/IQ3_S mix prefill 512, fp32 GEMM", "the same on the fp32 GEMM", specq, 512, 4,
        CF.inputs(2, 512, 2048), S, 10, "mfma", "mixiq prefill512 fp32", mode=GEMM_FP32)
    del specq
    spec2 = CF.c2_layer()
    out["configs[2] shape, prefill 512"] = run_layer_config(gpu, "configs[2] shape, prefill 512",
                                                            "configs[2]'s layer at prefill 512", spec2, 512, 4,
                                                            CF.inputs(2, 512, 2048), S, 10, "mfma", "c2 prefill512")
    return out


def qwen38_mix(CF):
    """The Qwen3.8 IQ2_XS checkpoint's expert formats (validation/rust-moe-layer-0.json:9-16) at configs[2]'s
    shape: IQ2_S gate/up, IQ3_S down, a gated shared expert in IQ4_XS (gate/up) and Q2_0 (down)."""
    from ingot_amd.moe import IQ2_S, IQ3_S, IQ4_XS, Q2_0
    return CF.make_layer(2, 0, 2048, 512, 10, 512, IQ2_S, IQ3_S, shared_ffn=512, shared_gate_kind=IQ4_XS,
                         shared_down_kind=Q2_0, shared_gated=True)


def profile_workload(args):
    """A short eager workload for rocprofv3 (--kernel-trace or --pmc), one
    configuration and batch per run (ingot_amd.profile_summary.WORKLOADS), then two 256 MiB
    device copies by the plain copy kernel (the counter calibration)."""
    from ingot_amd import configs as CF
    from ingot_amd.moe import Q4_K, Q6_K, Gpu, MoeLayer
    gpu = Gpu(0)

    def run(spec, T, copies, cfg, H, bf16=False):
        base = MoeLayer(gpu, spec)
        layers = [base] + [base.clone() for _ in range(copies - 1)]
        dx = gpu.to_device(CF.inputs(cfg, T, H, bf16=bf16))
        dout = gpu.buffer(4 * T * H)
        for rep in range(2):
            for l in layers:
                l.forward(dx, T, dout)
        gpu.synchronize()
        log(f"profile: configs[{cfg}] T={T} done")
        for l in layers:
            l.destroy()

    w = args.profile
    if w == "c1":
        run(CF.c1_layer(), 512, args.copies, 1, 2048)
    elif w == "c0":
        run(CF.c0_layer(), 1, 32, 0, 2048)
    elif w in ("c2b1", "c2b4"):
        run(CF.c2_layer(), 1 if w == "c2b1" else 4, 32, 2, 2048)
    elif w == "c3":
        run(CF.c3_layer(), 64, 2, 3, 4096, bf16=True)
    elif w in ("mix46b1", "mix46p"):
        spec = CF.make_layer(0, 0, 2048, 128, 8, 768, Q4_K, Q6_K, bias=None if w == "mix46b1" else "zipf")
        run(spec, 1 if w == "mix46b1" else 512, 32 if w == "mix46b1" else 8, 0, 2048)
    elif w in ("mixiqb1", "mixiqp"):
        run(qwen38_mix(CF), 1 if w == "mixiqb1" else 512, 32 if w == "mixiqb1" else 4, 2, 2048)
    elif w in ("c4b1", "c4b8"):
        T = 1 if w == "c4b1" else 8
        layers = [MoeLayer(gpu, CF.c4_layer(l)) for l in range(48)]
        da = gpu.to_device(CF.inputs(4, T, 2048))
        bufs = [gpu.buffer(4 * T * 2048), gpu.buffer(4 * T * 2048)]
        for rep in range(2):
            s_ = da
            for j, l in enumerate(layers):
                l.forward(s_, T, bufs[j & 1])
                s_ = bufs[j & 1]
        gpu.synchronize()
        log(f"profile: configs[4] T={T} done")
        for l in layers:
            l.destroy()
    n = 256 << 20
    a, b = gpu.buffer(n), gpu.buffer(n)
    a.upload(np.zeros(n // 4, np.float32))
    b.copy_from(a, n)
    b.copy_from(a, n)
    gpu.synchronize()
    log("profile: calibration copy of 256 MiB done")


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200, help="timed steps of the headline configs[1] prefill")
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=8, help="resident weight copies for the configs[1] prefill")
    ap.add_argument("--decode-steps", type=int, default=1000, help="timed steps of the decode configurations")
    ap.add_argument("--c3-steps", type=int, default=100)
    ap.add_argument("--c4-steps", type=int, default=20)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget of configs[1]")
    ap.add_argument("--only-headline", action="store_true", help="configs[0] and configs[1] only")
    ap.add_argument("--extra", action="store_true", help="also more format mixes ('extra_configs')")
    ap.add_argument("--extra-steps", type=int, default=100)
    ap.add_argument("--profile", choices=sorted(PROFILE_WORKLOADS),  # ingot_amd.profile_summary.WORKLOADS
                    help="run only a short eager workload for rocprofv3 and exit (no JSON line)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (the layer would shard by expert, "
              "with one all-reduce of the partial outputs)",
              file=sys.stderr)
        sys.exit(2)

    if args.profile:
        profile_workload(args)
        return

    from ingot_amd import configs as CF
    from ingot_amd.moe import Q4_K, Q6_K, Gpu

    gpu = Gpu(0)
    log(f"device: {gpu.name()}")
    cpu = 0.0 if args.no_cpu else args.cpu_seconds
    small = 0.0 if args.no_cpu else max(2.0, args.cpu_seconds / 3)
    configs = {}

    # the headline (prefill 512)
    spec1 = CF.c1_layer()
    x1 = CF.inputs(1, 512, 2048)
    c1 = run_layer_config(gpu, "configs[1] prefill 512",
                          "configs[1]: Qwen3-30B-A3B-shaped Q4_K MoE layer, prefill 512 tokens, Zipf router bias",
                          spec1, 512, args.copies, x1, args.steps, args.warmup, "mfma", "c1 prefill512", cpu_s=cpu)
    configs["configs[1] prefill 512"] = c1
    # decode b=1
    spec0 = CF.c0_layer()
    c0 = run_layer_config(gpu, "configs[0] decode b=1",
                          "configs[0]: Qwen3-30B-A3B-shaped Q4_K MoE layer, decode batch 1",
                          spec0, 1, 32, CF.inputs(0, 1, 2048), args.decode_steps, args.warmup, "hbm", "c0 b=1",
                          cpu_s=small, floor=True)
    configs["configs[0] decode b=1"] = c0
    del spec0
    if not args.only_headline:
        spec2 = CF.c2_layer()
        for T in (1, 4):
            configs[f"configs[2] b={T}"] = run_layer_config(
                gpu, f"configs[2] b={T}", f"configs[2]: 512 experts top-10 IQ2_XS + gated Q8_0 shared expert, "
                f"batch {T}", spec2, T, 32, CF.inputs(2, T, 2048), args.decode_steps, args.warmup, "hbm",
                f"c2 b={T}", cpu_s=small, floor=True)
        del spec2
        spec3 = CF.c3_layer()
        configs["configs[3] T=64"] = run_layer_config(
            gpu, "configs[3] T=64", "configs[3]: GLM-style sigmoid routing, H 4096, IQ3_XXS gate/up, IQ4_NL down, "
            "ungated shared expert, 64 tokens", spec3, 64, 2, CF.inputs(3, 64, 4096, bf16=True), args.c3_steps,
            args.warmup, "hbm", "c3 T=64", cpu_s=small)
        del spec3
        configs.update(run_c4(gpu, args.c4_steps, 2, small))
        # the real Qwen3-30B-A3B Q4_K_M format mix (Q6_K down in about a third of its layers)
        specm = CF.make_layer(0, 0, 2048, 128, 8, 768, Q4_K, Q6_K)
        configs["mix Q4_K/Q6_K b=1"] = run_layer_config(
            gpu, "mix Q4_K/Q6_K b=1", "Qwen3-30B-A3B Q4_K_M mix at configs[0]'s shape: Q4_K gate/up, Q6_K down, "
            "decode batch 1", specm, 1, 32, CF.inputs(0, 1, 2048), args.decode_steps, args.warmup, "hbm",
            "mix46 b=1", cpu_s=small, floor=True)
        specm.router_bias = spec1.router_bias
        configs["mix Q4_K/Q6_K prefill 512"] = run_layer_config(
            gpu, "mix Q4_K/Q6_K prefill 512", "the same mix at configs[1]'s shape: prefill 512, Zipf router bias",
            specm, 512, 8, CF.inputs(1, 512, 2048), args.steps, args.warmup, "mfma", "mix46 prefill512",
            cpu_s=small)
        del specm
        specq = qwen38_mix(CF)
        configs["mix IQ2_S/IQ3_S b=1"] = run_layer_config(
            gpu, "mix IQ2_S/IQ3_S b=1", "Qwen3.8 IQ2_XS checkpoint mix at configs[2]'s shape (IQ2_S gate/up, IQ3_S "
            "down, gated IQ4_XS/Q2_0 shared expert), decode batch 1", specq, 1, 32, CF.inputs(2, 1, 2048),
            args.decode_steps, args.warmup, "hbm", "mixiq b=1", cpu_s=small, floor=True)
        configs["mix IQ2_S/IQ3_S prefill 512"] = run_layer_config(
            gpu, "mix IQ2_S/IQ3_S prefill 512", "the same mix, prefill 512", specq, 512, 4, CF.inputs(2, 512, 2048),
            args.steps, args.warmup, "mfma", "mixiq prefill512", cpu_s=small)
        del specq
        # the reference prefills in 4096-token blocks (docs/ENGINE.md:29-31): the dispatch at 32,768 pairs
        configs["configs[1] layer prefill 4096"] = run_layer_config(
            gpu, "configs[1] layer prefill 4096", "configs[1]'s layer at the reference's 4096-token prefill block",
            spec1, 4096, 2, CF.inputs(1, 4096, 2048), 10, 2, "mfma", "c1 prefill4096")

    extra = extra_configs(gpu, args) if args.extra else None

    ms_step = c1["us_per_step"] * 1e-3
    rf = dict(c1["roofline"])
    line = {
        "metric": "MoE-layer tokens/s at prefill 512 (configs[1]); decode b=1 in 'decode'; every config in 'configs'",
        "value": c1["tokens_per_s"],
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: weights N(0,0.02) quantized to GGUF formats, x ~ N(0,1), seeded SplitMix64",
        "config": {"workload": "configs[1]: Qwen3-30B-A3B-shaped Q4_K MoE layer, prefill 512 tokens, Zipf router bias",
                   "hidden": 2048, "experts": 128, "top_k": 8, "ffn": 768, "tokens": 512, "format": "Q4_K",
                   "weight_copies": args.copies, "experts_touched": c1["experts_touched"],
                   "timing": f"median of {c1['launches']} event-timed graph launches of {c1['steps_per_launch']} "
                             f"steps, each over {c1['copies_per_launch']} weight copies"},
        "roofline": rf,
        "layer_frac_vs_fp32_mfma_peak": c1["frac_vs_fp32_mfma_peak"],
        "stages_us": c1["stages_us"],
        "decode": {"config": c0["config"], "tokens_per_s": c0["tokens_per_s"], "us_per_step": c0["us_per_step"],
                   "hbm_frac": c0["hbm_frac"], "roofline": c0["roofline"], "stages_us": c0["stages_us"],
                   "floor": c0["floor"], "step_over_chain_floor": c0["step_over_chain_floor"],
                   "cpu_baseline": c0.get("cpu_baseline")},
        "configs": configs,
        "cpu_baseline": c1.get("cpu_baseline"),
    }
    if extra is not None:
        line["extra_configs"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
