"""MoE-layer benchmark on one MI355X (BASELINE.json metric: MoE-layer tokens/s at
decode b=1 and prefill 512; % of HBM / MFMA roofline).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--copies C] [--no-cpu]

A step is one forward of the MoE layer over one batch of synthetic input that
is already resident in HBM:

* value (the headline line): configs[1], the Qwen3-30B-A3B-shaped Q4_K layer
  at prefill 512 tokens with Zipf-biased routing. K steps are captured in one
  HIP graph that cycles over C resident copies of the layer's weights (so the
  256 MB Infinity Cache cannot serve repeated weight reads) and timed between
  HIP events; value = 512 * K / elapsed.
* decode: configs[0] (same layer shape, decode batch 1) the same way over 32
  copies, reported in the "decode" object.
* roofline: the dominant kernel of the prefill step (the stage with the
  largest time), timed live by graph-captured replays with HIP events on the
  stream it runs on; achieved = its algorithmic FLOPs / duration, priced
  against the dense fp16 MFMA peak (the instructions it issues); traffic = its
  HBM bytes per launch from the committed rocprofv3 PMC summary in profiles/.
* cpu_baseline: the C++ CPU restatement of the layer (oracle/liboracle.so,
  fp32 accumulation, one thread per available core) timed on a bounded sample
  of the same workload. The reference (Rust + Metal) cannot run on Linux.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F32_PEAK_TFLOPS = 157.3
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16 MFMA, the datatype the prefill GEMMs issue
PROFILES = os.path.join(ROOT, "profiles")


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def prefill_stage_work(spec, ids, T):
    """Algorithmic FLOPs / bytes of each prefill stage (intermediates excluded from bytes)."""
    H, F, K, E = spec.hidden, spec.ffn, spec.top_k, spec.experts
    P = T * K
    touched = np.unique(ids).size
    bpe = spec.weight_bytes_per_expert()
    gu_bytes = touched * (spec.gate.rows * spec.gate.stride + spec.up.rows * spec.up.stride)
    dn_bytes = touched * spec.down.rows * spec.down.stride
    return {
        "router": {"flops": 2.0 * T * E * H, "bytes": 4.0 * (E * H + T * H + T * E)},
        "gate_up": {"flops": 2.0 * P * 2 * F * H, "bytes": float(gu_bytes)},
        "down": {"flops": 2.0 * P * F * H, "bytes": float(dn_bytes)},
        "layer": {"flops": 2.0 * P * 3 * F * H + 2.0 * T * E * H,
                  "bytes": float(touched * bpe + 4 * E * H + 2 * 4 * T * H), "touched": int(touched)},
    }


def time_graph(gpu, layers, dx, T, dout, steps, warmup):
    from ingot_amd.moe import Graph  # noqa: F401
    for l in layers:
        l.reserve(T)
        l.forward(dx, T, dout)
    gpu.synchronize()
    gpu.check_device_flags()
    gpu.graph_begin()
    for i in range(warmup):
        layers[i % len(layers)].forward(dx, T, dout)
    gw = gpu.graph_end()
    gpu.graph_begin()
    for i in range(steps):
        layers[i % len(layers)].forward(dx, T, dout)
    g = gpu.graph_end()
    if warmup:
        gw.launch()
    gpu.synchronize()
    ms = g.time(1)
    gw.destroy()
    g.destroy()
    return ms


def time_stages(layers, dx, T, dout, reps):
    """Mean us per launch of every stage that ran in the layers' last forward."""
    from ingot_amd.moe import (STAGE_COMBINE, STAGE_DISPATCH, STAGE_DOWN, STAGE_GATEUP, STAGE_ROUTE, STAGE_ROUTER,
                               time_stage)
    for l in layers:
        l.forward(dx, T, dout)
    out = {}
    for name, st in (("router", STAGE_ROUTER), ("route", STAGE_ROUTE), ("dispatch", STAGE_DISPATCH),
                     ("gate_up", STAGE_GATEUP), ("down", STAGE_DOWN), ("combine", STAGE_COMBINE)):
        kernel = layers[0].stage_kernel(st)
        if kernel:
            out[name] = {"us": 1e3 * time_stage(layers, st, reps), "kernel": kernel}
    layers[0].gpu.synchronize()
    return out


def measured_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, calibrated against the plain copy kernel), or None."""
    import glob
    import re
    for path in sorted(glob.glob(os.path.join(PROFILES, "*_pmc.md"))):
        text = open(path).read()
        if f"kernel: {kernel}" not in text:
            continue
        m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", text, re.M)
        if m:
            return int(m.group(1)), os.path.relpath(path, ROOT)
    return None, None


def profile_workload(args):
    """A short eager workload for rocprofv3 (--kernel-trace or --pmc): C1 prefill
    forwards over 8 weight copies, C0 decode forwards over 32 copies, then one
    256 MiB device copy by the plain copy kernel (the counter calibration)."""
    from ingot_amd import configs as CF
    from ingot_amd.moe import Gpu, MoeLayer
    gpu = Gpu(0)
    base = MoeLayer(gpu, CF.c1_layer())
    layers = [base] + [base.clone() for _ in range(args.copies - 1)]
    dx = gpu.to_device(CF.inputs(1, 512, 2048))
    dout = gpu.buffer(4 * 512 * 2048)
    for rep in range(2):
        for l in layers:
            l.forward(dx, 512, dout)
    gpu.synchronize()
    log("profile: prefill done")
    for l in layers:
        l.destroy()
    d0 = MoeLayer(gpu, CF.c0_layer())
    dl = [d0] + [d0.clone() for _ in range(args.decode_copies - 1)]
    dx0 = gpu.to_device(CF.inputs(0, 1, 2048))
    dout0 = gpu.buffer(4 * 2048)
    for rep in range(2):
        for l in dl:
            l.forward(dx0, 1, dout0)
    gpu.synchronize()
    log("profile: decode done")
    n = 256 << 20
    a, b = gpu.buffer(n), gpu.buffer(n)
    a.upload(np.zeros(n // 4, np.float32))
    b.copy_from(a, n)
    b.copy_from(a, n)
    gpu.synchronize()
    log("profile: calibration copy of 256 MiB done")


def layer_work(spec, ids, T):
    """Algorithmic bytes (touched weights, router, vectors, x and out) and FLOPs of one forward."""
    H, E, K, F = spec.hidden, spec.experts, spec.top_k, spec.ffn
    touched = int(np.unique(ids).size)
    nbytes = touched * spec.weight_bytes_per_expert() + 4 * E * H + 2 * 4 * T * H
    flops = 2.0 * T * K * 3 * F * H + 2.0 * T * E * H
    if spec.router_bias is not None:
        nbytes += 4 * E
    if spec.shared is not None:
        nbytes += sum(m.rows * m.stride for m in spec.shared)
        flops += 2.0 * T * 3 * spec.shared[0].rows * H
    if spec.shared_gate_vec is not None:
        nbytes += 4 * H
    if spec.norm_gain is not None:
        nbytes += 4 * H
    return nbytes, flops, touched


def time_steps(gpu, step, steps, warmup):
    """Mean ms of one step() captured `steps` times in a HIP graph (after a warm-up graph)."""
    step()
    gpu.synchronize()
    gpu.check_device_flags()
    gpu.graph_begin()
    for _ in range(warmup):
        step()
    gw = gpu.graph_end()
    gpu.graph_begin()
    for _ in range(steps):
        step()
    g = gpu.graph_end()
    gw.launch()
    gpu.synchronize()
    ms = g.time(1)
    gw.destroy()
    g.destroy()
    return ms / steps


def extra_configs(gpu, args):
    """configs[2], [3] and [4] (parity-test configurations) timed the same way, for the record."""
    from ingot_amd import configs as CF
    from ingot_amd.moe import MoeLayer
    out = {}

    def record(name, spec, ids, T, ms, copies, bound, stages=None):
        nbytes, flops, touched = layer_work(spec, ids, T)
        r = {"tokens": T, "us_per_step": ms * 1e3, "tokens_per_s": T / (ms * 1e-3), "experts_touched": touched,
             "weight_copies": copies, "bytes": nbytes, "hbm_frac": nbytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9),
             "flops": flops, "frac_vs_fp32_mfma_peak": flops / (ms * 1e-3) / (MFMA_F32_PEAK_TFLOPS * 1e12),
             "bound": bound}
        if stages:
            r["stages_us"] = {k: round(v["us"], 2) for k, v in stages.items()}
            r["stage_kernels"] = {k: v["kernel"] for k, v in stages.items()}
        out[name] = r
        log(f"{name}: {ms * 1e3:.1f} us/step, {r['tokens_per_s']:.0f} tok/s, HBM {100 * r['hbm_frac']:.1f} %, "
            f"fp32 MFMA {100 * r['frac_vs_fp32_mfma_peak']:.1f} %")
        if stages:
            log(f"  stages (us): " + ", ".join(f"{k} {v['us']:.1f} ({v['kernel']})" for k, v in stages.items()))

    def single(name, spec, T, copies, xin, bound, mode=None):
        base = MoeLayer(gpu, spec)
        layers = [base] + [base.clone() for _ in range(copies - 1)]
        if mode is not None:
            for l in layers:
                l.set_gemm_mode(mode)
        dx = gpu.to_device(xin)
        dout = gpu.buffer(4 * T * spec.hidden)
        dids = gpu.buffer(4 * T * spec.top_k)
        for l in layers:
            l.reserve(T)
        base.forward(dx, T, dout, dids)
        gpu.synchronize()
        ids = dids.download(np.uint32, T * spec.top_k)
        i = [0]

        def step():
            layers[i[0] % copies].forward(dx, T, dout)
            i[0] += 1
        ms = time_steps(gpu, step, args.extra_steps, 10)
        stages = time_stages(layers, dx, T, dout, 20)
        record(name, spec, ids, T, ms, copies, bound, stages)
        for l in layers:
            l.destroy()

    t0 = time.time()
    spec2 = CF.c2_layer()
    log(f"C2 layer synthesized in {time.time() - t0:.1f} s")
    for T in (1, 4):
        single(f"configs[2] b={T}", spec2, T, 32, CF.inputs(2, T, 2048), "hbm")
    single("configs[2] shape, prefill 512", spec2, 512, 4, CF.inputs(2, 512, 2048), "mfma")
    del spec2
    t0 = time.time()
    spec3 = CF.c3_layer()
    log(f"C3 layer synthesized in {time.time() - t0:.1f} s")
    single("configs[3] T=64", spec3, 64, 2, CF.inputs(3, 64, 4096, bf16=True), "hbm and mfma (ridge)")
    del spec3
    # The real checkpoints' format mixes at the graded shapes (for the record): Qwen3-30B-A3B
    # Q4_K_M (Q4_K gate/up, Q6_K down in about a third of its layers) and the Qwen3.8 IQ2_XS
    # mix (validation/rust-moe-layer-0.json:9-16).
    from ingot_amd.moe import IQ2_S, IQ3_S, IQ4_XS, Q2_0, Q4_K, Q6_K
    specm = CF.make_layer(0, 0, 2048, 128, 8, 768, Q4_K, Q6_K)
    single("Q4_K/Q6_K mix b=1", specm, 1, 32, CF.inputs(0, 1, 2048), "hbm")
    specm.router_bias = np.array([1.5 * np.log((e + 1.0) ** -1.1) for e in range(128)], np.float32)
    single("Q4_K/Q6_K mix prefill 512", specm, 512, 8, CF.inputs(0, 512, 2048), "mfma")
    del specm
    from ingot_amd.moe import Q5_K
    spec5 = CF.make_layer(0, 0, 2048, 128, 8, 768, Q5_K, Q5_K, bias="zipf")
    single("Q5_K prefill 512", spec5, 512, 8, CF.inputs(0, 512, 2048), "mfma")
    del spec5
    specq = CF.make_layer(2, 0, 2048, 512, 10, 512, IQ2_S, IQ3_S, shared_ffn=512, shared_gate_kind=IQ4_XS,
                          shared_down_kind=Q2_0, shared_gated=True)
    single("IQ2_S/IQ3_S + IQ4_XS/Q2_0 shared mix b=1", specq, 1, 32, CF.inputs(2, 1, 2048), "hbm")
    # Prefill of the same mix: IQ2_S gate/up on the f16 GEMM (IQ3_S down on the fp32 one), and
    # the whole layer forced onto the fp32 GEMM for comparison.
    from ingot_amd.moe import GEMM_FP32
    single("IQ2_S/IQ3_S mix prefill 512", specq, 512, 4, CF.inputs(2, 512, 2048), "mfma")
    single("IQ2_S/IQ3_S mix prefill 512, fp32 GEMM", specq, 512, 4, CF.inputs(2, 512, 2048), "mfma", GEMM_FP32)
    del specq
    # 48 independent layers, h <- h + MoE_l(RMSNorm_l(h)); one step = the whole stack.
    t0 = time.time()
    specs = [CF.c4_layer(l) for l in range(48)]
    layers = [MoeLayer(gpu, s) for s in specs]
    log(f"C4 stack synthesized and uploaded in {time.time() - t0:.1f} s")
    for T in (1, 8):
        da = gpu.to_device(CF.inputs(4, T, 2048))
        db = gpu.buffer(4 * T * 2048)
        idb = [gpu.buffer(4 * T * 8) for _ in layers]
        for l in layers:
            l.reserve(T)
        a, b = da, db
        for l, ib in zip(layers, idb):
            l.forward(a, T, b, ib)
            a, b = b, a
        gpu.synchronize()
        ids = [ib.download(np.uint32, T * 8) for ib in idb]

        def step():
            a, b = da, db
            for l in layers:
                l.forward(a, T, b)
                a, b = b, a
        ms = time_steps(gpu, step, max(2, args.extra_steps // 10), 2)
        nbytes = flops = 0
        touched = []
        for s, i in zip(specs, ids):
            nb, fl, tc = layer_work(s, i, T)
            nbytes += nb - 2 * 4 * T * 2048
            flops += fl
            touched.append(tc)
        nbytes += 2 * 4 * T * 2048
        r = {"tokens": T, "layers": 48, "us_per_step": ms * 1e3, "tokens_per_s": T / (ms * 1e-3),
             "experts_touched_mean": float(np.mean(touched)), "bytes": nbytes,
             "hbm_frac": nbytes / (ms * 1e-3) / (HBM_PEAK_GBS * 1e9), "flops": flops, "bound": "hbm"}
        out[f"configs[4] 48 layers b={T}"] = r
        log(f"C4 b={T}: {ms * 1e3:.1f} us per 48-layer step, {r['tokens_per_s']:.0f} tok/s, HBM {100 * r['hbm_frac']:.1f} %")
    for l in layers:
        l.destroy()
    return out


def cpu_baseline(spec, x, budget_s, label):
    from oracle import pyoracle as O
    cores = len(os.sched_getaffinity(0))
    st, _, _, _ = O.moe_forward(spec, x, O.F32, threads=cores)  # warm-up
    assert st == 0
    n, t0 = 0, time.perf_counter()
    while True:
        st, _, _, _ = O.moe_forward(spec, x, O.F32, threads=cores)
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 200:
            break
    T = x.shape[0]
    return {"value": T * n / el, "unit": "tokens/s", "cores": cores, "kind": "port",
            "sample": f"{label}: {n} forward(s) of {T} token(s), fp32 accumulation, {el:.1f} s"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--copies", type=int, default=8, help="resident weight copies for the prefill step")
    ap.add_argument("--decode-copies", type=int, default=32)
    ap.add_argument("--decode-steps", type=int, default=1000)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--extra", action="store_true",
                    help="also time configs[2], [3] and [4] and add them as 'extra_configs' (slower: synthesis)")
    ap.add_argument("--extra-steps", type=int, default=100)
    ap.add_argument("--profile", action="store_true",
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
    from ingot_amd.moe import Gpu, MoeLayer

    gpu = Gpu(0)
    log(f"device: {gpu.name()}")

    # ---------------- prefill 512 ----------------
    t0 = time.time()
    spec1 = CF.c1_layer()
    x1 = CF.inputs(1, 512, 2048)
    log(f"C1 layer synthesized in {time.time() - t0:.1f} s")
    base = MoeLayer(gpu, spec1)
    layers = [base] + [base.clone() for _ in range(args.copies - 1)]
    T = 512
    dx = gpu.to_device(x1)
    dout = gpu.buffer(4 * T * 2048)
    dids = gpu.buffer(4 * T * 8)
    base.forward(dx, T, dout, dids)
    gpu.synchronize()
    ids = dids.download(np.uint32, T * 8)
    ms = time_graph(gpu, layers, dx, T, dout, args.steps, args.warmup)
    ms_step = ms / args.steps
    log(f"prefill: {ms_step * 1e3:.1f} us/step over {args.steps} steps, {args.copies} copies")
    work = prefill_stage_work(spec1, ids, T)
    stages = time_stages(layers, dx, T, dout, 40)
    log("prefill stages (us): " + ", ".join(f"{k} {v['us']:.1f}" for k, v in stages.items()))
    dom = max(("gate_up", "down"), key=lambda k: stages[k]["us"])
    dflops = work[dom]["flops"]
    achieved = dflops / (stages[dom]["us"] * 1e-6) / 1e12
    traffic, traffic_src = measured_traffic(stages[dom]["kernel"])
    layer_tflops = work["layer"]["flops"] / (ms_step * 1e-3) / 1e12

    # ---------------- decode b=1 ----------------
    spec0 = CF.c0_layer()
    x0 = CF.inputs(0, 1, 2048)
    d0 = MoeLayer(gpu, spec0)
    dl = [d0] + [d0.clone() for _ in range(args.decode_copies - 1)]
    dx0 = gpu.to_device(x0)
    dout0 = gpu.buffer(4 * 2048)
    dms = time_graph(gpu, dl, dx0, 1, dout0, args.decode_steps, args.warmup)
    dms_step = dms / args.decode_steps
    d_bytes = 4 * 128 * 2048 + 8 * spec0.weight_bytes_per_expert() + 2 * 4 * 2048
    gu_bytes = 8 * (spec0.gate.rows * spec0.gate.stride + spec0.up.rows * spec0.up.stride) + 4 * 2048
    dn_bytes = 8 * spec0.down.rows * spec0.down.stride + 8 * 4 * 768 + 4 * 2048
    dstages = time_stages(dl, dx0, 1, dout0, 256)
    log(f"decode: {dms_step * 1e3:.2f} us/step; stages (us): " +
        ", ".join(f"{k} {v['us']:.2f}" for k, v in dstages.items()))
    decode = {
        "config": "configs[0]: Qwen3-30B-A3B-shaped Q4_K MoE layer, decode batch 1",
        "tokens_per_s": 1.0 / (dms_step * 1e-3),
        "us_per_step": dms_step * 1e3,
        "steps": args.decode_steps,
        "weight_copies": args.decode_copies,
        "layer_hbm": {"bytes": d_bytes, "achieved_GBs": d_bytes / (dms_step * 1e-3) / 1e9,
                      "frac": d_bytes / (dms_step * 1e-3) / 1e9 / HBM_PEAK_GBS},
        "kernels": {
            "gate_up": {"kernel": dstages["gate_up"]["kernel"], "us": dstages["gate_up"]["us"], "bytes": gu_bytes,
                        "achieved_GBs": gu_bytes / (dstages["gate_up"]["us"] * 1e-6) / 1e9},
            "down": {"kernel": dstages["down"]["kernel"], "us": dstages["down"]["us"], "bytes": dn_bytes,
                     "achieved_GBs": dn_bytes / (dstages["down"]["us"] * 1e-6) / 1e9},
            **{k: v for k, v in dstages.items() if k not in ("gate_up", "down")},
        },
    }

    extra = extra_configs(gpu, args) if args.extra else None

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(spec1, x1, args.cpu_seconds, "configs[1] prefill 512")
        cpu_d = cpu_baseline(spec0, x0, max(2.0, args.cpu_seconds / 4), "configs[0] decode b=1")
        decode["cpu_baseline"] = cpu_d
        log(f"cpu baseline: prefill {cpu['value']:.0f} tok/s, decode {cpu_d['value']:.1f} tok/s on {cpu['cores']} cores")

    line = {
        "metric": "MoE-layer tokens/s at prefill 512 (configs[1]); decode b=1 in 'decode'",
        "value": T / (ms_step * 1e-3),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp32",
        "data": "synthetic: weights N(0,0.02) quantized to Q4_K, x ~ N(0,1), seeded SplitMix64",
        "config": {"workload": "configs[1]: Qwen3-30B-A3B-shaped Q4_K MoE layer, prefill 512 tokens, Zipf router bias",
                   "hidden": 2048, "experts": 128, "top_k": 8, "ffn": 768, "tokens": T, "format": "Q4_K",
                   "weight_copies": args.copies, "experts_touched": work["layer"]["touched"]},
        "roofline": {"bound": "mfma", "kernel": stages[dom]["kernel"], "achieved": achieved,
                     "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": achieved / MFMA_F16_PEAK_TFLOPS,
                     "traffic": traffic, "traffic_source": traffic_src,
                     "kernel_us": stages[dom]["us"], "algorithmic_flops": dflops,
                     "issued_f16_frac": 2.0 * achieved / MFMA_F16_PEAK_TFLOPS,
                     "frac_vs_fp32_mfma_peak": achieved / MFMA_F32_PEAK_TFLOPS,
                     "note": "fp32-accurate products as two f16 MFMA products (A hi and lo) with fp32 "
                             "accumulation; peak = dense fp16 MFMA"},
        "layer_frac_vs_fp32_mfma_peak": layer_tflops / MFMA_F32_PEAK_TFLOPS,
        "stages_us": {k: round(v["us"], 2) for k, v in stages.items()},
        "decode": decode,
        "cpu_baseline": cpu,
    }
    if extra is not None:
        line["extra_configs"] = extra
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
