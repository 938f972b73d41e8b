#!/usr/bin/env python3
"""Benchmark of the fused Qwen3 SwiGLU MLP on one MI355X.

One step = one MLP layer ``out = x + down(silu(gate(x)) * up(x))`` at the Qwen3-27B shape
(hidden 5120, intermediate 17408) over M = 16 tokens (a speculative-verify block), bfp8 weights
(16-value groups sharing an 8-bit exponent), inputs resident in HBM.  Steps rotate over several
independently seeded layers so that no weight byte is served from L2 or the 256 MB last-level
cache; each layer's residual is the previous layer's output.  The timed region is bracketed by
device synchronisation and holds nothing but the forwards; a second pass of the same loop with
per-kernel HIP events on the forward's stream times the dominant (gate/up) kernel.

Prints one JSON line: metric, value (achieved HBM GB/s of the whole layer, algorithmic bytes
W + 4*M*H), ms_per_step, the gate/up kernel's roofline, the CPU baseline (the oracle's torch fp32
formula on this host's cores) and, unless --no-extras, the bf16-weight variant, the bf4 gate/up variant, the M = 1/32
sweep, one GPU's share of a two-way split layer, a 64-layer stack and the M = 2048 prefill chunk.
"""
import argparse
import json
import os
import platform
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
METRIC = "fused MLP µs/layer + achieved HBM GB/s (% of peak) at M=16, 27B shape, 1 GPU"
HBM_PEAK_GBS = 8000.0
BF16_MFMA_PEAK_TFLOPS = 2500.0


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def parse():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--workload", default="qwen3-27b-mlp-m16-bfp8")
    ap.add_argument("--rotate", type=int, default=8, help="distinct layers cycled through by the timed loop")
    ap.add_argument("--no-extras", action="store_true", help="skip the bf16 variant, sweep, stack and prefill")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="first run plain MIB-MiB device copies (scale for HBM byte counters)")
    return ap.parse_args()


def make_layers(pkg, workloads, wl, n, device, first_layer=0):
    layers = []
    for i in range(n):
        sd = workloads.state_dict(wl.hidden, wl.intermediate, layer=first_layer + i, device=device)
        layers.append(pkg.load_mlp_weights(device, sd, weight_format=wl.fmt))
        del sd
    return layers


def time_layers(pkg, layers, x, steps, warmup, profile=False, chain=True):
    """Runs `steps` forwards cycling through `layers`; returns (ms_per_step, kernel_ms dict).

    chain: each layer's residual is the previous layer's output (a residual stream, as in the
    decoder); x, the normalised MLP input, stays the same tensor.  profile: each projection kernel
    is launched with a start / stop HIP event pair (hipExtLaunchKernel: the dispatch's own
    timestamps on the forward's stream); the headline pass runs without them."""
    import ctypes

    import torch

    lib = pkg.lib()
    M, H = x.shape
    I = layers[0].intermediate
    ws = pkg.new_workspace(M, H, I, layers[0].fmt, x.device)
    outs = [x.clone(), x.clone(), x.clone()]
    for i in range(warmup):
        pkg.mlp_forward(x, layers[i % len(layers)], residual=outs[i % 3], out=outs[(i + 1) % 3], workspace=ws)
    events = []
    if profile:
        for _ in range(steps):
            evs = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
            for e in evs:
                e.record()  # materialise the handle
            events.append(evs)
    for o in outs:
        o.copy_(x)
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for i in range(steps):
        if profile:
            arr = (ctypes.c_void_p * 4)(*[e._as_parameter_.value for e in events[i]])
            lib.qmlp_set_profile_events(arr, 4)
        res = outs[i % 2] if chain else outs[2]
        pkg.mlp_forward(x, layers[i % len(layers)], residual=res, out=outs[(i + 1) % 2], workspace=ws)
    if profile:
        lib.qmlp_set_profile_events(None, 0)
    end.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    kern = {}
    if profile:
        for k, name in enumerate(("gate_up", "down")):
            kern[name] = statistics.fmean(ev[2 * k].elapsed_time(ev[2 * k + 1]) for ev in events)
    return ms, kern


def copy_calibration(mib, device):
    """Plain device-to-device copies of `mib` MiB (the reference point that scales the HBM byte
    counters of a profiling run: bytes read and written are both exactly mib MiB per copy)."""
    import torch

    n = mib << 20
    a = torch.empty(n, dtype=torch.uint8, device=device).fill_(1)
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    del a, b


# The sources that decide what the M <= 32 weight-streaming kernels read and write (their code,
# the packed layout and dequantisation helpers): a traffic figure measured on other sources
# describes other kernels.
TRAFFIC_SOURCES = ("qmlp_gemv.hip", "qmlp_common.h")


def kernel_source_hash():
    """sha256 (first 16 hex digits) over the gate/up kernel's sources, in TRAFFIC_SOURCES order."""
    import hashlib

    h = hashlib.sha256()
    csrc = os.path.join(ROOT, "tenstorrent.blackhole-qwen3.8-27b_amd", "csrc")
    for name in TRAFFIC_SOURCES:
        with open(os.path.join(csrc, name), "rb") as f:
            h.update(name.encode() + b"\0" + f.read())
    return h.hexdigest()[:16]


TRAFFIC_FILE = os.path.join("profiles", "gemv_m16_bfp8_traffic.md")


def read_traffic(workload):
    """HBM bytes per launch of the gate/up and down kernels from the committed counter summary.

    Returns ({"gate_up": bytes, "down": bytes} or None, note).  The summary is used only when it
    names this workload and was measured on the current kernel sources (its
    ``kernel_source_sha256`` line); otherwise the bench line reports no traffic rather than a stale
    figure."""
    path = os.path.join(ROOT, TRAFFIC_FILE)
    if not os.path.exists(path):
        return None, "no counter summary"
    vals = {}
    with open(path) as f:
        for line in f:
            if line.startswith("- ") and ":" in line:
                k, v = line[2:].split(":", 1)
                vals[k.strip()] = v.strip().strip("`")
    if vals.get("workload") != workload:
        return None, f"counter summary is for {vals.get('workload')}"
    if vals.get("kernel_source_sha256") != kernel_source_hash():
        return None, "counter summary was measured on other kernel sources"
    try:
        return {"gate_up": int(vals["hbm_bytes_per_launch_gate_up"]),
                "down": int(vals["hbm_bytes_per_launch_down"])}, TRAFFIC_FILE
    except (KeyError, ValueError):
        return None, "counter summary has no byte count"


def cpu_baseline(pkg, workloads, wl, device, seconds):
    """The oracle's restatement of the reference CPU path (torch fp32 formula,
    scripts/ci/mlp-sweep.py:121-126) on identically dequantised weights, this host's cores."""
    import numpy as np
    import torch

    if ROOT not in sys.path:
        sys.path.insert(0, ROOT)
    from oracle import bfp8 as obfp8
    from oracle import mlp as omlp

    # every core this process may run on (os.cpu_count() unless an affinity mask narrows it)
    threads = max(1, len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1))
    torch.set_num_threads(threads)
    sd = workloads.state_dict(wl.hidden, wl.intermediate, layer=0, device=device)
    w = {}
    for name in ("gate_proj", "up_proj", "down_proj"):
        t = sd[f"{name}.weight"]
        if wl.fmt == "bfp8":
            q, e8 = pkg.quantize_bfp8(t)
            w[name] = torch.from_numpy(obfp8.dequantize(q.cpu().numpy(), e8.cpu().numpy()))
        else:
            w[name] = t.float().cpu()
    del sd
    x = workloads.activations(wl.tokens, wl.hidden, gain=wl.gain, device=device).float().cpu()
    omlp.swiglu_torch(x, w["gate_proj"], w["up_proj"], w["down_proj"], residual=x)  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while len(times) < 5 or time.perf_counter() < t_end:
        t0 = time.perf_counter()
        omlp.swiglu_torch(x, w["gate_proj"], w["up_proj"], w["down_proj"], residual=x)
        times.append(time.perf_counter() - t0)
        if len(times) >= 2000:
            break
    med = statistics.median(times)
    cpu_model = platform.processor() or ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    cpu_model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {
        "value": round(wl.algorithmic_bytes() / med / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{len(times)} single-layer forwards of the same workload (median), torch fp32 on "
                  f"dequantised weights, {threads} threads (every core in this process's affinity mask), "
                  f"os.cpu_count()={os.cpu_count()}, {cpu_model}",
        "us_per_layer": round(med * 1e6, 1),
    }


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: the library runs the unsharded MLP on a single MI355X; "
              f"--gpus {args.gpus} (WORLD_SIZE={world}) is not supported.", file=sys.stderr)
        sys.exit(2)
    import torch

    sys.path.insert(0, ROOT)
    import __graft_entry__

    pkg = __graft_entry__.load_package()
    from qwen_mlp_amd import _lib, workloads

    library_hash = _lib.library_source_hash()  # lib() has refused a binary built from other sources
    _log(f"library {pkg.lib().qmlp_version().decode()}")

    dev = torch.device("cuda:0")
    wl = workloads.WORKLOADS[args.workload]
    _log(f"workload {wl.name}: generating {args.rotate} layers")
    layers = make_layers(pkg, workloads, wl, args.rotate, dev)
    x = workloads.activations(wl.tokens, wl.hidden, gain=wl.gain, device=dev)
    if args.calibrate_copy:
        _log(f"copy calibration: {args.calibrate_copy} MiB")
        copy_calibration(args.calibrate_copy, dev)
    _log(f"timing {args.steps} steps after {args.warmup} warm-up")
    ms, _ = time_layers(pkg, layers, x, args.steps, args.warmup)
    _log("per-kernel breakdown (HIP events on the forward's stream)")
    _, kern = time_layers(pkg, layers, x, args.steps, args.warmup, profile=True)
    layer_bytes = wl.algorithmic_bytes()
    value = layer_bytes / (ms / 1e3) / 1e9
    per = {"bfp8": 17 / 16, "bf4": 9 / 16, "bf16": 2}[wl.fmt]  # gate/up bytes per weight value
    gu_bytes = int(2 * wl.hidden * wl.intermediate * per + 2 * wl.tokens * wl.hidden)
    gu_ms = kern["gate_up"]
    gu_gbs = gu_bytes / (gu_ms / 1e3) / 1e9
    traffic, traffic_src = read_traffic(wl.name)
    dn_bytes = wl.algorithmic_bytes() - gu_bytes  # down weights + the out write (W + 4 M H in all)
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "us_per_layer": round(ms * 1e3, 2),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": {"bfp8": "f16-mfma/f32-acc (bfp8 weights)", "bf4": "f16-mfma/f32-acc (bf4 gate/up, bfp8 down)",
                  "bf16": "bf16-mfma/f32-acc"}[wl.fmt],
        "data": "synthetic: x ~ N(0,1)*U(0.5,1.5) gain, random-init weights N(0,0.02), seeds 1000/2000+",
        "config": {"workload": wl.name, "hidden": wl.hidden, "intermediate": wl.intermediate,
                   "tokens": wl.tokens, "weight_format": wl.fmt, "layers_rotated": args.rotate,
                   "algorithmic_bytes_per_layer": layer_bytes},
        "kernel_ms": {k: round(v, 5) for k, v in kern.items()},
        "roofline": {"kernel": "gate/up projection (gemv_kernel, 2 matrices)", "bound": "hbm",
                     "achieved": round(gu_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gu_gbs / HBM_PEAK_GBS, 4),
                     "traffic": traffic["gate_up"] if traffic else None, "traffic_source": traffic_src,
                     "traffic_over_algorithmic": round(traffic["gate_up"] / gu_bytes, 4) if traffic else None,
                     "kernel_source_sha256": kernel_source_hash(), "algorithmic_bytes_per_launch": gu_bytes,
                     "down": {"achieved": round(dn_bytes / (kern["down"] / 1e3) / 1e9, 2),
                              "frac": round(dn_bytes / (kern["down"] / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
                              "algorithmic_bytes_per_launch": dn_bytes,
                              "traffic": traffic["down"] if traffic else None,
                              "traffic_over_algorithmic": round(traffic["down"] / dn_bytes, 4) if traffic else None}},
        "library_source_sha16": library_hash,
    }
    if wl.tokens > 32:  # many-token chunks run the matrix-core kernels: bound by the MFMA peak
        gu_flops = 4 * wl.tokens * wl.hidden * wl.intermediate
        gu_tf = gu_flops / (gu_ms / 1e3) / 1e12
        kname = "tiled_kernel" if wl.fmt == "bf16" else "tiled32_kernel"
        result["roofline"] = {"kernel": f"gate/up projection ({kname}, 2 matrices)", "bound": "mfma",
                              "achieved": round(gu_tf, 1), "peak": BF16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
                              "frac": round(gu_tf / BF16_MFMA_PEAK_TFLOPS, 4), "traffic": None,
                              "algorithmic_flops_per_launch": gu_flops}
    del layers
    torch.cuda.empty_cache()
    if not args.no_extras:
        extras = {}
        # bf16-weight variant of the same layer (the 2x comparison)
        if wl.fmt == "bfp8":
            wb = workloads.Workload(wl.name.replace("bfp8", "bf16"), wl.hidden, wl.intermediate, wl.tokens, "bf16",
                                    wl.gain)
            _log("bf16-weight variant")
            lb = make_layers(pkg, workloads, wb, max(4, args.rotate // 2), dev)
            msb, _ = time_layers(pkg, lb, x, max(50, args.steps // 2), 10)
            del lb
            torch.cuda.empty_cache()
            extras["bf16_variant"] = {"us_per_layer": round(msb * 1e3, 2),
                                      "gbs": round(wb.algorithmic_bytes() / (msb / 1e3) / 1e9, 2),
                                      "bfp8_speedup": round(msb / ms, 3)}
            # bf4 gate/up + bfp8 down (the reference's weight formats) at the same width
            w4 = workloads.Workload(wl.name.replace("bfp8", "bf4"), wl.hidden, wl.intermediate, wl.tokens, "bf4",
                                    wl.gain)
            _log("bf4 gate/up variant")
            l4 = make_layers(pkg, workloads, w4, args.rotate, dev)
            ms4, _ = time_layers(pkg, l4, x, max(50, args.steps // 2), 10)
            _, k4 = time_layers(pkg, l4, x, max(50, args.steps // 2), 10, profile=True)
            del l4
            torch.cuda.empty_cache()
            gu4 = int(2 * w4.hidden * w4.intermediate * 9 / 16 + 2 * w4.tokens * w4.hidden)
            extras["bf4_variant"] = {"us_per_layer": round(ms4 * 1e3, 2),
                                     "gbs": round(w4.algorithmic_bytes() / (ms4 / 1e3) / 1e9, 2),
                                     "algorithmic_bytes_per_layer": w4.algorithmic_bytes(),
                                     "kernel_ms": {k: round(v, 5) for k, v in k4.items()},
                                     "gate_up_gbs": round(gu4 / (k4["gate_up"] / 1e3) / 1e9, 2),
                                     "speedup_vs_bfp8": round(ms / ms4, 3)}
            # width sweep
            sweep = {}
            lq = make_layers(pkg, workloads, wl, args.rotate, dev)
            for M in (1, 32, 64, 256):  # 64 / 256: the many-token kernels with every tile split
                xm = workloads.activations(M, wl.hidden, gain=wl.gain, device=dev)
                msm, _ = time_layers(pkg, lq, xm, max(50, args.steps // 2), 10)
                b = wl.weight_bytes() + 4 * M * wl.hidden
                sweep[f"M={M}"] = {"us_per_layer": round(msm * 1e3, 2), "gbs": round(b / (msm / 1e3) / 1e9, 2),
                                   "pct_hbm_peak": round(100 * b / (msm / 1e3) / 1e9 / HBM_PEAK_GBS, 2)}
            extras["width_sweep"] = sweep
            del lq
            torch.cuda.empty_cache()
            # one GPU's share of a two-way (TP2) split of the layer: I = 8704 (the all-reduce of the
            # [M, H] partials that completes the layer is not part of a one-GPU run)
            ws2 = workloads.WORKLOADS["qwen3-27b-tp2-share-m16-bfp8"]
            _log("TP2 share")
            l2 = make_layers(pkg, workloads, ws2, args.rotate, dev)
            ms2, _ = time_layers(pkg, l2, x, max(50, args.steps // 2), 10)
            del l2
            torch.cuda.empty_cache()
            extras["tp2_share_m16"] = {"intermediate": ws2.intermediate, "us_per_layer": round(ms2 * 1e3, 2),
                                       "gbs": round(ws2.algorithmic_bytes() / (ms2 / 1e3) / 1e9, 2),
                                       "algorithmic_bytes_per_layer": ws2.algorithmic_bytes()}
            # 64-layer stack, chained through the residual stream
            _log("64-layer stack")
            stack = make_layers(pkg, workloads, wl, 64, dev, first_layer=100)
            mss, _ = time_layers(pkg, stack, x, 128, 64)
            extras["stack64"] = {"layers": 64, "bytes": 64 * wl.algorithmic_bytes(),
                                 "ms_per_stack": round(mss * 64, 4), "us_per_layer": round(mss * 1e3, 2),
                                 "sustained_gbs": round(wl.algorithmic_bytes() / (mss / 1e3) / 1e9, 2)}
            del stack
            torch.cuda.empty_cache()
            # prefill chunk
            _log("prefill M=2048")
            wp = workloads.WORKLOADS["qwen3-27b-mlp-prefill-m2048-bfp8"]
            lp = make_layers(pkg, workloads, wp, 2, dev)
            xp = workloads.activations(wp.tokens, wp.hidden, gain=False, device=dev)
            msp, _ = time_layers(pkg, lp, xp, 20, 5)
            tflops = wp.flops() / (msp / 1e3) / 1e12
            extras["prefill_m2048"] = {"us_per_layer": round(msp * 1e3, 1), "tflops": round(tflops, 1),
                                       "mfma_util_vs_bf16_peak": round(tflops / BF16_MFMA_PEAK_TFLOPS, 4)}
            del lp
            torch.cuda.empty_cache()
        result["extras"] = extras
    if not args.no_cpu:
        _log("CPU baseline")
        result["cpu_baseline"] = cpu_baseline(pkg, workloads, wl, dev, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
