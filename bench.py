#!/usr/bin/env python3
"""W4A16 benchmark on one MI355X: HBM GB/s at M=1 and MFMA TFLOP/s at M=2048.

Step = one Qwen3-8B decode sweep at M=1: 36 layers x 7 projections (q, k, v, o,
gate, up, down), each a separate ``int4_matmul`` call on that layer's own
weights (3.69 GB of INT4 weights + scales, so nothing is served from the
256 MB Infinity Cache), captured once as a HIP graph and replayed.  ``value`` is
the sweep's algorithmic bytes / wall time per step, with everything resident in
HBM before the timed region.

Printed as one JSON line, with:
  roofline      the skinny kernel on gate_proj (K=4096, N=12288, M=1): algorithmic
                bytes per launch / average launch duration (HIP events around a
                graph of 36 back-to-back launches on distinct layers), against
                8 TB/s HBM.
  prefill       one Qwen3-8B layer at M=2048 (7 projections, config 4): TFLOP/s
                against 2.5 PFLOP/s dense bf16, plus the gate_proj GEMM alone.
  cpu_baseline  the reference's host path (dequantize with bf16 scales, then
                x @ w in bf16, engine/kernels/quant.py:264-266) restated in
                oracle/int4_oracle.cpu_path, timed on this host for one layer.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "inf-engine_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HBM_PEAK_GBS = 8000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "W4A16 GEMM: HBM GB/s (% of peak) at M=1; MFMA TFLOPS (% peak) at M=2048"


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def capture(fn, stream):
    """Run fn once eagerly on `stream` (creates workspaces), then capture it."""
    import torch

    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        out = fn()
    torch.cuda.synchronize()
    return g, out


def time_graph(g, stream, reps: int) -> float:
    """Average ms per replay, HIP events recorded on the replay stream."""
    import torch

    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(reps):
            g.replay()
        end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def cpu_baseline(host_layer, k_model: int) -> dict:
    import torch

    from oracle import int4_oracle as orc
    from w4a16 import synth

    threads = torch.get_num_threads()
    total_s = 0.0
    total_bytes = 0
    for name, k, n, packed, scale in host_layer:
        x = synth.make_activations(1, k, seed=5)
        orc.cpu_path(x, packed, scale)  # warmup
        times = []
        for _ in range(3):
            t0 = time.perf_counter()
            orc.cpu_path(x, packed, scale)
            times.append(time.perf_counter() - t0)
        total_s += statistics.median(times)
        total_bytes += synth.algorithmic_bytes(1, k, n)
    return {
        "value": round(total_bytes / total_s / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": (
            "one Qwen3-8B layer at M=1 (7 projections, 102.6 MB), median of 3 runs after 1 warmup per "
            f"projection, {total_s * 1e3:.1f} ms per layer; the 36-layer sweep is 36x this"
        ),
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py: this build measures one GPU only (the W4A16 kernels run on a single MI355X; "
            "multi-GPU sharding is a design note, not a measured path). Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2

    import torch

    from w4a16 import _native, int4_matmul, synth

    _native.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    layers = args.layers
    shapes = synth.QWEN3_8B

    # ---- weights: one distinct INT4 set per layer, resident in HBM ----
    t0 = time.perf_counter()
    weights = []
    for layer in range(layers):
        weights.append([synth.make_weight(k, n, seed=1000 * layer + i, device=dev) for i, (_, k, n) in enumerate(shapes)])
    xs = {k: synth.make_activations(1, k, seed=k, device=dev) for k in {k for _, k, _ in shapes}}
    torch.cuda.synchronize()
    log(f"generated {layers} layers of weights in {time.perf_counter() - t0:.1f}s")

    step_bytes = layers * sum(synth.algorithmic_bytes(1, k, n) for _, k, n in shapes)

    def sweep():
        outs = []
        for layer in range(layers):
            for (_, k, n), (packed, scale) in zip(shapes, weights[layer]):
                outs.append(int4_matmul(xs[k], packed, scale))
        return outs

    stream = torch.cuda.Stream()
    g_sweep, _ = capture(sweep, stream)

    for _ in range(args.warmup):
        g_sweep.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(args.steps):
            g_sweep.replay()
        end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_per_step = start.elapsed_time(end) / args.steps
    value = step_bytes / (ms_per_step * 1e-3) / 1e9
    log(f"sweep: {ms_per_step * 1e3:.1f} us/step, {value:.1f} GB/s (wall {wall * 1e3 / args.steps:.1f} ms/step)")

    # ---- per-projection launch durations (graph of `layers` launches each) ----
    per_proj = {}
    for i, (name, k, n) in enumerate(shapes):
        def proj(i=i, k=k):
            return [int4_matmul(xs[k], *weights[layer][i]) for layer in range(layers)]

        g, _ = capture(proj, stream)
        for _ in range(3):
            g.replay()
        us = time_graph(g, stream, 10) * 1e3 / layers
        gbs = synth.algorithmic_bytes(1, k, n) / (us * 1e-6) / 1e9
        per_proj[name] = {"us": round(us, 3), "GB/s": round(gbs, 1)}
        log(f"  {name:10s} K={k:5d} N={n:5d}: {us:7.2f} us/launch  {gbs:7.1f} GB/s")
        del g
    gate = per_proj["gate_proj"]
    gate_bytes = synth.algorithmic_bytes(1, 4096, 12288)
    roofline = {
        "bound": "hbm",
        "achieved": gate["GB/s"],
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(gate["GB/s"] / HBM_PEAK_GBS, 4),
        "traffic": None,
        "kernel": "skinny_kernel<1,16> (gate_proj K=4096 N=12288 M=1)",
        "bytes_per_launch": gate_bytes,
        "avg_launch_us": gate["us"],
    }

    # ---- prefill: one layer at M=2048 ----
    prefill = None
    if not args.no_prefill:
        m = 2048
        xp = {k: synth.make_activations(m, k, seed=k + 1, device=dev) for k in {k for _, k, _ in shapes}}

        def layer_fn():
            return [int4_matmul(xp[k], *weights[0][i]) for i, (_, k, n) in enumerate(shapes)]

        g, _ = capture(layer_fn, stream)
        for _ in range(3):
            g.replay()
        ms = time_graph(g, stream, max(3, args.steps // 2))
        flops = sum(synth.algorithmic_flops(m, k, n) for _, k, n in shapes)
        tflops = flops / (ms * 1e-3) / 1e12
        del g
        gi = 4  # gate_proj

        def gate_fn():
            return [int4_matmul(xp[4096], *weights[layer][gi]) for layer in range(4)]

        g, _ = capture(gate_fn, stream)
        g.replay()
        gms = time_graph(g, stream, 5) / 4
        gtf = synth.algorithmic_flops(m, 4096, 12288) / (gms * 1e-3) / 1e12
        del g
        prefill = {
            "workload": "qwen3-8b layer, M=2048, 7 projections",
            "ms_per_layer": round(ms, 4),
            "tflops": round(tflops, 2),
            "frac_of_bf16_peak": round(tflops / BF16_PEAK_TFLOPS, 4),
            "gate_proj_us": round(gms * 1e3, 2),
            "gate_proj_tflops": round(gtf, 2),
            "peak_tflops": BF16_PEAK_TFLOPS,
        }
        log(f"prefill layer M=2048: {ms * 1e3:.1f} us, {tflops:.1f} TFLOP/s; gate {gms * 1e3:.1f} us {gtf:.1f} TFLOP/s")
        del xp

    # ---- CPU baseline: the reference's host path on one layer ----
    cpu = None
    if not args.no_cpu_baseline:
        host_layer = [(name, k, n, p.cpu(), s.cpu()) for (name, k, n), (p, s) in zip(shapes, weights[0])]
        cpu = cpu_baseline(host_layer, 4096)
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads")

    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,0.02) bf16 weights quantized to int4 (group 128, fp32 scales), N(0,1) bf16 x",
        "config": {
            "workload": f"qwen3-8b decode M=1, {layers}-layer x 7-projection weight-streaming sweep (one HIP graph)",
            "M": 1,
            "layers": layers,
            "bytes_per_step": step_bytes,
            "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        },
        "per_projection_M1": per_proj,
        "roofline": roofline,
        "prefill": prefill,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
