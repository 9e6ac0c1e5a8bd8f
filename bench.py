#!/usr/bin/env python3
"""W4A16 benchmark on one MI355X: HBM GB/s at M=1 and MFMA TFLOP/s at M=2048.

Step = one Qwen3-8B decode sweep at M=1 (config 2): 36 layers x 7 projections
(q, k, v, o, gate, up, down), each a separate ``int4_matmul`` call on that
layer's own weights, which is the reference's own call pattern
(engine/llama_attention.py:83-85, engine/llama_mlp.py:30-33).  The 3.69 GB of
INT4 weights + scales exceed the 256 MB Infinity Cache, so every step streams
them from HBM.  The sweep is captured once as a HIP graph and replayed; inputs
are resident in HBM before the timed region.  ``value`` = algorithmic bytes of
the sweep / time per step.

The JSON line also carries:
  fused_sweep     the same 36 layers through ``int4_matmul_grouped``: q/k/v in
                  one launch, o, gate+up in one launch, down (4 launches/layer).
  per_projection  M=1 launch durations per projection.
  batched_decode  config 3: M in {4, 8, 16, 32} at gate/up and down.
  prefill         config 4: the seven projections at M=2048, per projection and
                  as a layer (drop-in and grouped), TFLOP/s vs 2.5 PFLOP/s, and
                  the vendor dense bf16 GEMM on the gate shape for comparison.
  roofline        decode kernel on gate_proj (K=4096, N=12288, M=1): algorithmic
                  bytes per launch / average launch duration, against 8 TB/s.
  roofline_prefill  the GEMM on gate_proj at M=2048 against dense bf16 MFMA peak.
  lm_head_M1      the dense bf16 lm_head GEMV at M=1 (Qwen3-8B vocab), GB/s.
  cpu_baseline    the reference's host path (dequantize with bf16 scales, then
                  x @ w in bf16, engine/kernels/quant.py:264-266), restated in
                  oracle/int4_oracle.cpu_path, timed on this host's usable
                  cores: config 1 in full, configs 2-4 per projection of one
                  layer, config 5 per projection at M=1.

Launch durations are HIP events on the launch stream around a graph of 36
back-to-back launches on distinct weights, divided by 36, so they include the
~1-2 us dispatch gap between graph kernels; rocprofv3's per-kernel average
excludes that gap.

    python bench.py [--steps K] [--warmup W] [--gpus 1]
    python bench.py --kernels-only [--copy-calibration]   # roofline kernels only (for rocprofv3)
"""

from __future__ import annotations

import argparse
import json
import os
import re
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
LAUNCHES = 36  # distinct weight sets per timed graph (one per layer)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic_gemv_gate_m1.md")
TRAFFIC_FILE_PREFILL = os.path.join(ROOT, "profiles", "traffic_gemm_gate_m2048.md")


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


def time_launches(fn, stream, reps: int = 10) -> float:
    """us per launch of `fn` (which issues LAUNCHES launches), from a captured graph."""
    g, _ = capture(fn, stream)
    for _ in range(3):
        g.replay()
    us = time_graph(g, stream, reps) * 1e3 / LAUNCHES
    del g
    return us


def read_traffic(path: str):
    """HBM bytes per launch recorded by the rocprofv3 --pmc summary at `path` (or None)."""
    try:
        with open(path) as f:
            text = f.read()
    except OSError:
        return None
    m = re.search(r"^traffic_bytes_per_launch:\s*([0-9.eE+]+)", text, re.M)
    return float(m.group(1)) if m else None


def _usable_cores() -> tuple[int, dict]:
    """Host cores this process may run on: the least of os.cpu_count(), the
    affinity mask and the cgroup CPU quota (a GPU box grants a share of its
    host)."""
    info = {"os_cpu_count": os.cpu_count()}
    n = os.cpu_count() or 1
    try:
        info["affinity"] = len(os.sched_getaffinity(0))
        n = min(n, info["affinity"])
    except (AttributeError, OSError):
        pass
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            info["cgroup_quota_cpus"] = round(int(quota) / int(period), 2)
            n = min(n, max(1, int(int(quota) / int(period))))
    except (OSError, ValueError):
        pass
    return n, info


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(budget_s: float) -> dict:
    """The reference's host path (engine/kernels/quant.py:264-266: dequantize
    with bf16 scales, then x @ w in bf16), restated in oracle.int4_oracle.cpu_path,
    timed on this host with torch using every usable core.

    Rows: config 1 in full; one layer of config 2 (7 projections, M=1); config
    3 (gate and down at M = 4..32); one layer of config 4 (7 projections at
    M=2048); config 5 per projection at M=1.  Each row: 1 warmup run (3 for
    M <= 32), then the median of 5 runs (3 at M >= 2048; fewer once the row
    has used its share of ``budget_s``).  ``value`` is the config-2 layer's
    GB/s, the unit of the headline metric.
    """
    import torch

    from oracle import int4_oracle as orc
    from w4a16 import synth

    cores, info = _usable_cores()
    torch.set_num_threads(cores)
    shapes8 = synth.QWEN3_8B
    rows_spec = [("config1", "qwen3-0.6b gate_proj", 1, *synth.QWEN3_06B_GATE[1:])]
    rows_spec += [("config2_layer", f"qwen3-8b {name}", 1, k, n) for name, k, n in shapes8]
    rows_spec += [("config3", f"qwen3-8b {name} M={m}", m, k, n)
                  for m in (4, 8, 16, 32) for name, k, n in shapes8 if name in ("gate_proj", "down_proj")]
    rows_spec += [("config4_layer", f"qwen3-8b {name} M=2048", 2048, k, n) for name, k, n in shapes8]
    rows_spec += [("config5", f"qwen3-32b {name}", 1, k, n) for name, k, n in synth.QWEN3_32B if name != "v_proj"
                  and name != "up_proj"]
    per_row = budget_s / len(rows_spec)
    rows = []
    t_start = time.perf_counter()
    weights = {}
    for cfg, label, m, k, n in rows_spec:
        if (k, n) not in weights:
            weights[(k, n)] = synth.make_weight(k, n, seed=k * 7 + n)
        packed, scale = weights[(k, n)]
        x = synth.make_activations(m, k, seed=m + k)
        for _ in range(3 if m <= 32 else 1):
            orc.cpu_path(x, packed, scale)
        times = []
        row_t0 = time.perf_counter()
        for _ in range(5 if m <= 32 else 3):
            t0 = time.perf_counter()
            orc.cpu_path(x, packed, scale)
            times.append(time.perf_counter() - t0)
            if time.perf_counter() - row_t0 > per_row and len(times) >= 1:
                break
        t = statistics.median(times)
        b = synth.algorithmic_bytes(m, k, n)
        f = synth.algorithmic_flops(m, k, n)
        rows.append({"config": cfg, "workload": label, "M": m, "K": k, "N": n, "runs": len(times),
                     "ms": round(t * 1e3, 3), "GB/s": round(b / t / 1e9, 3), "GFLOP/s": round(f / t / 1e9, 2)})
        log(f"  cpu {label:28s} M={m:5d}: {t * 1e3:9.2f} ms  {b / t / 1e9:7.3f} GB/s  {f / t / 1e9:8.2f} GFLOP/s")
    elapsed = time.perf_counter() - t_start
    layer = [r for r in rows if r["config"] == "config2_layer"]
    layer_bytes = sum(synth.algorithmic_bytes(1, r["K"], r["N"]) for r in layer)
    layer_s = sum(r["ms"] for r in layer) * 1e-3
    return {
        "value": round(layer_bytes / layer_s / 1e9, 3),
        "unit": "GB/s",
        "cores": torch.get_num_threads(),
        "kind": "port",
        "cpu_model": _cpu_model(),
        "os_cpu_count": info.get("os_cpu_count"),
        "usable_cores": info,
        "torch_threads": torch.get_num_threads(),
        "sample": (
            f"one Qwen3-8B layer at M=1 (7 projections, {layer_bytes / 1e6:.1f} MB algorithmic) timed per projection "
            f"({layer_s * 1e3:.1f} ms/layer; the 36-layer sweep would take 36x as long), plus the rows below, "
            f"{elapsed:.1f} s of CPU work in all on {torch.get_num_threads()} torch threads"
        ),
        "rows": rows,
    }


def make_layers(layers: int, shapes, dev):
    from w4a16 import synth

    return [
        [synth.make_weight(k, n, seed=1000 * layer + i, device=dev) for i, (_, k, n) in enumerate(shapes)]
        for layer in range(layers)
    ]


def roofline_decode(us: float) -> dict:
    from w4a16 import synth

    b = synth.algorithmic_bytes(1, 4096, 12288)
    ach = b / (us * 1e-6) / 1e9
    return {
        "bound": "hbm",
        "achieved": round(ach, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(ach / HBM_PEAK_GBS, 4),
        "traffic": read_traffic(TRAFFIC_FILE),
        "kernel": "gemv_kernel<8, 4, true, false, 1, false> (gate_proj K=4096 N=12288 M=1, one launch of int4_matmul)",
        "bytes_per_launch": b,
        "avg_launch_us": round(us, 3),
    }


def roofline_prefill(us: float) -> dict:
    from w4a16 import synth

    f = synth.algorithmic_flops(2048, 4096, 12288)
    ach = f / (us * 1e-6) / 1e12
    return {
        "bound": "mfma",
        "achieved": round(ach, 1),
        "peak": BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(ach / BF16_PEAK_TFLOPS, 4),
        "traffic": read_traffic(TRAFFIC_FILE_PREFILL),
        "kernel": "gemm_kernel<4, true, 1, false> (gate_proj K=4096 N=12288 M=2048), after rowsum_kernel",
        "flops_per_launch": f,
        "avg_launch_us": round(us, 3),
    }


KERNEL_SETS = ("gate_m1", "gate_m16", "gate_m32", "down_m32", "prefill_gate")


def kernels_only(args) -> int:
    """Only the roofline kernels (or the --kernels list), plus optionally a
    copy of known size, for rocprofv3 (kernel traces and counter passes)."""
    import torch

    from w4a16 import _native, int4_matmul, synth

    _native.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.Stream()
    if args.copy_calibration:
        # 256 MiB device-to-device copy: FETCH_SIZE / WRITE_SIZE of this dispatch
        # calibrate the counters against a known byte count.
        src = torch.empty(64 << 20, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy calibration: 3 x {src.numel() * 4} bytes read and written")
        del src, dst
    which = args.kernels.split(",") if args.kernels else ["gate_m1"] + ([] if args.no_prefill else ["prefill_gate"])
    for w in which:
        if w not in KERNEL_SETS:
            raise SystemExit(f"unknown kernel set {w!r}; choose from {KERNEL_SETS}")
    gate = [synth.make_weight(4096, 12288, seed=1000 * l + 4, device=dev) for l in range(LAUNCHES)]
    down = ([synth.make_weight(12288, 4096, seed=1000 * l + 6, device=dev) for l in range(LAUNCHES)]
            if "down_m32" in which else None)
    out = {}
    for w in which:
        if w == "prefill_gate":
            x = synth.make_activations(2048, 4096, seed=4097, device=dev)
            us = time_launches(lambda: [int4_matmul(x, *gate[l]) for l in range(LAUNCHES)], stream, reps=3)
            out["prefill_gate_m2048"] = roofline_prefill(us)
        else:
            m = int(w.split("_m")[1])
            k, ws = (12288, down) if w.startswith("down") else (4096, gate)
            x = synth.make_activations(m, k, seed=k + m, device=dev)
            us = time_launches(lambda: [int4_matmul(x, *ws[l]) for l in range(LAUNCHES)], stream)
            n = ws[0][0].shape[1]
            b = synth.algorithmic_bytes(m, k, n)
            out[w] = {"us": round(us, 3), "GB/s": round(b / (us * 1e-6) / 1e9, 1)}
            if w == "gate_m1":
                out["decode_gate_m1"] = roofline_decode(us)
        log(f"{w}: {us:.2f} us/launch")
    print(json.dumps(out), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--cpu-seconds", type=float, default=30.0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--no-32b", action="store_true", help="skip the Qwen3-32B (config 5) lines")
    ap.add_argument("--kernels-only", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true")
    ap.add_argument("--kernels", default="", help=f"--kernels-only: comma list of {KERNEL_SETS}")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print(
            "bench.py: this build measures one GPU only (the W4A16 kernels run on a single MI355X; "
            "multi-GPU sharding is a design note, not a measured path). Run with --gpus 1.",
            file=sys.stderr,
        )
        return 2
    if args.kernels_only:
        return kernels_only(args)

    import torch

    from w4a16 import _native, int4_matmul, int4_matmul_grouped, int4_swiglu, synth

    _native.load_library()
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    layers = args.layers
    shapes = synth.QWEN3_8B
    names = [s[0] for s in shapes]
    ix = {name: i for i, name in enumerate(names)}

    # ---- weights: one distinct INT4 set per layer, resident in HBM ----
    t0 = time.perf_counter()
    weights = make_layers(layers, shapes, dev)
    xs = {k: synth.make_activations(1, k, seed=k, device=dev) for k in {k for _, k, _ in shapes}}
    torch.cuda.synchronize()
    log(f"generated {layers} layers of weights in {time.perf_counter() - t0:.1f}s")

    step_bytes = layers * sum(synth.algorithmic_bytes(1, k, n) for _, k, n in shapes)
    stream = torch.cuda.Stream()

    def sweep():
        outs = []
        for layer in range(layers):
            for (_, k, n), (packed, scale) in zip(shapes, weights[layer]):
                outs.append(int4_matmul(xs[k], packed, scale))
        return outs

    def fused_layer(w, x4096):
        # q/k/v in one grouped launch, gate/up as one fused SwiGLU call whose
        # output h feeds down.
        qkv = int4_matmul_grouped(x4096, [w[ix["q_proj"]], w[ix["k_proj"]], w[ix["v_proj"]]])
        o = int4_matmul(x4096, *w[ix["o_proj"]])
        h = int4_swiglu(x4096, w[ix["gate_proj"]], w[ix["up_proj"]])
        d = int4_matmul(h, *w[ix["down_proj"]])
        return qkv + [o, h, d]

    def fused_sweep():
        return [fused_layer(weights[l], xs[4096]) for l in range(layers)]

    # ---- headline: drop-in sweep ----
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
    del g_sweep
    log(f"sweep: {ms_per_step * 1e3:.1f} us/step, {value:.1f} GB/s (wall {wall * 1e3 / args.steps:.1f} ms/step)")

    g_fused, _ = capture(fused_sweep, stream)
    for _ in range(args.warmup):
        g_fused.replay()
    fms = time_graph(g_fused, stream, args.steps)
    del g_fused
    fused = {
        "ms_per_step": round(fms, 5),
        "GB/s": round(step_bytes / (fms * 1e-3) / 1e9, 1),
        "frac_of_hbm_peak": round(step_bytes / (fms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "launches_per_step": 4 * layers,
    }
    log(f"fused sweep: {fms * 1e3:.1f} us/step, {fused['GB/s']} GB/s")

    # ---- per-projection launch durations at M=1 ----
    per_proj = {}
    for i, (name, k, n) in enumerate(shapes):
        us = time_launches(lambda i=i, k=k: [int4_matmul(xs[k], *weights[l % layers][i]) for l in range(LAUNCHES)],
                           stream)
        gbs = synth.algorithmic_bytes(1, k, n) / (us * 1e-6) / 1e9
        per_proj[name] = {"us": round(us, 3), "GB/s": round(gbs, 1)}
        log(f"  {name:10s} K={k:5d} N={n:5d}: {us:7.2f} us/launch  {gbs:7.1f} GB/s")
    us = time_launches(lambda: [int4_swiglu(xs[4096], weights[l % layers][ix["gate_proj"]],
                                            weights[l % layers][ix["up_proj"]]) for l in range(LAUNCHES)], stream)
    gbs = 2 * synth.algorithmic_bytes(1, 4096, 12288) / (us * 1e-6) / 1e9
    per_proj["swiglu_gate_up"] = {"us": round(us, 3), "GB/s": round(gbs, 1)}
    log(f"  swiglu gate+up     : {us:7.2f} us/launch  {gbs:7.1f} GB/s")
    roofline = roofline_decode(per_proj["gate_proj"]["us"])

    # ---- config 3: batched decode / verify ----
    batched = {}
    for m in (4, 8, 16, 32):
        xm = {k: synth.make_activations(m, k, seed=k + m, device=dev) for k in (4096, 12288)}
        for name in ("gate_proj", "down_proj"):
            i = ix[name]
            _, k, n = shapes[i]
            us = time_launches(lambda i=i, k=k: [int4_matmul(xm[k], *weights[l % layers][i]) for l in range(LAUNCHES)],
                               stream)
            gbs = synth.algorithmic_bytes(m, k, n) / (us * 1e-6) / 1e9
            tf = synth.algorithmic_flops(m, k, n) / (us * 1e-6) / 1e12
            batched[f"M{m}_{name}"] = {"us": round(us, 3), "GB/s": round(gbs, 1), "TFLOP/s": round(tf, 2)}
            log(f"  M={m:2d} {name:10s}: {us:7.2f} us/launch  {gbs:7.1f} GB/s  {tf:6.2f} TFLOP/s")
        del xm

    # ---- config 4: prefill at M=2048 ----
    prefill = None
    roof_pf = None
    if not args.no_prefill:
        m = 2048
        xp = {k: synth.make_activations(m, k, seed=k + 1, device=dev) for k in {k for _, k, _ in shapes}}
        proj = {}
        for i, (name, k, n) in enumerate(shapes):
            us = time_launches(lambda i=i, k=k: [int4_matmul(xp[k], *weights[l % layers][i]) for l in range(LAUNCHES)],
                               stream, reps=3)
            tf = synth.algorithmic_flops(m, k, n) / (us * 1e-6) / 1e12
            proj[name] = {"us": round(us, 2), "TFLOP/s": round(tf, 1)}
            log(f"  prefill {name:10s}: {us:8.2f} us  {tf:7.1f} TFLOP/s")
        us = time_launches(lambda: [int4_swiglu(xp[4096], weights[l % layers][ix["gate_proj"]],
                                                weights[l % layers][ix["up_proj"]]) for l in range(LAUNCHES)],
                           stream, reps=3)
        tf = 2 * synth.algorithmic_flops(m, 4096, 12288) / (us * 1e-6) / 1e12
        proj["swiglu_gate_up"] = {"us": round(us, 2), "TFLOP/s": round(tf, 1)}
        log(f"  prefill swiglu    : {us:8.2f} us  {tf:7.1f} TFLOP/s")
        # The practical ceiling on this chip: the vendor dense bf16 GEMM
        # (torch.matmul, hipBLASLt) on the gate shape, same activations, four
        # distinct N(0, 0.02) bf16 weights (not INT4; no dequantization).
        gen = torch.Generator(device=dev).manual_seed(7)
        wd = [torch.randn(4096, 12288, device=dev, dtype=torch.bfloat16, generator=gen).mul_(0.02) for _ in range(4)]
        us = time_launches(lambda: [xp[4096] @ wd[l % 4] for l in range(LAUNCHES)], stream, reps=3)
        del wd
        tf = synth.algorithmic_flops(m, 4096, 12288) / (us * 1e-6) / 1e12
        dense_ref = {"workload": "dense bf16 torch.matmul (hipBLASLt), M=2048 K=4096 N=12288",
                     "us": round(us, 2), "TFLOP/s": round(tf, 1)}
        log(f"  dense bf16 gate (hipBLASLt): {us:8.2f} us  {tf:7.1f} TFLOP/s")
        flops = sum(synth.algorithmic_flops(m, k, n) for _, k, n in shapes)

        def layer_fn():
            return [int4_matmul(xp[k], *weights[l][i]) for l in range(4) for i, (_, k, n) in enumerate(shapes)]

        def layer_fused():
            return [fused_layer(weights[l], xp[4096]) for l in range(4)]

        res = {}
        for tag, fn in (("drop_in", layer_fn), ("grouped", layer_fused)):
            g, _ = capture(fn, stream)
            g.replay()
            ms = time_graph(g, stream, 3) / 4
            del g
            res[tag] = {"us_per_layer": round(ms * 1e3, 1), "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1)}
            log(f"prefill layer ({tag}): {ms * 1e3:.1f} us, {res[tag]['TFLOP/s']} TFLOP/s")
        prefill = {
            "workload": "qwen3-8b, M=2048, 7 projections",
            "per_projection": proj,
            "layer": res,
            "dense_bf16_reference": dense_ref,
            "frac_of_bf16_peak": round(res["drop_in"]["TFLOP/s"] / BF16_PEAK_TFLOPS, 4),
            "peak_tflops": BF16_PEAK_TFLOPS,
        }
        roof_pf = roofline_prefill(proj["gate_proj"]["us"])
        del xp

    # ---- config 1: Qwen3-0.6B gate at M=1 (the reference's CPU-runnable case) ----
    _, k1, n1 = synth.QWEN3_06B_GATE
    w1 = [synth.make_weight(k1, n1, seed=60 + l, device=dev) for l in range(LAUNCHES)]
    x1 = synth.make_activations(1, k1, seed=61, device=dev)
    us = time_launches(lambda: [int4_matmul(x1, *w1[l]) for l in range(LAUNCHES)], stream)
    config1 = {"workload": "qwen3-0.6b gate_proj M=1 K=1024 N=3072", "us": round(us, 3),
               "GB/s": round(synth.algorithmic_bytes(1, k1, n1) / (us * 1e-6) / 1e9, 1)}
    log(f"config 1 (0.6B gate M=1): {us:.2f} us/launch, {config1['GB/s']} GB/s")
    del w1

    # ---- lm_head: the dense bf16 decode GEMV of the untied Qwen3-8B output projection ----
    from w4a16 import lm_head

    vocab, dmodel = 151936, 4096
    gen = torch.Generator(device=dev).manual_seed(5)
    w_lm = (torch.randn(vocab, dmodel, generator=gen, device=dev) * 0.02).bfloat16()
    x_lm = synth.make_activations(1, dmodel, seed=9, device=dev)
    us = time_launches(lambda: [lm_head(x_lm, w_lm) for _ in range(LAUNCHES)], stream, reps=3)
    lm_bytes = vocab * dmodel * 2 + dmodel * 2 + vocab * 2
    lm = {"workload": "qwen3-8b lm_head M=1 (151936 x 4096 dense bf16, 1.24 GB)", "us": round(us, 2),
          "GB/s": round(lm_bytes / (us * 1e-6) / 1e9, 1),
          "frac_of_hbm_peak": round(lm_bytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    log(f"lm_head M=1: {us:.1f} us/launch, {lm['GB/s']} GB/s")
    del w_lm
    torch.cuda.empty_cache()

    # ---- config 5: Qwen3-32B, 64-layer M=1 sweep and one M=4096 prefill layer ----
    config5 = None
    if not args.no_32b:
        del weights
        torch.cuda.empty_cache()
        shapes32 = synth.QWEN3_32B
        t0 = time.perf_counter()
        w32 = make_layers(synth.QWEN3_32B_LAYERS, shapes32, dev)
        x32 = {k: synth.make_activations(1, k, seed=k, device=dev) for k in {k for _, k, _ in shapes32}}
        torch.cuda.synchronize()
        log(f"generated {len(w32)} Qwen3-32B layers in {time.perf_counter() - t0:.1f}s")
        bytes32 = sum(synth.algorithmic_bytes(1, k, n) for _, k, n in shapes32) * len(w32)

        def sweep32():
            return [int4_matmul(x32[k], *w32[l][i]) for l in range(len(w32)) for i, (_, k, _) in enumerate(shapes32)]

        g32, _ = capture(sweep32, stream)
        for _ in range(2):
            g32.replay()
        ms32 = time_graph(g32, stream, max(3, args.steps // 2))
        del g32
        gbs32 = bytes32 / (ms32 * 1e-3) / 1e9
        log(f"config 5 (32B M=1, {len(w32)} layers): {ms32:.3f} ms/step, {gbs32:.1f} GB/s")
        config5 = {"decode_M1": {"layers": len(w32), "ms_per_step": round(ms32, 4), "GB/s": round(gbs32, 1),
                                 "frac_of_hbm_peak": round(gbs32 / HBM_PEAK_GBS, 4), "bytes_per_step": bytes32}}
        if not args.no_prefill:
            m = 4096
            xp32 = {k: synth.make_activations(m, k, seed=k + 2, device=dev) for k in {k for _, k, _ in shapes32}}

            def layer32():
                return [int4_matmul(xp32[k], *w32[0][i]) for i, (_, k, _) in enumerate(shapes32)]

            g, _ = capture(layer32, stream)
            g.replay()
            ms = time_graph(g, stream, 3)
            del g
            fl = sum(synth.algorithmic_flops(m, k, n) for _, k, n in shapes32)
            tf = fl / (ms * 1e-3) / 1e12
            log(f"config 5 (32B M=4096 layer): {ms * 1e3:.1f} us, {tf:.1f} TFLOP/s")
            config5["prefill_M4096_layer"] = {"us": round(ms * 1e3, 1), "TFLOP/s": round(tf, 1),
                                              "frac_of_bf16_peak": round(tf / BF16_PEAK_TFLOPS, 4)}
            del xp32
        del w32
        torch.cuda.empty_cache()

    # ---- CPU baseline: the reference's host path ----
    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(args.cpu_seconds)
        log(f"cpu baseline: {cpu['value']} GB/s on {cpu['cores']} threads ({cpu['cpu_model']})")

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
            "workload": f"qwen3-8b decode M=1 (config 2): {layers}-layer x 7-projection weight-streaming sweep, "
                        "one int4_matmul call per projection, replayed as one HIP graph",
            "M": 1,
            "layers": layers,
            "bytes_per_step": step_bytes,
            "frac_of_hbm_peak": round(value / HBM_PEAK_GBS, 4),
        },
        "fused_sweep": fused,
        "per_projection_M1": per_proj,
        "batched_decode": batched,
        "prefill": prefill,
        "config1_qwen3_06b": config1,
        "lm_head_M1": lm,
        "config5_qwen3_32b": config5,
        "roofline": roofline,
        "roofline_prefill": roof_pf,
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
