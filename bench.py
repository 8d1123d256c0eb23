"""Benchmark: the MoE forward layer on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config fine_grained] [--routing random]

Workload (default): the fine-grained layer, T=4096 tokens, D=1024, F=4096,
E=64 experts, top-2, bf16, uniform routing (2 distinct experts per token),
x ~ N(0,1), W1/W2 ~ N(0, 1/fan_in), softmax gates; synthetic, seeded.

A step is one whole layer (routing -> SDD+GELU -> DSD -> combine) replayed
from a HIP graph captured once, with inputs resident in HBM. Before each
step a 512 MiB buffer is zeroed (outside the step's events) so the 256 MB
Infinity Cache and the L2s start cold, as the reference's timing does with
its L2 flush. Timed: exactly K steps between synchronizations, each as the
reference's timing loop runs one (sparsebench/timing.py:15-29: flush, event, layer,
event, synchronize), with the events on the replay stream; ms_per_step is
their median and value is useful TFLOP/s = 2*2*T*k*D*F / step time (padding
FLOPs not counted).

Also reported (same JSON line): eager-mode layer time, per-stage times from
events at the layer's stage marks (each of SDD and DSD is exactly one kernel,
so its stage time is that kernel's duration on its stream), the roofline of
the dominant kernel, and the CPU baseline: the oracle's fp32 loop-over-experts
layer on this host's cores, on the benchmark's CPU configuration (T=256,
D=128, F=512, E=8) with os.cpu_count() threads and with 1 thread, plus the
GPU workload itself in fp32 for scale.

Before timing, the layer's output is checked against a plain-torch fp32
reference on the GPU (max |err| / max |ref| <= 2e-2); a wrong layer is not timed.
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import torch

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, published
MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16, published
FLUSH_BYTES = 512 * 1024 * 1024
REL_GATE = 2e-2


def parse_args() -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--config", default="fine_grained", choices=["fine_grained", "mixtral", "replay_sweep"])
    p.add_argument("--routing", default="random", choices=["random", "zipf_perm", "zipf"])
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu-baseline", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--no-stages", action="store_true", help="skip the eager per-stage breakdown")
    p.add_argument("--calibrate-copy", action="store_true",
                   help="only copy 1 GiB five times (torch's copy kernel): the reference point that scales "
                        "rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    p.add_argument("--kernel-loop", type=int, default=0,
                   help="after the bench, replay the graph N more times (for rocprofv3 runs)")
    return p.parse_args()


def fp32_reference_gpu(x, idx, gates, w1, w2) -> torch.Tensor:
    """Loop over experts in fp32 on the GPU (exact-erf GELU): the correctness gate."""
    out = torch.zeros(x.shape[0], x.shape[1], dtype=torch.float32, device=x.device)
    for e in range(w1.shape[0]):
        token, slot = torch.nonzero(idx == e, as_tuple=True)
        if token.numel():
            h = x[token].float() @ w1[e].float()
            h = 0.5 * h * (1.0 + torch.erf(h * 0.7071067811865476))
            out.index_add_(0, token, (h @ w2[e].float()) * gates[token, slot, None].float())
    return out


def algorithmic_bytes(shape, active_experts: int) -> dict[str, int]:
    """Bytes each stage must move at least: inputs read once, outputs written once, no padding."""
    t, d, f, k = shape.num_tokens, shape.d_model, shape.ffn_dim, shape.top_k
    n = t * k
    return {
        "sdd": t * d * 2 + active_experts * d * f * 2 + n * f * 2,
        "dsd": n * f * 2 + active_experts * f * d * 2 + n * d * 2,
        "combine": n * d * 2 + n * (2 + 4) + t * d * 2,
    }


def measured_traffic(config: str, routing: str, stage: str) -> int | None:
    """HBM bytes per launch of `stage` from the committed rocprofv3 FETCH/WRITE summary, if one exists."""
    import pathlib
    import re

    for path in sorted(pathlib.Path(__file__).resolve().parent.glob("profiles/traffic_*.md")):
        for line in path.read_text().splitlines():
            m = re.match(r"\s*traffic_bytes (\S+) (\S+) (.*)", line)
            if m and m.group(1) == config and m.group(2) == routing:
                values = dict(kv.split("=") for kv in m.group(3).split())
                if stage in values:
                    return int(values[stage])
    return None


def _time_cpu_layer(x, idx, gates, w1, w2, threads: int, warmup: int, runs: int, budget_s: float | None = None
                    ) -> list[float]:
    """Seconds per run of the oracle's fp32 loop-over-experts layer with `threads` torch threads."""
    from oracle.moe_ref import moe_reference  # CPU baseline leg only

    saved = torch.get_num_threads()
    torch.set_num_threads(threads)
    try:
        for _ in range(warmup):
            moe_reference(x, idx, gates, w1, w2)
        times: list[float] = []
        start = time.perf_counter()
        while len(times) < runs or (budget_s is not None and time.perf_counter() - start < budget_s
                                     and len(times) < 200):
            t0 = time.perf_counter()
            moe_reference(x, idx, gates, w1, w2)
            times.append(time.perf_counter() - t0)
        return times
    finally:
        torch.set_num_threads(saved)


def cpu_baseline(shape, routing: str, seed: int) -> dict:
    """The oracle's fp32 loop-over-experts layer (the algorithm of the
    reference's sparsebench/reference.py:49-61) on this host's cores.

    value: configuration 1 of the benchmark (T=256, D=128, F=512, E=8, top-2,
    seed 0), 3 warm-ups then the median of 20 runs, with os.cpu_count()
    threads; also with 1 thread. Extra: the benchmarked GPU workload itself
    in fp32 with torch's default thread count, repeated for about 10 s of
    CPU work (at least 3 runs), for scale.
    """
    from sparsebench_amd.workloads import SHAPES, make_layer

    cores = os.cpu_count() or 1
    small = SHAPES["cpu_reference"]
    x, idx, gates, w1, w2 = make_layer(small, "random", 0, device="cpu", dtype=torch.float32)
    small_flops = small.useful_flops

    def leg(threads: int) -> dict:
        sec = statistics.median(_time_cpu_layer(x, idx, gates, w1, w2, threads, warmup=3, runs=20))
        return {"value": round(small_flops / sec / 1e12, 6), "ms_per_sample": round(sec * 1e3, 4), "threads": threads}

    all_cores, one_core = leg(cores), leg(1)

    default_threads = torch.get_num_threads()
    bx, bidx, bgates, bw1, bw2 = make_layer(shape, routing, seed, device="cpu", dtype=torch.float32)
    times = _time_cpu_layer(bx, bidx, bgates, bw1, bw2, default_threads, warmup=1, runs=3, budget_s=10.0)
    sec = statistics.median(times)
    return {
        "value": all_cores["value"],
        "unit": "TFLOP/s",
        "cores": cores,
        "kind": "port",
        "sample": (f"benchmark configuration 1 (T={small.num_tokens}, D={small.d_model}, F={small.ffn_dim}, "
                   f"E={small.num_experts}, top-2, seed 0): oracle fp32 loop-over-experts layer "
                   f"(oracle/moe_ref.py), 3 warm-ups, median of 20 runs, torch CPU with os.cpu_count() = "
                   f"{cores} threads"),
        "ms_per_sample": all_cores["ms_per_sample"],
        "single_thread": one_core,
        "cpu_model": _cpu_model(),
        "os_cpu_count": cores,
        "gpu_workload_fp32": {
            "value": round(shape.useful_flops / sec / 1e12, 6), "unit": "TFLOP/s", "threads": default_threads,
            "ms_per_sample": round(sec * 1e3, 3),
            "sample": (f"the whole {shape.name} layer in fp32, {routing} routing, median of {len(times)} runs "
                       f"over {sum(times):.1f} s"),
        },
    }


def _cpu_model() -> str:
    """Model name as lscpu prints it (from /proc/cpuinfo when lscpu is absent)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.strip().startswith("Model name"):
                return line.split(":", 1)[1].strip()
    except (OSError, subprocess.SubprocessError):
        pass
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build's path is single-GPU (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        return 2
    if not torch.cuda.is_available():
        print("bench.py needs a GPU (MI355X)", file=sys.stderr)
        return 2
    if args.calibrate_copy:
        src = torch.ones(1 << 30, dtype=torch.uint8, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("copied 1 GiB x 5")
        return 0

    from sparsebench_amd.moe import moe_forward
    from sparsebench_amd.workloads import SHAPES, make_layer

    shape = SHAPES[args.config]
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    x, idx, gates, w1, w2 = make_layer(shape, args.routing, args.seed, device=dev)
    gates = gates.to(torch.bfloat16)
    active = int(torch.unique(idx).numel())
    print(f"[bench] {shape} routing={args.routing} active_experts={active}", flush=True)

    # ---- correctness gate ----
    out = moe_forward(x, idx, gates, w1, w2)
    ref = fp32_reference_gpu(x, idx, gates, w1, w2)
    rel = float((out.float() - ref).abs().max() / ref.abs().max())
    print(f"[bench] correctness: max rel err {rel:.3e} (gate {REL_GATE})", flush=True)
    if not rel <= REL_GATE:
        print(json.dumps({"error": f"wrong answer: max rel err {rel}"}))
        return 1
    del ref

    flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device=dev)
    stream = torch.cuda.Stream(device=dev)

    # ---- capture the layer once ----
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for _ in range(2):
            moe_forward(x, idx, gates, w1, w2)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        g_out = moe_forward(x, idx, gates, w1, w2)
    torch.cuda.synchronize()

    def timed_replays(n: int) -> list[float]:
        samples = []
        with torch.cuda.stream(stream):
            for _ in range(n):
                flush.zero_()
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record(stream)
                graph.replay()
                e.record(stream)
                e.synchronize()  # one step at a time, as the reference's timing loop
                samples.append((s, e))
        torch.cuda.synchronize()
        return [s.elapsed_time(e) for s, e in samples]

    timed_replays(args.warmup)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    samples = timed_replays(args.steps)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms = statistics.median(samples)
    assert torch.equal(g_out, moe_forward(x, idx, gates, w1, w2)), "graph replay differs from eager"
    print(f"[bench] graph replay: median {ms:.4f} ms over {args.steps} steps (min {min(samples):.4f})", flush=True)

    # ---- eager layer and per-stage times ----
    stages: dict[str, float] = {}
    eager_ms = None
    if not args.no_stages:
        per_stage: dict[str, list[float]] = {}
        totals = []
        for it in range(args.warmup + args.steps):
            flush.zero_()
            events: list[tuple[str, torch.cuda.Event]] = []

            def mark(stage: str) -> None:
                ev = torch.cuda.Event(enable_timing=True)
                ev.record()
                events.append((stage, ev))

            start = torch.cuda.Event(enable_timing=True)
            start.record()
            moe_forward(x, idx, gates, w1, w2, mark=mark)
            torch.cuda.synchronize()
            if it < args.warmup:
                continue
            prev = start
            for stage, ev in events:
                per_stage.setdefault(stage, []).append(prev.elapsed_time(ev))
                prev = ev
            totals.append(start.elapsed_time(events[-1][1]))
        stages = {s: round(statistics.median(v), 4) for s, v in per_stage.items()}
        eager_ms = round(statistics.median(totals), 4)
        print(f"[bench] eager: {eager_ms} ms, stages {stages}", flush=True)

    # ---- roofline of the dominant kernel (SDD or DSD, one kernel each) ----
    # Both matmul stages are reported; the top-level fields are the longer one's.
    nbytes = algorithmic_bytes(shape, active)
    roofline = None
    if stages:
        flops = shape.useful_flops // 2

        def stage_roofline(name: str, kms: float) -> dict:
            ai = flops / nbytes[name]
            traffic = measured_traffic(args.config, args.routing, name)
            entry = {"kernel": f"{name} stage (one kernel)", "kernel_ms": kms, "traffic": traffic,
                     "traffic_source": (f"profiles/traffic_*.md (rocprofv3 FETCH_SIZE / WRITE_SIZE of this bench "
                                        f"command, committed; not measured in this run)" if traffic is not None
                                        else None)}
            if ai < MFMA_BF16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9):
                achieved = nbytes[name] / (kms * 1e-3) / 1e9
                return {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBS, 4), **entry, "algorithmic_bytes": nbytes[name],
                        "useful_tflops": round(flops / (kms * 1e-3) / 1e12, 2)}
            achieved = flops / (kms * 1e-3) / 1e12
            return {"bound": "mfma", "achieved": round(achieved, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                    "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4), **entry, "useful_flops": flops}

        per_kernel = {"sdd": stage_roofline("sdd", stages["SDD + GELU (fused)"]),
                      "dsd": stage_roofline("dsd", stages["DSD"])}
        name = "sdd" if per_kernel["sdd"]["kernel_ms"] >= per_kernel["dsd"]["kernel_ms"] else "dsd"
        roofline = dict(per_kernel[name])
        roofline["stages"] = {k: {f: v[f] for f in ("bound", "achieved", "unit", "frac", "kernel_ms", "traffic")}
                              for k, v in per_kernel.items()}

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline ...", flush=True)
        cpu = cpu_baseline(shape, args.routing, args.seed)
        print(f"[bench] CPU baseline (config 1): {cpu['value']} TFLOP/s on {cpu['cores']} threads, "
              f"{cpu['single_thread']['value']} on 1 thread; {cpu['cpu_model']}", flush=True)

    if args.kernel_loop:
        with torch.cuda.stream(stream):
            for _ in range(args.kernel_loop):
                graph.replay()
        torch.cuda.synchronize()

    tflops = shape.useful_flops / (ms * 1e-3) / 1e12
    line = {
        "metric": (f"MoE fwd layer ms + useful TFLOP/s, D{shape.d_model} F{shape.ffn_dim} E{shape.num_experts}, "
                   f"{shape.num_tokens} tok top-{shape.top_k} bf16"),
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded x, routing, random-init weights)",
        "config": {"workload": f"{shape.name} MoE forward layer", "tokens": shape.num_tokens,
                   "d_model": shape.d_model, "ffn_dim": shape.ffn_dim, "experts": shape.num_experts,
                   "top_k": shape.top_k, "routing": args.routing, "block_size": 128,
                   "timing": "hipGraph replay, 512 MiB cache flush between steps, median"},
        "layer_ms_eager": eager_ms,
        "stages_ms": stages,
        "wall_s_timed_steps": round(wall, 4),
        "max_rel_err": rel,
        "roofline": roofline,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
