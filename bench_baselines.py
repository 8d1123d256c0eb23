"""Same-box comparison tables: this build's MoE layer against other ways of
computing it on the same MI355X (the measurements of the reference's
bench/bench_moe.py and bench/bench_token_rounding.py, made here).

    python bench_baselines.py                 # both tables, markdown on stdout
    python bench_baselines.py --only layer    # or: --only rounding, --only replay, --only ceilings, --only gemm

Layer pipelines (everything from the routing to the [T, D] output is timed,
host syncs included):
  ours          moe_forward: GPU routing -> SDD (+ gather, GELU) -> DSD -> combine;
                no host sync. Timed eagerly, and as a captured graph.
  grouped_mm    sort copies by expert -> torch._grouped_mm -> GELU ->
                torch._grouped_mm -> unsort -> weighted sum (torch ops, no sync).
  loop          per expert: x[tokens] @ w1[e] -> GELU -> @ w2[e], expert counts
                read on the host (syncs).

Token rounding (SonicMoE; the router's scores from workloads.router_scores):
  the layer on the plain top-k list and on the token-rounded list, for
  moe_forward_assigned and for the grouped_mm pipeline on the same list; the
  rounding step alone (routing.route_rounded: rounding, its list and its
  layout, no sync); and moe_forward_rounded (rounding fused into the layer).

Replay sweep (D=2048, F=768, E=128, top-2, Zipf over a
permutation): moe_forward captured once in a graph with buffers for
T=16384, then replayed with fresh seeded x, routing and gates (seeds 1-4)
at T' in {512, 2048, 8192, 16384}, the token count a device scalar read
on the GPU each replay. Each replay is checked bit for bit against an eager
moe_forward at T'.

Ceilings (the box's practical roofs, next to the published 8 TB/s and
2.5 PFLOP/s): streaming reads of 2 GiB with 16-byte vector loads and through
LDS DMA (sbp_read of libsparsebench_probe.so, the load path of SDD / DSD), a 1 GiB device copy, and
dense bf16 GEMMs through torch.matmul (hipBLASLt), with the weight as the
layer stores it ([K, N]) and transposed ([N, K]); --only gemm runs just these.

Every pipeline is checked against the fp32 loop reference before it is
timed (max error <= 3e-2 (1 + max |ref|), the reference's check). Timing: a
512 MiB buffer is zeroed before each step (outside the events), events on
the current stream, median of 20 after 3 warm-ups.
"""

from __future__ import annotations

import argparse
import statistics

import torch
import torch.nn.functional as F

from sparsebench_amd.moe import moe_forward, moe_forward_assigned, moe_forward_rounded
from sparsebench_amd.routing import route_rounded
from sparsebench_amd.token_rounding import token_rounding, top_k_assignments
from sparsebench_amd.workloads import SHAPES, make_layer, router_scores, routing_case, softmax_gates

TOL = 3e-2
FLUSH_BYTES = 512 << 20


def time_ms(fn, flush: torch.Tensor, steps: int = 20, warmup: int = 3) -> float:
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(steps):
        flush.zero_()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        fn()
        e.record()
        e.synchronize()
        times.append(s.elapsed_time(e))
    return statistics.median(times)


def reference_fp32(x, token, expert, weight, w1, w2) -> torch.Tensor:
    """Loop over experts in fp32 on the GPU (ground truth for the checks)."""
    out = torch.zeros(x.shape[0], x.shape[1], device=x.device)
    for e in range(w1.shape[0]):
        m = expert == e
        if m.any():
            y = F.gelu(x[token[m]].float() @ w1[e].float()) @ w2[e].float()
            out.index_add_(0, token[m], y * weight[m, None].float())
    return out


def checked(fn, ref: torch.Tensor, flush: torch.Tensor) -> float | str:
    err = (fn().float() - ref).abs().max().item()
    if err > TOL * (1 + ref.abs().max().item()):
        return f"wrong ({err:.3g})"
    return time_ms(fn, flush)


def grouped_mm_layer(x, token, expert, weight, w1, w2) -> torch.Tensor:
    """Grouped GEMM over a flat list: sort by expert, two torch._grouped_mm
    calls with GELU between, then the weighted sum back per token."""
    num_experts = w1.shape[0]
    order = torch.sort(expert, stable=True).indices
    counts = torch.zeros(num_experts, dtype=torch.int32, device=x.device).scatter_add_(
        0, expert, torch.ones_like(expert, dtype=torch.int32))
    offs = torch.cumsum(counts, 0, dtype=torch.int32)
    tok = token[order]
    h = F.gelu(torch._grouped_mm(x[tok], w1, offs=offs))
    y = torch._grouped_mm(h, w2, offs=offs).float() * weight[order, None].float()
    return torch.zeros(x.shape[0], x.shape[1], device=x.device).index_add_(0, tok, y).to(x.dtype)


def loop_layer(x, token, expert, weight, w1, w2) -> torch.Tensor:
    out = torch.zeros(x.shape[0], x.shape[1], device=x.device)
    order = torch.sort(expert, stable=True).indices
    counts = torch.bincount(expert, minlength=w1.shape[0]).tolist()  # host sync
    start = 0
    for e, n in enumerate(counts):
        if n:
            rows = order[start:start + n]
            y = F.gelu(x[token[rows]] @ w1[e]) @ w2[e]
            out.index_add_(0, token[rows], y.float() * weight[rows, None].float())
        start += n
    return out.to(x.dtype)


def graph_of(fn):
    fn()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fn()
    return g.replay


def fmt(v) -> str:
    return f"{v:.3f}" if isinstance(v, float) else str(v)


def layer_table(flush: torch.Tensor) -> list[str]:
    lines = ["| shape | routing | ours (graph) | ours (eager) | torch._grouped_mm | per-expert loop |",
             "|---|---|---:|---:|---:|---:|"]
    print("\n".join(lines), flush=True)
    for shape_name in ("fine_grained", "mixtral"):
        shape = SHAPES[shape_name]
        for routing in ("random", "zipf_perm"):
            x, idx, gates, w1, w2 = make_layer(shape, routing, 0)
            k = idx.shape[1]
            token = torch.arange(x.shape[0], device=x.device).repeat_interleave(k)
            expert, weight = idx.reshape(-1), gates.reshape(-1)
            ref = reference_fp32(x, token, expert, weight, w1, w2)
            row = [shape_name, routing]
            ours = lambda: moe_forward(x, idx, gates, w1, w2)  # noqa: E731
            t_eager = checked(ours, ref, flush)
            t_graph = time_ms(graph_of(ours), flush) if isinstance(t_eager, float) else "-"
            row += [fmt(t_graph), fmt(t_eager)]
            try:
                row.append(fmt(checked(lambda: grouped_mm_layer(x, token, expert, weight, w1, w2), ref, flush)))
            except RuntimeError as e:
                row.append(f"unavailable ({str(e).splitlines()[0][:60]})")
            row.append(fmt(checked(lambda: loop_layer(x, token, expert, weight, w1, w2), ref, flush)))
            lines.append("| " + " | ".join(row) + " |")
            print(lines[-1], flush=True)
            del x, idx, gates, w1, w2, ref
            torch.cuda.empty_cache()
    return lines


def rounding_table(flush: torch.Tensor) -> list[str]:
    lines = ["| shape | tokens | routing | ours top-k | ours TR | gain | ours TR fused: eager / graph | "
             "grouped_mm top-k | grouped_mm TR | rounding alone (ours): eager / graph |",
             "|---|---:|---|---:|---:|---:|---:|---:|---:|---:|"]
    print("\n".join(lines), flush=True)
    problems = [("fine_grained", 4096), ("fine_grained", 16384), ("mixtral", 4096)]
    for shape_name, num_tokens in problems:
        base = SHAPES[shape_name]
        shape = type(base)(base.name, num_tokens, base.d_model, base.ffn_dim, base.num_experts)
        x, _, _, w1, w2 = make_layer(shape, "random", 0)
        e = shape.num_experts
        for routing in ("uniform", "zipf"):
            scores = router_scores(routing, num_tokens, e).cuda()
            plain = top_k_assignments(scores, 2)
            rounded = token_rounding(scores, 2, 128)
            row = [shape_name, str(num_tokens), routing]
            t = {}
            for label, a in (("topk", plain), ("tr", rounded)):
                ref = reference_fp32(x, a.token, a.expert, a.weight, w1, w2)
                t["ours_" + label] = checked(
                    lambda a=a: moe_forward_assigned(x, a.token, a.expert, a.weight, w1, w2), ref, flush)
                try:
                    t["gmm_" + label] = checked(
                        lambda a=a: grouped_mm_layer(x, a.token, a.expert, a.weight, w1, w2), ref, flush)
                except RuntimeError as err:
                    t["gmm_" + label] = f"unavailable ({str(err).splitlines()[0][:40]})"
                if label == "tr":
                    fused = lambda: moe_forward_rounded(x, scores, 2, w1, w2)  # noqa: E731
                    t["fused"] = checked(fused, ref, flush)
                    t["fused_graph"] = time_ms(graph_of(fused), flush) if isinstance(t["fused"], float) else "-"
                del ref
            rounding = lambda: route_rounded(scores, 2, shape.ffn_dim, 128, 128)  # noqa: E731
            t["rounding"] = time_ms(rounding, flush)
            t["rounding_graph"] = time_ms(graph_of(rounding), flush)
            gain = (f"{t['ours_topk'] / t['ours_tr']:.2f}x"
                    if isinstance(t["ours_topk"], float) and isinstance(t["ours_tr"], float) else "-")
            row += [fmt(t["ours_topk"]), fmt(t["ours_tr"]), gain, f"{fmt(t['fused'])} / {fmt(t['fused_graph'])}",
                    fmt(t["gmm_topk"]), fmt(t["gmm_tr"]), f"{fmt(t['rounding'])} / {fmt(t['rounding_graph'])}"]
            lines.append("| " + " | ".join(row) + " |")
            print(lines[-1], flush=True)
        del x, w1, w2
        torch.cuda.empty_cache()
    return lines


def replay_table(flush: torch.Tensor) -> list[str]:
    lines = ["| T' | seed | replay ms | useful TFLOP/s | eager at T' (ms) | bit-identical to eager |",
             "|---:|---:|---:|---:|---:|---|"]
    print("\n".join(lines), flush=True)
    shape = SHAPES["replay_sweep"]
    t_max = shape.num_tokens
    x, idx, gates, w1, w2 = make_layer(shape, "zipf_perm", 0)
    valid = torch.tensor([t_max], dtype=torch.int32, device="cuda")
    run = lambda: moe_forward(x, idx, gates, w1, w2, valid_tokens=valid)  # noqa: E731
    run()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = run()
    flops_per_token = 2 * 2 * shape.top_k * shape.d_model * shape.ffn_dim
    for seed, t in zip((1, 2, 3, 4), (512, 2048, 8192, 16384)):
        g = torch.Generator(device="cuda").manual_seed(seed)  # fresh x, routing and gates, written in place
        x.copy_(torch.randn(t_max, shape.d_model, generator=g, device="cuda"))
        idx.copy_(routing_case("zipf_perm", t_max, shape.num_experts, seed, shape.top_k))
        gates.copy_(softmax_gates(t_max, shape.top_k, seed + 1, "cuda"))
        valid.fill_(t)
        graph.replay()
        torch.cuda.synchronize()
        eager = lambda t=t: moe_forward(x[:t], idx[:t], gates[:t], w1, w2)  # noqa: E731
        same = torch.equal(out[:t], eager())
        ms = time_ms(graph.replay, flush)
        ms_eager = time_ms(eager, flush)
        lines.append(f"| {t} | {seed} | {ms:.3f} | {flops_per_token * t / ms / 1e9:.0f} | {ms_eager:.3f} | {same} |")
        print(lines[-1], flush=True)
    del x, idx, gates, w1, w2, out
    torch.cuda.empty_cache()
    return lines


def read_probe():
    """sbp_read of libsparsebench_probe.so (a measurement tool built beside the
    library, not part of its C ABI): read a whole tensor once on the device."""
    import ctypes

    from sparsebench_amd import _lib

    probe = ctypes.CDLL(str(_lib.LIB_PATH.with_name("libsparsebench_probe.so")))
    probe.sbp_read.restype = ctypes.c_int
    probe.sbp_read.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_uint32, ctypes.c_void_p,
                               ctypes.c_void_p]
    probe.sbp_last_error.restype = ctypes.c_char_p

    def run(data: torch.Tensor, mode: str, sink: torch.Tensor) -> None:
        rc = probe.sbp_read(data.data_ptr(), data.numel() * data.element_size(), {"vector": 0, "lds_dma": 1}[mode],
                            0x9E3779B9, sink.data_ptr(), _lib.stream_of(data.device))
        if rc != 0:
            raise RuntimeError(probe.sbp_last_error().decode())

    return run


def ceilings_table(flush: torch.Tensor) -> list[str]:
    probe = read_probe()
    lines = ["| measurement | ms | rate | of published peak |", "|---|---:|---:|---:|"]
    print("\n".join(lines), flush=True)
    data = torch.ones(2 << 30, dtype=torch.uint8, device="cuda")
    sink = torch.zeros(256, dtype=torch.int32, device="cuda")
    for mode in ("vector", "lds_dma"):
        ms = time_ms(lambda: probe(data, mode, sink), flush)
        tbs = data.numel() / ms / 1e9
        lines.append(f"| read 2 GiB, {mode} | {ms:.3f} | {tbs:.2f} TB/s | {tbs / 8.0:.0%} |")
        print(lines[-1], flush=True)
    src, dst = data[: 1 << 30], data[1 << 30:]
    ms = time_ms(lambda: dst.copy_(src), flush)
    tbs = 2 * src.numel() / ms / 1e9
    lines.append(f"| copy 1 GiB (read + write) | {ms:.3f} | {tbs:.2f} TB/s | {tbs / 8.0:.0%} |")
    print(lines[-1], flush=True)
    del data, src, dst
    torch.cuda.empty_cache()
    return lines + gemm_table(flush, header=False)


def gemm_table(flush: torch.Tensor, header: bool = True) -> list[str]:
    """Dense bf16 GEMMs of the Mixtral-like stages' total shapes through torch.matmul (hipBLASLt), with the
    weight stored as the layer stores it (N-contiguous, [K, N]) and transposed (K-contiguous, [N, K])."""
    lines = ["| measurement | ms | rate | of published peak |", "|---|---:|---:|---:|"] if header else []
    if header:
        print("\n".join(lines), flush=True)
    for m, n, k in ((8192, 8192, 8192), (8192, 14336, 4096), (8192, 4096, 14336)):
        a = torch.randn(m, k, device="cuda", dtype=torch.bfloat16)
        b = torch.randn(k, n, device="cuda", dtype=torch.bfloat16)
        bt = b.t().contiguous()
        for label, fn in (("weight [K, N]", lambda: a @ b), ("weight [N, K]", lambda: a @ bt.t())):
            ms = time_ms(fn, flush)
            tf = 2 * m * n * k / ms / 1e9
            lines.append(f"| bf16 GEMM {m}x{n}x{k}, {label} (torch.matmul) | {ms:.3f} | {tf:.0f} TFLOP/s | {tf / 2500:.0%} |")
            print(lines[-1], flush=True)
        del a, b, bt
    return lines


def main() -> None:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--only", choices=["layer", "rounding", "replay", "ceilings", "gemm"])
    args = p.parse_args()
    if not torch.cuda.is_available():
        raise SystemExit("bench_baselines.py needs a GPU")
    flush = torch.empty(FLUSH_BYTES, dtype=torch.uint8, device="cuda")
    print(f"GPU: {torch.cuda.get_device_name()}, torch {torch.__version__}; times in ms, median of 20\n", flush=True)
    if args.only in (None, "layer"):
        print("## Whole layer, top-2 (T=4096)\n", flush=True)
        layer_table(flush)
        print(flush=True)
    if args.only in (None, "rounding"):
        print("## Token rounding (tile 128, top-2)\n", flush=True)
        rounding_table(flush)
        print(flush=True)
    if args.only in (None, "replay"):
        print("## Graph replay sweep (config 5: captured at T=16384)\n", flush=True)
        replay_table(flush)
        print(flush=True)
    if args.only in (None, "ceilings"):
        print("## Ceilings of this box\n", flush=True)
        ceilings_table(flush)
    if args.only == "gemm":
        print("## Dense GEMMs (hipBLASLt)\n", flush=True)
        gemm_table(flush)


if __name__ == "__main__":
    main()
