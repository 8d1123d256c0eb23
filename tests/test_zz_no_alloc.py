"""sb_routing_noalloc (routing with its scratch in a fixed device array)
against sb_routing (routing with a caller-owned workspace), through the C ABI.

Two calls in a row, the second on a smaller input, so the second call runs
on scratch the first one left behind. Every output must be bit-identical to
sb_routing's (integer layout work: the bar is exact), and sizes beyond the
fixed array are rejected before anything is enqueued. Up to 32768 copies
(32 chunks of 1024) the place kernel reads the per-chunk counts straight
from scratch; beyond, the offsets kernel scans them there in place first.
The sizes here are on both sides of that bound, each call smaller than the
one before.
"""

import ctypes

import pytest
import torch

from sparsebench_amd import _C
from sparsebench_amd._lib import lib, stream_of
from sparsebench_amd.workloads import routing_case

pytestmark = pytest.mark.gpu

SCRATCH_ELEMS = 1 << 19


def routing_outputs(num_copies: int, num_experts: int, ffn_dim: int, block_size: int, device) -> list[torch.Tensor]:
    max_rb, max_rows, _ = _C.routing_sizes(num_copies, num_experts, ffn_dim, block_size)
    opts = {"dtype": torch.int32, "device": device}
    # Filled with a sentinel so an output the kernels leave unwritten shows.
    return [torch.full((n,), -7, **opts) for n in (num_experts, num_experts + 1, max_rows, num_copies, max_rb,
                                                   max_rb + 1, max_rb * (ffn_dim // block_size), 1)]


def run_noalloc(idx: torch.Tensor, num_experts: int, ffn_dim: int, block_size: int, valid=None) -> list[torch.Tensor]:
    t, k = idx.shape
    outs = routing_outputs(t * k, num_experts, ffn_dim, block_size, idx.device)
    rc = lib().sb_routing_noalloc(idx.data_ptr(), 1 if idx.dtype == torch.int64 else 0, t, k, num_experts, ffn_dim,
                                  block_size, None if valid is None else valid.data_ptr(),
                                  *(o.data_ptr() for o in outs), stream_of(idx.device))
    assert rc == 0, lib().sb_last_error().decode()
    return outs


def run_with_workspace(idx: torch.Tensor, num_experts: int, ffn_dim: int, block_size: int,
                       valid=None) -> list[torch.Tensor]:
    t, k = idx.shape
    outs = routing_outputs(t * k, num_experts, ffn_dim, block_size, idx.device)
    _, _, ws = _C.routing_sizes(t * k, num_experts, ffn_dim, block_size)
    workspace = torch.empty(ws, dtype=torch.int32, device=idx.device)
    rc = lib().sb_routing(idx.data_ptr(), 1 if idx.dtype == torch.int64 else 0, t, k, num_experts, ffn_dim,
                          block_size, None if valid is None else valid.data_ptr(), workspace.data_ptr(),
                          *(o.data_ptr() for o in outs), stream_of(idx.device))
    assert rc == 0, lib().sb_last_error().decode()
    return outs


def assert_same(a: list[torch.Tensor], b: list[torch.Tensor]) -> None:
    torch.cuda.synchronize()
    names = ["tokens_per_expert", "padded_offsets", "row_token", "copy_row", "row_block_expert", "row_offsets",
             "col_indices", "error"]
    for name, x, y in zip(names, a, b):
        assert torch.equal(x, y), name


@pytest.mark.parametrize(("case", "num_experts", "block_size"), [("zipf", 64, 128), ("random", 1000, 16),
                                                                  ("empty_middle", 8, 4)])
def test_noalloc_matches_workspace_routing_twice(case: str, num_experts: int, block_size: int) -> None:
    ffn_dim = 4 * block_size
    big = routing_case(case, 20000, num_experts, seed=1).cuda()  # 40000 copies: 40 chunks
    small = routing_case(case, 17000, num_experts, seed=2).int().cuda()  # 34 chunks, over stale scratch
    tiny = routing_case(case, 777, num_experts, seed=3).cuda()  # 2 chunks, counts scanned by the place kernel
    for idx in (big, small, tiny):  # each call smaller: stale scratch from the one before must not leak in
        assert_same(run_noalloc(idx, num_experts, ffn_dim, block_size),
                    run_with_workspace(idx, num_experts, ffn_dim, block_size))


@pytest.mark.parametrize("num_tokens", [3000, 20000])
def test_noalloc_bad_ids_and_valid_tokens(num_tokens: int) -> None:
    idx = routing_case("random", num_tokens, 32, seed=3).cuda()
    idx[5, 1] = 32
    idx[17, 0] = -1
    valid = torch.tensor([2500], dtype=torch.int32, device="cuda")
    for v in (None, valid):
        assert_same(run_noalloc(idx, 32, 256, 128, v), run_with_workspace(idx, 32, 256, 128, v))


def test_noalloc_rejects_more_scratch_than_the_array() -> None:
    # ceil(T*k / 1024) * (E + 1) int32 of scratch: 1024 experts need over 512 chunks' worth.
    t, k, e = 300_000, 2, 1024
    _, _, ws = _C.routing_sizes(t * k, e, 256, 128)
    assert ws > SCRATCH_ELEMS
    idx = torch.zeros(t, k, dtype=torch.int32, device="cuda")
    outs = routing_outputs(t * k, e, 256, 128, idx.device)
    rc = lib().sb_routing_noalloc(idx.data_ptr(), 0, t, k, e, 256, 128, None, *(o.data_ptr() for o in outs),
                                  stream_of(idx.device))
    assert rc == 1
    assert "scratch" in lib().sb_last_error().decode()
    torch.cuda.synchronize()
    assert int(outs[0][0]) == -7  # nothing ran


@pytest.mark.parametrize("num_tokens", [4096, 17000])
def test_noalloc_under_graph_capture(num_tokens: int) -> None:
    # Captured after a first eager call on the device; every replay, with fresh
    # routing written in place between them, equals the workspace routing.
    idx = routing_case("zipf", num_tokens, 64, seed=4).cuda()
    run_noalloc(idx, 64, 512, 128)
    torch.cuda.synchronize()
    t, k = idx.shape
    outs = routing_outputs(t * k, 64, 512, 128, idx.device)
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        rc = lib().sb_routing_noalloc(idx.data_ptr(), 1, t, k, 64, 512, 128, None, *(o.data_ptr() for o in outs),
                                      ctypes.c_void_p(side.cuda_stream))
    assert rc == 0
    for seed in (5, 6, 7):
        idx.copy_(routing_case("zipf", num_tokens, 64, seed=seed).cuda())
        graph.replay()
        torch.cuda.synchronize()
        assert_same(outs, run_with_workspace(idx, 64, 512, 128))
