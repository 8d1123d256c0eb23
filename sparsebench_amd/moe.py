"""A full MoE layer forward on the gfx950 kernels, with no host sync
(the reference's sparsebench/moe.py:25-56).

    routing -> SDD + GELU -> DSD -> combine

Every buffer is sized for the worst case on the host, so the CPU never waits
for the GPU to learn how many rows routing produced: the kernels read the
real size from padded_offsets / row_offsets on the GPU.
"""

from __future__ import annotations

from collections.abc import Callable

import torch

from sparsebench_amd.routing import route_device
from sparsebench_amd.spmm import dsd, sdd

BLOCK_SIZE = 128
STAGES = ("routing", "SDD + GELU (fused)", "DSD", "combine")


def _no_mark(stage: str) -> None:
    pass


def combine(
    y: torch.Tensor, copy_row: torch.Tensor, expert_weight: torch.Tensor, valid_tokens: torch.Tensor | None = None
) -> torch.Tensor:
    """out[t] = sum_j y[copy_row[t*k + j]] * expert_weight[t, j], fp32 sum, bf16 out. One kernel."""
    from sparsebench_amd import _C

    return _C.combine_cuda(y, copy_row, expert_weight, valid_tokens)


def moe_forward(
    x: torch.Tensor,
    expert_idx: torch.Tensor,
    expert_weight: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    mark: Callable[[str], None] = _no_mark,
    valid_tokens: torch.Tensor | None = None,
) -> torch.Tensor:
    """x [T, D], expert_idx / expert_weight [T, k], w1 [E, D, F], w2 [E, F, D] -> [T, D].

    bf16 weights and activations, fp32 accumulation inside the kernels.
    mark(stage) is called right after each stage is launched (for per-stage
    timing with events). valid_tokens (optional int32 CUDA scalar T' <= T)
    restricts the layer to the first T' tokens without changing any shape,
    so a graph captured at T replays at any T' <= T; rows >= T' of the
    result are left unwritten.
    """
    num_experts, d_model, ffn_dim = w1.shape
    if w2.shape != (num_experts, ffn_dim, d_model):
        raise ValueError(f"w2 must be {(num_experts, ffn_dim, d_model)}, got {tuple(w2.shape)}")
    if x.shape[1] != d_model or expert_idx.shape != expert_weight.shape or expert_idx.shape[0] != x.shape[0]:
        raise ValueError("x must be [T, D] and expert_idx / expert_weight [T, k]")

    topo = route_device(expert_idx, num_experts, ffn_dim, BLOCK_SIZE, valid_tokens)
    mark("routing")
    h = sdd(x, w1, topo, gelu=True)
    mark("SDD + GELU (fused)")
    y = dsd(h, w2.view(num_experts * ffn_dim, d_model), topo, version=5)
    mark("DSD")
    out = combine(y, topo.copy_row, expert_weight, valid_tokens)
    mark("combine")
    return out
