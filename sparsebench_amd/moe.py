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

from sparsebench_amd.routing import AssignedRouting, route_assigned, route_device, route_rounded
from sparsebench_amd.spmm import dsd, sdd

BLOCK_SIZE = 128
STAGES = ("routing", "SDD + GELU (fused)", "DSD", "combine")

# The stage kernels the layer runs; every choice gives the same output bits.
#   expert_tiles   SDD / DSD on the layer kernels (sdd_experts_cuda /
#                  dsd_experts_cuda), else the per-row-block sdd / dsd.
_STAGE_OPTIONS = {"expert_tiles": True}


def set_stage_options(**options: bool) -> dict[str, bool]:
    """Sets the layer's stage choices (keys of _STAGE_OPTIONS) for this
    process and returns the previous values. For tests and measurements:
    outputs do not depend on them."""
    unknown = set(options) - set(_STAGE_OPTIONS)
    if unknown:
        raise ValueError(f"unknown stage options {sorted(unknown)}")
    previous = dict(_STAGE_OPTIONS)
    _STAGE_OPTIONS.update({k: bool(v) for k, v in options.items()})
    return previous


def _no_mark(stage: str) -> None:
    pass


def _expert_tiles(topo, d_model: int, ffn_dim: int) -> bool:
    """SDD / DSD on the layer kernels (the default), unless switched off or
    the shape needs the per-row-block kernels."""
    from sparsebench_amd import _C

    if not _STAGE_OPTIONS["expert_tiles"]:
        return False
    return _C.expert_tiles_fit(d_model, ffn_dim, topo.row_token.numel() // topo.block_size)


def _sdd_dsd(x, w1, w2, topo, mark):
    """H = gelu(x grouped @ w1), then y = H @ w2 on topo's rows; marks both stages."""
    from sparsebench_amd import _C

    num_experts, d_model, ffn_dim = w1.shape
    w2_cat = w2.view(num_experts * ffn_dim, d_model)
    if _expert_tiles(topo, d_model, ffn_dim):
        h = _C.sdd_experts_cuda(x, w1, topo, True)
        mark("SDD + GELU (fused)")
        y = _C.dsd_experts_cuda(h, w2_cat, topo)
    else:
        h = sdd(x, w1, topo, gelu=True)
        mark("SDD + GELU (fused)")
        y = dsd(h, w2_cat, topo, version=5)
    mark("DSD")
    return h, y


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
    _, y = _sdd_dsd(x, w1, w2, topo, mark)
    out = combine(y, topo.copy_row, expert_weight, valid_tokens)
    mark("combine")
    return out


def _assigned_layer(x, routing: AssignedRouting, weight_of_copy, w1, w2, mark, valid_tokens) -> torch.Tensor:
    from sparsebench_amd import _C

    mark("routing")
    _, y = _sdd_dsd(x, w1, w2, routing.topology, mark)
    out = _C.combine_assigned_cuda(y, routing.topology.copy_row, weight_of_copy, routing.token_offsets,
                                   routing.token_copies, x.shape[0], valid_tokens)
    mark("combine")
    return out


def moe_forward_assigned(
    x: torch.Tensor,
    token_of_copy: torch.Tensor,
    expert_of_copy: torch.Tensor,
    weight_of_copy: torch.Tensor,
    w1: torch.Tensor,
    w2: torch.Tensor,
    mark: Callable[[str], None] = _no_mark,
    valid_tokens: torch.Tensor | None = None,
) -> torch.Tensor:
    """The same layer for any routing given as a flat list (the reference's
    sparsebench/moe.py:59-91): copy c sends token_of_copy[c] to
    expert_of_copy[c] with weight weight_of_copy[c]. A token may have any
    number of copies, including none (its output row is 0), e.g. after token
    rounding. No host sync.

    The routing is moe_forward's with k = 1 and token ids from the list. The
    combine sums each token's copies in list order with fp32 accumulation,
    as the reference's index_add_ does on the CPU (on the GPU its order is not
    fixed), so the same list always gives the same bits, and a top-k list
    gives exactly moe_forward's result. A token id outside [0, T) is skipped
    and flagged in the routing's error word.
    """
    num_experts, d_model, ffn_dim = w1.shape
    if w2.shape != (num_experts, ffn_dim, d_model):
        raise ValueError(f"w2 must be {(num_experts, ffn_dim, d_model)}, got {tuple(w2.shape)}")
    if x.dim() != 2 or x.shape[1] != d_model:
        raise ValueError(f"x must be [T, {d_model}], got {tuple(x.shape)}")
    n = expert_of_copy.numel()
    if token_of_copy.numel() != n or weight_of_copy.numel() != n:
        raise ValueError("token_of_copy, expert_of_copy and weight_of_copy must have one entry per copy")
    if n == 0:  # host-known size: nothing routed anywhere
        return torch.zeros_like(x)
    routing = route_assigned(token_of_copy.reshape(-1), expert_of_copy.reshape(-1), x.shape[0], num_experts,
                             ffn_dim, BLOCK_SIZE, valid_tokens)
    return _assigned_layer(x, routing, weight_of_copy.reshape(-1), w1, w2, mark, valid_tokens)


def moe_forward_rounded(
    x: torch.Tensor,
    scores: torch.Tensor,
    k: int,
    w1: torch.Tensor,
    w2: torch.Tensor,
    tile: int = BLOCK_SIZE,
    mark: Callable[[str], None] = _no_mark,
) -> torch.Tensor:
    """The layer with token rounding fused into routing, no host sync:
    moe_forward_assigned(x, *token_rounding(scores, k, tile), w1, w2) without
    the sync token_rounding needs for its length. scores [T, E] fp32 router
    probabilities. Bit-identical to that two-step form."""
    num_experts, d_model, ffn_dim = w1.shape
    if w2.shape != (num_experts, ffn_dim, d_model):
        raise ValueError(f"w2 must be {(num_experts, ffn_dim, d_model)}, got {tuple(w2.shape)}")
    if x.dim() != 2 or x.shape[1] != d_model or scores.shape != (x.shape[0], num_experts):
        raise ValueError(f"x must be [T, {d_model}] and scores [T, {num_experts}]")
    routing = route_rounded(scores, k, ffn_dim, BLOCK_SIZE, tile)
    return _assigned_layer(x, routing, routing.weight_of_copy, w1, w2, mark, None)
