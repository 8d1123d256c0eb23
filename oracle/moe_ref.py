"""Floating-point references of the MoE layer and its stages (torch, CPU).
TEST INFRASTRUCTURE ONLY.

Expert e computes y = gelu(x @ w1[e]) @ w2[e] with the exact erf GELU
(F.gelu's default, as in the reference's sparsebench/reference.py:59 and
csrc/sdd.cu:41). Each token sums its k experts' outputs weighted by its gates.

    moe_reference            loop over experts (reference.py:49-61)
    moe_assigned_reference   the same for a routing given as a list (moe.py:59-91)
    per_token_reference      one token at a time (tests/test_reference.py:18-27)
    moe_blocksparse_reference through the layout: group, SDD, GELU, DSD,
                             combine (reference.py:64-114)
    sdd_blocks / dsd_rows    one stage each, from the definition
    combine_reference        moe.py:51-54: fp32 products, summed over k

Pins: per-token == loop (fp64), block-sparse == loop at 1e-10 (fp64), GELU
against math.erf, DSD block-wise == DSD through the dense matrix.
"""

from __future__ import annotations

import math

import numpy as np
import torch

from oracle.topology_ref import Layout, build_layout, row_block_of_nnz


def gelu_erf(v: torch.Tensor) -> torch.Tensor:
    """0.5 v (1 + erf(v / sqrt 2))."""
    return 0.5 * v * (1.0 + torch.erf(v * (1.0 / math.sqrt(2.0))))


def route(logits: torch.Tensor, k: int = 2) -> tuple[torch.Tensor, torch.Tensor]:
    """Top-k router, softmax over the k picked logits only (reference.py:19-29)."""
    if logits.dim() != 2 or not 0 < k <= logits.shape[1]:
        raise ValueError(f"need [T, E] logits with 0 < k <= E, got {tuple(logits.shape)} and k={k}")
    top, idx = torch.topk(logits, k, dim=-1)
    return idx, torch.softmax(top.float(), dim=-1).to(logits.dtype)


def check_shapes(x, expert_idx, expert_weight, w1, w2) -> None:
    """The shape checks of reference.py:32-46 (ValueError)."""
    if x.dim() != 2:
        raise ValueError(f"x must be [T, D], got {tuple(x.shape)}")
    num_tokens, d_model = x.shape
    if w1.dim() != 3 or w1.shape[1] != d_model:
        raise ValueError(f"w1 must be [E, {d_model}, F], got {tuple(w1.shape)}")
    num_experts, _, ffn_dim = w1.shape
    if w2.shape != (num_experts, ffn_dim, d_model):
        raise ValueError(f"w2 must be {(num_experts, ffn_dim, d_model)}, got {tuple(w2.shape)}")
    if expert_idx.dim() != 2 or expert_idx.shape[0] != num_tokens:
        raise ValueError(f"expert_idx must be [{num_tokens}, k], got {tuple(expert_idx.shape)}")
    if expert_weight.shape != expert_idx.shape:
        raise ValueError(f"expert_weight must match expert_idx shape {tuple(expert_idx.shape)}")


def moe_reference(x, expert_idx, expert_weight, w1, w2) -> torch.Tensor:
    """[T, D]: for each expert, its tokens through the MLP, added with their gate."""
    check_shapes(x, expert_idx, expert_weight, w1, w2)
    out = torch.zeros_like(x)
    for e in range(w1.shape[0]):
        token, slot = torch.nonzero(expert_idx == e, as_tuple=True)
        if token.numel():
            y = gelu_erf(x[token] @ w1[e]) @ w2[e]
            out.index_add_(0, token, y * expert_weight[token, slot, None])
    return out


def moe_assigned_reference(x, token, expert, weight, w1, w2) -> torch.Tensor:
    """[T, D] fp32 for a routing given as a list: copy c sends token[c] to
    expert[c] with weight[c]; tokens with no copy give 0 (the layer of
    sparsebench/moe.py:59-91, as the reference's tests/test_token_rounding.py:
    91-99 computes it). fp32 math on the given values, one expert at a time."""
    x, w1, w2 = x.float().cpu(), w1.float().cpu(), w2.float().cpu()
    token, expert = torch.as_tensor(token).long().cpu(), torch.as_tensor(expert).long().cpu()
    weight = torch.as_tensor(weight).float().cpu()
    out = torch.zeros(x.shape[0], x.shape[1])
    for e in range(w1.shape[0]):
        m = expert == e
        if m.any():
            y = gelu_erf(x[token[m]] @ w1[e]) @ w2[e]
            out.index_add_(0, token[m], y * weight[m, None])
    return out


def per_token_reference(x, expert_idx, expert_weight, w1, w2) -> torch.Tensor:
    """Token by token, choice by choice: no grouping at all."""
    out = torch.zeros_like(x)
    for t in range(x.shape[0]):
        for j in range(expert_idx.shape[1]):
            e = int(expert_idx[t, j])
            out[t] += expert_weight[t, j] * (gelu_erf(x[t] @ w1[e]) @ w2[e])
    return out


def group_tokens(x: torch.Tensor, row_token: np.ndarray) -> torch.Tensor:
    """[T, D] -> [P, D] in layout row order; padding rows (row_token < 0) are zero."""
    rt = torch.as_tensor(np.asarray(row_token), dtype=torch.long)
    xg = x[rt.clamp(min=0)]
    xg[rt < 0] = 0
    return xg


def bsr_to_dense(blocks: torch.Tensor, layout: Layout) -> torch.Tensor:
    """[nnz, bs, bs] -> dense [num_row_blocks*bs, E*F], zeros off the layout."""
    bs = layout.block_size
    nrb = layout.row_offsets.size - 1
    ncb = layout.num_experts * layout.ffn_blocks
    grid = blocks.new_zeros(nrb, ncb, bs, bs)
    rows = torch.as_tensor(row_block_of_nnz(layout), dtype=torch.long)
    cols = torch.as_tensor(layout.col_indices[: rows.numel()].astype(np.int64))
    grid[rows, cols] = blocks[: rows.numel()]
    return grid.permute(0, 2, 1, 3).reshape(nrb * bs, ncb * bs)


def dense_to_bsr(dense: torch.Tensor, layout: Layout) -> torch.Tensor:
    """Dense [num_row_blocks*bs, E*F] -> [nnz, bs, bs]; values off the layout dropped."""
    bs = layout.block_size
    nrb = layout.row_offsets.size - 1
    ncb = layout.num_experts * layout.ffn_blocks
    grid = dense.reshape(nrb, bs, ncb, bs).permute(0, 2, 1, 3)
    rows = torch.as_tensor(row_block_of_nnz(layout), dtype=torch.long)
    cols = torch.as_tensor(layout.col_indices[: rows.numel()].astype(np.int64))
    return grid[rows, cols].contiguous()


def sdd_blocks(x: torch.Tensor, w1: torch.Tensor, layout: Layout, gelu: bool = True) -> torch.Tensor:
    """[nnz, 128, 128]: block j of row block r = (gelu)(rows of r @ w1[e][:, j*bs:(j+1)*bs])."""
    bs = layout.block_size
    xg = group_tokens(x, layout.row_token[: layout.num_rows])
    out = []
    for r in range(layout.num_row_blocks):
        e = int(layout.row_block_expert[r])
        h = xg[r * bs:(r + 1) * bs] @ w1[e]
        if gelu:
            h = gelu_erf(h)
        out.append(h.reshape(bs, layout.ffn_blocks, bs).permute(1, 0, 2))
    if not out:
        return x.new_zeros(0, bs, bs)
    return torch.cat(out).contiguous()


def dsd_rows(blocks: torch.Tensor, w: torch.Tensor, layout: Layout) -> torch.Tensor:
    """[num_row_blocks*bs, D] = BSR @ w, block by block (any BSR layout)."""
    bs = layout.block_size
    nrb = layout.row_offsets.size - 1
    nnz = int(layout.row_offsets[-1])
    cols = torch.as_tensor(layout.col_indices[:nnz].astype(np.int64))
    w_blocks = w.view(-1, bs, w.shape[1])[cols]
    products = torch.bmm(blocks[:nnz], w_blocks)
    out = torch.zeros(nrb, bs, w.shape[1], dtype=products.dtype)
    out.index_add_(0, torch.as_tensor(row_block_of_nnz(layout), dtype=torch.long), products)
    return out.view(-1, w.shape[1])


def combine_reference(y_rows: torch.Tensor, copy_row: np.ndarray, expert_weight: torch.Tensor) -> torch.Tensor:
    """[T, D] fp32: sum_j fp32(y[copy_row[t*k+j]]) * fp32(w[t, j]); skipped copies (-1) add nothing."""
    num_tokens, k = expert_weight.shape
    cr = torch.as_tensor(np.asarray(copy_row), dtype=torch.long)
    rows = y_rows.float()[cr.clamp(min=0)] * (cr >= 0)[:, None]
    return (rows.view(num_tokens, k, -1) * expert_weight.float()[..., None]).sum(dim=1)


def moe_blocksparse_reference(x, expert_idx, expert_weight, w1, w2, block_size: int) -> torch.Tensor:
    """moe_reference computed through the block-sparse layout."""
    check_shapes(x, expert_idx, expert_weight, w1, w2)
    num_experts, d_model, ffn_dim = w1.shape
    layout = build_layout(expert_idx.numpy(), num_experts, ffn_dim, block_size)
    w1_cat = w1.permute(1, 0, 2).reshape(d_model, num_experts * ffn_dim)
    w2_cat = w2.reshape(num_experts * ffn_dim, d_model)
    h = dense_to_bsr(group_tokens(x, layout.row_token) @ w1_cat, layout)
    y = bsr_to_dense(gelu_erf(h), layout) @ w2_cat
    num_tokens, k = expert_weight.shape
    rows = y[torch.as_tensor(layout.copy_row.astype(np.int64))].view(num_tokens, k, -1)
    return (rows * expert_weight[..., None]).sum(dim=1)


def layer_reference_fp32(x, expert_idx, expert_weight, w1, w2) -> torch.Tensor:
    """fp32 ground truth for a bf16 layer: fp32 math on the same bf16 values, one expert at a time."""
    return moe_reference(x.float().cpu(), expert_idx.cpu(), expert_weight.float().cpu(), w1.float().cpu(),
                         w2.float().cpu())


def max_rel_err(out: torch.Tensor, ref: torch.Tensor) -> float:
    """max |out - ref| / max |ref| (the layer's 2e-2 gate)."""
    ref = ref.float().cpu()
    return float((out.float().cpu() - ref).abs().max() / ref.abs().max().clamp(min=1e-30))


__all__ = [
    "bsr_to_dense", "check_shapes", "combine_reference", "dense_to_bsr", "dsd_rows", "gelu_erf",
    "group_tokens", "layer_reference_fp32", "max_rel_err", "moe_blocksparse_reference", "moe_reference",
    "per_token_reference", "route", "sdd_blocks",
]
