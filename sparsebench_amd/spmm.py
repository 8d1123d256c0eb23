"""Block-sparse matmuls (the reference's sparsebench/spmm.py:9-43)."""

from __future__ import annotations

import torch

from sparsebench_amd.routing import DeviceTopology
from sparsebench_amd.topology import Topology


def dsd(
    blocks: torch.Tensor, w2_cat: torch.Tensor, topo: Topology | DeviceTopology, version: int = 1
) -> torch.Tensor:
    """out = H @ w2_cat, with H block-sparse in topo's layout.

    blocks [nnz, bs, bs] bf16, w2_cat [E*F, D] bf16 -> [num_row_blocks*bs, D] bf16.
    With a DeviceTopology everything is worst-case sized and nothing syncs.
    Rows of dead row blocks are zeros for versions 1-3 and left unwritten
    from version 4 on (the reference's contract; one kernel serves all codes).
    """
    from sparsebench_amd import _C

    bs = topo.block_size
    if blocks.dim() != 3 or blocks.shape[1:] != (bs, bs):
        raise ValueError(f"blocks must be [nnz, {bs}, {bs}] for this topology, got {tuple(blocks.shape)}")
    return _C.dsd_cuda(blocks, w2_cat, topo.row_offsets, topo.col_indices, version)


def sdd(x: torch.Tensor, w1: torch.Tensor, topo: Topology | DeviceTopology, gelu: bool = True) -> torch.Tensor:
    """H = (gelu)(x grouped by topo @ w1[expert]), on topo's blocks only.

    x [T, D] bf16, w1 [E, D, F] bf16 -> blocks [nnz, 128, 128] bf16 in topo's
    BSR order. Rows are gathered from x inside the kernel; blocks of dead row
    blocks are left unwritten. Needs block size 128, D % 64 == 0, F % 256 == 0.
    """
    from sparsebench_amd import _C

    if topo.block_size != 128:
        raise ValueError(f"sdd needs block size 128, got {topo.block_size}")
    return _C.sdd_cuda(
        x, w1, topo.row_token, topo.row_block_expert, topo.row_offsets, topo.col_indices.numel(), gelu
    )
