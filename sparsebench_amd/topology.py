"""The trimmed block-sparse layout (the Topology type of the reference's
sparsebench/topology.py:30-55).

Copies (t, j) -> c = t*k + j are sorted by expert, each expert's group padded
to a multiple of block_size. That gives P padded rows in row blocks of one
expert each; row block r owns BSR blocks row_offsets[r] .. row_offsets[r+1],
col_indices naming the column block (expert*ffn_blocks + j) of each.
The GPU builds it in sparsebench_amd.routing.
"""

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class Topology:
    block_size: int
    num_experts: int
    ffn_blocks: int  # F // block_size: column blocks per expert

    tokens_per_expert: torch.Tensor  # [E] int32, real copies per expert
    padded_offsets: torch.Tensor  # [E+1] int32, first padded row of each expert
    row_token: torch.Tensor  # [P] int32, source token of each row, -1 = padding
    copy_row: torch.Tensor  # [T*k] int32, padded row of copy (t, j) at t*k + j

    row_block_expert: torch.Tensor  # [P / block_size] int32
    row_offsets: torch.Tensor  # [P / block_size + 1] int32
    col_indices: torch.Tensor  # [nnz_blocks] int32

    @property
    def num_rows(self) -> int:
        return self.row_token.numel()

    @property
    def num_row_blocks(self) -> int:
        return self.row_block_expert.numel()

    @property
    def nnz_blocks(self) -> int:
        return self.col_indices.numel()
