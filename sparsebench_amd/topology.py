"""The trimmed block-sparse layout (the Topology type of the reference's
sparsebench/topology.py:25-50).

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
    ffn_blocks: int  # block columns of one expert's FFN (F / block_size)

    # All int32. E experts, T*k copies, P padded rows.
    tokens_per_expert: torch.Tensor  # [E]: copies routed to each expert
    padded_offsets: torch.Tensor  # [E+1]: expert e's rows start at [e]; [E] = P
    row_token: torch.Tensor  # [P]: token each row reads; padding rows hold -1
    copy_row: torch.Tensor  # [T*k]: row that copy c = t*k + j landed in

    row_block_expert: torch.Tensor  # [P / block_size]: owning expert per row block
    row_offsets: torch.Tensor  # [P / block_size + 1]: BSR row pointers
    col_indices: torch.Tensor  # [nnz]: block column of each stored block

    @property
    def num_rows(self) -> int:
        return self.row_token.numel()

    @property
    def num_row_blocks(self) -> int:
        return self.row_block_expert.numel()

    @property
    def nnz_blocks(self) -> int:
        return self.col_indices.numel()
