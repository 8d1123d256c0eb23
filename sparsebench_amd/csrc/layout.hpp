// The BSR side of a routing layout, written from padded_offsets and
// tokens_per_expert alone (shared by top-k routing and token rounding).
//
// Item i (one lane each, i over max(max_row_blocks * ffn_blocks + 1,
// max_rows)) writes
//   row_offsets[i]       = min(i, num_row_blocks) * ffn_blocks   (i <= max_rb)
//   col_indices[i]       = expert(r) * ffn_blocks + j, or -1 past the end
//   row_block_expert[r]  (at j == 0), -1 past the end
//   row_token[i]         = -1 for every row that holds no copy
// with r = i / ffn_blocks, j = i % ffn_blocks: the conventions of the
// reference's csrc/routing.cu:162-193, 248-249. Rows that hold a copy are
// written by the caller's own placement.
#pragma once

#include "common.hpp"

namespace sb {

constexpr int kMaxExperts = 1024;

// Last expert whose row range starts at or before `row` (offs in LDS):
// empty experts share a start with the next one, and "last" steps over them.
__device__ __forceinline__ int32_t expert_of_row(const int32_t* offs, int32_t num_experts, int32_t row) {
  int32_t lo = 0, hi = num_experts - 1;
  while (lo < hi) {
    const int32_t mid = (lo + hi + 1) >> 1;
    if (offs[mid] <= row) lo = mid;
    else hi = mid - 1;
  }
  return lo;
}

// offs[E+1] = padded_offsets, cnts[E] = tokens_per_expert, both in LDS.
__device__ __forceinline__ void layout_item(int64_t i, const int32_t* offs, const int32_t* cnts, int32_t num_experts,
                                            int32_t block_size, int32_t ffn_blocks, int32_t max_row_blocks,
                                            int64_t max_rows, int32_t* __restrict__ row_token,
                                            int32_t* __restrict__ row_block_expert,
                                            int32_t* __restrict__ row_offsets, int32_t* __restrict__ col_indices) {
  const int32_t num_rows = offs[num_experts];
  const int32_t num_row_blocks = num_rows / block_size;
  const int64_t bsr_items = static_cast<int64_t>(max_row_blocks) * ffn_blocks;
  if (i <= max_row_blocks) {
    const int32_t r = static_cast<int32_t>(i);
    row_offsets[r] = (r < num_row_blocks ? r : num_row_blocks) * ffn_blocks;
  }
  if (i < bsr_items) {
    const int32_t r = static_cast<int32_t>(i / ffn_blocks);
    const int32_t j = static_cast<int32_t>(i % ffn_blocks);
    const int32_t expert = r < num_row_blocks ? expert_of_row(offs, num_experts, r * block_size) : -1;
    col_indices[i] = expert < 0 ? -1 : expert * ffn_blocks + j;
    if (j == 0) row_block_expert[r] = expert;
  }
  if (i < max_rows) {
    const int32_t row = static_cast<int32_t>(i);
    bool copy_here = false;
    if (row < num_rows) {
      const int32_t e = expert_of_row(offs, num_experts, row);
      copy_here = row - offs[e] < cnts[e];
    }
    if (!copy_here) row_token[row] = -1;
  }
}

}  // namespace sb
