// One DSD tile of a row block on the LDS-DMA main loop (gemm_dma.hpp), the
// tile of the per-row-block kernels (dsd.hip).
#pragma once

#include "gemm_dma.hpp"

namespace sb {

// The same tile on the LDS-DMA mainloop (gemm_dma.hpp). A block of w that
// does not exist (bad column index) gets a zero-length buffer: its loads
// return zeros and it contributes nothing.
template <class Cfg>
struct DsdDmaSrc {
  static constexpr int kStepsPerBlock = Cfg::BM / Cfg::BK;
  // A row block's reduction is whole blocks (reduction_fits for any count).
  static_assert(!Cfg::APAIR || kStepsPerBlock % 2 == 0, "paired A needs an even step count per block");
  const uint16_t* blocks;
  const uint16_t* w;
  const int32_t* col_indices;
  int64_t w_rows;
  int32_t d_model, begin;
  uint32_t a_off[Cfg::kAInstr];
  uint32_t b_off[Cfg::kBInstr];
  __device__ __forceinline__ uint32_t a_voff(int q) const { return a_off[q]; }
  __device__ __forceinline__ uint32_t b_voff(int q) const { return b_off[q]; }
  __device__ __forceinline__ void a_src(int t, __amdgpu_buffer_rsrc_t* r, uint32_t* s) const {
    const int32_t p = begin + t / kStepsPerBlock;
    *r = make_rsrc(blocks + static_cast<int64_t>(p) * Cfg::BM * Cfg::BM, Cfg::BM * Cfg::BM * 2);
    *s = static_cast<uint32_t>(t % kStepsPerBlock) * (Cfg::BK * 2);
  }
  __device__ __forceinline__ void b_src(int t, __amdgpu_buffer_rsrc_t* r, uint32_t* s) const {
    const int32_t p = begin + t / kStepsPerBlock;
    const int64_t row0 = static_cast<int64_t>(col_indices[p]) * Cfg::BM;
    const bool ok = row0 >= 0 && row0 + Cfg::BM <= w_rows;
    *r = make_rsrc(w + (ok ? row0 : 0) * d_model, ok ? static_cast<uint32_t>(Cfg::BM) * d_model * 2u : 0u);
    *s = static_cast<uint32_t>(t % kStepsPerBlock) * (Cfg::BK * 2u) * static_cast<uint32_t>(d_model);
  }
};

// Tile `tile_id` of the row-block grid: bs x BN outputs of one row block,
// its blocks walked in K steps through col_indices. Ids past the grid's
// num_row_blocks * num_slices tiles do nothing.
template <class Cfg>
__device__ __forceinline__ void dsd_row_block_tile(uint8_t* __restrict__ lds, int tile_id,
                                                   const uint16_t* __restrict__ blocks,
                                                   const uint16_t* __restrict__ w,
                                                   const int32_t* __restrict__ row_offsets,
                                                   const int32_t* __restrict__ col_indices, uint16_t* __restrict__ out,
                                                   int64_t nnz, int64_t w_rows, int32_t num_row_blocks,
                                                   int32_t d_model, int32_t num_slices, int32_t zero_dead_rows,
                                                   int32_t group) {
  using ML = DmaMainloop<Cfg>;
  constexpr int BM = Cfg::BM, BN = Cfg::BN;
  if (tile_id >= num_row_blocks * num_slices) return;
  const int live_rb = zero_dead_rows ? num_row_blocks : live_row_blocks(row_offsets, num_row_blocks);
  const int tile = xcd_remap(tile_id, live_rb * num_slices);
  int rb, slice;
  tile_coords(tile, live_rb, num_slices, group, &rb, &slice);
  const int n0 = slice * BN;
  int32_t begin = row_offsets[rb];
  int32_t end = row_offsets[rb + 1];
  if (begin < 0 || end > nnz || end < begin) begin = end = 0;  // not a BSR row: treat as empty

  uint16_t* out_tile = out + static_cast<int64_t>(rb) * BM * d_model + n0;
  if (begin == end) {
    if (!zero_dead_rows) return;
    constexpr int kChunksPerRow = BN / 8;
    for (int q = threadIdx.x; q < BM * kChunksPerRow; q += Cfg::kThreads) {
      const int r = q / kChunksPerRow, c = q % kChunksPerRow;
      *reinterpret_cast<u32x4_t*>(out_tile + static_cast<int64_t>(r) * d_model + c * 8) = u32x4_t{0u, 0u, 0u, 0u};
    }
    return;
  }

  DsdDmaSrc<Cfg> src;
  src.blocks = blocks;
  src.w = w + n0;
  src.col_indices = col_indices;
  src.w_rows = w_rows;
  src.d_model = d_model;
  src.begin = begin;
  const ADmaPos<Cfg> ap;
#pragma unroll
  for (int q = 0; q < Cfg::kAInstr; ++q) src.a_off[q] = (ap.row[q] * BM + ap.chunk[q] * 8) * 2u;
  const BDmaPos<Cfg> bp;
#pragma unroll
  for (int q = 0; q < Cfg::kBInstr; ++q)
    src.b_off[q] = (static_cast<uint32_t>(bp.row[q]) * d_model + bp.col[q]) * 2u;

  typename ML::Acc acc;
  ML::run(lds, src, (end - begin) * DsdDmaSrc<Cfg>::kStepsPerBlock, acc);

  // bf16, staged in LDS, then whole row segments per store instruction.
  // Plain stores: the combine reads these rows right away, partly from L2.
  ML::stage_tile(lds, acc, [](float v) { return v; });
  ML::for_each_staged_chunk(lds, [&](int r, int col, u32x4_t v) {
    *reinterpret_cast<u32x4_t*>(out_tile + static_cast<int64_t>(r) * d_model + col) = v;
  });
}

}  // namespace sb
