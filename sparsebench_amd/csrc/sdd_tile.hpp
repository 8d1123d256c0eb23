// One SDD tile of a row block on the LDS-DMA main loop (gemm_dma.hpp): the
// tile of the per-row-block kernel (sdd.hip), and that kernel's default
// tile shape, which the MoE layer's SDD kernel (experts.hip) also uses.
#pragma once

#include "expert_chunks.hpp"
#include "gelu.hpp"
#include "gemm_dma.hpp"

namespace sb {

// The same tile on the LDS-DMA mainloop (gemm_dma.hpp): token rows are
// gathered by the buffer loads themselves, padding rows read out of range
// and land in LDS as zeros.
template <class Cfg>
struct SddDmaSrc {
  __amdgpu_buffer_rsrc_t x_rsrc, w_rsrc;
  uint32_t a_off[Cfg::kAInstr];
  uint32_t b_off[Cfg::kBInstr];
  uint32_t b_step_bytes;
  __device__ __forceinline__ uint32_t a_voff(int q) const { return a_off[q]; }
  __device__ __forceinline__ uint32_t b_voff(int q) const { return b_off[q]; }
  __device__ __forceinline__ void a_src(int t, __amdgpu_buffer_rsrc_t* r, uint32_t* s) const {
    *r = x_rsrc;
    *s = static_cast<uint32_t>(t) * (Cfg::BK * 2);
  }
  __device__ __forceinline__ void b_src(int t, __amdgpu_buffer_rsrc_t* r, uint32_t* s) const {
    *r = w_rsrc;
    *s = static_cast<uint32_t>(t) * b_step_bytes;
  }
};

// Tile `tile_id` of the row-block grid: 128 rows x BN FFN columns of one
// row block, written as BN/128 blocks. Ids past the grid's
// num_row_blocks * num_slices tiles, dead row blocks and row blocks that are
// not a routing layout's do nothing.
template <class Cfg, bool kFastGelu>
__device__ __forceinline__ void sdd_row_block_tile(uint8_t* __restrict__ lds, int tile_id,
                                                   const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                                                   const int32_t* __restrict__ row_token,
                                                   const int32_t* __restrict__ row_block_expert,
                                                   const int32_t* __restrict__ row_offsets, uint16_t* __restrict__ out,
                                                   int32_t num_tokens, int32_t d_model, int32_t ffn_dim,
                                                   int32_t num_experts, int32_t num_row_blocks, int32_t num_slices,
                                                   int32_t apply_gelu, int32_t group) {
  using ML = DmaMainloop<Cfg>;
  constexpr int BN = Cfg::BN;
  static_assert(Cfg::BM == kBS, "one row block per tile");
  if (tile_id >= num_row_blocks * num_slices) return;
  const int live_rb = live_row_blocks(row_offsets, num_row_blocks);
  const int tile = xcd_remap(tile_id, live_rb * num_slices);
  int rb, slice;
  tile_coords(tile, live_rb, num_slices, group, &rb, &slice);
  const int n0 = slice * BN;
  const int32_t begin = row_offsets[rb];
  const int32_t end = row_offsets[rb + 1];
  const int32_t ffn_blocks = ffn_dim / kBS;
  if (begin == end) return;
  const int32_t expert = row_block_expert[rb];
  if (end - begin != ffn_blocks || begin < 0 || end > num_row_blocks * ffn_blocks || expert < 0 ||
      expert >= num_experts)
    return;

  SddDmaSrc<Cfg> src;
  src.x_rsrc = make_rsrc(x, static_cast<uint32_t>(num_tokens) * static_cast<uint32_t>(d_model) * 2u);
  src.w_rsrc = make_rsrc(w1 + static_cast<int64_t>(expert) * d_model * ffn_dim,
                         static_cast<uint32_t>(d_model) * static_cast<uint32_t>(ffn_dim) * 2u);
  src.b_step_bytes = static_cast<uint32_t>(Cfg::BK) * static_cast<uint32_t>(ffn_dim) * 2u;
  const ADmaPos<Cfg> ap;
#pragma unroll
  for (int q = 0; q < Cfg::kAInstr; ++q) {
    const int32_t tok = row_token[static_cast<int64_t>(rb) * kBS + ap.row[q]];
    src.a_off[q] = (tok >= 0 && tok < num_tokens)
                        ? static_cast<uint32_t>(tok) * static_cast<uint32_t>(d_model) * 2u + ap.chunk[q] * 16u
                        : kOutOfRange;
  }
  const BDmaPos<Cfg> bp;
#pragma unroll
  for (int q = 0; q < Cfg::kBInstr; ++q)
    src.b_off[q] = (static_cast<uint32_t>(bp.row[q]) * ffn_dim + n0 + bp.col[q]) * 2u;

  typename ML::Acc acc;
  ML::run(lds, src, d_model / Cfg::BK, acc);

  // GELU, bf16, staged in LDS; then C[m, f] -> block begin + f/128, row m,
  // column f % 128, whole 256-byte block rows per store instruction. Plain
  // stores: DSD reads H right after, and a non-temporal hint here makes SDD
  // alone faster but the layer slower (DSD then misses on H).
  if (apply_gelu)
    ML::stage_tile(lds, acc, [](float v) { return kFastGelu ? gelu_erf_fast(v) : gelu_erf_libm(v); });
  else
    ML::stage_tile(lds, acc, [](float v) { return v; });
  uint16_t* blocks = out + static_cast<int64_t>(begin) * kBS * kBS;
  ML::for_each_staged_chunk(lds, [&](int m, int col, u32x4_t v) {
    const int f = n0 + col;
    *reinterpret_cast<u32x4_t*>(blocks + static_cast<int64_t>(f / kBS) * kBS * kBS + m * kBS + (f % kBS)) = v;
  });
}

// Default tile: 128 x 512 tiles of 8 waves (64 x 128 each), BK 32, a
// 3-stage ring, or a 4-stage one for a deep reduction (D >= 4096); 128 x 256
// tiles (BK 64 x 3 stages) when F is not a multiple of 512. From timing every
// variant on the benchmark shapes (MI355X, samples interleaved).
inline int default_sdd_variant(int64_t d_model, int64_t ffn_dim) {
  if (ffn_dim % 512 != 0) return 63;
  return d_model >= 4096 ? 62 : 65;
}

}  // namespace sb
