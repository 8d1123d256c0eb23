// One SDD tile of a row block on the LDS-DMA main loop (gemm_dma.hpp): the
// tile of the per-row-block kernel (sdd.hip), and that kernel's default
// tile shape, which the MoE layer's SDD kernel (experts.hip) also uses.
#pragma once

#include "expert_chunks.hpp"
#include "gelu.hpp"
#include "gemm_dma.hpp"

namespace sb {

// Sources of an SDD tile's K steps on the LDS-DMA main loop: token rows of
// x gathered by the loads themselves, and W1[e] as stored.
//
// x under 2 GiB (kWideX false): one buffer over x; a lane's 32-bit offset is
// its token row's chunk, and a padding row (no token) gets an out-of-range
// offset, so the buffer unit lands zeros in LDS without reading memory.
// x of 2 GiB or more (kWideX true): 32-bit offsets cannot reach every row,
// so each lane issues global_load_lds from its own 64-bit address, its row's
// chunk advanced by BK * 2 bytes per K step; a padding row's lane reads the
// 16 zero bytes of sdd_zero_chunk at every step instead.
static __device__ __attribute__((aligned(16))) uint32_t sdd_zero_chunk[4];

template <class Cfg, bool kWideX = false>
struct SddDmaSrc {
  static constexpr bool kGlobalA = kWideX;
  __amdgpu_buffer_rsrc_t x_rsrc, w_rsrc;
  uint32_t a_off[Cfg::kAInstr];
  uint32_t b_off[Cfg::kBInstr];
  uint32_t b_step_bytes;
  // Global form: this lane's address at step 0, and its advance per step.
  uint64_t a_addr[kWideX ? Cfg::kAInstr : 1];
  uint32_t a_step[kWideX ? Cfg::kAInstr : 1];
  __device__ __forceinline__ uint32_t a_voff(int q) const { return a_off[q]; }
  __device__ __forceinline__ uint32_t b_voff(int q) const { return b_off[q]; }
  __device__ __forceinline__ const void* a_global(int q, int t) const {
    return reinterpret_cast<const void*>(a_addr[q] + static_cast<uint64_t>(static_cast<uint32_t>(t)) * a_step[q]);
  }
  __device__ __forceinline__ void a_src(int t, __amdgpu_buffer_rsrc_t* r, uint32_t* s) const {
    *r = x_rsrc;
    *s = static_cast<uint32_t>(t) * (Cfg::BK * 2);
  }
  __device__ __forceinline__ void b_src(int t, __amdgpu_buffer_rsrc_t* r, uint32_t* s) const {
    *r = w_rsrc;
    *s = static_cast<uint32_t>(t) * b_step_bytes;
  }
  // Lane A position q reads token `tok` (< 0: a padding row), 16-byte chunk `chunk`.
  __device__ __forceinline__ void set_row(int q, int32_t tok, int chunk, const uint16_t* x, int32_t d_model) {
    if constexpr (kWideX) {
      const bool real = tok >= 0;
      a_addr[q] = real ? reinterpret_cast<uint64_t>(x + static_cast<int64_t>(tok) * d_model) + chunk * 16u
                       : reinterpret_cast<uint64_t>(&sdd_zero_chunk[0]);
      a_step[q] = real ? Cfg::BK * 2u : 0u;
      a_off[q] = 0;
    } else {
      a_off[q] = tok >= 0 ? static_cast<uint32_t>(tok) * static_cast<uint32_t>(d_model) * 2u + chunk * 16u
                          : kOutOfRange;
    }
  }
};

// Tile `tile_id` of the row-block grid: 128 rows x BN FFN columns of one
// row block, written as BN/128 blocks. Ids past the grid's
// num_row_blocks * num_slices tiles, dead row blocks and row blocks that are
// not a routing layout's do nothing.
template <class Cfg, bool kWideX>
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

  SddDmaSrc<Cfg, kWideX> src;
  src.x_rsrc = make_rsrc(x, kWideX ? 0u : static_cast<uint32_t>(num_tokens) * static_cast<uint32_t>(d_model) * 2u);
  src.w_rsrc = make_rsrc(w1 + static_cast<int64_t>(expert) * d_model * ffn_dim,
                         static_cast<uint32_t>(d_model) * static_cast<uint32_t>(ffn_dim) * 2u);
  src.b_step_bytes = static_cast<uint32_t>(Cfg::BK) * static_cast<uint32_t>(ffn_dim) * 2u;
  const ADmaPos<Cfg> ap;
#pragma unroll
  for (int q = 0; q < Cfg::kAInstr; ++q) {
    const int32_t tok = row_token[static_cast<int64_t>(rb) * kBS + ap.row[q]];
    src.set_row(q, (tok >= 0 && tok < num_tokens) ? tok : -1, ap.chunk[q], x, d_model);
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
    ML::stage_tile(lds, acc, [](float v) { return gelu_erf_fast(v); });
  else
    ML::stage_tile(lds, acc, [](float v) { return v; });
  uint16_t* blocks = out + static_cast<int64_t>(begin) * kBS * kBS;
  ML::for_each_staged_chunk(lds, [&](int m, int col, u32x4_t v) {
    const int f = n0 + col;
    *reinterpret_cast<u32x4_t*>(blocks + static_cast<int64_t>(f / kBS) * kBS * kBS + m * kBS + (f % kBS)) = v;
  });
}

// The tile shapes of the per-row-block SDD, from timing every shape tried on
// the benchmark configurations (MI355X, samples interleaved across shapes):
// 128 x 512 tiles of 8 waves (64 x 128 each: 8 MFMAs per 16-deep sub-step,
// enough to cover the LDS fragment reads), BK 32 through a 3-stage ring, or
// a 4-stage one for a deep reduction (D >= 4096), the x rows loaded two K
// steps at a time as whole 128-byte rows (APAIR); 128 x 256 tiles (BK 64 x 3
// stages) when F is not a multiple of 512. All: non-temporal W1 loads, the
// DMA of a later step and the next sub-step's fragment reads issued among
// the MFMAs (PIPE 3); the 4-stage tile also reads the next step's first
// fragments among the current step's last MFMAs (PIPE 5; in the 3-stage
// one that schedule spills inside the main loop).
using SddWideTile = DmaCfg<128, 512, 32, 3, 2, 4, 0, 2, 3, 1, 1>;
using SddDeepTile = DmaCfg<128, 512, 32, 4, 2, 4, 0, 2, 5, 1, 1>;
using SddNarrowTile = DmaCfg<128, 256, 64, 3, 2, 4, 0, 2, 3>;
// Half of the narrow tile (the layer's pair kernel splits a short last round
// of singles into column halves): the same ring and K steps, 64 x 32 per wave.
using SddNarrowHalfTile = DmaCfg<128, 128, 64, 3, 2, 4, 0, 2, 3>;
// Half of a 512-wide tile (the layer kernel splits a short last round of
// row-block tiles into column halves): 8 waves of 64 x 64, the 4-stage
// paired ring of the deep tile.
using SddHalfTile = DmaCfg<128, 256, 32, 4, 2, 4, 0, 2, 5, 1, 1>;

enum class SddTile { kWide, kDeep, kNarrow };

inline SddTile sdd_tile_for(int64_t d_model, int64_t ffn_dim) {
  if (ffn_dim % 512 != 0) return SddTile::kNarrow;
  return d_model >= 4096 ? SddTile::kDeep : SddTile::kWide;
}

// x of 2 GiB or more needs the 64-bit gather (SddDmaSrc's global form).
inline bool sdd_wide_x(int64_t num_tokens, int64_t d_model) {
  return num_tokens * d_model * 2 >= (int64_t{1} << 31) - 2 * d_model;
}

}  // namespace sb
