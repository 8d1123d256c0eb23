// SDD: the MoE's first matmul, written straight into the block-sparse layout
// (the operation of csrc/sdd.cu in the reference, built here for gfx950).
//
//   H blocks [nnz, 128, 128] = gelu( x[row_token] [P, D] @ W1[expert] [D, F] )
//
// Row block r (128 padded rows, one expert e) owns blocks row_offsets[r] + j,
// j < F/128, holding columns j*128 .. j*128+127 of e's FFN. One workgroup
// computes 128 rows x BN columns of one row block:
//   A  gathered inside the load: lane rows map through row_token to rows of
//      x; padding rows (row_token < 0) are zero registers, x is not read.
//   B  W1[e] rows k0 .. k0+63, columns n0 .. n0+BN-1, as stored.
//   epilogue  fp32 -> exact erf GELU -> bf16 (round to nearest even), written
//      as BN/128 blocks of 128 x 128 in BSR order, ready for DSD.
// Dead row blocks (no blocks) exit at once; tiles are ordered row block first
// and spread over the XCDs in contiguous ranges (xcd_remap). The tile code
// is sdd_row_block_tile (sdd_tile.hpp); the MoE layer's SDD kernel
// (experts.hip) shares its main loop and epilogue.

#include "expert_chunks.hpp"
#include "gelu.hpp"
#include "gemm_dma.hpp"
#include "sdd_tile.hpp"

namespace sb {
namespace {

template <class Cfg, bool kWideX>
__global__ void __launch_bounds__(Cfg::kThreads)
    sdd_dma_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                   const int32_t* __restrict__ row_token, const int32_t* __restrict__ row_block_expert,
                   const int32_t* __restrict__ row_offsets, uint16_t* __restrict__ out, int32_t num_tokens,
                   int32_t d_model, int32_t ffn_dim, int32_t num_experts, int32_t num_row_blocks, int32_t num_slices,
                   int32_t apply_gelu) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg::kLdsAlloc];
  sdd_row_block_tile<Cfg, kWideX>(lds, static_cast<int>(blockIdx.x), x, w1, row_token, row_block_expert,
                                  row_offsets, out, num_tokens, d_model, ffn_dim, num_experts, num_row_blocks,
                                  num_slices, apply_gelu, kTileGroup);
}

template <class Cfg, bool kWideX>
int launch_sdd(const void* x, const void* w1, const int32_t* row_token, const int32_t* row_block_expert,
               const int32_t* row_offsets, void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim,
               int64_t num_experts, int64_t num_row_blocks, int32_t apply_gelu, hipStream_t stream) {
  if (!reduction_fits<Cfg>(d_model))
    return fail(SB_ERR_INVALID, "sdd: D (%lld) is not a whole number of the tile's K steps",
                static_cast<long long>(d_model));
  const int32_t num_slices = static_cast<int32_t>(ffn_dim / Cfg::BN);
  const int64_t tiles = num_row_blocks * num_slices;
  sdd_dma_kernel<Cfg, kWideX><<<static_cast<uint32_t>(tiles), Cfg::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w1), row_token, row_block_expert, row_offsets,
      static_cast<uint16_t*>(out), static_cast<int32_t>(num_tokens), static_cast<int32_t>(d_model),
      static_cast<int32_t>(ffn_dim), static_cast<int32_t>(num_experts), static_cast<int32_t>(num_row_blocks),
      num_slices, apply_gelu);
  return check_launch("sdd");
}

template <bool kWideX, class... Args>
int dispatch_sdd(SddTile tile, Args... args) {
  switch (tile) {
    case SddTile::kWide: return launch_sdd<SddWideTile, kWideX>(args...);
    case SddTile::kDeep: return launch_sdd<SddDeepTile, kWideX>(args...);
    case SddTile::kNarrow: return launch_sdd<SddNarrowTile, kWideX>(args...);
  }
  return fail(SB_ERR_INVALID, "sdd: no tile for this shape");
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" int sb_sdd(const void* x, const void* w1, const int32_t* row_token, const int32_t* row_block_expert,
                      const int32_t* row_offsets, void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim,
                      int64_t num_experts, int64_t num_row_blocks, int32_t apply_gelu, void* stream) {
  constexpr int64_t kI32Max = 2147483647;
  if (num_row_blocks < 0) return fail(SB_ERR_INVALID, "sdd: row_offsets must have at least one entry");
  if (num_row_blocks == 0) return clear_ok();
  if (!x || !w1 || !row_token || !row_block_expert || !row_offsets || !out)
    return fail(SB_ERR_INVALID, "sdd: null buffer");
  if (!aligned16(x) || !aligned16(w1) || !aligned16(out))
    return fail(SB_ERR_INVALID, "x and w1 must be 16-byte aligned");
  if (d_model <= 0 || d_model % 64 != 0)
    return fail(SB_ERR_INVALID, "sdd needs D (%lld) to be a multiple of 64", static_cast<long long>(d_model));
  if (ffn_dim <= 0 || ffn_dim % 256 != 0)
    return fail(SB_ERR_INVALID, "sdd needs F (%lld) to be a multiple of 256", static_cast<long long>(ffn_dim));
  if (num_tokens <= 0 || num_tokens > kI32Max || num_experts <= 0 || num_experts > kI32Max)
    return fail(SB_ERR_INVALID, "sdd: bad token or expert count");
  // The reference's limits (csrc/sdd.cu:151-153): one expert's W1 and the
  // tile grid within int32. W1[e] is read through a buffer of up to 4 GB.
  if (num_row_blocks * (ffn_dim / 128) > kI32Max || ffn_dim * d_model > kI32Max ||
      num_tokens * d_model > (int64_t{1} << 62) || num_row_blocks * 128 > kI32Max)
    return fail(SB_ERR_INVALID, "problem too large");
  const hipStream_t s = as_stream(stream);
  const SddTile tile = sdd_tile_for(d_model, ffn_dim);
  if (sdd_wide_x(num_tokens, d_model))
    return dispatch_sdd<true>(tile, x, w1, row_token, row_block_expert, row_offsets, out, num_tokens, d_model, ffn_dim,
                              num_experts, num_row_blocks, apply_gelu, s);
  return dispatch_sdd<false>(tile, x, w1, row_token, row_block_expert, row_offsets, out, num_tokens, d_model, ffn_dim,
                             num_experts, num_row_blocks, apply_gelu, s);
}
