// DSD: block-sparse (BSR) x dense on gfx950 (the operation of the reference's
// csrc/dsd_v1.cu .. dsd_v5.cu, one kernel here for every version code).
//
//   out[r*bs + i, n] = sum_{p in [row_offsets[r], row_offsets[r+1])}
//                      sum_{kk < bs} blocks[p][i][kk] * w[col_indices[p]*bs + kk, n]
//
// One workgroup computes bs x BN outputs of one row block, walking its
// blocks in K steps through col_indices on the LDS-DMA MFMA tile loop
// (dsd_row_block_tile, dsd_tile.hpp). Dead row blocks are skipped, or written as zeros
// when zero_dead_rows is set (the contract of the reference's versions 1-3).
// Tiles are row block first and spread over the XCDs in contiguous ranges,
// so a row block's column slices and an expert's row blocks share an L2.

#include "dsd_tile.hpp"
#include "gemm_dma.hpp"

namespace sb {
namespace {

template <class Cfg>
__global__ void __launch_bounds__(Cfg::kThreads)
    dsd_dma_kernel(const uint16_t* __restrict__ blocks, const uint16_t* __restrict__ w,
                   const int32_t* __restrict__ row_offsets, const int32_t* __restrict__ col_indices,
                   uint16_t* __restrict__ out, int64_t nnz, int64_t w_rows, int32_t num_row_blocks, int32_t d_model,
                   int32_t num_slices, int32_t zero_dead_rows) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg::kLdsAlloc];
  dsd_row_block_tile<Cfg>(lds, static_cast<int>(blockIdx.x), blocks, w, row_offsets, col_indices, out, nnz, w_rows,
                          num_row_blocks, d_model, num_slices, zero_dead_rows, kTileGroup);
}

template <class Cfg>
int launch_dsd(const void* blocks, const void* w, const int32_t* row_offsets, const int32_t* col_indices, void* out,
               int64_t nnz, int64_t w_rows, int64_t num_row_blocks, int64_t d_model, int32_t zero_dead_rows,
               hipStream_t stream) {
  const int32_t num_slices = static_cast<int32_t>(d_model / Cfg::BN);
  const int64_t tiles = num_row_blocks * num_slices;
  dsd_dma_kernel<Cfg><<<static_cast<uint32_t>(tiles), Cfg::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(blocks), static_cast<const uint16_t*>(w), row_offsets, col_indices,
      static_cast<uint16_t*>(out), nnz, w_rows, static_cast<int32_t>(num_row_blocks), static_cast<int32_t>(d_model),
      num_slices, zero_dead_rows);
  return check_launch("dsd");
}

// Tile shapes for a block size BM, from timing every shape tried on the
// benchmark configurations (MI355X, samples interleaved across shapes):
//   D % 512 == 0   128 x 512 tiles, BK 32 through a 4-stage ring, 4 waves of
//                  128 x 128; with a deep reduction (K = F per expert >= 8192)
//                  8 waves of 64 x 128
//   D % 256 == 0   128 x 256 tiles, BK 64 x 3 stages, 8 waves
//   otherwise      128 x 128 tiles, BK 64 x 3 stages, 4 waves
// All with non-temporal W loads; the 256- and 512-wide ones issue the DMA of
// a later step and the next sub-step's fragment reads among the MFMAs, and
// the 512-wide ones load H two K steps at a time, as whole 128-byte rows
// (APAIR; a row's K is a multiple of 64, since bs is 64 or 128), and read
// the next step's first fragments among the current step's last MFMAs
// (PIPE 5).
template <int BM, class... Args>
int dispatch_dsd(int64_t d_model, int64_t row_k, Args... args) {
  if (d_model % 512 == 0) {
    if (row_k >= 8192) return launch_dsd<DmaCfg<BM, 512, 32, 4, 2, 4, 0, 2, 5, 1, 1>>(args...);
    return launch_dsd<DmaCfg<BM, 512, 32, 4, 1, 4, 0, 2, 5, 1, 1>>(args...);
  }
  if (d_model % 256 == 0) return launch_dsd<DmaCfg<BM, 256, 64, 3, 2, 4, 0, 2, 3>>(args...);
  return launch_dsd<DmaCfg<BM, 128, 64, 3, 2, 2, 0, 2, 0>>(args...);
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" int sb_dsd(const void* blocks, const void* w, const int32_t* row_offsets, const int32_t* col_indices,
                      void* out, int64_t nnz, int64_t w_rows, int64_t num_row_blocks, int64_t block_size,
                      int64_t d_model, int32_t zero_dead_rows, void* stream) {
  constexpr int64_t kI32Max = 2147483647;
  if (block_size != 64 && block_size != 128)
    return fail(SB_ERR_INVALID, "block size must be 64 or 128, got %lld", static_cast<long long>(block_size));
  if (d_model <= 0 || d_model % 128 != 0)
    return fail(SB_ERR_INVALID, "D (%lld) must be a positive multiple of 128", static_cast<long long>(d_model));
  if (num_row_blocks < 0) return fail(SB_ERR_INVALID, "row_offsets must have at least one entry");
  if (w_rows < 0 || w_rows % block_size != 0)
    return fail(SB_ERR_INVALID, "w rows (%lld) must be a multiple of the block size (%lld)",
                static_cast<long long>(w_rows), static_cast<long long>(block_size));
  if (nnz < 0) return fail(SB_ERR_INVALID, "blocks must be [nnz, bs, bs]");
  if (num_row_blocks * block_size > kI32Max) return fail(SB_ERR_INVALID, "too many row blocks");
  if (num_row_blocks * (d_model / 128) > kI32Max) return fail(SB_ERR_INVALID, "too many tiles for a 1-D grid");
  if (num_row_blocks == 0) return clear_ok();
  if (!blocks || !w || !row_offsets || !col_indices || !out) return fail(SB_ERR_INVALID, "dsd: null buffer");
  if (!aligned16(blocks) || !aligned16(w) || !aligned16(out))
    return fail(SB_ERR_INVALID, "blocks and w must be 16-byte aligned");
  // The reduction depth per row block, from the buffer shape (nnz /
  // num_row_blocks blocks per row), picks the deep-K tile.
  const int64_t row_k = nnz / num_row_blocks * block_size;
  const hipStream_t s = as_stream(stream);
  if (block_size == 128)
    return dispatch_dsd<128>(d_model, row_k, blocks, w, row_offsets, col_indices, out, nnz, w_rows, num_row_blocks,
                             d_model, zero_dead_rows, s);
  return dispatch_dsd<64>(d_model, row_k, blocks, w, row_offsets, col_indices, out, nnz, w_rows, num_row_blocks,
                          d_model, zero_dead_rows, s);
}
