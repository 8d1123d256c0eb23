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
// and spread over the XCDs in contiguous ranges (xcd_remap).

#include <type_traits>

#include "gemm_tile.hpp"

namespace sb {
namespace {

constexpr int kBS = 128;

__device__ __forceinline__ float gelu_erf(float v) { return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f)); }

template <class Cfg>
struct SddLoader {
  using ML = Mainloop<Cfg>;
  using BRow = typename Cfg::BRow;
  const uint16_t* x;
  const uint16_t* w_cols;  // W1[e] + n0
  int64_t d_model, ffn_dim;
  int32_t token[Cfg::kAChunks];

  __device__ __forceinline__ void load_a(int t, const typename ML::LoadPos& p, u32x4_t (&a)[Cfg::kAChunks]) const {
    const int k = t * Cfg::BK + p.a_chunk * 8;
#pragma unroll
    for (int j = 0; j < Cfg::kAChunks; ++j) {
      if (token[j] >= 0) {
        a[j] = *reinterpret_cast<const u32x4_t*>(x + token[j] * d_model + k);
      } else {
        a[j] = u32x4_t{0u, 0u, 0u, 0u};
      }
    }
  }

  __device__ __forceinline__ void load_b(int t, const typename ML::LoadPos& p, BRow (&b)[8]) const {
    const uint16_t* src = w_cols + (static_cast<int64_t>(t) * Cfg::BK + p.b_kgroup * 8) * ffn_dim + p.b_col;
#pragma unroll
    for (int r = 0; r < 8; ++r) b[r] = *reinterpret_cast<const BRow*>(src + r * ffn_dim);
  }
};

template <int BN>
__global__ void __launch_bounds__(256)
    sdd_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1, const int32_t* __restrict__ row_token,
               const int32_t* __restrict__ row_block_expert, const int32_t* __restrict__ row_offsets,
               uint16_t* __restrict__ out, int32_t num_tokens, int32_t d_model, int32_t ffn_dim, int32_t num_experts,
               int32_t num_row_blocks, int32_t num_slices, int32_t apply_gelu) {
  using Cfg = TileCfg<kBS, BN>;
  using ML = Mainloop<Cfg>;
  __shared__ __attribute__((aligned(16))) uint16_t lds[Cfg::kLdsElems];

  const int live = live_row_blocks(row_offsets, num_row_blocks) * num_slices;
  const int tile = xcd_remap(static_cast<int>(blockIdx.x), live);
  const int rb = tile / num_slices;
  const int n0 = (tile % num_slices) * BN;
  const int32_t begin = row_offsets[rb];
  const int32_t end = row_offsets[rb + 1];
  const int32_t ffn_blocks = ffn_dim / kBS;
  if (begin == end) return;  // dead row block: nothing to write
  const int32_t expert = row_block_expert[rb];
  // A live row block holds exactly its expert's F/128 blocks; anything else
  // is not a routing layout and is skipped rather than written out of range.
  if (end - begin != ffn_blocks || begin < 0 || end > num_row_blocks * ffn_blocks || expert < 0 ||
      expert >= num_experts)
    return;

  SddLoader<Cfg> ld;
  ld.x = x;
  ld.w_cols = w1 + static_cast<int64_t>(expert) * d_model * ffn_dim + n0;
  ld.d_model = d_model;
  ld.ffn_dim = ffn_dim;
  const typename ML::LoadPos pos = ML::load_pos();
#pragma unroll
  for (int j = 0; j < Cfg::kAChunks; ++j) {
    const int32_t tok = row_token[static_cast<int64_t>(rb) * kBS + pos.a_row[j]];
    ld.token[j] = (tok >= 0 && tok < num_tokens) ? tok : -1;
  }

  typename ML::Acc acc;
  ML::run(lds, ld, d_model / Cfg::BK, acc);

  // Column f of the expert's FFN -> block begin + f/128, column f % 128.
  uint16_t* blocks = out + static_cast<int64_t>(begin) * kBS * kBS;
#pragma unroll
  for (int j = 0; j < Cfg::TN; ++j) {
    const int f = n0 + ML::acc_col(j);
    uint16_t* col = blocks + static_cast<int64_t>(f / kBS) * kBS * kBS + (f % kBS);
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        float h = acc[i][j][v];
        if (apply_gelu) h = gelu_erf(h);
        col[ML::acc_row(i, v) * kBS] = f32_to_bf16(h);
      }
  }
}

template <int BN>
int launch_sdd(const void* x, const void* w1, const int32_t* row_token, const int32_t* row_block_expert,
               const int32_t* row_offsets, void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim,
               int64_t num_experts, int64_t num_row_blocks, int32_t apply_gelu, hipStream_t stream) {
  const int32_t num_slices = static_cast<int32_t>(ffn_dim / BN);
  const int64_t tiles = num_row_blocks * num_slices;
  sdd_kernel<BN><<<static_cast<uint32_t>(tiles), 256, 0, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w1), row_token, row_block_expert, row_offsets,
      static_cast<uint16_t*>(out), static_cast<int32_t>(num_tokens), static_cast<int32_t>(d_model),
      static_cast<int32_t>(ffn_dim), static_cast<int32_t>(num_experts), static_cast<int32_t>(num_row_blocks),
      num_slices, apply_gelu);
  return check_launch("sdd");
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
  if (num_row_blocks * (ffn_dim / 128) > kI32Max || ffn_dim * d_model > kI32Max ||
      num_tokens * d_model > (int64_t{1} << 62) || num_row_blocks * 128 > kI32Max)
    return fail(SB_ERR_INVALID, "problem too large");
  const hipStream_t s = as_stream(stream);
  // 256-column tiles read each gathered A tile half as often; 128-column
  // tiles double the workgroup count when there are too few row blocks to
  // fill 256 CUs a few times over.
  if (num_row_blocks * (ffn_dim / 256) >= 4 * 256)
    return launch_sdd<256>(x, w1, row_token, row_block_expert, row_offsets, out, num_tokens, d_model, ffn_dim,
                           num_experts, num_row_blocks, apply_gelu, s);
  return launch_sdd<128>(x, w1, row_token, row_block_expert, row_offsets, out, num_tokens, d_model, ffn_dim,
                         num_experts, num_row_blocks, apply_gelu, s);
}
