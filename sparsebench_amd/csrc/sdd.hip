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

#include "expert_chunks.hpp"
#include "gelu.hpp"
#include "gemm_dma.hpp"
#include "gemm_tile.hpp"
#include "sdd_tile.hpp"

namespace sb {
namespace {

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
    for (int r = 0; r < 8; ++r) b[r] = load_vec<Cfg::NTB, BRow>(src + r * ffn_dim);
  }
};

template <class Cfg, bool kFastGelu>
__global__ void __launch_bounds__(Cfg::kThreads)
    sdd_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1, const int32_t* __restrict__ row_token,
               const int32_t* __restrict__ row_block_expert, const int32_t* __restrict__ row_offsets,
               uint16_t* __restrict__ out, int32_t num_tokens, int32_t d_model, int32_t ffn_dim, int32_t num_experts,
               int32_t num_row_blocks, int32_t num_slices, int32_t apply_gelu, int32_t group) {
  using ML = Mainloop<Cfg>;
  constexpr int BN = Cfg::BN;
  static_assert(Cfg::BM == kBS, "one row block per tile");
  __shared__ __attribute__((aligned(16))) uint16_t lds[Cfg::kLdsElems];

  const int live_rb = live_row_blocks(row_offsets, num_row_blocks);
  const int tile = xcd_remap(static_cast<int>(blockIdx.x), live_rb * num_slices);
  int rb, slice;
  tile_coords(tile, live_rb, num_slices, group, &rb, &slice);
  const int n0 = slice * BN;
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
        if (apply_gelu) h = kFastGelu ? gelu_erf_fast(h) : gelu_erf_libm(h);
        col[ML::acc_row(i, v) * kBS] = f32_to_bf16(h);
      }
  }
}

template <class Cfg, bool kFastGelu>
__global__ void __launch_bounds__(Cfg::kThreads)
    sdd_dma_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                   const int32_t* __restrict__ row_token, const int32_t* __restrict__ row_block_expert,
                   const int32_t* __restrict__ row_offsets, uint16_t* __restrict__ out, int32_t num_tokens,
                   int32_t d_model, int32_t ffn_dim, int32_t num_experts, int32_t num_row_blocks, int32_t num_slices,
                   int32_t apply_gelu, int32_t group) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg::kLdsAlloc];
  sdd_row_block_tile<Cfg, kFastGelu>(lds, static_cast<int>(blockIdx.x), x, w1, row_token, row_block_expert,
                                     row_offsets, out, num_tokens, d_model, ffn_dim, num_experts, num_row_blocks,
                                     num_slices, apply_gelu, group);
}

// Persistent form (DmaMainloop::run_tiles): gridDim.x workgroups, about one
// per CU slot, each walking the tile list with stride gridDim.x through the
// same XCD remap and grouped order as the one-tile-per-workgroup kernel.
template <class Cfg, bool kFastGelu>
struct SddTiles {
  using ML = DmaMainloop<Cfg>;
  static constexpr int BN = Cfg::BN;
  // Per tile: the expert's W1 buffer, the column origin and this lane's
  // gathered x rows. Everything else is shared by all tiles.
  struct Tile {
    __amdgpu_buffer_rsrc_t w_rsrc;
    uint32_t a_off[Cfg::kAInstr];
    int steps;
    int32_t begin;
    int n0;
  };
  struct Src {
    __amdgpu_buffer_rsrc_t x_rsrc, w_rsrc;
    uint32_t b_step_bytes, n0_bytes;
    uint32_t a_off[Cfg::kAInstr];
    uint32_t b_off[Cfg::kBInstr];
    __device__ __forceinline__ void a_src(int k, __amdgpu_buffer_rsrc_t* r, uint32_t* off) const {
      *r = x_rsrc;
      *off = static_cast<uint32_t>(k) * (Cfg::BK * 2);
    }
    __device__ __forceinline__ void b_src(int k, __amdgpu_buffer_rsrc_t* r, uint32_t* off) const {
      *r = w_rsrc;
      *off = static_cast<uint32_t>(k) * b_step_bytes + n0_bytes;
    }
    __device__ __forceinline__ uint32_t a_voff(int q) const { return a_off[q]; }
    __device__ __forceinline__ uint32_t b_voff(int q) const { return b_off[q]; }
  };

  const uint16_t* x;
  const uint16_t* w1;
  const int32_t* row_token;
  const int32_t* row_block_expert;
  const int32_t* row_offsets;
  uint16_t* out;
  int32_t num_tokens, d_model, ffn_dim, num_experts, num_row_blocks, num_slices, apply_gelu, group;
  int live_rb, live_tiles, vtile;
  __amdgpu_buffer_rsrc_t x_rsrc;
  uint32_t b_step_bytes;
  uint32_t b_off[Cfg::kBInstr];  // this lane's W1 chunk at column origin 0

  __device__ __forceinline__ void init() {
    x_rsrc = make_rsrc(x, static_cast<uint32_t>(num_tokens) * static_cast<uint32_t>(d_model) * 2u);
    b_step_bytes = static_cast<uint32_t>(Cfg::BK) * static_cast<uint32_t>(ffn_dim) * 2u;
    const BDmaPos<Cfg> bp;
#pragma unroll
    for (int q = 0; q < Cfg::kBInstr; ++q) b_off[q] = (static_cast<uint32_t>(bp.row[q]) * ffn_dim + bp.col[q]) * 2u;
  }

  __device__ __forceinline__ Src source(const Tile& t) const {
    Src src;
    src.x_rsrc = x_rsrc;
    src.w_rsrc = t.w_rsrc;
    src.b_step_bytes = b_step_bytes;
    src.n0_bytes = static_cast<uint32_t>(t.n0) * 2u;
#pragma unroll
    for (int q = 0; q < Cfg::kAInstr; ++q) src.a_off[q] = t.a_off[q];
#pragma unroll
    for (int q = 0; q < Cfg::kBInstr; ++q) src.b_off[q] = b_off[q];
    return src;
  }

  // This lane's token for A DMA instruction q. The wave's rows are
  // consecutive: kAInstr * kARowsPerInstr of them, read with uniform
  // (scalar) loads and picked per lane with selects.
  __device__ __forceinline__ void lane_tokens(int rb, int32_t (&tok)[Cfg::kAInstr]) const {
    constexpr int kRows = Cfg::kAInstr * Cfg::kARowsPerInstr;
    const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
    const int32_t* rows = row_token + static_cast<int64_t>(rb) * kBS + wave * kRows;
    // readfirstlane pins each value to an SGPR: without it the compiler folds
    // the selects into one per-lane vector load, whose wait (vmcnt) would
    // also wait for the whole DMA queue.
    int32_t wt[kRows];
#pragma unroll
    for (int r = 0; r < kRows; ++r) wt[r] = __builtin_amdgcn_readfirstlane(rows[r]);
    const int lr = (threadIdx.x & 63) / Cfg::kAChunksPerRow;
#pragma unroll
    for (int q = 0; q < Cfg::kAInstr; ++q) {
      int32_t v = wt[q * Cfg::kARowsPerInstr];
#pragma unroll
      for (int r = 1; r < Cfg::kARowsPerInstr; ++r) v = lr == r ? wt[q * Cfg::kARowsPerInstr + r] : v;
      tok[q] = v;
    }
  }

  __device__ __forceinline__ bool next(Tile& t) {
    const int32_t ffn_blocks = ffn_dim / kBS;
    while (vtile < live_tiles) {
      const int tile = xcd_remap(vtile, live_tiles);
      vtile += gridDim.x;
      int rb, slice;
      tile_coords(tile, live_rb, num_slices, group, &rb, &slice);
      const int32_t begin = row_offsets[rb];
      const int32_t end = row_offsets[rb + 1];
      const int32_t expert = row_block_expert[rb];
      // Same skips as the one-tile kernel: dead, or not a routing layout.
      if (begin == end || end - begin != ffn_blocks || begin < 0 || end > num_row_blocks * ffn_blocks ||
          expert < 0 || expert >= num_experts)
        continue;
      // Uniform by construction; readfirstlane keeps them in SGPRs (a VGPR
      // n0 would make the buffer offset of every W load lane-divergent).
      t.n0 = __builtin_amdgcn_readfirstlane(slice * BN);
      t.begin = __builtin_amdgcn_readfirstlane(begin);
      t.steps = d_model / Cfg::BK;
      t.w_rsrc = make_rsrc(w1 + static_cast<int64_t>(expert) * d_model * ffn_dim,
                           static_cast<uint32_t>(d_model) * static_cast<uint32_t>(ffn_dim) * 2u);
      int32_t tok[Cfg::kAInstr];
      lane_tokens(rb, tok);
      const ADmaPos<Cfg> ap;
#pragma unroll
      for (int q = 0; q < Cfg::kAInstr; ++q)
        t.a_off[q] = (tok[q] >= 0 && tok[q] < num_tokens)
                         ? static_cast<uint32_t>(tok[q]) * static_cast<uint32_t>(d_model) * 2u + ap.chunk[q] * 16u
                         : kOutOfRange;
      return true;
    }
    return false;
  }

  __device__ __forceinline__ void epilogue(const Tile& t, typename ML::Acc& acc) const {
    uint16_t* blocks = out + static_cast<int64_t>(t.begin) * kBS * kBS;
#pragma unroll
    for (int jn = 0; jn < Cfg::TN; ++jn)
#pragma unroll
      for (int i = 0; i < Cfg::TM; ++i) {
        const int m = ML::out_row(i);
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int f = t.n0 + ML::out_col(jn, g);
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            v[e] = acc[jn][i][4 * g + e];
            if (apply_gelu) v[e] = kFastGelu ? gelu_erf_fast(v[e]) : gelu_erf_libm(v[e]);
          }
          *reinterpret_cast<u32x2_t*>(blocks + static_cast<int64_t>(f / kBS) * kBS * kBS + m * kBS + (f % kBS)) =
              u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
      }
  }
};

template <class Cfg, bool kFastGelu>
__global__ void __launch_bounds__(Cfg::kThreads)
    sdd_persistent_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                          const int32_t* __restrict__ row_token, const int32_t* __restrict__ row_block_expert,
                          const int32_t* __restrict__ row_offsets, uint16_t* __restrict__ out, int32_t num_tokens,
                          int32_t d_model, int32_t ffn_dim, int32_t num_experts, int32_t num_row_blocks,
                          int32_t num_slices, int32_t apply_gelu, int32_t group) {
  static_assert(Cfg::BM == kBS, "one row block per tile");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg::kLdsAlloc];
  SddTiles<Cfg, kFastGelu> sched;
  sched.x = x;
  sched.w1 = w1;
  sched.row_token = row_token;
  sched.row_block_expert = row_block_expert;
  sched.row_offsets = row_offsets;
  sched.out = out;
  sched.num_tokens = num_tokens;
  sched.d_model = d_model;
  sched.ffn_dim = ffn_dim;
  sched.num_experts = num_experts;
  sched.num_row_blocks = num_row_blocks;
  sched.num_slices = num_slices;
  sched.apply_gelu = apply_gelu;
  sched.group = group;
  sched.live_rb = live_row_blocks(row_offsets, num_row_blocks);
  sched.live_tiles = sched.live_rb * num_slices;
  sched.vtile = blockIdx.x;
  sched.init();
  DmaMainloop<Cfg>::run_tiles(lds, sched);
}

template <class Cfg, bool kFastGelu>
int launch_sdd_persistent(const void* x, const void* w1, const int32_t* row_token, const int32_t* row_block_expert,
                          const int32_t* row_offsets, void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim,
                          int64_t num_experts, int64_t num_row_blocks, int32_t apply_gelu, hipStream_t stream) {
  if (ffn_dim % Cfg::BN != 0) return fail(SB_ERR_INVALID, "sdd: F %% tile width != 0");
  const int32_t num_slices = static_cast<int32_t>(ffn_dim / Cfg::BN);
  const int64_t tiles = num_row_blocks * num_slices;
  static int occupancy = 0;
  int grid = 0;
  if (const int rc = persistent_grid(reinterpret_cast<const void*>(sdd_persistent_kernel<Cfg, kFastGelu>),
                                     Cfg::kThreads, tiles, &occupancy, &grid))
    return rc;
  sdd_persistent_kernel<Cfg, kFastGelu><<<static_cast<uint32_t>(grid), Cfg::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w1), row_token, row_block_expert, row_offsets,
      static_cast<uint16_t*>(out), static_cast<int32_t>(num_tokens), static_cast<int32_t>(d_model),
      static_cast<int32_t>(ffn_dim), static_cast<int32_t>(num_experts), static_cast<int32_t>(num_row_blocks),
      num_slices, apply_gelu, tile_group());
  return check_launch("sdd");
}

template <class Cfg, bool kFastGelu>
int launch_sdd_dma(const void* x, const void* w1, const int32_t* row_token, const int32_t* row_block_expert,
                   const int32_t* row_offsets, void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim,
                   int64_t num_experts, int64_t num_row_blocks, int32_t apply_gelu, hipStream_t stream) {
  if (ffn_dim % Cfg::BN != 0) return fail(SB_ERR_INVALID, "sdd: F %% tile width != 0");
  const int32_t num_slices = static_cast<int32_t>(ffn_dim / Cfg::BN);
  const int64_t tiles = num_row_blocks * num_slices;
  sdd_dma_kernel<Cfg, kFastGelu><<<static_cast<uint32_t>(tiles), Cfg::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w1), row_token, row_block_expert, row_offsets,
      static_cast<uint16_t*>(out), static_cast<int32_t>(num_tokens), static_cast<int32_t>(d_model),
      static_cast<int32_t>(ffn_dim), static_cast<int32_t>(num_experts), static_cast<int32_t>(num_row_blocks),
      num_slices, apply_gelu, tile_group());
  return check_launch("sdd");
}

template <class Cfg, bool kFastGelu>
int launch_sdd(const void* x, const void* w1, const int32_t* row_token, const int32_t* row_block_expert,
               const int32_t* row_offsets, void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim,
               int64_t num_experts, int64_t num_row_blocks, int32_t apply_gelu, hipStream_t stream) {
  const int32_t num_slices = static_cast<int32_t>(ffn_dim / Cfg::BN);
  const int64_t tiles = num_row_blocks * num_slices;
  sdd_kernel<Cfg, kFastGelu><<<static_cast<uint32_t>(tiles), Cfg::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w1), row_token, row_block_expert, row_offsets,
      static_cast<uint16_t*>(out), static_cast<int32_t>(num_tokens), static_cast<int32_t>(d_model),
      static_cast<int32_t>(ffn_dim), static_cast<int32_t>(num_experts), static_cast<int32_t>(num_row_blocks),
      num_slices, apply_gelu, tile_group());
  return check_launch("sdd");
}

// Tile variants (BM x BN, waves WM x WN, register prefetch depth). 0 = pick by shape.
template <bool kFastGelu, class... Args>
int dispatch_sdd(int variant, Args... args) {
  switch (variant) {
    case 1: return launch_sdd<TileCfg<128, 128, 2, 2, 1>, kFastGelu>(args...);
    case 2: return launch_sdd<TileCfg<128, 256, 2, 2, 1>, kFastGelu>(args...);
    case 3: return launch_sdd<TileCfg<128, 128, 2, 2, 2>, kFastGelu>(args...);
    case 4: return launch_sdd<TileCfg<128, 256, 2, 2, 2>, kFastGelu>(args...);
    case 5: return launch_sdd<TileCfg<128, 256, 2, 4, 1>, kFastGelu>(args...);
    case 6: return launch_sdd<TileCfg<128, 256, 2, 4, 2>, kFastGelu>(args...);
    case 7: return launch_sdd<TileCfg<128, 128, 2, 4, 1>, kFastGelu>(args...);
    case 8: return launch_sdd<TileCfg<128, 128, 2, 4, 2>, kFastGelu>(args...);
    case 11: return launch_sdd_dma<DmaCfg<128, 128, 64, 2>, kFastGelu>(args...);
    case 12: return launch_sdd_dma<DmaCfg<128, 128, 64, 3>, kFastGelu>(args...);
    case 13: return launch_sdd_dma<DmaCfg<128, 128, 32, 5>, kFastGelu>(args...);
    case 14: return launch_sdd_dma<DmaCfg<128, 256, 64, 2>, kFastGelu>(args...);
    case 15: return launch_sdd_dma<DmaCfg<128, 256, 64, 3>, kFastGelu>(args...);
    case 16: return launch_sdd_dma<DmaCfg<128, 256, 32, 6, 2, 4>, kFastGelu>(args...);
    case 17: return launch_sdd_dma<DmaCfg<128, 256, 64, 3, 2, 4>, kFastGelu>(args...);
    case 18: return launch_sdd_dma<DmaCfg<128, 128, 32, 4>, kFastGelu>(args...);
    case 19: return launch_sdd_dma<DmaCfg<128, 128, 32, 5, 2, 4>, kFastGelu>(args...);
    case 9: return launch_sdd<TileCfg<128, 128, 2, 4, 1, true>, kFastGelu>(args...);
    case 10: return launch_sdd<TileCfg<128, 128, 2, 2, 1, true>, kFastGelu>(args...);
    case 21: return launch_sdd_dma<DmaCfg<128, 128, 64, 2, 2, 2, 0, 2>, kFastGelu>(args...);
    case 22: return launch_sdd_dma<DmaCfg<128, 128, 64, 2, 2, 2, 2, 2>, kFastGelu>(args...);
    case 23: return launch_sdd_dma<DmaCfg<128, 128, 64, 3, 2, 2, 0, 2>, kFastGelu>(args...);
    case 24: return launch_sdd_dma<DmaCfg<128, 256, 64, 2, 2, 2, 0, 2>, kFastGelu>(args...);
    case 25: return launch_sdd_dma<DmaCfg<128, 256, 64, 3, 2, 4, 0, 2>, kFastGelu>(args...);
    case 26: return launch_sdd_dma<DmaCfg<128, 256, 64, 3, 2, 2, 0, 2>, kFastGelu>(args...);
    case 27: return launch_sdd_dma<DmaCfg<128, 128, 32, 5, 2, 2, 0, 2>, kFastGelu>(args...);
    case 31: return launch_sdd_dma<DmaCfg<128, 512, 64, 2, 1, 4, 0, 2>, kFastGelu>(args...);
    case 32: return launch_sdd_dma<DmaCfg<128, 512, 32, 4, 1, 4, 0, 2>, kFastGelu>(args...);
    case 33: return launch_sdd_dma<DmaCfg<128, 512, 32, 3, 1, 4, 0, 2>, kFastGelu>(args...);
    case 34: return launch_sdd_dma<DmaCfg<128, 256, 32, 3, 2, 4, 0, 2>, kFastGelu>(args...);
    case 35: return launch_sdd_dma<DmaCfg<128, 256, 32, 3, 2, 2, 0, 2>, kFastGelu>(args...);
    case 36: return launch_sdd_dma<DmaCfg<128, 256, 64, 2, 2, 4, 0, 2>, kFastGelu>(args...);
    case 37: return launch_sdd_dma<DmaCfg<128, 256, 32, 6, 2, 4, 0, 2>, kFastGelu>(args...);
    case 38: return launch_sdd_dma<DmaCfg<128, 256, 32, 5, 2, 4, 0, 2>, kFastGelu>(args...);
    case 39: return launch_sdd_dma<DmaCfg<128, 128, 32, 8, 2, 2, 0, 2>, kFastGelu>(args...);
    case 51: return launch_sdd_dma<DmaCfg<128, 256, 64, 3, 2, 4, 0, 2, 1>, kFastGelu>(args...);
    case 52: return launch_sdd_dma<DmaCfg<128, 512, 32, 4, 1, 4, 0, 2, 1>, kFastGelu>(args...);
    case 53: return launch_sdd_dma<DmaCfg<128, 256, 32, 5, 2, 4, 0, 2, 1>, kFastGelu>(args...);
    case 54: return launch_sdd_dma<DmaCfg<128, 256, 64, 3, 2, 4, 0, 2, 2>, kFastGelu>(args...);
    case 55: return launch_sdd_dma<DmaCfg<128, 512, 32, 4, 1, 4, 0, 2, 2>, kFastGelu>(args...);
    case 56: return launch_sdd_dma<DmaCfg<128, 512, 32, 4, 2, 4, 0, 2, 0>, kFastGelu>(args...);
    case 57: return launch_sdd_dma<DmaCfg<128, 512, 32, 4, 2, 4, 0, 2, 2>, kFastGelu>(args...);
    case 58: return launch_sdd_dma<DmaCfg<128, 512, 32, 4, 2, 4, 0, 2, 1>, kFastGelu>(args...);
    case 59: return launch_sdd_dma<DmaCfg<128, 512, 64, 2, 2, 4, 0, 2, 2>, kFastGelu>(args...);
    // The next step's DMA interleaved with the MFMAs (PIPE 3).
    case 61: return launch_sdd_dma<DmaCfg<128, 512, 64, 2, 2, 4, 0, 2, 3>, kFastGelu>(args...);
    case 62: return launch_sdd_dma<DmaCfg<128, 512, 32, 4, 2, 4, 0, 2, 3>, kFastGelu>(args...);
    case 63: return launch_sdd_dma<DmaCfg<128, 256, 64, 3, 2, 4, 0, 2, 3>, kFastGelu>(args...);
    case 64: return launch_sdd_dma<DmaCfg<128, 512, 32, 4, 1, 4, 0, 2, 3>, kFastGelu>(args...);
    case 65: return launch_sdd_dma<DmaCfg<128, 512, 32, 3, 2, 4, 0, 2, 3>, kFastGelu>(args...);
    case 41: return launch_sdd_persistent<DmaCfg<128, 256, 64, 3, 2, 4, 0, 2>, kFastGelu>(args...);
    case 43: return launch_sdd_persistent<DmaCfg<128, 128, 64, 2, 2, 2, 0, 2>, kFastGelu>(args...);
    case 44: return launch_sdd_persistent<DmaCfg<128, 256, 32, 3, 2, 4, 0, 2>, kFastGelu>(args...);
    default: return fail(SB_ERR_INVALID, "sdd: unknown tile variant %d", variant);
  }
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
  // Buffer offsets are 32-bit: x and one expert's W1 must each stay under 2 GB.
  if (num_tokens * d_model * 2 >= (int64_t{1} << 31) - 2 * d_model)
    return fail(SB_ERR_INVALID, "sdd: x too large for 32-bit buffer offsets");
  if (num_row_blocks * (ffn_dim / 128) > kI32Max || ffn_dim * d_model > kI32Max ||
      num_tokens * d_model > (int64_t{1} << 62) || num_row_blocks * 128 > kI32Max)
    return fail(SB_ERR_INVALID, "problem too large");
  const hipStream_t s = as_stream(stream);
  const int forced = tuning_override("SPARSEBENCH_SDD_VARIANT");
  const int gelu_mode = tuning_override("SPARSEBENCH_GELU_LIBM");
  // Default (default_sdd_variant): 128 x 512 tiles of 8 waves, each 64 x
  // 128 (8 MFMAs per 16-deep sub-step: enough work to cover the LDS
  // fragment reads, 2 waves per SIMD), non-temporal weight loads, the next
  // stage's DMA and the next sub-step's fragment reads issued among the
  // MFMAs.
  int variant = forced > 0 ? forced : default_sdd_variant(d_model, ffn_dim);
  if (ffn_dim % 512 != 0 && ((variant >= 31 && variant <= 33) || variant == 52 || (variant >= 55 && variant <= 59)))
    variant = 25;
  if (ffn_dim % 512 != 0 && (variant == 61 || variant == 62 || variant == 64 || variant == 65)) variant = 63;
  if (gelu_mode > 0)
    return dispatch_sdd<false>(variant, x, w1, row_token, row_block_expert, row_offsets, out, num_tokens, d_model,
                               ffn_dim, num_experts, num_row_blocks, apply_gelu, s);
  return dispatch_sdd<true>(variant, x, w1, row_token, row_block_expert, row_offsets, out, num_tokens, d_model,
                            ffn_dim, num_experts, num_row_blocks, apply_gelu, s);
}
