// The SDD and DSD stages of the MoE layer, each one kernel that tiles either
// by expert chunks or by row blocks, chosen on the device.
//
// The routing layout gives expert e n = tokens_per_expert[e] real rows,
// stored from padded row padded_offsets[e] in ceil(n / 128) row blocks, real
// rows first. The per-row-block kernels (sdd.hip, dsd.hip) stream all of an
// expert's weight columns once per row block and compute the padding rows.
// With near-uniform routing most experts hold a little more or less than
// one block, so a second, nearly empty row block streams the whole weight
// slice again (a third of SDD's HBM traffic at the fine-grained shape) and
// about a quarter of the MFMAs run on padding.
//
// Expert tiles (expert_chunks.hpp): a tile covers one chunk of one expert's
// rows, M = 32 R rows for the chunk's own R = ceil(rows / 32), with one row
// of waves, each owning a column strip of all R 32-row groups, on the
// LDS-DMA main loop (gemm_dma.hpp).
//   SDD  chunks of up to 192 rows (RMAX 6: an expert with 129-192 rows is
//        one tile), 512 columns per tile, 8 waves of 64 columns.
//   DSD  chunks of up to 256 rows (RMAX 8), 256 columns per tile, 4 waves
//        of 64 columns; at the fine-grained shape 64 experts x 4 slices is
//        one tile per CU. For a reduction of F >= 8192, 8 waves and chunks
//        of 256 rows whose last piece of up to 64 rows joins the chunk
//        before it (RMAX 10): at the Mixtral-like shape every expert is then
//        four chunks, 512 tiles in two rounds on 256 CUs, where a fifth,
//        nearly empty chunk per expert made 592 tiles and a third round.
// Rows of a chunk past its real rows are read as zeros (out-of-range DMA,
// no memory read). SDD writes all 32 R rows of a chunk (padding rows as
// GELU(0) = 0); DSD writes the real rows only. Padding rows past an
// expert's last 32-row group are written by neither: nothing in the layer
// reads them.
//
// Every workgroup computes the same choice from tokens_per_expert
// (expert_tiles_chosen): expert tiles for balanced routing, else row-block
// tiles with sb_sdd's / sb_dsd's default tile shape. Both live in one kernel
// so the choice costs nothing: two launches, one of them returning at once,
// cost about 10 us each (every workgroup holds up to 160 KB of LDS while it
// reads the counts). The row-block tiles run on the expert tiles' own code
// (sdd_chunk_tile / dsd_chunk_tile with the row block as a 128-row chunk,
// every row read and written, except that the 4-wave DSD reads and writes
// only the real 32-row groups of an expert of one row block), which also
// needs fewer dependent loads
// before the first DMA than the per-row-block kernels' tiles. Next to the
// expert tiles in one kernel, dsd_row_block_tile's main loop gets a full
// vmcnt(0) after every step's barrier from the compiler (its LDS-DMA alias
// tracking loses the stages apart), which serialises its loads and MFMAs.

#include "expert_chunks.hpp"
#include "gelu.hpp"
#include "gemm_dma.hpp"
#include "layout.hpp"
#include "sdd_tile.hpp"

namespace sb {
namespace {

// Main-loop configuration of an R-group tile: M = 32 R, K steps of 32, one
// row of WAVES waves, non-temporal weight loads, DMA issue spread over the
// MFMAs and the next step's first fragments read among the current step's
// last MFMAs (PIPE 5). With 8 waves (two per SIMD, at most 256 registers
// each) and six row groups, the 192 accumulators leave room for one set of
// A fragments only (PIPE 4); a bf16 tile over 160 KB is staged in two parts.
// 4-stage rings load A two K steps at a time, as whole 128-byte rows
// (APAIR); in the 3-stage rings of the taller SDD tiles the extra address
// registers would spill inside the main loop.
template <int R, int BN, int WAVES, int STAGES>
using ChunkCfg = DmaCfg<32 * R, BN, 32, STAGES, 1, WAVES, 0, 2, (WAVES == 8 && R >= 6) ? 4 : 5,
                        (32 * R * BN * 2 > 160 * 1024) ? 2 : 1, STAGES == 4 ? 1 : 0>;

template <class T>
struct Tag {
  using type = T;
};

// The DSD's tiles: as ChunkCfg, except that with 8 waves an even number of
// row groups is split between two rows of 4 waves (a 256 x 256 tile: 128 x
// 64 per wave, where one row of 8 waves would read all 256 A rows in every
// wave). At most 128 accumulators then, so always PIPE 5.
template <int R, int BN, int WAVES, int STAGES>
using DsdCfg = DmaCfg<32 * R, BN, 32, STAGES, (WAVES == 8 && R % 2 == 0) ? 2 : 1,
                      (WAVES == 8 && R % 2 == 0) ? WAVES / 2 : WAVES, 0, 2, 5, 1, STAGES == 4 ? 1 : 0>;

// A tile configuration cut to R row groups (R a multiple of its rows of
// waves, WM: DmaCfg asserts that each wave owns whole 32-row groups).
template <class Cfg, int R>
using RowsCfg = DmaCfg<32 * R, Cfg::BN, Cfg::BK, Cfg::STAGES, Cfg::WM, Cfg::WN, Cfg::CPA, Cfg::CPB, Cfg::PIPE,
                       Cfg::EPI_PARTS, Cfg::APAIR ? 1 : 0, Cfg::BSTAGES == Cfg::STAGES ? 0 : Cfg::BSTAGES>;

// LDS of the expert tiles of a kernel: the largest over its tile heights.
template <int BN, int WAVES, int STAGES, int R>
constexpr int chunk_lds_bytes() {
  if constexpr (R == 1) {
    return ChunkCfg<1, BN, WAVES, STAGES>::kLdsAlloc;
  } else {
    constexpr int a = ChunkCfg<R, BN, WAVES, STAGES>::kLdsAlloc;
    constexpr int b = chunk_lds_bytes<BN, WAVES, STAGES, R - 1>();
    return a > b ? a : b;
  }
}

constexpr int max_int(int a, int b) { return a > b ? a : b; }

// f(integral_constant<int, R>) for the chunk's R in 1 .. RMAX.
template <int RMAX, class F>
__device__ __forceinline__ void with_groups(int groups, F&& f) {
  static_for<1, RMAX + 1>([&](auto rc) {
    constexpr int R = decltype(rc)::value;
    if (groups == R) f(rc);
  });
}

// ------------------------------------------------------------------ SDD ---

template <class Cfg>
struct SddChunkSrc {
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

struct SddArgs {
  const uint16_t* x;
  const uint16_t* w1;
  const int32_t* row_token;
  uint16_t* out;
  int32_t num_tokens, d_model, ffn_dim;
  int32_t apply_gelu;
};

template <class Cfg>
__device__ __forceinline__ void sdd_chunk_tile(uint8_t* __restrict__ lds, const SddArgs& a, const Chunk& ch, int n0) {
  using ML = DmaMainloop<Cfg>;
  SddChunkSrc<Cfg> src;
  src.x_rsrc = make_rsrc(a.x, static_cast<uint32_t>(a.num_tokens) * static_cast<uint32_t>(a.d_model) * 2u);
  src.w_rsrc = make_rsrc(a.w1 + static_cast<int64_t>(ch.expert) * a.d_model * a.ffn_dim,
                         static_cast<uint32_t>(a.d_model) * static_cast<uint32_t>(a.ffn_dim) * 2u);
  src.b_step_bytes = static_cast<uint32_t>(Cfg::BK) * static_cast<uint32_t>(a.ffn_dim) * 2u;
  const ADmaPos<Cfg> ap;
#pragma unroll
  for (int q = 0; q < Cfg::kAInstr; ++q) {
    const int j = ap.row[q];  // row of the chunk; rows past BM belong to the rounded-up DMA area
    const int32_t tok = j < ch.rows ? a.row_token[ch.row0 + j] : -1;
    src.a_off[q] = (tok >= 0 && tok < a.num_tokens)
                       ? static_cast<uint32_t>(tok) * static_cast<uint32_t>(a.d_model) * 2u + ap.chunk[q] * 16u
                       : kOutOfRange;
  }
  const BDmaPos<Cfg> bp;
#pragma unroll
  for (int q = 0; q < Cfg::kBInstr; ++q)
    src.b_off[q] = (static_cast<uint32_t>(bp.row[q]) * a.ffn_dim + n0 + bp.col[q]) * 2u;

  typename ML::Acc acc;
  ML::run(lds, src, a.d_model / Cfg::BK, acc);

  // Padded row p -> row block p / 128, whose blocks are (p / 128) * F/128 + f/128.
  const int64_t ffn_blocks = a.ffn_dim / kBS;
  static_for<0, Cfg::EPI_PARTS>([&](auto pc) {
    constexpr int P = decltype(pc)::value;
    if (a.apply_gelu)
      ML::template stage_part<P>(lds, acc, [](float v) { return gelu_erf_fast(v); });
    else
      ML::template stage_part<P>(lds, acc, [](float v) { return v; });
    ML::for_each_staged_chunk(lds, [&](int m, int col, u32x4_t v) {
      const int p = ch.row0 + P * ML::kPartRows + m;
      const int f = n0 + col;
      *reinterpret_cast<u32x4_t*>(a.out + ((p / kBS) * ffn_blocks + f / kBS) * (kBS * kBS) + (p % kBS) * kBS +
                                  (f % kBS)) = v;
    });
  });
}

// Expert tiles of the DSD (defined below): 256 columns, chunks of up to 256
// rows, 4 waves; for a reduction of F >= 8192, 8 waves (as sb_dsd's
// row-block tiles) and a last piece of up to 64 rows joined to the chunk
// before it (tiles of up to 320 rows; with 4 waves the 320 accumulators of
// such a tile spill). The SDD's choice follows the DSD's, so both are
// needed here.
// The DSD's expert tiles need a reduction of at least kDsdExpertMinF (48
// K steps): over shorter ones the 256 x 256 tile's fixed costs (ring fill,
// a 256-row epilogue) outweigh the W2 traffic it saves, and the 128 x 512
// row-block tiles are faster even with balanced routing (F = 768: 187.1
// against 160.3 us at T = 16384; F = 1024: 116.6 against 102.5 us at
// T = 8192, D = 2048), while from F = 1536 on they are even or slower.
constexpr int kDsdBN = 256, kDsdStages = 4, kDsdDeepF = 8192, kDsdExpertMinF = 1536;
template <int WAVES>
constexpr int dsd_rmax() { return WAVES == 8 ? 10 : 8; }

// Expert tiles of the SDD: 8 waves, 512 columns, chunks of up to 192 rows;
// tiles of up to 128 rows have a 4-stage ring (4 x 40 KB fits the 160 KB),
// 160-row tiles a split one (2 A slots of 16 KB, 4 B stages of 32 KB), and
// 192-row tiles a 3-stage ring.
constexpr int kSddBN = 512, kSddWaves = 8, kSddRmax = 6, kSddStages = 3;
template <int R>
using SddChunkCfg = std::conditional_t<
    (R <= 4), ChunkCfg<R, kSddBN, kSddWaves, 4>,
    std::conditional_t<(R == 5), DmaCfg<160, kSddBN, 32, 2, 1, kSddWaves, 0, 2, 5, 1, 0, 4>,
                       ChunkCfg<R, kSddBN, kSddWaves, kSddStages>>>;
static_assert(SddChunkCfg<5>::kLdsAlloc <= 160 * 1024, "LDS");

template <class CfgB>
__global__ void __launch_bounds__(64 * kSddWaves)
    sdd_layer_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                     const int32_t* __restrict__ row_token, const int32_t* __restrict__ row_block_expert,
                     const int32_t* __restrict__ row_offsets, const int32_t* __restrict__ tokens_per_expert,
                     const int32_t* __restrict__ padded_offsets, uint16_t* __restrict__ out, int32_t num_tokens,
                     int32_t d_model, int32_t ffn_dim, int32_t num_experts, int32_t max_row_blocks,
                     int32_t apply_gelu, int32_t group, int32_t force, int32_t dsd_grid, int32_t cus_per_xcd,
                     int32_t tail_slack) {
  static_assert(CfgB::kThreads == 64 * kSddWaves && CfgB::BM == kBS, "row-block tiles: 128 rows, same workgroup");
  using CfgH = SddHalfTile;
  static_assert(CfgH::kThreads == CfgB::kThreads && 2 * CfgH::BN == CfgB::BN, "half tiles: same workgroup");
  __shared__ __attribute__((aligned(1024)))
  uint8_t lds[max_int(max_int(chunk_lds_bytes<kSddBN, kSddWaves, kSddStages, kSddRmax>(),
                               chunk_lds_bytes<kSddBN, kSddWaves, 4, 4>()),
                       max_int(CfgB::kLdsAlloc, CfgH::kLdsAlloc))];
  // Workgroups past both tilings' tiles leave before the summary: every
  // chunk starts a row block of its own, so there are at most live row
  // blocks x slices tiles either way, numbered up to kNumXcd - 1 chunk rows
  // past them by the XCD deal, plus the split halves of a short last round.
  // The counts are loaded alongside padded_offsets[E], ahead of the exit test.
  const int32_t first = expert_counts(tokens_per_expert, num_experts, 0);
  const int live_rb = __builtin_amdgcn_readfirstlane(padded_offsets[num_experts]) / kBS;
  if (static_cast<int>(blockIdx.x) >= (live_rb + kNumXcd) * (ffn_dim / kSddBN) + tail_slack) return;
  const LayoutSummary sum =
      summarize_layout<kSddRmax, 4, dsd_rmax<4>(), dsd_rmax<8>()>(tokens_per_expert, num_experts, first);
  const SddArgs a{x, w1, row_token, out, num_tokens, d_model, ffn_dim, apply_gelu};
  // The DSD's own choice (dsd_layer_kernel): its expert tiles when the
  // routing is balanced, F >= kDsdExpertMinF and its grid of dsd_grid
  // workgroups holds them all.
  const bool dsd_expert =
      force == 1 || (ffn_dim >= kDsdExpertMinF && expert_stage_runs(sum, num_experts, kGateDsd, force) &&
                     static_cast<int64_t>(ffn_dim >= kDsdDeepF ? sum.chunks_d : sum.chunks_c) * (d_model / kDsdBN) <=
                         dsd_grid);
  if (!(expert_stage_runs(sum, num_experts, kGateSdd, force, ffn_dim / kSddBN, cus_per_xcd * kNumXcd) &&
        dsd_expert)) {
    // Row blocks: the chunks of up to 128 rows are the live row blocks, in
    // order; every row is computed and written (padding rows read as zeros),
    // except past the last 32-row group of an expert of at most 96 rows when
    // the 4-wave DSD follows, which reads no further. The tiles of a short
    // last round run as column halves (split_tail).
    const int blocks = sum.chunks_b;
    const int slices = ffn_dim / CfgB::BN;
    const TailTile tt = split_tail(static_cast<int>(blockIdx.x), blocks * slices, cus_per_xcd);
    if (tt.tile >= blocks * slices) return;
    int rb, slice;
    tile_coords(tt.tile, blocks, slices, group, &rb, &slice);
    if (rb >= blocks || rb >= max_row_blocks) return;
    const int32_t expert = __builtin_amdgcn_readfirstlane(row_block_expert[rb]);
    if (expert < 0 || expert >= num_experts) return;
    Chunk ch{expert, rb * kBS, kBS, 4};
    const int32_t n = __builtin_amdgcn_readfirstlane(tokens_per_expert[expert]);
    if (ffn_dim < kDsdDeepF && n > 0 && n <= 3 * 32) {
      // An expert of one row block whose 4-wave DSD reads its real 32-row
      // groups only: compute and write those.
      ch.rows = n;
      ch.groups = (n + 31) / 32;
      if (tt.half < 0) {
        with_groups<3>(ch.groups, [&](auto rc) {
          sdd_chunk_tile<SddChunkCfg<decltype(rc)::value>>(lds, a, ch, slice * CfgB::BN);
        });
      } else if (ch.groups <= 2) {
        // The half tile's two rows of waves take an even number of groups.
        ch.groups = 2;
        sdd_chunk_tile<RowsCfg<CfgH, 2>>(lds, a, ch, slice * CfgB::BN + tt.half * CfgH::BN);
      } else {
        ch.groups = 4;
        sdd_chunk_tile<CfgH>(lds, a, ch, slice * CfgB::BN + tt.half * CfgH::BN);
      }
      return;
    }
    if (tt.half < 0)
      sdd_chunk_tile<CfgB>(lds, a, ch, slice * CfgB::BN);
    else
      sdd_chunk_tile<CfgH>(lds, a, ch, slice * CfgB::BN + tt.half * CfgH::BN);
    return;
  }
  // Expert tiles. When every expert is one chunk, the chunks are dealt to
  // the XCDs largest first (balanced_chunk_tile); an expert of several
  // chunks keeps them on one XCD, where they share its W1 columns in L2
  // (xcd_remap and groups of chunks x slices).
  const int chunks = sum.chunks_a;
  const int slices = ffn_dim / kSddBN;
  Chunk ch;
  int n0_slice = 0;
  if (chunks == sum.active) {
    int rank, slice;
    if (!balanced_chunk_tile(static_cast<int>(blockIdx.x), chunks, slices, &rank, &slice)) return;
    int32_t hist[kSddRmax + 1];
    single_chunk_hist<kSddRmax>(tokens_per_expert, num_experts, first, hist);
    ch = find_single_chunk_by_size<kSddRmax>(tokens_per_expert, num_experts, rank, first, hist);
    n0_slice = slice;
  } else {
    // Groups of `group` chunks x slices (tile_coords), largest chunks first
    // inside each group (lpt_group_tile).
    const int tile = xcd_remap(static_cast<int>(blockIdx.x), chunks * slices);
    if (tile >= chunks * slices) return;
    const int per_group = group * slices;
    const int g0 = (tile / per_group) * group;
    const int G = min(group, chunks - g0);
    const uint32_t big = big_chunks_of_group<kSddRmax>(tokens_per_expert, num_experts, g0, G, first);
    int pos, slice;
    lpt_group_tile(tile - (g0 / group) * per_group, G, slices, big, &pos, &slice);
    ch = find_chunk<kSddRmax>(tokens_per_expert, num_experts, __builtin_amdgcn_readfirstlane(g0 + pos), first);
    n0_slice = __builtin_amdgcn_readfirstlane(slice);
  }
  // Not a routing layout (the chunk would leave the buffers): skip it.
  if (ch.expert < 0 || ch.row0 < 0 || ch.groups < 1 || ch.groups > kSddRmax ||
      ch.row0 + 32 * ch.groups > max_row_blocks * kBS)
    return;
  with_groups<kSddRmax>(ch.groups, [&](auto rc) {
    constexpr int R = decltype(rc)::value;
    sdd_chunk_tile<SddChunkCfg<R>>(lds, a, ch, n0_slice * kSddBN);
  });
}

// The SDD for F % 512 != 0: 256-wide tiles over row-block pairs
// (expert_chunks.hpp). A pair is one 256 x 256 tile of 8 waves (two rows of
// 4, 128 x 64 each), so each W1 slice is streamed once per two row blocks
// of an expert instead of once per row block; a single is the per-row-block
// kernel's 128 x 256 tile. XCD x takes the x-th eighth of the pairs and the
// x-th eighth of the singles, each kind in expert order: every XCD gets the
// same mix of the two tile sizes (so no XCD's rounds are all pairs, which
// left its singles a round of their own), and an expert's units stay on a
// few neighbouring XCDs, which then stream its W1 from HBM once each. An XCD
// runs its pairs, then its singles, so the tiles handed to the CUs that
// free up last are the short ones; a unit's slices run side by side
// (sharing its x rows), and so do an expert's pairs (sharing its W1
// slices). Every padded row that a DSD tiling reads is written.
using SddPairTile = DmaCfg<256, 256, 32, 4, 2, 4, 0, 2, 5, 1, 1>;

template <class CfgP, class CfgS, class CfgSH>
__global__ void __launch_bounds__(CfgP::kThreads)
    sdd_pair_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ w1,
                    const int32_t* __restrict__ row_token, const int32_t* __restrict__ tokens_per_expert,
                    const int32_t* __restrict__ padded_offsets, uint16_t* __restrict__ out, int32_t num_tokens,
                    int32_t d_model, int32_t ffn_dim, int32_t num_experts, int32_t max_row_blocks,
                    int32_t apply_gelu, int32_t cus_per_xcd) {
  static_assert(CfgP::kThreads == CfgS::kThreads && CfgP::BN == CfgS::BN, "one workgroup and slice width");
  static_assert(CfgSH::kThreads == CfgS::kThreads && 2 * CfgSH::BN == CfgS::BN && CfgSH::BK == CfgS::BK,
                "a single's column halves: same workgroup and K steps");
  static_assert(CfgP::BM == 2 * kBS && CfgS::BM == kBS && CfgSH::BM == kBS, "pairs and singles of row blocks");
  __shared__ __attribute__((aligned(1024))) uint8_t lds[max_int(CfgP::kLdsAlloc, max_int(CfgS::kLdsAlloc,
                                                                                         CfgSH::kLdsAlloc))];
  // Workgroup bid is XCD bid % 8's tile bid / 8 (units x slices, unit-major,
  // a short last round of singles as column halves; pair_tile_for).
  const int32_t first = expert_counts(tokens_per_expert, num_experts, 0);
  const int live_rb = __builtin_amdgcn_readfirstlane(padded_offsets[num_experts]) / kBS;
  const int slices = ffn_dim / CfgP::BN;
  if (static_cast<int>(blockIdx.x) / kNumXcd >= pair_units_per_xcd(live_rb) * slices + cus_per_xcd / 2) return;
  const PairCounts pc = pair_counts(tokens_per_expert, num_experts, first);
  bool single;
  int k, slice, half;
  if (!pair_tile_for(static_cast<int>(blockIdx.x), pc.pairs, pc.singles, slices, cus_per_xcd, &single, &k, &slice,
                     &half))
    return;
  const Chunk ch = find_pair_unit(tokens_per_expert, num_experts, single, k, first);
  // Not a routing layout (the unit would leave the buffers): skip it.
  if (ch.expert < 0 || ch.expert >= num_experts || ch.row0 < 0 || ch.rows < 1 ||
      ch.row0 + 32 * ch.groups > max_row_blocks * kBS)
    return;
  const SddArgs a{x, w1, row_token, out, num_tokens, d_model, ffn_dim, apply_gelu};
  if (ch.groups == CfgP::BM / 32) {
    sdd_chunk_tile<CfgP>(lds, a, ch, slice * CfgP::BN);
    return;
  }
  // A single of an expert of one row block of at most 64 rows, whose 4-wave
  // DSD reads its real 32-row groups only: its first two groups.
  const int32_t n = __builtin_amdgcn_readfirstlane(tokens_per_expert[ch.expert]);
  const bool cut = ffn_dim < kDsdDeepF && n > 0 && n <= 64;
  if (cut) {
    Chunk c2 = ch;
    c2.rows = n;
    c2.groups = 2;
    if (half < 0)
      sdd_chunk_tile<RowsCfg<CfgS, 2>>(lds, a, c2, slice * CfgS::BN);
    else
      sdd_chunk_tile<RowsCfg<CfgSH, 2>>(lds, a, c2, slice * CfgS::BN + half * CfgSH::BN);
  } else if (half < 0) {
    sdd_chunk_tile<CfgS>(lds, a, ch, slice * CfgS::BN);
  } else {
    sdd_chunk_tile<CfgSH>(lds, a, ch, slice * CfgS::BN + half * CfgSH::BN);
  }
}

// ------------------------------------------------------------------ DSD ---

// A: the chunk's rows of H, read in place. All of H is one buffer; lane row
// j of the chunk sits in row block row0/128 + j/128 at row j % 128, so its
// offset from the chunk's first block of the K step is fixed per lane, and
// the step moves the scalar offset (4 steps of 32 per 128-wide block).
template <class Cfg>
struct DsdChunkSrc {
  static constexpr int kStepsPerBlock = kBS / Cfg::BK;
  __amdgpu_buffer_rsrc_t h_rsrc, w_rsrc;
  uint32_t h_base;  // byte offset of the chunk's first H block
  uint32_t w_step_bytes, n0_bytes;
  uint32_t a_off[Cfg::kAInstr];
  uint32_t b_off[Cfg::kBInstr];
  __device__ __forceinline__ uint32_t a_voff(int q) const { return a_off[q]; }
  __device__ __forceinline__ uint32_t b_voff(int q) const { return b_off[q]; }
  __device__ __forceinline__ void a_src(int t, __amdgpu_buffer_rsrc_t* r, uint32_t* s) const {
    *r = h_rsrc;
    *s = h_base + static_cast<uint32_t>(t / kStepsPerBlock) * (kBS * kBS * 2) +
         static_cast<uint32_t>(t % kStepsPerBlock) * (Cfg::BK * 2);
  }
  __device__ __forceinline__ void b_src(int t, __amdgpu_buffer_rsrc_t* r, uint32_t* s) const {
    *r = w_rsrc;
    *s = static_cast<uint32_t>(t) * w_step_bytes + n0_bytes;
  }
};

struct DsdArgs {
  const uint16_t* h;
  const uint16_t* w2;
  uint16_t* out;
  int64_t h_bytes;
  int32_t ffn_dim, d_model;
};

template <class Cfg>
__device__ __forceinline__ void dsd_chunk_tile(uint8_t* __restrict__ lds, const DsdArgs& a, const Chunk& ch, int n0) {
  using ML = DmaMainloop<Cfg>;
  const uint32_t ffn_blocks = static_cast<uint32_t>(a.ffn_dim / kBS);
  DsdChunkSrc<Cfg> src;
  src.h_rsrc = make_rsrc(a.h, static_cast<uint32_t>(a.h_bytes));
  src.h_base = static_cast<uint32_t>(ch.row0 / kBS) * ffn_blocks * (kBS * kBS * 2);
  src.w_rsrc = make_rsrc(a.w2 + static_cast<int64_t>(ch.expert) * a.ffn_dim * a.d_model,
                         static_cast<uint32_t>(a.ffn_dim) * static_cast<uint32_t>(a.d_model) * 2u);
  src.w_step_bytes = static_cast<uint32_t>(Cfg::BK) * static_cast<uint32_t>(a.d_model) * 2u;
  src.n0_bytes = static_cast<uint32_t>(n0) * 2u;
  const ADmaPos<Cfg> ap;
#pragma unroll
  for (int q = 0; q < Cfg::kAInstr; ++q) {
    const uint32_t j = static_cast<uint32_t>(ap.row[q]);
    src.a_off[q] = static_cast<int>(j) < ch.rows
                       ? ((j / kBS) * ffn_blocks * (kBS * kBS) + (j % kBS) * kBS) * 2u + ap.chunk[q] * 16u
                       : kOutOfRange;
  }
  const BDmaPos<Cfg> bp;
#pragma unroll
  for (int q = 0; q < Cfg::kBInstr; ++q)
    src.b_off[q] = (static_cast<uint32_t>(bp.row[q]) * a.d_model + bp.col[q]) * 2u;

  typename ML::Acc acc;
  ML::run(lds, src, a.ffn_dim / Cfg::BK, acc);

  ML::stage_tile(lds, acc, [](float v) { return v; });
  uint16_t* out_tile = a.out + static_cast<int64_t>(ch.row0) * a.d_model + n0;
  ML::for_each_staged_chunk(lds, [&](int m, int col, u32x4_t v) {
    if (m < ch.rows) *reinterpret_cast<u32x4_t*>(out_tile + static_cast<int64_t>(m) * a.d_model + col) = v;
  });
}

// Expert tiles of the DSD: 4 waves, 256 columns, chunks of up to 256 rows.
// Row-block tiles: 4 waves, 128 x CfgB::BN, every row of the row block read
// and written, as sb_dsd's default tile does, except for an expert of one
// row block, whose tile stops at its last real 32-row group (with few
// tokens most row blocks are such experts, and mostly padding: 93% of the
// rows at T = 512 of config 5); they run on the same tile code as the
// expert chunks (one H buffer, K steps through the row block's own F/128
// blocks, as the routing layout stores them).

template <class CfgB, int WAVES>
__global__ void __launch_bounds__(64 * WAVES)
    dsd_layer_kernel(const uint16_t* __restrict__ h, const uint16_t* __restrict__ w2,
                     const int32_t* __restrict__ tokens_per_expert, const int32_t* __restrict__ padded_offsets,
                     const int32_t* __restrict__ row_block_expert, uint16_t* __restrict__ out, int64_t h_bytes,
                     int32_t num_experts, int32_t ffn_dim, int32_t d_model, int32_t max_row_blocks, int32_t group,
                     int32_t force, int32_t tile_grid, int32_t cus_per_xcd, int32_t tail_slack) {
  static_assert(CfgB::kThreads == 64 * WAVES && CfgB::BM == kBS, "row-block tiles: 128 rows, same workgroup");
  using CfgH = DsdCfg<4, CfgB::BN / 2, WAVES, kDsdStages>;
  constexpr int kRmax = dsd_rmax<WAVES>();
  __shared__ __attribute__((aligned(1024)))
  uint8_t lds[max_int(chunk_lds_bytes<kDsdBN, WAVES, kDsdStages, kRmax>(), max_int(CfgB::kLdsAlloc, CfgH::kLdsAlloc))];
  // As in the SDD: at most live row blocks x D/256 tiles either way, plus
  // the split halves of a short last round.
  const int32_t first = expert_counts(tokens_per_expert, num_experts, 0);
  const int live_rb = __builtin_amdgcn_readfirstlane(padded_offsets[num_experts]) / kBS;
  if (static_cast<int>(blockIdx.x) >= live_rb * (d_model / kDsdBN) + tail_slack) return;
  const LayoutSummary sum = summarize_layout<kRmax, 4>(tokens_per_expert, num_experts, first);
  const DsdArgs a{h, w2, out, h_bytes, ffn_dim, d_model};
  // Expert tiles for balanced routing over a reduction of at least
  // kDsdExpertMinF. The grid may hold fewer workgroups than expert tiles
  // (see the launch): then the row blocks take the stage.
  const bool fits = static_cast<int64_t>(sum.chunks_a) * (d_model / kDsdBN) <= static_cast<int64_t>(tile_grid);
  const bool chosen = ffn_dim >= kDsdExpertMinF && expert_stage_runs(sum, num_experts, kGateDsd, force) && fits;
  if (!(chosen || force == 1)) {
    // Row blocks: the chunks of up to 128 rows are the live row blocks, in order.
    // The tiles of a short last round run as column halves (split_tail).
    const int blocks = sum.chunks_b;
    const int slices = d_model / CfgB::BN;
    const TailTile tt = split_tail(static_cast<int>(blockIdx.x), blocks * slices, cus_per_xcd);
    if (tt.tile >= blocks * slices) return;
    int rb, slice;
    tile_coords(tt.tile, blocks, slices, group, &rb, &slice);
    if (rb >= blocks || rb >= max_row_blocks) return;
    const int32_t expert = __builtin_amdgcn_readfirstlane(row_block_expert[rb]);
    if (expert < 0 || expert >= num_experts) return;
    Chunk ch{expert, rb * kBS, kBS, 4};
    if constexpr (WAVES == 4) {
      // An expert of one row block: its real 32-row groups only. No other
      // row block shares its W2 slice, so its tile running ahead of the
      // others costs no L2 sharing (skipping padding rows in every row
      // block was slower at the fine-grained shape for that reason). The
      // padding rows of y are then left unwritten; nothing reads them.
      const int32_t n = __builtin_amdgcn_readfirstlane(tokens_per_expert[expert]);
      if (n > 0 && n < kBS) {
        ch.rows = n;
        ch.groups = (n + 31) / 32;
      }
      with_groups<4>(ch.groups, [&](auto rc) {
        constexpr int R = decltype(rc)::value;
        if (tt.half < 0)
          dsd_chunk_tile<RowsCfg<CfgB, R>>(lds, a, ch, slice * CfgB::BN);
        else
          dsd_chunk_tile<RowsCfg<CfgH, R>>(lds, a, ch, slice * CfgB::BN + tt.half * CfgH::BN);
      });
    } else {
      if (tt.half < 0)
        dsd_chunk_tile<CfgB>(lds, a, ch, slice * CfgB::BN);
      else
        dsd_chunk_tile<CfgH>(lds, a, ch, slice * CfgB::BN + tt.half * CfgH::BN);
    }
    return;
  }
  const int chunks = sum.chunks_a;
  const int slices = d_model / kDsdBN;
  const int tile = xcd_remap(static_cast<int>(blockIdx.x), chunks * slices);
  int c, slice;
  if (chunks == sum.active || chunks > 32 * kNumXcd) {
    tile_coords(tile, chunks, slices, group, &c, &slice);
  } else {
    // Experts of several chunks: groups of ceil(chunks / 8) chunks x all
    // slices, about one XCD's share each, largest chunks first inside each
    // group (lpt_group_tile: an expert's merged last chunk of up to 320
    // rows, about 1.25 times a 256-row tile's time, runs in the first round,
    // so no CU runs two of them one after the other).
    if (tile >= chunks * slices) return;
    const int per = (chunks + kNumXcd - 1) / kNumXcd;
    const int g0 = (tile / (per * slices)) * per;
    const int G = min(per, chunks - g0);
    const uint32_t big = big_chunks_of_group<kRmax>(tokens_per_expert, num_experts, g0, G, first);
    int pos;
    lpt_group_tile(tile - g0 * slices, G, slices, big, &pos, &slice);
    c = __builtin_amdgcn_readfirstlane(g0 + pos);
    slice = __builtin_amdgcn_readfirstlane(slice);
  }
  if (c >= chunks) return;
  const Chunk ch = find_chunk<kRmax>(tokens_per_expert, num_experts, c, first);
  if (ch.expert < 0 || ch.row0 < 0 || ch.groups < 1 || ch.groups > kRmax ||
      ch.row0 + 32 * ch.groups > max_row_blocks * kBS)
    return;
  // Nine row groups run as ten (the tenth reads zeros): in one row of 8
  // waves, nine groups read 11 LDS fragments per 9 MFMAs against 9 per 10
  // split between two rows of 4.
  with_groups<kRmax>(ch.groups == 9 ? 10 : ch.groups, [&](auto rc) {
    constexpr int R = decltype(rc)::value;
    if constexpr (R != 9) {
      dsd_chunk_tile<DsdCfg<R, kDsdBN, WAVES, kDsdStages>>(lds, a, ch, slice * kDsdBN);
    }
  });
}

// --------------------------------------------------------------- launch ---

// CUs of the current device, read once per device.
int device_cus(int* cus_out) {
  constexpr int kMaxDevices = 64;
  static int cus[kMaxDevices] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return fail(SB_ERR_HIP, "dsd_experts: no current device");
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
      return fail(SB_ERR_HIP, "dsd_experts: cannot read the CU count");
    cus[dev] = n;
  }
  *cus_out = cus[dev];
  return SB_OK;
}

// Workgroups of dsd_layer_kernel: every row-block tile (the 512- or
// 256-wide tile of sb_dsd's default shape), or every expert tile up to four
// per CU if they can be more, and no more: workgroups past the chosen
// tiling's tiles still read the counts before they return. Expert e's
// ceil(n_e / 256) chunks are at most 1 + (n_e - 1) / 256, so there are at
// most min(E, N) + N / 256 of them for N routed rows, and N is at most
// 128 max_row_blocks - 127 E + 127 (max_row_blocks = floor((N + 127 E) /
// 128)). Expert tiles the grid cannot hold leave the stage to the row
// blocks (on the device). A function of the layout's sizes only, so the
// SDD's launch computes the same number for its own choice.
int dsd_layer_grid(int64_t max_row_blocks, int64_t num_experts, int64_t d_model, int32_t force, int64_t* grid) {
  int cus = 0;
  if (const int rc = device_cus(&cus)) return rc;
  const int64_t rows = std::min(max_row_blocks * kBS, std::max<int64_t>(0, max_row_blocks * kBS - (kBS - 1) * num_experts) +
                                                          (kBS - 1));
  const int64_t chunk_bound =
      std::min(max_row_blocks, std::min(num_experts, rows) + rows / Chunking<dsd_rmax<4>()>::kRows);
  static_assert(Chunking<dsd_rmax<4>()>::kRows == Chunking<dsd_rmax<8>()>::kRows, "one bound for both");
  const int64_t expert_tiles = chunk_bound * (d_model / kDsdBN);
  const int64_t forced_expert = force == 1 ? expert_tiles : 0;
  const int64_t rb_bn = d_model % 512 == 0 ? 512 : 256;
  *grid = std::max({std::min<int64_t>(expert_tiles, 4 * static_cast<int64_t>(cus)), forced_expert,
                    max_row_blocks * (d_model / rb_bn)});
  return SB_OK;
}

template <class CfgB>
int launch_sdd_layer(const void* x, const void* w1, const int32_t* row_token, const int32_t* row_block_expert,
                     const int32_t* row_offsets, const int32_t* tokens_per_expert, const int32_t* padded_offsets,
                     void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim, int64_t num_experts,
                     int64_t max_row_blocks, int32_t apply_gelu, int32_t force, hipStream_t stream) {
  // Both tilings have at most max_row_blocks x F/512 tiles (every chunk
  // starts a row block of its own).
  static_assert(CfgB::BN == kSddBN, "one grid for both tilings");
  if (!reduction_fits<CfgB>(d_model) || !reduction_fits<SddHalfTile>(d_model) ||
      !reduction_fits<ChunkCfg<4, kSddBN, kSddWaves, 4>>(d_model))
    return fail(SB_ERR_INVALID, "sdd_experts: D (%lld) is not a whole number of the tiles' K steps",
                static_cast<long long>(d_model));
  const int64_t tiles = max_row_blocks * (ffn_dim / kSddBN);
  int64_t dsd_grid = 0;  // no DSD expert tiles for D % 256 != 0
  if (d_model % kDsdBN == 0)
    if (const int rc = dsd_layer_grid(max_row_blocks, num_experts, d_model, force, &dsd_grid)) return rc;
  int cus = 0;
  if (const int rc = device_cus(&cus)) return rc;
  const int64_t slack = split_tail_slack(cus) + kNumXcd * (ffn_dim / kSddBN);
  sdd_layer_kernel<CfgB><<<static_cast<uint32_t>(tiles + slack), 64 * kSddWaves, 0, stream>>>(
      static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w1), row_token, row_block_expert, row_offsets,
      tokens_per_expert, padded_offsets, static_cast<uint16_t*>(out), static_cast<int32_t>(num_tokens),
      static_cast<int32_t>(d_model), static_cast<int32_t>(ffn_dim), static_cast<int32_t>(num_experts),
      static_cast<int32_t>(max_row_blocks), apply_gelu, kTileGroup, force,
      static_cast<int32_t>(std::min<int64_t>(dsd_grid, 2147483647)), cus / kNumXcd, static_cast<int32_t>(slack));
  return check_launch("sdd_experts");
}

int dispatch_sdd_layer(const void* x, const void* w1, const int32_t* row_token, const int32_t* row_block_expert,
                       const int32_t* row_offsets, const int32_t* tokens_per_expert, const int32_t* padded_offsets,
                       void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim, int64_t num_experts,
                       int64_t max_row_blocks, int32_t apply_gelu, int32_t force, hipStream_t stream) {
  // The row-block tile is sb_sdd's for the shape (sdd_tile_for).
  if (sdd_tile_for(d_model, ffn_dim) == SddTile::kDeep)
    return launch_sdd_layer<SddDeepTile>(x, w1, row_token, row_block_expert, row_offsets, tokens_per_expert,
                                         padded_offsets, out, num_tokens, d_model, ffn_dim, num_experts,
                                         max_row_blocks, apply_gelu, force, stream);
  return launch_sdd_layer<SddWideTile>(x, w1, row_token, row_block_expert, row_offsets, tokens_per_expert,
                                       padded_offsets, out, num_tokens, d_model, ffn_dim, num_experts, max_row_blocks,
                                       apply_gelu, force, stream);
}

int launch_sdd_pairs(const void* x, const void* w1, const int32_t* row_token, const int32_t* tokens_per_expert,
                     const int32_t* padded_offsets, void* out, int64_t num_tokens, int64_t d_model, int64_t ffn_dim,
                     int64_t num_experts, int64_t max_row_blocks, int32_t apply_gelu, hipStream_t stream) {
  if (!reduction_fits<SddPairTile>(d_model) || !reduction_fits<SddNarrowTile>(d_model) ||
      !reduction_fits<SddNarrowHalfTile>(d_model))
    return fail(SB_ERR_INVALID, "sdd_experts: D (%lld) is not a whole number of the tiles' K steps",
                static_cast<long long>(d_model));
  int cus = 0;
  if (const int rc = device_cus(&cus)) return rc;
  const int cus_per_xcd = cus / kNumXcd;
  // Each XCD's positions: its tiles, plus up to half its CUs for a split
  // last round (pair_tile_for).
  const int64_t grid =
      int64_t{kNumXcd} *
      (int64_t{pair_units_per_xcd(static_cast<int>(max_row_blocks))} * (ffn_dim / SddPairTile::BN) + cus_per_xcd / 2);
  sdd_pair_kernel<SddPairTile, SddNarrowTile, SddNarrowHalfTile>
      <<<static_cast<uint32_t>(grid), SddPairTile::kThreads, 0, stream>>>(
          static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(w1), row_token, tokens_per_expert,
          padded_offsets, static_cast<uint16_t*>(out), static_cast<int32_t>(num_tokens),
          static_cast<int32_t>(d_model), static_cast<int32_t>(ffn_dim), static_cast<int32_t>(num_experts),
          static_cast<int32_t>(max_row_blocks), apply_gelu, cus_per_xcd);
  return check_launch("sdd_experts");
}

template <class CfgB, int WAVES>
int launch_dsd_layer(const void* h, const void* w2, const int32_t* tokens_per_expert, const int32_t* padded_offsets,
                     const int32_t* row_block_expert, void* out, int64_t max_row_blocks, int64_t num_experts,
                     int64_t num_copies, int64_t ffn_dim, int64_t d_model, int32_t force, hipStream_t stream) {
  static_assert(CfgB::BN == 512 || CfgB::BN == 256, "row-block tile widths of dsd_layer_grid");
  if (!reduction_fits<CfgB>(ffn_dim) || !reduction_fits<DsdCfg<4, kDsdBN, WAVES, kDsdStages>>(ffn_dim))
    return fail(SB_ERR_INVALID, "dsd_experts: F (%lld) is not a whole number of the tiles' K steps",
                static_cast<long long>(ffn_dim));
  int64_t tiles = 0;
  if (const int rc = dsd_layer_grid(max_row_blocks, num_experts, d_model, force, &tiles)) return rc;
  const int64_t h_bytes = max_row_blocks * (ffn_dim / kBS) * kBS * kBS * 2;
  int cus = 0;
  if (const int rc = device_cus(&cus)) return rc;
  const int64_t slack = split_tail_slack(cus);
  dsd_layer_kernel<CfgB, WAVES><<<static_cast<uint32_t>(tiles + slack), 64 * WAVES, 0, stream>>>(
      static_cast<const uint16_t*>(h), static_cast<const uint16_t*>(w2), tokens_per_expert, padded_offsets,
      row_block_expert, static_cast<uint16_t*>(out), h_bytes, static_cast<int32_t>(num_experts),
      static_cast<int32_t>(ffn_dim), static_cast<int32_t>(d_model), static_cast<int32_t>(max_row_blocks),
      kTileGroup, force, static_cast<int32_t>(tiles), cus / kNumXcd, static_cast<int32_t>(slack));
  return check_launch("dsd_experts");
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" int sb_sdd_experts(const void* x, const void* w1, const int32_t* row_token,
                              const int32_t* row_block_expert, const int32_t* row_offsets,
                              const int32_t* tokens_per_expert, const int32_t* padded_offsets, void* out,
                              int64_t num_tokens, int64_t d_model, int64_t ffn_dim, int64_t num_experts,
                              int64_t max_row_blocks, int32_t apply_gelu, void* stream) {
  constexpr int64_t kI32Max = 2147483647;
  if (max_row_blocks < 0) return fail(SB_ERR_INVALID, "sdd_experts: negative row block count");
  if (max_row_blocks == 0) return clear_ok();
  if (!x || !w1 || !row_token || !row_block_expert || !row_offsets || !tokens_per_expert || !padded_offsets || !out)
    return fail(SB_ERR_INVALID, "sdd_experts: null buffer");
  if (!aligned16(x) || !aligned16(w1) || !aligned16(out))
    return fail(SB_ERR_INVALID, "x and w1 must be 16-byte aligned");
  if (d_model <= 0 || d_model % 64 != 0)
    return fail(SB_ERR_INVALID, "sdd needs D (%lld) to be a multiple of 64", static_cast<long long>(d_model));
  if (ffn_dim <= 0 || ffn_dim % 256 != 0)
    return fail(SB_ERR_INVALID, "sdd needs F (%lld) to be a multiple of 256", static_cast<long long>(ffn_dim));
  if (num_tokens <= 0 || num_tokens > kI32Max || num_experts <= 0 || num_experts > kMaxExperts)
    return fail(SB_ERR_INVALID, "sdd_experts: bad token or expert count");
  if (ffn_dim * d_model > kI32Max || max_row_blocks * kBS > kI32Max ||
      (max_row_blocks + kNumXcd) * (ffn_dim / kBS) > kI32Max - 65536)
    return fail(SB_ERR_INVALID, "problem too large");
  const int32_t force = expert_gate_override();
  // The layer kernels read x and W1[e] through 32-bit buffer offsets; x of
  // 2 GiB or more, or one expert's W1 of 2 GiB or more, go to the
  // per-row-block kernel, which gathers x with 64-bit addresses, as do
  // forced row blocks. F % 512 != 0 takes the row-block pairs (256 wide),
  // other widths the layer kernel (512 wide). The real rows are the same
  // bits every way.
  const bool offsets_fit = !sdd_wide_x(num_tokens, d_model) && ffn_dim * d_model * 2 < (int64_t{1} << 31);
  if (force == 2 || !offsets_fit)
    return sb_sdd(x, w1, row_token, row_block_expert, row_offsets, out, num_tokens, d_model, ffn_dim, num_experts,
                  max_row_blocks, apply_gelu, stream);
  if (ffn_dim % kSddBN != 0) {
    const int rc = launch_sdd_pairs(x, w1, row_token, tokens_per_expert, padded_offsets, out, num_tokens, d_model,
                                    ffn_dim, num_experts, max_row_blocks, apply_gelu, as_stream(stream));
    return rc ? rc : clear_ok();
  }
  const int rc = dispatch_sdd_layer(x, w1, row_token, row_block_expert, row_offsets, tokens_per_expert, padded_offsets,
                                    out, num_tokens, d_model, ffn_dim, num_experts, max_row_blocks, apply_gelu, force,
                                    as_stream(stream));
  return rc ? rc : clear_ok();
}

extern "C" int sb_dsd_experts(const void* h, const void* w2, const int32_t* tokens_per_expert,
                              const int32_t* padded_offsets, const int32_t* row_block_expert,
                              const int32_t* row_offsets, const int32_t* col_indices, void* out,
                              int64_t max_row_blocks, int64_t num_experts, int64_t num_copies, int64_t ffn_dim,
                              int64_t d_model, void* stream) {
  constexpr int64_t kI32Max = 2147483647;
  if (max_row_blocks < 0) return fail(SB_ERR_INVALID, "dsd_experts: negative row block count");
  if (max_row_blocks == 0) return clear_ok();
  if (!h || !w2 || !tokens_per_expert || !padded_offsets || !row_block_expert || !row_offsets || !col_indices || !out)
    return fail(SB_ERR_INVALID, "dsd_experts: null buffer");
  if (!aligned16(h) || !aligned16(w2) || !aligned16(out)) return fail(SB_ERR_INVALID, "dsd_experts: unaligned buffer");
  if (num_experts <= 0 || num_experts > kMaxExperts) return fail(SB_ERR_INVALID, "dsd_experts: bad expert count");
  if (num_copies <= 0) return fail(SB_ERR_INVALID, "dsd_experts: bad copy count");
  if (ffn_dim <= 0 || ffn_dim % kBS != 0)
    return fail(SB_ERR_INVALID, "dsd_experts: F (%lld) must be a multiple of 128", static_cast<long long>(ffn_dim));
  if (d_model <= 0 || d_model % kDsdBN != 0)
    return fail(SB_ERR_INVALID, "dsd_experts: D (%lld) must be a multiple of 256", static_cast<long long>(d_model));
  // H is read through one buffer and each expert's W2 through another, both
  // with 32-bit offsets.
  if (max_row_blocks * (ffn_dim / kBS) * kBS * kBS * 2 >= (int64_t{1} << 31) ||
      ffn_dim * d_model * 2 >= (int64_t{1} << 31))
    return fail(SB_ERR_INVALID, "dsd_experts: H or one expert's W2 too large for 32-bit buffer offsets");
  if (max_row_blocks * kBS * d_model > (int64_t{1} << 62) || max_row_blocks * (d_model / kDsdBN) > kI32Max - 65536)
    return fail(SB_ERR_INVALID, "problem too large");
  const int32_t force = expert_gate_override();
  // Row blocks forced: exactly sb_dsd version 5 (its default tile).
  if (force == 2)
    return sb_dsd(h, w2, row_offsets, col_indices, out, max_row_blocks * (ffn_dim / kBS), num_experts * ffn_dim,
                  max_row_blocks, kBS, d_model, 0, stream);
  const hipStream_t s = as_stream(stream);
  // Row-block tile: sb_dsd's 128 x 512 tile (4 waves, or 8 for K >= 8192);
  // 128 x 256 when D % 512 != 0. The expert tiles take the same wave count.
  auto launch = [&](auto cfg, auto waves) {  // cfg: Tag<row-block config>
    return launch_dsd_layer<typename decltype(cfg)::type, decltype(waves)::value>(
        h, w2, tokens_per_expert, padded_offsets, row_block_expert, out, max_row_blocks, num_experts, num_copies,
        ffn_dim, d_model, force, s);
  };
  using W4 = std::integral_constant<int, 4>;
  using W8 = std::integral_constant<int, 8>;
  const bool wide = d_model % 512 == 0, deep = ffn_dim >= kDsdDeepF;
  const int rc = wide ? (deep ? launch(Tag<DsdCfg<4, 512, 8, 4>>{}, W8{})
                              : launch(Tag<DsdCfg<4, 512, 4, 4>>{}, W4{}))
                      : (deep ? launch(Tag<DsdCfg<4, 256, 8, 4>>{}, W8{})
                              : launch(Tag<DsdCfg<4, 256, 4, 4>>{}, W4{}));
  return rc ? rc : clear_ok();
}
