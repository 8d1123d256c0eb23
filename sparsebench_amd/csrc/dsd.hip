// DSD: block-sparse (BSR) x dense on gfx950 (the operation of the reference's
// csrc/dsd_v1.cu .. dsd_v5.cu, one kernel here for every version code).
//
//   out[r*bs + i, n] = sum_{p in [row_offsets[r], row_offsets[r+1])}
//                      sum_{kk < bs} blocks[p][i][kk] * w[col_indices[p]*bs + kk, n]
//
// One workgroup computes bs x BN outputs of one row block, walking its
// blocks in K steps of 64 (two per block at bs = 128, one at bs = 64) on the
// shared MFMA tile loop. Dead row blocks are skipped, or written as zeros
// when zero_dead_rows is set (the contract of the reference's versions 1-3).
// Tiles are row block first and spread over the XCDs in contiguous ranges,
// so a row block's column slices and an expert's row blocks share an L2.

#include <type_traits>

#include "dsd_tile.hpp"
#include "gemm_dma.hpp"
#include "gemm_tile.hpp"

namespace sb {
namespace {

template <class Cfg>
struct DsdLoader {
  using ML = Mainloop<Cfg>;
  using BRow = typename Cfg::BRow;
  static constexpr int kStepsPerBlock = Cfg::BM / Cfg::BK;
  const uint16_t* blocks;
  const uint16_t* w_cols;  // w + n0
  const int32_t* col_indices;
  int64_t d_model, w_rows;
  int32_t begin;

  // Block p and the K offset inside it of K step t.
  __device__ __forceinline__ void step(int t, int32_t* p, int* kin) const {
    *p = begin + t / kStepsPerBlock;
    *kin = (t % kStepsPerBlock) * Cfg::BK;
  }

  __device__ __forceinline__ void load_a(int t, const typename ML::LoadPos& pos, u32x4_t (&a)[Cfg::kAChunks]) const {
    int32_t p;
    int kin;
    step(t, &p, &kin);
    const uint16_t* blk = blocks + static_cast<int64_t>(p) * Cfg::BM * Cfg::BM + kin + pos.a_chunk * 8;
#pragma unroll
    for (int j = 0; j < Cfg::kAChunks; ++j)
      a[j] = *reinterpret_cast<const u32x4_t*>(blk + static_cast<int64_t>(pos.a_row[j]) * Cfg::BM);
  }

  __device__ __forceinline__ void load_b(int t, const typename ML::LoadPos& pos, BRow (&b)[8]) const {
    int32_t p;
    int kin;
    step(t, &p, &kin);
    const int64_t row0 = static_cast<int64_t>(col_indices[p]) * Cfg::BM;
    if (row0 < 0 || row0 + Cfg::BM > w_rows) {  // not a block of w: contributes nothing
#pragma unroll
      for (int r = 0; r < 8; ++r) b[r] = BRow{};
      return;
    }
    const uint16_t* src = w_cols + (row0 + kin + pos.b_kgroup * 8) * d_model + pos.b_col;
#pragma unroll
    for (int r = 0; r < 8; ++r) b[r] = load_vec<Cfg::NTB, BRow>(src + r * d_model);
  }
};

template <class Cfg>
__global__ void __launch_bounds__(Cfg::kThreads)
    dsd_kernel(const uint16_t* __restrict__ blocks, const uint16_t* __restrict__ w,
               const int32_t* __restrict__ row_offsets, const int32_t* __restrict__ col_indices,
               uint16_t* __restrict__ out, int64_t nnz, int64_t w_rows, int32_t num_row_blocks, int32_t d_model,
               int32_t num_slices, int32_t zero_dead_rows, int32_t group) {
  using ML = Mainloop<Cfg>;
  constexpr int BM = Cfg::BM, BN = Cfg::BN;
  __shared__ __attribute__((aligned(16))) uint16_t lds[Cfg::kLdsElems];

  const int live_rb = zero_dead_rows ? num_row_blocks : live_row_blocks(row_offsets, num_row_blocks);
  const int tile = xcd_remap(static_cast<int>(blockIdx.x), live_rb * num_slices);
  int rb, slice;
  tile_coords(tile, live_rb, num_slices, group, &rb, &slice);
  const int n0 = slice * BN;
  int32_t begin = row_offsets[rb];
  int32_t end = row_offsets[rb + 1];
  if (begin < 0 || end > nnz || end < begin) begin = end = 0;  // not a BSR row: treat as empty

  uint16_t* out_tile = out + static_cast<int64_t>(rb) * BM * d_model + n0;
  if (begin == end) {
    if (!zero_dead_rows) return;
    // BM x BN zeros, 16 bytes per store.
    constexpr int kChunksPerRow = BN / 8;
    for (int q = threadIdx.x; q < BM * kChunksPerRow; q += Cfg::kThreads) {
      const int r = q / kChunksPerRow, c = q % kChunksPerRow;
      *reinterpret_cast<u32x4_t*>(out_tile + static_cast<int64_t>(r) * d_model + c * 8) = u32x4_t{0u, 0u, 0u, 0u};
    }
    return;
  }

  DsdLoader<Cfg> ld;
  ld.blocks = blocks;
  ld.w_cols = w + n0;
  ld.col_indices = col_indices;
  ld.d_model = d_model;
  ld.w_rows = w_rows;
  ld.begin = begin;

  typename ML::Acc acc;
  ML::run(lds, ld, (end - begin) * DsdLoader<Cfg>::kStepsPerBlock, acc);

#pragma unroll
  for (int j = 0; j < Cfg::TN; ++j) {
    uint16_t* col = out_tile + ML::acc_col(j);
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
      for (int v = 0; v < 16; ++v) col[static_cast<int64_t>(ML::acc_row(i, v)) * d_model] = f32_to_bf16(acc[i][j][v]);
  }
}

template <class Cfg>
__global__ void __launch_bounds__(Cfg::kThreads)
    dsd_dma_kernel(const uint16_t* __restrict__ blocks, const uint16_t* __restrict__ w,
                   const int32_t* __restrict__ row_offsets, const int32_t* __restrict__ col_indices,
                   uint16_t* __restrict__ out, int64_t nnz, int64_t w_rows, int32_t num_row_blocks, int32_t d_model,
                   int32_t num_slices, int32_t zero_dead_rows, int32_t group) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg::kLdsAlloc];
  dsd_row_block_tile<Cfg>(lds, static_cast<int>(blockIdx.x), blocks, w, row_offsets, col_indices, out, nnz, w_rows,
                          num_row_blocks, d_model, num_slices, zero_dead_rows, group);
}

// Persistent form (DmaMainloop::run_tiles): about one workgroup per CU slot,
// each walking the tile list with stride gridDim.x through the same XCD
// remap and grouped order as the one-tile kernel. A dead tile with
// zero_dead_rows set is a tile of zero K steps: its epilogue writes zeros.
template <class Cfg>
struct DsdTiles {
  using ML = DmaMainloop<Cfg>;
  static constexpr int BM = Cfg::BM, BN = Cfg::BN;
  static constexpr int kStepsPerBlock = BM / Cfg::BK;
  struct Tile {
    int steps;
    int32_t begin;
    int32_t rb;
    int n0;
  };
  struct Src {
    const uint16_t* blocks;
    const uint16_t* w;
    const int32_t* col_indices;
    int64_t w_rows;
    int32_t d_model, begin;
    uint32_t n0_bytes;
    uint32_t a_off[Cfg::kAInstr];
    uint32_t b_off[Cfg::kBInstr];
    __device__ __forceinline__ void a_src(int t, __amdgpu_buffer_rsrc_t* r, uint32_t* s) const {
      const int32_t p = begin + t / kStepsPerBlock;
      *r = make_rsrc(blocks + static_cast<int64_t>(p) * BM * BM, BM * BM * 2);
      *s = static_cast<uint32_t>(t % kStepsPerBlock) * (Cfg::BK * 2);
    }
    __device__ __forceinline__ void b_src(int t, __amdgpu_buffer_rsrc_t* r, uint32_t* s) const {
      const int32_t p = begin + t / kStepsPerBlock;
      const int64_t row0 = static_cast<int64_t>(col_indices[p]) * BM;
      const bool ok = row0 >= 0 && row0 + BM <= w_rows;
      *r = make_rsrc(w + (ok ? row0 : 0) * d_model, ok ? static_cast<uint32_t>(BM) * d_model * 2u : 0u);
      *s = static_cast<uint32_t>(t % kStepsPerBlock) * (Cfg::BK * 2u) * static_cast<uint32_t>(d_model) + n0_bytes;
    }
    __device__ __forceinline__ uint32_t a_voff(int q) const { return a_off[q]; }
    __device__ __forceinline__ uint32_t b_voff(int q) const { return b_off[q]; }
  };

  const uint16_t* blocks;
  const uint16_t* w;
  const int32_t* row_offsets;
  const int32_t* col_indices;
  uint16_t* out;
  int64_t nnz, w_rows;
  int32_t num_row_blocks, d_model, num_slices, zero_dead_rows, group;
  int live_rb, live_tiles, vtile;
  uint32_t a_off[Cfg::kAInstr];
  uint32_t b_off[Cfg::kBInstr];

  __device__ __forceinline__ void init() {
    const ADmaPos<Cfg> ap;
#pragma unroll
    for (int q = 0; q < Cfg::kAInstr; ++q) a_off[q] = (ap.row[q] * BM + ap.chunk[q] * 8) * 2u;
    const BDmaPos<Cfg> bp;
#pragma unroll
    for (int q = 0; q < Cfg::kBInstr; ++q) b_off[q] = (static_cast<uint32_t>(bp.row[q]) * d_model + bp.col[q]) * 2u;
  }

  __device__ __forceinline__ Src source(const Tile& t) const {
    Src src;
    src.blocks = blocks;
    src.w = w;
    src.col_indices = col_indices;
    src.w_rows = w_rows;
    src.d_model = d_model;
    src.begin = t.begin;
    src.n0_bytes = static_cast<uint32_t>(t.n0) * 2u;
#pragma unroll
    for (int q = 0; q < Cfg::kAInstr; ++q) src.a_off[q] = a_off[q];
#pragma unroll
    for (int q = 0; q < Cfg::kBInstr; ++q) src.b_off[q] = b_off[q];
    return src;
  }

  __device__ __forceinline__ bool next(Tile& t) {
    while (vtile < live_tiles) {
      const int tile = xcd_remap(vtile, live_tiles);
      vtile += gridDim.x;
      int rb, slice;
      tile_coords(tile, live_rb, num_slices, group, &rb, &slice);
      int32_t begin = row_offsets[rb];
      int32_t end = row_offsets[rb + 1];
      if (begin < 0 || end > nnz || end < begin) begin = end = 0;  // not a BSR row: treat as empty
      if (begin == end && !zero_dead_rows) continue;
      t.rb = __builtin_amdgcn_readfirstlane(rb);
      t.n0 = __builtin_amdgcn_readfirstlane(slice * BN);
      t.begin = __builtin_amdgcn_readfirstlane(begin);
      t.steps = __builtin_amdgcn_readfirstlane((end - begin) * kStepsPerBlock);
      return true;
    }
    return false;
  }

  __device__ __forceinline__ void epilogue(const Tile& t, typename ML::Acc& acc) const {
    uint16_t* out_tile = out + static_cast<int64_t>(t.rb) * BM * d_model + t.n0;
#pragma unroll
    for (int jn = 0; jn < Cfg::TN; ++jn)
#pragma unroll
      for (int i = 0; i < Cfg::TM; ++i) {
        uint16_t* row = out_tile + static_cast<int64_t>(ML::out_row(i)) * d_model;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const f32x16_t& a = acc[jn][i];
          *reinterpret_cast<u32x2_t*>(row + ML::out_col(jn, g)) =
              u32x2_t{pack_bf16x2(a[4 * g], a[4 * g + 1]), pack_bf16x2(a[4 * g + 2], a[4 * g + 3])};
        }
      }
  }
};

template <class Cfg>
__global__ void __launch_bounds__(Cfg::kThreads)
    dsd_persistent_kernel(const uint16_t* __restrict__ blocks, const uint16_t* __restrict__ w,
                          const int32_t* __restrict__ row_offsets, const int32_t* __restrict__ col_indices,
                          uint16_t* __restrict__ out, int64_t nnz, int64_t w_rows, int32_t num_row_blocks,
                          int32_t d_model, int32_t num_slices, int32_t zero_dead_rows, int32_t group) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg::kLdsAlloc];
  DsdTiles<Cfg> sched;
  sched.blocks = blocks;
  sched.w = w;
  sched.row_offsets = row_offsets;
  sched.col_indices = col_indices;
  sched.out = out;
  sched.nnz = nnz;
  sched.w_rows = w_rows;
  sched.num_row_blocks = num_row_blocks;
  sched.d_model = d_model;
  sched.num_slices = num_slices;
  sched.zero_dead_rows = zero_dead_rows;
  sched.group = group;
  sched.live_rb = zero_dead_rows ? num_row_blocks : live_row_blocks(row_offsets, num_row_blocks);
  sched.live_tiles = sched.live_rb * num_slices;
  sched.vtile = blockIdx.x;
  sched.init();
  DmaMainloop<Cfg>::run_tiles(lds, sched);
}

template <class Cfg>
int launch_dsd_persistent(const void* blocks, const void* w, const int32_t* row_offsets, const int32_t* col_indices,
                          void* out, int64_t nnz, int64_t w_rows, int64_t num_row_blocks, int64_t d_model,
                          int32_t zero_dead_rows, hipStream_t stream) {
  if (d_model % Cfg::BN != 0) return fail(SB_ERR_INVALID, "dsd: D %% tile width != 0");
  const int32_t num_slices = static_cast<int32_t>(d_model / Cfg::BN);
  const int64_t tiles = num_row_blocks * num_slices;
  static int occupancy = 0;
  int grid = 0;
  if (const int rc = persistent_grid(reinterpret_cast<const void*>(dsd_persistent_kernel<Cfg>), Cfg::kThreads, tiles,
                                     &occupancy, &grid))
    return rc;
  dsd_persistent_kernel<Cfg><<<static_cast<uint32_t>(grid), Cfg::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(blocks), static_cast<const uint16_t*>(w), row_offsets, col_indices,
      static_cast<uint16_t*>(out), nnz, w_rows, static_cast<int32_t>(num_row_blocks), static_cast<int32_t>(d_model),
      num_slices, zero_dead_rows, tile_group());
  return check_launch("dsd");
}

// ---- DSD with the combine fused into its epilogue (top-k routing) --------
//
// out[t, :] = bf16( sum_j fp32(y[copy_row[t*k+j], :]) * fp32(gate[t*k+j]) ),
// the combine of moe_forward, done by the tile that completes token t:
// every tile writes its rows of y, publishes them (release fence, agent
// scope: the XCDs' L2s are not coherent with each other), then counts each
// of its tokens in on counters[t][column slice]. The tile whose count
// completes a token (all its routed copies written for this slice) resets
// the counter, takes an acquire fence and sums the token's rows in slot
// order j, the order of combine_kernel, so the result is bit-identical to
// the unfused path and independent of timing. No tile waits on another.
// Extra workgroups past the tiles write zeros for tokens none of whose
// copies was routed (bad expert ids), as the unfused combine does.
template <typename G>
__device__ __forceinline__ float gate_value(const G* g, int64_t i);
template <>
__device__ __forceinline__ float gate_value<uint16_t>(const uint16_t* g, int64_t i) {
  return bf16_to_f32(g[i]);
}
template <>
__device__ __forceinline__ float gate_value<_Float16>(const _Float16* g, int64_t i) {
  return static_cast<float>(g[i]);
}
template <>
__device__ __forceinline__ float gate_value<float>(const float* g, int64_t i) {
  return g[i];
}

constexpr int kOrphanTokensPerGroup = 1024;

template <class Cfg, typename G>
__global__ void __launch_bounds__(Cfg::kThreads)
    dsd_combine_kernel(const uint16_t* __restrict__ blocks, const uint16_t* __restrict__ w,
                       const int32_t* __restrict__ row_offsets, const int32_t* __restrict__ col_indices,
                       const int32_t* __restrict__ row_token, const int32_t* __restrict__ copy_row,
                       const G* __restrict__ gates, uint16_t* y, uint16_t* __restrict__ out,
                       int32_t* __restrict__ counters, int64_t nnz, int64_t w_rows, int32_t num_row_blocks,
                       int32_t d_model, int32_t num_slices, int32_t num_tokens, int32_t k,
                       const int32_t* __restrict__ valid_tokens, int32_t num_tile_groups, int32_t group) {
  using ML = DmaMainloop<Cfg>;
  constexpr int BM = Cfg::BM, BN = Cfg::BN;
  constexpr int kChunksPerRow = BN / 8;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg::kLdsAlloc];
  // Tokens this tile completes, in the part of LDS the staged tile leaves free.
  static_assert(Cfg::kLdsAlloc >= ML::kStagedBytes + (BM + 1) * 4, "room for the finish list");
  int32_t* finish_token = reinterpret_cast<int32_t*>(lds + ML::kStagedBytes);
  int32_t& num_finish = finish_token[BM];
  const int tid = threadIdx.x;
  const int32_t limit = valid_tokens ? min(num_tokens, *valid_tokens) : num_tokens;

  if (static_cast<int32_t>(blockIdx.x) >= num_tile_groups) {
    // Tokens with no routed copy: a zero row, as the unfused combine writes.
    const int64_t base = static_cast<int64_t>(blockIdx.x - num_tile_groups) * kOrphanTokensPerGroup;
    for (int64_t t = base + tid; t < base + kOrphanTokensPerGroup && t < limit; t += Cfg::kThreads) {
      bool any = false;
      for (int32_t j = 0; j < k; ++j) any = any || copy_row[t * k + j] >= 0;
      if (!any)
        for (int32_t c = 0; c < d_model; c += 8)
          *reinterpret_cast<u32x4_t*>(out + t * d_model + c) = u32x4_t{0u, 0u, 0u, 0u};
    }
    return;
  }

  const int live_rb = live_row_blocks(row_offsets, num_row_blocks);
  const int tile = xcd_remap(static_cast<int>(blockIdx.x), live_rb * num_slices);
  int rb, slice;
  tile_coords(tile, live_rb, num_slices, group, &rb, &slice);
  const int n0 = slice * BN;
  int32_t begin = row_offsets[rb];
  int32_t end = row_offsets[rb + 1];
  if (begin < 0 || end > nnz || end < begin) begin = end = 0;
  if (begin == end) return;  // dead row block: holds no copy

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

  uint16_t* y_tile = y + static_cast<int64_t>(rb) * BM * d_model + n0;
  ML::stage_tile(lds, acc, [](float v) { return v; });
  ML::for_each_staged_chunk(lds, [&](int r, int col, u32x4_t v) {
    *reinterpret_cast<u32x4_t*>(y_tile + static_cast<int64_t>(r) * d_model + col) = v;
  });

  // Publish this tile's rows, then count its tokens in.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
  if (tid == 0) num_finish = 0;
  __syncthreads();
  if (tid < BM) {
    const int32_t t = row_token[static_cast<int64_t>(rb) * BM + tid];
    if (t >= 0 && t < limit) {
      int32_t routed = 0;
      for (int32_t j = 0; j < k; ++j) routed += copy_row[static_cast<int64_t>(t) * k + j] >= 0 ? 1 : 0;
      int32_t* ctr = counters + static_cast<int64_t>(t) * num_slices + slice;
      const int32_t before = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (before == routed - 1) {
        __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // ready for the next call
        finish_token[atomicAdd(&num_finish, 1)] = t;
      }
    }
  }
  __syncthreads();
  const int32_t nf = num_finish;
  if (nf == 0) return;
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
  for (int q = tid; q < nf * kChunksPerRow; q += Cfg::kThreads) {
#pragma clang fp contract(off)  // as sb_combine: products rounded, then added
    const int32_t t = finish_token[q / kChunksPerRow];
    const int col = n0 + (q % kChunksPerRow) * 8;
    float a[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int32_t j = 0; j < k; ++j) {
      const int64_t c = static_cast<int64_t>(t) * k + j;
      const int32_t row = copy_row[c];
      if (row < 0) continue;
      const float g = gate_value(gates, c);
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(y + static_cast<int64_t>(row) * d_model + col);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        a[2 * e] += __uint_as_float(v[e] << 16) * g;
        a[2 * e + 1] += __uint_as_float(v[e] & 0xffff0000u) * g;
      }
    }
    *reinterpret_cast<u32x4_t*>(out + static_cast<int64_t>(t) * d_model + col) =
        u32x4_t{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(a[4], a[5]), pack_bf16x2(a[6], a[7])};
  }
}

template <class Cfg, typename G>
int launch_dsd_combine(const void* blocks, const void* w, const int32_t* row_offsets, const int32_t* col_indices,
                       const int32_t* row_token, const int32_t* copy_row, const void* gates, void* y, void* out,
                       int32_t* counters, int64_t nnz, int64_t w_rows, int64_t num_row_blocks, int64_t d_model,
                       int64_t num_tokens, int32_t k, const int32_t* valid_tokens, hipStream_t stream) {
  if (d_model % Cfg::BN != 0) return fail(SB_ERR_INVALID, "dsd: D %% tile width != 0");
  const int32_t num_slices = static_cast<int32_t>(d_model / Cfg::BN);
  const int64_t tiles = num_row_blocks * num_slices;
  const int64_t orphan_groups = (num_tokens + kOrphanTokensPerGroup - 1) / kOrphanTokensPerGroup;
  dsd_combine_kernel<Cfg, G><<<static_cast<uint32_t>(tiles + orphan_groups), Cfg::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(blocks), static_cast<const uint16_t*>(w), row_offsets, col_indices, row_token,
      copy_row, static_cast<const G*>(gates), static_cast<uint16_t*>(y), static_cast<uint16_t*>(out), counters, nnz,
      w_rows, static_cast<int32_t>(num_row_blocks), static_cast<int32_t>(d_model), num_slices,
      static_cast<int32_t>(num_tokens), k, valid_tokens, static_cast<int32_t>(tiles), tile_group());
  return check_launch("dsd+combine");
}

template <typename G, class... Args>
int dispatch_dsd_combine(int variant, Args... args) {
  switch (variant) {
    case 25: return launch_dsd_combine<DmaCfg<128, 256, 64, 3, 2, 4, 0, 2>, G>(args...);
    case 32: return launch_dsd_combine<DmaCfg<128, 512, 32, 4, 1, 4, 0, 2>, G>(args...);
    case 58: return launch_dsd_combine<DmaCfg<128, 512, 32, 4, 2, 4, 0, 2, 1>, G>(args...);
    case 62: return launch_dsd_combine<DmaCfg<128, 512, 32, 4, 2, 4, 0, 2, 3>, G>(args...);
    case 63: return launch_dsd_combine<DmaCfg<128, 256, 64, 3, 2, 4, 0, 2, 3>, G>(args...);
    case 64: return launch_dsd_combine<DmaCfg<128, 512, 32, 4, 1, 4, 0, 2, 3>, G>(args...);
    default: return fail(SB_ERR_INVALID, "dsd+combine: unknown tile variant %d", variant);
  }
}

template <class Cfg>
int launch_dsd_dma(const void* blocks, const void* w, const int32_t* row_offsets, const int32_t* col_indices,
                   void* out, int64_t nnz, int64_t w_rows, int64_t num_row_blocks, int64_t d_model,
                   int32_t zero_dead_rows, hipStream_t stream) {
  if (d_model % Cfg::BN != 0) return fail(SB_ERR_INVALID, "dsd: D %% tile width != 0");
  const int32_t num_slices = static_cast<int32_t>(d_model / Cfg::BN);
  const int64_t tiles = num_row_blocks * num_slices;
  dsd_dma_kernel<Cfg><<<static_cast<uint32_t>(tiles), Cfg::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(blocks), static_cast<const uint16_t*>(w), row_offsets, col_indices,
      static_cast<uint16_t*>(out), nnz, w_rows, static_cast<int32_t>(num_row_blocks), static_cast<int32_t>(d_model),
      num_slices, zero_dead_rows, tile_group());
  return check_launch("dsd");
}

template <class Cfg>
int launch_dsd(const void* blocks, const void* w, const int32_t* row_offsets, const int32_t* col_indices, void* out,
               int64_t nnz, int64_t w_rows, int64_t num_row_blocks, int64_t d_model, int32_t zero_dead_rows,
               hipStream_t stream) {
  if (d_model % Cfg::BN != 0) return fail(SB_ERR_INVALID, "dsd: D %% tile width != 0");
  const int32_t num_slices = static_cast<int32_t>(d_model / Cfg::BN);
  const int64_t tiles = num_row_blocks * num_slices;
  dsd_kernel<Cfg><<<static_cast<uint32_t>(tiles), Cfg::kThreads, 0, stream>>>(
      static_cast<const uint16_t*>(blocks), static_cast<const uint16_t*>(w), row_offsets, col_indices,
      static_cast<uint16_t*>(out), nnz, w_rows, static_cast<int32_t>(num_row_blocks), static_cast<int32_t>(d_model),
      num_slices, zero_dead_rows, tile_group());
  return check_launch("dsd");
}

// Tile variants (BN, waves WM x WN, register prefetch depth) for a block size BM.
template <int BM, class... Args>
int dispatch_dsd(int variant, Args... args) {
  switch (variant) {
    case 1: return launch_dsd<TileCfg<BM, 128, 2, 2, 1>>(args...);
    case 2: return launch_dsd<TileCfg<BM, 256, 2, 2, 1>>(args...);
    case 3: return launch_dsd<TileCfg<BM, 128, 2, 2, 2>>(args...);
    case 4: return launch_dsd<TileCfg<BM, 256, 2, 2, 2>>(args...);
    case 5: return launch_dsd<TileCfg<BM, 256, 2, 4, 1>>(args...);
    case 6: return launch_dsd<TileCfg<BM, 256, 2, 4, 2>>(args...);
    case 7: return launch_dsd<TileCfg<BM, 128, 2, 4, 1>>(args...);
    case 8: return launch_dsd<TileCfg<BM, 128, 2, 4, 2>>(args...);
    case 11: return launch_dsd_dma<DmaCfg<BM, 128, 64, 2>>(args...);
    case 12: return launch_dsd_dma<DmaCfg<BM, 128, 64, 3>>(args...);
    case 13: return launch_dsd_dma<DmaCfg<BM, 128, 32, 5>>(args...);
    case 14: return launch_dsd_dma<DmaCfg<BM, 256, 64, 2>>(args...);
    case 15: return launch_dsd_dma<DmaCfg<BM, 256, 64, 3>>(args...);
    case 16:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 32, 6, 2, 4>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 32, 6>>(args...);
    case 17:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 64, 3, 2, 4>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 64, 3>>(args...);
    case 18: return launch_dsd_dma<DmaCfg<BM, 128, 32, 4>>(args...);
    case 19:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 128, 32, 5, 2, 4>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 128, 32, 5>>(args...);
    case 9: return launch_dsd<TileCfg<BM, 128, 2, 4, 1, true>>(args...);
    case 10: return launch_dsd<TileCfg<BM, 128, 2, 2, 1, true>>(args...);
    case 21: return launch_dsd_dma<DmaCfg<BM, 128, 64, 2, 2, 2, 0, 2>>(args...);
    case 22: return launch_dsd_dma<DmaCfg<BM, 128, 64, 2, 2, 2, 2, 2>>(args...);
    case 23: return launch_dsd_dma<DmaCfg<BM, 128, 64, 3, 2, 2, 0, 2>>(args...);
    case 24: return launch_dsd_dma<DmaCfg<BM, 256, 64, 2, 2, 2, 0, 2>>(args...);
    case 25:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 64, 3, 2, 4, 0, 2>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 64, 3, 2, 2, 0, 2>>(args...);
    case 26: return launch_dsd_dma<DmaCfg<BM, 256, 64, 3, 2, 2, 0, 2>>(args...);
    case 27: return launch_dsd_dma<DmaCfg<BM, 128, 32, 5, 2, 2, 0, 2>>(args...);
    case 31: return launch_dsd_dma<DmaCfg<BM, 512, 64, 2, 1, 4, 0, 2>>(args...);
    case 32: return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 1, 4, 0, 2>>(args...);
    case 33: return launch_dsd_dma<DmaCfg<BM, 512, 32, 3, 1, 4, 0, 2>>(args...);
    case 34:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 32, 3, 2, 4, 0, 2>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 32, 3, 2, 2, 0, 2>>(args...);
    case 35: return launch_dsd_dma<DmaCfg<BM, 256, 32, 3, 2, 2, 0, 2>>(args...);
    case 36:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 64, 2, 2, 4, 0, 2>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 64, 2, 2, 2, 0, 2>>(args...);
    case 51:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 64, 3, 2, 4, 0, 2, 1>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 64, 3, 2, 2, 0, 2, 1>>(args...);
    case 52: return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 1, 4, 0, 2, 1>>(args...);
    case 53:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 32, 5, 2, 4, 0, 2, 1>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 32, 5, 2, 2, 0, 2, 1>>(args...);
    case 54:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 64, 3, 2, 4, 0, 2, 2>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 64, 3, 2, 2, 0, 2, 2>>(args...);
    case 55: return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 1, 4, 0, 2, 2>>(args...);
    // 8 waves of 64 x 128 (a 64-row block takes the 4-wave form).
    case 56:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 2, 4, 0, 2, 0>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 1, 4, 0, 2, 0>>(args...);
    case 57:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 2, 4, 0, 2, 2>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 1, 4, 0, 2, 2>>(args...);
    case 58:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 2, 4, 0, 2, 1>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 1, 4, 0, 2, 1>>(args...);
    case 59:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 512, 64, 2, 2, 4, 0, 2, 2>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 512, 64, 2, 1, 4, 0, 2, 2>>(args...);
    // The next step's DMA interleaved with the MFMAs (PIPE 3).
    case 61:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 512, 64, 2, 2, 4, 0, 2, 3>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 512, 64, 2, 1, 4, 0, 2, 3>>(args...);
    case 62:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 2, 4, 0, 2, 3>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 1, 4, 0, 2, 3>>(args...);
    case 63:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 64, 3, 2, 4, 0, 2, 3>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 64, 3, 2, 2, 0, 2, 3>>(args...);
    case 64: return launch_dsd_dma<DmaCfg<BM, 512, 32, 4, 1, 4, 0, 2, 3>>(args...);
    case 65:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 512, 32, 3, 2, 4, 0, 2, 3>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 512, 32, 3, 1, 4, 0, 2, 3>>(args...);
    case 37:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 32, 6, 2, 4, 0, 2>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 32, 6, 2, 2, 0, 2>>(args...);
    case 38:
      if constexpr (BM == 128) return launch_dsd_dma<DmaCfg<BM, 256, 32, 5, 2, 4, 0, 2>>(args...);
      else return launch_dsd_dma<DmaCfg<BM, 256, 32, 5, 2, 2, 0, 2>>(args...);
    case 39: return launch_dsd_dma<DmaCfg<BM, 128, 32, 8, 2, 2, 0, 2>>(args...);
    case 41:
      if constexpr (BM == 128) return launch_dsd_persistent<DmaCfg<BM, 256, 64, 3, 2, 4, 0, 2>>(args...);
      else return launch_dsd_persistent<DmaCfg<BM, 256, 64, 3, 2, 2, 0, 2>>(args...);
    case 42: return launch_dsd_persistent<DmaCfg<BM, 512, 32, 4, 1, 4, 0, 2>>(args...);
    case 43: return launch_dsd_persistent<DmaCfg<BM, 128, 64, 2, 2, 2, 0, 2>>(args...);
    case 44:
      if constexpr (BM == 128) return launch_dsd_persistent<DmaCfg<BM, 256, 32, 3, 2, 4, 0, 2>>(args...);
      else return launch_dsd_persistent<DmaCfg<BM, 256, 32, 3, 2, 2, 0, 2>>(args...);
    case 45: return launch_dsd_persistent<DmaCfg<BM, 128, 64, 2>>(args...);
    default: return fail(SB_ERR_INVALID, "dsd: unknown tile variant %d", variant);
  }
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
  const hipStream_t s = as_stream(stream);
  const int forced = tuning_override("SPARSEBENCH_DSD_VARIANT");
  // Default, from timing every variant on the benchmark shapes (MI355X,
  // samples interleaved across variants): 128 x 512 tiles, BK 32 x 4-stage
  // LDS-DMA ring with non-temporal W loads, the next stage's DMA and the
  // next sub-step's fragment reads issued among the MFMAs; 4 waves of
  // 128 x 128. With a deep reduction (K = F per expert >= 8192, read from
  // the buffer shape: nnz / num_row_blocks blocks per row) 8 waves of
  // 64 x 128.
  const int64_t row_k = num_row_blocks > 0 ? nnz / num_row_blocks * block_size : 0;
  int variant = forced > 0 ? forced : (row_k >= 8192 ? 62 : 64);
  if (d_model % 256 != 0 && (variant == 2 || variant == 4 || variant == 5 || variant == 6 || variant == 14 ||
                             variant == 15 || variant == 16 || variant == 17 || variant == 24 || variant == 25 ||
                             variant == 26 || variant == 34 || variant == 35 || variant == 36 || variant == 37 ||
                             variant == 38 || variant == 41 || variant == 44 || variant == 51 || variant == 53 ||
                             variant == 54 || variant == 63))
    variant = 1;
  if (d_model % 512 != 0 &&
      ((variant >= 31 && variant <= 33) || variant == 42 || variant == 52 || (variant >= 55 && variant <= 59)))
    variant = d_model % 256 == 0 ? 25 : 21;
  if (d_model % 512 != 0 && (variant == 61 || variant == 62 || variant == 64 || variant == 65))
    variant = d_model % 256 == 0 ? 63 : 21;
  if (block_size == 128)
    return dispatch_dsd<128>(variant, blocks, w, row_offsets, col_indices, out, nnz, w_rows, num_row_blocks, d_model,
                             zero_dead_rows, s);
  return dispatch_dsd<64>(variant, blocks, w, row_offsets, col_indices, out, nnz, w_rows, num_row_blocks, d_model,
                          zero_dead_rows, s);
}

extern "C" int sb_dsd_combine(const void* blocks, const void* w, const int32_t* row_offsets,
                              const int32_t* col_indices, const int32_t* row_token, const int32_t* copy_row,
                              const void* gates, int32_t gate_dtype, void* y, void* out, int32_t* counters,
                              int64_t nnz, int64_t w_rows, int64_t num_row_blocks, int64_t d_model,
                              int64_t num_tokens, int32_t k, const int32_t* valid_tokens, void* stream) {
  constexpr int64_t kI32Max = 2147483647;
  if (d_model <= 0 || d_model % 256 != 0)
    return fail(SB_ERR_INVALID, "dsd+combine needs D (%lld) to be a multiple of 256", static_cast<long long>(d_model));
  if (num_row_blocks < 0 || w_rows < 0 || w_rows % 128 != 0 || nnz < 0)
    return fail(SB_ERR_INVALID, "dsd+combine: bad layout sizes");
  if (num_tokens <= 0 || num_tokens > kI32Max / 8 || k <= 0 || num_tokens * k > kI32Max)
    return fail(SB_ERR_INVALID, "dsd+combine: bad token count or k");
  if (num_row_blocks * 128 > kI32Max || num_row_blocks * (d_model / 128) > kI32Max)
    return fail(SB_ERR_INVALID, "dsd+combine: too many row blocks");
  if (!blocks || !w || !row_offsets || !col_indices || !row_token || !copy_row || !gates || !y || !out || !counters)
    return fail(SB_ERR_INVALID, "dsd+combine: null buffer");
  if (!aligned16(blocks) || !aligned16(w) || !aligned16(y) || !aligned16(out))
    return fail(SB_ERR_INVALID, "dsd+combine: blocks, w, y and out must be 16-byte aligned");
  if (num_row_blocks == 0) return clear_ok();
  const hipStream_t s = as_stream(stream);
  const int forced = tuning_override("SPARSEBENCH_DSD_VARIANT");
  const int64_t row_k = nnz / num_row_blocks * 128;
  int variant = forced == 25 || forced == 32 || forced == 58 || forced == 62 || forced == 63 || forced == 64
                    ? forced
                    : (row_k >= 8192 ? 62 : 64);
  if (d_model % 512 != 0 && variant != 25 && variant != 63) variant = 63;
  switch (gate_dtype) {
    case SB_DTYPE_BF16:
      return dispatch_dsd_combine<uint16_t>(variant, blocks, w, row_offsets, col_indices, row_token, copy_row, gates,
                                            y, out, counters, nnz, w_rows, num_row_blocks, d_model, num_tokens, k,
                                            valid_tokens, s);
    case SB_DTYPE_F16:
      return dispatch_dsd_combine<_Float16>(variant, blocks, w, row_offsets, col_indices, row_token, copy_row, gates,
                                            y, out, counters, nnz, w_rows, num_row_blocks, d_model, num_tokens, k,
                                            valid_tokens, s);
    case SB_DTYPE_F32:
      return dispatch_dsd_combine<float>(variant, blocks, w, row_offsets, col_indices, row_token, copy_row, gates, y,
                                         out, counters, nnz, w_rows, num_row_blocks, d_model, num_tokens, k,
                                         valid_tokens, s);
    default:
      return fail(SB_ERR_INVALID, "dsd+combine: unsupported gate dtype code %d", gate_dtype);
  }
}
