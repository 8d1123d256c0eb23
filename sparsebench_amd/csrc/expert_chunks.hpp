// The expert chunks of a routing layout, and the choice between the
// expert-major and the per-row-block kernels of the MoE layer.
//
// The layout gives expert e n = tokens_per_expert[e] real rows from padded
// row padded_offsets[e], in ceil(n / 128) row blocks, real rows first. A
// chunk is a run of up to 32 RMAX of those rows that one tile computes:
// chunks of S = 128 floor(32 RMAX / 128) rows, the last one holding what
// remains, and a last piece of at most 32 RMAX - S rows joined to the chunk
// before it. Every workgroup derives the chunks itself from
// tokens_per_expert with wave scans, so no launch or buffer is added.
#pragma once

#include "common.hpp"

namespace sb {

constexpr int kBS = 128;

// Chunks of an expert with n real rows, for tiles of at most 32 * RMAX rows.
template <int RMAX>
struct Chunking {
  static_assert(RMAX >= 4 && RMAX <= 10, "a tile holds one to two row blocks and a 64-row piece");
  static constexpr int kRows = kBS * ((32 * RMAX) / kBS);  // rows of a full chunk
  static constexpr int kMerge = 32 * RMAX - kRows;         // a last piece up to this size joins the one before
  __device__ __forceinline__ static int count(int32_t n) {
    if (n <= 0) return 0;
    const int c = (n + kRows - 1) / kRows;
    const int last = n - kRows * (c - 1);
    return c - ((c >= 2 && last <= kMerge) ? 1 : 0);
  }
};

// Inclusive prefix sum of v over the wave's 64 lanes (lane i gets lanes
// 0 .. i) by DPP moves, six VALU operations: row_shr 1, 2, 4 and 8 add up
// each row of 16 lanes, then row_bcast:15 adds row 0's total to row 1 and
// row 2's to row 3, and row_bcast:31 adds the total of rows 0-1 to rows 2
// and 3. A lane whose source lies outside its row, or whose row the row
// mask leaves out, adds the 0 it starts from. Every lane of the wave must
// be active. (A shuffle through LDS, ds_bpermute, is a round trip of its
// own: six dependent ones per scan made the layout summary and the chunk
// search a few microseconds of every tile's start.)
__device__ __forceinline__ int wave_inclusive_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

// The same scan with max, for v >= 0.
__device__ __forceinline__ int wave_inclusive_max(int v) {
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false));
  v = max(v, __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false));
  return v;
}

// Sum of v over the wave, as a uniform (scalar) value.
__device__ __forceinline__ int wave_inclusive_scan_total(int v) {
  return __builtin_amdgcn_readlane(wave_inclusive_scan(v), 63);
}

// Lane l's v, for a uniform l: a scalar read (v_readlane_b32).
__device__ __forceinline__ int lane_value(int v, int l) { return __builtin_amdgcn_readlane(v, l); }

// tokens_per_expert[base + lane] (0 past the experts) for one pass of 64
// experts. The addresses are uniform, so these are scalar loads: after a
// CU's first tile they hit its scalar cache, where per-lane vector loads
// go to L2 each time (about a microsecond while the CU's DMA streams run,
// before every tile's first load). v_writelane_b32 moves each value into
// its lane (this compiler has no builtin for it; the asm is not volatile,
// so the loads are still batched into wide scalar loads ahead of it). A
// partial last pass uses per-lane loads.
__device__ __forceinline__ int32_t expert_counts(const int32_t* __restrict__ tokens_per_expert, int32_t num_experts,
                                                 int base) {
  int32_t n = 0;
  base = __builtin_amdgcn_readfirstlane(base);  // uniform in every caller; said so for the scalar loads
  if (base + 64 <= num_experts) {
    // Wide loads (tokens_per_expert is 16-byte aligned, base a multiple
    // of 64), issued together before the first value is used.
    const int4* q = reinterpret_cast<const int4*>(tokens_per_expert + base);
    int4 c[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) c[j] = q[j];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int32_t v[4] = {c[j].x, c[j].y, c[j].z, c[j].w};
#pragma unroll
      for (int k = 0; k < 4; ++k)
        asm("v_writelane_b32 %0, %1, %2" : "+v"(n) : "s"(__builtin_amdgcn_readfirstlane(v[k])), "i"(4 * j + k));
    }
  } else {  // the last pass of an expert count that is not a multiple of 64
    const int lane = threadIdx.x & 63;
    if (base + lane < num_experts) n = tokens_per_expert[base + lane];
  }
  return n;
}

// The helpers below take `first`, the counts of the first pass
// (expert_counts(tokens_per_expert, num_experts, 0)), loaded once by the
// kernel; they load only the passes after it. Rebuilding the first pass's
// vector in every helper cost 64 v_writelane_b32 and a wait on the scalar
// loads each time.
struct Chunk {
  int32_t expert;  // -1: no such chunk
  int32_t row0;    // first padded row (a multiple of 128)
  int32_t rows;    // real rows, 1 .. 32 * groups
  int32_t groups;  // 32-row groups of the tile
};

// Padded rows of an expert with n real rows (the routing layout pads each
// expert to whole row blocks).
__device__ __forceinline__ int32_t padded_rows(int32_t n) { return n > 0 ? (n + kBS - 1) / kBS * kBS : 0; }

// Chunk c (0 <= c < the number of chunks) in expert order. Its first row is
// the expert's first padded row, the sum of the padded rows of the experts
// before it (padded_offsets[e] of the routing layout), computed here from the
// counts instead of loaded: one dependent load less before the tile's first.
template <int RMAX>
__device__ __forceinline__ Chunk find_chunk(const int32_t* __restrict__ tokens_per_expert, int32_t num_experts, int c,
                                            int32_t first) {
  Chunk ch{-1, 0, 0, 0};
  int before = 0;       // chunks of the experts before this pass
  int rows_before = 0;  // padded rows of the experts before this pass
  for (int base = 0; base < num_experts; base += 64) {
    const int32_t n = base == 0 ? first : expert_counts(tokens_per_expert, num_experts, base);
    const int cc = Chunking<RMAX>::count(n);
    const int incl = wave_inclusive_scan(cc);
    const int pincl = wave_inclusive_scan(padded_rows(n));
    const uint64_t reach = __ballot(before + incl > c);  // experts whose chunks run past c
    if (reach != 0) {
      const int l = __builtin_ctzll(reach);  // the first of them holds chunk c
      const int i = c - (before + lane_value(incl - cc, l));
      const int count = lane_value(cc, l);
      const int32_t n_e = lane_value(n, l);
      const int start = Chunking<RMAX>::kRows * i;
      ch.expert = base + l;
      ch.row0 = rows_before + lane_value(pincl - padded_rows(n), l) + start;
      ch.rows = i + 1 < count ? Chunking<RMAX>::kRows : n_e - start;
      ch.groups = (ch.rows + 31) / 32;
      break;
    }
    before += lane_value(incl, 63);
    rows_before += lane_value(pincl, 63);
  }
  ch.expert = __builtin_amdgcn_readfirstlane(ch.expert);
  ch.row0 = __builtin_amdgcn_readfirstlane(ch.row0);
  ch.rows = __builtin_amdgcn_readfirstlane(ch.rows);
  ch.groups = __builtin_amdgcn_readfirstlane(ch.groups);
  return ch;
}

// Largest-first order inside one tile group (the `group` chunks g0 .. g0+G-1
// that tile_coords walks slice by slice): the chunks with more than
// kRows / 32 row groups (an expert's last chunk with a joined piece) take
// the group's first tiles, all their slices, then the others slice by
// slice. Chunk p of the group is such a chunk iff bit p of the returned
// mask is set. One pass over the counts.
template <int RMAX>
__device__ __forceinline__ uint32_t big_chunks_of_group(const int32_t* __restrict__ tokens_per_expert,
                                                        int32_t num_experts, int g0, int G, int32_t first) {
  constexpr int kFull = Chunking<RMAX>::kRows / 32;
  uint32_t mask = 0;
  int before = 0;
  for (int base = 0; base < num_experts && before < g0 + G; base += 64) {
    const int32_t n = base == 0 ? first : expert_counts(tokens_per_expert, num_experts, base);
    const int c = Chunking<RMAX>::count(n);
    const int incl = wave_inclusive_scan(c);
    const int last = before + incl - 1;  // this expert's last chunk
    const int groups = c > 0 ? (n - Chunking<RMAX>::kRows * (c - 1) + 31) / 32 : 0;
    const uint32_t bit = (c > 0 && groups > kFull && last >= g0 && last < g0 + G) ? (1u << (last - g0)) : 0u;
    // Experts have distinct last chunks, so their bits are distinct and
    // the wave's sum is their union.
    mask |= static_cast<uint32_t>(wave_inclusive_scan_total(static_cast<int>(bit)));
    before += lane_value(incl, 63);
  }
  return __builtin_amdgcn_readfirstlane(mask);
}

// Local tile `local` of a group of G chunks x `slices` slices, largest
// first: the chunks of `big` (a mask over the group's positions) with all
// their slices, then the rest slice by slice.
__host__ __device__ __forceinline__ void lpt_group_tile(int local, int G, int slices, uint32_t big, int* pos,
                                                        int* slice) {
  const int nb = __builtin_popcount(big);
  uint32_t set = big;
  int idx;
  if (local < nb * slices) {
    idx = local % nb;
    *slice = local / nb;
  } else {
    local -= nb * slices;
    set = ~big & ((G >= 32 ? 0u : (1u << G)) - 1u);
    idx = local % (G - nb);
    *slice = local / (G - nb);
  }
  for (int i = 0; i < idx; ++i) set &= set - 1;  // drop the idx lowest members
  *pos = __builtin_ctz(set);
}

// The experts by tile size, for layouts where every expert is one chunk:
// hist[g] = experts of g row groups (ceil(n / 32) = g), g = 1 .. RMAX, from
// one ballot per g and pass (every wave computes the same values).
template <int RMAX>
__device__ __forceinline__ void single_chunk_hist(const int32_t* __restrict__ tokens_per_expert, int32_t num_experts,
                                                  int32_t first, int32_t (&hist)[RMAX + 1]) {
#pragma unroll
  for (int g = 0; g <= RMAX; ++g) hist[g] = 0;
#pragma unroll 1
  for (int base = 0; base < num_experts; base += 64) {
    const int32_t n = base == 0 ? first : expert_counts(tokens_per_expert, num_experts, base);
    const int groups = n > 0 ? (n + 31) / 32 : 0;
#pragma unroll
    for (int g = 1; g <= RMAX; ++g) hist[g] += __builtin_popcountll(__ballot(groups == g));
  }
}

// Chunk k (0 <= k < the number of experts with rows) in size order, for
// layouts where every expert is one chunk: by row-group count, largest
// first, in expert order within one count. The chunk's first row is the sum
// of the padded rows of the experts before it (padded_offsets[e] of the
// routing layout), computed from the counts.
template <int RMAX>
__device__ __forceinline__ Chunk find_single_chunk_by_size(const int32_t* __restrict__ tokens_per_expert,
                                                           int32_t num_experts, int k, int32_t first,
                                                           const int32_t (&hist)[RMAX + 1]) {
  Chunk ch{-1, 0, 0, 0};
  int g = RMAX;
  for (; g >= 1; --g) {  // the count that holds rank k, and k's rank within it
    if (k < hist[g]) break;
    k -= hist[g];
  }
  if (g < 1) return ch;
  int rows_before = 0;  // padded rows of the experts before this pass
  for (int base = 0; base < num_experts; base += 64) {
    const int32_t n = base == 0 ? first : expert_counts(tokens_per_expert, num_experts, base);
    const uint64_t match = __ballot(n > 0 && (n + 31) / 32 == g);
    const int cnt = __builtin_popcountll(match);
    if (k < cnt) {
      // The lane of the k-th match: its rank among the matches is k.
      const int below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(match >> 32),
                                                  __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(match), 0));
      const uint64_t hit = __ballot(n > 0 && (n + 31) / 32 == g && below == k);
      const int l = __builtin_ctzll(hit);
      const int pincl = wave_inclusive_scan(padded_rows(n));
      ch.expert = base + l;
      ch.row0 = rows_before + lane_value(pincl - padded_rows(n), l);
      ch.rows = lane_value(n, l);
      ch.groups = g;
      break;
    }
    k -= cnt;
    rows_before += wave_inclusive_scan_total(padded_rows(n));
  }
  ch.expert = __builtin_amdgcn_readfirstlane(ch.expert);
  ch.row0 = __builtin_amdgcn_readfirstlane(ch.row0);
  ch.rows = __builtin_amdgcn_readfirstlane(ch.rows);
  ch.groups = __builtin_amdgcn_readfirstlane(ch.groups);
  return ch;
}

// Row-block pairs, the SDD's units when F % 512 != 0 (256-wide tiles): an
// expert's row blocks two by two from its first, an odd last one alone. A
// pair is 256 padded rows (8 row groups), a single 128 (4); the tile
// computes every padded row, so padding rows come out as zeros, as from the
// per-row-block kernel (a single of an expert of at most 64 rows stops at
// its first 64 when the DSD's row-block tiles read no further). Units are
// numbered in expert order, pairs and singles each counted on their own.
struct PairCounts {
  int32_t pairs, singles;
};

// first: expert_counts(tokens_per_expert, num_experts, 0).
__device__ __forceinline__ PairCounts pair_counts(const int32_t* __restrict__ tokens_per_expert, int32_t num_experts,
                                                  int32_t first) {
  int p = 0, s = 0;
#pragma unroll 1
  for (int base = 0; base < num_experts; base += 64) {
    const int32_t n = base == 0 ? first : expert_counts(tokens_per_expert, num_experts, base);
    const int rb = n > 0 ? (n + kBS - 1) / kBS : 0;
    p += rb >> 1;
    s += rb & 1;
  }
  PairCounts c;
  c.pairs = wave_inclusive_scan_total(p);
  c.singles = wave_inclusive_scan_total(s);
  return c;
}

// The units of the pair kernel's workgroups: XCD x takes the x-th eighth of
// the pairs and the x-th eighth of the singles, each kind in expert order,
// and runs its pairs, then its singles, each unit's `slices` column slices
// side by side (pair_tile_for). An XCD holds at most this many units.
__host__ __device__ constexpr int pair_units_per_xcd(int units) { return units / kNumXcd + 2; }

// Workgroup bid (on XCD bid % 8) and its tile, with a short last round
// split. An XCD that runs n tiles on
// `cus` CUs has r = n % cus of them in its last round; when those are all
// singles, each runs as two column halves on workgroups of their own, so 2r
// CUs share the round (as split_tail does for row-block tiles), if 2r CUs
// are free when the round starts: pair tiles in the round before it (about
// 1.6 times a single's time) still hold their CUs then, and halves past the
// free CUs would wait for a round of their own. Workgroup bid gets unit k of
// its kind, column slice `slice` and `half`: -1 for the whole slice, else 0
// or 1; false past the XCD's tiles. An XCD uses positions up to n + cus / 2.
__host__ __device__ __forceinline__ bool pair_tile_for(int bid, int pairs, int singles, int slices, int cus,
                                                       bool* single, int* k, int* slice, int* half) {
  const int q = bid / kNumXcd, x = bid % kNumXcd;
  const int p_lo = pairs * x / kNumXcd, p_hi = pairs * (x + 1) / kNumXcd;
  const int s_lo = singles * x / kNumXcd, s_hi = singles * (x + 1) / kNumXcd;
  const int np = p_hi - p_lo, ns = s_hi - s_lo;
  const int n = (np + ns) * slices;
  const int whole = cus > 0 ? n - n % cus : n;  // tiles in whole rounds
  const int r = n - whole;
  const int pair_tiles = np * slices;
  const int busy = whole >= cus && pair_tiles > whole - cus ? pair_tiles - (whole - cus) : 0;
  int t = q, h = -1;
  if (r > 0 && 2 * r <= cus - busy && whole >= pair_tiles) {
    if (q >= whole + 2 * r) return false;
    if (q >= whole) {
      t = whole + (q - whole) / 2;
      h = (q - whole) % 2;
    }
  } else if (q >= n) {
    return false;
  }
  const int u = t / slices;
  *single = u >= np;
  *k = uniform(u >= np ? s_lo + u - np : p_lo + u);
  *slice = uniform(t % slices);
  *half = uniform(h);
  return true;
}

// Pair k (single = false) or single k (single = true), each kind counted in
// expert order. The chunk's first row is the sum of the padded rows of the
// experts before it (padded_offsets[e] of the routing layout), computed
// from the counts.
__device__ __forceinline__ Chunk find_pair_unit(const int32_t* __restrict__ tokens_per_expert, int32_t num_experts,
                                                bool single, int k, int32_t first) {
  Chunk ch{-1, 0, 0, 0};
  int rows_before = 0;  // padded rows of the experts before this pass
#pragma unroll 1
  for (int base = 0; base < num_experts; base += 64) {
    const int32_t n = base == 0 ? first : expert_counts(tokens_per_expert, num_experts, base);
    const int rb = n > 0 ? (n + kBS - 1) / kBS : 0;
    const int mine = single ? (rb & 1) : (rb >> 1);  // this expert's units of the kind
    const int incl = wave_inclusive_scan(mine);
    const int total = lane_value(incl, 63);
    if (k < total) {
      const int l = __builtin_ctzll(__ballot(incl > k));  // the expert that holds unit k
      const int i = k - (lane_value(incl, l) - lane_value(mine, l));
      const int first_rb = single ? lane_value(rb, l) - 1 : 2 * i;  // the unit's first row block in the expert
      const int pincl = wave_inclusive_scan(rb * kBS);
      ch.expert = base + l;
      ch.row0 = rows_before + lane_value(pincl - rb * kBS, l) + first_rb * kBS;
      ch.rows = min(lane_value(n, l) - first_rb * kBS, single ? kBS : 2 * kBS);
      ch.groups = single ? 4 : 8;
      break;
    }
    k -= total;
    rows_before += wave_inclusive_scan_total(rb * kBS);
  }
  ch.expert = __builtin_amdgcn_readfirstlane(ch.expert);
  ch.row0 = __builtin_amdgcn_readfirstlane(ch.row0);
  ch.rows = __builtin_amdgcn_readfirstlane(ch.rows);
  ch.groups = __builtin_amdgcn_readfirstlane(ch.groups);
  return ch;
}

// The XCD-balanced tile of workgroup bid over `chunks` chunks x `slices`
// column slices. The chunks in size order are dealt to the XCDs like cards
// in snake order (ranks 0-7 to XCDs 0-7, ranks 8-15 to XCDs 7-0, ...), so
// each XCD gets a like mix of large and small tiles; an XCD runs its chunks
// slice by slice, largest first, so the tiles dispatched last to the CUs
// that free up first are the smallest. Workgroups are handed to the XCDs
// round-robin by id. Returns false past the XCD's tiles (the grid needs up
// to kNumXcd x ceil(chunks / kNumXcd) x slices workgroups).
__host__ __device__ __forceinline__ bool balanced_chunk_tile(int bid, int chunks, int slices, int* rank, int* slice) {
  const int x = bid % kNumXcd, q = bid / kNumXcd;
  const int rows = chunks / kNumXcd, rem = chunks % kNumXcd;
  const int pos = (rows & 1) ? kNumXcd - 1 - x : x;  // x's place in the partial row
  const int n = rows + (pos < rem ? 1 : 0);           // chunks of XCD x
  if (n == 0 || q >= n * slices) return false;
  const int j = q % n;
  *slice = uniform(q / n);
  *rank = uniform(kNumXcd * j + ((j & 1) ? kNumXcd - 1 - x : x));
  return true;
}

// Which tiling computes a stage of the MoE layer: expert chunks or row
// blocks. Every workgroup of the stage's kernel makes the same choice from
// the same counts, so it costs no host sync.
//   kGateDsd  expert tiles when the routing is balanced: no expert holds
//             more than twice the mean rows (and, checked by the layer
//             kernels next to this gate, F >= 1536). Skewed routing keeps row
//             blocks: their tiles are all one size, and the many row blocks
//             of a popular expert run side by side and share its W2 lines
//             in L2, where chunks of very different sizes leave CUs idle.
//   kGateSdd  as kGateDsd, and either at most 256 rows per expert on
//             average (merging an expert's last, nearly empty row block
//             into one tile saves a whole stream of its W1 slice), or
//             fewer rounds of tiles over the CUs than the row blocks need
//             (large experts: each expert's last, nearly empty row block is
//             a tile of its own among the row blocks, which can add a
//             round; with as many rounds the row-block tiles are as fast
//             and need no summary of the layout). The SDD's
//             expert tiles leave padding rows past each expert's last
//             32-row group unwritten, so they must only feed the DSD's
//             expert tiles, which do not read them: the SDD takes its
//             expert tiles only when the DSD will take its own (kGateDsd,
//             and the DSD's grid holds all of its expert tiles; both
//             kernels compute that from the same counts and the same grid
//             size). A row-block DSD would read those rows, cold from HBM
//             rather than from the cache the SDD's stores warm (with skewed
//             routing that costs it more than the SDD gains), and write
//             their unspecified products to padding rows of its output.
enum ExpertGate : int32_t { kGateNone = 0, kGateDsd = 1, kGateSdd = 2 };

// What a workgroup needs to choose and to number its tiles, from one pass
// over tokens_per_expert (every wave computes the same values).
struct LayoutSummary {
  int64_t rows;      // real rows of all experts
  int32_t largest;   // real rows of the largest expert
  int32_t chunks_a;  // chunks of up to 32 RA rows
  int32_t chunks_b;  // chunks of up to 32 RB rows
  int32_t chunks_c;  // chunks of up to 32 RC rows (0 when RC is 0)
  int32_t chunks_d;  // chunks of up to 32 RD rows (0 when RD is 0)
  int32_t active;    // experts with at least one row
};

// first: expert_counts(tokens_per_expert, num_experts, 0), loaded by the
// caller ahead of its own first dependent load so the two overlap.
template <int RA, int RB, int RC = 0, int RD = 0>
__device__ __forceinline__ LayoutSummary summarize_layout(const int32_t* __restrict__ tokens_per_expert,
                                                          int32_t num_experts, int32_t first) {
  int64_t rows = 0;
  int32_t most = 0, ca = 0, cb = 0, cc = 0, cd = 0, act = 0;
#pragma unroll 1
  for (int base = 0; base < num_experts; base += 64) {
    const int32_t n = base == 0 ? first : expert_counts(tokens_per_expert, num_experts, base);
    const int32_t v = n > 0 ? n : 0;
    rows += v;
    most = max(most, v);
    act += v > 0 ? 1 : 0;
    ca += Chunking<RA>::count(v);
    cb += Chunking<RB>::count(v);
    if constexpr (RC > 0) cc += Chunking<RC>::count(v);
    if constexpr (RD > 0) cd += Chunking<RD>::count(v);
  }
  // A lane's row sum (under 2^35) is split at bit 16 so that each half's
  // sum over the wave stays under 2^31.
  LayoutSummary sum;
  const int64_t lo = wave_inclusive_scan_total(static_cast<int>(rows & 0xffff));
  const int64_t hi = wave_inclusive_scan_total(static_cast<int>(rows >> 16));
  sum.rows = (hi << 16) + lo;
  sum.largest = __builtin_amdgcn_readlane(wave_inclusive_max(most), 63);
  sum.chunks_a = wave_inclusive_scan_total(ca);
  sum.chunks_b = wave_inclusive_scan_total(cb);
  sum.chunks_c = RC > 0 ? wave_inclusive_scan_total(cc) : 0;
  sum.chunks_d = RD > 0 ? wave_inclusive_scan_total(cd) : 0;
  sum.active = wave_inclusive_scan_total(act);
  return sum;
}

__device__ __forceinline__ bool expert_tiles_chosen(const LayoutSummary& sum, int32_t num_experts, int32_t gate,
                                                    int32_t slices, int32_t cus) {
  const bool balanced = sum.rows > 0 && static_cast<int64_t>(sum.largest) * num_experts <= 2 * sum.rows;
  bool chosen = balanced;
  if (gate == kGateSdd) {
    // Rounds of 512-wide tiles over the CUs: large experts take the expert
    // chunks when these need fewer rounds than the row blocks.
    // 32-bit: the host bounds live row blocks x slices below 2^31 (a 64-bit
    // division is a long scalar sequence at every tile's start).
    const uint32_t c = static_cast<uint32_t>(cus);
    const uint32_t chunk_rounds = (static_cast<uint32_t>(sum.chunks_a) * static_cast<uint32_t>(slices) + c - 1) / c;
    const uint32_t block_rounds = (static_cast<uint32_t>(sum.chunks_b) * static_cast<uint32_t>(slices) + c - 1) / c;
    chosen = balanced && (sum.rows <= static_cast<int64_t>(256) * num_experts || chunk_rounds < block_rounds);
  }
  return __builtin_amdgcn_readfirstlane(chosen ? 1 : 0) != 0;
}

// Host side of the gate: the test hook SB_HOOK_EXPERT_GATE = 1 forces the
// expert tiles, 2 the row blocks; 0 (its default) chooses.
inline int32_t expert_gate_override() {
  const int32_t v = test_hook(SB_HOOK_EXPERT_GATE);
  return v == 1 || v == 2 ? v : 0;
}

// On the device: are the expert tiles of `gate`'s stage used?
// force: 0 choose, 1 always, 2 never.
__device__ __forceinline__ bool expert_stage_runs(const LayoutSummary& sum, int32_t num_experts, int32_t gate,
                                                  int32_t force, int32_t slices = 1, int32_t cus = 1) {
  if (force == 1) return true;
  if (force == 2) return false;
  return expert_tiles_chosen(sum, num_experts, gate, slices, cus);
}

}  // namespace sb
