// Routing -> block-sparse layout on gfx950, with no host sync.
//
// A copy is one (token, choice) pair, c = t*k + j. Copies are sorted by
// expert with a stable counting sort, padded per expert to a multiple of the
// block size, and described as BSR for the two matmuls. The result is the
// layout of sparsebench/topology.py:53-118 (reference), bit for bit, with the
// worst-case buffer conventions of csrc/routing.cu:162-193, 248-249.
//
// Launches, all on the caller's stream:
//   1. count    one workgroup per chunk of 1024 copies: per-expert counts of
//               the chunk, plus a count of bad ids in column E.
//   2. offsets  (only beyond kScanChunks chunks) one workgroup: exclusive
//               prefix of every expert's column over the chunks (in place),
//               tokens_per_expert, padded_offsets, error.
//   3. place    first C workgroups: each copy's row, ranked inside its wave
//               by ballot bit-slicing (no atomics, so the order is stable);
//               the remaining workgroups write row_offsets / col_indices /
//               row_block_expert and mark every non-copy row -1. Up to
//               kScanChunks chunks, every workgroup first sums the columns
//               of the counts itself (route_place_scan_kernel), in place of
//               step 2.
// Place's two roles touch disjoint memory and depend only on steps 1-2.

#include <mutex>

#include "common.hpp"
#include "layout.hpp"

namespace sb {
namespace {

constexpr int kChunk = 1024;             // copies per count/place workgroup, one per lane
constexpr int kWaves = kChunk / 64;      // 16 wave64s
constexpr int kLayoutItemsPerGroup = 1024;

__device__ __forceinline__ uint64_t lanes_below() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// Mask of the wave's lanes that hold a valid copy of the same expert as this
// lane: AND of one ballot per bit of the expert id. ceil(log2 E) ballots.
__device__ __forceinline__ uint64_t same_expert_lanes(bool valid, int32_t e, int num_bits) {
  uint64_t peers = __ballot(valid);
  for (int b = 0; b < num_bits; ++b) {
    const bool bit = (e >> b) & 1;
    const uint64_t ones = __ballot(valid && bit);
    peers &= bit ? ones : ~ones;
  }
  return peers;
}

// Where copy c's token comes from: c / k for top-k routing, or a list of
// token ids (one per copy) for a routing given as assignments.
template <typename Tok>
struct TokenSource {
  const Tok* __restrict__ ids;  // nullptr: token = c / k
  int32_t k;
  int64_t num_tokens;
  __device__ __forceinline__ int64_t token(int64_t c) const {
    return ids != nullptr ? static_cast<int64_t>(ids[c]) : c / k;
  }
};

// Expert of copy c, or -1 when the copy is skipped. A copy past the end or
// of a token >= *valid_tokens is skipped silently; a bad expert id (or a
// token id outside [0, T)) is skipped and reported through *bad.
template <typename Idx, typename Tok>
__device__ __forceinline__ int32_t read_expert(const Idx* __restrict__ idx, int64_t c, int64_t n,
                                               const TokenSource<Tok>& src, int32_t num_experts,
                                               const int32_t* __restrict__ valid_tokens, bool* bad,
                                               int32_t* token) {
  *bad = false;
  *token = -1;
  if (c >= n) return -1;
  const int64_t t = src.token(c);
  if (t < 0 || t >= src.num_tokens) {
    *bad = true;
    return -1;
  }
  if (valid_tokens != nullptr && t >= static_cast<int64_t>(*valid_tokens)) return -1;
  const Idx v = idx[c];
  if (v >= 0 && v < static_cast<Idx>(num_experts)) {
    *token = static_cast<int32_t>(t);
    return static_cast<int32_t>(v);
  }
  *bad = true;
  return -1;
}

template <typename Idx, typename Tok>
__global__ void __launch_bounds__(kChunk) route_count_kernel(const Idx* __restrict__ idx, int64_t n,
                                                             TokenSource<Tok> tokens, int32_t num_experts,
                                                             int32_t num_bits,
                                                             const int32_t* __restrict__ valid_tokens,
                                                             int32_t* __restrict__ counts) {
  __shared__ int32_t hist[kMaxExperts + 1];
  const int tid = threadIdx.x;
  for (int e = tid; e <= num_experts; e += kChunk) hist[e] = 0;
  __syncthreads();

  const int64_t c = static_cast<int64_t>(blockIdx.x) * kChunk + tid;
  bool bad;
  int32_t token;
  const int32_t e = read_expert(idx, c, n, tokens, num_experts, valid_tokens, &bad, &token);
  const bool valid = e >= 0;
  // One LDS add per distinct expert in the wave instead of one per copy:
  // skewed routing would otherwise serialize 64 adds on one address.
  const uint64_t peers = same_expert_lanes(valid, e, num_bits);
  if (valid && (peers & lanes_below()) == 0) atomicAdd(&hist[e], __popcll(peers));
  const uint64_t bad_lanes = __ballot(bad);
  if ((tid & 63) == 0 && bad_lanes != 0) atomicAdd(&hist[num_experts], __popcll(bad_lanes));
  __syncthreads();

  int32_t* row = counts + static_cast<int64_t>(blockIdx.x) * (num_experts + 1);
  for (int e2 = tid; e2 <= num_experts; e2 += kChunk) row[e2] = hist[e2];
}

// Inclusive scan over the 1024 lanes of one workgroup.
__device__ __forceinline__ int64_t block_inclusive_scan(int64_t v, int64_t* wave_sums) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  for (int d = 1; d < 64; d <<= 1) {
    const int64_t below = __shfl_up(v, d, 64);
    if (lane >= d) v += below;
  }
  if (lane == 63) wave_sums[wave] = v;
  __syncthreads();
  if (wave == 0) {
    int64_t s = lane < kWaves ? wave_sums[lane] : 0;
    for (int d = 1; d < kWaves; d <<= 1) {
      const int64_t below = __shfl_up(s, d, 64);
      if (lane >= d) s += below;
    }
    if (lane < kWaves) wave_sums[lane] = s;
  }
  __syncthreads();
  return v + (wave > 0 ? wave_sums[wave - 1] : 0);
}

__global__ void __launch_bounds__(kChunk) route_offsets_kernel(int32_t* __restrict__ counts, int32_t num_chunks,
                                                               int32_t num_experts, int32_t block_size,
                                                               int32_t* __restrict__ tokens_per_expert,
                                                               int32_t* __restrict__ padded_offsets,
                                                               int32_t* __restrict__ error) {
  __shared__ int64_t wave_sums[kWaves];
  const int tid = threadIdx.x;
  const int64_t stride = num_experts + 1;
  int64_t padded = 0;
  // Column col: copies of expert col (or bad ids, col == E) in each chunk,
  // replaced in place by the copies in all earlier chunks. The loads do not
  // depend on each other, so the unrolled walk keeps several in flight.
  for (int col = tid; col <= num_experts; col += kChunk) {
    int32_t total = 0;
    int32_t b = 0;
    for (; b + 4 <= num_chunks; b += 4) {
      int32_t* p = counts + b * stride + col;
      const int32_t c0 = p[0], c1 = p[stride], c2 = p[2 * stride], c3 = p[3 * stride];
      p[0] = total;
      p[stride] = total + c0;
      p[2 * stride] = total + c0 + c1;
      p[3 * stride] = total + c0 + c1 + c2;
      total += c0 + c1 + c2 + c3;
    }
    for (; b < num_chunks; ++b) {
      int32_t* p = counts + b * stride + col;
      const int32_t c0 = *p;
      *p = total;
      total += c0;
    }
    if (col < num_experts) {
      tokens_per_expert[col] = total;
      padded = (static_cast<int64_t>(total) + block_size - 1) / block_size * block_size;
    } else {
      error[0] = total > 0 ? 1 : 0;
    }
  }
  const int64_t incl = block_inclusive_scan(tid < num_experts ? padded : 0, wave_sums);
  if (tid < num_experts) padded_offsets[tid + 1] = static_cast<int32_t>(incl);
  if (tid == 0) padded_offsets[0] = 0;
}

template <typename Idx, typename Tok>
__global__ void __launch_bounds__(kChunk)
    route_place_kernel(const Idx* __restrict__ idx, int64_t n, TokenSource<Tok> tokens, int32_t num_experts,
                       int32_t num_bits,
                       const int32_t* __restrict__ valid_tokens, int32_t num_chunks,
                       const int32_t* __restrict__ chunk_base, const int32_t* __restrict__ tokens_per_expert,
                       const int32_t* __restrict__ padded_offsets, int32_t block_size, int32_t ffn_blocks,
                       int32_t max_row_blocks, int64_t max_rows, int32_t* __restrict__ copy_row,
                       int32_t* __restrict__ row_token, int32_t* __restrict__ row_block_expert,
                       int32_t* __restrict__ row_offsets, int32_t* __restrict__ col_indices) {
  __shared__ int32_t lds[kWaves * kMaxExperts];  // place: per-wave counts; layout: offsets + counts
  const int tid = threadIdx.x;

  if (static_cast<int32_t>(blockIdx.x) < num_chunks) {
    // ---- place: copy -> row, stable inside each expert ----
    const int lane = tid & 63;
    const int wave = tid >> 6;
    for (int i = tid; i < kWaves * num_experts; i += kChunk) lds[i] = 0;
    __syncthreads();

    const int64_t c = static_cast<int64_t>(blockIdx.x) * kChunk + tid;
    bool bad;
    int32_t token;
    const int32_t e = read_expert(idx, c, n, tokens, num_experts, valid_tokens, &bad, &token);
    const bool valid = e >= 0;
    const uint64_t peers = same_expert_lanes(valid, e, num_bits);
    const uint64_t lower = peers & lanes_below();
    if (valid && lower == 0) lds[wave * num_experts + e] = __popcll(peers);  // one writer per (wave, e)
    __syncthreads();
    (void)lane;

    if (valid) {
      int32_t before = 0;
      for (int w = 0; w < wave; ++w) before += lds[w * num_experts + e];
      const int32_t row = padded_offsets[e] +
                          chunk_base[static_cast<int64_t>(blockIdx.x) * (num_experts + 1) + e] + before +
                          __popcll(lower);
      copy_row[c] = row;
      row_token[row] = token;
    } else if (c < n) {
      copy_row[c] = -1;
    }
    return;
  }

  // ---- layout: BSR arrays and the -1 marks of non-copy rows ----
  int32_t* offs = lds;                    // [E+1] padded_offsets
  int32_t* cnts = lds + kMaxExperts + 1;  // [E] tokens_per_expert (E <= 1024, fits the array)
  for (int e = tid; e <= num_experts; e += kChunk) offs[e] = padded_offsets[e];
  for (int e = tid; e < num_experts; e += kChunk) cnts[e] = tokens_per_expert[e];
  __syncthreads();
  const int64_t i = static_cast<int64_t>(blockIdx.x - num_chunks) * kLayoutItemsPerGroup + tid;
  layout_item(i, offs, cnts, num_experts, block_size, ffn_blocks, max_row_blocks, max_rows, row_token,
              row_block_expert, row_offsets, col_indices);
}

// Place and layout for at most kScanChunks chunks, straight from the count
// kernel's per-chunk counts: each workgroup sums every expert's column
// itself (one lane per expert; num_chunks loads each), over the chunks
// before its own and over all of them, and scans the padded sizes in LDS.
// That replaces the one-workgroup offsets kernel and its launch. Workgroup 0
// also writes tokens_per_expert, padded_offsets and the error flag. The
// rest is route_place_kernel's placement and layout.
constexpr int kScanChunks = 32;

template <typename Idx, typename Tok>
__global__ void __launch_bounds__(kChunk)
    route_place_scan_kernel(const Idx* __restrict__ idx, int64_t n, TokenSource<Tok> tokens, int32_t num_experts,
                            int32_t num_bits, const int32_t* __restrict__ valid_tokens, int32_t num_chunks,
                            const int32_t* __restrict__ counts, int32_t block_size, int32_t ffn_blocks,
                            int32_t max_row_blocks, int64_t max_rows, int32_t* __restrict__ tokens_per_expert,
                            int32_t* __restrict__ padded_offsets, int32_t* __restrict__ error,
                            int32_t* __restrict__ copy_row, int32_t* __restrict__ row_token,
                            int32_t* __restrict__ row_block_expert, int32_t* __restrict__ row_offsets,
                            int32_t* __restrict__ col_indices) {
  __shared__ int32_t total[kMaxExperts];   // copies of each expert in all chunks
  __shared__ int32_t before[kMaxExperts];  // copies of each expert in the chunks before this one
  __shared__ int32_t offs[kMaxExperts + 1];
  __shared__ int32_t wave_counts[kWaves * kMaxExperts];
  __shared__ int64_t wave_sums[kWaves];
  const int tid = threadIdx.x;
  const bool placing = static_cast<int32_t>(blockIdx.x) < num_chunks;
  const int own = placing ? static_cast<int>(blockIdx.x) : num_chunks;
  const int64_t stride = num_experts + 1;
  // This lane's copy, read before the column sums so that its load waits
  // alongside theirs rather than after the scan.
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kChunk + tid;
  bool bad = false;
  int32_t token = -1;
  const int32_t e = placing ? read_expert(idx, c, n, tokens, num_experts, valid_tokens, &bad, &token) : -1;

  // Column tid (expert tid): all of its at most kScanChunks loads are issued
  // before the first is used, so they are in flight together.
  int32_t sum_before = 0, sum_all = 0;
  if (tid < num_experts) {
    int32_t v[kScanChunks];
#pragma unroll
    for (int b = 0; b < kScanChunks; ++b) v[b] = b < num_chunks ? counts[b * stride + tid] : 0;
#pragma unroll
    for (int b = 0; b < kScanChunks; ++b) {
      sum_before += b < own ? v[b] : 0;
      sum_all += v[b];
    }
    total[tid] = sum_all;
    before[tid] = sum_before;
  }
  const int64_t padded =
      tid < num_experts ? (static_cast<int64_t>(sum_all) + block_size - 1) / block_size * block_size : 0;
  const int64_t incl = block_inclusive_scan(padded, wave_sums);  // synchronizes the workgroup
  if (tid < num_experts) offs[tid + 1] = static_cast<int32_t>(incl);
  if (tid == 0) offs[0] = 0;
  if (blockIdx.x == 0) {
    if (tid < num_experts) {
      tokens_per_expert[tid] = sum_all;
      padded_offsets[tid + 1] = static_cast<int32_t>(incl);
    }
    if (tid == 0) {
      padded_offsets[0] = 0;
      int32_t bad = 0;  // column E: copies with a bad id
      for (int b = 0; b < num_chunks; ++b) bad += counts[b * stride + num_experts];
      error[0] = bad > 0 ? 1 : 0;
    }
  }

  if (placing) {
    for (int i = tid; i < kWaves * num_experts; i += kChunk) wave_counts[i] = 0;
    __syncthreads();
    const int wave = tid >> 6;
    const bool valid = e >= 0;
    const uint64_t peers = same_expert_lanes(valid, e, num_bits);
    const uint64_t lower = peers & lanes_below();
    if (valid && lower == 0) wave_counts[wave * num_experts + e] = __popcll(peers);
    __syncthreads();
    if (valid) {
      int32_t in_waves = 0;
      for (int w = 0; w < wave; ++w) in_waves += wave_counts[w * num_experts + e];
      const int32_t row = offs[e] + before[e] + in_waves + __popcll(lower);
      copy_row[c] = row;
      row_token[row] = token;
    } else if (c < n) {
      copy_row[c] = -1;
    }
    return;
  }
  __syncthreads();
  const int64_t i = static_cast<int64_t>(blockIdx.x - num_chunks) * kLayoutItemsPerGroup + tid;
  layout_item(i, offs, total, num_experts, block_size, ffn_blocks, max_row_blocks, max_rows, row_token,
              row_block_expert, row_offsets, col_indices);
}

int bits_for(int32_t num_experts) {
  int b = 0;
  while ((1 << b) < num_experts) ++b;
  return b;
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" int sb_routing_sizes(int64_t num_copies, int32_t num_experts, int32_t ffn_dim, int32_t block_size,
                                int64_t* max_row_blocks, int64_t* max_rows, int64_t* workspace_elems) {
  constexpr int64_t kI32Max = 2147483647;
  if (num_copies <= 0) return fail(SB_ERR_INVALID, "expert_idx must be [T, k] with T, k > 0");
  if (num_experts <= 0 || num_experts > kMaxExperts)
    return fail(SB_ERR_INVALID, "num_experts must be in [1, %d], got %d", kMaxExperts, num_experts);
  if (block_size <= 0) return fail(SB_ERR_INVALID, "block_size must be in [1, 2^31)");
  if (ffn_dim <= 0 || ffn_dim % block_size != 0)
    return fail(SB_ERR_INVALID, "ffn_dim (%d) must be a positive multiple of block_size (%d)", ffn_dim, block_size);
  if (num_copies > kI32Max) return fail(SB_ERR_INVALID, "problem too large for int32 indexing");
  const int64_t rb = (num_copies + static_cast<int64_t>(num_experts) * (block_size - 1)) / block_size;
  const int64_t rows = rb * block_size;
  const int64_t ffn_blocks = ffn_dim / block_size;
  if (rows > kI32Max / ffn_dim || rb * ffn_blocks >= kI32Max)
    return fail(SB_ERR_INVALID, "problem too large for int32 indexing");
  const int64_t chunks = (num_copies + kChunk - 1) / kChunk;
  if (max_row_blocks) *max_row_blocks = rb;
  if (max_rows) *max_rows = rows;
  if (workspace_elems) *workspace_elems = chunks * (num_experts + 1);
  return clear_ok();
}

namespace sb {
namespace {

// Routing of n copies whose tokens come from `tokens`: count, then place with
// the offsets scan inside for at most kScanChunks chunks; count, offsets and
// place beyond.
template <typename Idx, typename Tok>
int launch_routing(const Idx* idx, int64_t n, TokenSource<Tok> tokens, int32_t num_experts, int32_t ffn_dim,
                   int32_t block_size, const int32_t* valid_tokens, int32_t* workspace, int32_t* tokens_per_expert,
                   int32_t* padded_offsets, int32_t* row_token, int32_t* copy_row, int32_t* row_block_expert,
                   int32_t* row_offsets, int32_t* col_indices, int32_t* error, hipStream_t stream) {
  int64_t max_row_blocks = 0, max_rows = 0, ws = 0;
  if (int rc = sb_routing_sizes(n, num_experts, ffn_dim, block_size, &max_row_blocks, &max_rows, &ws)) return rc;
  const int32_t num_chunks = static_cast<int32_t>((n + kChunk - 1) / kChunk);
  const int32_t ffn_blocks = ffn_dim / block_size;
  const int num_bits = bits_for(num_experts);
  const int64_t layout_items = std::max<int64_t>(max_row_blocks * ffn_blocks + 1, max_rows);
  const int32_t layout_groups = static_cast<int32_t>((layout_items + kLayoutItemsPerGroup - 1) / kLayoutItemsPerGroup);

  route_count_kernel<Idx, Tok><<<num_chunks, kChunk, 0, stream>>>(idx, n, tokens, num_experts, num_bits,
                                                                  valid_tokens, workspace);
  if (int rc = check_launch("routing count")) return rc;
  if (num_chunks <= kScanChunks) {
    route_place_scan_kernel<Idx, Tok><<<num_chunks + layout_groups, kChunk, 0, stream>>>(
        idx, n, tokens, num_experts, num_bits, valid_tokens, num_chunks, workspace, block_size, ffn_blocks,
        static_cast<int32_t>(max_row_blocks), max_rows, tokens_per_expert, padded_offsets, error, copy_row, row_token,
        row_block_expert, row_offsets, col_indices);
    return check_launch("routing place");
  }
  route_offsets_kernel<<<1, kChunk, 0, stream>>>(workspace, num_chunks, num_experts, block_size, tokens_per_expert,
                                                 padded_offsets, error);
  if (int rc = check_launch("routing offsets")) return rc;
  route_place_kernel<Idx, Tok><<<num_chunks + layout_groups, kChunk, 0, stream>>>(
      idx, n, tokens, num_experts, num_bits, valid_tokens, num_chunks, workspace, tokens_per_expert, padded_offsets,
      block_size, ffn_blocks, static_cast<int32_t>(max_row_blocks), max_rows, copy_row, row_token, row_block_expert,
      row_offsets, col_indices);
  return check_launch("routing place");
}

}  // namespace
}  // namespace sb

extern "C" int sb_routing(const void* expert_idx, int32_t idx_is_i64, int64_t num_tokens, int32_t k,
                          int32_t num_experts, int32_t ffn_dim, int32_t block_size, const int32_t* valid_tokens,
                          int32_t* workspace, int32_t* tokens_per_expert, int32_t* padded_offsets,
                          int32_t* row_token, int32_t* copy_row, int32_t* row_block_expert, int32_t* row_offsets,
                          int32_t* col_indices, int32_t* error, void* stream_ptr) {
  if (num_tokens <= 0 || k <= 0) return fail(SB_ERR_INVALID, "expert_idx must be [T, k] with T, k > 0");
  const int64_t n = num_tokens * k;
  int64_t max_row_blocks = 0, max_rows = 0, ws = 0;
  if (int rc = sb_routing_sizes(n, num_experts, ffn_dim, block_size, &max_row_blocks, &max_rows, &ws)) return rc;
  if (!expert_idx || !workspace || !tokens_per_expert || !padded_offsets || !row_token || !copy_row ||
      !row_block_expert || !row_offsets || !col_indices || !error)
    return fail(SB_ERR_INVALID, "sb_routing: null buffer");
  const TokenSource<int32_t> tokens{nullptr, k, num_tokens};
  const hipStream_t stream = as_stream(stream_ptr);
  const int rc = idx_is_i64
                     ? launch_routing(static_cast<const int64_t*>(expert_idx), n, tokens, num_experts, ffn_dim,
                                      block_size, valid_tokens, workspace, tokens_per_expert, padded_offsets,
                                      row_token, copy_row, row_block_expert, row_offsets, col_indices, error, stream)
                     : launch_routing(static_cast<const int32_t*>(expert_idx), n, tokens, num_experts, ffn_dim,
                                      block_size, valid_tokens, workspace, tokens_per_expert, padded_offsets,
                                      row_token, copy_row, row_block_expert, row_offsets, col_indices, error, stream);
  return rc ? rc : clear_ok();
}

extern "C" int sb_routing_assigned(const void* expert_of_copy, int32_t expert_is_i64, const void* token_of_copy,
                                   int32_t token_is_i64, int64_t num_copies, int64_t num_tokens, int32_t num_experts,
                                   int32_t ffn_dim, int32_t block_size, const int32_t* valid_tokens,
                                   int32_t* workspace, int32_t* tokens_per_expert, int32_t* padded_offsets,
                                   int32_t* row_token, int32_t* copy_row, int32_t* row_block_expert,
                                   int32_t* row_offsets, int32_t* col_indices, int32_t* error, void* stream_ptr) {
  if (num_copies <= 0) return fail(SB_ERR_INVALID, "routing: the assignment list must not be empty");
  if (num_tokens <= 0 || num_tokens > 2147483647LL) return fail(SB_ERR_INVALID, "routing: bad token count");
  int64_t max_row_blocks = 0, max_rows = 0, ws = 0;
  if (int rc = sb_routing_sizes(num_copies, num_experts, ffn_dim, block_size, &max_row_blocks, &max_rows, &ws))
    return rc;
  if (!expert_of_copy || !token_of_copy || !workspace || !tokens_per_expert || !padded_offsets || !row_token ||
      !copy_row || !row_block_expert || !row_offsets || !col_indices || !error)
    return fail(SB_ERR_INVALID, "sb_routing_assigned: null buffer");
  const hipStream_t stream = as_stream(stream_ptr);
  auto run = [&](auto tok_ptr) {
    using Tok = std::remove_cv_t<std::remove_pointer_t<decltype(tok_ptr)>>;
    const TokenSource<Tok> tokens{tok_ptr, 1, num_tokens};
    return expert_is_i64
               ? launch_routing(static_cast<const int64_t*>(expert_of_copy), num_copies, tokens, num_experts,
                                ffn_dim, block_size, valid_tokens, workspace, tokens_per_expert, padded_offsets,
                                row_token, copy_row, row_block_expert, row_offsets, col_indices, error, stream)
               : launch_routing(static_cast<const int32_t*>(expert_of_copy), num_copies, tokens, num_experts,
                                ffn_dim, block_size, valid_tokens, workspace, tokens_per_expert, padded_offsets,
                                row_token, copy_row, row_block_expert, row_offsets, col_indices, error, stream);
  };
  const int rc = token_is_i64 ? run(static_cast<const int64_t*>(token_of_copy))
                              : run(static_cast<const int32_t*>(token_of_copy));
  return rc ? rc : clear_ok();
}

// ---- sb_routing_noalloc: sb_routing with its scratch in a fixed device array
//
// The only scratch of routing is the per-chunk expert counts that sb_routing
// takes as `workspace` (ceil(n / 1024) * (E + 1) int32). This entry point
// keeps them in `scratch`, a file-scope device array of kScratchElems int32
// (2 MiB) that every GPU the library runs on holds until the process ends,
// so a caller that cannot allocate (graph capture, a serving loop, a
// harness that forbids hipMalloc) passes only inputs and outputs.
//
// The host never names `scratch` itself (its host-side symbol is not a
// device address): on the first call on a device (the device of the call's
// stream), with that device current, hipGetSymbolAddress gives that
// device's copy, and the pointer is kept per device and passed to the
// kernels.
//
// Nothing in it has to start at zero: the count kernel writes every entry
// of the chunks it covers before the offsets kernel reads it. Calls that
// overlap on one GPU (two streams, or a graph replay beside an eager call)
// share the array and race.

namespace sb {
namespace {

constexpr int64_t kScratchElems = int64_t{1} << 19;

__device__ __attribute__((aligned(256))) int32_t scratch[kScratchElems];

// The array of the device that `stream` belongs to (the current device for
// the null stream): the kernels run there, whichever device is current.
int scratch_for_stream(hipStream_t stream, int32_t** out) {
  constexpr int kMaxDevices = 64;
  static std::mutex mu;
  static int32_t* ptrs[kMaxDevices] = {};
  int current = 0;
  if (hipGetDevice(&current) != hipSuccess) return fail(SB_ERR_HIP, "routing_noalloc: no current device");
  int dev = current;
  if (stream != nullptr) {
    hipDevice_t d = 0;
    if (hipStreamGetDevice(stream, &d) != hipSuccess)
      return fail(SB_ERR_HIP, "routing_noalloc: cannot read the stream's device");
    dev = static_cast<int>(d);
  }
  if (dev < 0 || dev >= kMaxDevices) return fail(SB_ERR_HIP, "routing_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (ptrs[dev] == nullptr) {
    // hipGetSymbolAddress answers for the current device: make the
    // stream's device current for the lookup, then restore the caller's.
    if (dev != current && hipSetDevice(dev) != hipSuccess)
      return fail(SB_ERR_HIP, "routing_noalloc: cannot select device %d", dev);
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (dev != current && hipSetDevice(current) != hipSuccess)
      return fail(SB_ERR_HIP, "routing_noalloc: cannot restore device %d", current);
    if (e != hipSuccess || p == nullptr)
      return fail(SB_ERR_HIP, "routing_noalloc: hipGetSymbolAddress of the scratch array failed: %s",
                  hipGetErrorString(e));
    ptrs[dev] = static_cast<int32_t*>(p);
  }
  *out = ptrs[dev];
  return SB_OK;
}

}  // namespace
}  // namespace sb

extern "C" int sb_routing_noalloc(const void* expert_idx, int32_t idx_is_i64, int64_t num_tokens, int32_t k,
                                  int32_t num_experts, int32_t ffn_dim, int32_t block_size,
                                  const int32_t* valid_tokens, int32_t* tokens_per_expert, int32_t* padded_offsets,
                                  int32_t* row_token, int32_t* copy_row, int32_t* row_block_expert,
                                  int32_t* row_offsets, int32_t* col_indices, int32_t* error, void* stream) {
  if (num_tokens <= 0 || k <= 0) return fail(SB_ERR_INVALID, "expert_idx must be [T, k] with T, k > 0");
  int64_t max_row_blocks = 0, max_rows = 0, ws = 0;
  if (int rc = sb_routing_sizes(num_tokens * k, num_experts, ffn_dim, block_size, &max_row_blocks, &max_rows, &ws))
    return rc;
  if (ws > kScratchElems)
    return fail(SB_ERR_INVALID,
                "routing_noalloc: %lld copies over %d experts need %lld int32 of scratch, more than the %lld of "
                "the fixed array (use sb_routing with a workspace)",
                static_cast<long long>(num_tokens * k), num_experts, static_cast<long long>(ws),
                static_cast<long long>(kScratchElems));
  int32_t* ws_ptr = nullptr;
  if (int rc = scratch_for_stream(as_stream(stream), &ws_ptr)) return rc;
  return sb_routing(expert_idx, idx_is_i64, num_tokens, k, num_experts, ffn_dim, block_size, valid_tokens, ws_ptr,
                    tokens_per_expert, padded_offsets, row_token, copy_row, row_block_expert, row_offsets,
                    col_indices, error, stream);
}
