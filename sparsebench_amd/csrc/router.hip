// Router side of the MoE layer on gfx950: plain top-k and token rounding
// (the reference's sparsebench/token_rounding.py: top_k_assignments at
// 39-46, round_counts at 49-55, token_rounding at 58-81), with the rounding
// fused into routing: scores go in, and out come the assignment list and
// the block-sparse layout that SDD / DSD / the assigned combine consume,
// with no host sync (the reference needs one, for nonzero()).
//
// Token rounding, per expert e (f_e = its top-k count):
//   target_e = f_e rounded to the nearest multiple of the tile, ties down,
//              at most floor(T / tile) * tile;
//   keep (t, e) for the target_e best tokens of column e, where picks keep
//   their score s and the others rank at s - 1, ties going to the lower
//   token (the reference's stable descending sort);
//   weight (t, e) = s[t, e] / sum of s over t's kept experts, the sum taken
//   in ascending expert order.
// The list is in (token, expert) order, like the reference's nonzero().
//
// Launches:
//   1. topk      one lane per token (one wave per token when E x k is
//                large): the k best experts (value, then lower index),
//                per-chunk pick counts, the shifted scores stored
//                expert-major, and (for top_k_assignments) the list itself.
//   2. targets   one workgroup: counts -> targets -> padded_offsets.
//   3. select    one workgroup per expert: radix select (4 passes of 8 bits)
//                of the target-th largest shifted score, then the keep
//                bitmask, its per-word prefix counts and row_token.
//   4. tokens    one wave per token: kept count and score total.
//   5. scan      one workgroup: token_offsets (and the list length).
//   6. emit      one wave per token: token / expert / weight / copy_row.
//   7. layout    row_offsets, col_indices, row_block_expert, -1 rows.

#include "common.hpp"
#include "layout.hpp"

namespace sb {
namespace {

constexpr int kTopkTokensPerGroup = 64;  // 4 waves x 16 tokens
constexpr int kTopkThreads = 256;
constexpr int kMaxPerLane = kMaxExperts / 64;
constexpr int kSelectThreads = 1024;
constexpr int kTokenWaves = 4;  // tokens kernel / emit kernel: waves per workgroup

// Order-preserving map of a float to uint32 (larger float -> larger key).
// -0 counts as +0 and every NaN as the largest value, as in a sort that
// compares values.
__device__ __forceinline__ uint32_t sort_key(float f) {
  if (f == 0.0f) f = 0.0f;
  uint32_t u = __float_as_uint(f);
  if (f != f) u = 0x7fc00000u;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Better of two (score, expert) candidates: higher score, then lower index.
__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
  return a > b || (a == b && ia < ib);
}

template <int PER>
__global__ void __launch_bounds__(kTopkThreads)
    router_topk_kernel(const float* __restrict__ scores, int64_t num_tokens, int32_t num_experts, int32_t k,
                       float* __restrict__ shifted, int32_t* __restrict__ chunk_counts,
                       int32_t* __restrict__ top_idx, float* __restrict__ top_weight) {
  // With E <= 256 the shifted scores go through an LDS tile [E][64 tokens]
  // so that the expert-major stores are 64-token rows, not scattered words.
  constexpr bool kTile = PER <= 4;
  constexpr int kTileStride = kTopkTokensPerGroup + 1;
  constexpr int kPerWave = kTopkTokensPerGroup / 4;
  // Tokens whose scores are loaded together (all loads in flight at once).
  constexpr int kBatch = PER <= 2 ? kPerWave : PER <= 4 ? 8 : 4;
  __shared__ int32_t hist[kMaxExperts];
  __shared__ float tile[kTile ? 64 * PER * kTileStride : 1];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (chunk_counts != nullptr)
    for (int e = tid; e < num_experts; e += kTopkThreads) hist[e] = 0;
  __syncthreads();

  const int64_t group_base = static_cast<int64_t>(blockIdx.x) * kTopkTokensPerGroup;
  for (int j0 = 0; j0 < kPerWave; j0 += kBatch) {
    float vb[kBatch][PER];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int64_t t = group_base + wave * kPerWave + j0 + b;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int e = lane + 64 * i;
        vb[b][i] = (t < num_tokens && e < num_experts) ? scores[t * num_experts + e] : 0.0f;
      }
    }
    // The k rounds of all kBatch tokens in lockstep: their shuffle chains
    // are independent, so they overlap instead of running one after another.
    uint32_t picked[kBatch];
    float total[kBatch];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      picked[b] = 0;
      total[b] = 0.0f;
    }
    for (int r = 0; r < k; ++r) {
      float bv[kBatch];
      int bi[kBatch];
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        bv[b] = 0.0f;
        bi[b] = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int e = lane + 64 * i;
          if (e < num_experts && !((picked[b] >> i) & 1u) && (bi[b] == 0x7fffffff || better(vb[b][i], e, bv[b], bi[b]))) {
            bv[b] = vb[b][i];
            bi[b] = e;
          }
        }
      }
      for (int d = 32; d >= 1; d >>= 1) {
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
          const float ov = __shfl_xor(bv[b], d, 64);
          const int oi = __shfl_xor(bi[b], d, 64);
          if (oi != 0x7fffffff && (bi[b] == 0x7fffffff || better(ov, oi, bv[b], bi[b]))) {
            bv[b] = ov;
            bi[b] = oi;
          }
        }
      }
#pragma unroll
      for (int b = 0; b < kBatch; ++b) {
        // bi[b]: the r-th best expert of token b, the same in every lane.
        if ((bi[b] & 63) == lane) picked[b] |= 1u << (bi[b] >> 6);
        total[b] += bv[b];  // in pick order, as a sum over the k picks
        const int64_t t = group_base + wave * kPerWave + j0 + b;
        if (lane == 0 && t < num_tokens) {
          if (top_idx != nullptr) top_idx[t * k + r] = bi[b];
          if (top_weight != nullptr) top_weight[t * k + r] = bv[b];  // raw score; normalized below
        }
      }
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int t_local = wave * kPerWave + j0 + b;
      const int64_t t = group_base + t_local;
      if (t >= num_tokens) break;
      // Weights: the picked scores over their sum (lane 0 reads back what it wrote).
      if (top_weight != nullptr && lane == 0)
        for (int r = 0; r < k; ++r) top_weight[t * k + r] = top_weight[t * k + r] / total[b];
      if (shifted != nullptr) {
#pragma unroll
        for (int i = 0; i < PER; ++i) {
          const int e = lane + 64 * i;
          if (e < num_experts) {
            const float sv = ((picked[b] >> i) & 1u) ? vb[b][i] : vb[b][i] - 1.0f;
            if constexpr (kTile) tile[e * kTileStride + t_local] = sv;
            else shifted[static_cast<int64_t>(e) * num_tokens + t] = sv;
          }
        }
      }
      if (chunk_counts != nullptr) {
#pragma unroll
        for (int i = 0; i < PER; ++i)
          if ((picked[b] >> i) & 1u) atomicAdd(&hist[lane + 64 * i], 1);
      }
    }
  }
  __syncthreads();
  if constexpr (kTile) {
    if (shifted != nullptr) {
      for (int i = tid; i < num_experts * kTopkTokensPerGroup; i += kTopkThreads) {
        const int e = i / kTopkTokensPerGroup, tl = i % kTopkTokensPerGroup;
        const int64_t t = group_base + tl;
        if (t < num_tokens) shifted[static_cast<int64_t>(e) * num_tokens + t] = tile[e * kTileStride + tl];
      }
    }
  }
  if (chunk_counts != nullptr)
    for (int e = tid; e < num_experts; e += kTopkThreads)
      chunk_counts[static_cast<int64_t>(blockIdx.x) * num_experts + e] = hist[e];
}

// Top-k with one lane per token (a wave of 64 tokens per workgroup, the
// same chunking as router_topk_kernel). The lane walks its token's row of
// scores in expert order and keeps the KMAX best in registers, sorted by
// (score desc, expert asc): each new (score, e) is bubbled in with
// compare-and-swap steps, so an equal score behind an earlier expert stays
// behind it. No lane talks to another, and the expert-major stores of the
// shifted scores are 64 consecutive tokens per instruction. The outputs are
// those of router_topk_kernel.
template <int KMAX>
__global__ void __launch_bounds__(64)
    router_topk_lane_kernel(const float* __restrict__ scores, int64_t num_tokens, int32_t num_experts, int32_t k,
                            float* __restrict__ shifted, int32_t* __restrict__ chunk_counts,
                            int32_t* __restrict__ top_idx, float* __restrict__ top_weight) {
  __shared__ int32_t hist[kMaxExperts];
  __shared__ uint32_t picked_bits[64 * (kMaxExperts / 32)];  // lane-major: this lane's picks, one bit per expert
  const int lane = threadIdx.x;
  const int words = (num_experts + 31) / 32;
  if (chunk_counts != nullptr)
    for (int e = lane; e < num_experts; e += 64) hist[e] = 0;
  for (int w = 0; w < words; ++w) picked_bits[lane * words + w] = 0u;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 64 + lane;
  const bool live = t < num_tokens;
  const float* row = scores + (live ? t : 0) * num_experts;

  float bv[KMAX];
  int bi[KMAX];
#pragma unroll
  for (int j = 0; j < KMAX; ++j) {
    bv[j] = 0.0f;
    bi[j] = 0x7fffffff;  // empty
  }
  auto offer = [&](float v, int e) {
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j < k && (bi[j] == 0x7fffffff || better(v, e, bv[j], bi[j]))) {
        const float tv = bv[j];
        const int ti = bi[j];
        bv[j] = v;
        bi[j] = e;
        v = tv;
        e = ti;
      }
    }
  };
  if (live) {
    int e = 0;
    if ((num_experts & 3) == 0 && (reinterpret_cast<uintptr_t>(scores) & 15) == 0) {
      // 16 scores (four 16-byte loads) in flight at a time.
      for (; e + 16 <= num_experts; e += 16) {
        float4 q[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) q[u] = *reinterpret_cast<const float4*>(row + e + 4 * u);
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          offer(q[u].x, e + 4 * u);
          offer(q[u].y, e + 4 * u + 1);
          offer(q[u].z, e + 4 * u + 2);
          offer(q[u].w, e + 4 * u + 3);
        }
      }
    }
    for (; e < num_experts; ++e) offer(row[e], e);
  }
  __syncthreads();  // hist and picked_bits cleared
  if (live) {
    float total = 0.0f;
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      if (j < k && bi[j] != 0x7fffffff) {
        total += bv[j];  // in pick order
        picked_bits[lane * words + (bi[j] >> 5)] |= 1u << (bi[j] & 31);
        if (chunk_counts != nullptr) atomicAdd(&hist[bi[j]], 1);
        if (top_idx != nullptr) top_idx[t * k + j] = bi[j];
      }
    }
    if (top_weight != nullptr)
#pragma unroll
      for (int j = 0; j < KMAX; ++j)
        if (j < k) top_weight[t * k + j] = bv[j] / total;
    if (shifted != nullptr) {
      for (int e = 0; e < num_experts; ++e) {
        const float v = row[e];
        const bool pick = (picked_bits[lane * words + (e >> 5)] >> (e & 31)) & 1u;
        shifted[static_cast<int64_t>(e) * num_tokens + t] = pick ? v : v - 1.0f;
      }
    }
  }
  if (chunk_counts != nullptr) {
    __syncthreads();
    for (int e = lane; e < num_experts; e += 64)
      chunk_counts[static_cast<int64_t>(blockIdx.x) * num_experts + e] = hist[e];
  }
}

// Inclusive scan over the lanes of one 1024-lane workgroup.
__device__ __forceinline__ int32_t block_scan_1024(int32_t v, int32_t* wave_sums, int32_t* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int d = 1; d < 64; d <<= 1) {
    const int32_t below = __shfl_up(v, d, 64);
    if (lane >= d) v += below;
  }
  if (lane == 63) wave_sums[wave] = v;
  __syncthreads();
  int32_t before = 0, all = 0;
  for (int w = 0; w < 16; ++w) {
    if (w < wave) before += wave_sums[w];
    all += wave_sums[w];
  }
  __syncthreads();
  *total = all;
  return v + before;
}

__global__ void __launch_bounds__(1024)
    router_targets_kernel(const int32_t* __restrict__ chunk_counts, int32_t num_chunks, int32_t num_experts,
                          int64_t num_tokens, int32_t tile, int32_t block_size, int32_t* __restrict__ target,
                          int32_t* __restrict__ padded_offsets, int32_t* __restrict__ error) {
  __shared__ int32_t counts[kMaxExperts];
  __shared__ int32_t wave_sums[16];
  const int tid = threadIdx.x;
  for (int e = tid; e < num_experts; e += 1024) counts[e] = 0;
  __syncthreads();
  // Column sums of chunk_counts [chunks, E], read in order, 8 loads in flight per lane.
  constexpr int kPer = 8;
  const int64_t total_items = static_cast<int64_t>(num_chunks) * num_experts;
  for (int64_t base = 0; base < total_items; base += 1024 * kPer) {
    int32_t v[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const int64_t i = base + u * 1024 + tid;
      v[u] = i < total_items ? chunk_counts[i] : 0;
    }
#pragma unroll
    for (int u = 0; u < kPer; ++u)
      if (v[u] != 0) atomicAdd(&counts[(base + u * 1024 + tid) % num_experts], v[u]);
  }
  __syncthreads();
  int32_t padded = 0;
  if (tid < num_experts) {
    const int32_t f = counts[tid];
    const int32_t low = f / tile * tile;
    const int32_t high = low + (f % tile > 0 ? tile : 0);
    int32_t rounded = (high - f < f - low) ? high : low;  // nearest, ties down
    const int64_t cap = num_tokens / tile * tile;
    if (rounded > cap) rounded = static_cast<int32_t>(cap);
    target[tid] = rounded;
    padded = (rounded + block_size - 1) / block_size * block_size;
  }
  int32_t total;
  const int32_t incl = block_scan_1024(padded, wave_sums, &total);
  if (tid < num_experts) padded_offsets[tid + 1] = incl;
  if (tid == 0) {
    padded_offsets[0] = 0;
    error[0] = 0;
  }
}

__device__ __forceinline__ uint64_t lanes_below() {
  const int lane = threadIdx.x & 63;
  return lane == 0 ? 0ull : (~0ull >> (64 - lane));
}

// hist[bin] += 1 for every active lane, one LDS atomic per distinct bin in
// the wave (lanes with the same bin found by one ballot per bin bit).
// Softmax scores share few top-byte values, so plain per-lane atomics
// would pile onto one or two addresses.
__device__ __forceinline__ void wave_hist_add(int32_t* hist, uint32_t bin, bool active) {
  uint64_t peers = __ballot(active);
#pragma unroll
  for (int b = 0; b < 8; ++b) {
    const bool bit = (bin >> b) & 1u;
    const uint64_t ones = __ballot(active && bit);
    peers &= bit ? ones : ~ones;
  }
  if (active && (peers & lanes_below()) == 0) atomicAdd(&hist[bin], __popcll(peers));
}

constexpr int kSelectLdsTokens = 32768;  // a column of up to this many keys stays in LDS (128 KB)

// One workgroup per expert e: which tokens it keeps, and their rows.
__global__ void __launch_bounds__(kSelectThreads)
    router_select_kernel(const float* __restrict__ shifted, int64_t num_tokens, const int32_t* __restrict__ target,
                         const int32_t* __restrict__ padded_offsets, uint32_t* __restrict__ keep_mask,
                         int32_t* __restrict__ keep_prefix, int32_t* __restrict__ row_token) {
  __shared__ uint32_t keys[kSelectLdsTokens];
  __shared__ int32_t hist[256];
  __shared__ int32_t wave_sums[16];
  __shared__ uint32_t s_prefix, s_prefix_mask;
  __shared__ int32_t s_remaining;
  __shared__ int64_t s_cut;
  const int tid = threadIdx.x;
  const int e = blockIdx.x;
  const float* col = shifted + static_cast<int64_t>(e) * num_tokens;
  const int32_t tgt = target[e];
  const int64_t words = (num_tokens + 31) / 32;
  uint32_t* mask = keep_mask + static_cast<int64_t>(e) * words;
  int32_t* pref = keep_prefix + static_cast<int64_t>(e) * words;

  // Keys of the column, computed once (in LDS when they fit).
  const bool in_lds = num_tokens <= kSelectLdsTokens;
  if (in_lds) {
    constexpr int kPer = 8;
    for (int64_t base = 0; base < num_tokens; base += kSelectThreads * kPer) {
      float v[kPer];
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int64_t t = base + u * kSelectThreads + tid;
        v[u] = t < num_tokens ? col[t] : 0.0f;
      }
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const int64_t t = base + u * kSelectThreads + tid;
        if (t < num_tokens) keys[t] = sort_key(v[u]);
      }
    }
    __syncthreads();
  }
  auto key_at = [&](int64_t t) -> uint32_t { return in_lds ? keys[t] : sort_key(col[t]); };

  // Threshold key and the last tie kept: keep t iff key > thr, or
  // key == thr and t <= cut.
  uint32_t thr = 0;
  int64_t cut = -1;
  bool keep_all = false, keep_none = false;
  if (tgt <= 0) {
    keep_none = true;
  } else if (tgt >= num_tokens) {
    keep_all = true;
  } else {
    if (tid == 0) {
      s_prefix = 0;
      s_prefix_mask = 0;
      s_remaining = tgt;
    }
    for (int shift = 24; shift >= 0; shift -= 8) {
      for (int b = tid; b < 256; b += kSelectThreads) hist[b] = 0;
      __syncthreads();
      const uint32_t pre = s_prefix, pmask = s_prefix_mask;
      for (int64_t base = 0; base < num_tokens; base += kSelectThreads) {  // same trip count in every lane
        const int64_t t = base + tid;
        const uint32_t key = t < num_tokens ? key_at(t) : 0u;
        wave_hist_add(hist, (key >> shift) & 255u, t < num_tokens && (key & pmask) == pre);
      }
      __syncthreads();
      if (tid < 64) {
        // Wave 0: lane l holds bins 255-4l .. 252-4l (descending). A suffix
        // count from the top finds the bin where the rem-th largest falls.
        const int32_t rem = s_remaining;
        int32_t c[4], own = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          c[q] = hist[255 - 4 * tid - q];
          own += c[q];
        }
        int32_t incl = own;  // keys in bins above and including this lane's four
        for (int d = 1; d < 64; d <<= 1) {
          const int32_t below = __shfl_up(incl, d, 64);
          if (tid >= d) incl += below;
        }
        int32_t above = incl - own;  // keys in higher bins than this lane's
        // The lane whose four bins reach rem: the first with incl >= rem.
        const uint64_t reach = __ballot(incl >= rem);
        if (reach != 0 && tid == __builtin_ctzll(reach)) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            if (above + c[q] >= rem) {
              s_prefix = pre | (static_cast<uint32_t>(255 - 4 * tid - q) << shift);
              s_prefix_mask = pmask | (255u << shift);
              s_remaining = rem - above;
              break;
            }
            above += c[q];
          }
        }
      }
      __syncthreads();
    }
    thr = s_prefix;
    const int32_t ties = s_remaining;  // keys == thr to keep, in token order
    // The ties-th token with key == thr.
    if (tid == 0) s_cut = num_tokens;
    int32_t carry = 0;
    for (int64_t base = 0; base < num_tokens; base += kSelectThreads) {
      const int64_t t = base + tid;
      const int32_t is_tie = (t < num_tokens && key_at(t) == thr) ? 1 : 0;
      int32_t chunk_total;
      const int32_t incl = block_scan_1024(is_tie, wave_sums, &chunk_total);
      if (is_tie && carry + incl == ties) s_cut = t;
      carry += chunk_total;
      if (carry >= ties) break;  // uniform: every thread has the same carry
    }
    __syncthreads();
    cut = s_cut;
  }

  // Keep bitmask, one 32-token word per lane.
  int32_t carry = 0;
  for (int64_t base = 0; base < words; base += kSelectThreads) {
    const int64_t w = base + tid;
    uint32_t bits = 0;
    if (w < words && !keep_none) {
      for (int b = 0; b < 32; ++b) {
        const int64_t t = w * 32 + b;
        if (t >= num_tokens) break;
        bool keep = keep_all;
        if (!keep_all) {
          const uint32_t key = key_at(t);
          keep = key > thr || (key == thr && t <= cut);
        }
        if (keep) bits |= 1u << b;
      }
    }
    const int32_t cnt = __popc(bits);
    int32_t chunk_total;
    const int32_t incl = block_scan_1024(cnt, wave_sums, &chunk_total);
    if (w < words) {
      mask[w] = bits;
      pref[w] = carry + incl - cnt;
      // Kept tokens take the expert's rows in token order.
      const int32_t row0 = padded_offsets[e] + carry + incl - cnt;
      uint32_t rest = bits;
      int32_t r = 0;
      while (rest != 0) {
        const int b = __builtin_ctz(rest);
        rest &= rest - 1;
        row_token[row0 + r] = static_cast<int32_t>(w * 32 + b);
        ++r;
      }
    }
    carry += chunk_total;
  }
}

// Kept experts of token t: bit e of word t/32 of expert e's mask.
__device__ __forceinline__ bool kept(const uint32_t* __restrict__ keep_mask, int64_t words, int32_t e, int64_t t) {
  return (keep_mask[static_cast<int64_t>(e) * words + (t >> 5)] >> (t & 31)) & 1u;
}

// One wave per token: number of kept experts and the sum of their scores,
// added in ascending expert order.
__global__ void __launch_bounds__(64 * kTokenWaves)
    router_tokens_kernel(const float* __restrict__ scores, int64_t num_tokens, int32_t num_experts,
                         const uint32_t* __restrict__ keep_mask, int32_t* __restrict__ kept_count,
                         float* __restrict__ kept_total) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kTokenWaves + (threadIdx.x >> 6);
  if (t >= num_tokens) return;
  const int64_t words = (num_tokens + 31) / 32;
  int32_t n = 0;
  float total = 0.0f;
  for (int e0 = 0; e0 < num_experts; e0 += 64) {
    const int e = e0 + lane;
    const bool keep = e < num_experts && kept(keep_mask, words, e, t);
    const float s = keep ? scores[t * num_experts + e] : 0.0f;
    uint64_t bal = __ballot(keep);
    n += __popcll(bal);
    while (bal != 0) {  // sequential, in expert order
      const int l = __builtin_ctzll(bal);
      bal &= bal - 1;
      total += __shfl(s, l, 64);
    }
  }
  if (lane == 0) {
    kept_count[t] = n;
    kept_total[t] = total;
  }
}

// token_offsets = exclusive scan of kept_count; token_offsets[T] = N.
// Each lane takes 16 consecutive tokens, so one workgroup scan covers 16K
// tokens (one pass at the benchmark sizes).
__global__ void __launch_bounds__(1024)
    router_scan_kernel(const int32_t* __restrict__ kept_count, int64_t num_tokens, int32_t* __restrict__ token_offsets,
                       int32_t* __restrict__ num_assignments) {
  __shared__ int32_t wave_sums[16];
  constexpr int kPer = 16;
  int32_t carry = 0;
  for (int64_t base = 0; base < num_tokens; base += 1024 * kPer) {
    const int64_t t0 = base + static_cast<int64_t>(threadIdx.x) * kPer;
    int32_t v[kPer];
    int32_t own = 0;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      v[u] = t0 + u < num_tokens ? kept_count[t0 + u] : 0;
      own += v[u];
    }
    int32_t chunk_total;
    const int32_t incl = block_scan_1024(own, wave_sums, &chunk_total);
    int32_t run = carry + incl - own;
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      if (t0 + u < num_tokens) token_offsets[t0 + u] = run;
      run += v[u];
    }
    carry += chunk_total;
  }
  if (threadIdx.x == 0) {
    token_offsets[num_tokens] = carry;
    num_assignments[0] = carry;
  }
}

// One wave per token: its assignments, in expert order; then the unused
// tail of copy_row (the capacity past N) is set to -1.
__global__ void __launch_bounds__(64 * kTokenWaves)
    router_emit_kernel(const float* __restrict__ scores, int64_t num_tokens, int32_t num_experts,
                       const uint32_t* __restrict__ keep_mask, const int32_t* __restrict__ keep_prefix,
                       const float* __restrict__ kept_total, const int32_t* __restrict__ token_offsets,
                       const int32_t* __restrict__ padded_offsets, int64_t capacity, int32_t* __restrict__ token_of_copy,
                       int32_t* __restrict__ expert_of_copy, float* __restrict__ weight_of_copy,
                       int32_t* __restrict__ copy_row) {
  const int lane = threadIdx.x & 63;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kTokenWaves + (threadIdx.x >> 6);
  const int64_t words = (num_tokens + 31) / 32;
  if (t < num_tokens) {
    const float total = kept_total[t];
    int32_t c = token_offsets[t];
    for (int e0 = 0; e0 < num_experts; e0 += 64) {
      const int e = e0 + lane;
      const bool keep = e < num_experts && kept(keep_mask, words, e, t);
      const uint64_t bal = __ballot(keep);
      if (keep) {
        const int64_t slot = c + __popcll(bal & ((1ull << lane) - 1ull));
        const uint32_t word = keep_mask[static_cast<int64_t>(e) * words + (t >> 5)];
        const int32_t rank = keep_prefix[static_cast<int64_t>(e) * words + (t >> 5)] +
                             __popc(word & ((1u << (t & 31)) - 1u));
        token_of_copy[slot] = static_cast<int32_t>(t);
        expert_of_copy[slot] = e;
        weight_of_copy[slot] = scores[t * num_experts + e] / total;
        copy_row[slot] = padded_offsets[e] + rank;
      }
      c += __popcll(bal);
    }
  }
  // Capacity tail.
  const int64_t n = token_offsets[num_tokens];
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = n + static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < capacity; i += stride) {
    token_of_copy[i] = -1;
    expert_of_copy[i] = -1;
    weight_of_copy[i] = 0.0f;
    copy_row[i] = -1;
  }
}

constexpr int kLayoutItems = 1024;

__global__ void __launch_bounds__(kLayoutItems)
    router_layout_kernel(const int32_t* __restrict__ padded_offsets, const int32_t* __restrict__ tokens_per_expert,
                         int32_t num_experts, int32_t block_size, int32_t ffn_blocks, int32_t max_row_blocks,
                         int64_t max_rows, int32_t* __restrict__ row_token, int32_t* __restrict__ row_block_expert,
                         int32_t* __restrict__ row_offsets, int32_t* __restrict__ col_indices) {
  __shared__ int32_t offs[kMaxExperts + 1];
  __shared__ int32_t cnts[kMaxExperts];
  for (int e = threadIdx.x; e <= num_experts; e += kLayoutItems) offs[e] = padded_offsets[e];
  for (int e = threadIdx.x; e < num_experts; e += kLayoutItems) cnts[e] = tokens_per_expert[e];
  __syncthreads();
  const int64_t i = static_cast<int64_t>(blockIdx.x) * kLayoutItems + threadIdx.x;
  layout_item(i, offs, cnts, num_experts, block_size, ffn_blocks, max_row_blocks, max_rows, row_token,
              row_block_expert, row_offsets, col_indices);
}

struct RouterSizes {
  int64_t max_assignments, workspace_elems, max_row_blocks, max_rows;
  int64_t chunks, words;
};

int router_sizes(int64_t num_tokens, int32_t num_experts, int32_t k, int32_t tile, int32_t block_size,
                 int32_t ffn_dim, RouterSizes* out) {
  constexpr int64_t kI32Max = 2147483647;
  if (num_tokens <= 0 || num_tokens > kI32Max / 2) return fail(SB_ERR_INVALID, "scores must be [T, E] with T > 0");
  if (num_experts <= 0 || num_experts > kMaxExperts)
    return fail(SB_ERR_INVALID, "num_experts must be in [1, %d], got %d", kMaxExperts, num_experts);
  if (k <= 0 || k > num_experts || k > 16)
    return fail(SB_ERR_INVALID, "k must be in [1, min(E, 16)], got %d", k);
  if (tile <= 0) return fail(SB_ERR_INVALID, "tile must be positive");
  // Rounding moves an expert by less than half a tile upwards.
  const int64_t cap = std::min<int64_t>(num_tokens * num_experts,
                                        num_tokens * k + static_cast<int64_t>(num_experts) * (tile / 2));
  int64_t rb = 0, rows = 0, ws_route = 0;
  if (int rc = sb_routing_sizes(cap, num_experts, ffn_dim, block_size, &rb, &rows, &ws_route)) return rc;
  out->max_assignments = cap;
  out->max_row_blocks = rb;
  out->max_rows = rows;
  out->chunks = (num_tokens + kTopkTokensPerGroup - 1) / kTopkTokensPerGroup;
  out->words = (num_tokens + 31) / 32;
  // chunk counts, target, shifted scores, keep mask, keep prefix, kept count, kept total
  out->workspace_elems = out->chunks * num_experts + num_experts + num_tokens * num_experts +
                         2 * out->words * num_experts + 2 * num_tokens;
  return SB_OK;
}

int launch_topk(const float* scores, int64_t num_tokens, int32_t num_experts, int32_t k, float* shifted,
                int32_t* chunk_counts, int32_t* top_idx, float* top_weight, hipStream_t s) {
  const uint32_t groups = static_cast<uint32_t>((num_tokens + kTopkTokensPerGroup - 1) / kTopkTokensPerGroup);
  const int per = (num_experts + 63) / 64;
  // A lane per token unless its insertion work (E x the rounded-up k) is
  // large; the test hook SB_HOOK_TOPK_KERNEL = 1 forces the wave form, 2
  // the lane form.
  const int kmax = k <= 1 ? 1 : k <= 2 ? 2 : k <= 4 ? 4 : k <= 8 ? 8 : 16;
  const int forced = test_hook(SB_HOOK_TOPK_KERNEL);
  if (forced == 2 || (forced != 1 && kmax * num_experts <= 2048)) {
#define SB_TOPK_LANE(K) \
  router_topk_lane_kernel<K><<<groups, 64, 0, s>>>(scores, num_tokens, num_experts, k, shifted, chunk_counts, top_idx, top_weight)
    if (k <= 1) SB_TOPK_LANE(1);
    else if (k <= 2) SB_TOPK_LANE(2);
    else if (k <= 4) SB_TOPK_LANE(4);
    else if (k <= 8) SB_TOPK_LANE(8);
    else SB_TOPK_LANE(16);
#undef SB_TOPK_LANE
    return check_launch("router top-k");
  }
#define SB_TOPK(P)                                                                                          \
  router_topk_kernel<P><<<groups, kTopkThreads, 0, s>>>(scores, num_tokens, num_experts, k, shifted, chunk_counts, \
                                                        top_idx, top_weight)
  if (per <= 1) SB_TOPK(1);
  else if (per <= 2) SB_TOPK(2);
  else if (per <= 4) SB_TOPK(4);
  else if (per <= 8) SB_TOPK(8);
  else SB_TOPK(kMaxPerLane);
#undef SB_TOPK
  return check_launch("router top-k");
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" int sb_router_sizes(int64_t num_tokens, int32_t num_experts, int32_t k, int32_t tile, int32_t block_size,
                               int32_t ffn_dim, int64_t* max_assignments, int64_t* max_row_blocks, int64_t* max_rows,
                               int64_t* workspace_elems) {
  RouterSizes z;
  if (int rc = router_sizes(num_tokens, num_experts, k, tile, block_size, ffn_dim, &z)) return rc;
  if (max_assignments) *max_assignments = z.max_assignments;
  if (max_row_blocks) *max_row_blocks = z.max_row_blocks;
  if (max_rows) *max_rows = z.max_rows;
  if (workspace_elems) *workspace_elems = z.workspace_elems;
  return clear_ok();
}

extern "C" int sb_router_topk(const float* scores, int64_t num_tokens, int32_t num_experts, int32_t k,
                              int32_t* top_idx, float* top_weight, void* stream) {
  if (num_tokens <= 0 || num_tokens > 2147483647LL / 16) return fail(SB_ERR_INVALID, "scores must be [T, E] with T > 0");
  if (num_experts <= 0 || num_experts > kMaxExperts)
    return fail(SB_ERR_INVALID, "num_experts must be in [1, %d], got %d", kMaxExperts, num_experts);
  if (k <= 0 || k > num_experts || k > 16) return fail(SB_ERR_INVALID, "k must be in [1, min(E, 16)], got %d", k);
  if (!scores || !top_idx || !top_weight) return fail(SB_ERR_INVALID, "router top-k: null buffer");
  if (int rc = launch_topk(scores, num_tokens, num_experts, k, nullptr, nullptr, top_idx, top_weight,
                           as_stream(stream)))
    return rc;
  return clear_ok();
}

extern "C" int sb_token_rounding(const float* scores, int64_t num_tokens, int32_t num_experts, int32_t k,
                                 int32_t tile, int32_t block_size, int32_t ffn_dim, int32_t* workspace,
                                 int32_t* token_of_copy, int32_t* expert_of_copy, float* weight_of_copy,
                                 int32_t* num_assignments, int32_t* token_offsets, int32_t* tokens_per_expert,
                                 int32_t* padded_offsets, int32_t* row_token, int32_t* copy_row,
                                 int32_t* row_block_expert, int32_t* row_offsets, int32_t* col_indices,
                                 int32_t* error, void* stream_ptr) {
  RouterSizes z;
  if (int rc = router_sizes(num_tokens, num_experts, k, tile, block_size, ffn_dim, &z)) return rc;
  if (!scores || !workspace || !token_of_copy || !expert_of_copy || !weight_of_copy || !num_assignments ||
      !token_offsets || !tokens_per_expert || !padded_offsets || !row_token || !copy_row || !row_block_expert ||
      !row_offsets || !col_indices || !error)
    return fail(SB_ERR_INVALID, "token rounding: null buffer");
  const hipStream_t s = as_stream(stream_ptr);
  const int64_t t = num_tokens;
  const int32_t e = num_experts;
  // Workspace carve-up (int32 elements; the float arrays share the 4-byte slots).
  int32_t* chunk_counts = workspace;
  int32_t* unused_target = chunk_counts + z.chunks * e;
  float* shifted = reinterpret_cast<float*>(unused_target + e);
  uint32_t* keep_mask = reinterpret_cast<uint32_t*>(shifted + t * e);
  int32_t* keep_prefix = reinterpret_cast<int32_t*>(keep_mask + z.words * e);
  int32_t* kept_count = keep_prefix + z.words * e;
  float* kept_total = reinterpret_cast<float*>(kept_count + t);

  if (int rc = launch_topk(scores, t, e, k, shifted, chunk_counts, nullptr, nullptr, s)) return rc;
  router_targets_kernel<<<1, 1024, 0, s>>>(chunk_counts, static_cast<int32_t>(z.chunks), e, t, tile, block_size,
                                           tokens_per_expert, padded_offsets, error);
  if (int rc = check_launch("token rounding targets")) return rc;
  router_select_kernel<<<e, kSelectThreads, 0, s>>>(shifted, t, tokens_per_expert, padded_offsets, keep_mask,
                                                    keep_prefix, row_token);
  if (int rc = check_launch("token rounding select")) return rc;
  const uint32_t token_groups = static_cast<uint32_t>((t + kTokenWaves - 1) / kTokenWaves);
  router_tokens_kernel<<<token_groups, 64 * kTokenWaves, 0, s>>>(scores, t, e, keep_mask, kept_count, kept_total);
  if (int rc = check_launch("token rounding totals")) return rc;
  router_scan_kernel<<<1, 1024, 0, s>>>(kept_count, t, token_offsets, num_assignments);
  if (int rc = check_launch("token rounding scan")) return rc;
  router_emit_kernel<<<token_groups, 64 * kTokenWaves, 0, s>>>(scores, t, e, keep_mask, keep_prefix, kept_total,
                                                               token_offsets, padded_offsets, z.max_assignments,
                                                               token_of_copy, expert_of_copy, weight_of_copy,
                                                               copy_row);
  if (int rc = check_launch("token rounding emit")) return rc;
  const int32_t ffn_blocks = ffn_dim / block_size;
  const int64_t layout_items = std::max<int64_t>(z.max_row_blocks * ffn_blocks + 1, z.max_rows);
  const uint32_t layout_groups = static_cast<uint32_t>((layout_items + kLayoutItems - 1) / kLayoutItems);
  router_layout_kernel<<<layout_groups, kLayoutItems, 0, s>>>(padded_offsets, tokens_per_expert, e, block_size,
                                                              ffn_blocks, static_cast<int32_t>(z.max_row_blocks),
                                                              z.max_rows, row_token, row_block_expert, row_offsets,
                                                              col_indices);
  if (int rc = check_launch("token rounding layout")) return rc;
  return clear_ok();
}
