// The MoE layer on a routing given as assignments (the path of
// sparsebench/moe.py:59-91 in the reference, moe_forward_assigned): copy c
// sends token[c] to expert[c] with weight[c]; a token may have any number of
// copies, including none.
//
// Routing is the top-k routing with k = 1 and token ids read from the list
// (sb_routing_assigned). What changes is the combine: a token's copies are
// no longer the k consecutive entries t*k .. t*k+k-1, so the reference sums
// them with index_add_ (atomics, order not fixed). Here two steps replace it:
//
//   token_csr   one workgroup: token_offsets[T+1] and token_copies, the
//               copies of each token in ascending copy order. Lists already
//               ordered by token (top-k lists, token rounding's output) take
//               a direct path: offsets from the run boundaries, copies = c.
//               Other lists: histogram, scan, placement, then each token's
//               few copies sorted, so the result does not depend on timing.
//   combine     out[t] = bf16( sum over t's copies, in copy order, of
//               fp32(y[copy_row[c]]) * fp32(weight[c]) ); 0 for no copies.
//
// Both are deterministic: the same list gives the same bits on every run.
// A token's copies are summed in list order, as the reference's index_add_
// does on the CPU, so a top-k list gives exactly the top-k combine's result.

#include "common.hpp"

namespace sb {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kCsrThreads = 1024;

// A copy is listed when routing placed it (copy_row >= 0; a bad expert or
// token id, or a token >= valid_tokens, gives -1) and its token is in range.
template <typename Tok>
__device__ __forceinline__ bool listed(const Tok* __restrict__ token, const int32_t* __restrict__ copy_row,
                                       int64_t c, int32_t num_tokens) {
  return copy_row[c] >= 0 && token[c] >= 0 && token[c] < static_cast<Tok>(num_tokens);
}

template <typename Tok>
__global__ void __launch_bounds__(kCsrThreads)
    token_csr_kernel(const Tok* __restrict__ token, const int32_t* __restrict__ copy_row, int64_t n,
                     int32_t num_tokens, int32_t* __restrict__ offsets, int32_t* __restrict__ copies) {
  __shared__ int32_t total_listed;
  const int tid = threadIdx.x;

  // Direct path: every copy listed and tokens non-decreasing.
  bool ordered = true;
  for (int64_t c = tid; c < n; c += kCsrThreads) {
    ordered = ordered && listed(token, copy_row, c, num_tokens) && (c == 0 || token[c] >= token[c - 1]);
  }
  if (__syncthreads_and(ordered)) {
    // offsets[t] = first copy of a token >= t: copy c starts the tokens
    // token[c-1]+1 .. token[c].
    for (int64_t c = tid; c < n; c += kCsrThreads) {
      const int64_t t = static_cast<int64_t>(token[c]);
      const int64_t prev = c == 0 ? -1 : static_cast<int64_t>(token[c - 1]);
      for (int64_t u = prev + 1; u <= t; ++u) offsets[u] = static_cast<int32_t>(c);
      copies[c] = static_cast<int32_t>(c);
    }
    const int64_t last = n > 0 ? static_cast<int64_t>(token[n - 1]) : -1;
    for (int64_t u = last + 1 + tid; u <= num_tokens; u += kCsrThreads) offsets[u] = static_cast<int32_t>(n);
    return;
  }

  // General path. offsets[t+1] counts token t's copies ...
  for (int64_t u = tid; u <= num_tokens; u += kCsrThreads) offsets[u] = 0;
  __syncthreads();
  for (int64_t c = tid; c < n; c += kCsrThreads)
    if (listed(token, copy_row, c, num_tokens)) atomicAdd(&offsets[static_cast<int64_t>(token[c]) + 1], 1);
  __syncthreads();
  // ... an inclusive scan of it gives offsets[t+1] = end of token t.
  __shared__ int32_t wave_sums[kCsrThreads / 64];
  int32_t carry = 0;
  const int lane = tid & 63, wave = tid >> 6;
  for (int64_t base = 1; base <= num_tokens; base += kCsrThreads) {
    const int64_t u = base + tid;
    int32_t v = u <= num_tokens ? offsets[u] : 0;
    for (int d = 1; d < 64; d <<= 1) {
      const int32_t below = __shfl_up(v, d, 64);
      if (lane >= d) v += below;
    }
    if (lane == 63) wave_sums[wave] = v;
    __syncthreads();
    int32_t before = carry;
    for (int w = 0; w < wave; ++w) before += wave_sums[w];
    int32_t chunk_total = 0;
    for (int w = 0; w < kCsrThreads / 64; ++w) chunk_total += wave_sums[w];
    if (u <= num_tokens) offsets[u] = v + before;
    carry += chunk_total;
    __syncthreads();
  }
  if (tid == 0) total_listed = carry;
  __syncthreads();
  // Placement: each copy takes a slot just below its token's end, which
  // walks offsets[t+1] down to the start of token t ...
  for (int64_t c = tid; c < n; c += kCsrThreads) {
    if (!listed(token, copy_row, c, num_tokens)) continue;
    const int32_t slot = atomicSub(&offsets[static_cast<int64_t>(token[c]) + 1], 1) - 1;
    copies[slot] = static_cast<int32_t>(c);
  }
  __syncthreads();
  // ... so offsets[t+1] now holds start(t): shift down by one, in passes
  // of 8 entries per thread. A pass reads only entries above its own range,
  // which earlier passes have not written.
  constexpr int kPer = 8;
  for (int64_t base = 0; base <= num_tokens; base += kPer * kCsrThreads) {
    int32_t shifted[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int64_t u = base + i * kCsrThreads + tid;
      shifted[i] = u < num_tokens ? offsets[u + 1] : total_listed;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int64_t u = base + i * kCsrThreads + tid;
      if (u <= num_tokens) offsets[u] = shifted[i];
    }
    __syncthreads();
  }
  // Each token's copies in ascending order (lists are a few entries long).
  for (int64_t u = tid; u < num_tokens; u += kCsrThreads) {
    const int32_t s = offsets[u], e = offsets[u + 1];
    for (int32_t i = s + 1; i < e; ++i) {
      const int32_t v = copies[i];
      int32_t j = i - 1;
      while (j >= s && copies[j] > v) {
        copies[j + 1] = copies[j];
        --j;
      }
      copies[j + 1] = v;
    }
  }
  // Unused tail of the copy list.
  for (int64_t c = static_cast<int64_t>(total_listed) + tid; c < n; c += kCsrThreads) copies[c] = -1;
}

template <typename G>
__device__ __forceinline__ float weight_f32(const G* g, int64_t i);
template <>
__device__ __forceinline__ float weight_f32<uint16_t>(const uint16_t* g, int64_t i) {
  return bf16_to_f32(g[i]);
}
template <>
__device__ __forceinline__ float weight_f32<_Float16>(const _Float16* g, int64_t i) {
  return static_cast<float>(g[i]);
}
template <>
__device__ __forceinline__ float weight_f32<float>(const float* g, int64_t i) {
  return g[i];
}

// One lane per 16 bytes (8 columns) of one token row.
template <typename G>
__global__ void __launch_bounds__(256)
    combine_assigned_kernel(const uint16_t* __restrict__ y, const int32_t* __restrict__ copy_row,
                            const G* __restrict__ weights, const int32_t* __restrict__ offsets,
                            const int32_t* __restrict__ copies, uint16_t* __restrict__ out, int64_t num_tokens,
                            int32_t chunks_per_row, int64_t y_rows, const int32_t* __restrict__ valid_tokens) {
  // Products rounded, then added (no fused multiply-add), as the reference's
  // index_add_ of rows.float() * weight.
#pragma clang fp contract(off)
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t t = item / chunks_per_row;
  const int32_t ch = static_cast<int32_t>(item % chunks_per_row);
  const int64_t limit = valid_tokens ? min(num_tokens, static_cast<int64_t>(*valid_tokens)) : num_tokens;
  if (t >= limit) return;
  const int64_t d_model = static_cast<int64_t>(chunks_per_row) * 8;
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  const int32_t s = offsets[t], e = offsets[t + 1];
  for (int32_t i = s; i < e; ++i) {
    const int32_t c = copies != nullptr ? copies[i] : i;  // no list: copies already in token order
    const int32_t row = c >= 0 ? copy_row[c] : -1;
    if (row < 0 || row >= y_rows) continue;
    const float g = weight_f32(weights, c);
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(y + row * d_model + ch * 8);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += __uint_as_float(v[q] << 16) * g;
      acc[2 * q + 1] += __uint_as_float(v[q] & 0xffff0000u) * g;
    }
  }
  u32x4_t o;
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
  *reinterpret_cast<u32x4_t*>(out + t * d_model + ch * 8) = o;
}

template <typename G>
int launch_combine_assigned(const void* y, const int32_t* copy_row, const void* weights, const int32_t* offsets,
                            const int32_t* copies, void* out, int64_t num_tokens, int64_t d_model, int64_t y_rows,
                            const int32_t* valid_tokens, hipStream_t stream) {
  const int32_t chunks = static_cast<int32_t>(d_model / 8);
  const int64_t groups = (num_tokens * chunks + 255) / 256;
  combine_assigned_kernel<G><<<static_cast<uint32_t>(groups), 256, 0, stream>>>(
      static_cast<const uint16_t*>(y), copy_row, static_cast<const G*>(weights), offsets, copies,
      static_cast<uint16_t*>(out), num_tokens, chunks, y_rows, valid_tokens);
  return check_launch("combine (assigned)");
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" int sb_token_csr(const void* token_of_copy, int32_t token_is_i64, const int32_t* copy_row,
                            int64_t num_copies, int64_t num_tokens, int32_t* token_offsets, int32_t* token_copies,
                            void* stream) {
  if (num_copies <= 0 || num_copies > 2147483647LL) return fail(SB_ERR_INVALID, "token_csr: bad copy count");
  if (num_tokens <= 0 || num_tokens > 2147483646LL) return fail(SB_ERR_INVALID, "token_csr: bad token count");
  if (!token_of_copy || !copy_row || !token_offsets || !token_copies)
    return fail(SB_ERR_INVALID, "token_csr: null buffer");
  const hipStream_t s = as_stream(stream);
  if (token_is_i64)
    token_csr_kernel<int64_t><<<1, kCsrThreads, 0, s>>>(static_cast<const int64_t*>(token_of_copy), copy_row,
                                                        num_copies, static_cast<int32_t>(num_tokens), token_offsets,
                                                        token_copies);
  else
    token_csr_kernel<int32_t><<<1, kCsrThreads, 0, s>>>(static_cast<const int32_t*>(token_of_copy), copy_row,
                                                        num_copies, static_cast<int32_t>(num_tokens), token_offsets,
                                                        token_copies);
  if (int rc = check_launch("token_csr")) return rc;
  return clear_ok();
}

extern "C" int sb_combine_assigned(const void* y, const int32_t* copy_row, const void* weights, int32_t weight_dtype,
                                   const int32_t* token_offsets, const int32_t* token_copies, void* out,
                                   int64_t num_tokens, int64_t d_model, int64_t y_rows, const int32_t* valid_tokens,
                                   void* stream) {
  if (num_tokens < 0) return fail(SB_ERR_INVALID, "combine: bad token count");
  if (d_model <= 0 || d_model % 8 != 0)
    return fail(SB_ERR_INVALID, "combine: D (%lld) must be a positive multiple of 8", static_cast<long long>(d_model));
  if (num_tokens == 0) return clear_ok();
  if (!y || !copy_row || !weights || !token_offsets || !out) return fail(SB_ERR_INVALID, "combine: null buffer");
  if (!aligned16(y) || !aligned16(out)) return fail(SB_ERR_INVALID, "combine: y and out must be 16-byte aligned");
  if ((num_tokens * (d_model / 8) + 255) / 256 > 2147483647LL) return fail(SB_ERR_INVALID, "combine: too many tokens");
  const hipStream_t s = as_stream(stream);
  switch (weight_dtype) {
    case SB_DTYPE_BF16:
      return launch_combine_assigned<uint16_t>(y, copy_row, weights, token_offsets, token_copies, out, num_tokens,
                                               d_model, y_rows, valid_tokens, s);
    case SB_DTYPE_F16:
      return launch_combine_assigned<_Float16>(y, copy_row, weights, token_offsets, token_copies, out, num_tokens,
                                               d_model, y_rows, valid_tokens, s);
    case SB_DTYPE_F32:
      return launch_combine_assigned<float>(y, copy_row, weights, token_offsets, token_copies, out, num_tokens,
                                            d_model, y_rows, valid_tokens, s);
    default:
      return fail(SB_ERR_INVALID, "combine: unsupported weight dtype code %d", weight_dtype);
  }
}
