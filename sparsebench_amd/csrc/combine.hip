// Combine: each token's k expert outputs, gate-weighted, in one pass
// (the step of sparsebench/moe.py:51-54 in the reference, which runs it as
// ~6 ATen launches over [T*k, D] -> [T, k, D] -> [T, D]).
//
//   out[t, :] = bf16( sum_j fp32(y[copy_row[t*k + j], :]) * fp32(gate[t, j]) )
//
// Bandwidth-bound: each lane owns 8 consecutive columns (16 bytes) of one
// token row, gathers the k rows with 16-byte loads and writes 16 bytes.

#include "common.hpp"

namespace sb {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <typename G>
__device__ __forceinline__ float gate_f32(const G* g, int64_t i);
template <>
__device__ __forceinline__ float gate_f32<uint16_t>(const uint16_t* g, int64_t i) {
  return bf16_to_f32(g[i]);
}
template <>
__device__ __forceinline__ float gate_f32<_Float16>(const _Float16* g, int64_t i) {
  return static_cast<float>(g[i]);
}
template <>
__device__ __forceinline__ float gate_f32<float>(const float* g, int64_t i) {
  return g[i];
}

template <typename G>
__global__ void __launch_bounds__(256)
    combine_kernel(const uint16_t* __restrict__ y, const int32_t* __restrict__ copy_row, const G* __restrict__ gates,
                   uint16_t* __restrict__ out, int64_t num_tokens, int32_t k, int32_t chunks_per_row, int64_t y_rows,
                   const int32_t* __restrict__ valid_tokens) {
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t t = item / chunks_per_row;
  const int32_t c = static_cast<int32_t>(item % chunks_per_row);
  const int64_t limit = valid_tokens ? min(num_tokens, static_cast<int64_t>(*valid_tokens)) : num_tokens;
  if (t >= limit) return;
  const int64_t d_model = static_cast<int64_t>(chunks_per_row) * 8;

  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int32_t j = 0; j < k; ++j) {
    const int32_t row = copy_row[t * k + j];
    if (row < 0 || row >= y_rows) continue;  // skipped copy (bad expert id)
    const float g = gate_f32(gates, t * k + j);
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(y + row * d_model + c * 8);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += __uint_as_float(v[q] << 16) * g;
      acc[2 * q + 1] += __uint_as_float(v[q] & 0xffff0000u) * g;
    }
  }
  u32x4_t o;
#pragma unroll
  for (int q = 0; q < 4; ++q) o[q] = pack_bf16x2(acc[2 * q], acc[2 * q + 1]);
  *reinterpret_cast<u32x4_t*>(out + t * d_model + c * 8) = o;
}

template <typename G>
int launch_combine(const void* y, const int32_t* copy_row, const void* gates, void* out, int64_t num_tokens,
                   int32_t k, int64_t d_model, int64_t y_rows, const int32_t* valid_tokens, hipStream_t stream) {
  const int32_t chunks = static_cast<int32_t>(d_model / 8);
  const int64_t items = num_tokens * chunks;
  const int64_t groups = (items + 255) / 256;
  combine_kernel<G><<<static_cast<uint32_t>(groups), 256, 0, stream>>>(
      static_cast<const uint16_t*>(y), copy_row, static_cast<const G*>(gates), static_cast<uint16_t*>(out),
      num_tokens, k, chunks, y_rows, valid_tokens);
  return check_launch("combine");
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" int sb_combine(const void* y, const int32_t* copy_row, const void* gates, int32_t gate_dtype, void* out,
                          int64_t num_tokens, int32_t k, int64_t d_model, int64_t y_rows,
                          const int32_t* valid_tokens, void* stream) {
  if (num_tokens < 0 || k <= 0) return fail(SB_ERR_INVALID, "combine: expert_weight must be [T, k] with k > 0");
  if (d_model <= 0 || d_model % 8 != 0)
    return fail(SB_ERR_INVALID, "combine: D (%lld) must be a positive multiple of 8", static_cast<long long>(d_model));
  if (num_tokens == 0) return clear_ok();
  if (!y || !copy_row || !gates || !out) return fail(SB_ERR_INVALID, "combine: null buffer");
  if (!aligned16(y) || !aligned16(out)) return fail(SB_ERR_INVALID, "combine: y and out must be 16-byte aligned");
  if ((num_tokens * (d_model / 8) + 255) / 256 > 2147483647LL) return fail(SB_ERR_INVALID, "combine: too many tokens");
  const hipStream_t s = as_stream(stream);
  switch (gate_dtype) {
    case SB_DTYPE_BF16:
      return launch_combine<uint16_t>(y, copy_row, gates, out, num_tokens, k, d_model, y_rows, valid_tokens, s);
    case SB_DTYPE_F16:
      return launch_combine<_Float16>(y, copy_row, gates, out, num_tokens, k, d_model, y_rows, valid_tokens, s);
    case SB_DTYPE_F32:
      return launch_combine<float>(y, copy_row, gates, out, num_tokens, k, d_model, y_rows, valid_tokens, s);
    default:
      return fail(SB_ERR_INVALID, "combine: unsupported gate dtype code %d", gate_dtype);
  }
}
