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

// KMAX > 0: k == KMAX, known at compile time, so the k row indices, then
// the k row loads, are all issued before the first is waited for (the
// loop below waits for each copy's row before it loads the next). KMAX ==
// 0: any k, one copy at a time. Either way the products are added in slot
// order j = 0 .. k-1, so the result is the same bits.
template <typename G, int KMAX>
__global__ void __launch_bounds__(256)
    combine_kernel(const uint16_t* __restrict__ y, const int32_t* __restrict__ copy_row, const G* __restrict__ gates,
                   uint16_t* __restrict__ out, int64_t num_tokens, int32_t k, int32_t chunks_per_row, int64_t y_rows,
                   const int32_t* __restrict__ valid_tokens) {
  // Products rounded, then added (no fused multiply-add): the reference's
  // rows.float() * weight, then .sum().
#pragma clang fp contract(off)
  const int64_t item = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  const int64_t t = item / chunks_per_row;
  const int32_t c = static_cast<int32_t>(item % chunks_per_row);
  const int64_t limit = valid_tokens ? min(num_tokens, static_cast<int64_t>(*valid_tokens)) : num_tokens;
  if (t >= limit) return;
  const int64_t d_model = static_cast<int64_t>(chunks_per_row) * 8;

  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  auto add = [&](const u32x4_t& v, float g) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      acc[2 * q] += __uint_as_float(v[q] << 16) * g;
      acc[2 * q + 1] += __uint_as_float(v[q] & 0xffff0000u) * g;
    }
  };
  if constexpr (KMAX > 0) {
    int32_t row[KMAX];
    float g[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      row[j] = copy_row[t * KMAX + j];
      g[j] = gate_f32(gates, t * KMAX + j);
    }
    u32x4_t v[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; ++j) {
      const bool ok = row[j] >= 0 && row[j] < y_rows;  // a skipped copy (bad expert id) adds nothing
      v[j] = ok ? *reinterpret_cast<const u32x4_t*>(y + row[j] * d_model + c * 8) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int j = 0; j < KMAX; ++j)
      if (row[j] >= 0 && row[j] < y_rows) add(v[j], g[j]);
  } else {
    for (int32_t j = 0; j < k; ++j) {
      const int32_t row = copy_row[t * k + j];
      if (row < 0 || row >= y_rows) continue;  // skipped copy (bad expert id)
      add(*reinterpret_cast<const u32x4_t*>(y + row * d_model + c * 8), gate_f32(gates, t * k + j));
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
  const uint32_t groups = static_cast<uint32_t>((num_tokens * chunks + 255) / 256);
  const auto* yp = static_cast<const uint16_t*>(y);
  const auto* gp = static_cast<const G*>(gates);
  auto* op = static_cast<uint16_t*>(out);
  auto run = [&](auto kmax) {
    combine_kernel<G, decltype(kmax)::value>
        <<<groups, 256, 0, stream>>>(yp, copy_row, gp, op, num_tokens, k, chunks, y_rows, valid_tokens);
  };
  switch (k) {
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 2>{}); break;
    case 4: run(std::integral_constant<int, 4>{}); break;
    case 8: run(std::integral_constant<int, 8>{}); break;
    default: run(std::integral_constant<int, 0>{}); break;
  }
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
