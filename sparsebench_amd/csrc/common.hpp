// Shared helpers for the gfx950 kernels and their C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <algorithm>
#include <string>
#include <type_traits>

#include "sparsebench_hip.h"

namespace sb {

// ---------------------------------------------------------------- errors ---

// Last error message of the calling host thread (read by sb_last_error).
std::string& last_error();

// printf-style: records the message and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

inline int clear_ok() {
  last_error().clear();
  return SB_OK;
}

// Checks the launch that was just enqueued (bad grid, missing code object).
inline int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(SB_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return SB_OK;
}

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------------ bf16 ---

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

// Round to nearest even; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  const uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x0040u);
  return static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f32_to_bf16(lo)) | (static_cast<uint32_t>(f32_to_bf16(hi)) << 16);
}

// ------------------------------------------------------------ scheduling ---

constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, each with its own L2

// Workgroups are handed to the XCDs round-robin by id. For ids in
// [0, live), return a permutation of [0, live) that gives each XCD one
// contiguous range of logical tiles, so tiles that share operands (the
// column slices of one row block, the row blocks of one expert) run on the
// same XCD and meet in its L2. Ids >= live map to themselves.
__device__ __forceinline__ int xcd_remap(int bid, int live) {
  if (bid >= live) return bid;
  const int per = live / kNumXcd;
  const int rem = live % kNumXcd;
  const int x = bid % kNumXcd;
  const int q = bid / kNumXcd;
  return x < rem ? x * (per + 1) + q : rem * (per + 1) + (x - rem) * per + q;
}

// Number of leading row blocks that can hold work. The routing layout puts
// every dead row block (no non-zero blocks) after the live ones and gives
// each live one the same block count, so the live prefix is
// total / per_row when row_offsets confirms it; otherwise all of them.
__device__ __forceinline__ int live_row_blocks(const int32_t* __restrict__ row_offsets, int num_row_blocks) {
  const int32_t total = row_offsets[num_row_blocks];
  const int32_t per_row = row_offsets[1] - row_offsets[0];
  if (per_row > 0 && total % per_row == 0) {
    const int32_t est = total / per_row;
    if (est <= num_row_blocks && row_offsets[est] == total) return est;
  }
  return num_row_blocks;
}

}  // namespace sb
