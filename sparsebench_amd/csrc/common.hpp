// Shared helpers for the gfx950 kernels and their C-ABI launchers.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
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

// Test hooks (sb_set_test_hook): process-wide overrides of a built-in
// choice, 0 keeping the choice. SB_HOOK_EXPERT_GATE forces one tiling of
// the layer kernels, SB_HOOK_TOPK_KERNEL one form of the top-k router.
// Only tests set them; the product path reads no environment.
int32_t test_hook(int32_t hook);

// Row blocks per tile group (see tile_coords).
constexpr int kTileGroup = 8;

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// ------------------------------------------------------------------ bf16 ---

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float(static_cast<uint32_t>(h) << 16); }

typedef __bf16 bf16x2_pack_t __attribute__((ext_vector_type(2)));

// fp32 -> bf16, round to nearest even, NaN kept (gfx950's v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2_pack_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
  return __builtin_bit_cast(uint32_t, v);
}

// ------------------------------------------------------------ scheduling ---

constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, each with its own L2

// A value every lane of the wave holds alike, said so for the compiler (a
// scalar register; v_readfirstlane). The tile schedules below are also
// compiled for the CPU (the tool library's shims, checked by
// tests/test_tile_schedules.py), where the value is returned as it is.
__host__ __device__ __forceinline__ int uniform(int v) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_readfirstlane(v);
#else
  return v;
#endif
}

// Workgroups are handed to the XCDs round-robin by id. For ids in
// [0, live), return a permutation of [0, live) that gives each XCD one
// contiguous range of logical tiles, so tiles that share operands (the
// column slices of one row block, the row blocks of one expert) run on the
// same XCD and meet in its L2. Ids >= live map to themselves.
__host__ __device__ __forceinline__ int xcd_remap(int bid, int live) {
  if (bid >= live) return bid;
  const int per = live / kNumXcd;
  const int rem = live % kNumXcd;
  const int x = bid % kNumXcd;
  const int q = bid / kNumXcd;
  return x < rem ? x * (per + 1) + q : rem * (per + 1) + (x - rem) * per + q;
}

// The same spread, with a short last round split. An XCD that runs n of the
// tiles on c CUs runs them in ceil(n / c) rounds; when its last round holds
// r <= c / 2 tiles, those r tiles are each split into two column halves that
// run as workgroups of their own, so 2r CUs share the round and it ends
// sooner (a half tile takes a little over half the time of a whole one).
// Workgroup bid gets logical tile `tile` (>= tiles: no work) and `half`:
// -1 for the whole tile, else 0 or 1. The grid needs up to
// kNumXcd * (ceil(tiles / kNumXcd) + c / 2) workgroups; ids past an XCD's
// share get tile = tiles.
struct TailTile {
  int tile, half;
};
__host__ __device__ __forceinline__ TailTile split_tail(int bid, int tiles, int cus_per_xcd) {
  const int per = tiles / kNumXcd;
  const int rem = tiles % kNumXcd;
  const int x = bid % kNumXcd;
  const int q = bid / kNumXcd;
  const int n = per + (x < rem ? 1 : 0);
  const int start = x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per;
  const int r = cus_per_xcd > 0 ? n % cus_per_xcd : 0;
  const int split = (r > 0 && 2 * r <= cus_per_xcd) ? r : 0;
  const int whole = n - split;
  TailTile t{tiles, -1};
  if (q < whole) {
    t.tile = start + q;
  } else if (q < whole + 2 * split) {
    t.tile = start + whole + (q - whole) / 2;
    t.half = (q - whole) % 2;
  }
  t.tile = uniform(t.tile);
  t.half = uniform(t.half);
  return t;
}

// Extra workgroups a grid of split_tail needs beyond its tiles.
__host__ __device__ inline int64_t split_tail_slack(int cus) { return kNumXcd * (cus / kNumXcd / 2 + 1); }

// Logical tile -> (row block, column slice) for the live region: tiles are
// taken in groups of `group` row blocks, walking down the group one column
// slice at a time, so the tiles that run together on one XCD cover a few
// row blocks x a few slices and share both their A rows and their W columns
// in that XCD's L2. Tiles past the live region map row block first.
// All arguments are wave-uniform; the results are made so explicitly: the
// integer divisions run on the vector unit, and a result left in a VGPR
// stays live across the caller's main loop (the layer kernels, which use
// all 512 registers, spilled it to scratch).
__host__ __device__ __forceinline__ void tile_coords(int tile, int live_rb, int slices, int group, int* rb,
                                                     int* slice) {
  int r, s;
  if (tile >= live_rb * slices || group <= 1) {
    r = tile / slices;
    s = tile % slices;
  } else {
    const int per_group = group * slices;
    const int g = tile / per_group;
    const int first = g * group;
    const int size = group < live_rb - first ? group : live_rb - first;
    const int local = tile - g * per_group;
    r = first + local % size;
    s = local / size;
  }
  *rb = uniform(r);
  *slice = uniform(s);
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
