// The bf16 MFMA tile loop shared by SDD and DSD on gfx950.
//
// One workgroup of WM x WN wave64s computes a BM x BN fp32 tile
//     acc += A[BM, K] @ B[K, BN]
// in K steps of 64 with v_mfma_f32_32x32x16_bf16. Each wave owns a
// (BM/WM) x (BN/WN) sub-tile, i.e. TM x TN blocks of 32 x 32.
//
// Operands. Both GEMMs read A with K contiguous (gathered token rows of x for
// SDD, the rows of a 128 x 128 H block for DSD) and B with N contiguous (rows
// of W1[e] or W2). MFMA wants every lane to hold 8 consecutive K values of
// one row (A) or one column (B), so B is transposed on its way into LDS:
// each lane loads an 8(K) x NC(N) patch (8 row loads, coalesced along N over
// the wave), transposes it in registers with v_perm_b32, and writes NC
// K-contiguous 16-byte chunks. LDS then holds both tiles K-contiguous,
// 64 K = 128 bytes = 8 chunks per row, chunk c of row r stored at
// c ^ swz(r): consecutive rows spread over all banks for the fragment reads
// (32 rows, one chunk) and for the B transpose writes (rows NC apart).
//
// Pipeline: LDS double buffer, plus PF K steps prefetched in registers. The
// global loads for step t+PF are issued before the MFMAs of step t; step t+1
// is written to the other LDS buffer after them: one barrier per K step.
//
// The caller supplies a loader with
//   load_a(t, pos, u32x4 (&a)[kAChunks])   this lane's A chunks of K step t
//   load_b(t, pos, BRow (&b)[8])           this lane's 8 B rows of K step t
// (zeros where there is no data) and consumes acc after run().
#pragma once

#include "common.hpp"

namespace sb {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x1_t __attribute__((ext_vector_type(1)));

template <int NC>
struct BRowOf;
template <>
struct BRowOf<8> { using type = u32x4_t; };
template <>
struct BRowOf<4> { using type = u32x2_t; };
template <>
struct BRowOf<2> { using type = u32x1_t; };

// NTB: load B (the weights) with the non-temporal hint.
template <int BM_, int BN_, int WM_ = 2, int WN_ = 2, int PF_ = 1, bool NTB_ = false>
struct TileCfg {
  static constexpr bool NTB = NTB_;
  static constexpr int BM = BM_;
  static constexpr int BN = BN_;
  static constexpr int BK = 64;
  static constexpr int WM = WM_, WN = WN_;             // waves along M and N
  static constexpr int PF = PF_;                       // K steps prefetched in registers
  static constexpr int kThreads = 64 * WM * WN;
  static constexpr int WTM = BM / WM, WTN = BN / WN;   // wave sub-tile
  static constexpr int TM = WTM / 32, TN = WTN / 32;   // 32 x 32 MFMA blocks per wave
  static constexpr int kAChunks = BM * (BK / 8) / kThreads;  // 16-byte A chunks per lane per K step
  static constexpr int kBCols = BN * BK / 8 / kThreads;      // B columns per lane (each 8 K deep)
  static constexpr int kBGroups = BN / kBCols;               // lanes along N in the B load
  static constexpr int kAElems = BM * BK;
  static constexpr int kStageElems = BM * BK + BN * BK;
  static constexpr int kLdsElems = 2 * kStageElems;
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "waves own whole 32 x 32 MFMA blocks");
  static_assert(kAChunks >= 1 && BM * (BK / 8) % kThreads == 0, "A chunks must divide over the lanes");
  static_assert(kBCols == 2 || kBCols == 4 || kBCols == 8, "B patch is 8 K x 2, 4 or 8 N");
  static_assert(kBGroups * 8 == kThreads, "8 K groups of 8 rows cover BK");
  static_assert(PF == 1 || PF == 2, "prefetch depth 1 or 2");
  using BRow = typename BRowOf<kBCols>::type;
};

// 8- or 16-byte global load, optionally with the non-temporal hint.
template <bool NT, class V>
__device__ __forceinline__ V load_vec(const uint16_t* p) {
  const V* q = reinterpret_cast<const V*>(p);
  if constexpr (NT) return __builtin_nontemporal_load(q);
  else return *q;
}

// Chunk position of logical chunk c in LDS row r.
__device__ __forceinline__ int swz(int r) { return (r ^ (r >> 3)) & 7; }
__device__ __forceinline__ int lds_off(int r, int c) { return r * 64 + ((c ^ swz(r)) << 3); }

// 8 rows x NC bf16 -> NC columns x 8 bf16 (K pairs packed low/high).
template <int NC, class In>
__device__ __forceinline__ void transpose_patch(const In (&in)[8], u32x4_t (&out)[NC]) {
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const uint32_t sel = (i & 1) ? 0x07060302u : 0x05040100u;
#pragma unroll
    for (int p = 0; p < 4; ++p) out[i][p] = __builtin_amdgcn_perm(in[2 * p + 1][i >> 1], in[2 * p][i >> 1], sel);
  }
}

template <class Cfg>
struct Mainloop {
  using BRow = typename Cfg::BRow;
  using Acc = f32x16_t[Cfg::TM][Cfg::TN];

  // This lane's place in the A and B loads (fixed for the whole loop).
  struct LoadPos {
    int a_row[Cfg::kAChunks];  // tile row of each A chunk
    int a_chunk;               // K chunk (0..7), the same for all of them
    int b_kgroup;              // B rows 8*b_kgroup .. +7
    int b_col;                 // first of kBCols B columns
  };

  struct Regs {
    u32x4_t a[Cfg::kAChunks];
    BRow b[8];
  };

  __device__ __forceinline__ static LoadPos load_pos() {
    LoadPos p;
    const int tid = threadIdx.x;
#pragma unroll
    for (int j = 0; j < Cfg::kAChunks; ++j) p.a_row[j] = (tid + j * Cfg::kThreads) >> 3;
    p.a_chunk = tid & 7;
    p.b_kgroup = tid / Cfg::kBGroups;
    p.b_col = (tid % Cfg::kBGroups) * Cfg::kBCols;
    return p;
  }

  template <class Loader>
  __device__ __forceinline__ static void load(Loader& ld, int t, const LoadPos& p, Regs& r) {
    ld.load_a(t, p, r.a);
    ld.load_b(t, p, r.b);
  }

  __device__ __forceinline__ static void store_stage(uint16_t* stage, const LoadPos& p, const Regs& r) {
#pragma unroll
    for (int j = 0; j < Cfg::kAChunks; ++j)
      *reinterpret_cast<u32x4_t*>(stage + lds_off(p.a_row[j], p.a_chunk)) = r.a[j];
    uint16_t* bs = stage + Cfg::kAElems;
    u32x4_t t[Cfg::kBCols];
    transpose_patch<Cfg::kBCols>(r.b, t);
#pragma unroll
    for (int i = 0; i < Cfg::kBCols; ++i)
      *reinterpret_cast<u32x4_t*>(bs + lds_off(p.b_col + i, p.b_kgroup)) = t[i];
  }

  __device__ __forceinline__ static void compute_stage(const uint16_t* stage, Acc& acc) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
    const uint16_t* as = stage;
    const uint16_t* bs = stage + Cfg::kAElems;
#pragma unroll
    for (int s = 0; s < Cfg::BK / 16; ++s) {
      const int chunk = 2 * s + (lane >> 5);
      bf16x8_t a[Cfg::TM], b[Cfg::TN];
#pragma unroll
      for (int i = 0; i < Cfg::TM; ++i) {
        const int r = wm * Cfg::WTM + i * 32 + (lane & 31);
        a[i] = *reinterpret_cast<const bf16x8_t*>(as + lds_off(r, chunk));
      }
#pragma unroll
      for (int j = 0; j < Cfg::TN; ++j) {
        const int r = wn * Cfg::WTN + j * 32 + (lane & 31);
        b[j] = *reinterpret_cast<const bf16x8_t*>(bs + lds_off(r, chunk));
      }
#pragma unroll
      for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
        for (int j = 0; j < Cfg::TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[i], b[j], acc[i][j], 0, 0, 0);
    }
  }

  template <class Loader>
  __device__ __forceinline__ static void run(uint16_t* lds, Loader& ld, int num_steps, Acc& acc) {
#pragma unroll
    for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
      for (int j = 0; j < Cfg::TN; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[i][j][v] = 0.0f;
    if (num_steps <= 0) return;

    const LoadPos pos = load_pos();
    if constexpr (Cfg::PF == 1) {
      Regs r;
      load(ld, 0, pos, r);
      store_stage(lds, pos, r);
      __syncthreads();
      for (int t = 0; t < num_steps; ++t) {
        const bool more = t + 1 < num_steps;
        if (more) load(ld, t + 1, pos, r);
        compute_stage(lds + (t & 1) * Cfg::kStageElems, acc);
        if (more) store_stage(lds + ((t + 1) & 1) * Cfg::kStageElems, pos, r);
        __syncthreads();
      }
    } else {
      // Two register sets: the loads of step t+2 are in flight during the
      // MFMAs of step t while step t+1's data is already waiting.
      Regs r[2];
      load(ld, 0, pos, r[0]);
      if (num_steps > 1) load(ld, 1, pos, r[1]);
      store_stage(lds, pos, r[0]);
      __syncthreads();
      for (int t = 0; t < num_steps; t += 2) {
        // even step t: compute buffer 0, r[1] holds t+1, r[0] is free
        if (t + 2 < num_steps) load(ld, t + 2, pos, r[0]);
        compute_stage(lds, acc);
        if (t + 1 >= num_steps) break;
        store_stage(lds + Cfg::kStageElems, pos, r[1]);
        __syncthreads();
        // odd step t+1: compute buffer 1, r[0] holds t+2, r[1] is free
        if (t + 3 < num_steps) load(ld, t + 3, pos, r[1]);
        compute_stage(lds + Cfg::kStageElems, acc);
        if (t + 2 < num_steps) store_stage(lds, pos, r[0]);
        __syncthreads();
      }
    }
  }

  // Tile coordinates of accumulator value v of block (i, j) for this lane:
  // the 32 x 32 MFMA result layout (column = lane % 32, four groups of four
  // consecutive rows).
  __device__ __forceinline__ static int acc_row(int i, int v) {
    const int lane = threadIdx.x & 63;
    const int wm = (threadIdx.x >> 6) / Cfg::WN;
    return wm * Cfg::WTM + i * 32 + (v >> 2) * 8 + (lane >> 5) * 4 + (v & 3);
  }
  __device__ __forceinline__ static int acc_col(int j) {
    const int lane = threadIdx.x & 63;
    const int wn = (threadIdx.x >> 6) % Cfg::WN;
    return wn * Cfg::WTN + j * 32 + (lane & 31);
  }
};

}  // namespace sb
