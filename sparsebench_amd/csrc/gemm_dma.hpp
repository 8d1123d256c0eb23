// The bf16 MFMA tile loop of SDD and DSD on gfx950, fed by LDS DMA.
//
// One workgroup of 4 wave64s (2 x 2) computes a BM x BN fp32 tile
//     C[BM, BN] = A[BM, K] @ B[K, BN]
// in K steps of 64. A has K contiguous (gathered token rows of x for SDD,
// rows of an H block for DSD); B has N contiguous (rows of W1[e] or W2).
//
// Global -> LDS: buffer_load_dwordx4 ... lds. Each wave instruction writes
// 1 KB of LDS (64 lanes x 16 bytes, consecutive) with no register staging,
// into a STAGES-deep ring; the loads for step t+STAGES-1 are issued before
// the MFMAs of step t and waited for with s_waitcnt vmcnt, so up to
// STAGES-1 steps stay in flight. A lane whose buffer offset is out of range
// gets zeros: the padding rows of SDD are filled that way, with no read.
//
// LDS layouts (both swizzled at 16-byte granularity, the swizzle applied by
// choosing which global chunk each lane fetches):
//   A  [BM][64] bf16, 128 B per row; logical chunk c of row r sits at
//      c ^ swzA(r), swzA(r) = (r ^ r >> 3) & 7.
//   B  [64][BN] bf16 as stored (row = k); logical chunk c of row k sits at
//      c ^ 4 (k & 3).
// Fragments (v_mfma_f32_32x32x16_bf16, operands swapped so that the result
// is C transposed and each lane holds 4 consecutive output columns):
//   W side (MFMA src A, 32 n x 16 k): two ds_read_b64_tr_b16 per block;
//      within each 16-lane group, lane j points at row k0 + j/4, columns
//      n0 + 4 (j % 4) .. +3, and lane i receives rows k0 .. k0+3 of column
//      n0 + i. Groups 0/1 cover k 0-7 (two reads), groups 2/3 k 8-15.
//   A side (MFMA src B, 16 k x 32 m): one ds_read_b128 of 8 consecutive k.
// Both sides hold k = 8 (lane / 32) + 0..7 of the 16-step, in the same order.
#pragma once

#include <type_traits>

#include "common.hpp"

namespace sb {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) i16x4_t lds_i16x4_t;

// Raw buffer resource word 3 for gfx9-family (CDNA) untyped loads.
constexpr int kBufferFlags = 0x00020000;
// Out-of-range buffer offset: loads there return zeros. Every valid offset
// (voffset + soffset) stays below 2^31, so this never wraps into range.
constexpr uint32_t kOutOfRange = 0x80000000u;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t num_bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), static_cast<int>(num_bytes),
                                           kBufferFlags);
}

__device__ __forceinline__ void wait_lgkmcnt0() {
  // gfx9 encoding of s_waitcnt lgkmcnt(0), vmcnt and expcnt left at their maximum.
  __builtin_amdgcn_s_waitcnt(15 | (3 << 14) | (7 << 4));
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N <= 63, "vmcnt range");
  // gfx9 encoding of s_waitcnt vmcnt(N), other counters left at their maximum.
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// CPA / CPB: cache policy of the A / B loads (buffer instruction bits; 2 = nt,
// a streaming hint that keeps the read-once weight stream from displacing
// reusable lines).
// PIPE: fragment schedule inside a K step. 0: per 16-deep sub-step, read
// its fragments then run its MFMAs (the compiler schedules). 1: two
// fragment register sets, sub-step s+1's LDS reads issued among sub-step
// s's MFMAs (scheduling groups pin the interleave). 2: the two register
// sets without the pinned interleave. 3: as 1, and the DMA of the step
// STAGES-1 ahead is issued among the MFMAs too, not as a burst after the
// barrier (a burst of DMA instructions holds each wave at issue until the
// address unit takes them, which delays its MFMAs). 4: as 3 with the A
// fragments single-buffered: each is read again for the next sub-step
// right after its last MFMA of this one (TM x 4 fewer registers, for tall
// tiles whose accumulators leave no room for a second set). 5: as 3, with
// the wait and barrier of step t+1 moved into step t's last sub-step, ahead
// of its MFMAs, and step t+1's first fragments read among them: otherwise
// every step starts with a barrier and LDS reads and no MFMA to cover them.
// EPI_PARTS: the epilogue stages the bf16 tile through LDS in this many
// parts of BM / EPI_PARTS rows (a 192 x 512 tile does not fit at once).
// APAIR: A is loaded two K steps at a time, as whole 128-byte rows (BK 32):
// a 64-byte row piece costs the address and data units a whole cache line,
// so pairing halves the A lines per byte. A pair m (K steps 2m, 2m+1) sits
// in A slot m % 2, B of step t in ring slot t % STAGES (STAGES 3 or 4).
// BSTAGES (0: as STAGES): a B ring deeper than the A ring (PIPE 5,
// unpaired): A of step t in slot t % STAGES, loaded STAGES-1 steps ahead,
// B in slot t % BSTAGES, loaded BSTAGES-1 steps ahead (DmaMainloop::
// run_split_xs). For tall tiles whose A area leaves no room for a fourth
// whole stage: the weight stream, whose misses go to HBM, keeps its lead.
template <int BM_, int BN_, int BK_, int STAGES_, int WM_ = 2, int WN_ = 2, int CPA_ = 0, int CPB_ = 0, int PIPE_ = 0,
          int EPI_PARTS_ = 1, int APAIR_ = 0, int BSTAGES_ = 0>
struct DmaCfg {
  static constexpr int BM = BM_, BN = BN_, BK = BK_, STAGES = STAGES_;
  static constexpr int BSTAGES = BSTAGES_ > 0 ? BSTAGES_ : STAGES_;
  static constexpr bool SPLIT = BSTAGES != STAGES;
  static constexpr int CPA = CPA_, CPB = CPB_;
  static constexpr int PIPE = PIPE_;
  static constexpr int EPI_PARTS = EPI_PARTS_;
  static constexpr bool APAIR = APAIR_ != 0;
  static constexpr int WM = WM_, WN = WN_;
  static constexpr int kWaves = WM * WN;
  static constexpr int kThreads = 64 * kWaves;
  static constexpr int WTM = BM / WM, WTN = BN / WN;
  static constexpr int TM = WTM / 32, TN = WTN / 32;
  static constexpr int kABK = APAIR ? 2 * BK : BK;  // K width of one A slot
  static constexpr int kARowBytes = kABK * 2;
  static constexpr int kAChunksPerRow = kABK / 8;
  // DMA instructions per wave for one A slot, and its area. When BM rows do
  // not split into whole 1 KB rows per wave, the area is rounded up: the
  // DMA rows past BM are loaded out of range (zeros, no memory read) and
  // never read back.
  static constexpr int kAInstr = (BM * kARowBytes + 1024 * kWaves - 1) / (1024 * kWaves);
  static constexpr int kABytes = kAInstr * kWaves * 1024;
  static constexpr int kBRowBytes = BN * 2;
  static constexpr int kBBytes = BK * kBRowBytes;
  static constexpr int kStageBytes = kABytes + kBBytes;
  static constexpr int kLdsBytes =
      APAIR ? 2 * kABytes + STAGES * kBBytes : (SPLIT ? STAGES * kABytes + BSTAGES * kBBytes : STAGES * kStageBytes);
  // LDS of a kernel: the ring, or the part of the bf16 output tile staged
  // through it in the epilogue if that is larger.
  static constexpr int kStagedPartBytes = BM * BN * 2 / EPI_PARTS;
  static constexpr int kLdsAlloc = kLdsBytes > kStagedPartBytes ? kLdsBytes : kStagedPartBytes;
  static constexpr int kBInstr = kBBytes / 1024 / kWaves;
  static constexpr int kLoadsPerStep = kAInstr + kBInstr;
  // The wait at the top of step t: step t's loads (and its A pair) are
  // complete once at most the loads issued after them are outstanding.
  // Unpaired: the STAGES-2 later steps'. Paired (see DmaMainloop::run):
  // STAGES-2 steps' B, and for odd t one A pair.
  static constexpr int kLaterLoads = (STAGES - 2) * kLoadsPerStep;
  static constexpr int kLaterLoadsEven = (STAGES - 2) * kBInstr;
  static constexpr int kLaterLoadsOdd = kAInstr + (STAGES - 2) * kBInstr;
  static constexpr int kARowsPerInstr = 1024 / kARowBytes;
  static constexpr int kBRowsPerInstr = kBRowBytes >= 1024 ? 1 : 1024 / kBRowBytes;
  static_assert(kBRowBytes <= 1024, "one DMA row per instruction at most");
  static constexpr int kBChunksPerRow = BN / 8;
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(BN == 128 || BN == 256 || BN == 512, "BN");
  static_assert(WTM % 32 == 0 && WTN % 32 == 0, "waves own whole 32 x 32 blocks");
  static_assert(kAInstr >= 1 && kABytes >= BM * kARowBytes, "the A area holds BM rows");
  static_assert(kBInstr >= 1 && kBInstr * kWaves * 1024 == kBBytes, "B step splits into whole 1 KB DMA rows");
  static_assert(STAGES >= 2 && STAGES <= 8, "STAGES");
  static_assert(kLdsAlloc <= 160 * 1024, "LDS");
  static_assert((APAIR ? kLaterLoadsOdd : kLaterLoads) <= 63, "vmcnt");
  static_assert(!APAIR || (BK == 32 && (STAGES == 3 || STAGES == 4) && (PIPE == 3 || PIPE == 4 || PIPE == 5)),
                "paired A: BK 32, a 3- or 4-stage B ring, DMA among the MFMAs");
  static_assert(EPI_PARTS == 1 || (WM == 1 && TM % EPI_PARTS == 0), "epilogue parts of whole row groups");
  static_assert(!SPLIT || (!APAIR && PIPE == 5 && BSTAGES > STAGES && STAGES >= 2 && BSTAGES <= 8),
                "a deeper B ring: unpaired PIPE 5");
  // The split ring's wait: loads issued after step t's A, in steady state.
  static constexpr int kSplitLater = kBInstr + (STAGES - 2) * (kAInstr + kBInstr);
  static_assert(!SPLIT || kSplitLater + kBInstr <= 63, "vmcnt");
};

// Whether a reduction of k elements runs on Cfg's main loop: whole K steps,
// and with APAIR an even number of them (run_paired and run_paired_xs load
// A two steps at a time and count their waits for an even count; with an
// odd one the last pair is never loaded). Every launch of a paired tile
// checks it on the host next to its other shape checks.
template <class Cfg>
constexpr bool reduction_fits(int64_t k) {
  return k > 0 && k % Cfg::BK == 0 && (!Cfg::APAIR || (k / Cfg::BK) % 2 == 0);
}

// A rows are BK/8 16-byte chunks: logical chunk c of row r sits at c ^ swz_a(r).
// 16 consecutive rows read at one logical chunk hit 16 different 16-byte bank
// groups of the 256-byte bank span.
template <int BK>
__device__ __forceinline__ int swz_a(int r) {
  if constexpr (BK == 64) return (r ^ (r >> 3)) & 7;  // 2 rows per 256 B
  else return (r >> 2) & 3;                             // 4 rows per 256 B
}

// This lane's LDS row / chunk for A DMA instruction q, and the logical
// chunk it must fetch.
template <class Cfg>
struct ADmaPos {
  int row[Cfg::kAInstr];
  int chunk[Cfg::kAInstr];  // logical 16-byte chunk (8 k values)
  __device__ __forceinline__ ADmaPos() {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int q = 0; q < Cfg::kAInstr; ++q) {
      row[q] = Cfg::kARowsPerInstr * (Cfg::kAInstr * wave + q) + lane / Cfg::kAChunksPerRow;
      chunk[q] = (lane % Cfg::kAChunksPerRow) ^ swz_a<Cfg::kABK>(row[q]);
    }
  }
};

template <class Cfg>
struct BDmaPos {
  int row[Cfg::kBInstr];    // k row within the step
  int col[Cfg::kBInstr];    // first of 8 n columns (logical)
  __device__ __forceinline__ BDmaPos() {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int q = 0; q < Cfg::kBInstr; ++q) {
      row[q] = Cfg::kBRowsPerInstr * (Cfg::kBInstr * wave + q) + lane / Cfg::kBChunksPerRow;
      const int p = lane % Cfg::kBChunksPerRow;
      col[q] = 8 * (p ^ (4 * (row[q] & 3)));
    }
  }
};

// Scheduling groups for one sub-step: MFMA, then up to kPer DS reads,
// kMfma times (mask 0x008 = MFMA, 0x100 = DS read).
template <int Q, int kMfma, int kReads, int kPer>
__device__ __forceinline__ void sched_interleave() {
  if constexpr (Q < kMfma) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int left = kReads - Q * kPer;
    constexpr int n = left <= 0 ? 0 : (left < kPer ? left : kPer);
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x100, n, 0);
    sched_interleave<Q + 1, kMfma, kReads, kPer>();
  }
}

// f(integral_constant<int, I>) for I = B .. E-1, in order.
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// PIPE 3 scheduling groups for one sub-step of kMfma MFMAs: after MFMA Q
// come up to kPer of the next sub-step's kReads DS reads, and the DMA
// instructions whose turn it is, kDma of them spread evenly over the MFMAs
// (masks: 0x008 MFMA, 0x100 DS read, 0x020 VMEM read).
template <int Q, int kMfma, int kReads, int kPer, int kDma>
__device__ __forceinline__ void sched_substep_with_dma() {
  if constexpr (Q < kMfma) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    constexpr int left = kReads - Q * kPer;
    constexpr int n = left <= 0 ? 0 : (left < kPer ? left : kPer);
    if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x100, n, 0);
    constexpr int due = (Q + 1) * kDma / kMfma - Q * kDma / kMfma;
    if constexpr (due > 0) __builtin_amdgcn_sched_group_barrier(0x020, due, 0);
    sched_substep_with_dma<Q + 1, kMfma, kReads, kPer, kDma>();
  }
}

// s_waitcnt vmcnt(later * L) for a run-time `later` in [0, MAXL].
template <int L, int MAXL>
__device__ __forceinline__ void wait_steps(int later) {
  if constexpr (MAXL <= 0) {
    wait_vmcnt<0>();
  } else {
    if (later >= MAXL) wait_vmcnt<MAXL * L>();
    else wait_steps<L, MAXL - 1>(later);
  }
}

// Per-step sources, supplied by the kernel:
//   a_src(t, &rsrc, &soffset), b_src(t, &rsrc, &soffset)
// and fixed per-lane offsets a_voff(q), q < kAInstr, b_voff(q), q < kBInstr
// (bytes). A source with kGlobalA = true gives A as per-lane 64-bit
// addresses instead, a_global(q, t), loaded with global_load_lds (same LDS
// destination, same vmcnt accounting).
template <class Src, class = void>
struct GlobalA : std::false_type {};
template <class Src>
struct GlobalA<Src, std::void_t<decltype(Src::kGlobalA)>> : std::bool_constant<Src::kGlobalA> {};

template <class Cfg>
struct DmaMainloop {
  using Acc = f32x16_t[Cfg::TN][Cfg::TM];  // acc[j][i]: C^T block (n block j, m block i)

  // The DMA and compute() take their LDS slots through __restrict__ pointers:
  // the DMA of step t+STAGES-1 writes different slots than the ones step t
  // reads, and saying so lets the compiler drop the vmcnt(0) it would
  // otherwise put before every LDS read (which serializes loads and MFMAs).
  // Slots of K step t: its A (shared by a stage pair with APAIR) and its B.
  __device__ __forceinline__ static uint8_t* a_slot(uint8_t* lds, int t) {
    if constexpr (Cfg::APAIR) return lds + ((t >> 1) & 1) * Cfg::kABytes;
    else if constexpr (Cfg::SPLIT) return lds + (t % Cfg::STAGES) * Cfg::kABytes;
    else return lds + (t % Cfg::STAGES) * Cfg::kStageBytes;
  }
  __device__ __forceinline__ static uint8_t* b_slot(uint8_t* lds, int t) {
    if constexpr (Cfg::APAIR) return lds + 2 * Cfg::kABytes + (t % Cfg::STAGES) * Cfg::kBBytes;
    else if constexpr (Cfg::SPLIT) return lds + Cfg::STAGES * Cfg::kABytes + (t % Cfg::BSTAGES) * Cfg::kBBytes;
    else return lds + (t % Cfg::STAGES) * Cfg::kStageBytes + Cfg::kABytes;
  }

  // The DMA instructions of the A slot that starts at K step `ta` (if
  // kWithA) and of K step `tb`'s B (if kWithB): dma(q), q < kCount, issues
  // this wave's instruction q (A rows first, then B rows). Unpaired: ta = tb.
  template <class Src, bool kWithA = true, bool kWithB = true>
  struct StepDma {
    static constexpr int kA = kWithA ? Cfg::kAInstr : 0;
    static constexpr int kCount = kA + (kWithB ? Cfg::kBInstr : 0);
    uint8_t* __restrict__ a_dst;
    uint8_t* __restrict__ b_dst;
    __amdgpu_buffer_rsrc_t ra, rb;
    uint32_t sa, sb;
    const Src& src;
    int wave, t;
    __device__ __forceinline__ StepDma(uint8_t* __restrict__ a_dst_, int ta, uint8_t* __restrict__ b_dst_, int tb,
                                       const Src& src_)
        : a_dst(a_dst_), b_dst(b_dst_), src(src_), t(ta) {
      wave = threadIdx.x >> 6;
      // The scalar offsets are uniform by contract; saying so keeps the
      // compiler from wrapping each load in a per-lane waterfall loop when
      // it cannot prove it.
      if constexpr (kWithA) {
        src.a_src(ta, &ra, &sa);
        sa = __builtin_amdgcn_readfirstlane(sa);
      }
      if constexpr (kWithB) {
        src.b_src(tb, &rb, &sb);
        sb = __builtin_amdgcn_readfirstlane(sb);
      }
    }
    __device__ __forceinline__ void operator()(int q) const {
      if (q < kA) {
        lds_void_t* dst = (lds_void_t*)(a_dst + (Cfg::kAInstr * wave + q) * 1024);
        if constexpr (GlobalA<Src>::value)
          __builtin_amdgcn_global_load_lds(src.a_global(q, t), dst, 16, 0, Cfg::CPA);
        else
          __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, dst, 16, src.a_voff(q), sa, 0, Cfg::CPA);
      } else {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_void_t*)(b_dst + (Cfg::kBInstr * wave + q - kA) * 1024),
                                                 16, src.b_voff(q - kA), sb, 0, Cfg::CPB);
      }
    }
  };

  // Unpaired: the loads of K step u, A and B.
  template <class Src>
  __device__ __forceinline__ static StepDma<Src, true> step_dma(uint8_t* __restrict__ lds, int u, const Src& src) {
    return StepDma<Src, true>(a_slot(lds, u), u, b_slot(lds, u), u, src);
  }
  // Paired: A pair m's loads (from K step 2m) with step u's B, or u's B only.
  template <class Src>
  __device__ __forceinline__ static StepDma<Src, true> pair_dma(uint8_t* __restrict__ lds, int m, int u,
                                                               const Src& src) {
    return StepDma<Src, true>(a_slot(lds, 2 * m), 2 * m, b_slot(lds, u), u, src);
  }
  template <class Src>
  __device__ __forceinline__ static StepDma<Src, false> b_dma(uint8_t* __restrict__ lds, int u, const Src& src) {
    return StepDma<Src, false>(nullptr, 0, b_slot(lds, u), u, src);
  }
  template <class Src>
  __device__ __forceinline__ static StepDma<Src, true, false> a_dma(uint8_t* __restrict__ lds, int m, const Src& src) {
    return StepDma<Src, true, false>(a_slot(lds, 2 * m), 2 * m, nullptr, 0, src);
  }
  template <class Dma>
  __device__ __forceinline__ static void issue_all(const Dma& dma) {
#pragma unroll
    for (int q = 0; q < Dma::kCount; ++q) dma(q);
  }
  // The first step's loads, B before A: B (the weights) needs no load of its
  // own to address, while A's offsets may wait on one (the SDD's token rows),
  // so B's fetch starts under that wait. Step 0's last load is then its A,
  // and the loads issued after it are those of the later steps, as counted
  // by every wait below.
  template <class Dma>
  __device__ __forceinline__ static void issue_b_first(const Dma& dma) {
#pragma unroll
    for (int q = Dma::kA; q < Dma::kCount; ++q) dma(q);
#pragma unroll
    for (int q = 0; q < Dma::kA; ++q) dma(q);
  }

  struct NoDma {
    static constexpr int kCount = 0;
    __device__ __forceinline__ void operator()(int) const {}
  };

  __device__ __forceinline__ static void compute(const uint8_t* __restrict__ as, const uint8_t* __restrict__ bs,
                                                 int khalf, Acc& acc) {
    compute(as, bs, khalf, acc, NoDma{});
  }

  // The lane's LDS offsets for its MMA fragments, fixed for the tile.
  //   A side (MFMA src B): row m = wm*WTM + 32 i + lane % 32, 8 k values
  //   of chunk 2s + kc, kc = 4 khalf + lane / 32.
  //   W side (MFMA src A): lane j of its 16-group reads row (k0 + j/4),
  //   columns n0 + 16 (group % 2) + 4 (j % 4); chunk block (4 chunks =
  //   64 B) of n block jn is XORed with (k & 3) = j / 4.
  struct Frags {
    int a_row_off[Cfg::TM], a_swz[Cfg::TM], b_off[Cfg::TN];
    int h;
    __device__ __forceinline__ Frags() {
      const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
      const int wm = wave / Cfg::WN, wn = wave % Cfg::WN;
      h = lane >> 5;
#pragma unroll
      for (int i = 0; i < Cfg::TM; ++i) {
        const int r = wm * Cfg::WTM + 32 * i + (lane & 31);
        a_row_off[i] = r * Cfg::kARowBytes;
        a_swz[i] = swz_a<Cfg::kABK>(r);
      }
      const int g = lane >> 4, jj = lane & 15;
      const int krow = 8 * (g >> 1) + (jj >> 2);
#pragma unroll
      for (int jn = 0; jn < Cfg::TN; ++jn) {
        const int blk = (wn * Cfg::WTN) / 32 + jn;  // 32-column block index
        const int chunk = 4 * (blk ^ (jj >> 2)) + 2 * (g & 1) + ((jj & 3) >> 1);
        b_off[jn] = krow * Cfg::kBRowBytes + chunk * 16 + (jj & 1) * 8;
      }
    }
    // Sub-step s's A fragment of row group i (K half `khalf` of a paired slot).
    __device__ __forceinline__ bf16x8_t read_a1(const uint8_t* __restrict__ as, int khalf, int s, int i) const {
      const int kc = 4 * khalf + h;
      return *reinterpret_cast<const bf16x8_t*>(as + a_row_off[i] + (((2 * s + kc) ^ a_swz[i]) << 4));
    }
    __device__ __forceinline__ void read_a(const uint8_t* __restrict__ as, int khalf, int s,
                                           bf16x8_t (&a)[Cfg::TM]) const {
#pragma unroll
      for (int i = 0; i < Cfg::TM; ++i) a[i] = read_a1(as, khalf, s, i);
    }
    __device__ __forceinline__ void read_b(const uint8_t* __restrict__ bs, int s, bf16x8_t (&b)[Cfg::TN]) const {
#pragma unroll
      for (int jn = 0; jn < Cfg::TN; ++jn) {
        const uint8_t* p = bs + b_off[jn] + 16 * s * Cfg::kBRowBytes;
        const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p));
        const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + 4 * Cfg::kBRowBytes));
        b[jn] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
      }
    }
  };
  __device__ __forceinline__ static void mfmas(Acc& acc, const bf16x8_t (&a)[Cfg::TM], const bf16x8_t (&b)[Cfg::TN]) {
#pragma unroll
    for (int jn = 0; jn < Cfg::TN; ++jn)
#pragma unroll
      for (int i = 0; i < Cfg::TM; ++i)
        acc[jn][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[jn], a[i], acc[jn][i], 0, 0, 0);
  }

  // One K step's fragments and MFMAs, from A slot `as` (K half `khalf` of
  // it with APAIR, else 0) and B slot `bs`. With PIPE 3 and 4, dma(q) for
  // q < Dma::kCount is called among the MFMAs (a later step's loads, into
  // other slots), spread evenly by the scheduling groups.
  template <class Dma>
  __device__ __forceinline__ static void compute(const uint8_t* __restrict__ as, const uint8_t* __restrict__ bs,
                                                 int khalf, Acc& acc, const Dma& dma) {
    const Frags fr;
    constexpr int kSub = Cfg::BK / 16;
    auto read_a = [&](int s, bf16x8_t (&a)[Cfg::TM]) { fr.read_a(as, khalf, s, a); };
    auto read_b = [&](int s, bf16x8_t (&b)[Cfg::TN]) { fr.read_b(bs, s, b); };
    auto mfmas = [&](const bf16x8_t (&a)[Cfg::TM], const bf16x8_t (&b)[Cfg::TN]) { DmaMainloop::mfmas(acc, a, b); };
    if constexpr (Cfg::PIPE == 4) {
      constexpr int kDma = Dma::kCount;
      auto read_a1 = [&](int sub, int i) { return fr.read_a1(as, khalf, sub, i); };
      bf16x8_t a[Cfg::TM], b[2][Cfg::TN];
      read_a(0, a);
      read_b(0, b[0]);
      static_for<0, kSub>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        if constexpr (s + 1 < kSub) read_b(s + 1, b[(s + 1) & 1]);
        static_for<0, Cfg::TM>([&](auto ic) {
          constexpr int i = decltype(ic)::value;
#pragma unroll
          for (int jn = 0; jn < Cfg::TN; ++jn)
            acc[jn][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[s & 1][jn], a[i], acc[jn][i], 0, 0, 0);
          if constexpr (s + 1 < kSub) a[i] = read_a1(s + 1, i);
          // This sub-step's share of the DMA, spread over its row groups.
          constexpr int q0 = s * kDma / kSub + i * (kDma / kSub) / Cfg::TM;
          constexpr int q1 = s * kDma / kSub + (i + 1 == Cfg::TM ? kDma / kSub : (i + 1) * (kDma / kSub) / Cfg::TM);
#pragma unroll
          for (int q = q0; q < q1; ++q) dma(q);
        });
      });
      // Whatever the division leaves over.
#pragma unroll
      for (int q = kSub * (kDma / kSub); q < kDma; ++q) dma(q);
      return;
    }
    if constexpr (Cfg::PIPE == 3) {
      constexpr int kMfma = Cfg::TM * Cfg::TN;
      constexpr int kReads = Cfg::TM + 2 * Cfg::TN;
      constexpr int kPer = (kReads + kMfma - 1) / kMfma;
      constexpr int kDma = Dma::kCount;
      bf16x8_t a[2][Cfg::TM], b[2][Cfg::TN];
      read_a(0, a[0]);
      read_b(0, b[0]);
      // Each sub-step is its own scheduling region (sched_barrier), holding
      // its MFMAs, the next sub-step's fragment reads and its share of the
      // DMA instructions, so the DMA spreads over the whole step.
      static_for<0, kSub>([&](auto sc) {
        constexpr int s = decltype(sc)::value;
        if constexpr (s + 1 < kSub) {
          read_a(s + 1, a[(s + 1) & 1]);
          read_b(s + 1, b[(s + 1) & 1]);
        }
        mfmas(a[s & 1], b[s & 1]);
#pragma unroll
        for (int q = s * kDma / kSub; q < (s + 1) * kDma / kSub; ++q) dma(q);
        if constexpr (s == 0) __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);  // sub-step 0's own reads
        sched_substep_with_dma<0, kMfma, (s + 1 < kSub ? kReads : 0), kPer,
                               (s + 1) * kDma / kSub - s * kDma / kSub>();
        __builtin_amdgcn_sched_barrier(0);
      });
      return;
    }
    if constexpr (Cfg::PIPE == 0) {
#pragma unroll
      for (int s = 0; s < kSub; ++s) {
        bf16x8_t a[Cfg::TM], b[Cfg::TN];
        read_a(s, a);
        read_b(s, b);
        mfmas(a, b);
      }
    } else {
      bf16x8_t a[2][Cfg::TM], b[2][Cfg::TN];
      read_a(0, a[0]);
      read_b(0, b[0]);
#pragma unroll
      for (int s = 0; s < kSub; ++s) {
        if (s + 1 < kSub) {
          read_a(s + 1, a[(s + 1) & 1]);
          read_b(s + 1, b[(s + 1) & 1]);
        }
        mfmas(a[s & 1], b[s & 1]);
      }
      if constexpr (Cfg::PIPE == 1) {
        // Interleave: the first sub-step's reads, then per later sub-step
        // its MFMAs alternating with the next sub-step's reads.
        constexpr int kMfma = Cfg::TM * Cfg::TN;
        constexpr int kReads = Cfg::TM + 2 * Cfg::TN;
        constexpr int kPer = (kReads + kMfma - 1) / kMfma;
        __builtin_amdgcn_sched_group_barrier(0x100, kReads, 0);  // DS reads of sub-step 0
#pragma unroll
        for (int s = 0; s < kSub; ++s) {
          if (s + 1 < kSub) sched_interleave<0, kMfma, kReads, kPer>();
          else __builtin_amdgcn_sched_group_barrier(0x008, kMfma, 0);
        }
      }
    }
  }

  using FragA = bf16x8_t[2][Cfg::TM];
  using FragB = bf16x8_t[2][Cfg::TN];

  // PIPE 5: one K step whose first sub-step's fragments are already in
  // a[0] / b[0]. The sub-steps before the last read the next sub-step's
  // fragments and issue this step's DMA among their MFMAs. The last one
  // first completes this step's LDS reads, waits for the next step's loads
  // (wait()), passes the barrier and reads the next step's first fragments
  // (slots nas / nbs) into a[0] / b[0], and then runs its MFMAs over those
  // reads' latency. All of this step's loads are issued before the wait, so
  // its counts are the ones a wait at the top of the next step would use.
  template <bool kNext, class Dma, class Wait>
  __device__ __forceinline__ static void compute_xs(const uint8_t* __restrict__ as, const uint8_t* __restrict__ bs,
                                                    int khalf, Acc& acc, const Dma& dma, const Frags& fr, FragA& a,
                                                    FragB& b, const uint8_t* __restrict__ nas,
                                                    const uint8_t* __restrict__ nbs, int nkhalf, const Wait& wait) {
    constexpr int kSub = Cfg::BK / 16;
    static_assert(kSub % 2 == 0, "the last sub-step uses the second register set");
    constexpr int kMfma = Cfg::TM * Cfg::TN;
    constexpr int kReads = Cfg::TM + 2 * Cfg::TN;
    constexpr int kPer = (kReads + kMfma - 1) / kMfma;
    constexpr int kDma = Dma::kCount;
    auto mfmas = [&](const bf16x8_t (&fa)[Cfg::TM], const bf16x8_t (&fb)[Cfg::TN]) { DmaMainloop::mfmas(acc, fa, fb); };
    static_for<0, kSub>([&](auto sc) {
      constexpr int s = decltype(sc)::value;
      if constexpr (s + 1 < kSub) {
        fr.read_a(as, khalf, s + 1, a[(s + 1) & 1]);
        fr.read_b(bs, s + 1, b[(s + 1) & 1]);
        mfmas(a[s & 1], b[s & 1]);
        constexpr int q0 = s * kDma / (kSub - 1), q1 = (s + 1) * kDma / (kSub - 1);
#pragma unroll
        for (int q = q0; q < q1; ++q) dma(q);
        sched_substep_with_dma<0, kMfma, kReads, kPer, q1 - q0>();
        __builtin_amdgcn_sched_barrier(0);
      } else {
        if constexpr (kNext) {
          wait_lgkmcnt0();  // this step's slots are read to their end before the barrier
          wait();
          __builtin_amdgcn_s_barrier();
          fr.read_a(nas, nkhalf, 0, a[0]);
          fr.read_b(nbs, 0, b[0]);
        }
        mfmas(a[s & 1], b[s & 1]);
        if constexpr (kNext) sched_interleave<0, kMfma, kReads, kPer>();
        __builtin_amdgcn_sched_barrier(0);
      }
    });
  }

  struct NoWait {
    __device__ __forceinline__ void operator()() const {}
  };
  template <int N>
  struct WaitVm {
    __device__ __forceinline__ void operator()() const { wait_vmcnt<N>(); }
  };

  // PIPE 5, paired A: the schedule of run_paired, each step's wait and
  // barrier moved into the step before it.
  template <class Src>
  __device__ __forceinline__ static void run_paired_xs(uint8_t* lds, const Src& src, int n, Acc& acc) {
    constexpr int S = Cfg::STAGES;
    constexpr int kA = Cfg::kAInstr, kB = Cfg::kBInstr;
    const Frags fr;
    FragA a;
    FragB b;
    issue_all(b_dma(lds, 0, src));
    issue_all(a_dma(lds, 0, src));
#pragma unroll
    for (int u = 1; u < S - 1; ++u)
      if (u < n) issue_all(b_dma(lds, u, src));
    if (S == 4 && n == 2) wait_vmcnt<kB>();
    else wait_vmcnt<Cfg::kLaterLoadsEven>();
    __builtin_amdgcn_s_barrier();
    fr.read_a(a_slot(lds, 0), 0, 0, a[0]);
    fr.read_b(b_slot(lds, 0), 0, b[0]);
    int t = 0;
    for (; t + S < n; t += 2) {
      compute_xs<true>(a_slot(lds, t), b_slot(lds, t), 0, acc, pair_dma(lds, t / 2 + 1, t + S - 1, src), fr, a, b,
                       a_slot(lds, t + 1), b_slot(lds, t + 1), 1, WaitVm<Cfg::kLaterLoadsOdd>{});
      compute_xs<true>(a_slot(lds, t + 1), b_slot(lds, t + 1), 1, acc, b_dma(lds, t + S, src), fr, a, b,
                       a_slot(lds, t + 2), b_slot(lds, t + 2), 0, WaitVm<Cfg::kLaterLoadsEven>{});
    }
    if (S == 4 && t + 2 < n) {  // t = n - 4, the last step that loads
      compute_xs<true>(a_slot(lds, t), b_slot(lds, t), 0, acc, pair_dma(lds, t / 2 + 1, t + 3, src), fr, a, b,
                       a_slot(lds, t + 1), b_slot(lds, t + 1), 1, WaitVm<kA + 2 * kB>{});
      ++t;
    }
    for (; t + 1 < n; ++t) {  // nothing left to load; the step after t has n - 2 - t after it
      const int later = n - 2 - t;
      auto w = [later] {
        if (later >= 2) wait_vmcnt<kA + 2 * kB>();
        else if (later == 1) wait_vmcnt<kB>();
        else wait_vmcnt<0>();
      };
      compute_xs<true>(a_slot(lds, t), b_slot(lds, t), t & 1, acc, NoDma{}, fr, a, b, a_slot(lds, t + 1),
                       b_slot(lds, t + 1), (t + 1) & 1, w);
    }
    compute_xs<false>(a_slot(lds, t), b_slot(lds, t), t & 1, acc, NoDma{}, fr, a, b, nullptr, nullptr, 0, NoWait{});
  }

  // s_waitcnt vmcnt(n) for a run-time n in [0, MAX].
  template <int MAX>
  __device__ __forceinline__ static void wait_vmcnt_upto(int n) {
    static_for<0, MAX + 1>([&](auto c) {
      if (n == decltype(c)::value) wait_vmcnt<decltype(c)::value>();
    });
  }

  // PIPE 5 with the deeper B ring (SPLIT). Step u issues A of step
  // u+STAGES-1, then B of step u+BSTAGES-1, each if it exists; the prologue
  // is steps -(BSTAGES-1) .. -1 of the same rule. Loads complete in issue
  // order and A of a step is issued after its B, so step t's data is in
  // once at most the loads issued after its A are outstanding: that step's
  // B (of step t+BSTAGES-STAGES) and the A and B of the STAGES-2 steps
  // after it, those that exist (split_later).
  __device__ __forceinline__ static int split_later(int t, int n) {
    constexpr int SA = Cfg::STAGES, SB = Cfg::BSTAGES;
    int later = t + SB - SA < n ? Cfg::kBInstr : 0;
#pragma unroll
    for (int d = 2 - SA; d <= -1; ++d) {
      later += t + d + SA - 1 < n ? Cfg::kAInstr : 0;
      later += t + d + SB - 1 < n ? Cfg::kBInstr : 0;
    }
    return later;
  }

  template <class Src>
  __device__ __forceinline__ static void run_split_xs(uint8_t* lds, const Src& src, int n, Acc& acc) {
    constexpr int SA = Cfg::STAGES, SB = Cfg::BSTAGES;
    const Frags fr;
    FragA a;
    FragB b;
    auto a_load = [&](int u) { return StepDma<Src, true, false>(a_slot(lds, u), u, nullptr, 0, src); };
#pragma unroll
    for (int u = -(SB - 1); u < 0; ++u) {
      if (u + SA - 1 >= 0 && u + SA - 1 < n) issue_all(a_load(u + SA - 1));
      if (u + SB - 1 < n) issue_all(b_dma(lds, u + SB - 1, src));
    }
    wait_vmcnt_upto<Cfg::kSplitLater>(split_later(0, n));
    __builtin_amdgcn_s_barrier();
    fr.read_a(a_slot(lds, 0), 0, 0, a[0]);
    fr.read_b(b_slot(lds, 0), 0, b[0]);
    int t = 0;
    // Both loads of each step exist.
    for (; t + SB - 1 < n && t + 1 < n; ++t)
      compute_xs<true>(a_slot(lds, t), b_slot(lds, t), 0, acc,
                       StepDma<Src, true, true>(a_slot(lds, t + SA - 1), t + SA - 1, b_slot(lds, t + SB - 1),
                                                t + SB - 1, src),
                       fr, a, b, a_slot(lds, t + 1), b_slot(lds, t + 1), 0,
                       [&] { wait_vmcnt_upto<Cfg::kSplitLater>(split_later(t + 1, n)); });
    // Only A loads left.
    for (; t + SA - 1 < n && t + 1 < n; ++t)
      compute_xs<true>(a_slot(lds, t), b_slot(lds, t), 0, acc, a_load(t + SA - 1), fr, a, b, a_slot(lds, t + 1),
                       b_slot(lds, t + 1), 0, [&] { wait_vmcnt_upto<Cfg::kSplitLater>(split_later(t + 1, n)); });
    // Nothing left to load.
    for (; t + 1 < n; ++t)
      compute_xs<true>(a_slot(lds, t), b_slot(lds, t), 0, acc, NoDma{}, fr, a, b, a_slot(lds, t + 1),
                       b_slot(lds, t + 1), 0, [&] { wait_vmcnt_upto<Cfg::kSplitLater>(split_later(t + 1, n)); });
    compute_xs<false>(a_slot(lds, t), b_slot(lds, t), 0, acc, NoDma{}, fr, a, b, nullptr, nullptr, 0, NoWait{});
  }

  // PIPE 5, unpaired.
  template <class Src>
  __device__ __forceinline__ static void run_xs(uint8_t* lds, const Src& src, int n, Acc& acc) {
    constexpr int S = Cfg::STAGES;
    const Frags fr;
    FragA a;
    FragB b;
    issue_b_first(step_dma(lds, 0, src));
#pragma unroll
    for (int s = 1; s < S - 1; ++s)
      if (s < n) issue_all(step_dma(lds, s, src));
    wait_steps<Cfg::kLoadsPerStep, S - 2>(n - 1);
    __builtin_amdgcn_s_barrier();
    fr.read_a(a_slot(lds, 0), 0, 0, a[0]);
    fr.read_b(b_slot(lds, 0), 0, b[0]);
    int t = 0;
    for (; t + S - 1 < n; ++t)
      compute_xs<true>(a_slot(lds, t), b_slot(lds, t), 0, acc, step_dma(lds, t + S - 1, src), fr, a, b,
                       a_slot(lds, t + 1), b_slot(lds, t + 1), 0, WaitVm<Cfg::kLaterLoads>{});
    for (; t + 1 < n; ++t) {
      const int later = n - 2 - t;
      compute_xs<true>(a_slot(lds, t), b_slot(lds, t), 0, acc, NoDma{}, fr, a, b, a_slot(lds, t + 1),
                       b_slot(lds, t + 1), 0, [later] { wait_steps<Cfg::kLoadsPerStep, S - 2>(later); });
    }
    compute_xs<false>(a_slot(lds, t), b_slot(lds, t), 0, acc, NoDma{}, fr, a, b, nullptr, nullptr, 0, NoWait{});
  }

  // Paired schedule (APAIR), for an even step count n: the prologue loads
  // A pair 0, then B of steps 0 .. STAGES-2. Step t then loads B of step
  // t+STAGES-1 and, if t is even, A pair t/2+1 (A first), each while it
  // exists: an A slot is refilled once the pair before it has been read to
  // its end, so A runs two steps ahead and B STAGES-1. The wait at the top
  // of step t counts the loads issued after step t's last one: B of the
  // STAGES-2 steps after it (the last of them issued with A pair t/2 when t
  // is even and STAGES is 4), plus, for odd t, the A pair its successor
  // step issued. In the last steps fewer loads follow: with STAGES 4 the
  // last four steps wait for 2B (and load A pair n/2-1 and the last B), A+2B,
  // B and nothing; with STAGES 3 the last two wait for B and nothing (and so
  // do the only two steps of n = 2 with STAGES 4).
  template <class Src>
  __device__ __forceinline__ static void run_paired(uint8_t* lds, const Src& src, int n, Acc& acc) {
    constexpr int S = Cfg::STAGES;
    issue_all(b_dma(lds, 0, src));
    issue_all(a_dma(lds, 0, src));
#pragma unroll
    for (int u = 1; u < S - 1; ++u)
      if (u < n) issue_all(b_dma(lds, u, src));
    int t = 0;
    for (; t + S < n; t += 2) {
      wait_vmcnt<Cfg::kLaterLoadsEven>();
      __builtin_amdgcn_s_barrier();
      compute(a_slot(lds, t), b_slot(lds, t), 0, acc, pair_dma(lds, t / 2 + 1, t + S - 1, src));
      wait_vmcnt<Cfg::kLaterLoadsOdd>();
      __builtin_amdgcn_s_barrier();
      compute(a_slot(lds, t + 1), b_slot(lds, t + 1), 1, acc, b_dma(lds, t + S, src));
    }
    if (S == 4 && t + 2 < n) {  // t = n - 4, the last step that loads (n = 2 has none)
      wait_vmcnt<2 * Cfg::kBInstr>();
      __builtin_amdgcn_s_barrier();
      compute(a_slot(lds, t), b_slot(lds, t), 0, acc, pair_dma(lds, t / 2 + 1, t + 3, src));
      ++t;
    }
    for (; t < n; ++t) {  // nothing left to load; `later` steps follow
      const int later = n - 1 - t;
      if (later >= 2) wait_vmcnt<Cfg::kAInstr + 2 * Cfg::kBInstr>();
      else if (later == 1) wait_vmcnt<Cfg::kBInstr>();
      else wait_vmcnt<0>();
      __builtin_amdgcn_s_barrier();
      compute(a_slot(lds, t), b_slot(lds, t), t & 1, acc);
    }
  }

  // num_steps: with APAIR an even count (reduction_fits).
  template <class Src>
  __device__ __forceinline__ static void run(uint8_t* lds, const Src& src, int num_steps, Acc& acc) {
#pragma unroll
    for (int jn = 0; jn < Cfg::TN; ++jn)
#pragma unroll
      for (int i = 0; i < Cfg::TM; ++i)
#pragma unroll
        for (int v = 0; v < 16; ++v) acc[jn][i][v] = 0.0f;
    if (num_steps <= 0) return;
    if constexpr (Cfg::PIPE == 5) {
      if constexpr (Cfg::APAIR) run_paired_xs(lds, src, num_steps, acc);
      else if constexpr (Cfg::SPLIT) run_split_xs(lds, src, num_steps, acc);
      else run_xs(lds, src, num_steps, acc);
      return;
    }
    if constexpr (Cfg::APAIR) {
      run_paired(lds, src, num_steps, acc);
      return;
    }
    issue_b_first(step_dma(lds, 0, src));
#pragma unroll
    for (int s = 1; s < Cfg::STAGES - 1; ++s)
      if (s < num_steps) issue_all(step_dma(lds, s, src));
    if constexpr (Cfg::PIPE == 3 || Cfg::PIPE == 4) {
      // Steps that issue a later step's loads, among their MFMAs; at the top
      // of each, the loads of steps t .. t+STAGES-2 have been issued.
      int t = 0;
      for (; t + Cfg::STAGES - 1 < num_steps; ++t) {
        wait_vmcnt<Cfg::kLaterLoads>();
        __builtin_amdgcn_s_barrier();
        compute(a_slot(lds, t), b_slot(lds, t), 0, acc, step_dma(lds, t + Cfg::STAGES - 1, src));
      }
      // The last STAGES-1 steps issue nothing.
      for (; t < num_steps; ++t) {
        wait_steps<Cfg::kLoadsPerStep, Cfg::STAGES - 2>(num_steps - 1 - t);
        __builtin_amdgcn_s_barrier();
        compute(a_slot(lds, t), b_slot(lds, t), 0, acc);
      }
      return;
    }
    for (int t = 0; t < num_steps; ++t) {
      // Step t's loads are complete once at most the later issued steps
      // (t+1 .. t+STAGES-2, if they exist) are outstanding.
      wait_steps<Cfg::kLoadsPerStep, Cfg::STAGES - 2>(min(num_steps - 1 - t, Cfg::STAGES - 2));
      // Every wave's step-t data is in LDS, and every wave is done with
      // step t-1's stage, which the next issue overwrites.
      __builtin_amdgcn_s_barrier();
      if (t + Cfg::STAGES - 1 < num_steps) issue_all(step_dma(lds, t + Cfg::STAGES - 1, src));
      compute(a_slot(lds, t), b_slot(lds, t), 0, acc);
    }
  }

  // Epilogue through LDS. A lane's results are 4 consecutive columns of 32
  // different rows, so storing them straight to memory writes each cache
  // line in 16-byte pieces. Instead the tile is written to LDS as bf16,
  // rows of BN*2 bytes, 16-byte chunk c of row r at chunk c ^ (r & 15)
  // (the 32 rows of one store spread over 16 bank groups), and read back
  // one 16-byte chunk per lane in row order: each wave instruction then
  // stores whole row segments. The ring is free once the last step has been
  // computed; the caller passes its base. fn(v) maps an fp32 result
  // (activation, or identity) before rounding to bf16.
  static constexpr int kStagedBytes = Cfg::kStagedPartBytes;
  static_assert(kStagedBytes <= Cfg::kLdsAlloc, "staged tile fits the kernel's LDS");
  static constexpr int kPartGroups = Cfg::TM / Cfg::EPI_PARTS;  // 32-row groups per part (WM == 1 when split)
  static constexpr int kPartRows = Cfg::BM / Cfg::EPI_PARTS;
  static_assert(Cfg::BN >= 128, "16 chunks per row at least");

  __device__ __forceinline__ static int staged_offset(int r, int chunk) {
    return r * (Cfg::BN * 2) + ((chunk ^ (r & 15)) << 4);
  }

  template <class Fn>
  __device__ __forceinline__ static void stage_tile(uint8_t* __restrict__ lds, Acc& acc, Fn fn) {
    static_assert(Cfg::EPI_PARTS == 1, "split epilogue: stage_part");
    stage_part<0>(lds, acc, fn);
  }

  // Part P of the tile: its row groups P * kPartGroups .. +kPartGroups,
  // staged as rows 0 .. kPartRows of LDS.
  template <int P, class Fn>
  __device__ __forceinline__ static void stage_part(uint8_t* __restrict__ lds, Acc& acc, Fn fn) {
    __syncthreads();  // every wave is done reading the ring (or the previous part)
#pragma unroll
    for (int jn = 0; jn < Cfg::TN; ++jn)
#pragma unroll
      for (int i = P * kPartGroups; i < (P + 1) * kPartGroups; ++i) {
        const int m = out_row(i) - P * kPartRows;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int n = out_col(jn, g);
          float v[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = fn(acc[jn][i][4 * g + e]);
          *reinterpret_cast<u32x2_t*>(lds + staged_offset(m, n >> 3) + (n & 7) * 2) =
              u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
        }
      }
    __syncthreads();
  }

  // fn(r, col, chunk16): every 16-byte chunk of the staged tile, row by row
  // (col = first of its 8 columns), consecutive lanes on consecutive chunks.
  template <class Fn>
  __device__ __forceinline__ static void for_each_staged_chunk(const uint8_t* __restrict__ lds, Fn fn) {
    constexpr int kChunksPerRow = Cfg::BN / 8;
    constexpr int kChunks = kPartRows * kChunksPerRow;
    static_assert(kChunks % Cfg::kThreads == 0, "whole passes");
#pragma unroll
    for (int q0 = 0; q0 < kChunks; q0 += Cfg::kThreads) {
      const int q = q0 + static_cast<int>(threadIdx.x);
      const int r = q / kChunksPerRow, c = q % kChunksPerRow;
      fn(r, c * 8, *reinterpret_cast<const u32x4_t*>(lds + staged_offset(r, c)));
    }
  }

  // Output coordinates of acc[jn][i][v] for this lane: the MFMA computed C^T,
  // so lane % 32 is the C row and v selects the column:
  //   m = wm*WTM + 32 i + lane % 32
  //   n = wn*WTN + 32 jn + 8 (v / 4) + 4 (lane / 32) + v % 4
  // Values v = 4g .. 4g+3 are four consecutive columns.
  __device__ __forceinline__ static int out_row(int i) {
    const int lane = threadIdx.x & 63, wm = (threadIdx.x >> 6) / Cfg::WN;
    return wm * Cfg::WTM + 32 * i + (lane & 31);
  }
  __device__ __forceinline__ static int out_col(int jn, int g) {
    const int lane = threadIdx.x & 63, wn = (threadIdx.x >> 6) % Cfg::WN;
    return wn * Cfg::WTN + 32 * jn + 8 * g + 4 * (lane >> 5);
  }
};

}  // namespace sb
