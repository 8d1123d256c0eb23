// Read-bandwidth probes: a measurement tool beside the library, built into
// libsparsebench_probe.so (not part of libsparsebench_hip.so's C ABI).
// bench_baselines.py uses it for the practical read ceilings of the roofline.
//
//   int sbp_read(data, bytes, mode, key, sink, stream)
//     mode 0: 16-byte vector loads over a grid of 8 workgroups per CU;
//     mode 1: LDS DMA (buffer_load ... lds), the load path of the SDD / DSD
//             main loops, one workgroup per MiB (bytes a multiple of 1 MiB).
//   What is read is folded into one word per lane, stored to sink[0..256)
//   only if it equals key, so no load can be dropped. Returns 0, or 1 for a
//   bad argument and 2 for a failed launch, with sbp_last_error() set.

#include "common.hpp"
#include "gemm_dma.hpp"

namespace sb {
namespace {

// Streaming reads, for the roofline's practical ceilings: how fast this
// device's memory can be read with plain 16-byte vector loads, and through
// LDS DMA (buffer_load ... lds) the way the SDD / DSD main loops read it.
// Each lane folds what it read into one word, stored only when that word
// equals `key` (which the caller picks so that it practically never does),
// so no load can be dropped.
constexpr int kProbeThreads = 256;

__global__ void __launch_bounds__(kProbeThreads)
    read_vec_kernel(const u32x4_t* __restrict__ p, int64_t n16, uint32_t key, uint32_t* __restrict__ sink) {
  constexpr int kUnroll = 4;
  uint32_t acc = 0;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * kProbeThreads * kUnroll;
  for (int64_t base = static_cast<int64_t>(blockIdx.x) * kProbeThreads * kUnroll + threadIdx.x; base < n16;
       base += stride) {
    u32x4_t v[kUnroll];
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) {
      const int64_t i = base + static_cast<int64_t>(u) * kProbeThreads;
      v[u] = i < n16 ? __builtin_nontemporal_load(p + i) : u32x4_t{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int u = 0; u < kUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
  }
  if (acc == key) sink[threadIdx.x] = acc;
}

// One workgroup per chunk of chunk_bytes, through a ring of kDmaStages
// stages of 256 lanes x kDmaLoads x 16 bytes (32 KB), the loads of stage
// s+3 issued before stage s is waited for.
constexpr int kDmaLoads = 8, kDmaStages = 4;
constexpr uint32_t kDmaStage = kProbeThreads * kDmaLoads * 16;

__global__ void __launch_bounds__(kProbeThreads)
    read_dma_kernel(const uint8_t* __restrict__ p, uint32_t chunk_bytes, uint32_t key, uint32_t* __restrict__ sink) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[kDmaStage * kDmaStages];
  const __amdgpu_buffer_rsrc_t rsrc = make_rsrc(p + static_cast<int64_t>(blockIdx.x) * chunk_bytes, chunk_bytes);
  const int steps = static_cast<int>(chunk_bytes / kDmaStage);
  const int wave = threadIdx.x >> 6;
  const uint32_t lane_off = (threadIdx.x & 63) * 16u;
  auto issue = [&](int s) {
    uint8_t* stage = lds + (s % kDmaStages) * kDmaStage;
#pragma unroll
    for (int q = 0; q < kDmaLoads; ++q) {
      const uint32_t row = static_cast<uint32_t>(q * kProbeThreads + wave * 64) * 16u;  // 1 KB per wave instruction
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void_t*)(stage + row), 16, lane_off,
                                               __builtin_amdgcn_readfirstlane(s * kDmaStage + row), 0, 0);
    }
  };
  for (int s = 0; s < kDmaStages - 1 && s < steps; ++s) issue(s);
  uint32_t acc = 0;
  for (int s = 0; s < steps; ++s) {
    if (s + kDmaStages - 1 < steps) {
      issue(s + kDmaStages - 1);
      wait_vmcnt<(kDmaStages - 1) * kDmaLoads>();  // stage s is in; the 3 later ones may be in flight
    } else {
      wait_vmcnt<0>();
    }
    __syncthreads();
    acc ^= *reinterpret_cast<const uint32_t*>(lds + (s % kDmaStages) * kDmaStage + threadIdx.x * 16);
    __syncthreads();  // the stage is free before it is loaded again
  }
  if (acc == key) sink[threadIdx.x] = acc;
}

const char* g_probe_error = "";

int probe_fail(int code, const char* msg) {
  g_probe_error = msg;
  return code;
}

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" const char* sbp_last_error(void) { return g_probe_error; }

extern "C" int sbp_read(const void* data, int64_t bytes, int32_t mode, uint32_t key, uint32_t* sink, void* stream) {
  if (!data || !sink) return probe_fail(1, "read_probe: null buffer");
  if (!aligned16(data)) return probe_fail(1, "read_probe: data must be 16-byte aligned");
  const hipStream_t s = as_stream(stream);
  if (mode == 0) {
    if (bytes <= 0 || bytes % 16 != 0) return probe_fail(1, "read_probe: bytes must be a positive multiple of 16");
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      return probe_fail(2, "read_probe: no CU count");
    read_vec_kernel<<<static_cast<uint32_t>(cus) * 8, kProbeThreads, 0, s>>>(static_cast<const u32x4_t*>(data),
                                                                                 bytes / 16, key, sink);
  } else if (mode == 1) {
    constexpr int64_t kChunk = 1 << 20;  // 32 stages per workgroup
    if (bytes <= 0 || bytes % kChunk != 0) return probe_fail(1, "read_probe: DMA mode reads whole MiB");
    if (bytes / kChunk > 2147483647LL) return probe_fail(1, "read_probe: too many chunks");
    read_dma_kernel<<<static_cast<uint32_t>(bytes / kChunk), kProbeThreads, 0, s>>>(
        static_cast<const uint8_t*>(data), static_cast<uint32_t>(kChunk), key, sink);
  } else {
    return probe_fail(1, "read_probe: mode must be 0 (vector loads) or 1 (LDS DMA)");
  }
  if (hipGetLastError() != hipSuccess) return probe_fail(2, "read_probe: kernel launch failed");
  g_probe_error = "";
  return 0;
}
