// arch_probe (the reference's csrc/smoke.cu), the read-bandwidth probes and
// the library's error state.

#include "common.hpp"
#include "gemm_dma.hpp"

namespace sb {

std::string& last_error() {
  thread_local std::string msg;
  return msg;
}

int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return code;
}

namespace {

// The number comes from the target the code object was compiled for, so a
// fallback path (another architecture, an interpreter) cannot produce it.
__global__ void arch_probe_kernel(int32_t* __restrict__ out, int64_t n) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) {
#if defined(__gfx950__)
    out[i] = 950;
#else
    out[i] = -1;
#endif
  }
}

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

}  // namespace
}  // namespace sb

using namespace sb;

extern "C" const char* sb_last_error(void) { return last_error().c_str(); }

extern "C" int32_t sb_version(void) { return 1; }

extern "C" int sb_arch_probe(int32_t* out, int64_t n, void* stream) {
  if (n <= 0) return fail(SB_ERR_INVALID, "arch_probe: n must be positive, got %lld", static_cast<long long>(n));
  const int64_t groups = (n + 255) / 256;
  if (groups > 2147483647LL) return fail(SB_ERR_INVALID, "arch_probe: n too large for a 1D grid");
  if (!out) return fail(SB_ERR_INVALID, "arch_probe: null buffer");
  arch_probe_kernel<<<static_cast<uint32_t>(groups), 256, 0, as_stream(stream)>>>(out, n);
  if (int rc = check_launch("arch_probe")) return rc;
  return clear_ok();
}

extern "C" int sb_read_probe(const void* data, int64_t bytes, int32_t mode, uint32_t key, uint32_t* sink,
                             void* stream) {
  if (!data || !sink) return fail(SB_ERR_INVALID, "read_probe: null buffer");
  if (!aligned16(data)) return fail(SB_ERR_INVALID, "read_probe: data must be 16-byte aligned");
  const hipStream_t s = as_stream(stream);
  if (mode == 0) {
    if (bytes <= 0 || bytes % 16 != 0) return fail(SB_ERR_INVALID, "read_probe: bytes must be a positive multiple of 16");
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
      return fail(SB_ERR_HIP, "read_probe: no CU count");
    read_vec_kernel<<<static_cast<uint32_t>(cus) * 8, kProbeThreads, 0, s>>>(static_cast<const u32x4_t*>(data),
                                                                                 bytes / 16, key, sink);
  } else if (mode == 1) {
    constexpr int64_t kChunk = 1 << 20;  // 32 stages per workgroup
    if (bytes <= 0 || bytes % kChunk != 0) return fail(SB_ERR_INVALID, "read_probe: DMA mode reads whole MiB");
    if (bytes / kChunk > 2147483647LL) return fail(SB_ERR_INVALID, "read_probe: too many chunks");
    read_dma_kernel<<<static_cast<uint32_t>(bytes / kChunk), kProbeThreads, 0, s>>>(
        static_cast<const uint8_t*>(data), static_cast<uint32_t>(kChunk), key, sink);
  } else {
    return fail(SB_ERR_INVALID, "read_probe: mode must be 0 (vector loads) or 1 (LDS DMA), got %d", mode);
  }
  if (int rc = check_launch("read_probe")) return rc;
  return clear_ok();
}
