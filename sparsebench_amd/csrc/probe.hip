// arch_probe (the reference's csrc/smoke.cu) and the library's error state.

#include "common.hpp"

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
