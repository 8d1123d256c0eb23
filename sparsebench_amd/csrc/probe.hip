// arch_probe (the reference's csrc/smoke.cu), the library's error state and
// its test hooks.

#include <atomic>

#include "common.hpp"

namespace sb {

std::string& last_error() {
  thread_local std::string msg;
  return msg;
}

namespace {
std::atomic<int32_t> g_test_hooks[SB_NUM_TEST_HOOKS];
}  // namespace

int32_t test_hook(int32_t hook) {
  return hook >= 0 && hook < SB_NUM_TEST_HOOKS ? g_test_hooks[hook].load(std::memory_order_relaxed) : 0;
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

extern "C" int sb_set_test_hook(int32_t hook, int32_t value) {
  if (hook < 0 || hook >= SB_NUM_TEST_HOOKS) return fail(SB_ERR_INVALID, "unknown test hook %d", hook);
  g_test_hooks[hook].store(value, std::memory_order_relaxed);
  return clear_ok();
}

extern "C" int sb_arch_probe(int32_t* out, int64_t n, void* stream) {
  if (n <= 0) return fail(SB_ERR_INVALID, "arch_probe: n must be positive, got %lld", static_cast<long long>(n));
  const int64_t groups = (n + 255) / 256;
  if (groups > 2147483647LL) return fail(SB_ERR_INVALID, "arch_probe: n too large for a 1D grid");
  if (!out) return fail(SB_ERR_INVALID, "arch_probe: null buffer");
  arch_probe_kernel<<<static_cast<uint32_t>(groups), 256, 0, as_stream(stream)>>>(out, n);
  if (int rc = check_launch("arch_probe")) return rc;
  return clear_ok();
}
