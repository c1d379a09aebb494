// Status codes, error text and the thread-local record of the last failed HIP call.
#include <hip/hip_runtime.h>

#include <atomic>

#include "q4llm.h"

namespace q4 {

static thread_local int g_last_hip_error = 0;

int hip_fail(hipError_t e) {
  g_last_hip_error = static_cast<int>(e);
  return Q4_ERR_HIP;
}

}  // namespace q4

extern "C" const char* q4llm_status_string(int status) {
  switch (status) {
    case Q4_OK: return "ok";
    case Q4_ERR_NULL: return "a required pointer is NULL";
    case Q4_ERR_SHAPE: return "sizes violate the documented shape rules";
    case Q4_ERR_ALIGN: return "a pointer is not aligned as documented";
    case Q4_ERR_DTYPE: return "unknown or unsupported dtype code";
    case Q4_ERR_WORKSPACE: return "workspace missing or too small";
    case Q4_ERR_RANGE: return "position, bucket or length out of range";
    case Q4_ERR_UNSUPPORTED: return "request outside this build's documented limits";
    case Q4_ERR_HIP: return "HIP runtime error (see q4llm_last_hip_error)";
    default: return "unknown status";
  }
}

extern "C" int q4llm_last_hip_error(void) { return q4::g_last_hip_error; }

extern "C" int q4llm_abi_version(void) { return 2; }

// Kernel-choice overrides (tests and sweeps): one atomic per key, read by the launch paths with a
// relaxed load (q4::debug_override in q4_internal.h). Each holds value ^ Q4_DBG_UNSET, so the
// zero-initialised store reads as "unset" from before any constructor runs.
namespace q4 {
std::atomic<int> g_debug[Q4_DBG_COUNT] = {};
}  // namespace q4

extern "C" int q4_debug_override(int key, int value) {
  if (key < 0 || key >= Q4_DBG_COUNT) return Q4_ERR_RANGE;
  q4::g_debug[key].store(value ^ Q4_DBG_UNSET, std::memory_order_relaxed);
  return Q4_OK;
}

extern "C" int q4_debug_override_get(int key, int* value) {
  if (key < 0 || key >= Q4_DBG_COUNT) return Q4_ERR_RANGE;
  if (!value) return Q4_ERR_NULL;
  *value = q4::g_debug[key].load(std::memory_order_relaxed) ^ Q4_DBG_UNSET;
  return Q4_OK;
}

extern "C" void q4_debug_clear(void) {
  for (auto& v : q4::g_debug) v.store(0, std::memory_order_relaxed);
}
