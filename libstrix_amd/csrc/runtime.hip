// SPDX-License-Identifier: MIT
// Error slot, arch gate and version query of the C ABI.
//
// The reference reports failures as c10::Error from TORCH_CHECK
// (csrc/gemm/w8a8_wmma_gemm.hip:803-860) and gates on the device arch once
// per process (csrc/gemm/w8a8_wmma_gemm.hip:757-763). Here every entry point
// returns a status code and keeps the message in a per-thread slot that the
// host layer turns into a RuntimeError with the same text.
#include <string.h>

#include <atomic>

#include "capi_internal.h"

namespace strix {

static thread_local char g_err[1024] = {0};

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

// Per-device facts, computed once (devices never change): arch verdict
// (0 unknown, 1 gfx950, 2 other) and compute-unit count.
static std::atomic<int> g_arch[64];
static std::atomic<int> g_cus[64];

static int query_device(int dev) {
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, dev) != hipSuccess)
    return set_error(STRIX_ERR_DEVICE, "libstrix_amd: cannot query device %d", dev);
  g_cus[dev].store(prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 1, std::memory_order_relaxed);
  g_arch[dev].store(strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 2, std::memory_order_release);
  return STRIX_OK;
}

int check_arch() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess)
    return set_error(STRIX_ERR_DEVICE, "libstrix_amd: no HIP device available");
  if (dev < 0 || dev >= 64)
    return set_error(STRIX_ERR_DEVICE, "libstrix_amd: device index %d out of range", dev);
  if (g_arch[dev].load(std::memory_order_acquire) == 0) {
    int rc = query_device(dev);
    if (rc != STRIX_OK) return rc;
  }
  if (g_arch[dev].load(std::memory_order_acquire) != 1)
    return set_error(STRIX_ERR_DEVICE,
                     "libstrix_amd targets gfx950 (MI355X, wave64 MFMA) GPUs only");
  return STRIX_OK;
}

int cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (g_arch[dev].load(std::memory_order_acquire) == 0 && query_device(dev) != STRIX_OK) return 256;
  return g_cus[dev].load(std::memory_order_relaxed);
}

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(STRIX_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return STRIX_OK;
}

}  // namespace strix

extern "C" {

const char* strix_last_error(void) { return strix::g_err; }

int strix_abi_version(void) { return STRIX_ABI_VERSION; }

}  // extern "C"
