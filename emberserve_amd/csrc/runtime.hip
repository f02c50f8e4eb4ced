// Library-wide entry points: ABI version, status strings and the per-device error word
// that index-checking kernels set (see ember_read_errors in include/ember_ops.h).
#include <atomic>

#include "ember_common.h"

namespace {

// One word per device; kernels OR EMBER_ERR_* bits into it with a vector atomic.
__device__ uint32_t g_error_word = 0;

constexpr int kMaxDevices = 64;
std::atomic<uint32_t*> g_error_word_addr[kMaxDevices];

}  // namespace

namespace ember {

__host__ uint32_t* device_error_word() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  uint32_t* p = g_error_word_addr[dev].load(std::memory_order_acquire);
  if (p != nullptr) return p;
  void* addr = nullptr;
  // The host-side name of a __device__ variable is not a device address: resolve it once
  // per device, with that device current.
  if (hipGetSymbolAddress(&addr, HIP_SYMBOL(g_error_word)) != hipSuccess) return nullptr;
  p = static_cast<uint32_t*>(addr);
  g_error_word_addr[dev].store(p, std::memory_order_release);
  return p;
}

__host__ int device_cu_count() {
  static std::atomic<int> cached[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) return 0;
  cached[dev].store(n, std::memory_order_relaxed);
  return n;
}

}  // namespace ember

extern "C" {

int ember_abi_version(void) { return 16; }

const char* ember_status_string(int status) {
  switch (status) {
    case EMBER_OK: return "ok";
    case EMBER_EINVAL: return "invalid argument (shape, stride, dtype or pointer)";
    case EMBER_EALIGN: return "misaligned operand";
    case EMBER_ELAUNCH: return "kernel launch failed";
    case EMBER_ENODEV: return "no HIP device or HIP runtime call failed";
    case EMBER_ETOOBIG: return "the call needs more scratch than the no-allocation entry point holds";
    default: return "unknown status";
  }
}

int ember_read_errors(uint32_t* flags, int clear) {
  uint32_t* p = ember::device_error_word();
  if (p == nullptr) return EMBER_ENODEV;
  if (hipDeviceSynchronize() != hipSuccess) return EMBER_ENODEV;
  uint32_t v = 0;
  if (hipMemcpy(&v, p, sizeof(v), hipMemcpyDeviceToHost) != hipSuccess) return EMBER_ENODEV;
  if (flags != nullptr) *flags = v;
  if (clear) {
    const uint32_t zero = 0;
    if (hipMemcpy(p, &zero, sizeof(zero), hipMemcpyHostToDevice) != hipSuccess) return EMBER_ENODEV;
  }
  return EMBER_OK;
}

}  // extern "C"
