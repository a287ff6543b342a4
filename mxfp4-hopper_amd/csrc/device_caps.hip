// Per-device launch parameters, queried once per device id and cached.
#include <atomic>

#include "omo_internal.h"

namespace omo_hip {

namespace {

constexpr int kMaxDevices = 64;
// 0 = not queried yet; a racing first query on two host threads writes the
// same values.
std::atomic<int> g_cus[kMaxDevices];
std::atomic<int> g_lds[kMaxDevices];

}  // namespace

DeviceCaps current_device_caps() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return DeviceCaps{256, 65536};
  int cus = g_cus[dev].load(std::memory_order_acquire);  // pairs with the release store below
  int lds = g_lds[dev].load(std::memory_order_relaxed);
  if (cus == 0) {
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || lds <= 0)
      lds = 65536;
    g_lds[dev].store(lds, std::memory_order_relaxed);
    g_cus[dev].store(cus, std::memory_order_release);
  }
  return DeviceCaps{cus, lds};
}

}  // namespace omo_hip
