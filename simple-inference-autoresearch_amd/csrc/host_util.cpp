// Host helpers shared by every entry point.
#include "host_util.hpp"

#include <mutex>
#include <string.h>

namespace sia {

namespace {
thread_local char g_msg[512] = "";

struct OccKey {
  const void* k;
  int block;
  size_t lds;
  int dev;
  int occ;
};
std::mutex g_mu;
OccKey g_occ[256];
int g_nocc = 0;
DeviceInfo g_dev[64];
}  // namespace

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_msg, sizeof(g_msg), fmt, ap);
  va_end(ap);
  return code;
}

const char* last_message() { return g_msg; }

const DeviceInfo& device_info() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    static DeviceInfo none;
    return none;
  }
  std::lock_guard<std::mutex> lock(g_mu);
  DeviceInfo& d = g_dev[dev];
  if (d.id != dev) {
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) == hipSuccess) {
      d.cus = prop.multiProcessorCount;
      d.gfx950 = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
      d.id = dev;
    }
  }
  return d;
}

int kernel_occupancy(const void* kernel, int block, size_t lds) {
  int dev = 0;
  (void)hipGetDevice(&dev);
  {
    std::lock_guard<std::mutex> lock(g_mu);
    for (int i = 0; i < g_nocc; ++i)
      if (g_occ[i].k == kernel && g_occ[i].block == block && g_occ[i].lds == lds && g_occ[i].dev == dev)
        return g_occ[i].occ;
  }
  if (lds > 65536) {
    if (hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
      return 0;
  }
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, block, lds) != hipSuccess) return 0;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_nocc < 256) g_occ[g_nocc++] = OccKey{kernel, block, lds, dev, n};
  return n;
}

}  // namespace sia
