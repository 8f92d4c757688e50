// Process-wide pieces of libmkq: error strings and cached device properties.
#include <stdio.h>
#include <string.h>

#include "mkq_host.h"

namespace mkq {

namespace {
thread_local char g_last_error[512] = {0};
constexpr int kMaxDevices = 64;
int g_cu_count[kMaxDevices] = {0};
int g_max_lds[kMaxDevices] = {0};
}  // namespace

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_last_error[0] = 0; }

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  return dev;
}

int cu_count() {
  int dev = current_device();
  if (dev < 0 || dev >= kMaxDevices) return 256;
  if (g_cu_count[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    g_cu_count[dev] = n;
  }
  return g_cu_count[dev];
}

int max_lds_per_block() {
  int dev = current_device();
  if (dev < 0 || dev >= kMaxDevices) return 65536;
  if (g_max_lds[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess || n <= 0)
      n = 65536;
    g_max_lds[dev] = n;
  }
  return g_max_lds[dev];
}

}  // namespace mkq

extern "C" const char* mkq_last_error(void) { return mkq::g_last_error; }

extern "C" int mkq_abi_version(void) { return 100; }
