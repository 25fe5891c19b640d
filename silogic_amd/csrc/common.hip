// Error state and device queries shared by every entry point.
#include <stdarg.h>

#include <mutex>

#include "slg_common.h"

namespace slg {

static thread_local std::string g_last_error;

void set_error(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
}

namespace {
constexpr int kMaxDevices = 64;
int g_cus[kMaxDevices];
int g_lds[kMaxDevices];
std::once_flag g_once[kMaxDevices];

void query(int dev) {
  int v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) v = 256;
  g_cus[dev] = v;
  v = 0;
  if (hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
    v = 65536;
  g_lds[dev] = v;
}

int current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
  std::call_once(g_once[dev], query, dev);
  return dev;
}
}  // namespace

int device_cus() { return g_cus[current_device()]; }
int device_lds_bytes() { return g_lds[current_device()]; }

}  // namespace slg

extern "C" {

const char* slg_last_error(void) { return slg::g_last_error.c_str(); }

int slg_version(void) { return 1; }

int slg_device_cus(void) { return slg::device_cus(); }

}  // extern "C"
