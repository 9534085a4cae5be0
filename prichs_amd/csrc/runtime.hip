// runtime.hip -- error reporting and device queries of libprichs_hip.so.
#include <cstdarg>
#include <mutex>

#include "common.hpp"

namespace prichs {

namespace {
thread_local char g_last_error[512] = {0};

void vset(const char *fmt, va_list ap) { vsnprintf(g_last_error, sizeof g_last_error, fmt, ap); }
}  // namespace

void set_error(const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vset(fmt, ap);
  va_end(ap);
}

int fail(int code, const char *fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vset(fmt, ap);
  va_end(ap);
  return code;
}

int device_cu_count() {
  static std::mutex mu;
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0) return -1;
  std::lock_guard<std::mutex> lock(mu);
  if (dev < 64 && cache[dev] > 0) return cache[dev];
  int n = 0;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return -1;
  if (dev < 64) cache[dev] = n;
  return n;
}

}  // namespace prichs

extern "C" const char *prichs_last_error(void) { return prichs::g_last_error; }

extern "C" void prichs_clear_error(void) { prichs::g_last_error[0] = 0; }

extern "C" int prichs_abi_version(void) { return 200; }

// Capabilities of the current device for the roofline (all outputs may be
// NULL): compute units, peak engine clock and memory clock in kHz, memory
// bus width in bits.
extern "C" int prichs_device_caps(int *cus, int *clock_khz, int *mem_clock_khz,
                                  int *mem_bus_bits) {
  int dev = 0;
  PRICHS_HIP_TRY(hipGetDevice(&dev), "device_caps: no HIP device");
  struct Q {
    int *out;
    hipDeviceAttribute_t attr;
  } qs[] = {{cus, hipDeviceAttributeMultiprocessorCount},
            {clock_khz, hipDeviceAttributeClockRate},
            {mem_clock_khz, hipDeviceAttributeMemoryClockRate},
            {mem_bus_bits, hipDeviceAttributeMemoryBusWidth}};
  for (const Q &q : qs)
    if (q.out) PRICHS_HIP_TRY(hipDeviceGetAttribute(q.out, q.attr, dev), "device_caps");
  return PRICHS_OK;
}
