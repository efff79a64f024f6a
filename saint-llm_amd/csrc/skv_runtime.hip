// Error state and version query of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include "skv_common.h"

namespace skv {

static thread_local char g_last_error[512] = "";

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    return set_error(SKV_EHIP, "%s: HIP launch failed: %s", what, hipGetErrorString(e));
  }
  return SKV_OK;
}

namespace {

// Per device, read once: compute units and XCDs (XCCs).  A device whose
// query fails counts as one XCD of 256 compute units; an XCD count that is
// not a power of two counts as one (placement then ignores the XCDs, and
// kernels place blocks with shifts and masks).
struct Topology {
  int cus = 0;
  int xcds = 0;
};

Topology topology() {
  static Topology topo[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    return Topology{256, 1};
  }
  Topology& t = topo[dev];
  if (t.cus <= 0) {
    int cus = 0, xcds = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) {
      (void)hipGetLastError();
      cus = 256;
    }
    if (hipDeviceGetAttribute(&xcds, hipDeviceAttributeNumberOfXccs, dev) != hipSuccess || xcds <= 0) {
      (void)hipGetLastError();
      xcds = 1;
    }
    if (xcds & (xcds - 1)) xcds = 1;
    t.xcds = xcds;
    t.cus = cus;
  }
  return t;
}

}  // namespace

int device_cus() { return topology().cus; }

int device_xcds() { return topology().xcds; }

}  // namespace skv

extern "C" int skv_abi_version(void) { return SKV_ABI_VERSION; }

extern "C" const char* skv_last_error(void) { return skv::g_last_error; }
