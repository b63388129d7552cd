// Host-side error channel and version of libquantpack_hip.so.
#include "qp_common.h"

namespace qp {

static thread_local std::string g_last_error;

void set_error(const std::string &msg) { g_last_error = msg; }

int fail(int code, const std::string &msg) {
  g_last_error = msg;
  return code;
}

// Status of the launch just issued on this thread: 0 or the hipError_t it raised.
int launch_status() {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    g_last_error = std::string("kernel launch failed: ") + hipGetErrorString(e);
    return (int)e;
  }
  return QP_OK;
}

// Compute units of the current device (cached per device).
int device_cus() {
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (!cached[dev]) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

}  // namespace qp

extern "C" const char *qp_last_error(void) { return qp::g_last_error.c_str(); }

extern "C" const char *qp_version(void) { return "quantpack-hip 0.1.0 gfx950"; }
