// grm_common.hip -- error plumbing and runtime description shared by the
// MLA and GQA halves of libgrm_hip_router.so.
#include "grm_common.hpp"

#include <stdio.h>
#include <string.h>

namespace grm {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }
void clear_error() { g_last_error.clear(); }

int fail(int code, const char* what) {
  g_last_error = what ? what : "";
  return code;
}

int fail_hip(hipError_t rc, const char* what) {
  std::string msg = what ? what : "hip call";
  msg += ": ";
  msg += hipGetErrorString(rc);
  g_last_error = msg;
  return hip_code(rc);
}

}  // namespace grm

extern "C" const char* grm_hip_last_error(void) {
  return grm::g_last_error.c_str();
}

extern "C" int grm_hip_runtime_info(char* out, size_t out_cap) {
  if (!out || out_cap == 0) return grm::fail(-1, "null output buffer");
  int dev = 0;
  hipDeviceProp_t prop;
  hipError_t rc = hipGetDevice(&dev);
  if (rc == hipSuccess) rc = hipGetDeviceProperties(&prop, dev);
  int n = 0;
  if (rc != hipSuccess) {
    n = snprintf(out, out_cap,
                 "{\"library\":\"grm_hip_router\",\"device\":null,"
                 "\"error\":\"%s\"}",
                 hipGetErrorString(rc));
  } else {
    n = snprintf(out, out_cap,
                 "{\"library\":\"grm_hip_router\",\"device\":%d,"
                 "\"name\":\"%s\",\"arch\":\"%s\",\"compute_units\":%d,"
                 "\"hbm_bytes\":%zu,\"clock_khz\":%d}",
                 dev, prop.name, prop.gcnArchName, prop.multiProcessorCount,
                 static_cast<size_t>(prop.totalGlobalMem), prop.clockRate);
  }
  return (n < 0 || static_cast<size_t>(n) >= out_cap) ? grm::fail(-1, "buffer too small") : 0;
}
