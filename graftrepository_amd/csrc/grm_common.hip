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

// Merge `count` candidates per query (query q reads in + q*in_stride) into
// out + q*k; one block per query.  Clears flags[q] when flags is given.
__global__ __launch_bounds__(kMergeWaves * kWave) void topk_merge_kernel(
    const Cand* __restrict__ in, uint32_t count, size_t in_stride, int k,
    Cand* __restrict__ out, unsigned* __restrict__ flags) {
  __shared__ Cand s_lists[kMergeWaves][kMaxTopK];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const Cand* src = in + blockIdx.x * in_stride;
  WaveList G;
  wl_init(G);
  wl_consume_global(G, k, src, count, static_cast<uint32_t>(wave), kMergeWaves);
  if (lane < kMaxTopK) s_lists[wave][lane] = wl_entry(G);
  __syncthreads();
  if (wave == 0) {
    WaveList B;
    block_merge<kMergeWaves>(s_lists, k, B);
    if (lane < k) out[static_cast<size_t>(blockIdx.x) * k + lane] = wl_entry(B);
    if (lane == 0 && flags) flags[blockIdx.x] = 0u;
  }
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
