// grm_common.hip -- error plumbing and runtime description shared by the
// MLA and GQA halves of libgrm_hip_router.so.
#include "grm_common.hpp"

#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <atomic>

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

void host_topk_merge(const Cand* in, size_t count, int k, Cand* out) {
  int n = 0;
  for (size_t i = 0; i < count; ++i) {
    const Cand& c = in[i];
    if (!isfinite(c.score) || c.id == kNoId) continue;
    if (n == k && !better(c.score, c.id, out[k - 1].score, out[k - 1].id)) continue;
    int pos = n < k ? n : k - 1;
    while (pos > 0 && better(c.score, c.id, out[pos - 1].score, out[pos - 1].id)) {
      out[pos] = out[pos - 1];
      --pos;
    }
    out[pos] = c;
    if (n < k) ++n;
  }
  for (int j = n; j < k; ++j) {
    out[j].score = __builtin_nanf("");
    out[j].slot = kNoSlot;
    out[j].id = kNoId;
  }
}

int reserve_mapped(MappedCands* m, size_t count) {
  if (count <= m->count && m->host) return 0;
  release_mapped(m);
  void* h = nullptr;
  GRM_HIP_CHECK(hipHostMalloc(&h, count * sizeof(Cand),
                              hipHostMallocMapped | hipHostMallocCoherent));
  void* d = nullptr;
  hipError_t rc = hipHostGetDevicePointer(&d, h, 0);
  if (rc != hipSuccess) {
    (void)hipHostFree(h);
    return fail_hip(rc, "hipHostGetDevicePointer");
  }
  m->host = static_cast<Cand*>(h);
  m->dev = static_cast<Cand*>(d);
  m->count = count;
  return 0;
}

bool blocking_sync() {
  static const bool blocking = [] {
    const char* env = getenv("GRM_HIP_BLOCKING_SYNC");
    return env && env[0] == '1';
  }();
  return blocking;
}

int wait_event(hipEvent_t ev) {
  if (blocking_sync()) {
    GRM_HIP_CHECK(hipEventSynchronize(ev));
    return 0;
  }
  for (;;) {
    const hipError_t e = hipEventQuery(ev);
    if (e == hipSuccess) return 0;
    if (e != hipErrorNotReady) return fail_hip(e, "hipEventQuery");
  }
}

int begin_flags(MappedBuf* buf, size_t max, unsigned* seq) {
  if (buf->bytes < max * sizeof(unsigned)) {
    GRM_CHECK_RC(reserve_mapped_bytes(buf, max * sizeof(unsigned)));
    memset(buf->host, 0, max * sizeof(unsigned));
    *seq = 0;
  }
  if (++*seq == 0) *seq = 1;  // 0 is what a fresh buffer holds
  return 0;
}

int wait_flags(const MappedBuf& buf, unsigned seq, size_t n, hipEvent_t ev) {
  const volatile unsigned* f = static_cast<const volatile unsigned*>(buf.host);
  size_t i = 0;
  for (uint64_t spin = 1;; ++spin) {
    while (i < n && f[i] == seq) ++i;
    if (i == n) break;
    if (spin % 256 == 0) {
      const hipError_t e = hipEventQuery(ev);
      if (e == hipSuccess) {
        while (i < n && f[i] == seq) ++i;
        if (i == n) break;
        return fail(-1, "route finished without its completion flags");
      }
      if (e != hipErrorNotReady) return fail_hip(e, "hipEventQuery");
    }
  }
  std::atomic_thread_fence(std::memory_order_acquire);
  return 0;
}

int wait_tagged(const Cand* entries, size_t n, unsigned seq, hipEvent_t ev) {
  const volatile uint32_t* tags = reinterpret_cast<const volatile uint32_t*>(entries);
  const uint32_t tag = route_tag(seq);
  // the slot field is the second word of each 16-byte entry
  for (size_t i = 0; i < n; ++i) {
    for (uint64_t spin = 1; tags[4 * i + 1] != tag; ++spin) {
      if (spin % 256 == 0) {
        const hipError_t e = hipEventQuery(ev);
        if (e == hipSuccess) {
          if (tags[4 * i + 1] == tag) break;
          return fail(-1, "route finished without its list entries");
        }
        if (e != hipErrorNotReady) return fail_hip(e, "hipEventQuery");
      }
    }
  }
  std::atomic_thread_fence(std::memory_order_acquire);
  return 0;
}

constexpr size_t kStampHead = 2;  // start tick, route number

int reserve_stamps(MappedBuf* buf, size_t max) {
  const size_t bytes = (kStampHead + max) * sizeof(unsigned long long);
  if (buf->bytes < bytes) {
    GRM_CHECK_RC(reserve_mapped_bytes(buf, bytes));
    memset(buf->host, 0, bytes);
  }
  return 0;
}

RouteStamps route_stamps(const MappedBuf& buf, size_t first) {
  unsigned long long* d = static_cast<unsigned long long*>(buf.dev);
  return RouteStamps{d, d + kStampHead + first};
}

int stamps_elapsed(const MappedBuf& buf, unsigned seq, size_t first, size_t n, hipEvent_t ev,
                   double ticks_per_ms, float* ms) {
  const volatile unsigned long long* st = static_cast<const volatile unsigned long long*>(buf.host);
  if (st[1] != seq) {
    GRM_CHECK_RC(wait_event(ev));
    if (st[1] != seq) return fail(-1, "route finished without its start stamp");
  }
  std::atomic_thread_fence(std::memory_order_acquire);
  const unsigned long long t0 = st[0];
  unsigned long long t1 = t0;
  // A timed block's end tick below t0 is an earlier route's (the stream
  // ran those kernels before this route's first timed one started); it is
  // replaced before the route's event completes.
  bool stale = false;
  for (size_t i = first; i < n; ++i) stale |= st[kStampHead + i] < t0;
  if (stale) {
    GRM_CHECK_RC(wait_event(ev));
    std::atomic_thread_fence(std::memory_order_acquire);
  }
  for (size_t i = first; i < n; ++i) {
    const unsigned long long e = st[kStampHead + i];
    if (e < t0) return fail(-1, "route finished without its end stamps");
    if (e > t1) t1 = e;
  }
  *ms = static_cast<float>(static_cast<double>(t1 - t0) / ticks_per_ms);
  return 0;
}

bool event_timing() {
  const char* env = getenv("GRM_HIP_ROUTE_TIMING");
  return env && strcmp(env, "events") == 0;
}

double wall_ticks_per_ms(int device) {
  int khz = 0;
  if (hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device) != hipSuccess) {
    (void)hipGetLastError();
    return 0.0;
  }
  return khz > 0 ? static_cast<double>(khz) : 0.0;
}

int reserve_mapped_bytes(MappedBuf* m, size_t bytes) {
  if (bytes <= m->bytes && m->host) return 0;
  release_mapped_bytes(m);
  void* h = nullptr;
  GRM_HIP_CHECK(hipHostMalloc(&h, bytes ? bytes : 1,
                              hipHostMallocMapped | hipHostMallocCoherent));
  void* d = nullptr;
  hipError_t rc = hipHostGetDevicePointer(&d, h, 0);
  if (rc != hipSuccess) {
    (void)hipHostFree(h);
    return fail_hip(rc, "hipHostGetDevicePointer");
  }
  m->host = h;
  m->dev = d;
  m->bytes = bytes;
  return 0;
}

void release_mapped_bytes(MappedBuf* m) {
  if (m->host) (void)hipHostFree(m->host);
  m->host = nullptr;
  m->dev = nullptr;
  m->bytes = 0;
}

void release_mapped(MappedCands* m) {
  if (m->host) (void)hipHostFree(m->host);
  m->host = nullptr;
  m->dev = nullptr;
  m->count = 0;
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

// dst[i] = src[i] for the 16-byte words [0, n16) and the tail bytes
// [16 * n16, bytes), grid-stride.
__global__ __launch_bounds__(256) void fetch_kernel(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                                    size_t n16, size_t bytes) {
  const size_t stride = static_cast<size_t>(gridDim.x) * blockDim.x;
  for (size_t i = static_cast<size_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n16; i += stride) {
    dst[i] = src[i];
  }
  if (blockIdx.x == 0 && threadIdx.x < bytes - n16 * 16) {
    reinterpret_cast<unsigned char*>(dst)[n16 * 16 + threadIdx.x] =
        reinterpret_cast<const unsigned char*>(src)[n16 * 16 + threadIdx.x];
  }
}

int fetch_async(void* dst, const void* src_mapped, size_t bytes, hipStream_t stream) {
  if (bytes == 0) return 0;
  const size_t n16 = bytes / 16;
  const unsigned blocks = static_cast<unsigned>(std::max<size_t>(1, std::min<size_t>((n16 + 255) / 256, 1024)));
  fetch_kernel<<<blocks, 256, 0, stream>>>(static_cast<uint4*>(dst), static_cast<const uint4*>(src_mapped), n16,
                                           bytes);
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
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
