// payload.hip -- packed graft payloads unpacked on the device.
//
// A packed tensor (core/graft_quant.py:177-217) is two arrays:
//   * int8 codes [..., groups, group_size];
//   * fp32 scales [..., groups, 1].
// Codes were quantised along the last axis (:93-131).  They unpack as
// fp16(fp32(code) * scale) (:136-144).  The law is the same for every
// storage depth: codes of depth below 8 use a narrower range of the same
// int8 container.
//
// The reference dequantises a packed node payload on the host and uploads
// the fp16 arrays (core/graft_arena.py:3479-3492).  Here the codes and
// scales are what crosses PCIe: 1 + 4/group_size bytes per value instead
// of 2.  A kernel then writes the fp16 values in HBM.  That kernel is
// HBM-bound at 1 + 4/group_size + 2 bytes per value; the scale is read
// once per group, and the writes are the bulk.

#include "grm_common.hpp"

#include <hip/hip_fp16.h>

#include <vector>

namespace grm {
namespace payload {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;

// One value: fp32 product, then fp16 round-to-nearest-even.  The empty asm
// keeps the product a value of its own; without it the compiler fuses the
// multiply and the conversion into v_fma_mixlo_f16, which rounds the exact
// product once and differs from the law when the fp32 rounding crosses an
// fp16 rounding boundary.
__device__ inline uint32_t dq(int code, float scale) {
  float p = static_cast<float>(code) * scale;
  asm volatile("" : "+v"(p));
  const _Float16 h = static_cast<_Float16>(p);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
}

// Two codes (bytes b and b+1 of w) to two packed fp16 values.
__device__ inline uint32_t dq2(uint32_t w, int b, float scale) {
  const int c0 = static_cast<int>(static_cast<int8_t>((w >> (8 * b)) & 0xffu));
  const int c1 = static_cast<int>(static_cast<int8_t>((w >> (8 * b + 8)) & 0xffu));
  return dq(c0, scale) | (dq(c1, scale) << 16);
}

// Eight values per thread per step: an 8-byte code load and a 16-byte
// store, all eight in one group (GS a multiple of 8).  Grid-stride over
// n8 = n / 8 steps.
template <int GS>
__global__ __launch_bounds__(kThreads) void dequant8_kernel(const u32x2* __restrict__ codes,
                                                            const float* __restrict__ scales,
                                                            uint64_t n8, u32x4* __restrict__ out) {
  static_assert(GS % 8 == 0, "eight values per group step");
  constexpr uint64_t kPer = GS / 8;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n8;
       i += stride) {
    const u32x2 c = __builtin_nontemporal_load(codes + i);
    const float s = scales[i / kPer];
    u32x4 o;
    o.x = dq2(c.x, 0, s);
    o.y = dq2(c.x, 2, s);
    o.z = dq2(c.y, 0, s);
    o.w = dq2(c.y, 2, s);
    __builtin_nontemporal_store(o, out + i);
  }
}

// Any group size: one value per thread per step.
__global__ __launch_bounds__(kThreads) void dequant1_kernel(const int8_t* __restrict__ codes,
                                                            const float* __restrict__ scales,
                                                            uint64_t n, uint64_t group_size,
                                                            uint16_t* __restrict__ out) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kThreads;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * kThreads + threadIdx.x; i < n;
       i += stride) {
    out[i] = static_cast<uint16_t>(dq(codes[i], scales[i / group_size]));
  }
}

// Library-owned stream and staging per device (default priority; they live
// until the process ends).
struct DeviceCtx {
  hipStream_t stream = nullptr;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
  unsigned char* stage = nullptr;
  size_t stage_bytes = 0;
  int cus = 0;
};

std::vector<DeviceCtx>& contexts() {
  static std::vector<DeviceCtx> ctx;
  return ctx;
}

int device_ctx(DeviceCtx** out) {
  int dev = 0;
  GRM_HIP_CHECK(hipGetDevice(&dev));
  auto& all = contexts();
  if (static_cast<size_t>(dev) >= all.size()) all.resize(static_cast<size_t>(dev) + 1);
  DeviceCtx& c = all[static_cast<size_t>(dev)];
  if (!c.stream) {
    GRM_HIP_CHECK(hipStreamCreateWithFlags(&c.stream, hipStreamNonBlocking));
    GRM_HIP_CHECK(hipEventCreate(&c.ev0));
    GRM_HIP_CHECK(hipEventCreate(&c.ev1));
    GRM_HIP_CHECK(hipDeviceGetAttribute(&c.cus, hipDeviceAttributeMultiprocessorCount, dev));
  }
  *out = &c;
  return 0;
}

bool valid_args(uint64_t n_values, uint32_t group_size) {
  return group_size > 0 && n_values % group_size == 0;
}

// Enqueue the dequant of n values (codes/scales/out device pointers).
int enqueue(DeviceCtx* c, const void* codes, const void* scales, uint64_t n, uint32_t gs,
            void* out) {
  if (n == 0) return 0;
  // One step per thread: a grid that covers the data measures 6.7 TB/s on
  // 1 Gi values, against 5.1 TB/s for a grid-stride loop over 32 blocks
  // per CU (each thread's load-convert-store chain then serialises).  The
  // stride loop stays for counts beyond the cap, which keeps blocks x
  // threads within the 2^32 - 1 work items a grid dimension may hold.
  const uint64_t max_blocks = 0xffffffffull / kThreads;
  (void)c->cus;
  const bool vec = gs % 8 == 0 && (reinterpret_cast<uintptr_t>(codes) % 8) == 0 &&
                   (reinterpret_cast<uintptr_t>(out) % 16) == 0;
  if (vec && (gs == 32 || gs == 64 || gs == 128)) {
    const uint64_t n8 = n / 8;
    const uint32_t blocks =
        static_cast<uint32_t>(std::min<uint64_t>((n8 + kThreads - 1) / kThreads, max_blocks));
    const auto* cp = static_cast<const u32x2*>(codes);
    const auto* sp = static_cast<const float*>(scales);
    auto* op = static_cast<u32x4*>(out);
    if (gs == 32) dequant8_kernel<32><<<blocks, kThreads, 0, c->stream>>>(cp, sp, n8, op);
    else if (gs == 64) dequant8_kernel<64><<<blocks, kThreads, 0, c->stream>>>(cp, sp, n8, op);
    else dequant8_kernel<128><<<blocks, kThreads, 0, c->stream>>>(cp, sp, n8, op);
  } else {
    const uint32_t blocks =
        static_cast<uint32_t>(std::min<uint64_t>((n + kThreads - 1) / kThreads, max_blocks));
    dequant1_kernel<<<blocks, kThreads, 0, c->stream>>>(
        static_cast<const int8_t*>(codes), static_cast<const float*>(scales), n, gs,
        static_cast<uint16_t*>(out));
  }
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

constexpr uint64_t kStageValues = 64ull << 20;  // values per upload chunk

}  // namespace payload
}  // namespace grm

using grm::payload::DeviceCtx;

// ------------------------------------------------------------ device memory

extern "C" int grm_hip_device_alloc(uint64_t bytes, void** out_ptr) {
  if (!out_ptr) return grm::fail(-1, "null output pointer");
  *out_ptr = nullptr;
  if (bytes == 0) return grm::fail(-1, "zero-byte allocation");
  GRM_HIP_CHECK(hipMalloc(out_ptr, bytes));
  return 0;
}

extern "C" int grm_hip_device_free(void* ptr) {
  if (ptr) GRM_HIP_CHECK(hipFree(ptr));
  return 0;
}

extern "C" int grm_hip_copy_to_host(void* host, const void* device, uint64_t bytes) {
  if ((!host || !device) && bytes) return grm::fail(-1, "null pointer");
  if (bytes) GRM_HIP_CHECK(hipMemcpy(host, device, bytes, hipMemcpyDeviceToHost));
  return 0;
}

extern "C" int grm_hip_copy_to_device(void* device, const void* host, uint64_t bytes) {
  if ((!host || !device) && bytes) return grm::fail(-1, "null pointer");
  if (bytes) GRM_HIP_CHECK(hipMemcpy(device, host, bytes, hipMemcpyHostToDevice));
  return 0;
}

// ---------------------------------------------------------------- payloads

extern "C" int grm_hip_payload_dequant(const void* d_codes, const void* d_scales,
                                       uint64_t n_values, uint32_t group_size, void* d_out_f16,
                                       float* elapsed_ms) {
  if (!grm::payload::valid_args(n_values, group_size)) {
    return grm::fail(-1, "group_size must be > 0 and divide n_values");
  }
  if (n_values && (!d_codes || !d_scales || !d_out_f16)) return grm::fail(-1, "null pointer");
  DeviceCtx* c = nullptr;
  GRM_CHECK_RC(grm::payload::device_ctx(&c));
  GRM_HIP_CHECK(hipEventRecord(c->ev0, c->stream));
  GRM_CHECK_RC(grm::payload::enqueue(c, d_codes, d_scales, n_values, group_size, d_out_f16));
  GRM_HIP_CHECK(hipEventRecord(c->ev1, c->stream));
  GRM_HIP_CHECK(hipEventSynchronize(c->ev1));
  if (elapsed_ms) GRM_HIP_CHECK(hipEventElapsedTime(elapsed_ms, c->ev0, c->ev1));
  grm::clear_error();
  return 0;
}

extern "C" int grm_hip_payload_upload(const void* h_codes, const void* h_scales,
                                      uint64_t n_values, uint32_t group_size, void* d_out_f16,
                                      float* elapsed_ms) {
  if (!grm::payload::valid_args(n_values, group_size)) {
    return grm::fail(-1, "group_size must be > 0 and divide n_values");
  }
  if (n_values && (!h_codes || !h_scales || !d_out_f16)) return grm::fail(-1, "null pointer");
  DeviceCtx* c = nullptr;
  GRM_CHECK_RC(grm::payload::device_ctx(&c));
  // Chunks of whole groups; the staging area holds one chunk's codes and
  // scales (codes first, scales 256-byte aligned after them).
  uint64_t chunk = std::min<uint64_t>(n_values, grm::payload::kStageValues);
  chunk = std::max<uint64_t>(group_size, chunk / group_size * group_size);
  const size_t codes_bytes = (static_cast<size_t>(chunk) + 255) / 256 * 256;
  const size_t need = codes_bytes + static_cast<size_t>(chunk / group_size) * 4;
  if (c->stage_bytes < need) {
    if (c->stage) GRM_HIP_CHECK(hipFree(c->stage));
    c->stage = nullptr;
    c->stage_bytes = 0;
    GRM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&c->stage), need));
    c->stage_bytes = need;
  }
  const auto* hc = static_cast<const unsigned char*>(h_codes);
  const auto* hs = static_cast<const float*>(h_scales);
  auto* out = static_cast<uint16_t*>(d_out_f16);
  GRM_HIP_CHECK(hipEventRecord(c->ev0, c->stream));
  for (uint64_t off = 0; off < n_values; off += chunk) {
    const uint64_t n = std::min<uint64_t>(chunk, n_values - off);
    const uint64_t groups = n / group_size;
    GRM_HIP_CHECK(hipMemcpyAsync(c->stage, hc + off, n, hipMemcpyHostToDevice, c->stream));
    GRM_HIP_CHECK(hipMemcpyAsync(c->stage + codes_bytes, hs + off / group_size, groups * 4,
                                 hipMemcpyHostToDevice, c->stream));
    GRM_CHECK_RC(grm::payload::enqueue(c, c->stage, c->stage + codes_bytes, n, group_size,
                                       out + off));
  }
  GRM_HIP_CHECK(hipEventRecord(c->ev1, c->stream));
  GRM_HIP_CHECK(hipEventSynchronize(c->ev1));
  if (elapsed_ms) GRM_HIP_CHECK(hipEventElapsedTime(elapsed_ms, c->ev0, c->ev1));
  grm::clear_error();
  return 0;
}
