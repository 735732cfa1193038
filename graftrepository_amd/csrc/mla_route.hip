// mla_route.hip -- MLA latent-centroid route on gfx950.
//
// Law (cpp/grm_runtime.cpp:3518-3545 exact_mla_entry_score, :4299-4361
// route_mla_arena, row norms :3232-3241):
//   score(node) = float( dot / (qnorm * (double)norm_f + 1e-8) )
//   dot   = sum_d (double)q_d * (double)r_d, sequential in d
//   qnorm = sqrt(sum_d (double)q_d^2)        norm_f = float(sqrt(sum (double)r_d^2))
// Every node is scored with exactly these fp64 operations in this order, so
// scores are bit-identical to the reference's CPU router and the ranking
// needs no re-check.  fp64 costs nothing here: the kernel streams 4 bytes
// (fp32 bank) or 2 bytes (bf16 bank) per multiply-add and is bound by HBM.
//
// Bank layout in HBM ("chunk planes"): a row is cut into 16-byte chunks (4
// fp32 or 8 bf16 values); slots are grouped in tiles of 64 and chunk c of
// slot tile*64+l lives at [c][tile][l].  Lane l of a wavefront owns one slot
// and walks its row in d order (the law's order); every load instruction of
// a wave reads 1 KiB of contiguous memory, and waves working on neighbouring
// tiles read neighbouring KiB of the same plane, which keeps DRAM rows open
// the way a plain sequential stream does.
//
// Top-k is fused: each wave keeps a distributed top-k list (grm_common.hpp),
// blocks merge their waves' lists in LDS and write their k best entries to
// mapped host memory, where the host merges the per-block lists after the
// kernel's completion event -- the score vector never leaves registers.
//
// Batched queries on a bf16 bank take the matrix-core path (mla_batch.hpp):
// an MFMA screen of 32 slots x up to 256 queries per wave keeps a per-lane
// shortlist, a merge kernel certifies each query's top-k against a proven
// bound on the screen's rounding error and rescores the shortlist with the
// exact law; queries without a certificate are routed again here.
#include "grm_common.hpp"
#include "grm_hip_router.h"

#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <limits>
#include <mutex>
#include <set>
#include <unordered_map>
#include <vector>

namespace grm {
namespace mla {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr uint32_t kMaxDim = 4096;
constexpr int kRouteWaves = 4;           // waves per block, plain kernel
constexpr int kPipeWaves = 16;           // waves per block, pipelined kernel
constexpr uint32_t kStageRows = 1u << 16;  // rows per attach staging batch

// ------------------------------------------------------------------ kernels

template <int DT>
__device__ inline double chunk_dot(u32x4 v, const double* __restrict__ q,
                                   double acc) {
  // fma(r, q, acc) == acc + r*q exactly: r*q has <= 48 significant bits.
  if constexpr (DT == kF32) {
    acc = fma(static_cast<double>(__uint_as_float(v.x)), q[0], acc);
    acc = fma(static_cast<double>(__uint_as_float(v.y)), q[1], acc);
    acc = fma(static_cast<double>(__uint_as_float(v.z)), q[2], acc);
    acc = fma(static_cast<double>(__uint_as_float(v.w)), q[3], acc);
  } else {
    acc = fma(static_cast<double>(__uint_as_float(v.x << 16)), q[0], acc);
    acc = fma(static_cast<double>(__uint_as_float(v.x & 0xffff0000u)), q[1], acc);
    acc = fma(static_cast<double>(__uint_as_float(v.y << 16)), q[2], acc);
    acc = fma(static_cast<double>(__uint_as_float(v.y & 0xffff0000u)), q[3], acc);
    acc = fma(static_cast<double>(__uint_as_float(v.z << 16)), q[4], acc);
    acc = fma(static_cast<double>(__uint_as_float(v.z & 0xffff0000u)), q[5], acc);
    acc = fma(static_cast<double>(__uint_as_float(v.w << 16)), q[6], acc);
    acc = fma(static_cast<double>(__uint_as_float(v.w & 0xffff0000u)), q[7], acc);
  }
  return acc;
}

// Dot product of this lane's row with the query, d ascending.
template <int DT>
__device__ inline double tile_dot(const u32x4* __restrict__ p, uint32_t chunks,
                                  size_t plane, const double* __restrict__ qd) {
  constexpr int EPC = DT == kF32 ? 4 : 8;
  constexpr uint32_t kBatch = 8;
  double acc = 0.0;
  uint32_t c = 0;
  for (; c + kBatch <= chunks; c += kBatch) {
    u32x4 v[kBatch];
#pragma unroll
    for (uint32_t j = 0; j < kBatch; ++j) {
      v[j] = __builtin_nontemporal_load(p + static_cast<size_t>(c + j) * plane);
    }
#pragma unroll
    for (uint32_t j = 0; j < kBatch; ++j) {
      acc = chunk_dot<DT>(v[j], qd + (c + j) * EPC, acc);
    }
  }
  for (; c < chunks; ++c) {
    acc = chunk_dot<DT>(__builtin_nontemporal_load(p + static_cast<size_t>(c) * plane),
                        qd + c * EPC, acc);
  }
  return acc;
}

// One query against every slot; each block writes its k best entries to
// block_out[blockIdx.x*k ..), then (with done) seq to done[blockIdx.x];
// with stamps a timed route's start and end ticks (RouteStamps).
template <int DT, int NW>
__global__ __launch_bounds__(NW * kWave) void mla_route_kernel(
    const u32x4* __restrict__ tiles, const float* __restrict__ norms,
    const uint64_t* __restrict__ ids, uint32_t num_tiles, uint32_t chunks,
    size_t plane, uint32_t dim, uint32_t dim_pad,
    const void* __restrict__ query, int query_dtype, int k,
    Cand* __restrict__ block_out, unsigned* __restrict__ done, unsigned seq, RouteStamps stamps) {
  route_start_stamp(stamps, seq);
  extern __shared__ double qd[];
  __shared__ double s_qnorm;
  __shared__ Cand s_lists[NW][kMaxTopK];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;

  for (uint32_t d = tid; d < dim_pad; d += NW * kWave) {
    double v = 0.0;
    if (d < dim) {
      v = query_dtype == kBF16
              ? static_cast<double>(bf16_to_f32(static_cast<const uint16_t*>(query)[d]))
              : static_cast<double>(static_cast<const float*>(query)[d]);
    }
    qd[d] = v;
  }
  __syncthreads();
  if (tid == 0) {
    double acc = 0.0;  // cpp/grm_runtime.cpp:4310-4314, sequential
    for (uint32_t d = 0; d < dim; ++d) acc = fma(qd[d], qd[d], acc);
    s_qnorm = sqrt(acc);
  }
  __syncthreads();
  const double qnorm = s_qnorm;

  WaveList L;
  wl_init(L);
  for (uint32_t t = blockIdx.x * NW + wave; t < num_tiles; t += gridDim.x * NW) {
    const double dot = tile_dot<DT>(
        tiles + static_cast<size_t>(t) * kWave + lane, chunks, plane, qd);
    const uint32_t slot = t * kWave + lane;
    const float nrm = norms[slot];  // NaN marks an empty or evicted slot
    const double den = qnorm * static_cast<double>(nrm) + 1.0e-8;
    const float s = static_cast<float>(dot / den);
    const bool need = isfinite(s) && s >= L.th_s;
    uint64_t id = kNoId;
    if (need) id = ids[slot];
    wl_consume(L, k, s, id, slot, need);
  }

  block_topk_write<NW>(L, k, s_lists, block_out, done ? route_tag(seq) : kNoSlot);
  block_done_flag(done, seq, stamps.end);
}

// Stage the query as doubles in LDS (zero beyond dim).
__device__ inline void stage_query(double* qd, const void* __restrict__ query,
                                   int query_dtype, uint32_t dim,
                                   uint32_t dim_pad) {
  for (uint32_t d = threadIdx.x; d < dim_pad; d += blockDim.x) {
    double v = 0.0;
    if (d < dim) {
      v = query_dtype == kBF16
              ? static_cast<double>(bf16_to_f32(static_cast<const uint16_t*>(query)[d]))
              : static_cast<double>(static_cast<const float*>(query)[d]);
    }
    qd[d] = v;
  }
}

template <int DT, int B>
__device__ inline double batch_dot(const u32x4 (&v)[B],
                                   const double* __restrict__ q, double acc) {
  constexpr int EPC = DT == kF32 ? 4 : 8;
#pragma unroll
  for (int j = 0; j < B; ++j) acc = chunk_dot<DT>(v[j], q + j * EPC, acc);
  return acc;
}

// Software-pipelined variant for rows of a whole number of B-chunk batches:
// while a batch is folded into the fp64 dot product the next batch (of the
// same tile or the wave's next tile) is already in flight, and the row norm
// of the next tile is fetched ahead of its data.  Arithmetic and order are
// those of mla_route_kernel.
template <int DT, int NW, int B>
__global__ __launch_bounds__(NW * kWave) void mla_route_pipe_kernel(
    const u32x4* __restrict__ tiles, const float* __restrict__ norms,
    const uint64_t* __restrict__ ids, uint32_t num_tiles, uint32_t chunks,
    size_t plane, uint32_t dim, uint32_t dim_pad,
    const void* __restrict__ query, int query_dtype, int k,
    Cand* __restrict__ block_out, unsigned* __restrict__ done, unsigned seq, RouteStamps stamps) {
  route_start_stamp(stamps, seq);
  constexpr int EPC = DT == kF32 ? 4 : 8;
  extern __shared__ double qd[];
  __shared__ double s_qnorm;
  __shared__ Cand s_lists[NW][kMaxTopK];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const uint32_t stride = gridDim.x * NW;
  const uint32_t nb = chunks / B;
  // Beyond-the-end prefetches read tile 0's first batch (cache resident).
  auto batch_ptr = [&](uint32_t t, uint32_t b) {
    return t < num_tiles
               ? tiles + static_cast<size_t>(b) * B * plane + static_cast<size_t>(t) * kWave + lane
               : tiles + lane;
  };
  auto load = [&](u32x4 (&v)[B], const u32x4* p) {
#pragma unroll
    for (int j = 0; j < B; ++j) v[j] = __builtin_nontemporal_load(p + j * plane);
  };

  uint32_t t = blockIdx.x * NW + wave;
  uint32_t b = 0;
  u32x4 bufA[B], bufB[B];
  float nrm_cur = norms[(t < num_tiles ? t : 0) * kWave + lane];
  load(bufA, batch_ptr(t, 0));

  stage_query(qd, query, query_dtype, dim, dim_pad);
  __syncthreads();
  if (tid == 0) {
    double acc = 0.0;  // cpp/grm_runtime.cpp:4310-4314, sequential
    for (uint32_t d = 0; d < dim; ++d) acc = fma(qd[d], qd[d], acc);
    s_qnorm = sqrt(acc);
  }
  __syncthreads();
  const double qnorm = s_qnorm;

  WaveList L;
  wl_init(L);
  auto finish = [&](uint32_t tt, double dot, float nrm) {
    const uint32_t slot = tt * kWave + lane;
    const double den = qnorm * static_cast<double>(nrm) + 1.0e-8;
    const float s = static_cast<float>(dot / den);
    const bool need = isfinite(s) && s >= L.th_s;
    uint64_t id = kNoId;
    if (need) id = ids[slot];
    wl_consume(L, k, s, id, slot, need);
  };
  double acc = 0.0;
  float nrm_next = 0.0f;
  while (t < num_tiles) {
    uint32_t tn = t, bn = b + 1;
    if (bn == nb) {
      tn = t + stride;
      bn = 0;
      nrm_next = norms[(tn < num_tiles ? tn : 0) * kWave + lane];
    }
    load(bufB, batch_ptr(tn, bn));
    acc = batch_dot<DT, B>(bufA, qd + b * B * EPC, acc);
    if (bn == 0) {
      finish(t, acc, nrm_cur);
      acc = 0.0;
      nrm_cur = nrm_next;
    }
    t = tn;
    b = bn;
    if (t >= num_tiles) break;

    tn = t;
    bn = b + 1;
    if (bn == nb) {
      tn = t + stride;
      bn = 0;
      nrm_next = norms[(tn < num_tiles ? tn : 0) * kWave + lane];
    }
    load(bufA, batch_ptr(tn, bn));
    acc = batch_dot<DT, B>(bufB, qd + b * B * EPC, acc);
    if (bn == 0) {
      finish(t, acc, nrm_cur);
      acc = 0.0;
      nrm_cur = nrm_next;
    }
    t = tn;
    b = bn;
  }
  block_topk_write<NW>(L, k, s_lists, block_out, done ? route_tag(seq) : kNoSlot);
  block_done_flag(done, seq, stamps.end);
}

// Place staged row-major rows into their tile slots and compute row norms
// (cpp/grm_runtime.cpp:3232-3241).  rows: [count][dim] of DT; slots/ids may be
// null (contiguous slots from slot0 / ids = slot).  norm_range[0] tracks the
// smallest positive norm ever placed, norm_range[1] the largest finite one
// (float bits, atomicMin / atomicMax).  A row holding a non-finite value
// has a NaN or infinite dot product with every query, so the law scores it
// NaN whatever its norm; such a row is stored as zeros with a NaN norm,
// which every route scores NaN as well (0 / NaN), and which the batched
// screen's products can then never overflow on.
template <int DT>
__global__ void mla_place_rows_kernel(const void* __restrict__ rows,
                                      uint64_t count, uint32_t dim,
                                      uint32_t chunks, size_t plane,
                                      const uint64_t* __restrict__ slots,
                                      const uint64_t* __restrict__ ids,
                                      uint64_t slot0, u32x4* __restrict__ tiles,
                                      float* __restrict__ norms,
                                      uint64_t* __restrict__ slot_ids,
                                      unsigned* __restrict__ norm_range) {
  constexpr int EPC = DT == kF32 ? 4 : 8;
  for (uint64_t r = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
       r < count; r += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint64_t slot = slots ? slots[r] : slot0 + r;
    const uint64_t tile = slot / kWave;
    const uint32_t lane = static_cast<uint32_t>(slot % kWave);
    u32x4* dst = tiles + tile * kWave + lane;
    double acc = 0.0;
    for (uint32_t c = 0; c < chunks; ++c) {
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      for (int e = 0; e < EPC; ++e) {
        const uint32_t d = c * EPC + e;
        float f = 0.0f;
        uint32_t bits = 0u;
        if (d < dim) {
          if constexpr (DT == kF32) {
            f = static_cast<const float*>(rows)[r * dim + d];
            bits = __float_as_uint(f);
          } else {
            bits = static_cast<const uint16_t*>(rows)[r * dim + d];
            f = bf16_to_f32(bits);
          }
          acc = fma(static_cast<double>(f), static_cast<double>(f), acc);
        }
        if constexpr (DT == kF32) {
          w[e] = bits;
        } else {
          w[e / 2] |= (e & 1) ? (bits << 16) : bits;
        }
      }
      u32x4 v;
      v.x = w[0];
      v.y = w[1];
      v.z = w[2];
      v.w = w[3];
      dst[static_cast<size_t>(c) * plane] = v;
    }
    // squares of finite fp32 / bf16 values cannot overflow fp64
    const bool finite_row = isfinite(acc);
    if (!finite_row) {
      const u32x4 zero = {0u, 0u, 0u, 0u};
      for (uint32_t c = 0; c < chunks; ++c) dst[static_cast<size_t>(c) * plane] = zero;
    }
    const float nf = finite_row ? static_cast<float>(sqrt(acc)) : __builtin_nanf("");
    norms[slot] = nf;
    slot_ids[slot] = ids ? ids[r] : slot;
    // norm range (non-negative floats order like their bits)
    if (nf > 0.0f && isfinite(nf)) {
      atomicMin(norm_range, __float_as_uint(nf));
      atomicMax(norm_range + 1, __float_as_uint(nf));
    }
  }
}

__global__ void mla_evict_kernel(const uint64_t* __restrict__ slots,
                                 uint64_t count, float* __restrict__ norms,
                                 uint64_t* __restrict__ slot_ids) {
  for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
       i < count; i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint64_t s = slots[i];
    norms[s] = __uint_as_float(0xffffffffu);
    slot_ids[s] = kNoId;
  }
}

}  // namespace mla
}  // namespace grm

#include "mla_batch.hpp"

using grm::Cand;
using grm::kBF16;
using grm::kF16;
using grm::kF32;
using grm::kNoId;
using grm::mla::u32x4;

// ------------------------------------------------------------------ host side

struct MlaDeviceArena {
  int device = 0;
  int dtype = kF32;
  uint32_t dim = 0;
  uint32_t dim_pad = 0;
  uint32_t epc = 4;
  uint32_t chunks = 0;
  uint32_t planes = 0;      // chunk planes allocated: chunks, or (bf16) the batched screen's 2*KS
  uint64_t capacity = 0;    // slots, multiple of 64
  uint64_t high_water = 0;  // slots [0, high_water) may hold live rows
  uint64_t live = 0;
  uint64_t epoch = 0;
  u32x4* d_tiles = nullptr;
  float* d_norms = nullptr;
  uint64_t* d_ids = nullptr;
  std::vector<uint64_t> slot_id;  // kNoId when free
  std::unordered_map<uint64_t, uint64_t> slot_of;
  std::set<uint64_t> free_slots;  // freed slots below high_water
  void* d_queries = nullptr;
  size_t d_queries_bytes = 0;
  float* d_latent_q = nullptr;  // route key formed from a device latent (dim floats)
  uint64_t* d_fbits = nullptr;  // per-slot route filter bits (capacity), 0 until set
  float* d_fnorms = nullptr;    // per-route norms with filtered-out slots NaN (capacity)
  const float* route_norms = nullptr;  // set around a filtered route: norms it reads
  bool no_batch = false;               // set around a filtered route: single-query path only
  grm::MappedCands blocks_out;  // per-query, per-block top-k (host mapped)
  // per-(query, block) completion flags (host mapped) and the number the
  // last flag-waiting route stored there
  grm::MappedBuf done_flags;
  unsigned route_seq = 0;
  // device-clock stamps of timed single-query routes on the flag path
  // (host mapped), and the clock's ticks per ms (0: stream events)
  grm::MappedBuf stamps;
  double ticks_per_ms = 0.0;
  std::vector<Cand> merged;
  void* h_stage = nullptr;
  size_t h_stage_bytes = 0;
  void* d_stage = nullptr;
  size_t d_stage_bytes = 0;
  hipStream_t stream = nullptr;
  hipStream_t side = nullptr;
  hipEvent_t ev_start = nullptr;
  hipEvent_t ev_stop = nullptr;
  hipEvent_t ev_mut = nullptr;
  bool mut_pending = false;
  unsigned* d_min_norm = nullptr;  // [smallest positive, largest finite] row norm placed (float bits)
  // batched route (bf16 banks): pass buffers and per-query results
  uint16_t* d_qpad = nullptr;
  size_t d_qpad_count = 0;
  float* d_inv_qn = nullptr;
  size_t d_inv_qn_count = 0;
  uint32_t* d_entries = nullptr;   // screen result planes
  size_t d_entries_count = 0;
  grm::MappedCands batch_out;
  grm::MappedBuf batch_status;
  // host queries staged for fetch_async (GRM_HIP_QUERY_COPY=dma: the copy
  // engine instead)
  grm::MappedBuf q_map;
  bool query_dma = false;
  int batch_min = 4;         // timed queries per call from which the batched path runs
  bool ring = true;          // full 256-query passes on the ring screen (GRM_HIP_BATCH_RING=0: off)
  float* d_winv = nullptr;   // slot weights of the ring screen (capacity), for bank epoch winv_epoch
  size_t d_winv_count = 0;
  uint64_t winv_epoch = ~0ull;
  size_t lds_max = 65536;    // dynamic LDS one block may use
  uint64_t batch_queries = 0;    // queries screened on the matrix cores
  uint64_t batch_fallbacks = 0;  // of those, routed again on the single-query path
  uint64_t batch_passes = 0;     // screen passes
  uint64_t single_queries = 0;   // queries through the single-query kernel
  std::vector<hipEvent_t> screen_ev;  // begin/end pairs around timed screens
  float screen_ms = 0.0f;        // screen-kernel time of the last batched route
  bool pipeline = true;     // software-pipelined kernel when rows allow it
  uint32_t cus = 256;       // compute units of the device
  uint32_t max_blocks = 0;  // plain-kernel grid cap (4 blocks per CU)
};

// Per-block top-k lists of the allocation-free route (see route_noalloc).
constexpr size_t kScratchCands = 16384;  // 256 KiB
static __device__ __align__(256) Cand scratch[kScratchCands];

namespace {

size_t elem_size(int dtype) { return dtype == kF32 ? 4 : 2; }

void destroy_arena(MlaDeviceArena* a) {
  if (!a) return;
  (void)hipSetDevice(a->device);
  if (a->stream) (void)hipStreamSynchronize(a->stream);
  if (a->side) (void)hipStreamSynchronize(a->side);
  if (a->d_tiles) (void)hipFree(a->d_tiles);
  if (a->d_norms) (void)hipFree(a->d_norms);
  if (a->d_ids) (void)hipFree(a->d_ids);
  if (a->d_queries) (void)hipFree(a->d_queries);
  if (a->d_latent_q) (void)hipFree(a->d_latent_q);
  if (a->d_fbits) (void)hipFree(a->d_fbits);
  if (a->d_fnorms) (void)hipFree(a->d_fnorms);
  if (a->d_stage) (void)hipFree(a->d_stage);
  if (a->d_min_norm) (void)hipFree(a->d_min_norm);
  if (a->d_qpad) (void)hipFree(a->d_qpad);
  if (a->d_inv_qn) (void)hipFree(a->d_inv_qn);
  if (a->d_entries) (void)hipFree(a->d_entries);
  if (a->d_winv) (void)hipFree(a->d_winv);
  grm::release_mapped(&a->batch_out);
  grm::release_mapped_bytes(&a->batch_status);
  grm::release_mapped_bytes(&a->q_map);
  grm::release_mapped(&a->blocks_out);
  grm::release_mapped_bytes(&a->done_flags);
  grm::release_mapped_bytes(&a->stamps);
  if (a->h_stage) (void)hipHostFree(a->h_stage);
  if (a->ev_start) (void)hipEventDestroy(a->ev_start);
  if (a->ev_stop) (void)hipEventDestroy(a->ev_stop);
  if (a->ev_mut) (void)hipEventDestroy(a->ev_mut);
  for (hipEvent_t e : a->screen_ev) (void)hipEventDestroy(e);
  if (a->stream) (void)hipStreamDestroy(a->stream);
  if (a->side) (void)hipStreamDestroy(a->side);
  delete a;
}

template <typename T>
int reserve_device(T** ptr, size_t* have, size_t want) {
  if (want <= *have && *ptr) return 0;
  if (*ptr) {
    GRM_HIP_CHECK(hipFree(*ptr));
    *ptr = nullptr;
    *have = 0;
  }
  GRM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(ptr), want * sizeof(T)));
  *have = want;
  return 0;
}

template <typename T>
int reserve_pinned(T** ptr, size_t* have, size_t want) {
  if (want <= *have && *ptr) return 0;
  if (*ptr) {
    GRM_HIP_CHECK(hipHostFree(*ptr));
    *ptr = nullptr;
    *have = 0;
  }
  GRM_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(ptr), want * sizeof(T),
                              hipHostMallocDefault));
  *have = want;
  return 0;
}

int wait_mutations(MlaDeviceArena* a) {
  if (a->mut_pending) {
    GRM_HIP_CHECK(hipEventSynchronize(a->ev_mut));
    a->mut_pending = false;
  }
  return 0;
}

// Launch the placement kernel over `count` staged rows on `stream`.
int launch_place(MlaDeviceArena* a, const void* d_rows, uint64_t count,
                 const uint64_t* d_slots, const uint64_t* d_ids, uint64_t slot0,
                 hipStream_t stream) {
  if (count == 0) return 0;
  const unsigned threads = 256;
  const unsigned blocks = static_cast<unsigned>(
      std::min<uint64_t>((count + threads - 1) / threads, 4096));
  if (a->dtype == kF32) {
    grm::mla::mla_place_rows_kernel<kF32><<<blocks, threads, 0, stream>>>(
        d_rows, count, a->dim, a->chunks, a->capacity, d_slots, d_ids, slot0,
        a->d_tiles, a->d_norms, a->d_ids, a->d_min_norm);
  } else {
    grm::mla::mla_place_rows_kernel<kBF16><<<blocks, threads, 0, stream>>>(
        d_rows, count, a->dim, a->chunks, a->capacity, d_slots, d_ids, slot0,
        a->d_tiles, a->d_norms, a->d_ids, a->d_min_norm);
  }
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

int create_arena(const void* rows, int dtype, uint64_t nodes, int dim,
                 const uint64_t* node_ids, uint64_t capacity,
                 MlaDeviceArena** out) {
  if (!out) return grm::fail(-1, "null output arena pointer");
  *out = nullptr;
  if (dim <= 0 || static_cast<uint32_t>(dim) > grm::mla::kMaxDim) {
    return grm::fail(-1, "dim must be in [1, 4096]");
  }
  if (dtype != kF32 && dtype != kBF16) {
    return grm::fail(-1, "MLA bank dtype must be F32 or BF16");
  }
  if (nodes > 0 && !rows) return grm::fail(-1, "null rows with nonzero nodes");
  if (capacity < nodes) capacity = nodes;
  if (capacity == 0) return grm::fail(-1, "bank needs nodes or capacity");
  if (capacity > (1ull << 31)) return grm::fail(-1, "capacity above 2^31 slots");
  auto* a = new MlaDeviceArena();
  int rc = 0;
  auto bail = [&](int code) {
    destroy_arena(a);
    return code;
  };
  if (hipGetDevice(&a->device) != hipSuccess) a->device = 0;
  a->dtype = dtype;
  a->dim = static_cast<uint32_t>(dim);
  a->epc = dtype == kF32 ? 4 : 8;
  a->dim_pad = (a->dim + a->epc - 1) / a->epc * a->epc;
  a->chunks = a->dim_pad / a->epc;
  // bf16 banks get zero planes up to the batched screen's 16-dimension
  // K-steps (16, 32 or 36 planes), which it then reads unconditionally
  a->planes = a->chunks;
  if (dtype == kBF16) {
    for (uint32_t p : {16u, 32u, 36u}) {
      if (a->chunks <= p) {
        a->planes = p;
        break;
      }
    }
  }
  a->capacity = (capacity + grm::kWave - 1) / grm::kWave * grm::kWave;
  {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, a->device) != hipSuccess ||
        cus <= 0) {
      cus = 256;
    }
    a->cus = static_cast<uint32_t>(cus);
    a->max_blocks = static_cast<uint32_t>(cus) * 4;
  }
  if (const char* env = getenv("GRM_HIP_MLA_BLOCKS")) {
    const long v = strtol(env, nullptr, 10);
    if (v >= 1 && v <= 65536) a->max_blocks = static_cast<uint32_t>(v);
  }
  if (const char* env = getenv("GRM_HIP_MLA_PIPELINE")) a->pipeline = env[0] != '0';
  if (const char* env = getenv("GRM_HIP_BATCH_RING")) a->ring = env[0] != '0';
  if (const char* env = getenv("GRM_HIP_QUERY_COPY")) a->query_dma = strcmp(env, "dma") == 0;
  a->ticks_per_ms = grm::wall_ticks_per_ms(a->device);
  if (const char* env = getenv("GRM_HIP_MLA_BATCH_MIN")) {
    const long v = strtol(env, nullptr, 10);
    if (v >= 1) a->batch_min = static_cast<int>(std::min<long>(v, 1l << 30));
  }
  {
    int lds = 0;
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeSharedMemPerBlockOptin, a->device) == hipSuccess &&
        lds > 0) {
      a->lds_max = static_cast<size_t>(lds);
    } else if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerBlock, a->device) ==
                   hipSuccess &&
               lds > 0) {
      a->lds_max = static_cast<size_t>(lds);
    }
  }
  a->slot_id.assign(a->capacity, kNoId);
  if (node_ids) {
    a->slot_of.reserve(nodes * 2);
    for (uint64_t i = 0; i < nodes; ++i) {
      if (!a->slot_of.emplace(node_ids[i], i).second) {
        return bail(grm::fail(-1, "duplicate node id"));
      }
      a->slot_id[i] = node_ids[i];
    }
  } else {
    a->slot_of.reserve(nodes * 2);
    for (uint64_t i = 0; i < nodes; ++i) {
      a->slot_of.emplace(i, i);
      a->slot_id[i] = i;
    }
  }
  const size_t tile_bytes = static_cast<size_t>(a->planes) * grm::kWave * 16;
  const size_t tiles = a->capacity / grm::kWave;
#define BAIL_HIP(expr)                                  \
  do {                                                  \
    hipError_t e_ = (expr);                             \
    if (e_ != hipSuccess) return bail(grm::fail_hip(e_, #expr)); \
  } while (0)
  BAIL_HIP(hipStreamCreateWithFlags(&a->stream, hipStreamDefault));
  BAIL_HIP(hipStreamCreateWithFlags(&a->side, hipStreamNonBlocking));
  BAIL_HIP(hipEventCreate(&a->ev_start));
  BAIL_HIP(hipEventCreate(&a->ev_stop));
  BAIL_HIP(hipEventCreateWithFlags(&a->ev_mut, hipEventDisableTiming));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_tiles), tiles * tile_bytes));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_norms), a->capacity * sizeof(float)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_ids), a->capacity * sizeof(uint64_t)));
  BAIL_HIP(hipMemsetAsync(a->d_tiles, 0, tiles * tile_bytes, a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_norms, 0xff, a->capacity * sizeof(float), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_ids, 0xff, a->capacity * sizeof(uint64_t), a->stream));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_min_norm), 2 * sizeof(unsigned)));
  {
    const unsigned range0[2] = {0x7f800000u, 0u};
    BAIL_HIP(hipMemcpyAsync(a->d_min_norm, range0, sizeof(range0), hipMemcpyHostToDevice,
                            a->stream));
    BAIL_HIP(hipStreamSynchronize(a->stream));
  }
  if (nodes > 0) {
    const size_t row_bytes = static_cast<size_t>(a->dim) * elem_size(dtype);
    const uint64_t batch = std::min<uint64_t>(nodes, grm::mla::kStageRows);
    rc = reserve_device(reinterpret_cast<unsigned char**>(&a->d_stage),
                        &a->d_stage_bytes,
                        batch * (row_bytes + sizeof(uint64_t)));
    if (rc) return bail(rc);
    for (uint64_t r0 = 0; r0 < nodes; r0 += batch) {
      const uint64_t n = std::min<uint64_t>(batch, nodes - r0);
      unsigned char* d_rows = static_cast<unsigned char*>(a->d_stage);
      uint64_t* d_idbuf = reinterpret_cast<uint64_t*>(d_rows + batch * row_bytes);
      BAIL_HIP(hipMemcpyAsync(d_rows,
                              static_cast<const unsigned char*>(rows) + r0 * row_bytes,
                              n * row_bytes, hipMemcpyHostToDevice, a->stream));
      if (node_ids) {
        BAIL_HIP(hipMemcpyAsync(d_idbuf, node_ids + r0, n * sizeof(uint64_t),
                                hipMemcpyHostToDevice, a->stream));
      }
      rc = launch_place(a, d_rows, n, nullptr, node_ids ? d_idbuf : nullptr,
                        r0, a->stream);
      if (rc) return bail(rc);
      // The staging buffer is reused by the next batch.
      BAIL_HIP(hipStreamSynchronize(a->stream));
    }
  }
  BAIL_HIP(hipStreamSynchronize(a->stream));
#undef BAIL_HIP
  a->high_water = nodes;
  a->live = nodes;
  *out = a;
  grm::clear_error();
  return 0;
}

// Launch geometry of the single-query route kernel.
struct SingleGeom {
  uint32_t num_tiles = 0, blocks = 0, nw = 0;
  int batch = 0;  // chunks per pipelined load batch (0: plain kernel)
};

SingleGeom single_geom(const MlaDeviceArena* a) {
  SingleGeom g;
  g.num_tiles = static_cast<uint32_t>((a->high_water + grm::kWave - 1) / grm::kWave);
  // The pipelined kernel runs one 16-wave block per CU (4 waves per SIMD);
  // the plain kernel (rows that do not split into whole batches) 4-wave
  // blocks, 4 per CU.
  if (a->pipeline) {
    for (int b : {9, 8, 6}) {
      if (a->chunks % b == 0) {
        g.batch = b;
        break;
      }
    }
  }
  g.nw = g.batch ? grm::mla::kPipeWaves : grm::mla::kRouteWaves;
  const uint32_t cap = g.batch ? std::min(a->cus, a->max_blocks) : a->max_blocks;
  g.blocks = std::max<uint32_t>(1, std::min((g.num_tiles + g.nw - 1) / g.nw, cap));
  return g;
}

// One query (device pointer q) through the single-query kernel; its
// per-block top-k lands at bout (g.blocks * topk entries), and with done
// its blocks' completion flags at done[0, g.blocks).
int launch_single(MlaDeviceArena* a, const SingleGeom& g, const void* q, int q_dtype, int topk,
                  Cand* bout, unsigned* done = nullptr,
                  const grm::RouteStamps& st = grm::RouteStamps{nullptr, nullptr}) {
  const size_t lds = static_cast<size_t>(a->dim_pad) * sizeof(double);
  const dim3 grid(g.blocks), block(g.nw * grm::kWave);
  const float* nrm = a->route_norms ? a->route_norms : a->d_norms;
#define GRM_MLA_ARGS                                                                  \
  a->d_tiles, nrm, a->d_ids, g.num_tiles, a->chunks, a->capacity, a->dim, a->dim_pad, q, \
      q_dtype, topk, bout, done, a->route_seq, st
  constexpr int PW = grm::mla::kPipeWaves;
  constexpr int RW = grm::mla::kRouteWaves;
  if (a->dtype == kF32) {
    switch (g.batch) {
      case 9: grm::mla::mla_route_pipe_kernel<kF32, PW, 9><<<grid, block, lds, a->stream>>>(GRM_MLA_ARGS); break;
      case 8: grm::mla::mla_route_pipe_kernel<kF32, PW, 8><<<grid, block, lds, a->stream>>>(GRM_MLA_ARGS); break;
      case 6: grm::mla::mla_route_pipe_kernel<kF32, PW, 6><<<grid, block, lds, a->stream>>>(GRM_MLA_ARGS); break;
      default: grm::mla::mla_route_kernel<kF32, RW><<<grid, block, lds, a->stream>>>(GRM_MLA_ARGS); break;
    }
  } else {
    switch (g.batch) {
      case 9: grm::mla::mla_route_pipe_kernel<kBF16, PW, 9><<<grid, block, lds, a->stream>>>(GRM_MLA_ARGS); break;
      case 8: grm::mla::mla_route_pipe_kernel<kBF16, PW, 8><<<grid, block, lds, a->stream>>>(GRM_MLA_ARGS); break;
      case 6: grm::mla::mla_route_pipe_kernel<kBF16, PW, 6><<<grid, block, lds, a->stream>>>(GRM_MLA_ARGS); break;
      default: grm::mla::mla_route_kernel<kBF16, RW><<<grid, block, lds, a->stream>>>(GRM_MLA_ARGS); break;
    }
  }
#undef GRM_MLA_ARGS
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

void write_cands(const Cand* c, int topk, uint64_t* out_ids, float* out_scores) {
  for (int j = 0; j < topk; ++j) {
    const bool ok = isfinite(c[j].score) && c[j].id != kNoId;
    out_ids[j] = ok ? c[j].id : kNoId;
    if (out_scores) out_scores[j] = ok ? c[j].score : __builtin_nanf("");
  }
}

// Batched-route plan: K-steps of 16 dims (template), LDS row stride.
struct BatchPlan {
  int ks = 0;        // 8, 16 or 18
  int stride = 0;    // bf16 elements per staged query row
  int qp_max = 0;    // queries per pass (multiple of 32, <= 256)
  int ibits = 0;     // width of the slot code the screen writes into its values
  bool ring = false;   // full passes run mla_batch_ring_kernel
  int ibits_ring = 0;  // its slot code width (one sub-stream per block)
};

// Slot code width of the batched screen: 4 bits of result register, the
// lane half, and enough bits for the longest run of tiles one screen
// wavefront walks.  The code costs the screen bound 2^(ibits-23) relative,
// so banks whose runs would need more than 16 bits route on the
// single-query path instead.
constexpr int kMaxSlotCodeBits = 16;

bool batch_plan(const MlaDeviceArena* a, int q_timed, BatchPlan* p) {
  if (a->dtype != kBF16 || q_timed < a->batch_min) return false;
  const uint32_t ks_need = (a->chunks + 1) / 2;
  p->ks = ks_need <= 8 ? 8 : (ks_need <= 16 ? 16 : (ks_need <= 18 ? 18 : 0));
  if (p->ks == 0 || a->planes < 2u * p->ks) return false;
  // 16*ks >= dim_pad always (ks covers the row's chunks); the screen
  // kernel takes this stride as a compile-time constant of its KS
  p->stride = 16 * p->ks + 8;
  const size_t row = std::max(static_cast<size_t>(p->stride) * 2,
                              static_cast<size_t>(grm::mla::kEntryPlanes) * grm::mla::kBatchWaves * 4);
  int qp = grm::mla::kBatchMaxCols;
  while (qp >= 32 && static_cast<size_t>(qp) * row > a->lds_max) qp /= 2;
  if (qp < 32) return false;
  // the merge holds kMergePer sub-streams (screen wavefronts) per thread
  if (static_cast<size_t>(a->cus) * grm::mla::kBatchWaves >
      static_cast<size_t>(grm::mla::kMergeLoaders) * grm::mla::kMergePer) {
    return false;
  }
  if (a->dim > grm::mla::kBatchMaxDim) return false;
  const uint32_t n_tiles32 = static_cast<uint32_t>((a->high_water + 31) / 32);
  auto code_bits = [&](uint32_t n_sub) {
    const uint32_t max_run = (n_tiles32 + n_sub - 1) / n_sub;
    int ibits = 5;
    while ((1u << (ibits - 5)) < max_run) ++ibits;
    return ibits;
  };
  const int ibits = code_bits(static_cast<uint32_t>(a->cus) * grm::mla::kBatchWaves);
  if (ibits > kMaxSlotCodeBits) return false;
  p->ibits = ibits;
  p->qp_max = qp;
  p->ibits_ring = code_bits(static_cast<uint32_t>(a->cus));
  p->ring = a->ring && qp == grm::mla::kRingQueries && p->ibits_ring <= kMaxSlotCodeBits &&
            grm::mla::RingShape<18>::kLds <= a->lds_max;
  return true;
}

// A pass of ct column tiles runs on the ring screen when the plan allows
// it and the pass is full (more than 128 queries, padded to 256).
bool ring_pass(const BatchPlan& p, int ct) { return p.ring && ct == 8; }
uint32_t pass_subs(const MlaDeviceArena* a, const BatchPlan& p, int ct) {
  return static_cast<uint32_t>(a->cus) * (ring_pass(p, ct) ? 1u : static_cast<uint32_t>(grm::mla::kBatchWaves));
}
int pass_ibits(const BatchPlan& p, int ct) { return ring_pass(p, ct) ? p.ibits_ring : p.ibits; }

// The ring screen's slot weights, formed again when the bank changed.
int ensure_weights(MlaDeviceArena* a) {
  GRM_CHECK_RC(reserve_device(&a->d_winv, &a->d_winv_count, static_cast<size_t>(a->capacity)));
  if (a->winv_epoch != a->epoch) {
    const unsigned blocks = static_cast<unsigned>((a->capacity + 255) / 256);
    grm::mla::mla_batch_weights_kernel<<<blocks, 256, 0, a->stream>>>(a->d_norms, a->capacity,
                                                                     a->d_winv);
    GRM_HIP_CHECK(hipGetLastError());
    a->winv_epoch = a->epoch;
  }
  return 0;
}

template <int KS, bool kProbe = false>
int launch_ring(MlaDeviceArena* a, uint32_t n_tiles32, int ibits, uint32_t* planes) {
  using RS = grm::mla::RingShape<KS>;
  auto kern = grm::mla::mla_batch_ring_kernel<KS, kProbe>;
  GRM_CHECK_RC(ensure_weights(a));
  GRM_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                    hipFuncAttributeMaxDynamicSharedMemorySize,
                                    static_cast<int>(RS::kLds)));
  kern<<<a->cus, grm::mla::kRingWaves * grm::kWave, RS::kLds, a->stream>>>(
      a->d_tiles, a->d_winv, a->capacity, n_tiles32, a->d_qpad, ibits, planes);
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

template <int KS, int CT, bool kProbe = false>
int launch_screen(MlaDeviceArena* a, uint32_t n_tiles32, int stride, int ibits, size_t lds,
                  uint32_t* planes) {
  auto kern = grm::mla::mla_batch_screen_kernel<KS, CT, kProbe>;
  if (lds > 65536) {
    GRM_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)));
  }
  kern<<<a->cus, grm::mla::kBatchWaves * grm::kWave, lds, a->stream>>>(
      a->d_tiles, a->d_norms, a->capacity, a->chunks, n_tiles32, a->d_qpad, stride, ibits, planes);
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

template <bool kProbe>
int dispatch_screen(MlaDeviceArena* a, const BatchPlan& p, int ct, uint32_t n_tiles32, size_t lds,
                    uint32_t* planes) {
  if (ring_pass(p, ct)) {
    switch (p.ks) {
      case 8: return launch_ring<8, kProbe>(a, n_tiles32, p.ibits_ring, planes);
      case 16: return launch_ring<16, kProbe>(a, n_tiles32, p.ibits_ring, planes);
      default: return launch_ring<18, kProbe>(a, n_tiles32, p.ibits_ring, planes);
    }
  }
  const int ibits = p.ibits;
#define GRM_SCREEN_CT(KS)                                                                        \
  switch (ct) {                                                                                  \
    case 1: return launch_screen<KS, 1, kProbe>(a, n_tiles32, p.stride, ibits, lds, planes);     \
    case 2: return launch_screen<KS, 2, kProbe>(a, n_tiles32, p.stride, ibits, lds, planes);     \
    case 4: return launch_screen<KS, 4, kProbe>(a, n_tiles32, p.stride, ibits, lds, planes);     \
    default: return launch_screen<KS, 8, kProbe>(a, n_tiles32, p.stride, ibits, lds, planes);    \
  }
  switch (p.ks) {
    case 8: GRM_SCREEN_CT(8);
    case 16: GRM_SCREEN_CT(16);
    default: GRM_SCREEN_CT(18);
  }
#undef GRM_SCREEN_CT
}

// Screen-bound constants: gamma bounds the fp32 accumulation of 16*ks
// products in 32x32x16 steps (with the MFMA's internal order unknown),
// delta the rounding of an fp32 query to bf16.
double batch_gamma(const BatchPlan& p) { return 2.0 * (16.0 * p.ks + 2.0 * p.ks) * ldexp(1.0, -24); }
double batch_delta(int q_dtype) { return q_dtype == kF32 ? ldexp(1.0, -8) : 0.0; }

// LDS of a screen pass of qp queries: the staged queries, later the
// block's result rows.
size_t batch_lds(const BatchPlan& p, int qp) {
  return std::max(static_cast<size_t>(qp) * p.stride * 2,
                  static_cast<size_t>(grm::mla::kEntryPlanes) * qp * grm::mla::kBatchWaves * 4);
}

// One pass: queries [0, qc) at q (device, dim values each) through the
// screen and the merge; results at out[0, qc*topk), certificates at
// status[0, qc).  ev (optional) is a pair of events recorded around the
// screen kernel.
int enqueue_batch_pass(MlaDeviceArena* a, const BatchPlan& p, const unsigned char* q, int q_dtype,
                       int qc, int topk, Cand* out, unsigned* status, hipEvent_t* ev) {
  const int ct = qc <= 32 ? 1 : (qc <= 64 ? 2 : (qc <= 128 ? 4 : 8));
  const int qp = 32 * ct;
  grm::mla::mla_batch_qprep_kernel<<<qp, grm::kWave, 0, a->stream>>>(
      q, q_dtype, qc, a->dim, p.stride, a->d_qpad, a->d_inv_qn);
  GRM_HIP_CHECK(hipGetLastError());
  const uint32_t n_tiles32 = static_cast<uint32_t>((a->high_water + 31) / 32);
  const uint32_t n_waves = pass_subs(a, p, ct);
  const int ibits = pass_ibits(p, ct);
  const size_t lds = batch_lds(p, qp);
  if (ev) GRM_HIP_CHECK(hipEventRecord(ev[0], a->stream));
  GRM_CHECK_RC(dispatch_screen<false>(a, p, ct, n_tiles32, lds, a->d_entries));
  if (ev) GRM_HIP_CHECK(hipEventRecord(ev[1], a->stream));
  const double gamma = batch_gamma(p);
  const double delta = batch_delta(q_dtype);
  grm::mla::mla_batch_merge_kernel<<<qc, grm::mla::kMergeThreads, 0, a->stream>>>(
      a->d_entries, n_waves, qp, n_tiles32, ibits, a->d_inv_qn, a->d_tiles, a->d_norms, a->d_ids,
      a->capacity, a->dim, q, q_dtype, a->dim, gamma, delta, a->d_min_norm, topk, out, status);
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

// Completion flags a route may wait on (one per query and route block).
constexpr size_t kMaxDoneFlags = 8192;

int route_impl(MlaDeviceArena* a, const void* queries, int q_dtype,
               bool on_device, int q_count, int dim, int warmup, int topk,
               uint64_t* out_ids, float* out_scores, float* elapsed_ms) {
  if (!a || !queries || !out_ids) return grm::fail(-1, "null argument");
  if (dim != static_cast<int>(a->dim)) return grm::fail(-1, "query dim does not match bank");
  if (q_dtype != kF32 && q_dtype != kBF16) return grm::fail(-1, "query dtype must be F32 or BF16");
  if (q_count <= 0 || warmup < 0 || warmup >= q_count) {
    return grm::fail(-1, "need query_count > 0 and 0 <= warmup < query_count");
  }
  if (topk <= 0 || topk > grm::kMaxTopK || static_cast<uint64_t>(topk) > a->live) {
    return grm::fail(-1, "topk must be in [1, 16] and <= live nodes");
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  const size_t qbytes = static_cast<size_t>(q_count) * a->dim * elem_size(q_dtype);
  const SingleGeom g = single_geom(a);
  const size_t per_q = static_cast<size_t>(g.blocks) * topk;
  const unsigned char* qbase = static_cast<const unsigned char*>(queries);
  if (!on_device) {
    // through a pinned, device-mapped buffer and a copy kernel on the
    // route's stream (fetch_async), as the GQA routes take theirs
    GRM_CHECK_RC(reserve_device(reinterpret_cast<unsigned char**>(&a->d_queries),
                                &a->d_queries_bytes, qbytes));
    GRM_CHECK_RC(grm::reserve_mapped_bytes(&a->q_map, qbytes));
    memcpy(a->q_map.host, queries, qbytes);
    if (a->query_dma) {
      GRM_HIP_CHECK(hipMemcpyAsync(a->d_queries, a->q_map.host, qbytes, hipMemcpyHostToDevice, a->stream));
    } else {
      GRM_CHECK_RC(grm::fetch_async(a->d_queries, a->q_map.dev, qbytes, a->stream));
    }
    qbase = static_cast<const unsigned char*>(a->d_queries);
  }
  if (a->mut_pending) GRM_HIP_CHECK(hipStreamWaitEvent(a->stream, a->ev_mut, 0));
  const size_t qstride = static_cast<size_t>(a->dim) * elem_size(q_dtype);
  BatchPlan bp;
  const bool batched = !a->no_batch && batch_plan(a, q_count - warmup, &bp);
  a->screen_ms = 0.0f;
  std::vector<int> redo;  // queries for the single-query kernel
  if (batched) {
    GRM_CHECK_RC(reserve_device(&a->d_qpad, &a->d_qpad_count, static_cast<size_t>(bp.qp_max) * bp.stride));
    GRM_CHECK_RC(reserve_device(&a->d_inv_qn, &a->d_inv_qn_count, static_cast<size_t>(bp.qp_max)));
    GRM_CHECK_RC(reserve_device(&a->d_entries, &a->d_entries_count,
                                static_cast<size_t>(grm::mla::kEntryPlanes) * bp.qp_max * a->cus *
                                    grm::mla::kBatchWaves));
    GRM_CHECK_RC(grm::reserve_mapped(&a->batch_out, static_cast<size_t>(q_count) * topk));
    GRM_CHECK_RC(grm::reserve_mapped_bytes(&a->batch_status, static_cast<size_t>(q_count) * sizeof(unsigned)));
    unsigned* st = static_cast<unsigned*>(a->batch_status.dev);
    const int timed_passes = (q_count - warmup + bp.qp_max - 1) / bp.qp_max;
    while (a->screen_ev.size() < 2 * static_cast<size_t>(timed_passes)) {
      hipEvent_t e = nullptr;
      GRM_HIP_CHECK(hipEventCreate(&e));
      a->screen_ev.push_back(e);
    }
    const int segments[2][2] = {{0, warmup}, {warmup, q_count}};
    int tp = 0;
    for (int si = 0; si < 2; ++si) {
      if (si == 1) GRM_HIP_CHECK(hipEventRecord(a->ev_start, a->stream));
      for (int q0 = segments[si][0]; q0 < segments[si][1]; q0 += bp.qp_max) {
        const int qc = std::min(bp.qp_max, segments[si][1] - q0);
        hipEvent_t* ev = si == 1 ? &a->screen_ev[2 * tp++] : nullptr;
        GRM_CHECK_RC(enqueue_batch_pass(a, bp, qbase + q0 * qstride, q_dtype, qc, topk,
                                        a->batch_out.dev + static_cast<size_t>(q0) * topk, st + q0,
                                        ev));
        a->batch_passes += 1;
      }
    }
    GRM_HIP_CHECK(hipEventRecord(a->ev_stop, a->stream));
    GRM_CHECK_RC(grm::wait_event(a->ev_stop));
    if (elapsed_ms) GRM_HIP_CHECK(hipEventElapsedTime(elapsed_ms, a->ev_start, a->ev_stop));
    a->screen_ms = 0.0f;
    for (int i = 0; i < tp; ++i) {
      float ms = 0.0f;
      GRM_HIP_CHECK(hipEventElapsedTime(&ms, a->screen_ev[2 * i], a->screen_ev[2 * i + 1]));
      a->screen_ms += ms;
    }
    const unsigned* hs = static_cast<const unsigned*>(a->batch_status.host);
    for (int qi = 0; qi < q_count; ++qi) {
      if (hs[qi] == 1u) {
        write_cands(a->batch_out.host + static_cast<size_t>(qi) * topk, topk,
                    out_ids + static_cast<size_t>(qi) * topk,
                    out_scores ? out_scores + static_cast<size_t>(qi) * topk : nullptr);
      } else {
        redo.push_back(qi);
      }
    }
    a->batch_queries += static_cast<uint64_t>(q_count);
    a->batch_fallbacks += redo.size();
  } else {
    for (int qi = 0; qi < q_count; ++qi) redo.push_back(qi);
  }
  if (!redo.empty()) {
    a->single_queries += redo.size();
    GRM_CHECK_RC(grm::reserve_mapped(&a->blocks_out, per_q * redo.size()));
    // The host sees completion through per-block flags in host memory, as
    // soon as the last block stores its flag (no stream event on the
    // path).  A timed route without a batched pass does too when the
    // device reports its constant clock: its device time is then the
    // clock's ticks from the first timed launch's start to the last flag
    // (RouteStamps; GRM_HIP_ROUTE_TIMING=events keeps stream events).
    const size_t n_flags = static_cast<size_t>(g.blocks) * redo.size();
    const bool flaggable = n_flags <= kMaxDoneFlags && !grm::blocking_sync();
    const bool clocked =
        elapsed_ms && !batched && flaggable && a->ticks_per_ms > 0.0 && !grm::event_timing();
    const bool flags = flaggable && (!elapsed_ms || clocked);
    unsigned* d_done = nullptr;
    if (flags) {
      GRM_CHECK_RC(grm::begin_flags(&a->done_flags, kMaxDoneFlags, &a->route_seq));
      d_done = static_cast<unsigned*>(a->done_flags.dev);
    }
    if (clocked) GRM_CHECK_RC(grm::reserve_stamps(&a->stamps, kMaxDoneFlags));
    // Uncertified batched queries add their time to the timed segment.
    bool started = false;
    for (size_t j = 0; j < redo.size(); ++j) {
      const int qi = redo[j];
      grm::RouteStamps st{nullptr, nullptr};
      if (clocked) st = grm::route_stamps(a->stamps, j * g.blocks);
      if (!started && elapsed_ms && (batched || qi == warmup)) {
        if (!clocked) GRM_HIP_CHECK(hipEventRecord(a->ev_start, a->stream));
        started = true;
      } else {
        st.start = nullptr;
      }
      GRM_CHECK_RC(launch_single(a, g, qbase + qi * qstride, q_dtype, topk,
                                 a->blocks_out.dev + j * per_q,
                                 d_done ? d_done + j * g.blocks : nullptr, st));
    }
    GRM_HIP_CHECK(hipEventRecord(a->ev_stop, a->stream));
    if (flags) {
      GRM_CHECK_RC(grm::wait_flags(a->done_flags, a->route_seq, n_flags, a->ev_stop));
      GRM_CHECK_RC(grm::wait_tagged(a->blocks_out.host, per_q * redo.size(), a->route_seq, a->ev_stop));
    } else {
      GRM_CHECK_RC(grm::wait_event(a->ev_stop));
    }
    if (clocked) {
      GRM_CHECK_RC(grm::stamps_elapsed(a->stamps, a->route_seq, static_cast<size_t>(warmup) * g.blocks, n_flags,
                                       a->ev_stop, a->ticks_per_ms, elapsed_ms));
    } else if (elapsed_ms) {
      float ms = 0.0f;
      GRM_HIP_CHECK(hipEventElapsedTime(&ms, a->ev_start, a->ev_stop));
      *elapsed_ms = batched ? *elapsed_ms + ms : ms;
    }
    a->merged.resize(topk);
    for (size_t j = 0; j < redo.size(); ++j) {
      const int qi = redo[j];
      grm::host_topk_merge(a->blocks_out.host + j * per_q, per_q, topk, a->merged.data());
      write_cands(a->merged.data(), topk, out_ids + static_cast<size_t>(qi) * topk,
                  out_scores ? out_scores + static_cast<size_t>(qi) * topk : nullptr);
    }
  }
  grm::clear_error();
  return 0;
}

int stage_upload(MlaDeviceArena* a, size_t bytes, void** host, void** dev) {
  GRM_CHECK_RC(wait_mutations(a));
  GRM_CHECK_RC(reserve_pinned(reinterpret_cast<unsigned char**>(&a->h_stage),
                              &a->h_stage_bytes, bytes));
  GRM_CHECK_RC(reserve_device(reinterpret_cast<unsigned char**>(&a->d_stage),
                              &a->d_stage_bytes, bytes));
  *host = a->h_stage;
  *dev = a->d_stage;
  return 0;
}

// Route key of one latent block, core/kv_graft.py:131-142
// (latent_centroid):
//   c = latent.astype(float32).mean(0);  key = c / (||c|| + 1e-8).
// The mean follows numpy's float32 reduce over axis 0 as mean() runs it
// (with a where mask, so from the identity): the accumulator starts at
// +0.0 (an all -0 column sums to +0), rows add in order, and one fp32
// division by the token count follows.  The norm is taken in
// fp64 and rounded to fp32.  The reference's comes from a BLAS dot in fp32
// whose summation order depends on the host CPU, so the key agrees with it
// to that dot's rounding (up to dim * 2^-24 of |c|^2), not bit for bit.
// normalize = 0 writes the mean alone.
//
// Columns are split over blocks, kLatentCols per block.  A block stages
// its strip of up to kLatentRows tokens in LDS at once (16-byte loads when
// rows allow them), then thread c adds column c over those tokens in order.
// The adds of a column stay one serial chain, as the law has them.  A
// one-block kernel then takes the norm and scales the key.
constexpr int kLatentThreads = 256;
constexpr uint32_t kLatentCols = 32;
constexpr uint32_t kLatentRows = 512;  // 64 KiB of fp32 strip per pass

__global__ __launch_bounds__(kLatentThreads) void latent_mean_kernel(
    const void* __restrict__ latent, int dtype, uint64_t tokens, uint32_t dim,
    uint64_t row_stride, float* __restrict__ out) {
  __shared__ float s_strip[kLatentRows * kLatentCols];  // [row][column]
  const uint32_t c0 = blockIdx.x * kLatentCols;
  const uint32_t width = min(kLatentCols, dim - c0);
  const uint32_t esize = dtype == kF32 ? 4u : 2u;
  const uint32_t epv = 16u / esize;  // values per 16-byte load
  const bool vec = width % epv == 0 && row_stride % epv == 0 && c0 % epv == 0 &&
                   reinterpret_cast<uintptr_t>(latent) % 16 == 0;
  auto cvt = [&](uint16_t b) -> float {
    return dtype == kBF16 ? grm::bf16_to_f32(b) : static_cast<float>(__builtin_bit_cast(_Float16, b));
  };
  float acc = 0.0f;  // column c0 + threadIdx.x (threads below width)
  for (uint64_t t0 = 0; t0 < tokens; t0 += kLatentRows) {
    const uint32_t rows = static_cast<uint32_t>(min<uint64_t>(kLatentRows, tokens - t0));
    if (vec) {
      const uint32_t per_row = width / epv;
      const uint32_t nv = rows * per_row;
      constexpr int kBatch = 8;
      for (uint32_t base = 0; base < nv; base += kBatch * kLatentThreads) {
        u32x4 v[kBatch];
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const uint32_t i = base + k * kLatentThreads + threadIdx.x;
          const uint64_t e = (t0 + i / per_row) * row_stride + c0 + (i % per_row) * epv;
          v[k] = i < nv ? *reinterpret_cast<const u32x4*>(
                              static_cast<const unsigned char*>(latent) + e * esize)
                        : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int k = 0; k < kBatch; ++k) {
          const uint32_t i = base + k * kLatentThreads + threadIdx.x;
          if (i >= nv) continue;
          float* dst = s_strip + (i / per_row) * kLatentCols + (i % per_row) * epv;
          if (dtype == kF32) {
            dst[0] = __uint_as_float(v[k].x);
            dst[1] = __uint_as_float(v[k].y);
            dst[2] = __uint_as_float(v[k].z);
            dst[3] = __uint_as_float(v[k].w);
          } else {
            const uint32_t w[4] = {v[k].x, v[k].y, v[k].z, v[k].w};
#pragma unroll
            for (int q = 0; q < 8; ++q) dst[q] = cvt(static_cast<uint16_t>(w[q / 2] >> (16 * (q % 2))));
          }
        }
      }
    } else {
      for (uint32_t i = threadIdx.x; i < rows * width; i += kLatentThreads) {
        const uint32_t r = i / width, c = i % width;
        const uint64_t e = (t0 + r) * row_stride + c0 + c;
        s_strip[r * kLatentCols + c] =
            dtype == kF32 ? static_cast<const float*>(latent)[e]
                          : cvt(static_cast<const uint16_t*>(latent)[e]);
      }
    }
    __syncthreads();
    if (threadIdx.x < width) {
      float a = acc;
#pragma unroll 8
      for (uint32_t r = 0; r < rows; ++r) a += s_strip[r * kLatentCols + threadIdx.x];
      acc = a;
    }
    __syncthreads();
  }
  if (threadIdx.x < width) out[c0 + threadIdx.x] = acc / static_cast<float>(tokens);
}

__global__ __launch_bounds__(kLatentThreads) void latent_normalize_kernel(uint32_t dim,
                                                                          float* __restrict__ out) {
  __shared__ double s_ss[kLatentThreads / grm::kWave];
  double ss = 0.0;
  for (uint32_t d = threadIdx.x; d < dim; d += kLatentThreads) {
    ss += static_cast<double>(out[d]) * static_cast<double>(out[d]);
  }
  for (int off = grm::kWave / 2; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  if ((threadIdx.x & (grm::kWave - 1)) == 0) s_ss[threadIdx.x / grm::kWave] = ss;
  __syncthreads();
  double total = 0.0;
  for (int w = 0; w < kLatentThreads / grm::kWave; ++w) total += s_ss[w];
  const float denom = static_cast<float>(sqrt(total)) + 1e-8f;
  for (uint32_t d = threadIdx.x; d < dim; d += kLatentThreads) out[d] = out[d] / denom;
}

// Route filters (cpp/grm_runtime.cpp:3074-3104, every filter value known,
// bits as route_filter_bits :2793-2838): a node passes when, for each
// category c with filters (bit c of cats), its bits meet that category's
// 16-bit mask, held at shift 16c in fmask.  Slots that do not pass get a
// NaN norm, the marker the route kernels already skip; the filtered route
// reads this copy in place of the bank's norms.
__global__ void mla_filter_norms_kernel(const float* __restrict__ norms,
                                        const uint64_t* __restrict__ fbits, uint64_t n,
                                        uint64_t fmask, uint32_t cats, float* __restrict__ out) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride) {
    const uint64_t hit = fbits[i] & fmask;
    bool ok = true;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if ((cats >> c) & 1u) ok = ok && ((hit >> (16 * c)) & 0xffffull) != 0;
    }
    out[i] = ok ? norms[i] : __builtin_nanf("");
  }
}

__global__ void mla_zero_bits_kernel(const uint64_t* __restrict__ slots, uint64_t n,
                                     uint64_t* __restrict__ fbits) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride) {
    fbits[slots[i]] = 0ull;
  }
}

__global__ void mla_scatter_bits_kernel(const uint64_t* __restrict__ slot_bits, uint64_t n,
                                        uint64_t* __restrict__ fbits) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) fbits[slot_bits[2 * i]] = slot_bits[2 * i + 1];
}

// Law scores (cpp/grm_runtime.cpp:3518-3545) of listed slots: the query
// staged in fp64, its norm summed in d order (as the route kernels), and
// per slot the fp64 dot in d order, then float(dot / (qnorm * norm_f +
// 1e-8)); NaN where that is not finite or the slot is empty.  One block;
// thread i scores slots i, i + blockDim.x, ...
template <int DT>
__global__ __launch_bounds__(256) void mla_score_slots_kernel(
    const u32x4* __restrict__ tiles, const float* __restrict__ norms, size_t plane,
    uint32_t chunks, uint32_t dim, uint32_t dim_pad, const void* __restrict__ query,
    int query_dtype, const uint64_t* __restrict__ slots, uint64_t n, float* __restrict__ out) {
  constexpr int EPC = DT == kF32 ? 4 : 8;
  extern __shared__ double qd[];
  __shared__ double s_qnorm;
  grm::mla::stage_query(qd, query, query_dtype, dim, dim_pad);
  __syncthreads();
  if (threadIdx.x == 0) {
    double acc = 0.0;
    for (uint32_t d = 0; d < dim; ++d) acc = fma(qd[d], qd[d], acc);
    s_qnorm = sqrt(acc);
  }
  __syncthreads();
  const double qnorm = s_qnorm;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint64_t slot = slots[i];
    // the route kernels' own chunk fold, chunks in order (zero past dim)
    double acc = 0.0;
    for (uint32_t c = 0; c < chunks; ++c) {
      acc = grm::mla::chunk_dot<DT>(tiles[static_cast<size_t>(c) * plane + slot], qd + c * EPC,
                                    acc);
    }
    const float nrm = norms[slot];
    const float sc = static_cast<float>(acc / (qnorm * static_cast<double>(nrm) + 1.0e-8));
    out[i] = isfinite(sc) ? sc : __builtin_nanf("");
  }
}

int enqueue_latent_query(MlaDeviceArena* a, const void* d_latent, int dtype, uint64_t tokens,
                         uint64_t row_stride, int normalize, float* d_out) {
  if (!d_latent || !d_out) return grm::fail(-1, "null pointer");
  if (dtype != kF32 && dtype != kBF16 && dtype != kF16) {
    return grm::fail(-1, "latent dtype must be F32, BF16 or F16");
  }
  if (tokens == 0) return grm::fail(-1, "latent has no tokens");
  if (tokens >= (1ull << 24)) return grm::fail(-1, "token count above 2^24");
  if (row_stride == 0) row_stride = a->dim;
  if (row_stride < a->dim) return grm::fail(-1, "row stride below the bank dim");
  GRM_HIP_CHECK(hipSetDevice(a->device));
  const uint32_t dim = static_cast<uint32_t>(a->dim);
  latent_mean_kernel<<<(dim + kLatentCols - 1) / kLatentCols, kLatentThreads, 0, a->stream>>>(
      d_latent, dtype, tokens, dim, row_stride, d_out);
  GRM_HIP_CHECK(hipGetLastError());
  if (normalize) latent_normalize_kernel<<<1, kLatentThreads, 0, a->stream>>>(dim, d_out);
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

// ------------------------------------------------ allocation-free route
//
// grm_mla_hip_route_noalloc keeps the single-query kernel's per-block top-k
// lists in `scratch`, a file-scope device array, instead of memory the
// library allocates; a merge kernel then writes the k best of those lists
// straight to the caller's device outputs.  Each GPU holds its own copy of
// the array from load to process end, and host code reaches it only through
// the address hipGetSymbolAddress returns for the current device (the
// array's name in host code is a host-side stand-in, not a device address).
// Every call on one GPU shares that GPU's array, so calls on one GPU are
// serialised by a per-device mutex held from the first launch until the
// bank's stream has drained (on the error path too): two host threads
// routing different banks on one GPU take turns and each gets its own
// answer.  Queries run one after another on the bank's stream, so one
// query's lists fit the array: up to kScratchCands entries (grid blocks x
// topk; 1024 blocks x 16 at most with the default grid cap).  Each block
// writes all k of its entries before the merge reads them, so nothing in
// the array has to start at zero.
constexpr int kScratchDevices = 64;

std::mutex g_scratch_mu;
Cand* g_scratch_ptr[kScratchDevices] = {};
// Held by a call from its first launch until its stream has drained.
std::mutex g_noalloc_mu[kScratchDevices];

// Device address of this device's scratch (the device must be current).
int scratch_for(int device, Cand** out) {
  if (device < 0 || device >= kScratchDevices) return grm::fail(-1, "device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    GRM_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) return grm::fail(-1, "scratch symbol has no device address");
    g_scratch_ptr[device] = static_cast<Cand*>(p);
  }
  *out = g_scratch_ptr[device];
  return 0;
}

// k best of `count` per-block entries, written as ids and scores (unfilled:
// UINT64_MAX and NaN); one block.
__global__ __launch_bounds__(grm::kMergeWaves * grm::kWave) void mla_merge_out_kernel(
    const Cand* __restrict__ in, uint32_t count, int k, uint64_t* __restrict__ out_ids,
    float* __restrict__ out_scores) {
  __shared__ Cand s_lists[grm::kMergeWaves][grm::kMaxTopK];
  const int lane = threadIdx.x & (grm::kWave - 1);
  const int wave = threadIdx.x / grm::kWave;
  grm::WaveList G;
  grm::wl_init(G);
  grm::wl_consume_global(G, k, in, count, static_cast<uint32_t>(wave), grm::kMergeWaves);
  if (lane < grm::kMaxTopK) s_lists[wave][lane] = grm::wl_entry(G);
  __syncthreads();
  if (wave == 0) {
    grm::WaveList B;
    grm::block_merge<grm::kMergeWaves>(s_lists, k, B);
    if (lane < k) {
      const bool ok = isfinite(B.s) && B.id != kNoId;
      out_ids[lane] = ok ? B.id : kNoId;
      if (out_scores) out_scores[lane] = ok ? B.s : __builtin_nanf("");
    }
  }
}

int route_noalloc(MlaDeviceArena* a, const void* d_queries, int q_dtype, int q_count, int dim,
                  int topk, uint64_t* d_out_ids, float* d_out_scores) {
  if (!a || !d_queries || !d_out_ids) return grm::fail(-1, "null argument");
  if (dim != static_cast<int>(a->dim)) return grm::fail(-1, "query dim does not match bank");
  if (q_dtype != kF32 && q_dtype != kBF16) return grm::fail(-1, "query dtype must be F32 or BF16");
  if (q_count <= 0) return grm::fail(-1, "need query_count > 0");
  if (topk <= 0 || topk > grm::kMaxTopK || static_cast<uint64_t>(topk) > a->live) {
    return grm::fail(-1, "topk must be in [1, 16] and <= live nodes");
  }
  const SingleGeom g = single_geom(a);
  const size_t per_q = static_cast<size_t>(g.blocks) * topk;
  if (per_q > kScratchCands) {
    return grm::fail(-1, "route grid blocks x topk exceed the 16384-entry scratch");
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  Cand* lists = nullptr;
  GRM_CHECK_RC(scratch_for(a->device, &lists));
  std::lock_guard<std::mutex> hold(g_noalloc_mu[a->device]);
  const size_t qstride = static_cast<size_t>(a->dim) * elem_size(q_dtype);
  const unsigned char* qbase = static_cast<const unsigned char*>(d_queries);
  auto launch_all = [&]() -> int {
    if (a->mut_pending) GRM_HIP_CHECK(hipStreamWaitEvent(a->stream, a->ev_mut, 0));
    for (int qi = 0; qi < q_count; ++qi) {
      GRM_CHECK_RC(launch_single(a, g, qbase + qi * qstride, q_dtype, topk, lists));
      mla_merge_out_kernel<<<1, grm::kMergeWaves * grm::kWave, 0, a->stream>>>(
          lists, static_cast<uint32_t>(per_q), topk,
          d_out_ids + static_cast<size_t>(qi) * topk,
          d_out_scores ? d_out_scores + static_cast<size_t>(qi) * topk : nullptr);
      GRM_HIP_CHECK(hipGetLastError());
    }
    return 0;
  };
  const int rc = launch_all();
  // Drain before the lock is released, also when a launch failed part way:
  // kernels already queued still write this GPU's scratch.
  const hipError_t sync = hipStreamSynchronize(a->stream);
  if (rc != 0) return rc;
  GRM_HIP_CHECK(sync);
  a->single_queries += static_cast<uint64_t>(q_count);
  grm::clear_error();
  return 0;
}

}  // namespace

// ============================================================ reference ABI

extern "C" int grm_mla_cuda_arena_create(const float* rows_host, int nodes,
                                         int dim, MlaDeviceArena** out_arena) {
  if (!rows_host || !out_arena || nodes <= 0 || dim <= 0) {
    return grm::fail(-1, "invalid MLA arena arguments");
  }
  return create_arena(rows_host, kF32, static_cast<uint64_t>(nodes), dim,
                      nullptr, static_cast<uint64_t>(nodes), out_arena);
}

extern "C" int grm_mla_cuda_arena_route(MlaDeviceArena* arena,
                                        const float* queries_host,
                                        int query_count, int dim, int warmup,
                                        int topk, uint64_t* out_topk_host,
                                        float* elapsed_ms_host) {
  if (!arena || !queries_host || query_count <= 0 || dim <= 0 ||
      !elapsed_ms_host) {
    return grm::fail(-1, "invalid MLA route arguments");
  }
  return route_impl(arena, queries_host, kF32, false, query_count, dim, warmup,
                    topk, out_topk_host, nullptr, elapsed_ms_host);
}

extern "C" int grm_mla_cuda_arena_route_device(MlaDeviceArena* arena,
                                               const float* d_queries,
                                               int query_count, int dim,
                                               int warmup, int topk,
                                               uint64_t* out_topk_host,
                                               float* elapsed_ms_host) {
  if (!arena || !elapsed_ms_host) return grm::fail(-1, "invalid MLA route arguments");
  return route_impl(arena, d_queries, kF32, true, query_count, dim, warmup,
                    topk, out_topk_host, nullptr, elapsed_ms_host);
}

extern "C" int grm_mla_cuda_upload_queries(const float* host_buf,
                                           size_t num_floats,
                                           float** out_device_ptr) {
  if (!host_buf || !out_device_ptr || num_floats == 0) {
    return grm::fail(-1, "invalid upload arguments");
  }
  *out_device_ptr = nullptr;
  float* d = nullptr;
  GRM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&d), num_floats * sizeof(float)));
  hipError_t rc = hipMemcpy(d, host_buf, num_floats * sizeof(float), hipMemcpyHostToDevice);
  if (rc != hipSuccess) {
    (void)hipFree(d);
    return grm::fail_hip(rc, "hipMemcpy");
  }
  *out_device_ptr = d;
  return 0;
}

extern "C" int grm_mla_cuda_free_device_ptr(float* device_ptr) {
  if (!device_ptr) return 0;
  GRM_HIP_CHECK(hipFree(device_ptr));
  return 0;
}

extern "C" int grm_mla_cuda_arena_destroy(MlaDeviceArena* arena) {
  destroy_arena(arena);
  return 0;
}

extern "C" int grm_mla_cublas_route(const float* rows_host,
                                    const float* queries_host, int nodes,
                                    int dim, int query_count, int warmup,
                                    int topk, uint64_t* out_topk_host,
                                    float* elapsed_ms_host) {
  MlaDeviceArena* arena = nullptr;
  int rc = grm_mla_cuda_arena_create(rows_host, nodes, dim, &arena);
  if (rc != 0) return rc;
  rc = grm_mla_cuda_arena_route(arena, queries_host, query_count, dim, warmup,
                                topk, out_topk_host, elapsed_ms_host);
  const int drc = grm_mla_cuda_arena_destroy(arena);
  return rc != 0 ? rc : drc;
}

// =============================================================== extensions

extern "C" int grm_mla_hip_bank_create(const void* rows_host, int row_dtype,
                                       uint64_t nodes, int dim,
                                       const uint64_t* node_ids,
                                       uint64_t capacity,
                                       MlaDeviceArena** out_arena) {
  return create_arena(rows_host, row_dtype, nodes, dim, node_ids, capacity,
                      out_arena);
}

extern "C" int grm_mla_hip_route(MlaDeviceArena* arena, const void* queries,
                                 int query_dtype, int queries_on_device,
                                 int query_count, int dim, int warmup,
                                 int topk, uint64_t* out_ids_host,
                                 float* out_scores_host,
                                 float* elapsed_ms_host) {
  return route_impl(arena, queries, query_dtype, queries_on_device != 0,
                    query_count, dim, warmup, topk, out_ids_host,
                    out_scores_host, elapsed_ms_host);
}

extern "C" int grm_mla_hip_route_noalloc(MlaDeviceArena* arena, const void* d_queries,
                                         int query_dtype, int query_count, int dim, int topk,
                                         uint64_t* d_out_ids, float* d_out_scores) {
  return route_noalloc(arena, d_queries, query_dtype, query_count, dim, topk, d_out_ids,
                       d_out_scores);
}

extern "C" int grm_mla_hip_latent_query(MlaDeviceArena* arena, const void* d_latent,
                                        int latent_dtype, uint64_t tokens,
                                        uint64_t row_stride, int normalize, float* d_out) {
  if (!arena) return grm::fail(-1, "null arena");
  GRM_CHECK_RC(enqueue_latent_query(arena, d_latent, latent_dtype, tokens, row_stride,
                                    normalize, d_out));
  GRM_HIP_CHECK(hipStreamSynchronize(arena->stream));
  grm::clear_error();
  return 0;
}

extern "C" int grm_mla_hip_route_latent(MlaDeviceArena* arena, const void* d_latent,
                                        int latent_dtype, uint64_t tokens,
                                        uint64_t row_stride, int topk,
                                        uint64_t* out_ids_host, float* out_scores_host,
                                        float* elapsed_ms_host) {
  if (!arena) return grm::fail(-1, "null arena");
  if (!arena->d_latent_q) {
    GRM_HIP_CHECK(hipSetDevice(arena->device));
    GRM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&arena->d_latent_q),
                            static_cast<size_t>(arena->dim) * sizeof(float)));
  }
  // The key is formed on the route stream; the route that follows on the
  // same stream reads it there, with no copy to the host in between.
  GRM_CHECK_RC(enqueue_latent_query(arena, d_latent, latent_dtype, tokens, row_stride, 1,
                                    arena->d_latent_q));
  return route_impl(arena, arena->d_latent_q, kF32, true, 1, static_cast<int>(arena->dim), 0,
                    topk, out_ids_host, out_scores_host, elapsed_ms_host);
}

extern "C" int grm_mla_hip_set_filter_bits(MlaDeviceArena* a, const uint64_t* node_ids,
                                           const uint64_t* bits, uint64_t count) {
  if (!a || (count > 0 && (!node_ids || !bits))) return grm::fail(-1, "invalid arguments");
  std::vector<uint64_t> pairs;
  pairs.reserve(2 * count);
  for (uint64_t i = 0; i < count; ++i) {
    auto it = a->slot_of.find(node_ids[i]);
    if (it == a->slot_of.end()) return grm::fail(-1, "filter bits for an id that is not live");
    pairs.push_back(it->second);
    pairs.push_back(bits[i]);
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  GRM_CHECK_RC(wait_mutations(a));
  if (!a->d_fbits) {
    GRM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&a->d_fbits),
                            a->capacity * sizeof(uint64_t)));
    GRM_HIP_CHECK(hipMemsetAsync(a->d_fbits, 0, a->capacity * sizeof(uint64_t), a->stream));
  }
  if (count > 0) {
    void* h = nullptr;
    void* d = nullptr;
    GRM_CHECK_RC(stage_upload(a, pairs.size() * sizeof(uint64_t), &h, &d));
    memcpy(h, pairs.data(), pairs.size() * sizeof(uint64_t));
    GRM_HIP_CHECK(hipMemcpyAsync(d, h, pairs.size() * sizeof(uint64_t), hipMemcpyHostToDevice,
                                 a->stream));
    mla_scatter_bits_kernel<<<static_cast<unsigned>((count + 255) / 256), 256, 0, a->stream>>>(
        static_cast<const uint64_t*>(d), count, a->d_fbits);
    GRM_HIP_CHECK(hipGetLastError());
  }
  GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
  grm::clear_error();
  return 0;
}

extern "C" int grm_mla_hip_route_filtered(MlaDeviceArena* a, const void* query, int query_dtype,
                                          int query_on_device, int topk, uint64_t filter_mask,
                                          uint32_t filter_categories, uint64_t* out_ids_host,
                                          float* out_scores_host, float* elapsed_ms_host) {
  if (!a) return grm::fail(-1, "null arena");
  if (filter_categories & ~0xfu) return grm::fail(-1, "filter categories are bits 0..3");
  if (filter_categories == 0) {
    return route_impl(a, query, query_dtype, query_on_device != 0, 1, static_cast<int>(a->dim), 0,
                      topk, out_ids_host, out_scores_host, elapsed_ms_host);
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  if (!a->d_fnorms) {
    GRM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&a->d_fnorms), a->capacity * sizeof(float)));
  }
  if (!a->d_fbits) {
    // no bits set on any node: every node fails an active category
    GRM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(&a->d_fbits),
                            a->capacity * sizeof(uint64_t)));
    GRM_HIP_CHECK(hipMemsetAsync(a->d_fbits, 0, a->capacity * sizeof(uint64_t), a->stream));
  }
  if (a->mut_pending) GRM_HIP_CHECK(hipStreamWaitEvent(a->stream, a->ev_mut, 0));
  // every slot the route scans: whole 64-slot tiles up to the high water
  // (capacity is a multiple of 64; the tail slots stay NaN)
  const uint64_t n = (a->high_water + grm::kWave - 1) / grm::kWave * grm::kWave;
  if (n > 0) {
    const unsigned blocks =
        static_cast<unsigned>(std::min<uint64_t>((n + 255) / 256, static_cast<uint64_t>(a->cus) * 16));
    mla_filter_norms_kernel<<<blocks, 256, 0, a->stream>>>(a->d_norms, a->d_fbits, n, filter_mask,
                                                          filter_categories, a->d_fnorms);
    GRM_HIP_CHECK(hipGetLastError());
  }
  a->route_norms = a->d_fnorms;
  a->no_batch = true;
  const int rc = route_impl(a, query, query_dtype, query_on_device != 0, 1,
                            static_cast<int>(a->dim), 0, topk, out_ids_host, out_scores_host,
                            elapsed_ms_host);
  a->route_norms = nullptr;
  a->no_batch = false;
  return rc;
}

namespace grm {
// Whether `count` appends fit once `n_drop` live rows are evicted (the
// device store checks this before it replaces an entry's keys).
bool mla_append_fits(const MlaDeviceArena* a, uint64_t n_drop, uint64_t count) {
  const uint64_t live = a->live >= n_drop ? a->live - n_drop : 0;
  return count <= a->capacity - live;
}
}  // namespace grm

extern "C" int grm_mla_hip_score_nodes(MlaDeviceArena* a, const void* query_host,
                                       int query_dtype, const uint64_t* node_ids, uint64_t count,
                                       float* out_scores_host) {
  if (!a || !query_host || (count > 0 && (!node_ids || !out_scores_host))) {
    return grm::fail(-1, "invalid arguments");
  }
  if (query_dtype != kF32 && query_dtype != kBF16) return grm::fail(-1, "query dtype must be F32 or BF16");
  if (count == 0) return 0;
  std::vector<uint64_t> slots(count);
  for (uint64_t i = 0; i < count; ++i) {
    auto it = a->slot_of.find(node_ids[i]);
    if (it == a->slot_of.end()) return grm::fail(-1, "score of an id that is not live");
    slots[i] = it->second;
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  GRM_CHECK_RC(wait_mutations(a));
  const size_t qbytes = static_cast<size_t>(a->dim) * (query_dtype == kF32 ? 4 : 2);
  const size_t sbytes = count * sizeof(uint64_t);
  const size_t obytes = count * sizeof(float);
  const size_t q_off = 0, s_off = (qbytes + 255) / 256 * 256, o_off = s_off + (sbytes + 255) / 256 * 256;
  void* h = nullptr;
  void* d = nullptr;
  GRM_CHECK_RC(stage_upload(a, o_off + obytes, &h, &d));
  memcpy(static_cast<unsigned char*>(h) + q_off, query_host, qbytes);
  memcpy(static_cast<unsigned char*>(h) + s_off, slots.data(), sbytes);
  GRM_HIP_CHECK(hipMemcpyAsync(d, h, o_off, hipMemcpyHostToDevice, a->stream));
  auto* dq = static_cast<unsigned char*>(d) + q_off;
  auto* ds = reinterpret_cast<const uint64_t*>(static_cast<unsigned char*>(d) + s_off);
  auto* dout = reinterpret_cast<float*>(static_cast<unsigned char*>(d) + o_off);
  const size_t lds = static_cast<size_t>(a->dim_pad) * sizeof(double);
  // one thread per listed node, spread over the compute units; each block
  // stages the query itself
  const unsigned blocks = static_cast<unsigned>(
      std::min<uint64_t>((count + 255) / 256, static_cast<uint64_t>(a->cus) * 4));
  if (a->dtype == kF32) {
    mla_score_slots_kernel<kF32><<<blocks, 256, lds, a->stream>>>(a->d_tiles, a->d_norms, a->capacity,
                                                             a->chunks, a->dim, a->dim_pad, dq,
                                                             query_dtype, ds, count, dout);
  } else {
    mla_score_slots_kernel<kBF16><<<blocks, 256, lds, a->stream>>>(a->d_tiles, a->d_norms, a->capacity,
                                                              a->chunks, a->dim, a->dim_pad, dq,
                                                              query_dtype, ds, count, dout);
  }
  GRM_HIP_CHECK(hipGetLastError());
  GRM_HIP_CHECK(hipMemcpyAsync(static_cast<unsigned char*>(h) + o_off, dout, obytes,
                               hipMemcpyDeviceToHost, a->stream));
  GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
  memcpy(out_scores_host, static_cast<unsigned char*>(h) + o_off, obytes);
  grm::clear_error();
  return 0;
}

extern "C" int grm_mla_hip_append(MlaDeviceArena* a, const void* rows_host,
                                  int row_dtype, uint64_t count,
                                  const uint64_t* node_ids,
                                  uint64_t* out_epoch) {
  if (!a || (count > 0 && (!rows_host || !node_ids))) {
    return grm::fail(-1, "invalid append arguments");
  }
  if (row_dtype != a->dtype) return grm::fail(-1, "append dtype differs from bank");
  if (count == 0) {
    if (out_epoch) *out_epoch = a->epoch;
    return 0;
  }
  {
    std::unordered_map<uint64_t, int> seen;
    seen.reserve(count * 2);
    for (uint64_t i = 0; i < count; ++i) {
      if (a->slot_of.count(node_ids[i]) || !seen.emplace(node_ids[i], 1).second) {
        return grm::fail(-1, "append id already live or repeated");
      }
      if (node_ids[i] == kNoId) return grm::fail(-1, "node id UINT64_MAX is reserved");
    }
  }
  const uint64_t room = a->free_slots.size() + (a->capacity - a->high_water);
  if (count > room) return grm::fail(-3, "MLA bank capacity exceeded");
  GRM_HIP_CHECK(hipSetDevice(a->device));
  const size_t row_bytes = static_cast<size_t>(a->dim) * elem_size(a->dtype);
  const size_t bytes = count * (2 * sizeof(uint64_t) + row_bytes);
  void* h = nullptr;
  void* d = nullptr;
  GRM_CHECK_RC(stage_upload(a, bytes, &h, &d));
  uint64_t* h_slots = static_cast<uint64_t*>(h);
  uint64_t* h_ids = h_slots + count;
  unsigned char* h_rows = reinterpret_cast<unsigned char*>(h_ids + count);
  std::vector<uint64_t> taken;
  taken.reserve(count);
  for (uint64_t i = 0; i < count; ++i) {
    uint64_t slot;
    if (!a->free_slots.empty()) {
      slot = *a->free_slots.begin();
      a->free_slots.erase(a->free_slots.begin());
    } else {
      slot = a->high_water++;
    }
    h_slots[i] = slot;
    h_ids[i] = node_ids[i];
    a->slot_id[slot] = node_ids[i];
    a->slot_of[node_ids[i]] = slot;
  }
  memcpy(h_rows, rows_host, count * row_bytes);
  uint64_t* d_slots = static_cast<uint64_t*>(d);
  uint64_t* d_ids = d_slots + count;
  unsigned char* d_rows = reinterpret_cast<unsigned char*>(d_ids + count);
  GRM_HIP_CHECK(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, a->side));
  GRM_CHECK_RC(launch_place(a, d_rows, count, d_slots, d_ids, 0, a->side));
  GRM_HIP_CHECK(hipEventRecord(a->ev_mut, a->side));
  a->mut_pending = true;
  a->live += count;
  a->epoch += 1;
  if (out_epoch) *out_epoch = a->epoch;
  grm::clear_error();
  return 0;
}

extern "C" int grm_mla_hip_evict(MlaDeviceArena* a, const uint64_t* node_ids,
                                 uint64_t count, uint64_t* out_epoch) {
  if (!a || (count > 0 && !node_ids)) return grm::fail(-1, "invalid evict arguments");
  if (count == 0) {
    if (out_epoch) *out_epoch = a->epoch;
    return 0;
  }
  std::vector<uint64_t> slots;
  slots.reserve(count);
  {
    std::unordered_map<uint64_t, int> seen;
    seen.reserve(count * 2);
    for (uint64_t i = 0; i < count; ++i) {
      auto it = a->slot_of.find(node_ids[i]);
      if (it == a->slot_of.end() || !seen.emplace(node_ids[i], 1).second) {
        return grm::fail(-1, "evict id not live or repeated");
      }
      slots.push_back(it->second);
    }
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  const size_t bytes = count * sizeof(uint64_t);
  void* h = nullptr;
  void* d = nullptr;
  GRM_CHECK_RC(stage_upload(a, bytes, &h, &d));
  memcpy(h, slots.data(), bytes);
  GRM_HIP_CHECK(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, a->side));
  const unsigned threads = 256;
  const unsigned blocks = static_cast<unsigned>(std::min<uint64_t>((count + threads - 1) / threads, 1024));
  grm::mla::mla_evict_kernel<<<blocks, threads, 0, a->side>>>(
      static_cast<const uint64_t*>(d), count, a->d_norms, a->d_ids);
  GRM_HIP_CHECK(hipGetLastError());
  if (a->d_fbits) {
    // a slot reused by a later append starts with no filter bits
    mla_zero_bits_kernel<<<blocks, threads, 0, a->side>>>(static_cast<const uint64_t*>(d), count,
                                                          a->d_fbits);
    GRM_HIP_CHECK(hipGetLastError());
  }
  GRM_HIP_CHECK(hipEventRecord(a->ev_mut, a->side));
  a->mut_pending = true;
  for (uint64_t s : slots) {
    a->slot_of.erase(a->slot_id[s]);
    a->slot_id[s] = kNoId;
    a->free_slots.insert(s);
  }
  // Trailing free slots shrink the scanned range.
  while (a->high_water > 0 && a->slot_id[a->high_water - 1] == kNoId) {
    a->free_slots.erase(a->high_water - 1);
    a->high_water -= 1;
  }
  a->live -= count;
  a->epoch += 1;
  if (out_epoch) *out_epoch = a->epoch;
  grm::clear_error();
  return 0;
}

extern "C" int grm_mla_hip_sync(MlaDeviceArena* a) {
  if (!a) return grm::fail(-1, "null arena");
  GRM_HIP_CHECK(hipSetDevice(a->device));
  return wait_mutations(a);
}

extern "C" int grm_mla_hip_bank_info(MlaDeviceArena* a, uint64_t* out6) {
  if (!a || !out6) return grm::fail(-1, "null argument");
  out6[0] = a->live;
  out6[1] = a->capacity;
  out6[2] = a->high_water;
  out6[3] = a->epoch;
  out6[4] = a->dim;
  out6[5] = static_cast<uint64_t>(a->dtype);
  return 0;
}

extern "C" int grm_mla_hip_route_stats(MlaDeviceArena* a, uint64_t* out4) {
  if (!a || !out4) return grm::fail(-1, "null argument");
  out4[0] = a->batch_queries;
  out4[1] = a->batch_fallbacks;
  out4[2] = a->single_queries;
  out4[3] = a->batch_passes;
  return 0;
}

extern "C" int grm_mla_hip_screen_ms(MlaDeviceArena* a, float* ms) {
  if (!a || !ms) return grm::fail(-1, "null argument");
  *ms = a->screen_ms;
  return 0;
}

// ------------------------------------------------------- screen-bound probe
//
// Test entry: runs the batched route's screen (the same kernel, in its
// probe form) over every slot of a small bf16 bank and returns each
// screened score s~ with its query's bound B, so a test can hold
// |s~ - law score| <= B for every (query, node) pair.  Not on any route
// path; allocates its own buffers.
extern "C" int grm_mla_hip_probe_screen(MlaDeviceArena* a, const void* queries_host,
                                        int query_dtype, int query_count, float* out_values_host,
                                        double* out_bounds_host, uint64_t* out_slot_ids_host) {
  if (!a || !queries_host || !out_values_host || !out_bounds_host) {
    return grm::fail(-1, "null argument");
  }
  if (query_dtype != kF32 && query_dtype != kBF16) return grm::fail(-1, "query dtype must be F32 or BF16");
  BatchPlan p;
  if (!batch_plan(a, std::numeric_limits<int>::max(), &p)) {
    return grm::fail(-1, "bank has no batched screen (bf16 rows, dim <= 288)");
  }
  if (query_count <= 0 || query_count > p.qp_max) return grm::fail(-1, "query_count out of range");
  const int ct = query_count <= 32 ? 1 : (query_count <= 64 ? 2 : (query_count <= 128 ? 4 : 8));
  const int qp = 32 * ct;
  const uint64_t n = a->high_water;
  if (n == 0) return grm::fail(-1, "empty bank");
  if (a->capacity * static_cast<uint64_t>(qp) > (1ull << 26)) {
    return grm::fail(-1, "probe is for banks of at most 2^26 / 256 slots");
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  struct Buf {
    void* p = nullptr;
    ~Buf() {
      if (p) (void)hipFree(p);
    }
  } d_q, d_planes, d_vals, d_bounds;
  const size_t qbytes = static_cast<size_t>(query_count) * a->dim * elem_size(query_dtype);
  GRM_HIP_CHECK(hipMalloc(&d_q.p, qbytes));
  GRM_HIP_CHECK(hipMalloc(&d_planes.p, static_cast<size_t>(qp) * a->capacity * sizeof(uint32_t)));
  GRM_HIP_CHECK(hipMalloc(&d_vals.p, static_cast<size_t>(query_count) * n * sizeof(float)));
  GRM_HIP_CHECK(hipMalloc(&d_bounds.p, static_cast<size_t>(query_count) * sizeof(double)));
  GRM_CHECK_RC(reserve_device(&a->d_qpad, &a->d_qpad_count, static_cast<size_t>(p.qp_max) * p.stride));
  GRM_CHECK_RC(reserve_device(&a->d_inv_qn, &a->d_inv_qn_count, static_cast<size_t>(p.qp_max)));
  if (a->mut_pending) GRM_HIP_CHECK(hipStreamWaitEvent(a->stream, a->ev_mut, 0));
  GRM_HIP_CHECK(hipMemcpyAsync(d_q.p, queries_host, qbytes, hipMemcpyHostToDevice, a->stream));
  grm::mla::mla_batch_qprep_kernel<<<qp, grm::kWave, 0, a->stream>>>(
      d_q.p, query_dtype, query_count, a->dim, p.stride, a->d_qpad, a->d_inv_qn);
  GRM_HIP_CHECK(hipGetLastError());
  const uint32_t n_tiles32 = static_cast<uint32_t>((n + 31) / 32);
  GRM_CHECK_RC(dispatch_screen<true>(a, p, ct, n_tiles32, batch_lds(p, qp),
                                     static_cast<uint32_t*>(d_planes.p)));
  grm::mla::mla_batch_probe_finish_kernel<<<query_count, grm::kWave, 0, a->stream>>>(
      static_cast<const uint32_t*>(d_planes.p), a->capacity, static_cast<uint32_t>(n), a->d_inv_qn,
      d_q.p, query_dtype, a->dim, a->dim, batch_gamma(p), batch_delta(query_dtype), a->d_min_norm,
      pass_ibits(p, ct), static_cast<float*>(d_vals.p), static_cast<double*>(d_bounds.p));
  GRM_HIP_CHECK(hipGetLastError());
  GRM_HIP_CHECK(hipMemcpyAsync(out_values_host, d_vals.p, static_cast<size_t>(query_count) * n * sizeof(float),
                               hipMemcpyDeviceToHost, a->stream));
  GRM_HIP_CHECK(hipMemcpyAsync(out_bounds_host, d_bounds.p, static_cast<size_t>(query_count) * sizeof(double),
                               hipMemcpyDeviceToHost, a->stream));
  if (out_slot_ids_host) {
    GRM_HIP_CHECK(hipMemcpyAsync(out_slot_ids_host, a->d_ids, n * sizeof(uint64_t),
                                 hipMemcpyDeviceToHost, a->stream));
  }
  GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
  grm::clear_error();
  return 0;
}
