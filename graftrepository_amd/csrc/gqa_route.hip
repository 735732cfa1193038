// gqa_route.hip -- exact ragged GQA route on gfx950.
//
// Law (cpp/grm_runtime.cpp:2980-3029 gqa_raw_score; core/graft_arena.py:2888-2900):
//   score(node) = float( (sum_h best_h) / H )                 h ascending, fp64
//   best_h      = max over (query token qi, key token t) of |dot| / sqrt(hd)
//   dot         = sum_d (double)q[h][qi][d] * (double)k[h/R][t][d], d ascending
// A node with zero key tokens scores 0.0; any non-finite query or key value
// makes the score NaN (never ranked).  Stacked routing layers are folded
// into the head axes by the caller (kv head g of layer y -> y*KV+g).
//
// Bank layout in HBM: ragged CSR.  Node slot i owns tokens
// [tok_off[i], tok_off[i]+len[i]) of the token arena; its block is
// [kv][len][hd] values of the storage dtype (f32, bf16, f16 or int8 codes
// with per-(token, group) scales, dequantised as fp16(code*scale),
// core/graft_quant.py:136-144).  No padding is stored or read.
//
// Route = (1) head-max kernel: one wavefront per (slot, 64-token chunk, kv
// head); lane t owns one key token, computes its R*Qt dot products in the
// law's d order in fp64, and the wave folds |dot|/sqrt(hd) into the
// per-(slot, head) maximum with a 64-bit atomicMax on the bit pattern
// (non-negative doubles order like their bits, so the result does not depend
// on scheduling); (2) finalize kernel: per slot the fp64 head sum in h order,
// the fused top-k, and a re-zero of the maxima for the next call.
#include "grm_common.hpp"
#include "grm_hip_router.h"

#include <hip/hip_fp16.h>
#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <set>
#include <unordered_map>
#include <vector>

namespace grm {
namespace gqa {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;          // key tokens per head-max wavefront
constexpr int kUnitWaves = 4;       // wavefronts per head-max block
constexpr int kFinWaves = 4;        // wavefronts per finalize block
constexpr int kMaxRQ = 32;          // R * Qt supported by the exact kernel
constexpr uint32_t kMaxHeadDim = 512;

// Work item: one 64-token chunk of one slot (all kv heads).
struct Item {
  uint32_t slot;
  uint32_t t0;
};

__device__ inline float dequant_i8(int code, float scale) {
  return __half2float(__float2half(static_cast<float>(code) * scale));
}

__device__ inline float load_scale(const unsigned char* __restrict__ scales,
                                   int scale_dtype, uint64_t idx) {
  if (scale_dtype == kF16) {
    return __half2float(reinterpret_cast<const __half*>(scales)[idx]);
  }
  return reinterpret_cast<const float*>(scales)[idx];
}

// Decode the 16-byte chunk at element index `e0` of a key row into floats.
// Returns the number of elements (EPC) decoded.
template <int KDT>
__device__ inline void decode_chunk(u32x4 v, const unsigned char* __restrict__ scales,
                                    int scale_dtype, uint64_t scale_idx,
                                    float* out) {
  if constexpr (KDT == kF32) {
    out[0] = __uint_as_float(v.x);
    out[1] = __uint_as_float(v.y);
    out[2] = __uint_as_float(v.z);
    out[3] = __uint_as_float(v.w);
  } else if constexpr (KDT == kBF16) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else if constexpr (KDT == kF16) {
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      __half_raw lo, hi;
      lo.x = static_cast<unsigned short>(w[i] & 0xffffu);
      hi.x = static_cast<unsigned short>(w[i] >> 16);
      out[2 * i] = __half2float(__half(lo));
      out[2 * i + 1] = __half2float(__half(hi));
    }
  } else {
    const float s = load_scale(scales, scale_dtype, scale_idx);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int code = static_cast<int>(static_cast<int8_t>((w[i] >> (8 * b)) & 0xffu));
        out[4 * i + b] = dequant_i8(code, s);
      }
    }
  }
}

template <int KDT>
struct KeyTraits {
  static constexpr int kEsize = KDT == kF32 ? 4 : (KDT == kI8 ? 1 : 2);
  static constexpr int kEpc = 16 / kEsize;  // elements per 16-byte chunk
};

// Exact per-(slot, head) maxima.  Grid: one wavefront per (item, kv head).
// hmax[slot * H + h] holds the running max of |dot|/sqrt(hd) as double bits.
template <int KDT, int RQ>
__global__ __launch_bounds__(kUnitWaves * kWave) void gqa_exact_heads_kernel(
    const unsigned char* __restrict__ keys,
    const unsigned char* __restrict__ scales, int scale_dtype, int group_size,
    const uint64_t* __restrict__ tok_off, const uint32_t* __restrict__ lens,
    const Item* __restrict__ items, uint32_t n_items, int kv, int hd, int R,
    int Qt, const void* __restrict__ query, int q_dtype, double denom,
    unsigned long long* __restrict__ hmax, int H,
    unsigned* __restrict__ qbad) {
  using T = KeyTraits<KDT>;
  extern __shared__ double qs[];  // [kUnitWaves][RQ][hd]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const uint64_t unit = static_cast<uint64_t>(blockIdx.x) * kUnitWaves + wave;
  const bool active = unit < static_cast<uint64_t>(n_items) * kv;
  const uint32_t item_i = active ? static_cast<uint32_t>(unit / kv) : 0;
  const int g = active ? static_cast<int>(unit % kv) : 0;
  double* q = qs + static_cast<size_t>(wave) * RQ * hd;
  const int rq_used = R * Qt;

  // Stage this kv head's R*Qt query rows as doubles (rows >= R*Qt are 0).
  bool bad = false;
  for (int i = lane; i < RQ * hd; i += kWave) {
    const int rq = i / hd;
    const int d = i - rq * hd;
    double v = 0.0;
    if (active && rq < rq_used) {
      const int r = rq / Qt;
      const int qi = rq - r * Qt;
      const uint64_t src = (static_cast<uint64_t>(g * R + r) * Qt + qi) * hd + d;
      const float f = q_dtype == kBF16
                          ? bf16_to_f32(static_cast<const uint16_t*>(query)[src])
                          : static_cast<const float*>(query)[src];
      bad = bad || !isfinite(f);
      v = static_cast<double>(f);
    }
    q[i] = v;
  }
  if (__ballot(bad) != 0ull && lane == 0) atomicOr(qbad, 1u);
  __syncthreads();
  if (!active) return;

  const Item it = items[item_i];
  const uint32_t L = lens[it.slot];
  const uint32_t t = it.t0 + lane;
  const bool has = t < L;
  double acc[RQ];
#pragma unroll
  for (int j = 0; j < RQ; ++j) acc[j] = 0.0;
  if (has) {
    const uint64_t row = (tok_off[it.slot] * kv + static_cast<uint64_t>(g) * L + t);
    const u32x4* p = reinterpret_cast<const u32x4*>(keys + row * hd * T::kEsize);
    const int groups = KDT == kI8 ? hd / group_size : 1;
    for (int c = 0; c < hd / T::kEpc; ++c) {
      const u32x4 v = p[c];
      float f[T::kEpc];
      const int e0 = c * T::kEpc;
      const uint64_t sidx = KDT == kI8 ? row * groups + e0 / group_size : 0;
      decode_chunk<KDT>(v, scales, scale_dtype, sidx, f);
#pragma unroll
      for (int e = 0; e < T::kEpc; ++e) {
        const double kd = static_cast<double>(f[e]);
#pragma unroll
        for (int j = 0; j < RQ; ++j) acc[j] = fma(kd, q[j * hd + e0 + e], acc[j]);
      }
    }
  }
  // best_h over this lane's token, then over the wave's tokens.
  for (int r = 0; r < R; ++r) {
    double m = 0.0;
#pragma unroll
    for (int j = 0; j < RQ; ++j) {
      if (j / Qt == r && j < rq_used && has) {
        const double v = fabs(acc[j]) / denom;
        m = (v > m || isnan(v)) ? v : m;
      }
    }
    unsigned long long bits = __double_as_longlong(m);
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const unsigned long long o = __shfl_xor(bits, off);
      bits = o > bits ? o : bits;
    }
    if (lane == 0) atomicMax(hmax + static_cast<uint64_t>(it.slot) * H + g * R + r, bits);
  }
}

// Finalize: exact score per slot; each block writes its k best entries to
// block_out for topk_merge_kernel (which also clears the query flag).
__global__ __launch_bounds__(kFinWaves * kWave) void gqa_finalize_kernel(
    unsigned long long* __restrict__ hmax, int H, uint32_t n_slots,
    const uint32_t* __restrict__ lens, const uint32_t* __restrict__ flags,
    const uint64_t* __restrict__ ids, const unsigned* __restrict__ qbad, int k,
    Cand* __restrict__ block_out) {
  __shared__ Cand s_lists[kFinWaves][kMaxTopK];
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const bool q_bad = *qbad != 0u;
  WaveList L;
  wl_init(L);
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t base = blockIdx.x * blockDim.x + wave * kWave; base < n_slots;
       base += stride) {
    const uint32_t slot = base + lane;
    float s = __builtin_nanf("");
    bool valid = false;
    if (slot < n_slots) {
      const uint32_t f = flags[slot];
      if (f & 1u) {  // live
        const uint32_t len = lens[slot];
        if (len == 0) {
          s = 0.0f;
        } else {
          // Read and re-zero the maxima of every scored slot (NaN bits of a
          // non-finite node included) so the next call starts from zero.
          double total = 0.0;
          unsigned long long* hm = hmax + static_cast<uint64_t>(slot) * H;
          for (int h = 0; h < H; ++h) {
            total += __longlong_as_double(hm[h]);
            hm[h] = 0ull;
          }
          if ((f & 2u) && !q_bad) {  // all key and query values finite
            s = static_cast<float>(total / static_cast<double>(H));
          }
        }
        valid = isfinite(s);
      }
    }
    const bool need = valid && s >= L.th_s;
    uint64_t id = kNoId;
    if (need) id = ids[slot];
    wl_consume(L, k, s, id, slot, need);
  }
  block_topk_write<kFinWaves>(L, k, s_lists, block_out);
}

// Per-slot key statistics for appended/created slots: bit 1 of flags is set
// when every decoded key value is finite.  One wave per (item, kv head).
template <int KDT>
__global__ __launch_bounds__(kUnitWaves * kWave) void gqa_key_stats_kernel(
    const unsigned char* __restrict__ keys,
    const unsigned char* __restrict__ scales, int scale_dtype, int group_size,
    const uint64_t* __restrict__ tok_off, const uint32_t* __restrict__ lens,
    const Item* __restrict__ items, uint32_t n_items, int kv, int hd,
    uint32_t* __restrict__ nonfinite) {
  using T = KeyTraits<KDT>;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const uint64_t unit = static_cast<uint64_t>(blockIdx.x) * kUnitWaves + wave;
  if (unit >= static_cast<uint64_t>(n_items) * kv) return;
  const Item it = items[unit / kv];
  const int g = static_cast<int>(unit % kv);
  const uint32_t L = lens[it.slot];
  const uint32_t t = it.t0 + lane;
  bool bad = false;
  if (t < L) {
    const uint64_t row = (tok_off[it.slot] * kv + static_cast<uint64_t>(g) * L + t);
    const u32x4* p = reinterpret_cast<const u32x4*>(keys + row * hd * T::kEsize);
    const int groups = KDT == kI8 ? hd / group_size : 1;
    for (int c = 0; c < hd / T::kEpc; ++c) {
      float f[T::kEpc];
      const int e0 = c * T::kEpc;
      decode_chunk<KDT>(p[c], scales, scale_dtype,
                        KDT == kI8 ? row * groups + e0 / group_size : 0, f);
#pragma unroll
      for (int e = 0; e < T::kEpc; ++e) bad = bad || !isfinite(f[e]);
    }
  }
  if (__ballot(bad) != 0ull && lane == 0) atomicOr(nonfinite + it.slot, 1u);
}

// flags[slot] = live | finite<<1, ids/offsets/lens written for the listed
// slots (metadata arrays packed back to back in `meta`).
__global__ void gqa_set_slots_kernel(const uint64_t* __restrict__ meta,
                                     uint64_t count,
                                     uint64_t* __restrict__ tok_off,
                                     uint32_t* __restrict__ lens,
                                     uint64_t* __restrict__ ids,
                                     uint32_t* __restrict__ flags,
                                     uint32_t* __restrict__ nonfinite) {
  // meta: [count slots][count tok_off][count lens][count ids]
  for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
       i < count; i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint64_t s = meta[i];
    tok_off[s] = meta[count + i];
    lens[s] = static_cast<uint32_t>(meta[2 * count + i]);
    ids[s] = meta[3 * count + i];
    flags[s] = 0u;  // finite bit set by gqa_commit_slots_kernel
    nonfinite[s] = 0u;
  }
}

__global__ void gqa_commit_slots_kernel(const uint64_t* __restrict__ slots,
                                        uint64_t count,
                                        uint32_t* __restrict__ flags,
                                        const uint32_t* __restrict__ nonfinite) {
  for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
       i < count; i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint64_t s = slots[i];
    flags[s] = 1u | (nonfinite[s] ? 0u : 2u);
  }
}

__global__ void gqa_evict_kernel(const uint64_t* __restrict__ slots,
                                 uint64_t count, uint32_t* __restrict__ flags,
                                 uint64_t* __restrict__ ids) {
  for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
       i < count; i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    flags[slots[i]] = 0u;
    ids[slots[i]] = kNoId;
  }
}

__global__ void gqa_clear_flag_kernel(unsigned* __restrict__ flag) { *flag = 0u; }

}  // namespace gqa
}  // namespace grm

using grm::Cand;
using grm::kBF16;
using grm::kF16;
using grm::kF32;
using grm::kI8;
using grm::kNoId;
using grm::gqa::Item;

// ------------------------------------------------------------------ host side

struct GqaDeviceArena {
  int device = 0;
  int key_dtype = kF32;
  int scale_dtype = kF32;
  int group_size = 0;
  uint32_t kv = 0;
  uint32_t hd = 0;
  uint64_t cap_nodes = 0;
  uint64_t cap_tokens = 0;
  uint64_t used_tokens = 0;  // bump pointer of the token arena
  uint64_t high_water = 0;   // slots [0, high_water) may be live
  uint64_t live = 0;
  uint64_t epoch = 0;
  unsigned char* d_keys = nullptr;
  unsigned char* d_scales = nullptr;
  uint64_t* d_tok_off = nullptr;
  uint32_t* d_len = nullptr;
  uint64_t* d_ids = nullptr;
  uint32_t* d_flags = nullptr;
  uint32_t* d_nonfinite = nullptr;
  // host mirrors
  std::vector<uint64_t> tok_off;
  std::vector<uint32_t> len;
  std::vector<uint64_t> slot_id;  // kNoId when free
  std::unordered_map<uint64_t, uint64_t> slot_of;
  std::set<uint64_t> free_slots;
  // route work list, rebuilt when the epoch moves
  Item* d_items = nullptr;
  size_t d_items_count = 0;
  uint64_t n_items = 0;
  uint64_t items_epoch = ~0ull;
  unsigned long long* d_hmax = nullptr;
  size_t d_hmax_count = 0;
  int hmax_heads = 0;
  grm::MappedCands blocks_out;  // per-query, per-block top-k (host mapped)
  std::vector<Cand> merged;
  unsigned* d_qbad = nullptr;  // set when a query value is non-finite
  void* d_queries = nullptr;
  size_t d_queries_bytes = 0;
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
  uint32_t fin_blocks = 256;
};

namespace {

size_t key_esize(int dt) { return dt == kF32 ? 4 : (dt == kI8 ? 1 : 2); }
size_t scale_esize(int dt) { return dt == kF16 ? 2 : 4; }

uint64_t row_values(const GqaDeviceArena* a) { return static_cast<uint64_t>(a->kv) * a->hd; }
uint64_t scale_groups(const GqaDeviceArena* a) {
  return a->key_dtype == kI8 ? a->hd / static_cast<uint32_t>(a->group_size) : 0;
}
size_t token_key_bytes(const GqaDeviceArena* a) { return row_values(a) * key_esize(a->key_dtype); }
size_t token_scale_bytes(const GqaDeviceArena* a) {
  return a->key_dtype == kI8 ? static_cast<size_t>(a->kv) * scale_groups(a) * scale_esize(a->scale_dtype) : 0;
}

template <typename T>
int reserve_device(T** ptr, size_t* have, size_t want) {
  if (want <= *have && *ptr) return 0;
  if (*ptr) {
    GRM_HIP_CHECK(hipFree(*ptr));
    *ptr = nullptr;
    *have = 0;
  }
  GRM_HIP_CHECK(hipMalloc(reinterpret_cast<void**>(ptr), std::max<size_t>(1, want) * sizeof(T)));
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
  GRM_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(ptr), std::max<size_t>(1, want) * sizeof(T),
                              hipHostMallocDefault));
  *have = want;
  return 0;
}

void destroy_arena(GqaDeviceArena* a) {
  if (!a) return;
  (void)hipSetDevice(a->device);
  if (a->stream) (void)hipStreamSynchronize(a->stream);
  if (a->side) (void)hipStreamSynchronize(a->side);
  void* dev[] = {a->d_keys, a->d_scales, a->d_tok_off, a->d_len, a->d_ids, a->d_flags,
                 a->d_nonfinite, a->d_items, a->d_hmax, a->d_qbad, a->d_queries, a->d_stage};
  for (void* p : dev) {
    if (p) (void)hipFree(p);
  }
  grm::release_mapped(&a->blocks_out);
  if (a->h_stage) (void)hipHostFree(a->h_stage);
  if (a->ev_start) (void)hipEventDestroy(a->ev_start);
  if (a->ev_stop) (void)hipEventDestroy(a->ev_stop);
  if (a->ev_mut) (void)hipEventDestroy(a->ev_mut);
  if (a->stream) (void)hipStreamDestroy(a->stream);
  if (a->side) (void)hipStreamDestroy(a->side);
  delete a;
}

int wait_mutations(GqaDeviceArena* a) {
  if (a->mut_pending) {
    GRM_HIP_CHECK(hipEventSynchronize(a->ev_mut));
    a->mut_pending = false;
  }
  return 0;
}

std::vector<Item> make_items(const GqaDeviceArena* a, const uint64_t* slots, uint64_t count) {
  std::vector<Item> items;
  for (uint64_t i = 0; i < count; ++i) {
    const uint64_t s = slots[i];
    for (uint32_t t0 = 0; t0 < a->len[s]; t0 += grm::gqa::kChunk) {
      items.push_back(Item{static_cast<uint32_t>(s), t0});
    }
  }
  return items;
}

int launch_stats(GqaDeviceArena* a, const Item* d_items, uint64_t n_items, hipStream_t st) {
  if (n_items == 0) return 0;
  const uint64_t units = n_items * a->kv;
  const unsigned blocks = static_cast<unsigned>((units + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves);
  const unsigned threads = grm::gqa::kUnitWaves * grm::kWave;
#define GRM_STATS(KDT)                                                              \
  grm::gqa::gqa_key_stats_kernel<KDT><<<blocks, threads, 0, st>>>(                  \
      a->d_keys, a->d_scales, a->scale_dtype, a->group_size, a->d_tok_off, a->d_len, \
      d_items, static_cast<uint32_t>(n_items), static_cast<int>(a->kv),             \
      static_cast<int>(a->hd), a->d_nonfinite)
  switch (a->key_dtype) {
    case kF32: GRM_STATS(kF32); break;
    case kBF16: GRM_STATS(kBF16); break;
    case kF16: GRM_STATS(kF16); break;
    default: GRM_STATS(kI8); break;
  }
#undef GRM_STATS
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

int stage_buffers(GqaDeviceArena* a, size_t bytes, unsigned char** h, unsigned char** d) {
  GRM_CHECK_RC(wait_mutations(a));
  GRM_CHECK_RC(reserve_pinned(reinterpret_cast<unsigned char**>(&a->h_stage), &a->h_stage_bytes, bytes));
  GRM_CHECK_RC(reserve_device(reinterpret_cast<unsigned char**>(&a->d_stage), &a->d_stage_bytes, bytes));
  *h = static_cast<unsigned char*>(a->h_stage);
  *d = static_cast<unsigned char*>(a->d_stage);
  return 0;
}

// Place `count` nodes whose keys (and scales) are packed back to back in
// host memory at the bump pointer; `slots` are already assigned on the host.
// Everything runs on `st`; the staging buffer stays busy until `st` passes
// the recorded mutation event.
int place_nodes(GqaDeviceArena* a, const std::vector<uint64_t>& slots,
                const std::vector<uint64_t>& ids, const uint64_t* tok_counts,
                const void* keys_host, const void* scales_host, hipStream_t st) {
  const uint64_t count = slots.size();
  uint64_t tokens = 0;
  for (uint64_t i = 0; i < count; ++i) tokens += tok_counts[i];
  const uint64_t first_tok = a->used_tokens;
  std::vector<uint64_t> offs(count);
  {
    uint64_t t = first_tok;
    for (uint64_t i = 0; i < count; ++i) {
      offs[i] = t;
      t += tok_counts[i];
    }
  }
  const size_t kbytes = tokens * token_key_bytes(a);
  const size_t sbytes = tokens * token_scale_bytes(a);
  std::vector<Item> items;
  for (uint64_t i = 0; i < count; ++i) {
    for (uint64_t t0 = 0; t0 < tok_counts[i]; t0 += grm::gqa::kChunk) {
      items.push_back(Item{static_cast<uint32_t>(slots[i]), static_cast<uint32_t>(t0)});
    }
  }
  const size_t meta_bytes = 4 * count * sizeof(uint64_t);
  const size_t item_bytes = items.size() * sizeof(Item);
  const size_t align = 256;
  const size_t o_items = (meta_bytes + align - 1) / align * align;
  const size_t o_keys = (o_items + item_bytes + align - 1) / align * align;
  const size_t o_scales = (o_keys + kbytes + align - 1) / align * align;
  const size_t total = o_scales + sbytes;
  unsigned char* h = nullptr;
  unsigned char* d = nullptr;
  GRM_CHECK_RC(stage_buffers(a, total, &h, &d));
  uint64_t* meta = reinterpret_cast<uint64_t*>(h);
  for (uint64_t i = 0; i < count; ++i) {
    meta[i] = slots[i];
    meta[count + i] = offs[i];
    meta[2 * count + i] = tok_counts[i];
    meta[3 * count + i] = ids[i];
  }
  memcpy(h + o_items, items.data(), item_bytes);
  if (kbytes) memcpy(h + o_keys, keys_host, kbytes);
  if (sbytes) memcpy(h + o_scales, scales_host, sbytes);
  GRM_HIP_CHECK(hipMemcpyAsync(d, h, total, hipMemcpyHostToDevice, st));
  if (kbytes) {
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_keys + first_tok * token_key_bytes(a), d + o_keys, kbytes,
                                 hipMemcpyDeviceToDevice, st));
  }
  if (sbytes) {
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_scales + first_tok * token_scale_bytes(a), d + o_scales,
                                 sbytes, hipMemcpyDeviceToDevice, st));
  }
  const unsigned threads = 256;
  const unsigned blocks = static_cast<unsigned>(std::min<uint64_t>((count + threads - 1) / threads, 1024));
  grm::gqa::gqa_set_slots_kernel<<<blocks, threads, 0, st>>>(
      reinterpret_cast<const uint64_t*>(d), count, a->d_tok_off, a->d_len, a->d_ids, a->d_flags,
      a->d_nonfinite);
  GRM_HIP_CHECK(hipGetLastError());
  GRM_CHECK_RC(launch_stats(a, reinterpret_cast<const Item*>(d + o_items), items.size(), st));
  grm::gqa::gqa_commit_slots_kernel<<<blocks, threads, 0, st>>>(
      reinterpret_cast<const uint64_t*>(d), count, a->d_flags, a->d_nonfinite);
  GRM_HIP_CHECK(hipGetLastError());
  // host mirrors
  for (uint64_t i = 0; i < count; ++i) {
    const uint64_t s = slots[i];
    a->tok_off[s] = offs[i];
    a->len[s] = static_cast<uint32_t>(tok_counts[i]);
    a->slot_id[s] = ids[i];
    a->slot_of[ids[i]] = s;
  }
  a->used_tokens += tokens;
  return 0;
}

int create_arena(const void* keys, int key_dtype, const void* scales, int scale_dtype,
                 int group_size, const uint64_t* tok_offsets, uint64_t nodes, int kv_heads,
                 int head_dim, const uint64_t* node_ids, uint64_t cap_nodes, uint64_t cap_tokens,
                 GqaDeviceArena** out) {
  if (!out) return grm::fail(-1, "null output arena pointer");
  *out = nullptr;
  if (kv_heads <= 0 || head_dim <= 0 || static_cast<uint32_t>(head_dim) > grm::gqa::kMaxHeadDim) {
    return grm::fail(-1, "kv_heads must be > 0 and head_dim in [1, 512]");
  }
  if (key_dtype < kF32 || key_dtype > kI8) return grm::fail(-1, "unknown key dtype");
  const int epc = static_cast<int>(16 / key_esize(key_dtype));
  if (head_dim % epc != 0) return grm::fail(-1, "head_dim * element size must be a multiple of 16 bytes");
  if (key_dtype == kI8) {
    if (scale_dtype != kF32 && scale_dtype != kF16) return grm::fail(-1, "scale dtype must be F32 or F16");
    if (group_size <= 0 || group_size % 16 != 0 || head_dim % group_size != 0) {
      return grm::fail(-1, "group_size must divide head_dim and be a multiple of 16");
    }
    if (nodes > 0 && !scales) return grm::fail(-1, "null scales for an INT8 bank");
  }
  if (nodes > 0 && (!keys || !tok_offsets)) return grm::fail(-1, "null keys or offsets");
  if (nodes > 0 && tok_offsets[0] != 0) return grm::fail(-1, "tok_offsets[0] must be 0");
  uint64_t tokens = 0;
  std::vector<uint64_t> counts(nodes);
  for (uint64_t i = 0; i < nodes; ++i) {
    if (tok_offsets[i + 1] < tok_offsets[i]) return grm::fail(-1, "tok_offsets must be non-decreasing");
    counts[i] = tok_offsets[i + 1] - tok_offsets[i];
    if (counts[i] > 0xffffffffull) return grm::fail(-1, "node too long");
  }
  if (nodes > 0) tokens = tok_offsets[nodes];
  cap_nodes = std::max(cap_nodes, nodes);
  cap_tokens = std::max(cap_tokens, tokens);
  if (cap_nodes == 0) return grm::fail(-1, "bank needs nodes or capacity");
  if (cap_nodes >= 0xffffffffull) return grm::fail(-1, "node capacity too large");
  auto* a = new GqaDeviceArena();
  auto bail = [&](int code) {
    destroy_arena(a);
    return code;
  };
  if (hipGetDevice(&a->device) != hipSuccess) a->device = 0;
  a->key_dtype = key_dtype;
  a->scale_dtype = key_dtype == kI8 ? scale_dtype : kF32;
  a->group_size = key_dtype == kI8 ? group_size : 0;
  a->kv = static_cast<uint32_t>(kv_heads);
  a->hd = static_cast<uint32_t>(head_dim);
  a->cap_nodes = cap_nodes;
  a->cap_tokens = cap_tokens;
  a->tok_off.assign(cap_nodes, 0);
  a->len.assign(cap_nodes, 0);
  a->slot_id.assign(cap_nodes, kNoId);
  std::vector<uint64_t> ids(nodes), slots(nodes);
  a->slot_of.reserve(nodes * 2);
  for (uint64_t i = 0; i < nodes; ++i) {
    ids[i] = node_ids ? node_ids[i] : i;
    slots[i] = i;
    if (ids[i] == kNoId || !a->slot_of.emplace(ids[i], i).second) {
      return bail(grm::fail(-1, "duplicate or reserved node id"));
    }
  }
  a->slot_of.clear();
#define BAIL_HIP(expr)                                              \
  do {                                                              \
    hipError_t e_ = (expr);                                         \
    if (e_ != hipSuccess) return bail(grm::fail_hip(e_, #expr));    \
  } while (0)
  BAIL_HIP(hipStreamCreateWithFlags(&a->stream, hipStreamDefault));
  BAIL_HIP(hipStreamCreateWithFlags(&a->side, hipStreamNonBlocking));
  BAIL_HIP(hipEventCreate(&a->ev_start));
  BAIL_HIP(hipEventCreate(&a->ev_stop));
  BAIL_HIP(hipEventCreateWithFlags(&a->ev_mut, hipEventDisableTiming));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_keys), std::max<size_t>(16, cap_tokens * token_key_bytes(a))));
  if (key_dtype == kI8) {
    BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_scales), std::max<size_t>(16, cap_tokens * token_scale_bytes(a))));
  }
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_tok_off), cap_nodes * sizeof(uint64_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_len), cap_nodes * sizeof(uint32_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_ids), cap_nodes * sizeof(uint64_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_flags), cap_nodes * sizeof(uint32_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_nonfinite), cap_nodes * sizeof(uint32_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_qbad), sizeof(unsigned)));
  BAIL_HIP(hipMemsetAsync(a->d_tok_off, 0, cap_nodes * sizeof(uint64_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_len, 0, cap_nodes * sizeof(uint32_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_ids, 0xff, cap_nodes * sizeof(uint64_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_flags, 0, cap_nodes * sizeof(uint32_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_nonfinite, 0, cap_nodes * sizeof(uint32_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_qbad, 0, sizeof(unsigned), a->stream));
  BAIL_HIP(hipStreamSynchronize(a->stream));
#undef BAIL_HIP
  if (const char* env = getenv("GRM_HIP_GQA_FIN_BLOCKS")) {
    const long v = strtol(env, nullptr, 10);
    if (v >= 1 && v <= 65536) a->fin_blocks = static_cast<uint32_t>(v);
  }
  // Upload in batches of whole nodes so the pinned staging stays bounded.
  const size_t kb = token_key_bytes(a), sb = token_scale_bytes(a);
  const uint64_t batch_tokens_cap = std::max<uint64_t>(1, (256ull << 20) / std::max<size_t>(1, kb + sb));
  uint64_t i0 = 0;
  while (i0 < nodes) {
    uint64_t i1 = i0, tok = 0;
    while (i1 < nodes && (i1 == i0 || tok + counts[i1] <= batch_tokens_cap)) {
      tok += counts[i1];
      ++i1;
    }
    std::vector<uint64_t> bslots(slots.begin() + i0, slots.begin() + i1);
    std::vector<uint64_t> bids(ids.begin() + i0, ids.begin() + i1);
    const unsigned char* kptr = static_cast<const unsigned char*>(keys) + tok_offsets[i0] * kb;
    const unsigned char* sptr = scales ? static_cast<const unsigned char*>(scales) + tok_offsets[i0] * sb : nullptr;
    int rc = place_nodes(a, bslots, bids, counts.data() + i0, kptr, sptr, a->stream);
    if (rc) return bail(rc);
    if (hipStreamSynchronize(a->stream) != hipSuccess) return bail(grm::fail(-1, "create upload failed"));
    i0 = i1;
  }
  a->high_water = nodes;
  a->live = nodes;
  *out = a;
  grm::clear_error();
  return 0;
}

int ensure_items(GqaDeviceArena* a) {
  if (a->items_epoch == a->epoch && a->d_items) return 0;
  std::vector<uint64_t> live_slots;
  live_slots.reserve(a->live);
  for (uint64_t s = 0; s < a->high_water; ++s) {
    if (a->slot_id[s] != kNoId) live_slots.push_back(s);
  }
  std::vector<Item> items = make_items(a, live_slots.data(), live_slots.size());
  GRM_CHECK_RC(reserve_device(&a->d_items, &a->d_items_count, items.size()));
  if (!items.empty()) {
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_items, items.data(), items.size() * sizeof(Item),
                                 hipMemcpyHostToDevice, a->stream));
    GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
  }
  a->n_items = items.size();
  a->items_epoch = a->epoch;
  return 0;
}

int launch_exact(GqaDeviceArena* a, const void* q, int q_dtype, int H, int Qt, int rq_pad) {
  if (a->n_items == 0) return 0;
  const int R = H / static_cast<int>(a->kv);
  const uint64_t units = a->n_items * a->kv;
  const unsigned blocks = static_cast<unsigned>((units + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves);
  const unsigned threads = grm::gqa::kUnitWaves * grm::kWave;
  const size_t lds = static_cast<size_t>(grm::gqa::kUnitWaves) * rq_pad * a->hd * sizeof(double);
  const double denom = sqrt(static_cast<double>(a->hd));
#define GRM_EXACT(KDT, RQ)                                                                  \
  grm::gqa::gqa_exact_heads_kernel<KDT, RQ><<<blocks, threads, lds, a->stream>>>(          \
      a->d_keys, a->d_scales, a->scale_dtype, a->group_size, a->d_tok_off, a->d_len,       \
      a->d_items, static_cast<uint32_t>(a->n_items), static_cast<int>(a->kv),              \
      static_cast<int>(a->hd), R, Qt, q, q_dtype, denom, a->d_hmax, H, a->d_qbad)
#define GRM_EXACT_RQ(KDT)                       \
  switch (rq_pad) {                             \
    case 1: GRM_EXACT(KDT, 1); break;           \
    case 2: GRM_EXACT(KDT, 2); break;           \
    case 4: GRM_EXACT(KDT, 4); break;           \
    case 8: GRM_EXACT(KDT, 8); break;           \
    case 16: GRM_EXACT(KDT, 16); break;         \
    default: GRM_EXACT(KDT, 32); break;         \
  }
  switch (a->key_dtype) {
    case kF32: GRM_EXACT_RQ(kF32); break;
    case kBF16: GRM_EXACT_RQ(kBF16); break;
    case kF16: GRM_EXACT_RQ(kF16); break;
    default: GRM_EXACT_RQ(kI8); break;
  }
#undef GRM_EXACT_RQ
#undef GRM_EXACT
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

int route_impl(GqaDeviceArena* a, const void* queries, int q_dtype, bool on_device, int q_count,
               int H, int Qt, int warmup, int topk, uint64_t* out_ids, float* out_scores,
               float* elapsed_ms) {
  if (!a || !queries || !out_ids) return grm::fail(-1, "null argument");
  if (q_dtype != kF32 && q_dtype != kBF16) return grm::fail(-1, "query dtype must be F32 or BF16");
  if (q_count <= 0 || H <= 0 || Qt <= 0 || H % static_cast<int>(a->kv) != 0) {
    return grm::fail(-1, "need query_count, heads, tokens > 0 and heads % kv_heads == 0");
  }
  if (warmup < 0 || warmup >= q_count) return grm::fail(-1, "need 0 <= warmup < query_count");
  if (topk <= 0 || topk > grm::kMaxTopK || static_cast<uint64_t>(topk) > a->live) {
    return grm::fail(-1, "topk must be in [1, 16] and <= live nodes");
  }
  const int R = H / static_cast<int>(a->kv);
  if (R * Qt > grm::gqa::kMaxRQ) return grm::fail(-1, "(heads / kv_heads) * query_tokens above 32");
  int rq_pad = 1;
  while (rq_pad < R * Qt) rq_pad *= 2;
  if (static_cast<size_t>(grm::gqa::kUnitWaves) * rq_pad * a->hd * sizeof(double) > 65536) {
    return grm::fail(-1, "(heads / kv_heads) * query_tokens * head_dim above 2048");
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  if (a->mut_pending) GRM_HIP_CHECK(hipStreamWaitEvent(a->stream, a->ev_mut, 0));
  GRM_CHECK_RC(ensure_items(a));
  if (a->hmax_heads != H || a->d_hmax_count < a->cap_nodes * static_cast<size_t>(H)) {
    GRM_CHECK_RC(reserve_device(&a->d_hmax, &a->d_hmax_count, a->cap_nodes * static_cast<size_t>(H)));
    GRM_HIP_CHECK(hipMemsetAsync(a->d_hmax, 0, a->d_hmax_count * sizeof(unsigned long long), a->stream));
    a->hmax_heads = H;
  }
  const uint32_t n_slots = static_cast<uint32_t>(a->high_water);
  const uint32_t per_block = grm::gqa::kFinWaves * grm::kWave;
  const uint32_t fin_blocks = std::max<uint32_t>(1, std::min<uint32_t>((n_slots + per_block - 1) / per_block, a->fin_blocks));
  const size_t per_q = static_cast<size_t>(fin_blocks) * topk;
  GRM_CHECK_RC(grm::reserve_mapped(&a->blocks_out, per_q * q_count));
  const size_t qvals = static_cast<size_t>(H) * Qt * a->hd;
  const size_t qstride = qvals * (q_dtype == kF32 ? 4 : 2);
  const unsigned char* qbase = static_cast<const unsigned char*>(queries);
  if (!on_device) {
    GRM_CHECK_RC(reserve_device(reinterpret_cast<unsigned char**>(&a->d_queries), &a->d_queries_bytes,
                                qstride * q_count));
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_queries, queries, qstride * q_count, hipMemcpyHostToDevice, a->stream));
    qbase = static_cast<const unsigned char*>(a->d_queries);
  }
  for (int qi = 0; qi < q_count; ++qi) {
    if (qi == warmup) GRM_HIP_CHECK(hipEventRecord(a->ev_start, a->stream));
    const void* q = qbase + qi * qstride;
    GRM_CHECK_RC(launch_exact(a, q, q_dtype, H, Qt, rq_pad));
    grm::gqa::gqa_finalize_kernel<<<fin_blocks, per_block, 0, a->stream>>>(
        a->d_hmax, H, n_slots, a->d_len, a->d_flags, a->d_ids, a->d_qbad, topk,
        a->blocks_out.dev + static_cast<size_t>(qi) * per_q);
    GRM_HIP_CHECK(hipGetLastError());
    grm::gqa::gqa_clear_flag_kernel<<<1, 1, 0, a->stream>>>(a->d_qbad);
    GRM_HIP_CHECK(hipGetLastError());
  }
  GRM_HIP_CHECK(hipEventRecord(a->ev_stop, a->stream));
  GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
  if (elapsed_ms) GRM_HIP_CHECK(hipEventElapsedTime(elapsed_ms, a->ev_start, a->ev_stop));
  a->merged.resize(topk);
  for (int qi = 0; qi < q_count; ++qi) {
    grm::host_topk_merge(a->blocks_out.host + static_cast<size_t>(qi) * per_q, per_q, topk,
                         a->merged.data());
    for (int j = 0; j < topk; ++j) {
      const Cand& c = a->merged[j];
      const bool ok = isfinite(c.score) && c.id != kNoId;
      out_ids[static_cast<size_t>(qi) * topk + j] = ok ? c.id : kNoId;
      if (out_scores) out_scores[static_cast<size_t>(qi) * topk + j] = ok ? c.score : __builtin_nanf("");
    }
  }
  grm::clear_error();
  return 0;
}

}  // namespace

// ============================================================ reference ABI

extern "C" int grm_gqa_cuda_arena_create(const float* keys_host, int nodes, int kv_heads,
                                         int key_tokens, int head_dim,
                                         GqaDeviceArena** out_arena) {
  if (!keys_host || !out_arena || nodes <= 0 || kv_heads <= 0 || key_tokens <= 0 ||
      head_dim <= 0) {
    return grm::fail(-1, "invalid GQA arena arguments");
  }
  std::vector<uint64_t> offs(static_cast<size_t>(nodes) + 1);
  for (int i = 0; i <= nodes; ++i) offs[i] = static_cast<uint64_t>(i) * key_tokens;
  return create_arena(keys_host, kF32, nullptr, kF32, 0, offs.data(), static_cast<uint64_t>(nodes),
                      kv_heads, head_dim, nullptr, static_cast<uint64_t>(nodes), offs.back(),
                      out_arena);
}

extern "C" int grm_gqa_cuda_arena_route(GqaDeviceArena* arena, const float* queries_host,
                                        int query_count, int query_heads, int query_tokens,
                                        int warmup, int topk, uint64_t* out_topk_host,
                                        float* elapsed_ms_host) {
  if (!arena || !queries_host || query_count <= 0 || query_heads <= 0 || query_tokens <= 0 ||
      !elapsed_ms_host) {
    return grm::fail(-1, "invalid GQA route arguments");
  }
  return route_impl(arena, queries_host, kF32, false, query_count, query_heads, query_tokens,
                    warmup, topk, out_topk_host, nullptr, elapsed_ms_host);
}

extern "C" int grm_gqa_cuda_arena_route_device(GqaDeviceArena* arena, const float* d_queries,
                                               int query_count, int query_heads,
                                               int query_tokens, int warmup, int topk,
                                               uint64_t* out_topk_host, float* elapsed_ms_host) {
  if (!arena || !elapsed_ms_host) return grm::fail(-1, "invalid GQA route arguments");
  return route_impl(arena, d_queries, kF32, true, query_count, query_heads, query_tokens, warmup,
                    topk, out_topk_host, nullptr, elapsed_ms_host);
}

extern "C" int grm_gqa_cuda_upload_queries(const float* host_buf, size_t num_floats,
                                           float** out_device_ptr) {
  return grm_mla_cuda_upload_queries(host_buf, num_floats, out_device_ptr);
}

extern "C" int grm_gqa_cuda_free_device_ptr(float* device_ptr) {
  return grm_mla_cuda_free_device_ptr(device_ptr);
}

extern "C" int grm_gqa_cuda_arena_destroy(GqaDeviceArena* arena) {
  destroy_arena(arena);
  return 0;
}

extern "C" int grm_gqa_cublas_route(const float* keys_host, const float* queries_host, int nodes,
                                    int kv_heads, int key_tokens, int query_count,
                                    int query_heads, int query_tokens, int head_dim, int warmup,
                                    int topk, uint64_t* out_topk_host, float* elapsed_ms_host) {
  GqaDeviceArena* arena = nullptr;
  int rc = grm_gqa_cuda_arena_create(keys_host, nodes, kv_heads, key_tokens, head_dim, &arena);
  if (rc != 0) return rc;
  rc = grm_gqa_cuda_arena_route(arena, queries_host, query_count, query_heads, query_tokens,
                                warmup, topk, out_topk_host, elapsed_ms_host);
  const int drc = grm_gqa_cuda_arena_destroy(arena);
  return rc != 0 ? rc : drc;
}

// =============================================================== extensions

extern "C" int grm_gqa_hip_bank_create(const void* keys_host, int key_dtype,
                                       const void* scales_host, int scale_dtype, int group_size,
                                       const uint64_t* tok_offsets, uint64_t nodes, int kv_heads,
                                       int head_dim, const uint64_t* node_ids,
                                       uint64_t capacity_nodes, uint64_t capacity_tokens,
                                       GqaDeviceArena** out_arena) {
  return create_arena(keys_host, key_dtype, scales_host, scale_dtype, group_size, tok_offsets,
                      nodes, kv_heads, head_dim, node_ids, capacity_nodes, capacity_tokens,
                      out_arena);
}

extern "C" int grm_gqa_hip_route(GqaDeviceArena* arena, const void* queries, int query_dtype,
                                 int queries_on_device, int query_count, int query_heads,
                                 int query_tokens, int warmup, int topk, uint64_t* out_ids_host,
                                 float* out_scores_host, float* elapsed_ms_host) {
  return route_impl(arena, queries, query_dtype, queries_on_device != 0, query_count, query_heads,
                    query_tokens, warmup, topk, out_ids_host, out_scores_host, elapsed_ms_host);
}

extern "C" int grm_gqa_hip_append(GqaDeviceArena* a, const void* keys_host,
                                  const void* scales_host, const uint64_t* tok_counts,
                                  uint64_t count, const uint64_t* node_ids, uint64_t* out_epoch) {
  if (!a || (count > 0 && (!tok_counts || !node_ids))) return grm::fail(-1, "invalid append arguments");
  if (count == 0) {
    if (out_epoch) *out_epoch = a->epoch;
    return 0;
  }
  uint64_t tokens = 0;
  {
    std::unordered_map<uint64_t, int> seen;
    seen.reserve(count * 2);
    for (uint64_t i = 0; i < count; ++i) {
      if (node_ids[i] == kNoId || a->slot_of.count(node_ids[i]) ||
          !seen.emplace(node_ids[i], 1).second) {
        return grm::fail(-1, "append id already live, repeated or reserved");
      }
      if (tok_counts[i] > 0xffffffffull) return grm::fail(-1, "node too long");
      tokens += tok_counts[i];
    }
  }
  if (tokens > 0 && !keys_host) return grm::fail(-1, "null keys");
  if (tokens > 0 && a->key_dtype == kI8 && !scales_host) return grm::fail(-1, "null scales");
  const uint64_t room = a->free_slots.size() + (a->cap_nodes - a->high_water);
  if (count > room) return grm::fail(-3, "GQA bank node capacity exceeded");
  if (tokens > a->cap_tokens - a->used_tokens) {
    return grm::fail(-3, "GQA bank token capacity exceeded (compact or grow)");
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  std::vector<uint64_t> slots(count), ids(node_ids, node_ids + count);
  std::vector<uint64_t> taken;
  for (uint64_t i = 0; i < count; ++i) {
    if (!a->free_slots.empty()) {
      slots[i] = *a->free_slots.begin();
      a->free_slots.erase(a->free_slots.begin());
    } else {
      slots[i] = a->high_water++;
    }
  }
  GRM_CHECK_RC(place_nodes(a, slots, ids, tok_counts, keys_host, scales_host, a->side));
  GRM_HIP_CHECK(hipEventRecord(a->ev_mut, a->side));
  a->mut_pending = true;
  a->live += count;
  a->epoch += 1;
  if (out_epoch) *out_epoch = a->epoch;
  grm::clear_error();
  return 0;
}

extern "C" int grm_gqa_hip_evict(GqaDeviceArena* a, const uint64_t* node_ids, uint64_t count,
                                 uint64_t* out_epoch) {
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
  unsigned char* h = nullptr;
  unsigned char* d = nullptr;
  GRM_CHECK_RC(stage_buffers(a, count * sizeof(uint64_t), &h, &d));
  memcpy(h, slots.data(), count * sizeof(uint64_t));
  GRM_HIP_CHECK(hipMemcpyAsync(d, h, count * sizeof(uint64_t), hipMemcpyHostToDevice, a->side));
  const unsigned threads = 256;
  const unsigned blocks = static_cast<unsigned>(std::min<uint64_t>((count + threads - 1) / threads, 1024));
  grm::gqa::gqa_evict_kernel<<<blocks, threads, 0, a->side>>>(reinterpret_cast<const uint64_t*>(d),
                                                               count, a->d_flags, a->d_ids);
  GRM_HIP_CHECK(hipGetLastError());
  GRM_HIP_CHECK(hipEventRecord(a->ev_mut, a->side));
  a->mut_pending = true;
  for (uint64_t s : slots) {
    a->slot_of.erase(a->slot_id[s]);
    a->slot_id[s] = kNoId;
    a->len[s] = 0;
    a->free_slots.insert(s);
  }
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

extern "C" int grm_gqa_hip_compact(GqaDeviceArena* a) {
  if (!a) return grm::fail(-1, "null arena");
  GRM_HIP_CHECK(hipSetDevice(a->device));
  GRM_CHECK_RC(wait_mutations(a));
  // Live slots in token order; each moves down to the running offset.  The
  // destination never overlaps a later source, so in-order copies are safe
  // on one stream.
  std::vector<uint64_t> order;
  for (uint64_t s = 0; s < a->high_water; ++s) {
    if (a->slot_id[s] != kNoId) order.push_back(s);
  }
  std::sort(order.begin(), order.end(),
            [&](uint64_t x, uint64_t y) { return a->tok_off[x] < a->tok_off[y]; });
  const size_t kb = token_key_bytes(a), sb = token_scale_bytes(a);
  uint64_t dst = 0;
  std::vector<uint64_t> new_off(order.size());
  for (size_t i = 0; i < order.size(); ++i) {
    const uint64_t s = order[i];
    const uint64_t src = a->tok_off[s];
    const uint64_t n = a->len[s];
    if (src != dst && n > 0) {
      if (src - dst >= n) {
        GRM_HIP_CHECK(hipMemcpyAsync(a->d_keys + dst * kb, a->d_keys + src * kb, n * kb,
                                     hipMemcpyDeviceToDevice, a->stream));
        if (sb) {
          GRM_HIP_CHECK(hipMemcpyAsync(a->d_scales + dst * sb, a->d_scales + src * sb, n * sb,
                                       hipMemcpyDeviceToDevice, a->stream));
        }
      } else {
        // Overlapping move: copy token by token in ascending order.
        for (uint64_t t = 0; t < n; ++t) {
          GRM_HIP_CHECK(hipMemcpyAsync(a->d_keys + (dst + t) * kb, a->d_keys + (src + t) * kb, kb,
                                       hipMemcpyDeviceToDevice, a->stream));
          if (sb) {
            GRM_HIP_CHECK(hipMemcpyAsync(a->d_scales + (dst + t) * sb, a->d_scales + (src + t) * sb,
                                         sb, hipMemcpyDeviceToDevice, a->stream));
          }
        }
      }
    }
    new_off[i] = dst;
    dst += n;
  }
  for (size_t i = 0; i < order.size(); ++i) a->tok_off[order[i]] = new_off[i];
  GRM_HIP_CHECK(hipMemcpyAsync(a->d_tok_off, a->tok_off.data(), a->cap_nodes * sizeof(uint64_t),
                               hipMemcpyHostToDevice, a->stream));
  GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
  a->used_tokens = dst;
  a->epoch += 1;
  grm::clear_error();
  return 0;
}

extern "C" int grm_gqa_hip_sync(GqaDeviceArena* a) {
  if (!a) return grm::fail(-1, "null arena");
  GRM_HIP_CHECK(hipSetDevice(a->device));
  return wait_mutations(a);
}

extern "C" int grm_gqa_hip_bank_info(GqaDeviceArena* a, uint64_t* out8) {
  if (!a || !out8) return grm::fail(-1, "null argument");
  out8[0] = a->live;
  out8[1] = a->cap_nodes;
  out8[2] = a->used_tokens;
  out8[3] = a->cap_tokens;
  out8[4] = a->epoch;
  out8[5] = a->kv;
  out8[6] = a->hd;
  out8[7] = static_cast<uint64_t>(a->key_dtype);
  return 0;
}
