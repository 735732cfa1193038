// grm_common.hpp -- shared pieces of the gfx950 GRM route library:
// error plumbing, the ranked-candidate type, the tie law, and the wave-wide
// top-k list every route kernel uses.
//
// Tie law (cpp/grm_runtime.cpp:75-82, score_node_better): higher score first,
// equal scores by lower node id; non-finite scores never enter a ranking
// (scripts/grm_mla_cuda_probe.py:136-152).
#pragma once

#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include <string>

namespace grm {

constexpr int kWave = 64;
constexpr int kMaxTopK = 16;
constexpr uint64_t kNoId = ~0ull;
constexpr uint32_t kNoSlot = 0xffffffffu;

enum Dtype : int { kF32 = 0, kBF16 = 1, kF16 = 2, kI8 = 3 };

// ------------------------------------------------------------------ errors

void set_error(const std::string& msg);
void clear_error();

inline int hip_code(hipError_t rc) {
  return rc == hipSuccess ? 0 : 1000 + static_cast<int>(rc);
}

int fail(int code, const char* what);
int fail_hip(hipError_t rc, const char* what);

#define GRM_HIP_CHECK(expr)                                       \
  do {                                                            \
    hipError_t grm_rc_ = (expr);                                  \
    if (grm_rc_ != hipSuccess) return ::grm::fail_hip(grm_rc_, #expr); \
  } while (0)

#define GRM_CHECK_RC(expr)                \
  do {                                    \
    int grm_rc2_ = (expr);                \
    if (grm_rc2_ != 0) return grm_rc2_;   \
  } while (0)

// ------------------------------------------------------------- candidates

// One ranked entry: score, bank slot, node id (16 bytes).
struct Cand {
  float score;
  uint32_t slot;
  uint64_t id;
};
static_assert(sizeof(Cand) == 16, "Cand must stay 16 bytes");

__host__ __device__ inline bool better(float s, uint64_t id, float ts,
                                       uint64_t tid) {
  return s > ts || (s == ts && id < tid);
}

__device__ inline float bf16_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// --------------------------------------------------------- wave top-k list
//
// A sorted list of `k` entries distributed over one wavefront: lane j < k
// holds entry j (best first).  `th_*` caches entry k-1, the bar a new
// candidate must beat; it is wave-uniform.
struct WaveList {
  float s;
  uint32_t slot;
  uint64_t id;
  float th_s;
  uint64_t th_id;
};

__device__ inline void wl_init(WaveList& L) {
  L.s = -INFINITY;
  L.slot = kNoSlot;
  L.id = kNoId;
  L.th_s = -INFINITY;
  L.th_id = kNoId;
}

// Wave-uniform copies of lane `src` (src must be wave-uniform).
__device__ inline float lane_f32(float v, int src) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), src));
}
__device__ inline uint32_t lane_u32(uint32_t v, int src) {
  return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), src));
}
__device__ inline uint64_t lane_u64(uint64_t v, int src) {
  const uint32_t lo = lane_u32(static_cast<uint32_t>(v), src);
  const uint32_t hi = lane_u32(static_cast<uint32_t>(v >> 32), src);
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

__device__ inline void wl_refresh(WaveList& L, int k) {
  L.th_s = lane_f32(L.s, k - 1);
  L.th_id = lane_u64(L.id, k - 1);
}

// Cross-lane moves through the VALU's data-parallel primitives (gfx9 DPP
// encodings) instead of LDS permutes: a lane whose source row is masked
// off keeps its own value.  Every lane of the wavefront must be active.
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(static_cast<int>(v), static_cast<int>(v), kCtrl, kRowMask, 0xf, false));
}
template <int kCtrl, int kRowMask = 0xf>
__device__ __forceinline__ float dpp_f32(float v) {
  return __uint_as_float(dpp_u32<kCtrl, kRowMask>(__float_as_uint(v)));
}

// Largest v over the wavefront (wave-uniform): quad swaps (lanes ^1, ^2),
// rotations by 4 and 8 within each row of 16, then rows 0 -> 1 and 2 -> 3
// (row broadcast of lane 15) and rows 0-1 -> 2-3 (of lane 31), so lane
// 63 ends with the maximum.
__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, dpp_f32<0xb1>(v));        // quad_perm [1,0,3,2]
  v = fmaxf(v, dpp_f32<0x4e>(v));        // quad_perm [2,3,0,1]
  v = fmaxf(v, dpp_f32<0x124>(v));       // row_ror:4
  v = fmaxf(v, dpp_f32<0x128>(v));       // row_ror:8
  v = fmaxf(v, dpp_f32<0x142, 0xa>(v));  // row_bcast:15 into rows 1, 3
  v = fmaxf(v, dpp_f32<0x143, 0xc>(v));  // row_bcast:31 into rows 2, 3
  return lane_f32(v, kWave - 1);
}

// Lane l gets v of lane l - 1 (wave_shr:1; lane 0 keeps its own).
__device__ __forceinline__ uint32_t wave_shr1_u32(uint32_t v) { return dpp_u32<0x138>(v); }

// Offer one candidate per lane (`valid` lanes only) and keep the best k of
// list + candidates.  Each iteration extracts the best remaining candidate
// (a max-reduction of the scores, then the lowest id among lanes holding
// that score) and inserts it, so the loop runs at most k times and not at
// all once no lane beats the bar.
__device__ inline void wl_consume(WaveList& L, int k, float s, uint64_t id,
                                  uint32_t slot, bool valid) {
  const int lane = __lane_id();
  bool cand = valid && better(s, id, L.th_s, L.th_id);
  uint64_t mask = __ballot(cand);
  while (mask != 0ull) {
    int bl;
    if (__popcll(mask) == 1) {
      bl = __ffsll(static_cast<long long>(mask)) - 1;
    } else {
      const float bs = wave_max_f32(cand ? s : -INFINITY);
      const uint64_t tie = __ballot(cand && s == bs);
      if (__popcll(tie) == 1) {
        bl = __ffsll(static_cast<long long>(tie)) - 1;
      } else {
        uint64_t bid = (cand && s == bs) ? id : kNoId;
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
          const uint64_t o = __shfl_xor(bid, off);
          bid = o < bid ? o : bid;
        }
        bl = __ffsll(static_cast<long long>(__ballot(cand && s == bs && id == bid))) - 1;
      }
    }
    const float ws = lane_f32(s, bl);
    const uint64_t wid = lane_u64(id, bl);
    const uint32_t wslot = lane_u32(slot, bl);
    // Entries ahead of the winner form a prefix of the sorted list.
    const bool ahead = lane < k && better(L.s, L.id, ws, wid);
    const int pos = __popcll(__ballot(ahead));
    const float ps = __uint_as_float(wave_shr1_u32(__float_as_uint(L.s)));
    const uint64_t pid = (static_cast<uint64_t>(wave_shr1_u32(static_cast<uint32_t>(L.id >> 32))) << 32) |
                         wave_shr1_u32(static_cast<uint32_t>(L.id));
    const uint32_t pslot = wave_shr1_u32(L.slot);
    if (lane == pos) {
      L.s = ws;
      L.id = wid;
      L.slot = wslot;
    } else if (lane > pos && lane < k) {
      L.s = ps;
      L.id = pid;
      L.slot = pslot;
    }
    wl_refresh(L, k);
    if (lane == bl) cand = false;
    cand = cand && better(s, id, L.th_s, L.th_id);
    mask = __ballot(cand);
  }
}

__device__ inline Cand wl_entry(const WaveList& L) {
  Cand c;
  c.score = L.s;
  c.slot = L.slot;
  c.id = L.id;
  return c;
}

// Merge the per-wave lists of a block (written to `lists[wave][0..k)`) into
// wave 0's list.  Caller synchronises the block before and reads the result
// from wave 0 after.
template <int NW, int CAP>
__device__ inline void block_merge(Cand (*lists)[CAP], int k, WaveList& out) {
  const int lane = __lane_id();
  wl_init(out);
  for (int base = 0; base < NW * k; base += kWave) {
    const int i = base + lane;
    const bool v = i < NW * k;
    Cand c;
    c.score = -INFINITY;
    c.slot = kNoSlot;
    c.id = kNoId;
    if (v) c = lists[i / k][i % k];
    wl_consume(out, k, c.score, c.id, c.slot, v && isfinite(c.score));
  }
}

// Consume `count` candidates from global memory into the list (one wave,
// strided by `stride_waves` waves starting at wave index `w`).
__device__ inline void wl_consume_global(WaveList& L, int k,
                                         const Cand* __restrict__ src,
                                         uint32_t count, uint32_t w,
                                         uint32_t stride_waves) {
  // Up to kPrefetch candidates per lane are loaded before any is consumed so
  // the loads overlap instead of paying one memory latency per 64 entries.
  constexpr int kPrefetch = 8;
  const int lane = __lane_id();
  const uint32_t step = stride_waves * kWave;
  for (uint32_t base = w * kWave; base < count; base += step * kPrefetch) {
    Cand c[kPrefetch];
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) {
      const uint32_t i = base + p * step + lane;
      c[p].score = -INFINITY;
      c[p].slot = kNoSlot;
      c[p].id = kNoId;
      if (i < count) c[p] = src[i];
    }
#pragma unroll
    for (int p = 0; p < kPrefetch; ++p) {
      if (base + p * step < count) {
        wl_consume(L, k, c[p].score, c[p].id, c[p].slot, isfinite(c[p].score));
      }
    }
  }
}


// Tag of route number `seq` in the slot field of a host-bound list entry
// (store_entry): the high bit keeps it apart from every real slot (all
// below 2^31) and from kNoSlot, so an entry of an earlier route, tagged or
// not, never carries the current route's tag (for 2^30 routes in a row).
__host__ __device__ constexpr uint32_t route_tag(unsigned seq) {
  return 0x80000000u | (seq & 0x3FFFFFFFu);
}

// A list entry bound for host memory on the completion-flag path, as one
// 16-byte store, its slot field replaced by `tag` (route_tag): the host
// takes an entry only once it carries the tag (wait_tagged), as it may see
// a block's flag before that block's earlier stores to other lines.  Host
// code never reads the slot of such an entry.  With tag kNoSlot the entry
// is stored as it is.
__device__ inline void store_entry(Cand* __restrict__ dst, Cand c, uint32_t tag) {
  if (tag != kNoSlot) c.slot = tag;
  typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));
  u32x4_t v;
  v.x = __float_as_uint(c.score);
  v.y = c.slot;
  v.z = static_cast<uint32_t>(c.id);
  v.w = static_cast<uint32_t>(c.id >> 32);
  *reinterpret_cast<u32x4_t*>(dst) = v;
}

// Block epilogue shared by the route kernels: merge the block's wave lists
// in LDS and write the block's k best entries to block_out[blockIdx.x*k ..)
// (tagged with `tag` unless it is kNoSlot, store_entry).  Must be reached
// by every thread of the block.  Device-side lists are merged by
// topk_merge_kernel, launched next on the same stream; the kernel boundary
// orders the writes, so no device-scope fence (an L2 write-back on gfx950)
// is paid per block.
template <int NW, int CAP>
__device__ inline void block_topk_write(WaveList& L, int k,
                                        Cand (*s_lists)[CAP],
                                        Cand* __restrict__ block_out,
                                        uint32_t tag = kNoSlot) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  if (lane < CAP) s_lists[wave][lane] = wl_entry(L);
  __syncthreads();
  if (wave == 0) {
    WaveList B;
    block_merge<NW>(s_lists, k, B);
    if (lane < k) store_entry(block_out + static_cast<size_t>(blockIdx.x) * k + lane, wl_entry(B), tag);
  }
}

// Device-clock stamps of a timed route that reports completion through
// flags, in host-mapped memory (null pointers when the route is untimed
// or timed by stream events): the route's first timed kernel stores its
// start tick and the route's number at start[0], start[1]
// (route_start_stamp); each block that stores a completion flag first
// stores its end tick at end[flag index].  The clock is the device's
// constant-rate one (wall_clock64), so the difference is device time
// whatever the shader clock does.
struct RouteStamps {
  unsigned long long* start;
  unsigned long long* end;
};

// Start tick of a route: the grid's first block (blocks start in index
// order) stores it as the kernel begins, with the route's number in the
// same 16-byte store, so a host that reads the number reads the tick.
__device__ inline void route_start_stamp(const RouteStamps& st, unsigned seq) {
  if (st.start && blockIdx.x == 0 && blockIdx.y == 0 && threadIdx.x == 0) {
    typedef unsigned long long u64x2_t __attribute__((ext_vector_type(2)));
    u64x2_t v;
    v.x = wall_clock64();
    v.y = seq;
    *reinterpret_cast<u64x2_t*>(st.start) = v;
  }
}

// Completion flag of a block whose list went to host-mapped memory (after
// block_topk_write, where wave 0 wrote the list): once wave 0's stores are
// complete it stores seq at done[blockIdx.x], after its end tick at
// end[blockIdx.x] when `end` is given.  No-op when done is null.
__device__ inline void block_done_flag(unsigned* __restrict__ done, unsigned seq,
                                       unsigned long long* __restrict__ end = nullptr) {
  if (done && threadIdx.x < kWave) {
    if (end && threadIdx.x == 0) end[blockIdx.x] = wall_clock64();
    __threadfence_system();
    if (threadIdx.x == 0) done[blockIdx.x] = seq;
  }
}

constexpr int kMergeWaves = 4;

// Host side: keep the best k of `count` candidates (tie law above) in out,
// best first; unfilled entries get score NaN, id kNoId, slot kNoSlot.
void host_topk_merge(const Cand* in, size_t count, int k, Cand* out);

// Wait until `ev` has completed by polling it: a route's result is read
// the moment its last kernel ends instead of after a blocking wake-up.
// With GRM_HIP_BLOCKING_SYNC=1 in the environment the wait blocks instead.
int wait_event(hipEvent_t ev);
// True when GRM_HIP_BLOCKING_SYNC=1 asks for blocking waits.
bool blocking_sync();


// Pinned host buffer of raw bytes that the device reads and writes directly
// (mapped, coherent).
struct MappedBuf {
  void* host = nullptr;
  void* dev = nullptr;
  size_t bytes = 0;
};
int reserve_mapped_bytes(MappedBuf* m, size_t bytes);
void release_mapped_bytes(MappedBuf* m);

// Completion flags in host-mapped memory: a route kernel's blocks store
// the route's number there once their results are in host memory
// (block_done_flag), and the host waits on the flags instead of a stream
// event.  begin_flags puts a buffer of `max` flags in place (zeroed when
// new) and advances *seq to the route's number (never 0); wait_flags
// polls flags [0, n) until all hold seq, checking `ev` (recorded after the
// route's kernels) now and then, so a route whose kernels fail or store no
// flags returns an error instead of spinning.
int begin_flags(MappedBuf* buf, size_t max, unsigned* seq);
int wait_flags(const MappedBuf& buf, unsigned seq, size_t n, hipEvent_t ev);
// After wait_flags: wait until each of the n host-mapped list entries at
// `entries` carries route_tag(seq) in its slot field (store_entry), so no
// entry of an earlier route is read; an error if `ev` (recorded after the
// route's kernels) completes and an entry still lacks the tag.
int wait_tagged(const Cand* entries, size_t n, unsigned seq, hipEvent_t ev);

// Device-clock timing of a flagged route (RouteStamps).  reserve_stamps
// puts a buffer in place for `max` flags: two start words, then one end
// tick per flag; route_stamps gives the device pointers, with the end
// ticks from flag `first` on.  stamps_elapsed, once wait_flags has seen
// flags [0, n) hold seq, gives the route's device time in ms: the latest
// end tick of the timed flags [first, n) less the start tick, at
// `ticks_per_ms`.  As with list entries, the host may see a flag before
// the stores ahead of it: a start stamp of another route, or a timed end
// tick below the start tick (an earlier route's), is waited for through
// `ev` and is an error if the kernels end without the new one.
// wall_ticks_per_ms: the constant clock's rate on `device` (0 when the
// device does not report it; such routes keep stream events).
int reserve_stamps(MappedBuf* buf, size_t max);
RouteStamps route_stamps(const MappedBuf& buf, size_t first);
int stamps_elapsed(const MappedBuf& buf, unsigned seq, size_t first, size_t n, hipEvent_t ev,
                   double ticks_per_ms, float* ms);
double wall_ticks_per_ms(int device);
// True when GRM_HIP_ROUTE_TIMING=events asks timed routes to keep stream
// events (and their wait) instead of flags and the device clock; read at
// each route.
bool event_timing();

// Pinned host buffer the device writes directly (mapped, coherent): the
// route kernels leave their per-block results there so the final merge
// needs neither a merge launch nor a device-to-host copy call.
struct MappedCands {
  Cand* host = nullptr;
  Cand* dev = nullptr;
  size_t count = 0;
};
int reserve_mapped(MappedCands* m, size_t count);
void release_mapped(MappedCands* m);

// Copy `bytes` from host-mapped pinned memory (src: its device address) to
// device memory dst on `stream` with a copy kernel.  For a route's small
// per-call upload (a query) the kernel runs on the route's own queue right
// before the route's kernels; a copy engine's transfer would first be
// handed over between queues, which costs more than the transfer itself.
int fetch_async(void* dst, const void* src_mapped, size_t bytes, hipStream_t stream);

// Merge `count` candidates per query (query q reads in + q*in_stride) into
// out + q*k; one block of kMergeWaves waves per query.  Clears flags[q] when
// flags is given.  Defined in grm_common.hip.
__global__ void topk_merge_kernel(const Cand* __restrict__ in, uint32_t count,
                                  size_t in_stride, int k,
                                  Cand* __restrict__ out,
                                  unsigned* __restrict__ flags);

}  // namespace grm
