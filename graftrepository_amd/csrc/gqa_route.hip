// gqa_route.hip -- ragged GQA route on gfx950: bank lifecycle, route
// orchestration and the C ABI.  Device code lives in gqa_kernels.hpp.
//
// Bank layout in HBM: ragged CSR.  Node slot i owns token rows
// [tok_off[i], tok_off[i] + L') of the token arena, L' = len[i] rounded up
// to 8; its block holds kv * L' * hd values of the storage dtype (f32,
// bf16, f16 or int8 codes with per-(token, group) scales) as chunk planes
// per kv head: chunk c (64 bytes when the row allows) of token t of head g
// at c*L' + t within the head's block (gqa_kernels.hpp).  The rounding
// puts every 8-token run of a plane on its own 128-byte lines, so streams
// never share a line; the rows past len[i] are never read.
//
// Route (bf16 / fp16 / int8 banks, head_dim 64, 128 or 256):
//   when (heads / kv) * query_tokens <= 4 the exact path below streams the
//   bank at the HBM rate by itself; otherwise
//   prep -> screen (MFMA, all key tokens) -> select -> shortlist/certify ->
//   exact rescore of the shortlist -> exact finalize; the host merges the
//   shortlist's exact scores.  A query whose shortlist is not certified, or
//   whose values are non-finite or leave the fp16 range, is routed again
//   on the exact path, so every result follows the law.
// fp32 banks (head_dim 64, 128 or 256) keep an fp16 copy of their keys
// beside the fp32 rows: the screens read the copy, with its rounding in
// their bound, and every exact recomputation reads the fp32 rows.
// Route (other shapes): exact path over every node.
#include "gqa_kernels.hpp"
#include "grm_hip_router.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <set>
#include <unordered_map>
#include <vector>

using grm::Cand;
using grm::kBF16;
using grm::kF16;
using grm::kF32;
using grm::kI8;
using grm::kNoId;
using grm::kNoSlot;
using grm::gqa::Item;
using grm::gqa::u32x4;

// ------------------------------------------------------------------ host side

struct GqaDeviceArena {
  int device = 0;
  int key_dtype = kF32;
  int scale_dtype = kF32;
  int group_size = 0;
  uint32_t kv = 0;
  uint32_t hd = 0;
  int piece_shift = 0;  // log2 of the 16-byte pieces per plane chunk
  uint64_t cap_nodes = 0;
  uint64_t cap_tokens = 0;
  uint64_t used_tokens = 0;  // bump pointer of the token arena
  uint64_t high_water = 0;   // slots [0, high_water) may be live
  uint64_t live = 0;
  uint64_t epoch = 0;
  unsigned char* d_keys = nullptr;
  unsigned char* d_scales = nullptr;
  // fp32 banks: fp16 copy of the keys (chunks of 4 pieces) for the screens
  unsigned char* d_skeys = nullptr;
  uint64_t* d_tok_off = nullptr;
  uint32_t* d_len = nullptr;
  uint64_t* d_ids = nullptr;
  uint32_t* d_flags = nullptr;  // bit 0 live, bit 1 all key values finite
  // store route: per-slot route filter bits (host copy uploaded when it
  // changed), a filtered route's copy of the flags, and the flags a route
  // reads (d_flags unless a filtered route set its copy)
  std::vector<uint64_t> fbits;
  bool fbits_dirty = false;
  uint64_t* d_fbits = nullptr;
  size_t d_fbits_count = 0;
  uint32_t* d_fflags = nullptr;
  size_t d_fflags_count = 0;
  const uint32_t* route_flags = nullptr;
  // listed-slot scoring (grm_gqa_hip_score_nodes)
  Item* d_sitems = nullptr;
  size_t d_sitems_count = 0;
  uint32_t* d_sslots = nullptr;
  size_t d_sslots_count = 0;
  float* d_sout = nullptr;
  size_t d_sout_count = 0;
  uint32_t* d_nonfinite = nullptr;
  unsigned* d_kmax = nullptr;   // float bits: max key norm per slot
  // host mirrors
  std::vector<uint64_t> tok_off;
  std::vector<uint32_t> len;
  std::vector<uint64_t> slot_id;  // kNoId when free
  std::unordered_map<uint64_t, uint64_t> slot_of;
  std::set<uint64_t> free_slots;
  // route work list, rebuilt when the epoch moves
  // Key tokens per work item of the route passes (screen and refine, the
  // exact path): a screen-and-refine item refines its columns' best rows
  // once at its end, so longer items read fewer rows again -- 512 for
  // banks the screen reads exactly (4-token route 0.229 -> 0.214 ms p50 on
  // the 512-node bf16 bank), 256 for fp32 banks screened through their
  // fp16 copy, whose refine gathers fp32 rows per wavefront (fp32
  // hand-over 0.205 against 0.207 ms device at 512); and per candidate
  // item of the bound-and-verify exact step, which is set by the
  // candidates' tokens and measured best at 256.
  uint32_t chunk = 512;
  uint32_t cand_chunk = 256;
  Item* d_items = nullptr;
  size_t d_items_count = 0;
  // the same items by decreasing token count in 64-token classes, address
  // order within a class (screen-and-refine passes with a heavy refine)
  Item* d_items_sized = nullptr;
  size_t d_items_sized_count = 0;
  uint64_t n_items = 0;
  uint64_t n_cand_items = 0;  // the live nodes' items at cand_chunk tokens
  // one item per live node with key tokens (all of them), for the
  // screen-only pass of the bound-and-verify path
  Item* d_units = nullptr;
  size_t d_units_count = 0;
  uint64_t n_units = 0;
  uint64_t items_epoch = ~0ull;
  uint32_t max_len = 0;  // longest live node
  // per-(query, head, slot) maxima, head-major per query (double bits)
  unsigned long long* d_hmax = nullptr;
  size_t d_hmax_count = 0;
  grm::MappedCands blocks_out;  // per-query, per-block top-k (host mapped)
  // per-(query, finalize block) completion flags (host mapped) and the
  // number the last route stored there
  grm::MappedBuf done_flags;
  unsigned route_seq = 0;
  // device-clock stamps of timed routes on the flag path (host mapped),
  // and the clock's ticks per ms (0: timed routes use stream events)
  grm::MappedBuf stamps;
  double ticks_per_ms = 0.0;
  unsigned* d_qbad = nullptr;   // per (query, kv head): non-finite query value
  size_t d_qbad_count = 0;
  // exact path
  double* d_q64 = nullptr;      // query rows as doubles (gqa_q64_kernel)
  size_t d_q64_count = 0;
  // screen-and-refine path
  int screen_mode = -1;  // -1 whenever the shape allows, 0 never
  // item order of screen-and-refine passes: -1 by the pass's shape, 0
  // address (slot) order, 1 by decreasing size
  int sr_order = -1;
  // bound-and-verify path (batched queries): -1 when a pass has more than
  // 16 query columns per kv head, 0 never, 1 whenever the screen runs
  int bound_mode = -1;
  // bound and verify of one wide query: the exact check on the columns the
  // screen cannot rule out only (GRM_HIP_GQA_SPARSE=0: every column)
  bool sparse_exact = true;
  // a single query's screen-only passes take up to 128 columns each at
  // head dims up to 128 (GRM_HIP_GQA_WIDE_SMAX=0: 64)
  bool wide_smax = true;
  // ... or, with at least smax_split (2 or 4) passes of 64 columns, that
  // many passes to a launch, which streams the bank once for all of them
  // (GRM_HIP_GQA_SMAX_SPLIT=0: one launch per pass).  A 64-token query
  // (R = 4, 4 passes) measured 0.776 ms in passes of 128 and 0.726 ms split
  // 4 ways; 2 passes split 2 ways were slower than one pass of 128.
  int smax_split = 4;
  unsigned* d_hmaxf = nullptr;   // screened maxima per (query, head, q token, slot), float bits
  size_t d_hmaxf_count = 0;
  float4* d_colinfo = nullptr;   // per (kv head, column): coef, eabs, scale, bad
  size_t d_colinfo_count = 0;
  float2* d_lbub = nullptr;      // per (query, slot): score bounds
  size_t d_lbub_count = 0;
  Cand* d_blists = nullptr;      // per (query, bounds block): k best lower bounds
  size_t d_blists_count = 0;
  uint32_t* d_cslots = nullptr;  // per (query): candidate slots
  size_t d_cslots_count = 0;
  uint32_t* d_ccount = nullptr;  // per query: candidate count; [qb_max]: exact items
  size_t d_ccount_count = 0;
  Item* d_citems = nullptr;      // exact work items of the candidates
  size_t d_citems_count = 0;
  uint64_t bv_routes = 0;        // passes routed by bound and verify
  uint64_t sr_routes = 0;        // passes routed by screen and refine
  uint64_t exact_routes = 0;     // queries routed by the exact path
  std::map<std::pair<const void*, size_t>, int> resident;  // blocks per CU by (kernel, LDS bytes)
  uint64_t routes = 0;          // route calls
  std::vector<Cand> merged;
  void* d_queries = nullptr;
  size_t d_queries_bytes = 0;
  // pinned staging of host queries (the route's own; mutations stage
  // through h_stage on the side stream)
  grm::MappedBuf q_map;
  bool query_dma = false;  // GRM_HIP_QUERY_COPY=dma: copy engine instead of fetch_async
  bool query_split = true;  // fp32 queries split into two MFMA-type parts (launch_sr_pass)
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
  uint32_t fin_blocks = 1024;
  // Exact-path wavefronts; the default gives every (kv head, item) pair a
  // wavefront of its own, a smaller count makes them walk several pairs.
  uint32_t exact_waves = 1u << 30;
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

// As reserve_device, and zero-filled on (re)allocation.
template <typename T>
int reserve_device_zero(T** ptr, size_t* have, size_t want, hipStream_t st) {
  if (want <= *have && *ptr) return 0;
  GRM_CHECK_RC(reserve_device(ptr, have, want));
  GRM_HIP_CHECK(hipMemsetAsync(*ptr, 0, std::max<size_t>(1, want) * sizeof(T), st));
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
  void* dev[] = {a->d_keys,   a->d_scales,  a->d_tok_off, a->d_len,    a->d_ids,   a->d_skeys,
                 a->d_flags,  a->d_nonfinite, a->d_kmax,  a->d_items,  a->d_items_sized, a->d_hmax,
                 a->d_qbad,   a->d_queries, a->d_stage,   a->d_q64,    a->d_hmaxf,
                 a->d_colinfo, a->d_lbub,   a->d_blists,  a->d_cslots, a->d_ccount,
                 a->d_citems, a->d_units,   a->d_fbits,   a->d_fflags,  a->d_sitems,
                 a->d_sslots, a->d_sout};
  for (void* p : dev) {
    if (p) (void)hipFree(p);
  }
  grm::release_mapped(&a->blocks_out);
  grm::release_mapped_bytes(&a->done_flags);
  grm::release_mapped_bytes(&a->stamps);
  if (a->h_stage) (void)hipHostFree(a->h_stage);
  grm::release_mapped_bytes(&a->q_map);
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

// Token rows a node of `len` tokens occupies in the planes.
uint64_t padded_len(uint64_t len) { return (len + grm::gqa::kTokAlign - 1) & ~uint64_t(grm::gqa::kTokAlign - 1); }

void append_items(std::vector<Item>& items, uint32_t slot, uint64_t base, uint64_t len,
                  uint32_t chunk) {
  for (uint64_t t0 = 0; t0 < len; t0 += chunk) {
    Item it;
    it.base = base;
    it.slot = slot;
    it.t0 = static_cast<uint32_t>(t0);
    it.count = static_cast<uint32_t>(std::min<uint64_t>(chunk, len - t0));
    it.len = static_cast<uint32_t>(padded_len(len));
    it.q = 0;
    it.pad = 0;
    items.push_back(it);
  }
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
// host memory ([kv][len][hd] per node) at the bump pointer; `slots` are
// already assigned on the host.  With src_rows > 0 the host keys are a
// dense bank instead: node i's block is [kv][src_rows][hd] at
// i * kv * src_rows * hd values, of which the first len rows per kv head
// are placed.  The staging copy takes the padded row
// layout of the bank, so a staged row and its bank row share an index.
// Everything runs on `st`; the staging buffer stays busy until `st` passes
// the recorded mutation event.
int place_nodes(GqaDeviceArena* a, const std::vector<uint64_t>& slots,
                const std::vector<uint64_t>& ids, const uint64_t* tok_counts,
                const void* keys_host, const void* scales_host, hipStream_t st,
                uint64_t src_rows = 0) {
  const uint64_t count = slots.size();
  uint64_t tokens = 0;  // padded token rows
  for (uint64_t i = 0; i < count; ++i) tokens += padded_len(tok_counts[i]);
  const uint64_t first_tok = a->used_tokens;
  std::vector<uint64_t> offs(count);
  {
    uint64_t t = first_tok;
    for (uint64_t i = 0; i < count; ++i) {
      offs[i] = t;
      t += padded_len(tok_counts[i]);
    }
  }
  const size_t kbytes = tokens * token_key_bytes(a);
  const size_t sbytes = tokens * token_scale_bytes(a);
  std::vector<Item> items;
  for (uint64_t i = 0; i < count; ++i) {
    append_items(items, static_cast<uint32_t>(slots[i]), offs[i] * a->kv, tok_counts[i], 64);
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
  {
    const size_t rk = static_cast<size_t>(a->hd) * key_esize(a->key_dtype);  // bytes per key row
    const size_t rs = token_scale_bytes(a) / a->kv;                         // bytes per scale row
    const unsigned char* ksrc = static_cast<const unsigned char*>(keys_host);
    const unsigned char* ssrc = static_cast<const unsigned char*>(scales_host);
    for (uint64_t i = 0; i < count; ++i) {
      const uint64_t L = tok_counts[i], Lp = padded_len(L);
      const uint64_t row = (offs[i] - first_tok) * a->kv;
      const uint64_t Ls = src_rows ? src_rows : L;  // source rows per kv head
      for (uint32_t g = 0; g < a->kv; ++g) {
        if (L == 0) break;
        memcpy(h + o_keys + (row + g * Lp) * rk, ksrc + g * Ls * rk, L * rk);
        if (rs) {
          memcpy(h + o_scales + (row + g * Lp) * rs, ssrc, L * rs);
          ssrc += L * rs;
        }
      }
      ksrc += (src_rows || L ? a->kv : 0) * Ls * rk;
    }
  }
  GRM_HIP_CHECK(hipMemcpyAsync(d, h, total, hipMemcpyHostToDevice, st));
  const unsigned threads = 256;
  const unsigned blocks = static_cast<unsigned>(std::min<uint64_t>((count + threads - 1) / threads, 1024));
  grm::gqa::gqa_set_slots_kernel<<<blocks, threads, 0, st>>>(
      reinterpret_cast<const uint64_t*>(d), count, a->d_tok_off, a->d_len, a->d_ids, a->d_flags,
      a->d_nonfinite, a->d_kmax);
  GRM_HIP_CHECK(hipGetLastError());
  if (!items.empty()) {
    // staged rows -> chunk planes, with the key statistics
    const dim3 grid(static_cast<unsigned>((items.size() + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves),
                    a->kv);
    const unsigned pthreads = grm::gqa::kUnitWaves * grm::kWave;
#define GRM_PLACE(KDT)                                                                          \
  grm::gqa::gqa_place_kernel<KDT><<<grid, pthreads, 0, st>>>(                                    \
      reinterpret_cast<const u32x4*>(d + o_keys), d + o_scales, first_tok * a->kv, a->d_keys,    \
      a->d_scales, a->scale_dtype, a->group_size, reinterpret_cast<const Item*>(d + o_items),    \
      static_cast<uint32_t>(items.size()), static_cast<int>(a->hd), a->piece_shift,           \
      a->d_nonfinite, a->d_kmax, a->d_skeys)
    switch (a->key_dtype) {
      case kF32: GRM_PLACE(kF32); break;
      case kBF16: GRM_PLACE(kBF16); break;
      case kF16: GRM_PLACE(kF16); break;
      default: GRM_PLACE(kI8); break;
    }
#undef GRM_PLACE
    GRM_HIP_CHECK(hipGetLastError());
  }
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

// A bank from CSR host keys (tok_offsets: node i's [kv][len][hd] block at
// value tok_offsets[i] * kv * hd), or with dense_rows > 0 from a dense
// host bank of dense_rows rows per (node, kv head) of which node i keeps
// the first tok_offsets[i + 1] - tok_offsets[i] (place_nodes).
int create_arena(const void* keys, int key_dtype, const void* scales, int scale_dtype,
                 int group_size, const uint64_t* tok_offsets, uint64_t nodes, int kv_heads,
                 int head_dim, const uint64_t* node_ids, uint64_t cap_nodes, uint64_t cap_tokens,
                 GqaDeviceArena** out, uint64_t dense_rows = 0) {
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
    if (counts[i] > 0xffffffffull - 8) return grm::fail(-1, "node too long");
  }
  if (nodes > 0) tokens = tok_offsets[nodes];
  cap_nodes = std::max(cap_nodes, nodes);
  cap_tokens = std::max(cap_tokens, tokens);
  // room for the row padding of every node slot
  cap_tokens += (grm::gqa::kTokAlign - 1) * cap_nodes;
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
  {
    const size_t row_bytes = static_cast<size_t>(head_dim) * key_esize(key_dtype);
    // fp32 banks without an fp16 copy take the lane-per-token exact path,
    // which streams best from 16-byte pieces; the others read whole
    // 64-byte chunks (an fp32 bank with a copy gathers single rows for
    // its exact recomputations, one 64-byte chunk per 16 values)
    const char* env = getenv("GRM_HIP_GQA_SHADOW");
    const bool shadow = key_dtype == kF32 && (head_dim == 64 || head_dim == 128 || head_dim == 256) &&
                        !(env && env[0] == '0');
    a->piece_shift = key_dtype == kF32 && !shadow
                         ? 0
                         : (row_bytes % 64 == 0 ? 2 : (row_bytes % 32 == 0 ? 1 : 0));
  }
  a->cap_nodes = cap_nodes;
  a->cap_tokens = cap_tokens;
  a->tok_off.assign(cap_nodes, 0);
  a->len.assign(cap_nodes, 0);
  a->slot_id.assign(cap_nodes, kNoId);
  a->chunk = key_dtype == kF32 ? 256 : 512;
  if (const char* env = getenv("GRM_HIP_GQA_CHUNK")) {
    const long v = strtol(env, nullptr, 10);
    if (v >= 16 && v <= 4096 && v % 16 == 0) a->chunk = static_cast<uint32_t>(v);
  }
  if (const char* env = getenv("GRM_HIP_GQA_CAND_CHUNK")) {
    const long v = strtol(env, nullptr, 10);
    if (v >= 16 && v <= 4096 && v % 16 == 0) a->cand_chunk = static_cast<uint32_t>(v);
  }
  if (const char* env = getenv("GRM_HIP_GQA_SCREEN")) a->screen_mode = env[0] != '0' ? -1 : 0;
  if (const char* env = getenv("GRM_HIP_QUERY_COPY")) a->query_dma = strcmp(env, "dma") == 0;
  if (const char* env = getenv("GRM_HIP_GQA_SPLIT")) a->query_split = env[0] != '0';
  a->ticks_per_ms = grm::wall_ticks_per_ms(a->device);
  if (const char* env = getenv("GRM_HIP_GQA_SR_ORDER")) {
    a->sr_order = strcmp(env, "slot") == 0 ? 0 : (strcmp(env, "size") == 0 ? 1 : -1);
  }
  if (const char* env = getenv("GRM_HIP_GQA_SPARSE")) a->sparse_exact = env[0] != '0';
  if (const char* env = getenv("GRM_HIP_GQA_WIDE_SMAX")) a->wide_smax = env[0] != '0';
  if (const char* env = getenv("GRM_HIP_GQA_SMAX_SPLIT")) {
    const long v = strtol(env, nullptr, 10);
    a->smax_split = (v == 2 || v == 4) ? static_cast<int>(v) : 0;
  }
  if (const char* env = getenv("GRM_HIP_GQA_BOUND")) {
    a->bound_mode = env[0] == '0' ? 0 : (env[0] == '1' ? 1 : -1);
  }
  if (const char* env = getenv("GRM_HIP_GQA_EXACT_WAVES")) {
    const long v = strtol(env, nullptr, 10);
    if (v >= 64 && v <= (1l << 30)) a->exact_waves = static_cast<uint32_t>(v);
  }
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
  if (key_dtype == kF32 && a->piece_shift == 2) {
    // the fp16 copy of an fp32 bank's keys (GRM_HIP_GQA_SHADOW=0: none)
    BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_skeys), cap_tokens * row_values(a) * 2));
  }
  if (key_dtype == kI8) {
    BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_scales), std::max<size_t>(16, cap_tokens * token_scale_bytes(a))));
  }
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_tok_off), cap_nodes * sizeof(uint64_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_len), cap_nodes * sizeof(uint32_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_ids), cap_nodes * sizeof(uint64_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_flags), cap_nodes * sizeof(uint32_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_nonfinite), cap_nodes * sizeof(uint32_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_kmax), cap_nodes * sizeof(unsigned)));
  BAIL_HIP(hipMemsetAsync(a->d_tok_off, 0, cap_nodes * sizeof(uint64_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_len, 0, cap_nodes * sizeof(uint32_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_ids, 0xff, cap_nodes * sizeof(uint64_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_flags, 0, cap_nodes * sizeof(uint32_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_nonfinite, 0, cap_nodes * sizeof(uint32_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_kmax, 0, cap_nodes * sizeof(unsigned), a->stream));
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
    while (i1 < nodes && (i1 == i0 || tok + padded_len(counts[i1]) <= batch_tokens_cap)) {
      tok += padded_len(counts[i1]);
      ++i1;
    }
    std::vector<uint64_t> bslots(slots.begin() + i0, slots.begin() + i1);
    std::vector<uint64_t> bids(ids.begin() + i0, ids.begin() + i1);
    const unsigned char* kptr = static_cast<const unsigned char*>(keys) +
                                (dense_rows ? i0 * dense_rows : tok_offsets[i0]) * kb;
    const unsigned char* sptr = scales ? static_cast<const unsigned char*>(scales) + tok_offsets[i0] * sb : nullptr;
    int rc = place_nodes(a, bslots, bids, counts.data() + i0, kptr, sptr, a->stream, dense_rows);
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
  std::vector<Item> items, units;
  items.reserve(a->live * 2);
  units.reserve(a->live);
  uint32_t max_len = 0;
  uint64_t n_cand_items = 0;
  for (uint64_t s = 0; s < a->high_water; ++s) {
    if (a->slot_id[s] == kNoId) continue;
    append_items(items, static_cast<uint32_t>(s), a->tok_off[s] * a->kv, a->len[s], a->chunk);
    n_cand_items += (a->len[s] + a->cand_chunk - 1) / a->cand_chunk;
    if (a->len[s] > 0) {
      append_items(units, static_cast<uint32_t>(s), a->tok_off[s] * a->kv, a->len[s], a->len[s]);
    }
    max_len = std::max(max_len, a->len[s]);
  }
  // The screen-only pass hands units to its waves round robin (wave w
  // takes w, w + S, w + 2S, ...).  In order of decreasing token count, any
  // two waves' totals differ by at most the longest unit minus the
  // shortest, and the pass ends on short units; in slot order the totals
  // of lognormal node lengths spread by about 10 %.  A counting sort on
  // the token count (capped at 2^16) keeps this O(units).
  if (units.size() > 1) {
    constexpr uint32_t kKeys = 1u << 16;
    std::vector<uint32_t> start(kKeys + 1, 0);
    auto key = [&](const Item& u) { return kKeys - 1 - std::min<uint32_t>(u.count, kKeys - 1); };
    for (const Item& u : units) ++start[key(u) + 1];
    for (uint32_t k = 0; k < kKeys; ++k) start[k + 1] += start[k];
    std::vector<Item> sorted(units.size());
    for (const Item& u : units) sorted[start[key(u)]++] = u;
    units.swap(sorted);
  }
  std::vector<Item> sized(items);
  std::stable_sort(sized.begin(), sized.end(), [](const Item& x, const Item& y) {
    return (x.count + 63) / 64 > (y.count + 63) / 64;
  });
  GRM_CHECK_RC(reserve_device(&a->d_items, &a->d_items_count, items.size()));
  GRM_CHECK_RC(reserve_device(&a->d_items_sized, &a->d_items_sized_count, items.size()));
  GRM_CHECK_RC(reserve_device(&a->d_units, &a->d_units_count, units.size()));
  if (!items.empty()) {
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_items, items.data(), items.size() * sizeof(Item),
                                 hipMemcpyHostToDevice, a->stream));
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_items_sized, sized.data(), sized.size() * sizeof(Item),
                                 hipMemcpyHostToDevice, a->stream));
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_units, units.data(), units.size() * sizeof(Item),
                                 hipMemcpyHostToDevice, a->stream));
    GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
  }
  a->n_items = items.size();
  a->n_cand_items = n_cand_items;
  a->n_units = units.size();
  a->max_len = max_len;
  a->items_epoch = a->epoch;
  return 0;
}

int rq_pad_of(int rq) {
  int p = 1;
  while (p < rq) p *= 2;
  return p;
}

// One pass over part of a route's query: heads g*R + r0 .. +rc of every kv
// head g, tokens t0 .. +qc (see "Query passes" in gqa_kernels.hpp).
struct QPass {
  int r0 = 0, rc = 0, t0 = 0, qc = 0;
};

// Passes that cover R heads per kv head x Qt tokens with at most `cmax`
// query columns (rc * qc) each: the whole query when it fits, else runs of
// tokens of all R heads, else (R > cmax) runs of heads of one token.
std::vector<QPass> query_passes(int R, int Qt, int cmax) {
  std::vector<QPass> out;
  if (R * Qt <= cmax) {
    out.push_back({0, R, 0, Qt});
  } else if (R <= cmax) {
    const int qc = cmax / R;
    for (int t0 = 0; t0 < Qt; t0 += qc) out.push_back({0, R, t0, std::min(qc, Qt - t0)});
  } else {
    for (int t0 = 0; t0 < Qt; ++t0) {
      for (int r0 = 0; r0 < R; r0 += cmax) out.push_back({r0, std::min(cmax, R - r0), t0, 1});
    }
  }
  return out;
}

// Byte offset of a pass's first query value (head r0, token t0 of kv head
// 0) from the query's start.
size_t pass_query_offset(const GqaDeviceArena* a, int Qt, const QPass& ps, int q_dtype) {
  return (static_cast<size_t>(ps.r0) * Qt + ps.t0) * a->hd * (q_dtype == kF32 ? 4 : 2);
}

// Maxima for up to qb queries; all zero between routes (the finalize
// kernel re-zeroes what it reads).
int ensure_hmax(GqaDeviceArena* a, int H, int qb) {
  const size_t want = static_cast<size_t>(qb) * a->cap_nodes * static_cast<size_t>(H);
  return reserve_device_zero(&a->d_hmax, &a->d_hmax_count, want, a->stream);
}

// Exact scores and per-block top-k of every slot, or (slot_list given) of
// the listed candidate slots of each query.
int launch_finalize(GqaDeviceArena* a, int H, int qb, int topk, uint32_t fin_blocks, Cand* bout,
                    const uint32_t* slot_list = nullptr, const uint32_t* list_count = nullptr,
                    unsigned* done = nullptr, unsigned long long* end_stamps = nullptr) {
  const uint32_t per_block = grm::gqa::kFinWaves * grm::kWave;
  grm::gqa::gqa_finalize_kernel<<<dim3(fin_blocks, qb), per_block, 0, a->stream>>>(
      a->d_hmax, a->cap_nodes * static_cast<size_t>(H), a->cap_nodes, H,
      static_cast<uint32_t>(a->high_water), a->d_len,
      a->route_flags ? a->route_flags : a->d_flags, a->d_ids, a->d_qbad,
      static_cast<int>(a->kv), topk, bout, slot_list, list_count, a->cap_nodes, done,
      a->route_seq, end_stamps);
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

// --------------------------------------------------------------- exact path

// Query rows of pass `ps` of queries [0, qb) at q (the query's start) as
// doubles in d_q64; d_qbad records non-finite values (written by the first
// pass, raised by later ones: flags_or).
int launch_q64(GqaDeviceArena* a, const void* q, int q_dtype, int qb, int H, int Qt,
               const QPass& ps, bool flags_or) {
  const int R = H / static_cast<int>(a->kv);
  const int rq_pad = rq_pad_of(ps.rc * ps.qc);
  GRM_CHECK_RC(reserve_device(&a->d_q64, &a->d_q64_count,
                              static_cast<size_t>(qb) * a->kv * a->hd * rq_pad));
  GRM_CHECK_RC(reserve_device(&a->d_qbad, &a->d_qbad_count, static_cast<size_t>(qb) * a->kv));
  // a block per (kv head, query); wide passes (a whole query of many
  // tokens) take 1024 threads
  const unsigned q64_threads = rq_pad >= 64 ? 1024u : 256u;
  grm::gqa::gqa_q64_kernel<<<dim3(a->kv, qb), q64_threads, 0, a->stream>>>(
      static_cast<const unsigned char*>(q) + pass_query_offset(a, Qt, ps, q_dtype), q_dtype,
      static_cast<size_t>(H) * Qt * a->hd, Qt, ps.qc, static_cast<int>(a->hd),
      static_cast<int>(a->kv), R, ps.rc, rq_pad, a->d_q64, a->d_qbad, flags_or ? 1 : 0);
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

// Exact maxima of pass `ps` (rows in d_q64, launch_q64) of the bank's items
// against query 0, or (n_items_dev given) of the device-built list `items`
// (at most max_items), each item against its own query.
int launch_exact(GqaDeviceArena* a, int H, const QPass& ps, const Item* items = nullptr,
                 uint64_t max_items = 0, const uint32_t* n_items_dev = nullptr) {
  if (!n_items_dev) {
    items = a->d_items;
    max_items = a->n_items;
  }
  if (max_items == 0) return 0;
  const int R = H / static_cast<int>(a->kv);
  const int rq_pad = rq_pad_of(ps.rc * ps.qc);
  if (rq_pad > grm::gqa::kMaxRQ) return grm::fail(-1, "exact pass wider than 32 columns");
  // Persistent stream: about exact_waves wavefronts, each walking the
  // (kv head, item) pairs w, w+W, ...; device-built lists get a fixed
  // number of waves, since their length is known only on the device
  const uint64_t pairs = n_items_dev ? std::min<uint64_t>(max_items * a->kv, 8192) : max_items * a->kv;
  if (max_items * a->kv >= 0xffffffffull) return grm::fail(-1, "too many work items");
  const uint64_t bx = std::min<uint64_t>((pairs + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves,
                                         (a->exact_waves + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves);
  const dim3 grid(static_cast<unsigned>(std::max<uint64_t>(1, bx)));
  const unsigned threads = grm::gqa::kUnitWaves * grm::kWave;
  const double denom = sqrt(static_cast<double>(a->hd));
#define GRM_EXACT(KDT, RQ)                                                                  \
  grm::gqa::gqa_exact_kernel<KDT, RQ, grm::gqa::exact_stage_chunks<KDT, RQ>()><<<grid, threads, 0, a->stream>>>( \
      a->d_keys, a->d_scales, a->scale_dtype, a->group_size, items,                         \
      static_cast<uint32_t>(max_items), n_items_dev, static_cast<int>(a->kv),                 \
      static_cast<int>(a->hd), a->piece_shift, R, ps.rc, ps.qc, a->d_q64, denom,              \
      a->d_hmax + static_cast<size_t>(ps.r0) * a->cap_nodes,                                   \
      a->cap_nodes * static_cast<size_t>(H), a->cap_nodes)
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

// Enqueue the exact route of one query, in passes of at most 32 query
// columns per kv head; its per-block top-k lands at bout.
int enqueue_exact(GqaDeviceArena* a, const void* q, int q_dtype, int H, int Qt, int topk,
                  uint32_t fin_blocks, Cand* bout) {
  GRM_CHECK_RC(ensure_hmax(a, H, 1));
  const auto passes = query_passes(H / static_cast<int>(a->kv), Qt, grm::gqa::kMaxRQ);
  for (size_t i = 0; i < passes.size(); ++i) {
    GRM_CHECK_RC(launch_q64(a, q, q_dtype, 1, H, Qt, passes[i], i > 0));
    GRM_CHECK_RC(launch_exact(a, H, passes[i]));
  }
  return launch_finalize(a, H, 1, topk, fin_blocks, bout);
}

void write_result(const Cand* merged, int topk, uint64_t* out_ids, float* out_scores) {
  for (int j = 0; j < topk; ++j) {
    const Cand& c = merged[j];
    const bool ok = isfinite(c.score) && c.id != kNoId;
    out_ids[j] = ok ? c.id : kNoId;
    if (out_scores) out_scores[j] = ok ? c.score : __builtin_nanf("");
  }
}

// ---------------------------------------------------- screen-and-refine path

struct SrPlan {
  int R = 0, Qt = 0, H = 0;
  int KS = 0;        // head_dim / 32
  int qb_max = 0;    // queries per pass (<= 64 columns)
  int mfma = kBF16;  // MFMA operand type
  std::vector<QPass> passes;  // query passes of one query (one unless R*Qt > 64)
};

// Maxima memory per pass is bounded by this many bytes (when one query
// alone needs more, passes take one query).
constexpr size_t kMaxHmaxBytes = 2ull << 30;

// The plane the screens read and its element type: the keys themselves,
// or an fp32 bank's fp16 copy.
const unsigned char* screen_keys(const GqaDeviceArena* a) { return a->d_skeys ? a->d_skeys : a->d_keys; }
int screen_dtype(const GqaDeviceArena* a) { return a->d_skeys ? kF16 : a->key_dtype; }

bool sr_plan(const GqaDeviceArena* a, int H, int Qt, SrPlan* p) {
  if (a->screen_mode == 0 || screen_dtype(a) == kF32) return false;
  if (a->hd != 64 && a->hd != 128 && a->hd != 256) return false;
  if (!a->d_skeys && a->piece_shift != 2) return false;  // the screen reads 64-byte chunks
  const int R = H / static_cast<int>(a->kv);
  p->R = R;
  p->Qt = Qt;
  p->H = H;
  p->KS = static_cast<int>(a->hd / 32);
  p->passes = query_passes(R, Qt, grm::gqa::kMaxCols);
  const size_t per_q = a->cap_nodes * static_cast<size_t>(H) * sizeof(unsigned long long);
  // a query wider than one pass is routed alone, its passes one after another
  const int cols1 = p->passes.size() == 1 ? R * Qt : grm::gqa::kMaxCols;
  p->qb_max = p->passes.size() == 1
                  ? std::max(1, std::min(grm::gqa::kMaxCols / cols1,
                                         static_cast<int>(std::max<size_t>(1, kMaxHmaxBytes / per_q))))
                  : 1;
  p->mfma = screen_dtype(a) == kBF16 ? kBF16 : kF16;
  return true;
}

// Device buffers of screen-and-refine passes of up to p.qb_max queries.
int prepare_sr(GqaDeviceArena* a, const SrPlan& p) {
  GRM_CHECK_RC(reserve_device(&a->d_qbad, &a->d_qbad_count, static_cast<size_t>(p.qb_max) * a->kv));
  return ensure_hmax(a, p.H, p.qb_max);
}

// Screen-bound constants of one route (per query column, see
// gqa_sr_kernel and gqa_smax_kernel):
//   gamma  fp32 accumulation of hd products, MFMA internal order unknown
//   delta  rounding of an fp32 query value to the MFMA type
//   sigma_q, sigma_k  a query / key value near zero flushed or rounded
//   sigma_p  a product lost to fp32 underflow
//   emax   the exponent under which scaled query values stay
//   eps_rel, eps_abs  an fp32 bank's fp16 key copy: rounding to nearest
//          even moves a value by at most 2^-11 of it, or 2^-25 below the
//          fp16 normal range
struct ScreenBound {
  double gamma = 0, delta = 0, sigma_q = 0, sigma_k = 0, sigma_p = 0;
  double eps_rel = 0, eps_abs = 0;
  int emax = 0;
};

ScreenBound screen_bound(const GqaDeviceArena* a, const SrPlan& p, int q_dtype) {
  ScreenBound b;
  b.gamma = 2.0 * (a->hd + 2.0 * p.KS) * ldexp(1.0, -24);
  if (p.mfma == kBF16) {
    b.delta = q_dtype == kF32 ? ldexp(1.0, -8) : 0.0;
    b.sigma_q = b.sigma_k = b.sigma_p = ldexp(1.0, -125);
    b.emax = 126;
  } else {
    b.delta = q_dtype == kF32 ? ldexp(1.0, -11) : 0.0;
    b.sigma_q = b.sigma_k = ldexp(1.0, -14);
    b.sigma_p = 0.0;
    b.emax = 15;
  }
  if (a->d_skeys) {
    b.eps_rel = ldexp(1.0, -11);
    b.eps_abs = ldexp(1.0, -25);
  }
  return b;
}

// One screen-and-refine launch: query pass `pi` of queries [0, qb) at qptr
// (the queries' start) against every (item, kv head), folding into the
// maxima; the first pass writes the query flags, later ones raise them.
int launch_sr_pass(GqaDeviceArena* a, const SrPlan& p, const ScreenBound& eb,
                   const unsigned char* qptr, int q_dtype, int qb, size_t pi,
                   const grm::RouteStamps& st) {
  const int kv = static_cast<int>(a->kv);
  const QPass& ps = p.passes[pi];
  if (a->n_items == 0) {
    // no key tokens at all: only the query flags are needed
    return launch_q64(a, qptr, q_dtype, qb, p.H, p.Qt, ps, pi > 0);
  }
  const int cols = qb * ps.rc * ps.qc;
  const int nt_need = (cols + 15) / 16;
  const int NT = nt_need <= 1 ? 1 : (nt_need <= 2 ? 2 : 4);
  const unsigned char* qpass = qptr + pass_query_offset(a, p.Qt, ps, q_dtype);
  unsigned long long* hpass = a->d_hmax + static_cast<size_t>(ps.r0) * a->cap_nodes;
  const size_t q_elems = static_cast<size_t>(p.H) * p.Qt * a->hd;
  // kv heads fastest, so the resident blocks sweep the bank in address
  // order (a node's kv-head blocks are contiguous); item blocks on x only
  // past the grid's y limit
  const uint64_t item_blocks = (a->n_items + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves;
  const int g_fast = item_blocks <= 65535 ? 1 : 0;
  const dim3 grid = g_fast ? dim3(a->kv, static_cast<unsigned>(item_blocks))
                           : dim3(static_cast<unsigned>(item_blocks), a->kv);
  const unsigned threads = grm::gqa::kUnitWaves * grm::kWave;
  const size_t hstride = a->cap_nodes * static_cast<size_t>(p.H);
  const double denom = sqrt(static_cast<double>(a->hd));
  // Item order: address order streams best (C4 shape, one query token:
  // 192 us against 198 us by size), and with items of 512 tokens (whole
  // nodes there) also for 4 query tokens (207 against 209 us).  Items of
  // 256 tokens with a heavier refine (more columns, or an fp32 bank's rows
  // read again in fp32) go by decreasing size: the waves of short items at
  // the launch's end even out the refines' cost (4 tokens: 221 us against
  // 252 us; fp32 bank: 215 us against 227 us).
  // GRM_HIP_GQA_SR_ORDER=slot / size fixes either.
  const bool by_size = a->sr_order >= 0 ? a->sr_order == 1
                                        : (a->d_skeys != nullptr || (cols > 4 && a->chunk <= 256));
  // fp32 queries over at most 8 columns: each column's remainder after its
  // rounding to the MFMA type rides in an idle column slot (gqa_sr_kernel,
  // query_frags), so the query's rounding leaves the bound: per value
  // |q - hi - lo| <= u^2 |q| + (1 + u) sigma_q (u the type's unit
  // roundoff), and the two fp32 accumulations plus their sum stay within
  // (gamma (1 + 3u) + 2^-24) ||q|| ||k||, so gamma' = gamma (1 + 2^-6) +
  // 2^-23, delta' = u^2 and sigma_q' = 2 sigma_q bound it
  // (GRM_HIP_GQA_SPLIT=0: no split).
  const int split = a->query_split && q_dtype == kF32 && NT == 1 && cols <= 8 ? 1 : 0;
  ScreenBound sb = eb;
  if (split) {
    const double u = p.mfma == kBF16 ? ldexp(1.0, -8) : ldexp(1.0, -11);
    sb.delta = u * u;
    sb.gamma = eb.gamma * (1.0 + ldexp(1.0, -6)) + ldexp(1.0, -23);
    sb.sigma_q = 2.0 * eb.sigma_q;
  }
  const Item* sr_items = by_size ? a->d_items_sized : a->d_items;
  // query columns in rows of hd + 4 floats: <= 66,560 bytes
  const size_t lds = static_cast<size_t>(cols) * (a->hd + 4) * sizeof(float);
#define GRM_SR(KDT, KS, NTT, XF)                                                                \
  if (lds > 65536) {                                                                            \
    GRM_HIP_CHECK(hipFuncSetAttribute(                                                          \
        reinterpret_cast<const void*>(grm::gqa::gqa_sr_kernel<KDT, KS, NTT, XF>),               \
        hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)));                    \
  }                                                                                             \
  grm::gqa::gqa_sr_kernel<KDT, KS, NTT, XF><<<grid, threads, lds, a->stream>>>(                 \
      screen_keys(a), a->d_keys, a->d_scales, a->scale_dtype, a->group_size, sr_items,          \
      static_cast<uint32_t>(a->n_items), kv, p.R, p.Qt, ps.rc, ps.qc, qpass, q_dtype, q_elems,  \
      qb, sb.emax, sb.gamma, sb.delta, sb.sigma_q, sb.sigma_k, sb.sigma_p, sb.eps_rel,          \
      sb.eps_abs, a->d_qbad, pi > 0 ? 1 : 0, reinterpret_cast<const float*>(a->d_kmax), denom,   \
      hpass, hstride, a->cap_nodes, g_fast, split, st, a->route_seq)
#define GRM_SR_NT(KDT, KS, XF)                 \
  switch (NT) {                                \
    case 1: GRM_SR(KDT, KS, 1, XF); break;     \
    case 2: GRM_SR(KDT, KS, 2, XF); break;     \
    default: GRM_SR(KDT, KS, 4, XF); break;    \
  }
#define GRM_SR_KS(KDT, XF)                     \
  switch (p.KS) {                              \
    case 2: GRM_SR_NT(KDT, 2, XF); break;      \
    case 4: GRM_SR_NT(KDT, 4, XF); break;      \
    default: GRM_SR_NT(KDT, 8, XF); break;     \
  }
  if (a->d_skeys) {
    GRM_SR_KS(kF16, true);
  } else {
    switch (a->key_dtype) {
      case kBF16: GRM_SR_KS(kBF16, false); break;
      case kF16: GRM_SR_KS(kF16, false); break;
      default: GRM_SR_KS(kI8, false); break;
    }
  }
#undef GRM_SR_KS
#undef GRM_SR_NT
#undef GRM_SR
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

// Enqueue the screen-and-refine route of queries [0, qb) at qptr (device,
// `qstride` bytes apart): its query passes one after another, all folding
// into the same maxima, then the finalize.  Their per-block top-k lands at
// bout, and with `done` the finalize blocks' completion flags at
// done[0, qb*fin_blocks).  With st.start the first pass stores the route's
// start tick, with st.end the finalize blocks their end ticks
// (RouteStamps).  Launches only (prepare_sr allocates).
int enqueue_sr(GqaDeviceArena* a, const SrPlan& p, const unsigned char* qptr, int q_dtype, int qb,
               int topk, uint32_t fin_blocks, Cand* bout, unsigned* done,
               const grm::RouteStamps& st) {
  const ScreenBound eb = screen_bound(a, p, q_dtype);
  for (size_t pi = 0; pi < p.passes.size(); ++pi) {
    const grm::RouteStamps sp{pi == 0 ? st.start : nullptr, nullptr};
    GRM_CHECK_RC(launch_sr_pass(a, p, eb, qptr, q_dtype, qb, pi, sp));
  }
  return launch_finalize(a, p.H, qb, topk, fin_blocks, bout, nullptr, nullptr, done, st.end);
}

// ------------------------------------------------------ bound-and-verify path

constexpr uint32_t kCandFinBlocks = 16;  // finalize blocks per query over candidates

// Bound and verify keeps the screened maxima of every column of the
// query (one screen launch per query pass of at most 64 columns per kv
// head, all into one set of rows) and verifies the candidates in exact
// passes of at most 32 columns.
// By default passes of more than 24 query columns per kv head take it: on
// the 512-node bank (R = 4) screen and refine is faster up to 5 query
// tokens (0.355 against 0.595 ms at 5) and bound and verify from 8 (0.422
// against 0.471 ms; 2.61 against 3.61 ms at 64 tokens).
bool use_bound(const GqaDeviceArena* a, const SrPlan& p, int qb) {
  if (a->bound_mode == 0) return false;
  if (a->bound_mode == 1) return true;
  return qb * p.R * p.Qt > 24;
}

// Column parameters of a bounds block beyond this many bytes are read
// from global memory instead of LDS.
constexpr size_t kBoundsStageBytes = 32768;
// Queries with at least this many (head, query token) cells per node take
// the bounds kernel with lanes over heads, in up to kWideBlocks blocks.
constexpr int kWideCells = 1024;
constexpr uint32_t kWideBlocks = 1024;

// Grid (P, kv) of the persistent screen kernel `fn`: as many blocks as
// the device holds resident at once (a block that had to wait for a slot
// would start its whole share of the items when the others finish), and
// no more than there are items to give every wave one.
int persistent_grid(GqaDeviceArena* a, const void* fn, unsigned threads, size_t lds, dim3* grid,
                    uint32_t walkers_per_block = grm::gqa::kUnitWaves) {
  const std::pair<const void*, size_t> key(fn, lds);
  auto it = a->resident.find(key);
  int per_cu = 0;
  if (it == a->resident.end()) {
    GRM_HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, static_cast<int>(threads), lds));
    per_cu = std::max(1, per_cu);
    a->resident.emplace(key, per_cu);
  } else {
    per_cu = it->second;
  }
  int cus = 256;
  GRM_HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, a->device));
  const uint64_t resident = static_cast<uint64_t>(std::max(1, cus)) * static_cast<uint64_t>(per_cu);
  const uint64_t px = std::max<uint64_t>(
      1, std::min<uint64_t>((a->n_units + walkers_per_block - 1) / walkers_per_block,
                            std::max<uint64_t>(1, resident / a->kv)));
  *grid = dim3(static_cast<unsigned>(px), a->kv);
  return 0;
}

// Device buffers of bound-and-verify passes of up to p.qb_max queries.
int prepare_bv(GqaDeviceArena* a, const SrPlan& p, int topk, uint32_t fin_blocks) {
  const size_t qbm = static_cast<size_t>(p.qb_max);
  const size_t cap = a->cap_nodes;
  GRM_CHECK_RC(reserve_device(&a->d_hmaxf, &a->d_hmaxf_count,
                              qbm * static_cast<size_t>(p.H) * p.Qt * cap));
  GRM_CHECK_RC(reserve_device(&a->d_colinfo, &a->d_colinfo_count,
                              static_cast<size_t>(a->kv) * qbm * p.R * p.Qt));
  GRM_CHECK_RC(reserve_device(&a->d_lbub, &a->d_lbub_count, qbm * cap));
  GRM_CHECK_RC(reserve_device(&a->d_blists, &a->d_blists_count,
                              qbm * std::max(fin_blocks, kWideBlocks) * static_cast<size_t>(topk)));
  GRM_CHECK_RC(reserve_device(&a->d_cslots, &a->d_cslots_count, qbm * cap));
  GRM_CHECK_RC(reserve_device(&a->d_ccount, &a->d_ccount_count, qbm + 1));
  GRM_CHECK_RC(reserve_device(&a->d_citems, &a->d_citems_count,
                              std::max<size_t>(1, qbm * a->n_cand_items)));
  GRM_CHECK_RC(reserve_device(&a->d_q64, &a->d_q64_count,
                              qbm * a->kv * a->hd * rq_pad_of(p.R * p.Qt)));
  return 0;
}

// Screen-only pass of queries [0, qb) at qptr over every (node, kv head)
// work unit: the largest screened |q~.k| per column and node into
// d_hmaxf (one run of colstride cells per (slot, kv head)), the columns'
// bound parameters into d_colinfo.
int launch_smax(GqaDeviceArena* a, const SrPlan& p, const unsigned char* qptr, int q_dtype, int qb,
                int colstride, const QPass* passes, int np) {
  const int kv = static_cast<int>(a->kv);
  if (np != 1 && np != 2 && np != 4) return grm::fail(-1, "1, 2 or 4 screen passes per launch");
  grm::gqa::SmaxPasses sp{};
  int cols = 0;
  for (int i = 0; i < np; ++i) {
    sp.r0[i] = passes[i].r0;
    sp.rc[i] = passes[i].rc;
    sp.t0[i] = passes[i].t0;
    sp.qc[i] = passes[i].qc;
    cols = std::max(cols, qb * passes[i].rc * passes[i].qc);
  }
  const int tiles = (cols + 15) / 16;
  const int NT = tiles <= 1 ? 1 : (tiles <= 2 ? 2 : (tiles <= 4 ? 4 : 8));
  if (cols > grm::gqa::kMaxSmaxCols || (NT == 8 && p.KS > 4) || (np > 1 && (NT > 4 || p.KS > 4))) {
    return grm::fail(-1, "screen-only pass wider than its kernel");
  }
  const bool fact = a->key_dtype == kI8 && static_cast<uint32_t>(a->group_size) == a->hd;
  // error-bound constants as in enqueue_sr; rho: the INT8 row scale
  // factored out of the dot product (fp32 product then fp16 rounding of
  // code*scale, and the fp32 product of the screened value by the scale)
  const ScreenBound eb = screen_bound(a, p, q_dtype);
  const double gamma = eb.gamma, delta = eb.delta, sigma_q = eb.sigma_q, sigma_k = eb.sigma_k,
               sigma_p = eb.sigma_p;
  const int emax = eb.emax;
  const double rho = fact ? ldexp(1.0, -11) + ldexp(1.0, -21) : 0.0;
  const size_t q_elems = static_cast<size_t>(p.H) * p.Qt * a->hd;
  const unsigned threads = (np == 1 ? grm::gqa::kUnitWaves : 8) * grm::kWave;
  if (a->n_units > 0) {
    // one LDS region of NT*16 columns per pass when passes are split
    const size_t lds = np == 1 ? static_cast<size_t>(cols) * a->hd * sizeof(float)
                               : static_cast<size_t>(np) * NT * 16 * a->hd * sizeof(float);
#define GRM_SMAX_NP(KDT, KS, NTT, FACT, SF16, NPP)                                                \
  do {                                                                                            \
    auto fn = grm::gqa::gqa_smax_kernel<KDT, KS, NTT, FACT, SF16, NPP>;                           \
    dim3 grid;                                                                                    \
    GRM_CHECK_RC(persistent_grid(a, reinterpret_cast<const void*>(fn), threads, lds, &grid,       \
                                 NPP == 1 ? grm::gqa::kUnitWaves : 8 / NPP));                     \
    fn<<<grid, threads, lds, a->stream>>>(                                                        \
        screen_keys(a), a->d_scales, a->scale_dtype, a->group_size, a->d_units,                   \
        static_cast<uint32_t>(a->n_units), kv, p.R, p.Qt, sp, qptr,                               \
        q_dtype, q_elems, qb, emax,                                                               \
        gamma, delta, rho, sigma_q, sigma_k, sigma_p, eb.eps_rel, eb.eps_abs, a->d_colinfo,        \
        a->d_hmaxf, colstride);                                                                   \
  } while (0)
#define GRM_SMAX(KDT, KS, NTT, FACT, SF16)                                        \
  do {                                                                            \
    if (np == 1) {                                                                \
      GRM_SMAX_NP(KDT, KS, NTT, FACT, SF16, 1);                                   \
    } else if (np == 2) {                                                         \
      GRM_SMAX_NP(KDT, KS, (NTT <= 4 ? NTT : 4), FACT, SF16, (KS <= 4 ? 2 : 1));  \
    } else {                                                                      \
      GRM_SMAX_NP(KDT, KS, (NTT <= 4 ? NTT : 4), FACT, SF16, (KS <= 4 ? 4 : 1));  \
    }                                                                             \
  } while (0)
#define GRM_SMAX_NT(KDT, KS, FACT, SF16)               \
  switch (NT) {                                        \
    case 1: GRM_SMAX(KDT, KS, 1, FACT, SF16); break;   \
    case 2: GRM_SMAX(KDT, KS, 2, FACT, SF16); break;   \
    case 4: GRM_SMAX(KDT, KS, 4, FACT, SF16); break;   \
    default: GRM_SMAX_NP(KDT, KS, (KS <= 4 ? 8 : 4), FACT, SF16, 1); break; \
  }
#define GRM_SMAX_KS(KDT, FACT, SF16)                   \
  switch (p.KS) {                                      \
    case 2: GRM_SMAX_NT(KDT, 2, FACT, SF16); break;    \
    case 4: GRM_SMAX_NT(KDT, 4, FACT, SF16); break;    \
    default: GRM_SMAX_NT(KDT, 8, FACT, SF16); break;   \
  }
    const bool sf16 = a->scale_dtype == kF16;
    switch (screen_dtype(a)) {
      case kBF16: GRM_SMAX_KS(kBF16, false, false); break;
      case kF16: GRM_SMAX_KS(kF16, false, false); break;
      default:
        if (fact && sf16) {
          GRM_SMAX_KS(kI8, true, true);
        } else if (fact) {
          GRM_SMAX_KS(kI8, true, false);
        } else if (sf16) {
          GRM_SMAX_KS(kI8, false, true);
        } else {
          GRM_SMAX_KS(kI8, false, false);
        }
        break;
    }
#undef GRM_SMAX_KS
#undef GRM_SMAX_NT
#undef GRM_SMAX
#undef GRM_SMAX_NP
    GRM_HIP_CHECK(hipGetLastError());
  }
  return 0;
}

// Enqueue one bound-and-verify pass over queries [0, qb) at qptr; query
// j's top-k candidates (kCandFinBlocks lists of k) land at bout + j*per_q.
int enqueue_bv(GqaDeviceArena* a, const SrPlan& p, const unsigned char* qptr, int q_dtype, int qb,
               int topk, uint32_t fin_blocks, Cand* bout, size_t per_q) {
  const int kv = static_cast<int>(a->kv);
  const int RQ = p.R * p.Qt;
  const int cols = qb * RQ;
  const int H = p.H;
  const bool fact = a->key_dtype == kI8 && static_cast<uint32_t>(a->group_size) == a->hd;
  // screened maxima: one run of colstride cells per (slot, kv head)
  const int colstride = p.qb_max * RQ;
  (void)cols;
  // exact passes of at most 32 columns per kv head
  const std::vector<QPass> xpasses = query_passes(p.R, p.Qt, grm::gqa::kMaxRQ);
  // 1. the query flags, and the query rows as doubles for a single exact
  // pass (with several, each loads its own rows before it runs)
  const QPass whole{0, p.R, 0, p.Qt};
  GRM_CHECK_RC(launch_q64(a, qptr, q_dtype, qb, H, p.Qt, xpasses.size() == 1 ? xpasses[0] : whole, false));
  // 2. screened maxima of every (column, node), one launch per screen
  // pass: a single query wider than one pass takes passes of up to 128
  // columns where the query fragments fit the registers (head dim <= 128)
  const bool single_wide = qb == 1 && p.passes.size() > 1 && p.KS <= 4;
  if (single_wide && a->smax_split > 1 && p.passes.size() >= static_cast<size_t>(a->smax_split)) {
    // passes of 64 columns, up to smax_split of them per launch
    const std::vector<QPass>& sp = p.passes;
    for (size_t i = 0; i < sp.size();) {
      const size_t left = sp.size() - i;
      const int np = left >= static_cast<size_t>(a->smax_split) ? a->smax_split : (left >= 2 ? 2 : 1);
      GRM_CHECK_RC(launch_smax(a, p, qptr, q_dtype, qb, colstride, &sp[i], np));
      i += static_cast<size_t>(np);
    }
  } else {
    const bool wide_passes = a->wide_smax && single_wide;
    const std::vector<QPass> spasses =
        wide_passes ? query_passes(p.R, p.Qt, grm::gqa::kMaxSmaxCols) : p.passes;
    for (const QPass& ps : spasses) GRM_CHECK_RC(launch_smax(a, p, qptr, q_dtype, qb, colstride, &ps, 1));
  }
  // 3. score bounds, the k best lower bounds per block (with no key tokens
  // at all the column parameters are never used: every live node has no
  // tokens and scores 0)
  const size_t ci_bytes = static_cast<size_t>(H) * p.Qt * sizeof(float4);
  const bool staged = ci_bytes <= kBoundsStageBytes;
  const bool wide = H * p.Qt >= kWideCells;
  const uint32_t n_slots = static_cast<uint32_t>(a->high_water);
  // the bounds blocks, and so the candidates kernel's lists per query: a
  // wavefront per slot (wide), else a lane per slot and about two rounds
  // of slots per wavefront (a block's fixed cost -- column parameters,
  // list merge -- would dominate one round)
  constexpr uint32_t kBoundsSlots = 2 * grm::gqa::kFinWaves * grm::kWave;
  const uint32_t bblocks =
      wide ? std::max<uint32_t>(1, std::min<uint32_t>(kWideBlocks, (n_slots + grm::gqa::kFinWaves - 1) /
                                                                        grm::gqa::kFinWaves))
           : (std::max<uint32_t>(1, std::min<uint32_t>(fin_blocks, (n_slots + kBoundsSlots - 1) / kBoundsSlots)) +
              7u) / 8u * 8u;  // a multiple of 8 (the kernel's XCD mapping)
#define GRM_BOUNDS(ST)                                                                           \
  grm::gqa::gqa_bounds_kernel<ST><<<dim3(qb * bblocks), grm::gqa::kFinWaves * grm::kWave,         \
                                    ST ? ci_bytes : 0, a->stream>>>(                             \
      a->d_hmaxf, colstride, a->cap_nodes, H, p.Qt, p.R, colstride, kv,                          \
      static_cast<uint32_t>(a->high_water), a->d_len,                                            \
      a->route_flags ? a->route_flags : a->d_flags, a->d_ids, a->d_kmax,                         \
      a->d_colinfo, a->d_qbad, fact ? 1 : 0, static_cast<int>(a->hd), topk, a->d_lbub,           \
      a->d_blists, a->d_ccount, p.qb_max + 1, qb)
  if (wide) {
    grm::gqa::gqa_bounds_wide_kernel<<<dim3(qb, bblocks), grm::gqa::kFinWaves * grm::kWave, 0,
                                       a->stream>>>(
        a->d_hmaxf, colstride, a->cap_nodes, H, p.Qt, p.R, colstride, kv, n_slots, a->d_len,
        a->route_flags ? a->route_flags : a->d_flags, a->d_ids, a->d_kmax, a->d_colinfo, a->d_qbad,
        fact ? 1 : 0, static_cast<int>(a->hd), topk, a->d_lbub, a->d_blists, a->d_ccount, p.qb_max + 1);
  } else if (staged) {
    GRM_BOUNDS(true);
  } else {
    GRM_BOUNDS(false);
  }
#undef GRM_BOUNDS
  GRM_HIP_CHECK(hipGetLastError());
  // 4. candidates and their exact work items, each query's slots split
  // over blocks of about four rounds of the block's wavefronts
  const uint32_t cblocks = std::max<uint32_t>(
      1, std::min<uint32_t>(64, (n_slots + 4 * grm::gqa::kCandWaves * grm::kWave - 1) /
                                    (4 * grm::gqa::kCandWaves * grm::kWave)));
  grm::gqa::gqa_cands_kernel<<<dim3(qb, cblocks), grm::gqa::kCandWaves * grm::kWave, 0, a->stream>>>(
      a->d_blists, bblocks, topk, a->d_lbub, a->cap_nodes, static_cast<uint32_t>(a->high_water),
      a->d_tok_off, a->d_len, kv, a->cand_chunk, a->d_cslots, a->d_ccount, a->d_citems,
      a->d_ccount + p.qb_max);
  GRM_HIP_CHECK(hipGetLastError());
  // 5. the law on the candidates, then their exact scores and top-k: one
  // query wider than an exact pass takes only the columns its screen
  // cannot rule out (the query's rows as doubles are all in q64 from step
  // 1), others the exact kernel pass by pass
  if (qb == 1 && a->sparse_exact) {
    const uint64_t pairs = a->cap_nodes * a->kv;
    const unsigned blocks = static_cast<unsigned>(
        std::max<uint64_t>(1, std::min<uint64_t>((pairs + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves, 2048)));
    const int rqp = rq_pad_of(p.R * p.Qt);
    const double denom = sqrt(static_cast<double>(a->hd));
#define GRM_SPARSE(KDT)                                                                           \
  grm::gqa::gqa_exact_sparse_kernel<KDT><<<blocks, grm::gqa::kUnitWaves * grm::kWave,           \
                                           grm::gqa::kUnitWaves * grm::gqa::kSparseCols *       \
                                               a->hd * sizeof(double),                           \
                                           a->stream>>>(                                         \
      a->d_keys, a->d_scales, a->scale_dtype, a->group_size, a->piece_shift, a->d_cslots,        \
      a->d_ccount, kv, p.R, p.Qt, static_cast<int>(a->hd), colstride, a->d_hmaxf, a->d_colinfo,  \
      a->d_kmax, fact ? 1 : 0, a->d_tok_off, a->d_len, a->d_q64, rqp, denom, a->d_hmax,          \
      a->cap_nodes)
    switch (a->key_dtype) {
      case kF32: GRM_SPARSE(kF32); break;
      case kBF16: GRM_SPARSE(kBF16); break;
      case kF16: GRM_SPARSE(kF16); break;
      default: GRM_SPARSE(kI8); break;
    }
#undef GRM_SPARSE
    GRM_HIP_CHECK(hipGetLastError());
  } else {
    for (size_t i = 0; i < xpasses.size(); ++i) {
      if (xpasses.size() > 1) GRM_CHECK_RC(launch_q64(a, qptr, q_dtype, qb, H, p.Qt, xpasses[i], true));
      GRM_CHECK_RC(launch_exact(a, H, xpasses[i], a->d_citems,
                                static_cast<uint64_t>(qb) * a->n_cand_items, a->d_ccount + p.qb_max));
    }
  }
  (void)per_q;
  return launch_finalize(a, H, qb, topk, std::min(kCandFinBlocks, fin_blocks), bout, a->d_cslots,
                         a->d_ccount);
}

// Completion flags a route may wait on (one per query and finalize block).
constexpr size_t kMaxDoneFlags = 4096;

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
  GRM_HIP_CHECK(hipSetDevice(a->device));
  if (a->mut_pending) GRM_HIP_CHECK(hipStreamWaitEvent(a->stream, a->ev_mut, 0));
  GRM_CHECK_RC(ensure_items(a));
  a->routes += 1;
  const size_t qvals = static_cast<size_t>(H) * Qt * a->hd;
  const size_t qstride = qvals * (q_dtype == kF32 ? 4 : 2);
  const unsigned char* qbase = static_cast<const unsigned char*>(queries);
  if (!on_device) {
    // Host queries go through a pinned, device-mapped buffer, which a copy
    // kernel on the route's stream reads (fetch_async): a copy from
    // pageable memory stages through the runtime's own buffers (about 30 us
    // more per call for a 64 KiB query, 12 us for 32 KiB), and a copy
    // engine's transfer is handed over to the route's queue.  The buffer is
    // free again once the previous route returned (every route waits for
    // its stream before returning).
    const size_t qbytes = qstride * q_count;
    GRM_CHECK_RC(reserve_device(reinterpret_cast<unsigned char**>(&a->d_queries), &a->d_queries_bytes, qbytes));
    GRM_CHECK_RC(grm::reserve_mapped_bytes(&a->q_map, qbytes));
    memcpy(a->q_map.host, queries, qbytes);
    if (a->query_dma) {
      GRM_HIP_CHECK(hipMemcpyAsync(a->d_queries, a->q_map.host, qbytes, hipMemcpyHostToDevice, a->stream));
    } else {
      GRM_CHECK_RC(grm::fetch_async(a->d_queries, a->q_map.dev, qbytes, a->stream));
    }
    qbase = static_cast<const unsigned char*>(a->d_queries);
  }
  const uint32_t n_slots = static_cast<uint32_t>(a->high_water);
  const uint32_t fin_blocks = std::max<uint32_t>(
      1, std::min<uint32_t>((n_slots + grm::gqa::kFinSlots - 1) / grm::gqa::kFinSlots, a->fin_blocks));
  const size_t per_q = static_cast<size_t>(fin_blocks) * topk;
  GRM_CHECK_RC(grm::reserve_mapped(&a->blocks_out, per_q * q_count));
  a->merged.resize(topk);
  SrPlan plan;
  const bool use_sr = sr_plan(a, H, Qt, &plan);
  if (use_sr) GRM_CHECK_RC(prepare_sr(a, plan));
  // Screen-and-refine routes report completion through per-block flags in
  // host memory, which the host sees as soon as the last finalize block
  // stores its flag (no stream event on the path).  A timed route does too
  // when every pass is screen and refine and the device reports its
  // constant clock: its device time is then the clock's ticks from the
  // first timed kernel's start to the last flag (RouteStamps) instead of
  // stream events around the kernels (GRM_HIP_ROUTE_TIMING=events keeps
  // the events).
  const size_t n_flags = static_cast<size_t>(q_count) * fin_blocks;
  const bool flaggable = use_sr && n_flags <= kMaxDoneFlags && !grm::blocking_sync();
  const bool clocked = elapsed_ms && flaggable && a->ticks_per_ms > 0.0 && !grm::event_timing() &&
                       a->n_items > 0 && !use_bound(a, plan, std::min(plan.qb_max, q_count));
  bool flags = flaggable && (!elapsed_ms || clocked);
  unsigned* d_done = nullptr;
  if (flags) {
    GRM_CHECK_RC(grm::begin_flags(&a->done_flags, kMaxDoneFlags, &a->route_seq));
    d_done = static_cast<unsigned*>(a->done_flags.dev);
  }
  if (clocked) GRM_CHECK_RC(grm::reserve_stamps(&a->stamps, kMaxDoneFlags));
  // where each query's per-block lists are, and how many entries they hold
  std::vector<uint32_t> q_entries(q_count, static_cast<uint32_t>(per_q));
  std::vector<size_t> q_off(q_count);
  for (int qi = 0; qi < q_count; ++qi) q_off[qi] = static_cast<size_t>(qi) * per_q;
  bool bv_ready = false;
  // untimed warmup queries first, then the timed ones
  const int segments[2][2] = {{0, warmup}, {warmup, q_count}};
  for (int si = 0; si < 2; ++si) {
    const auto& seg = segments[si];
    if (si == 1 && elapsed_ms && !clocked) GRM_HIP_CHECK(hipEventRecord(a->ev_start, a->stream));
    if (use_sr) {
      for (int q0 = seg[0]; q0 < seg[1]; q0 += plan.qb_max) {
        const int qb = std::min(plan.qb_max, seg[1] - q0);
        if (use_bound(a, plan, qb)) {
          flags = false;
          if (!bv_ready) {
            GRM_CHECK_RC(prepare_bv(a, plan, topk, fin_blocks));
            bv_ready = true;
          }
          GRM_CHECK_RC(enqueue_bv(a, plan, qbase + static_cast<size_t>(q0) * qstride, q_dtype, qb,
                                  topk, fin_blocks, a->blocks_out.dev + static_cast<size_t>(q0) * per_q,
                                  per_q));
          // the candidates' lists of the pass's queries are packed back to back
          const uint32_t ent = std::min(kCandFinBlocks, fin_blocks) * topk;
          for (int j = 0; j < qb; ++j) {
            q_entries[q0 + j] = ent;
            q_off[q0 + j] = static_cast<size_t>(q0) * per_q + static_cast<size_t>(j) * ent;
          }
          a->bv_routes += 1;
        } else {
          // the timed segment's first launch stores the start tick
          grm::RouteStamps st{nullptr, nullptr};
          if (clocked) {
            st = grm::route_stamps(a->stamps, static_cast<size_t>(q0) * fin_blocks);
            if (si == 0 || q0 != seg[0]) st.start = nullptr;
          }
          GRM_CHECK_RC(enqueue_sr(a, plan, qbase + static_cast<size_t>(q0) * qstride, q_dtype, qb, topk,
                                  fin_blocks, a->blocks_out.dev + static_cast<size_t>(q0) * per_q,
                                  d_done ? d_done + static_cast<size_t>(q0) * fin_blocks : nullptr, st));
          a->sr_routes += 1;
        }
      }
    } else {
      for (int qi = seg[0]; qi < seg[1]; ++qi) {
        GRM_CHECK_RC(enqueue_exact(a, qbase + static_cast<size_t>(qi) * qstride, q_dtype, H, Qt, topk,
                                   fin_blocks, a->blocks_out.dev + static_cast<size_t>(qi) * per_q));
        a->exact_routes += 1;
      }
    }
  }
  GRM_HIP_CHECK(hipEventRecord(a->ev_stop, a->stream));
  if (flags) {
    GRM_CHECK_RC(grm::wait_flags(a->done_flags, a->route_seq, n_flags, a->ev_stop));
    for (int qi = 0; qi < q_count; ++qi) {
      GRM_CHECK_RC(grm::wait_tagged(a->blocks_out.host + q_off[qi], q_entries[qi], a->route_seq, a->ev_stop));
    }
  } else {
    GRM_CHECK_RC(grm::wait_event(a->ev_stop));
  }
  for (int qi = 0; qi < q_count; ++qi) {
    grm::host_topk_merge(a->blocks_out.host + q_off[qi], q_entries[qi], topk, a->merged.data());
    write_result(a->merged.data(), topk, out_ids + static_cast<size_t>(qi) * topk,
                 out_scores ? out_scores + static_cast<size_t>(qi) * topk : nullptr);
  }
  if (clocked) {
    GRM_CHECK_RC(grm::stamps_elapsed(a->stamps, a->route_seq, static_cast<size_t>(warmup) * fin_blocks, n_flags,
                                     a->ev_stop, a->ticks_per_ms, elapsed_ms));
  } else if (elapsed_ms) {
    GRM_HIP_CHECK(hipEventElapsedTime(elapsed_ms, a->ev_start, a->ev_stop));
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
  // The dense bank is zero-padded to key_tokens rows per (node, kv head).
  // A key row of zeros adds |q.0| = 0 to a maximum that starts at 0, so
  // the trailing tokens whose rows are zero in every kv head leave the
  // law's score unchanged and are not placed; one token always stays
  // (a node with no tokens scores 0.0 even against a non-finite query,
  // which the law scores NaN over a zero key row).
  const uint64_t rowv = static_cast<uint64_t>(kv_heads) * head_dim;  // values per token, all kv heads
  const uint64_t block = static_cast<uint64_t>(key_tokens) * rowv;
  std::vector<uint64_t> offs(static_cast<size_t>(nodes) + 1, 0);
  for (int i = 0; i < nodes; ++i) {
    const uint32_t* node = reinterpret_cast<const uint32_t*>(keys_host) + static_cast<uint64_t>(i) * block;
    uint64_t len = static_cast<uint64_t>(key_tokens);
    for (; len > 1; --len) {
      bool zero = true;
      for (int g = 0; g < kv_heads && zero; ++g) {
        const uint32_t* row = node + (static_cast<uint64_t>(g) * key_tokens + len - 1) * head_dim;
        for (int d = 0; d < head_dim; ++d) {
          if (row[d] & 0x7fffffffu) {
            zero = false;
            break;
          }
        }
      }
      if (!zero) break;
    }
    offs[i + 1] = offs[i] + len;
  }
  return create_arena(keys_host, kF32, nullptr, kF32, 0, offs.data(), static_cast<uint64_t>(nodes),
                      kv_heads, head_dim, nullptr, static_cast<uint64_t>(nodes), offs.back(),
                      out_arena, static_cast<uint64_t>(key_tokens));
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
      if (tok_counts[i] > 0xffffffffull - 8) return grm::fail(-1, "node too long");
      tokens += padded_len(tok_counts[i]);
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
  // a slot taken by an append starts with no route filter bits
  if (!a->fbits.empty()) {
    for (uint64_t sl : slots) {
      if (sl < a->fbits.size() && a->fbits[sl] != 0) {
        a->fbits[sl] = 0;
        a->fbits_dirty = true;
      }
    }
  }
  // the route work lists follow the host mirrors; rebuilding them here
  // keeps the next route from paying for it
  GRM_CHECK_RC(ensure_items(a));
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
  GRM_CHECK_RC(ensure_items(a));  // as after an append
  if (out_epoch) *out_epoch = a->epoch;
  grm::clear_error();
  return 0;
}

namespace grm {
// Whether appending nodes of tok_counts[0, count) fits once the live ids
// drop[0, n_drop) are evicted, compacting the token arena if it must (the
// device store checks this before it replaces an entry's keys, so a
// replace that cannot fit leaves the old entry in place).
bool gqa_append_fits(const GqaDeviceArena* a, const uint64_t* drop, uint64_t n_drop,
                     const uint64_t* tok_counts, uint64_t count) {
  uint64_t dropped = 0, drop_pad = 0;
  for (uint64_t i = 0; i < n_drop; ++i) {
    auto it = a->slot_of.find(drop[i]);
    if (it == a->slot_of.end()) continue;
    dropped += 1;
    drop_pad += padded_len(a->len[it->second]);
  }
  const uint64_t room = a->free_slots.size() + (a->cap_nodes - a->high_water) + dropped;
  if (count > room) return false;
  uint64_t need = 0;
  for (uint64_t i = 0; i < count; ++i) need += padded_len(tok_counts[i]);
  if (need <= a->cap_tokens - a->used_tokens) return true;
  uint64_t live_pad = 0;  // what a compaction keeps
  for (const auto& kv : a->slot_of) live_pad += padded_len(a->len[kv.second]);
  return live_pad - drop_pad + need <= a->cap_tokens;
}
}  // namespace grm

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
  const size_t hb = a->d_skeys ? row_values(a) * 2 : 0;  // fp16 copy bytes per token
  uint64_t dst = 0;
  std::vector<uint64_t> new_off(order.size());
  for (size_t i = 0; i < order.size(); ++i) {
    const uint64_t s = order[i];
    const uint64_t src = a->tok_off[s];
    const uint64_t n = padded_len(a->len[s]);
    if (src != dst && n > 0) {
      if (src - dst >= n) {
        GRM_HIP_CHECK(hipMemcpyAsync(a->d_keys + dst * kb, a->d_keys + src * kb, n * kb,
                                     hipMemcpyDeviceToDevice, a->stream));
        if (sb) {
          GRM_HIP_CHECK(hipMemcpyAsync(a->d_scales + dst * sb, a->d_scales + src * sb, n * sb,
                                       hipMemcpyDeviceToDevice, a->stream));
        }
        if (hb) {
          GRM_HIP_CHECK(hipMemcpyAsync(a->d_skeys + dst * hb, a->d_skeys + src * hb, n * hb,
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
          if (hb) {
            GRM_HIP_CHECK(hipMemcpyAsync(a->d_skeys + (dst + t) * hb, a->d_skeys + (src + t) * hb,
                                         hb, hipMemcpyDeviceToDevice, a->stream));
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
  GRM_CHECK_RC(ensure_items(a));  // as after an append
  grm::clear_error();
  return 0;
}

extern "C" int grm_gqa_hip_sync(GqaDeviceArena* a) {
  if (!a) return grm::fail(-1, "null arena");
  GRM_HIP_CHECK(hipSetDevice(a->device));
  return wait_mutations(a);
}

// ---------------------------------------------------------------- store route

namespace {

// Upload the host copy of the route filter bits when it changed.
int sync_filter_bits(GqaDeviceArena* a) {
  if (a->fbits.size() < a->cap_nodes) {
    a->fbits.resize(a->cap_nodes, 0);
    a->fbits_dirty = true;
  }
  if (!a->d_fbits || a->fbits_dirty) {
    GRM_CHECK_RC(reserve_device(&a->d_fbits, &a->d_fbits_count, a->cap_nodes));
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_fbits, a->fbits.data(), a->cap_nodes * sizeof(uint64_t),
                                 hipMemcpyHostToDevice, a->stream));
    a->fbits_dirty = false;
  }
  return 0;
}

}  // namespace

extern "C" int grm_gqa_hip_set_filter_bits(GqaDeviceArena* a, const uint64_t* node_ids,
                                           const uint64_t* bits, uint64_t count) {
  if (!a || (count > 0 && (!node_ids || !bits))) return grm::fail(-1, "invalid arguments");
  if (a->fbits.size() < a->cap_nodes) a->fbits.resize(a->cap_nodes, 0);
  std::vector<uint64_t> slots(count);
  for (uint64_t i = 0; i < count; ++i) {
    auto it = a->slot_of.find(node_ids[i]);
    if (it == a->slot_of.end()) return grm::fail(-1, "filter bits for an id that is not live");
    slots[i] = it->second;
  }
  for (uint64_t i = 0; i < count; ++i) a->fbits[slots[i]] = bits[i];
  if (count > 0) a->fbits_dirty = true;
  grm::clear_error();
  return 0;
}

extern "C" int grm_gqa_hip_route_filtered(GqaDeviceArena* a, const void* query, int query_dtype,
                                          int query_on_device, int query_heads, int query_tokens,
                                          int topk, uint64_t filter_mask, uint32_t filter_categories,
                                          uint64_t* out_ids_host, float* out_scores_host,
                                          float* elapsed_ms_host) {
  if (!a) return grm::fail(-1, "null arena");
  if (filter_categories & ~0xfu) return grm::fail(-1, "filter categories are bits 0..3");
  if (filter_categories == 0) {
    return route_impl(a, query, query_dtype, query_on_device != 0, 1, query_heads, query_tokens,
                      0, topk, out_ids_host, out_scores_host, elapsed_ms_host);
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  GRM_CHECK_RC(sync_filter_bits(a));
  GRM_CHECK_RC(reserve_device(&a->d_fflags, &a->d_fflags_count, a->cap_nodes));
  if (a->mut_pending) GRM_HIP_CHECK(hipStreamWaitEvent(a->stream, a->ev_mut, 0));
  const uint64_t n = a->high_water;
  if (n > 0) {
    const unsigned blocks = static_cast<unsigned>(std::min<uint64_t>((n + 255) / 256, 4096));
    grm::gqa::gqa_filter_flags_kernel<<<blocks, 256, 0, a->stream>>>(
        a->d_flags, a->d_fbits, n, filter_mask, filter_categories, a->d_fflags);
    GRM_HIP_CHECK(hipGetLastError());
  }
  a->route_flags = a->d_fflags;
  const int rc = route_impl(a, query, query_dtype, query_on_device != 0, 1, query_heads,
                            query_tokens, 0, topk, out_ids_host, out_scores_host, elapsed_ms_host);
  a->route_flags = nullptr;
  return rc;
}

extern "C" int grm_gqa_hip_score_nodes(GqaDeviceArena* a, const void* query_host, int query_dtype,
                                       int query_heads, int query_tokens, const uint64_t* node_ids,
                                       uint64_t count, float* out_scores_host) {
  if (!a || !query_host || (count > 0 && (!node_ids || !out_scores_host))) {
    return grm::fail(-1, "invalid arguments");
  }
  if (query_dtype != kF32 && query_dtype != kBF16) return grm::fail(-1, "query dtype must be F32 or BF16");
  if (query_heads <= 0 || query_tokens <= 0 || query_heads % static_cast<int>(a->kv) != 0) {
    return grm::fail(-1, "need heads, tokens > 0 and heads % kv_heads == 0");
  }
  if (count == 0) return 0;
  // distinct slots (a slot's maxima are read once), results mapped back
  std::vector<uint32_t> slots;
  std::unordered_map<uint64_t, uint32_t> pos;
  std::vector<uint32_t> where(count);
  for (uint64_t i = 0; i < count; ++i) {
    auto it = a->slot_of.find(node_ids[i]);
    if (it == a->slot_of.end()) return grm::fail(-1, "score of an id that is not live");
    auto ins = pos.emplace(it->second, static_cast<uint32_t>(slots.size()));
    if (ins.second) slots.push_back(static_cast<uint32_t>(it->second));
    where[i] = ins.first->second;
  }
  std::vector<Item> items;
  for (uint32_t sl : slots) {
    if (a->len[sl] > 0) append_items(items, sl, a->tok_off[sl] * a->kv, a->len[sl], a->chunk);
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  GRM_CHECK_RC(wait_mutations(a));
  const int H = query_heads;
  const int Qt = query_tokens;
  const size_t qbytes = static_cast<size_t>(H) * Qt * a->hd * (query_dtype == kF32 ? 4 : 2);
  GRM_CHECK_RC(reserve_device(reinterpret_cast<unsigned char**>(&a->d_queries), &a->d_queries_bytes,
                              qbytes));
  GRM_CHECK_RC(reserve_device(&a->d_sitems, &a->d_sitems_count, items.size() + 1));
  GRM_CHECK_RC(reserve_device(&a->d_sslots, &a->d_sslots_count, slots.size() + 1));
  GRM_CHECK_RC(reserve_device(&a->d_sout, &a->d_sout_count, slots.size()));
  GRM_CHECK_RC(ensure_hmax(a, H, 1));
  GRM_HIP_CHECK(hipMemcpyAsync(a->d_queries, query_host, qbytes, hipMemcpyHostToDevice, a->stream));
  // slot list, then the item count behind it (the exact kernel reads its
  // item count from the device)
  std::vector<uint32_t> sl_and_count(slots);
  sl_and_count.push_back(static_cast<uint32_t>(items.size()));
  GRM_HIP_CHECK(hipMemcpyAsync(a->d_sslots, sl_and_count.data(), sl_and_count.size() * sizeof(uint32_t),
                               hipMemcpyHostToDevice, a->stream));
  if (!items.empty()) {
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_sitems, items.data(), items.size() * sizeof(Item),
                                 hipMemcpyHostToDevice, a->stream));
  }
  const auto passes = query_passes(H / static_cast<int>(a->kv), Qt, grm::gqa::kMaxRQ);
  for (size_t i = 0; i < passes.size(); ++i) {
    GRM_CHECK_RC(launch_q64(a, a->d_queries, query_dtype, 1, H, Qt, passes[i], i > 0));
    if (!items.empty()) {
      GRM_CHECK_RC(launch_exact(a, H, passes[i], a->d_sitems, items.size(),
                                a->d_sslots + slots.size()));
    }
  }
  const unsigned blocks = static_cast<unsigned>((slots.size() + 255) / 256);
  grm::gqa::gqa_slot_scores_kernel<<<blocks, 256, 0, a->stream>>>(
      a->d_hmax, a->cap_nodes, H, a->d_sslots, slots.size(), a->d_len, a->d_flags, a->d_qbad,
      static_cast<int>(a->kv), a->d_sout);
  GRM_HIP_CHECK(hipGetLastError());
  std::vector<float> out(slots.size());
  GRM_HIP_CHECK(hipMemcpyAsync(out.data(), a->d_sout, out.size() * sizeof(float), hipMemcpyDeviceToHost,
                               a->stream));
  GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
  for (uint64_t i = 0; i < count; ++i) out_scores_host[i] = out[where[i]];
  grm::clear_error();
  return 0;
}

extern "C" int grm_gqa_hip_route_stats(GqaDeviceArena* a, uint64_t* out4) {
  if (!a || !out4) return grm::fail(-1, "null argument");
  out4[0] = a->routes;
  out4[1] = a->sr_routes;
  out4[2] = a->bv_routes;
  out4[3] = a->exact_routes;
  return 0;
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

// ------------------------------------------------------- screen-bound probe
//
// Test entry: runs the screen-only kernel of the bound-and-verify path (one
// query, one pass: heads/kv_heads x query_tokens <= 64 columns per kv head)
// over every node with key tokens and returns, per (slot < node capacity,
// kv head g,
// column cg = r*Qt + t of head g*R + r at query token t), the largest
// screened value over the node's tokens in the screen's scaled units,
// out_maxima[(slot*kv + g)*R*Qt + cg] (0 for nodes without tokens); per
// column the bound parameters {coef, eabs, scale, kcap},
// out_colinfo[(g*R*Qt + cg)*4 ..]; per slot the key norm bound K the
// bound uses, out_knorm[slot]; and the slots' node ids.  For every node
// with K < kcap the screen obeys |m - scale * max_t |q.k_t|| <= coef * K +
// eabs.  Not on any route path; allocates its own query buffer.
extern "C" int grm_gqa_hip_probe_screen(GqaDeviceArena* a, const void* query_host, int query_dtype,
                                        int query_heads, int query_tokens, float* out_maxima_host,
                                        float* out_colinfo_host, double* out_knorm_host,
                                        uint64_t* out_slot_ids_host) {
  if (!a || !query_host || !out_maxima_host || !out_colinfo_host || !out_knorm_host) {
    return grm::fail(-1, "null argument");
  }
  if (query_dtype != kF32 && query_dtype != kBF16) return grm::fail(-1, "query dtype must be F32 or BF16");
  if (query_heads <= 0 || query_tokens <= 0 || query_heads % static_cast<int>(a->kv) != 0) {
    return grm::fail(-1, "need heads, tokens > 0 and heads % kv_heads == 0");
  }
  SrPlan p;
  if (!sr_plan(a, query_heads, query_tokens, &p) || p.passes.size() != 1) {
    return grm::fail(-1, "bank or query has no screen pass (bf16/f16/int8 keys, head_dim 64/128/256, <= 64 columns)");
  }
  const uint64_t n = a->cap_nodes;
  const int colstride = p.R * p.Qt;
  GRM_HIP_CHECK(hipSetDevice(a->device));
  struct Buf {
    void* p = nullptr;
    ~Buf() {
      if (p) (void)hipFree(p);
    }
  } d_q;
  const size_t qbytes = static_cast<size_t>(query_heads) * query_tokens * a->hd * (query_dtype == kF32 ? 4 : 2);
  GRM_HIP_CHECK(hipMalloc(&d_q.p, qbytes));
  const size_t cells = static_cast<size_t>(a->cap_nodes) * a->kv * colstride;
  GRM_CHECK_RC(reserve_device(&a->d_hmaxf, &a->d_hmaxf_count, cells));
  GRM_CHECK_RC(reserve_device(&a->d_colinfo, &a->d_colinfo_count,
                              static_cast<size_t>(a->kv) * grm::gqa::kMaxCols));
  if (a->mut_pending) GRM_HIP_CHECK(hipStreamWaitEvent(a->stream, a->ev_mut, 0));
  GRM_CHECK_RC(ensure_items(a));
  if (a->n_units == 0) return grm::fail(-1, "no node has key tokens");
  GRM_HIP_CHECK(hipMemcpyAsync(d_q.p, query_host, qbytes, hipMemcpyHostToDevice, a->stream));
  GRM_HIP_CHECK(hipMemsetAsync(a->d_hmaxf, 0, cells * sizeof(unsigned), a->stream));
  GRM_CHECK_RC(launch_smax(a, p, static_cast<const unsigned char*>(d_q.p), query_dtype, 1, colstride,
                           &p.passes[0], 1));
  const size_t out_cells = static_cast<size_t>(n) * a->kv * colstride;
  GRM_HIP_CHECK(hipMemcpyAsync(out_maxima_host, a->d_hmaxf, out_cells * sizeof(float),
                               hipMemcpyDeviceToHost, a->stream));
  GRM_HIP_CHECK(hipMemcpyAsync(out_colinfo_host, a->d_colinfo,
                               static_cast<size_t>(a->kv) * colstride * sizeof(float4),
                               hipMemcpyDeviceToHost, a->stream));
  std::vector<unsigned> km(n);
  GRM_HIP_CHECK(hipMemcpyAsync(km.data(), a->d_kmax, n * sizeof(unsigned), hipMemcpyDeviceToHost,
                               a->stream));
  if (out_slot_ids_host) {
    GRM_HIP_CHECK(hipMemcpyAsync(out_slot_ids_host, a->d_ids, n * sizeof(uint64_t),
                                 hipMemcpyDeviceToHost, a->stream));
  }
  GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
  const bool fact = a->key_dtype == kI8 && static_cast<uint32_t>(a->group_size) == a->hd;
  for (uint64_t s = 0; s < n; ++s) {
    float f;
    memcpy(&f, &km[s], sizeof(f));
    out_knorm_host[s] = grm::gqa::screen_key_norm(f, fact, static_cast<int>(a->hd));
  }
  grm::clear_error();
  return 0;
}
