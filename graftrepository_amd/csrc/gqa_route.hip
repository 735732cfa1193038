// gqa_route.hip -- ragged GQA route on gfx950: bank lifecycle, route
// orchestration and the C ABI.  Device code lives in gqa_kernels.hpp.
//
// Bank layout in HBM: ragged CSR.  Node slot i owns tokens
// [tok_off[i], tok_off[i]+len[i]) of the token arena; its block is
// [kv][len][hd] values of the storage dtype (f32, bf16, f16 or int8 codes
// with per-(token, group) scales).  No padding is stored or read.
//
// Route (bf16 / fp16 / int8 banks, head_dim 64, 128 or 256):
//   prep -> screen (MFMA, all key tokens) -> select -> shortlist/certify ->
//   exact rescore of the shortlist -> exact finalize; the host merges the
//   shortlist's exact scores.  A query whose shortlist is not certified, or
//   whose values are non-finite or leave the fp16 range, is routed again
//   on the exact path, so every result follows the law.
// Route (fp32 banks and other shapes): exact path over every node.
#include "gqa_kernels.hpp"
#include "grm_hip_router.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
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
  uint32_t* d_flags = nullptr;  // bit 0 live, bit 1 all key values finite
  uint32_t* d_nonfinite = nullptr;
  unsigned* d_kmax = nullptr;   // float bits: max key norm per slot
  // host mirrors
  std::vector<uint64_t> tok_off;
  std::vector<uint32_t> len;
  std::vector<uint64_t> slot_id;  // kNoId when free
  std::unordered_map<uint64_t, uint64_t> slot_of;
  std::set<uint64_t> free_slots;
  // route work list, rebuilt when the epoch moves
  uint32_t chunk = 64;  // key tokens per work item
  Item* d_items = nullptr;
  size_t d_items_count = 0;
  uint64_t n_items = 0;
  uint64_t items_epoch = ~0ull;
  uint32_t max_len = 0;  // longest live node
  // exact path
  unsigned long long* d_hmax = nullptr;
  size_t d_hmax_count = 0;
  int hmax_heads = 0;
  grm::MappedCands blocks_out;  // per-query, per-block top-k (host mapped)
  unsigned* d_qbad = nullptr;   // set when a query value is non-finite
  // screen path
  bool screen = true;
  u32x4* d_bfrag = nullptr;
  size_t d_bfrag_count = 0;
  float* d_coef = nullptr;
  size_t d_coef_count = 0;
  unsigned* d_qflags = nullptr;
  size_t d_qflags_count = 0;
  unsigned* d_hms = nullptr;
  size_t d_hms_count = 0;
  int hms_heads = 0;
  Cand* d_bu = nullptr;
  size_t d_bu_count = 0;
  Cand* d_bl = nullptr;
  size_t d_bl_count = 0;
  uint32_t* d_shortlist = nullptr;
  size_t d_shortlist_count = 0;
  unsigned long long* d_hex = nullptr;
  size_t d_hex_count = 0;
  grm::MappedCands short_out;  // exact scores of the shortlists (host mapped)
  grm::MappedBuf qstate;       // per query: prep flags, then status (host mapped)
  uint32_t sel_blocks = 256;
  uint32_t screen_waves = 8192;  // persistent screen wavefronts (all kv heads)
  uint64_t routes = 0;          // route calls
  uint64_t fallbacks = 0;       // queries re-routed on the exact path
  std::vector<Cand> merged;
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
  void* dev[] = {a->d_keys,  a->d_scales, a->d_tok_off, a->d_len,   a->d_ids,
                 a->d_flags, a->d_nonfinite, a->d_kmax, a->d_items, a->d_hmax,
                 a->d_qbad,  a->d_queries, a->d_stage,  a->d_bfrag, a->d_coef,
                 a->d_hms,   a->d_bu,     a->d_bl,      a->d_shortlist, a->d_hex,
                 a->d_qflags};
  for (void* p : dev) {
    if (p) (void)hipFree(p);
  }
  grm::release_mapped(&a->blocks_out);
  grm::release_mapped(&a->short_out);
  grm::release_mapped_bytes(&a->qstate);
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

void append_items(std::vector<Item>& items, uint32_t slot, uint64_t base, uint64_t len,
                  uint32_t chunk) {
  for (uint64_t t0 = 0; t0 < len; t0 += chunk) {
    Item it;
    it.base = base;
    it.slot = slot;
    it.t0 = static_cast<uint32_t>(t0);
    it.count = static_cast<uint32_t>(std::min<uint64_t>(chunk, len - t0));
    it.len = static_cast<uint32_t>(len);
    items.push_back(it);
  }
}

int launch_stats(GqaDeviceArena* a, const Item* d_items, uint64_t n_items, hipStream_t st) {
  if (n_items == 0) return 0;
  const dim3 grid(static_cast<unsigned>((n_items + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves), a->kv);
  const unsigned threads = grm::gqa::kUnitWaves * grm::kWave;
#define GRM_STATS(KDT)                                                              \
  grm::gqa::gqa_key_stats_kernel<KDT><<<grid, threads, 0, st>>>(                    \
      a->d_keys, a->d_scales, a->scale_dtype, a->group_size, d_items,               \
      static_cast<uint32_t>(n_items), static_cast<int>(a->hd), a->d_nonfinite, a->d_kmax)
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
      a->d_nonfinite, a->d_kmax);
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
  // Larger banks use longer work items so the grid stays near a few
  // hundred thousand wavefronts.
  a->chunk = cap_tokens * a->kv > (8ull << 20) ? 256 : 64;
  if (const char* env = getenv("GRM_HIP_GQA_CHUNK")) {
    const long v = strtol(env, nullptr, 10);
    if (v >= 16 && v <= 4096 && v % 16 == 0) a->chunk = static_cast<uint32_t>(v);
  }
  if (const char* env = getenv("GRM_HIP_GQA_SCREEN")) a->screen = env[0] != '0';
  {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, a->device) != hipSuccess ||
        cus <= 0) {
      cus = 256;
    }
    a->screen_waves = static_cast<uint32_t>(cus) * 16;  // 4 per SIMD
  }
  if (const char* env = getenv("GRM_HIP_GQA_SCREEN_WAVES")) {
    const long v = strtol(env, nullptr, 10);
    if (v >= 64 && v <= (1l << 22)) a->screen_waves = static_cast<uint32_t>(v);
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
  if (key_dtype == kI8) {
    BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_scales), std::max<size_t>(16, cap_tokens * token_scale_bytes(a))));
  }
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_tok_off), cap_nodes * sizeof(uint64_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_len), cap_nodes * sizeof(uint32_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_ids), cap_nodes * sizeof(uint64_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_flags), cap_nodes * sizeof(uint32_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_nonfinite), cap_nodes * sizeof(uint32_t)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_kmax), cap_nodes * sizeof(unsigned)));
  BAIL_HIP(hipMalloc(reinterpret_cast<void**>(&a->d_qbad), sizeof(unsigned)));
  BAIL_HIP(hipMemsetAsync(a->d_tok_off, 0, cap_nodes * sizeof(uint64_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_len, 0, cap_nodes * sizeof(uint32_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_ids, 0xff, cap_nodes * sizeof(uint64_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_flags, 0, cap_nodes * sizeof(uint32_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_nonfinite, 0, cap_nodes * sizeof(uint32_t), a->stream));
  BAIL_HIP(hipMemsetAsync(a->d_kmax, 0, cap_nodes * sizeof(unsigned), a->stream));
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
  std::vector<Item> items;
  items.reserve(a->live * 2);
  uint32_t max_len = 0;
  for (uint64_t s = 0; s < a->high_water; ++s) {
    if (a->slot_id[s] == kNoId) continue;
    append_items(items, static_cast<uint32_t>(s), a->tok_off[s] * a->kv, a->len[s], a->chunk);
    max_len = std::max(max_len, a->len[s]);
  }
  GRM_CHECK_RC(reserve_device(&a->d_items, &a->d_items_count, items.size()));
  if (!items.empty()) {
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_items, items.data(), items.size() * sizeof(Item),
                                 hipMemcpyHostToDevice, a->stream));
    GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
  }
  a->n_items = items.size();
  a->max_len = max_len;
  a->items_epoch = a->epoch;
  return 0;
}

int rq_pad_of(int rq) {
  int p = 1;
  while (p < rq) p *= 2;
  return p;
}

// --------------------------------------------------------------- exact path

int launch_exact_heads(GqaDeviceArena* a, const void* q, int q_dtype, int H, int Qt) {
  if (a->n_items == 0) return 0;
  const int R = H / static_cast<int>(a->kv);
  const int rq_pad = rq_pad_of(R * Qt);
  const dim3 grid(static_cast<unsigned>((a->n_items + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves), a->kv);
  const unsigned threads = grm::gqa::kUnitWaves * grm::kWave;
  const size_t lds = static_cast<size_t>(rq_pad) * a->hd * sizeof(double);
  const double denom = sqrt(static_cast<double>(a->hd));
#define GRM_EXACT(KDT, RQ)                                                                  \
  grm::gqa::gqa_exact_heads_kernel<KDT, RQ><<<grid, threads, lds, a->stream>>>(            \
      a->d_keys, a->d_scales, a->scale_dtype, a->group_size, a->d_items,                   \
      static_cast<uint32_t>(a->n_items), static_cast<int>(a->hd), R, Qt, q, q_dtype, denom,  \
      a->d_hmax, a->cap_nodes, a->d_qbad)
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

// Enqueue the exact route of one query; its per-block top-k lands in
// blocks_out at `bout`.
int enqueue_exact(GqaDeviceArena* a, const void* q, int q_dtype, int H, int Qt, int topk,
                  uint32_t fin_blocks, Cand* bout) {
  if (a->hmax_heads != H || a->d_hmax_count < a->cap_nodes * static_cast<size_t>(H)) {
    GRM_CHECK_RC(reserve_device(&a->d_hmax, &a->d_hmax_count, a->cap_nodes * static_cast<size_t>(H)));
    GRM_HIP_CHECK(hipMemsetAsync(a->d_hmax, 0, a->d_hmax_count * sizeof(unsigned long long), a->stream));
    a->hmax_heads = H;
  }
  GRM_CHECK_RC(launch_exact_heads(a, q, q_dtype, H, Qt));
  const uint32_t per_block = grm::gqa::kFinWaves * grm::kWave;
  grm::gqa::gqa_finalize_kernel<<<fin_blocks, per_block, 0, a->stream>>>(
      a->d_hmax, a->cap_nodes, H, static_cast<uint32_t>(a->high_water), a->d_len, a->d_flags,
      a->d_ids, a->d_qbad, topk, bout);
  GRM_HIP_CHECK(hipGetLastError());
  grm::gqa::gqa_clear_flags_kernel<<<1, 64, 0, a->stream>>>(a->d_qbad, 1);
  GRM_HIP_CHECK(hipGetLastError());
  return 0;
}

void write_result(const Cand* merged, int topk, uint64_t* out_ids, float* out_scores) {
  for (int j = 0; j < topk; ++j) {
    const Cand& c = merged[j];
    const bool ok = isfinite(c.score) && c.id != kNoId;
    out_ids[j] = ok ? c.id : kNoId;
    if (out_scores) out_scores[j] = ok ? c.score : __builtin_nanf("");
  }
}

// -------------------------------------------------------------- screen path

struct ScreenPlan {
  int R = 0, Qt = 0, H = 0;
  int KS = 0;        // head_dim / 32
  int qb_max = 0;    // queries per screen pass (<= 64 columns)
  int M = 0;         // shortlist length
  int mfma = kBF16;  // MFMA operand type
};

bool screen_plan(const GqaDeviceArena* a, int H, int Qt, int topk, ScreenPlan* p) {
  if (!a->screen || a->key_dtype == kF32) return false;
  if (a->hd != 64 && a->hd != 128 && a->hd != 256) return false;
  const int R = H / static_cast<int>(a->kv);
  if (R * Qt > 64) return false;
  p->R = R;
  p->Qt = Qt;
  p->H = H;
  p->KS = static_cast<int>(a->hd / 32);
  p->qb_max = std::max(1, 64 / (R * Qt));
  p->M = std::min(grm::gqa::kMaxShort - 1, std::max(16, 2 * topk));
  p->mfma = a->key_dtype == kBF16 ? kBF16 : kF16;
  return true;
}

// Enqueue the screen route of queries [q0, q0+qb) of a call of q_total
// queries (device pointer `qbase`, `qstride` bytes per query).  Shortlist
// exact scores land in short_out at q0*M; qstate holds the queries' prep
// flags at [q] and certificate status at [q_total + q].
int enqueue_screen(GqaDeviceArena* a, const ScreenPlan& p, const unsigned char* qbase,
                   size_t qstride, int q_dtype, int q0, int qb, int q_total, int topk) {
  const int kv = static_cast<int>(a->kv);
  const int cols = qb * p.R * p.Qt;
  const int NT = (cols + 15) / 16;
  const int ntp = NT <= 1 ? 1 : (NT <= 2 ? 2 : 4);
  const int H = p.H;
  const int M = p.M;
  const int mU = M + 1;
  GRM_CHECK_RC(reserve_device(&a->d_bfrag, &a->d_bfrag_count,
                              static_cast<size_t>(kv) * ntp * p.KS * grm::kWave));
  GRM_CHECK_RC(reserve_device(&a->d_coef, &a->d_coef_count, static_cast<size_t>(p.qb_max)));
  if (a->hms_heads != H || a->d_hms_count < static_cast<size_t>(p.qb_max) * a->cap_nodes * H) {
    a->d_hms_count = 0;
    GRM_CHECK_RC(reserve_device_zero(&a->d_hms, &a->d_hms_count,
                                     static_cast<size_t>(p.qb_max) * a->cap_nodes * H, a->stream));
    a->hms_heads = H;
  }
  const uint32_t n_slots = static_cast<uint32_t>(a->high_water);
  const uint32_t per_block = grm::gqa::kFinWaves * grm::kWave;
  const uint32_t nblk = std::max<uint32_t>(1, std::min<uint32_t>((n_slots + per_block - 1) / per_block, a->sel_blocks));
  GRM_CHECK_RC(reserve_device(&a->d_bu, &a->d_bu_count, static_cast<size_t>(qb) * nblk * mU));
  GRM_CHECK_RC(reserve_device(&a->d_bl, &a->d_bl_count, static_cast<size_t>(qb) * nblk * topk));
  GRM_CHECK_RC(reserve_device(&a->d_shortlist, &a->d_shortlist_count, static_cast<size_t>(p.qb_max) * M));
  if (a->d_hex_count < static_cast<size_t>(p.qb_max) * M * H) {
    a->d_hex_count = 0;
    GRM_CHECK_RC(reserve_device_zero(&a->d_hex, &a->d_hex_count, static_cast<size_t>(p.qb_max) * M * H,
                                     a->stream));
  }
  GRM_CHECK_RC(reserve_device(&a->d_qflags, &a->d_qflags_count, static_cast<size_t>(p.qb_max)));
  // 1. query prep (fragments, error coefficient, flags)
  grm::gqa::gqa_clear_flags_kernel<<<(qb + 63) / 64, 64, 0, a->stream>>>(a->d_qflags, qb);
  GRM_HIP_CHECK(hipGetLastError());
  const unsigned char* qptr = qbase + static_cast<size_t>(q0) * qstride;
  const double gamma = 2.0 * (a->hd + 2.0 * p.KS) * ldexp(1.0, -24);
  double delta = 0.0, sigma = 0.0;
  if (p.mfma == kBF16) {
    delta = q_dtype == kF32 ? ldexp(1.0, -8) : 0.0;
    sigma = ldexp(1.0, -130);
  } else {
    delta = q_dtype == kF32 ? ldexp(1.0, -11) : 0.0;
    sigma = ldexp(1.0, -25);
  }
  if (p.mfma == kBF16) {
    grm::gqa::gqa_query_prep_kernel<kBF16><<<kv + qb, 256, 0, a->stream>>>(
        qptr, q_dtype, qb, H, p.Qt, static_cast<int>(a->hd), kv, p.R, ntp, p.KS, a->d_bfrag,
        a->d_qflags, a->d_coef, gamma, delta, sigma);
  } else {
    grm::gqa::gqa_query_prep_kernel<kF16><<<kv + qb, 256, 0, a->stream>>>(
        qptr, q_dtype, qb, H, p.Qt, static_cast<int>(a->hd), kv, p.R, ntp, p.KS, a->d_bfrag,
        a->d_qflags, a->d_coef, gamma, delta, sigma);
  }
  GRM_HIP_CHECK(hipGetLastError());
  // 2. screen
  if (a->n_items > 0) {
    // Persistent stream: about screen_waves wavefronts in all, spread over
    // the kv heads (grid y); each walks items w, w+W, ...
    const uint64_t per_plane = std::max<uint64_t>(1, a->screen_waves / a->kv);
    const uint64_t bx = std::min<uint64_t>((a->n_items + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves,
                                           (per_plane + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves);
    const dim3 grid(static_cast<unsigned>(std::max<uint64_t>(1, bx)), a->kv);
    const unsigned threads = grm::gqa::kUnitWaves * grm::kWave;
    const size_t hstride = a->cap_nodes * static_cast<size_t>(H);
#define GRM_SCREEN(KDT, KS, NTT)                                                              \
  grm::gqa::gqa_screen_kernel<KDT, KS, NTT><<<grid, threads, 0, a->stream>>>(                 \
      a->d_keys, a->d_scales, a->scale_dtype, a->group_size, a->d_items,                      \
      static_cast<uint32_t>(a->n_items), p.R, p.Qt, cols, a->d_bfrag, a->d_hms, hstride,      \
      a->cap_nodes)
#define GRM_SCREEN_NT(KDT, KS)                 \
  switch (ntp) {                               \
    case 1: GRM_SCREEN(KDT, KS, 1); break;     \
    case 2: GRM_SCREEN(KDT, KS, 2); break;     \
    default: GRM_SCREEN(KDT, KS, 4); break;    \
  }
#define GRM_SCREEN_KS(KDT)                     \
  switch (p.KS) {                              \
    case 2: GRM_SCREEN_NT(KDT, 2); break;      \
    case 4: GRM_SCREEN_NT(KDT, 4); break;      \
    default: GRM_SCREEN_NT(KDT, 8); break;     \
  }
    switch (a->key_dtype) {
      case kBF16: GRM_SCREEN_KS(kBF16); break;
      case kF16: GRM_SCREEN_KS(kF16); break;
      default: GRM_SCREEN_KS(kI8); break;
    }
#undef GRM_SCREEN_KS
#undef GRM_SCREEN_NT
#undef GRM_SCREEN
    GRM_HIP_CHECK(hipGetLastError());
  }
  // 3. select, 4. shortlist + certificate
  const float inv_scale = static_cast<float>(1.0 / (H * sqrt(static_cast<double>(a->hd))));
  const float slack_rel = static_cast<float>((H + 8) * ldexp(1.0, -22));
  grm::gqa::gqa_select_kernel<<<dim3(nblk, qb), per_block, 0, a->stream>>>(
      a->d_hms, a->cap_nodes * static_cast<size_t>(H), a->cap_nodes, H, n_slots, a->d_len,
      a->d_flags, a->d_ids,
      reinterpret_cast<const float*>(a->d_kmax), a->d_coef, inv_scale, slack_rel, mU, topk,
      a->d_bu, a->d_bl);
  GRM_HIP_CHECK(hipGetLastError());
  unsigned* out_flags = static_cast<unsigned*>(a->qstate.dev) + q0;
  unsigned* out_status = static_cast<unsigned*>(a->qstate.dev) + q_total + q0;
  grm::gqa::gqa_shortlist_kernel<<<qb, per_block, 0, a->stream>>>(
      a->d_bu, a->d_bl, nblk, mU, topk, M, a->d_shortlist, a->d_qflags, out_flags, out_status);
  GRM_HIP_CHECK(hipGetLastError());
  // 5. exact rescore of the shortlist, 6. exact scores out
  const int rq_pad = rq_pad_of(p.R * p.Qt);
  const uint32_t max_chunks = std::max<uint32_t>(1, (a->max_len + grm::kWave - 1) / grm::kWave);
  const uint64_t units = static_cast<uint64_t>(qb) * M * max_chunks;
  const dim3 rgrid(static_cast<unsigned>((units + grm::gqa::kUnitWaves - 1) / grm::gqa::kUnitWaves), a->kv);
  const size_t lds = static_cast<size_t>(grm::gqa::kUnitWaves) * rq_pad * a->hd * sizeof(double);
  const double denom = sqrt(static_cast<double>(a->hd));
  const size_t q_elems = static_cast<size_t>(H) * p.Qt * a->hd;
#define GRM_RESCORE(KDT, RQ)                                                                  \
  grm::gqa::gqa_rescore_kernel<KDT, RQ><<<rgrid, grm::gqa::kUnitWaves * grm::kWave, lds, a->stream>>>( \
      a->d_keys, a->d_scales, a->scale_dtype, a->group_size, a->d_tok_off, a->d_len,           \
      a->d_shortlist, M, qb, max_chunks, kv, static_cast<int>(a->hd), p.R, p.Qt, qptr,          \
      q_dtype, q_elems, denom, a->d_hex)
#define GRM_RESCORE_RQ(KDT)                     \
  switch (rq_pad) {                             \
    case 1: GRM_RESCORE(KDT, 1); break;         \
    case 2: GRM_RESCORE(KDT, 2); break;         \
    case 4: GRM_RESCORE(KDT, 4); break;         \
    case 8: GRM_RESCORE(KDT, 8); break;         \
    case 16: GRM_RESCORE(KDT, 16); break;       \
    default: GRM_RESCORE(KDT, 32); break;       \
  }
  switch (a->key_dtype) {
    case kBF16: GRM_RESCORE_RQ(kBF16); break;
    case kF16: GRM_RESCORE_RQ(kF16); break;
    default: GRM_RESCORE_RQ(kI8); break;
  }
#undef GRM_RESCORE_RQ
#undef GRM_RESCORE
  GRM_HIP_CHECK(hipGetLastError());
  const uint32_t total = static_cast<uint32_t>(qb) * M;
  grm::gqa::gqa_rescore_finalize_kernel<<<(total + 255) / 256, 256, 0, a->stream>>>(
      a->d_hex, H, a->d_shortlist, total, a->d_len, a->d_ids,
      a->short_out.dev + static_cast<size_t>(q0) * M);
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
  if (static_cast<size_t>(rq_pad_of(R * Qt)) * a->hd * sizeof(double) * grm::gqa::kUnitWaves > 65536) {
    return grm::fail(-1, "(heads / kv_heads) * query_tokens * head_dim above 2048");
  }
  GRM_HIP_CHECK(hipSetDevice(a->device));
  if (a->mut_pending) GRM_HIP_CHECK(hipStreamWaitEvent(a->stream, a->ev_mut, 0));
  GRM_CHECK_RC(ensure_items(a));
  a->routes += 1;
  const size_t qvals = static_cast<size_t>(H) * Qt * a->hd;
  const size_t qstride = qvals * (q_dtype == kF32 ? 4 : 2);
  const unsigned char* qbase = static_cast<const unsigned char*>(queries);
  if (!on_device) {
    GRM_CHECK_RC(reserve_device(reinterpret_cast<unsigned char**>(&a->d_queries), &a->d_queries_bytes,
                                qstride * q_count));
    GRM_HIP_CHECK(hipMemcpyAsync(a->d_queries, queries, qstride * q_count, hipMemcpyHostToDevice, a->stream));
    qbase = static_cast<const unsigned char*>(a->d_queries);
  }
  const uint32_t n_slots = static_cast<uint32_t>(a->high_water);
  const uint32_t per_block = grm::gqa::kFinWaves * grm::kWave;
  const uint32_t fin_blocks = std::max<uint32_t>(1, std::min<uint32_t>((n_slots + per_block - 1) / per_block, a->fin_blocks));
  const size_t per_q = static_cast<size_t>(fin_blocks) * topk;
  a->merged.resize(topk);
  ScreenPlan plan;
  const bool use_screen = screen_plan(a, H, Qt, topk, &plan);
  std::vector<int> redo;
  if (use_screen) {
    GRM_CHECK_RC(grm::reserve_mapped(&a->short_out, static_cast<size_t>(q_count) * plan.M));
    GRM_CHECK_RC(grm::reserve_mapped_bytes(&a->qstate, static_cast<size_t>(q_count) * 2 * sizeof(unsigned)));
    // untimed warmup queries first, then the timed ones
    int q0 = 0;
    const int segments[2][2] = {{0, warmup}, {warmup, q_count}};
    for (const auto& seg : segments) {
      if (seg[0] == warmup) GRM_HIP_CHECK(hipEventRecord(a->ev_start, a->stream));
      for (q0 = seg[0]; q0 < seg[1]; q0 += plan.qb_max) {
        const int qb = std::min(plan.qb_max, seg[1] - q0);
        GRM_CHECK_RC(enqueue_screen(a, plan, qbase, qstride, q_dtype, q0, qb, q_count, topk));
      }
    }
    GRM_HIP_CHECK(hipEventRecord(a->ev_stop, a->stream));
    GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
    const unsigned* st = static_cast<const unsigned*>(a->qstate.host);
    for (int qi = 0; qi < q_count; ++qi) {
      const unsigned flags = st[qi], certified = st[q_count + qi];
      if (flags != 0u || certified != 1u) {
        redo.push_back(qi);
        continue;
      }
      grm::host_topk_merge(a->short_out.host + static_cast<size_t>(qi) * plan.M, plan.M, topk,
                           a->merged.data());
      write_result(a->merged.data(), topk, out_ids + static_cast<size_t>(qi) * topk,
                   out_scores ? out_scores + static_cast<size_t>(qi) * topk : nullptr);
    }
    a->fallbacks += redo.size();
  } else {
    for (int qi = 0; qi < q_count; ++qi) redo.push_back(qi);
  }
  if (!redo.empty()) {
    GRM_CHECK_RC(grm::reserve_mapped(&a->blocks_out, per_q * redo.size()));
    if (!use_screen) {
      if (warmup > 0) {
        for (int qi = 0; qi < warmup; ++qi) {
          GRM_CHECK_RC(enqueue_exact(a, qbase + qi * qstride, q_dtype, H, Qt, topk, fin_blocks,
                                     a->blocks_out.dev + static_cast<size_t>(qi) * per_q));
        }
      }
      GRM_HIP_CHECK(hipEventRecord(a->ev_start, a->stream));
      for (int qi = warmup; qi < q_count; ++qi) {
        GRM_CHECK_RC(enqueue_exact(a, qbase + qi * qstride, q_dtype, H, Qt, topk, fin_blocks,
                                   a->blocks_out.dev + static_cast<size_t>(qi) * per_q));
      }
      GRM_HIP_CHECK(hipEventRecord(a->ev_stop, a->stream));
    } else {
      for (size_t j = 0; j < redo.size(); ++j) {
        GRM_CHECK_RC(enqueue_exact(a, qbase + redo[j] * qstride, q_dtype, H, Qt, topk, fin_blocks,
                                   a->blocks_out.dev + j * per_q));
      }
    }
    GRM_HIP_CHECK(hipStreamSynchronize(a->stream));
    for (size_t j = 0; j < redo.size(); ++j) {
      const int qi = redo[j];
      grm::host_topk_merge(a->blocks_out.host + j * per_q, per_q, topk, a->merged.data());
      write_result(a->merged.data(), topk, out_ids + static_cast<size_t>(qi) * topk,
                   out_scores ? out_scores + static_cast<size_t>(qi) * topk : nullptr);
    }
  }
  if (elapsed_ms) GRM_HIP_CHECK(hipEventElapsedTime(elapsed_ms, a->ev_start, a->ev_stop));
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
