// store.hip -- the store's route calls over the device node banks.
//
// The reference keeps route entries in its CPU store and routes them there
// (cpp/grm_runtime_c.h:381-436):
//   * grm_store_set_route / _set_route_multi / _set_route_list /
//     _clear_route / _set_route_metadata keep a node's route key(s),
//     lexical keys and route metadata;
//   * grm_store_route / _route_filtered run route_mla_arena
//     (cpp/grm_runtime.cpp:4299-4361), grm_store_route_gqa runs
//     route_gqa_raw (:4498-4881).
// This file serves those calls, with the same names, argument lists, return
// codes and output conventions, over a device bank (an MLA or a ragged GQA
// bank of this library): the route keys live in HBM, the lexical keys and
// route metadata on the host beside them.  The store here holds route
// entries only; nodes, payloads and the rest of the CPU store stay where
// they are.  A handle comes from grm_hip_store_create_mla / _gqa.
//
// The laws, in the order the reference applies them:
//   * an entry takes part when it passes the route filters (:3053-3104):
//     per category with filter values, its value must be one of them (a
//     known value compares as a bit, an unknown one as a string; an empty
//     metadata value is the entry default, cpp/grm_runtime.hpp:483-494);
//   * MLA: score = exact law score + hits / |query lexical keys| in float
//     (:3107-3170), non-finite sums dropped, order (score desc, id asc);
//   * GQA without lexical keys: the raw law score, order (raw desc, id asc);
//     with lexical keys: raw / (max raw over the entries taking part +
//     1e-8) + hits / |query lexical keys| in float, same order.
// How the device answers them: the lexical bonus is never negative and
// (for GQA) the normalisation is monotone, so an entry without lexical
// hits that makes the top k is in the bank's filtered top k; the answer is
// that top k, plus every entry with hits (scored exactly on the device),
// ranked by the law.  For GQA the normalisation can round distinct raw
// scores to one value, so the bank's top k+1 is fetched and the top k is
// kept only when its last score lies above the (k+1)-th's normalised raw
// score; otherwise every entry taking part is scored exactly.
//
// Entries with several route keys (multi-row MLA, multi-key GQA;
// set_route_multi / set_route_list with key_count != 1) score the maximum
// of their keys' finite law scores, NaN when none is finite
// (cpp/grm_runtime.cpp:3518-3545 exact_mla_entry_score, :3031-3051
// max_gqa_raw_score).  Their keys live in a second bank of the same kind
// under internal ids; every route scores all of them exactly on the device
// (one score_nodes call) and folds each entry's maximum in beside the main
// bank's filtered top k, so the answer is the law's whenever the main
// bank's is.  An entry with no key never scores.
//
// Limits: topk <= 16 (the device route's list length); MLA keys of the
// store's dim; GQA keys of whole [kv_heads][L][head_dim] blocks.  Calls on
// one handle are serialized by its mutex.

#include "grm_common.hpp"
#include "grm_hip_router.h"

#include <algorithm>
#include <cmath>
#include <mutex>
#include <set>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

namespace grm {
// Room checks of the bank files: a replace runs only when the new keys fit
// once the entry's old keys are gone, so a put that cannot fit leaves the
// old entry in place.
bool mla_append_fits(const MlaDeviceArena* a, uint64_t n_drop, uint64_t count);
bool gqa_append_fits(const GqaDeviceArena* a, const uint64_t* drop, uint64_t n_drop,
                     const uint64_t* tok_counts, uint64_t count);
}  // namespace grm

namespace {

constexpr int kMla = 0;
constexpr int kGqa = 1;
constexpr uint64_t kNone = ~0ull;

// known route filter values and their bits (cpp/grm_runtime.cpp:2788-2838):
// category c at bit 16c, value j at bit 16c + j
const char* const kKnown[4][8] = {
    {"turn", "doc", "digest", "era", "fact", "task_state", "recall", "cull_span"},
    {"conversation", "project", "user", "task", "global", "session", nullptr, nullptr},
    {"volatile", "session", "project", "permanent", nullptr, nullptr, nullptr, nullptr},
    {"ephemeral", "stable", "mutable", "immutable", nullptr, nullptr, nullptr, nullptr},
};
// a new route entry's metadata (cpp/grm_runtime.hpp:483-494)
const char* const kDefaultMeta[4] = {"turn", "conversation", "session", "ephemeral"};
// per-query string-match bit of a category: unused by every known value
constexpr int kMatchBit = 15;

uint64_t known_bit(int cat, const std::string& v) {
  for (int j = 0; j < 8 && kKnown[cat][j]; ++j) {
    if (v == kKnown[cat][j]) return 1ull << (16 * cat + j);
  }
  return 0;
}

// '\n'-joined keys, empty items dropped (cpp/grm_runtime.cpp:5196-5209)
std::vector<std::string> split_keys(const char* text) {
  std::vector<std::string> out;
  if (!text) return out;
  std::string cur;
  for (const char* p = text; *p; ++p) {
    if (*p == '\n') {
      if (!cur.empty()) out.push_back(cur);
      cur.clear();
    } else {
      cur.push_back(*p);
    }
  }
  if (!cur.empty()) out.push_back(cur);
  return out;
}

struct Entry {
  std::vector<std::string> lex;
  std::string meta[4];
  uint64_t bits = 0;
  // an entry with no key or several: its keys' ids on the multi-key bank
  bool multi = false;
  std::vector<uint64_t> mkeys;
};

}  // namespace

struct grm_store_handle {
  int dialect = kMla;
  MlaDeviceArena* mla = nullptr;
  GqaDeviceArena* gqa = nullptr;
  uint32_t dim = 0;      // MLA key length
  uint32_t kv = 0;       // GQA kv heads
  uint32_t hd = 0;       // GQA head dim
  uint64_t cap_nodes = 0, cap_tokens = 0;  // the main bank's, for the multi-key bank
  // keys of entries with several keys (created on first use)
  MlaDeviceArena* mla_multi = nullptr;
  GqaDeviceArena* gqa_multi = nullptr;
  uint64_t next_mkey = 0;
  std::unordered_set<uint64_t> multi;  // node ids of entries with multi set
  std::unordered_map<uint64_t, Entry> entries;
  std::unordered_map<std::string, std::unordered_set<uint64_t>> index;  // lexical key -> nodes
  std::mutex mu;
};

namespace {

uint64_t entry_bits(const Entry& e) {
  uint64_t b = 0;
  for (int c = 0; c < 4; ++c) b |= known_bit(c, e.meta[c]);
  return b;
}

int set_bits(grm_store_handle* h, const std::vector<uint64_t>& ids, const std::vector<uint64_t>& bits) {
  if (ids.empty()) return 0;
  return h->dialect == kMla
             ? grm_mla_hip_set_filter_bits(h->mla, ids.data(), bits.data(), ids.size())
             : grm_gqa_hip_set_filter_bits(h->gqa, ids.data(), bits.data(), ids.size());
}

void unindex(grm_store_handle* h, uint64_t nid, const Entry& e) {
  for (const auto& s : std::set<std::string>(e.lex.begin(), e.lex.end())) {
    auto it = h->index.find(s);
    if (it == h->index.end()) continue;
    it->second.erase(nid);
    if (it->second.empty()) h->index.erase(it);
  }
}

// Take an entry's key(s) off its bank and its lexical keys out of the index
// (the entry itself stays in h->entries).
int drop_keys(grm_store_handle* h, uint64_t nid, const Entry& e) {
  if (e.multi) {
    if (!e.mkeys.empty()) {
      const int rc = h->dialect == kMla
                         ? grm_mla_hip_evict(h->mla_multi, e.mkeys.data(), e.mkeys.size(), nullptr)
                         : grm_gqa_hip_evict(h->gqa_multi, e.mkeys.data(), e.mkeys.size(), nullptr);
      if (rc != 0) return rc;
    }
    h->multi.erase(nid);
  } else {
    const uint64_t id = nid;
    const int rc = h->dialect == kMla ? grm_mla_hip_evict(h->mla, &id, 1, nullptr)
                                      : grm_gqa_hip_evict(h->gqa, &id, 1, nullptr);
    if (rc != 0) return rc;
  }
  unindex(h, nid, e);
  return 0;
}

// GQA append with one compaction and retry when the token space is short.
int gqa_append(GqaDeviceArena* a, const float* keys, const uint64_t* tokens, uint64_t count,
               const uint64_t* ids) {
  int rc = grm_gqa_hip_append(a, keys, nullptr, tokens, count, ids, nullptr);
  if (rc == -3) {
    // token space: reclaim evicted nodes' tokens and try once more
    const int crc = grm_gqa_hip_compact(a);
    if (crc != 0) return crc;
    rc = grm_gqa_hip_append(a, keys, nullptr, tokens, count, ids, nullptr);
  }
  return rc;
}

// Key tokens of a GQA key of len values (whole [kv][L][hd] blocks).
int gqa_tokens(const grm_store_handle* h, uint64_t len, uint64_t* tokens) {
  const uint64_t row = static_cast<uint64_t>(h->kv) * h->hd;
  if (len % row != 0) return grm::fail(-1, "GQA route key is not whole [kv_heads][L][head_dim] blocks");
  *tokens = len / row;
  return 0;
}

// A new entry starts from the default metadata, a replaced one keeps its
// own (cpp/grm_runtime.cpp:2877-2902).
Entry new_entry(const grm_store_handle* h, uint64_t nid, const char* lexical) {
  Entry e;
  auto found = h->entries.find(nid);
  for (int c = 0; c < 4; ++c) e.meta[c] = found != h->entries.end() ? found->second.meta[c] : kDefaultMeta[c];
  e.lex = split_keys(lexical);
  e.bits = entry_bits(e);
  return e;
}

// Put an entry with `count` route keys (keys[i], lens[i] values) on the
// multi-key bank, replacing the node's entry if it has one.
int put_multi(grm_store_handle* h, uint64_t nid, const std::vector<const float*>& keys,
              const std::vector<uint64_t>& lens, const char* lexical) {
  if (nid == kNone) return grm::fail(-1, "node id UINT64_MAX is reserved");
  const uint64_t count = keys.size();
  std::vector<uint64_t> tokens(count);
  uint64_t total = 0;
  for (uint64_t i = 0; i < count; ++i) {
    if (lens[i] > 0 && !keys[i]) return grm::fail(-1, "null route key with nonzero length");
    if (h->dialect == kMla) {
      if (lens[i] != h->dim) return grm::fail(-1, "route key length does not match the store dim");
    } else {
      GRM_CHECK_RC(gqa_tokens(h, lens[i], &tokens[i]));
    }
    total += lens[i];
  }
  if (count > 0 && !h->mla_multi && !h->gqa_multi) {
    if (h->dialect == kMla) {
      GRM_CHECK_RC(grm_mla_hip_bank_create(nullptr, GRM_DTYPE_F32, 0, static_cast<int>(h->dim),
                                           nullptr, std::max<uint64_t>(h->cap_nodes, 64), &h->mla_multi));
    } else {
      const uint64_t zero = 0;
      GRM_CHECK_RC(grm_gqa_hip_bank_create(nullptr, GRM_DTYPE_F32, nullptr, GRM_DTYPE_F32, 0, &zero, 0,
                                           static_cast<int>(h->kv), static_cast<int>(h->hd), nullptr,
                                           std::max<uint64_t>(h->cap_nodes, 1),
                                           std::max<uint64_t>(h->cap_tokens, 8), &h->gqa_multi));
    }
  }
  Entry e = new_entry(h, nid, lexical);
  auto found = h->entries.find(nid);
  if (count > 0) {
    // the old keys leave the multi-key bank only when the entry had several
    const std::vector<uint64_t> none;
    const std::vector<uint64_t>& old_keys =
        found != h->entries.end() && found->second.multi ? found->second.mkeys : none;
    const bool fits = h->dialect == kMla
                          ? grm::mla_append_fits(h->mla_multi, old_keys.size(), count)
                          : grm::gqa_append_fits(h->gqa_multi, old_keys.data(), old_keys.size(),
                                                 tokens.data(), count);
    if (!fits) return grm::fail(-3, "multi-key bank capacity exceeded; the entry is unchanged");
  }
  if (found != h->entries.end()) {
    GRM_CHECK_RC(drop_keys(h, nid, found->second));
    h->entries.erase(found);  // its old keys are gone
  }
  e.multi = true;
  if (count > 0) {
    std::vector<float> flat;
    flat.reserve(total);
    for (uint64_t i = 0; i < count; ++i) flat.insert(flat.end(), keys[i], keys[i] + lens[i]);
    e.mkeys.resize(count);
    for (uint64_t i = 0; i < count; ++i) e.mkeys[i] = h->next_mkey++;
    const int rc = h->dialect == kMla
                       ? grm_mla_hip_append(h->mla_multi, flat.data(), GRM_DTYPE_F32, count,
                                            e.mkeys.data(), nullptr)
                       : gqa_append(h->gqa_multi, flat.data(), tokens.data(), count, e.mkeys.data());
    if (rc != 0) return rc;
  }
  for (const auto& s : e.lex) h->index[s].insert(nid);
  h->multi.insert(nid);
  h->entries[nid] = std::move(e);
  return 0;
}

// Put a single route key on the main bank (see new_entry for metadata).
int put_entry(grm_store_handle* h, uint64_t nid, const float* key, uint64_t len,
              const char* lexical) {
  if (nid == kNone) return grm::fail(-1, "node id UINT64_MAX is reserved");
  if (len > 0 && !key) return grm::fail(-1, "null route key with nonzero length");
  uint64_t tokens = 0;
  if (h->dialect == kMla) {
    if (len != h->dim) return grm::fail(-1, "route key length does not match the store dim");
  } else {
    GRM_CHECK_RC(gqa_tokens(h, len, &tokens));
  }
  Entry e = new_entry(h, nid, lexical);
  auto found = h->entries.find(nid);
  // the old key leaves this bank only when it is a single key
  const bool drops_here = found != h->entries.end() && !found->second.multi;
  const bool fits = h->dialect == kMla
                        ? grm::mla_append_fits(h->mla, drops_here ? 1 : 0, 1)
                        : grm::gqa_append_fits(h->gqa, &nid, drops_here ? 1 : 0, &tokens, 1);
  if (!fits) return grm::fail(-3, "route bank capacity exceeded; the entry is unchanged");
  if (found != h->entries.end()) {
    GRM_CHECK_RC(drop_keys(h, nid, found->second));
    h->entries.erase(found);  // its old key is gone
  }
  const int rc = h->dialect == kMla ? grm_mla_hip_append(h->mla, key, GRM_DTYPE_F32, 1, &nid, nullptr)
                                    : gqa_append(h->gqa, key, &tokens, 1, &nid);
  if (rc != 0) return rc;
  for (const auto& s : e.lex) h->index[s].insert(nid);
  h->entries[nid] = e;
  return set_bits(h, {nid}, {e.bits});
}

struct Filters {
  uint64_t mask = 0;  // device filter mask
  uint32_t cats = 0;  // categories with filters
  std::vector<std::string> values[4];
  bool strings[4] = {false, false, false, false};  // category filtered by an unknown value
};

Filters make_filters(const char* kinds, const char* scopes, const char* durs, const char* muts) {
  Filters f;
  const char* in[4] = {kinds, scopes, durs, muts};
  for (int c = 0; c < 4; ++c) {
    f.values[c] = split_keys(in[c]);
    if (f.values[c].empty()) continue;
    f.cats |= 1u << c;
    uint64_t m = 0;
    bool all_known = true;
    for (const auto& v : f.values[c]) {
      const uint64_t b = known_bit(c, v);
      all_known = all_known && b != 0;
      m |= b;
    }
    if (all_known) {
      f.mask |= m;
    } else {
      f.strings[c] = true;
      f.mask |= 1ull << (16 * c + kMatchBit);
    }
  }
  return f;
}

bool passes(const Entry& e, const Filters& f) {
  for (int c = 0; c < 4; ++c) {
    if (!((f.cats >> c) & 1u)) continue;
    if (std::find(f.values[c].begin(), f.values[c].end(), e.meta[c]) == f.values[c].end()) {
      return false;
    }
  }
  return true;
}

// Score listed nodes exactly on the device (NaN where not finite), on the
// main bank or (multi) the multi-key bank.
int score_nodes(grm_store_handle* h, const float* query, uint64_t heads, uint64_t tokens,
                const std::vector<uint64_t>& ids, std::vector<float>* out, bool multi = false) {
  out->assign(ids.size(), std::nanf(""));
  if (ids.empty()) return 0;
  return h->dialect == kMla
             ? grm_mla_hip_score_nodes(multi ? h->mla_multi : h->mla, query, GRM_DTYPE_F32,
                                       ids.data(), ids.size(), out->data())
             : grm_gqa_hip_score_nodes(multi ? h->gqa_multi : h->gqa, query, GRM_DTYPE_F32,
                                       static_cast<int>(heads), static_cast<int>(tokens), ids.data(),
                                       ids.size(), out->data());
}

// Law scores of the multi-key entries taking part: the maximum of each
// entry's finite key scores; entries with none are left out.
int score_multi(grm_store_handle* h, const float* query, uint64_t heads, uint64_t tokens,
                const Filters& f, std::unordered_map<uint64_t, float>* out) {
  std::vector<uint64_t> keys, owner;
  for (uint64_t nid : h->multi) {
    const Entry& e = h->entries.at(nid);
    if (!passes(e, f)) continue;
    for (uint64_t k : e.mkeys) {
      keys.push_back(k);
      owner.push_back(nid);
    }
  }
  std::vector<float> sc;
  GRM_CHECK_RC(score_nodes(h, query, heads, tokens, keys, &sc, true));
  for (size_t i = 0; i < keys.size(); ++i) {
    if (!std::isfinite(sc[i])) continue;
    auto ins = out->emplace(owner[i], sc[i]);
    if (!ins.second && sc[i] > ins.first->second) ins.first->second = sc[i];
  }
  return 0;
}

struct Ranked {
  float score;
  uint64_t id;
};

bool ranked_better(const Ranked& a, const Ranked& b) {
  if (a.score != b.score) return a.score > b.score;
  return a.id < b.id;
}

// The route: filtered device top k (k_fetch entries), the lexical bonus,
// the law's order.  GQA routes pass heads/tokens; MLA passes heads = 0.
int route(grm_store_handle* h, const float* query, uint64_t heads, uint64_t tokens,
          const char* lexical, const Filters& f, uint64_t topk, uint64_t* out_ids,
          float* out_scores, uint64_t out_cap, uint64_t* out_count) {
  *out_count = 0;
  if (topk == 0 || h->entries.empty()) return 0;
  if (topk > static_cast<uint64_t>(grm::kMaxTopK)) return grm::fail(-1, "topk above 16 is not served on the device");
  const std::vector<std::string> lex = split_keys(lexical);
  const bool gqa = h->dialect == kGqa;
  // categories filtered by unknown values: the per-query match bit on the
  // entries whose value is listed, for this route only
  std::vector<uint64_t> temp_ids, temp_bits, back_bits;
  std::unordered_map<uint64_t, size_t> temp_at;
  for (int c = 0; c < 4; ++c) {
    if (!f.strings[c]) continue;
    const auto& vals = f.values[c];
    const uint64_t bit = 1ull << (16 * c + kMatchBit);
    for (const auto& kvp : h->entries) {
      if (kvp.second.multi) continue;  // not on the main bank
      if (std::find(vals.begin(), vals.end(), kvp.second.meta[c]) == vals.end()) continue;
      auto ins = temp_at.emplace(kvp.first, temp_ids.size());
      if (ins.second) {
        temp_ids.push_back(kvp.first);
        temp_bits.push_back(kvp.second.bits | bit);
        back_bits.push_back(kvp.second.bits);
      } else {
        temp_bits[ins.first->second] |= bit;
      }
    }
  }
  GRM_CHECK_RC(set_bits(h, temp_ids, temp_bits));
  // entries on the main bank (one key each)
  const uint64_t live = h->entries.size() - h->multi.size();
  const uint64_t want = gqa && !lex.empty() ? topk + 1 : topk;
  const int kf = static_cast<int>(std::min<uint64_t>({want, live, static_cast<uint64_t>(grm::kMaxTopK)}));
  std::vector<uint64_t> ids(kf, kNone);
  std::vector<float> sc(kf, std::nanf(""));
  int rc = 0;
  if (kf > 0) {
    rc = gqa ? grm_gqa_hip_route_filtered(h->gqa, query, GRM_DTYPE_F32, 0, static_cast<int>(heads),
                                          static_cast<int>(tokens), kf, f.mask, f.cats, ids.data(),
                                          sc.data(), nullptr)
             : grm_mla_hip_route_filtered(h->mla, query, GRM_DTYPE_F32, 0, kf, f.mask, f.cats,
                                          ids.data(), sc.data(), nullptr);
  }
  const int rc2 = set_bits(h, temp_ids, back_bits);
  if (rc != 0) return rc;
  if (rc2 != 0) return rc2;
  std::unordered_map<uint64_t, float> base;  // node -> law score (MLA) or raw (GQA), finite
  std::vector<Ranked> fetched;
  for (int j = 0; j < kf; ++j) {
    if (ids[j] != kNone && std::isfinite(sc[j])) {
      base.emplace(ids[j], sc[j]);
      fetched.push_back({sc[j], ids[j]});
    }
  }
  // every multi-key entry taking part, scored exactly
  std::unordered_map<uint64_t, float> mbase;
  GRM_CHECK_RC(score_multi(h, query, heads, tokens, f, &mbase));
  float mmax = 0.0f;  // largest |raw| among them (GQA normalisation)
  for (const auto& kvp : mbase) {
    base.emplace(kvp.first, kvp.second);
    mmax = std::max(mmax, std::fabs(kvp.second));
  }
  if (lex.empty()) {
    // no bonus: the main bank's filtered order is the law's; the
    // multi-key entries join it by score
    std::vector<Ranked> all = fetched;
    for (const auto& kvp : mbase) all.push_back({kvp.second, kvp.first});
    std::sort(all.begin(), all.end(), ranked_better);
    const uint64_t n = std::min<uint64_t>({static_cast<uint64_t>(all.size()), topk, out_cap});
    for (uint64_t i = 0; i < n; ++i) {
      out_ids[i] = all[i].id;
      if (out_scores) out_scores[i] = all[i].score;
    }
    *out_count = n;
    return 0;
  }
  // lexical hits: each query key found among the entry's keys counts once
  std::unordered_map<uint64_t, uint64_t> hits;
  for (const auto& s : lex) {
    auto it = h->index.find(s);
    if (it == h->index.end()) continue;
    for (uint64_t nid : it->second) hits[nid] += 1;
  }
  std::vector<uint64_t> need;
  for (const auto& kvp : hits) {
    const Entry& e = h->entries.at(kvp.first);
    if (!e.multi && passes(e, f) && !base.count(kvp.first)) need.push_back(kvp.first);
  }
  std::vector<float> extra;
  GRM_CHECK_RC(score_nodes(h, query, heads, tokens, need, &extra));
  for (size_t i = 0; i < need.size(); ++i) {
    if (std::isfinite(extra[i])) base.emplace(need[i], extra[i]);
  }
  const float den = static_cast<float>(lex.size());
  auto bonus_of = [&](uint64_t nid) -> float {
    auto it = hits.find(nid);
    if (it == hits.end() || !passes(h->entries.at(nid), f)) return 0.0f;
    return static_cast<float>(it->second) / den;
  };
  std::vector<Ranked> ranked;
  if (!gqa) {
    for (const auto& kvp : base) {
      const float total = kvp.second + bonus_of(kvp.first);
      if (std::isfinite(total)) ranked.push_back({total, kvp.first});
    }
    std::sort(ranked.begin(), ranked.end(), ranked_better);
  } else {
    // raw >= 0, so the largest |raw| taking part is the bank's first result
    auto rank_gqa = [&](const std::unordered_map<uint64_t, float>& raws, float max_abs) {
      std::vector<Ranked> r;
      const float norm = max_abs + 1.0e-8f;
      for (const auto& kvp : raws) r.push_back({kvp.second / norm + bonus_of(kvp.first), kvp.first});
      std::sort(r.begin(), r.end(), ranked_better);
      return r;
    };
    const float max_abs = std::max(fetched.empty() ? 0.0f : std::fabs(fetched.front().score), mmax);
    ranked = rank_gqa(base, max_abs);
    const bool all_fetched = static_cast<int>(fetched.size()) < kf || fetched.size() >= live;
    if (!all_fetched) {
      const float norm = max_abs + 1.0e-8f;
      const float r_last = fetched.back().score;
      // An entry the bank did not return (and without lexical hits) has
      // raw <= r_last.  With k + 1 fetched, it normalises to at most
      // guard = fl(r_last / norm), so the top k is certain when the k-th
      // ranked score lies above guard.  When the fetch stopped at the
      // kernels' cap (k = 16, so only k fetched), the last fetched entry
      // is itself one of the k: an unfetched entry with raw == r_last has
      // a higher node id (the bank's tie law) and ranks after it, and one
      // with raw < r_last normalises to at most fl(pred(r_last) / norm), so
      // the top k is certain when the k-th ranked score lies above that.
      const float guard = kf > static_cast<int>(topk)
                              ? r_last / norm
                              : std::nextafter(r_last, -INFINITY) / norm;
      const bool sure = ranked.size() >= topk && ranked[topk - 1].score > guard;
      if (!sure) {
        // every entry taking part, scored exactly
        std::vector<uint64_t> all;
        for (const auto& kvp : h->entries) {
          if (!kvp.second.multi && passes(kvp.second, f)) all.push_back(kvp.first);
        }
        std::vector<float> raw;
        GRM_CHECK_RC(score_nodes(h, query, heads, tokens, all, &raw));
        std::unordered_map<uint64_t, float> every(mbase);
        float mx = mmax;
        for (size_t i = 0; i < all.size(); ++i) {
          if (!std::isfinite(raw[i])) continue;
          every.emplace(all[i], raw[i]);
          mx = std::max(mx, std::fabs(raw[i]));
        }
        ranked = rank_gqa(every, mx);
      }
    }
  }
  const uint64_t n = std::min<uint64_t>({static_cast<uint64_t>(ranked.size()), topk, out_cap});
  for (uint64_t i = 0; i < n; ++i) {
    out_ids[i] = ranked[i].id;
    if (out_scores) out_scores[i] = ranked[i].score;
  }
  *out_count = n;
  return 0;
}

int check_out(uint64_t* out_ids, uint64_t out_cap, uint64_t* out_count) {
  if (!out_count) return grm::fail(-1, "null out_count");
  if (!out_ids && out_cap > 0) return grm::fail(-1, "null output buffer with nonzero capacity");
  return 0;
}

}  // namespace

// ================================================================ create

extern "C" int grm_hip_store_create_mla(int dim, uint64_t capacity, int row_dtype,
                                        grm_store_handle** out_handle) {
  if (!out_handle || dim <= 0) return grm::fail(-1, "invalid store arguments");
  if (row_dtype != GRM_DTYPE_F32 && row_dtype != GRM_DTYPE_BF16) {
    return grm::fail(-1, "MLA store rows are F32 or BF16");
  }
  if (row_dtype != GRM_DTYPE_F32) {
    return grm::fail(-1, "the store takes fp32 route keys; its bank holds them as F32");
  }
  auto* h = new grm_store_handle();
  h->dialect = kMla;
  h->dim = static_cast<uint32_t>(dim);
  h->cap_nodes = capacity;
  const int rc = grm_mla_hip_bank_create(nullptr, row_dtype, 0, dim, nullptr,
                                         std::max<uint64_t>(capacity, 64), &h->mla);
  if (rc != 0) {
    delete h;
    return rc;
  }
  *out_handle = h;
  return 0;
}

extern "C" int grm_hip_store_create_gqa(int kv_heads, int head_dim, uint64_t capacity_nodes,
                                        uint64_t capacity_tokens, grm_store_handle** out_handle) {
  if (!out_handle || kv_heads <= 0 || head_dim <= 0) return grm::fail(-1, "invalid store arguments");
  auto* h = new grm_store_handle();
  h->dialect = kGqa;
  h->kv = static_cast<uint32_t>(kv_heads);
  h->hd = static_cast<uint32_t>(head_dim);
  h->cap_nodes = capacity_nodes;
  h->cap_tokens = capacity_tokens;
  const uint64_t zero = 0;
  const int rc = grm_gqa_hip_bank_create(nullptr, GRM_DTYPE_F32, nullptr, GRM_DTYPE_F32, 0, &zero, 0,
                                         kv_heads, head_dim, nullptr,
                                         std::max<uint64_t>(capacity_nodes, 1),
                                         std::max<uint64_t>(capacity_tokens, 8), &h->gqa);
  if (rc != 0) {
    delete h;
    return rc;
  }
  *out_handle = h;
  return 0;
}

extern "C" void grm_hip_store_destroy(grm_store_handle* h) {
  if (!h) return;
  if (h->mla) grm_mla_cuda_arena_destroy(h->mla);
  if (h->gqa) grm_gqa_cuda_arena_destroy(h->gqa);
  if (h->mla_multi) grm_mla_cuda_arena_destroy(h->mla_multi);
  if (h->gqa_multi) grm_gqa_cuda_arena_destroy(h->gqa_multi);
  delete h;
}

// ================================================== reference route surface

extern "C" int grm_store_set_route(grm_store_handle* h, uint64_t node_id, const float* route_key,
                                   uint64_t route_len, const char* lexical_keys) {
  if (!h) return grm::fail(-1, "invalid set_route arguments");
  std::lock_guard<std::mutex> lock(h->mu);
  const int rc = put_entry(h, node_id, route_key, route_len, lexical_keys);
  if (rc == 0) grm::clear_error();
  return rc;
}

extern "C" int grm_store_set_route_multi(grm_store_handle* h, uint64_t node_id,
                                         const float* route_keys, uint64_t key_count,
                                         uint64_t route_len, const char* lexical_keys) {
  if (!h) return grm::fail(-1, "invalid set_route_multi arguments");
  if (!route_keys && key_count > 0 && route_len > 0) return grm::fail(-1, "null route keys with nonzero shape");
  if (key_count == 1) return grm_store_set_route(h, node_id, route_keys, route_len, lexical_keys);
  std::vector<const float*> keys(key_count);
  std::vector<uint64_t> lens(key_count, route_len);
  for (uint64_t k = 0; k < key_count; ++k) keys[k] = route_keys ? route_keys + k * route_len : nullptr;
  std::lock_guard<std::mutex> lock(h->mu);
  const int rc = put_multi(h, node_id, keys, lens, lexical_keys);
  if (rc == 0) grm::clear_error();
  return rc;
}

extern "C" int grm_store_set_route_list(grm_store_handle* h, uint64_t node_id,
                                        const float* route_values, uint64_t value_count,
                                        const uint64_t* route_offsets, uint64_t key_count,
                                        const char* lexical_keys) {
  // argument checks in the reference's order (cpp/grm_runtime.cpp:6691-6731)
  if (!h) return grm::fail(-1, "invalid set_route_list arguments");
  if (!route_values && value_count > 0) return grm::fail(-1, "null route values with nonzero length");
  if (!route_offsets && key_count > 0) return grm::fail(-1, "null route offsets with nonzero key count");
  if (key_count == 0 && value_count != 0) return grm::fail(-1, "route values require route offsets");
  if (key_count > 0 && route_offsets[0] != 0) return grm::fail(-1, "route offsets must start at zero");
  if (key_count > 0 && route_offsets[key_count] != value_count) {
    return grm::fail(-1, "route offsets must end at value_count");
  }
  std::vector<const float*> keys(key_count);
  std::vector<uint64_t> lens(key_count);
  for (uint64_t k = 0; k < key_count; ++k) {
    if (route_offsets[k + 1] < route_offsets[k] || route_offsets[k + 1] > value_count) {
      return grm::fail(-1, "invalid route key offsets");
    }
    keys[k] = route_values ? route_values + route_offsets[k] : nullptr;
    lens[k] = route_offsets[k + 1] - route_offsets[k];
  }
  if (key_count == 1) return grm_store_set_route(h, node_id, keys[0], lens[0], lexical_keys);
  std::lock_guard<std::mutex> lock(h->mu);
  const int rc = put_multi(h, node_id, keys, lens, lexical_keys);
  if (rc == 0) grm::clear_error();
  return rc;
}

extern "C" int grm_store_clear_route(grm_store_handle* h, uint64_t node_id) {
  if (!h) return grm::fail(-1, "invalid clear_route arguments");
  std::lock_guard<std::mutex> lock(h->mu);
  auto it = h->entries.find(node_id);
  if (it == h->entries.end()) return 0;  // no route entry: nothing to clear
  GRM_CHECK_RC(drop_keys(h, node_id, it->second));
  h->entries.erase(it);
  grm::clear_error();
  return 0;
}

extern "C" int grm_store_set_route_metadata(grm_store_handle* h, uint64_t node_id, const char* kind,
                                            const char* scope, const char* durability,
                                            const char* mutability) {
  if (!h) return grm::fail(-1, "invalid set_route_metadata arguments");
  std::lock_guard<std::mutex> lock(h->mu);
  auto it = h->entries.find(node_id);
  if (it == h->entries.end()) return 0;  // no route entry: left alone (:2922-2946)
  const char* in[4] = {kind, scope, durability, mutability};
  for (int c = 0; c < 4; ++c) {
    if (in[c] && in[c][0]) it->second.meta[c] = in[c];
  }
  it->second.bits = entry_bits(it->second);
  // a multi-key entry's filters are applied on the host
  const int rc = it->second.multi ? 0 : set_bits(h, {node_id}, {it->second.bits});
  if (rc == 0) grm::clear_error();
  return rc;
}

extern "C" int grm_store_route(grm_store_handle* h, const float* query, uint64_t query_len,
                               const char* lexical_keys, uint64_t topk, uint64_t* out_node_ids,
                               uint64_t out_cap, uint64_t* out_count) {
  return grm_store_route_filtered(h, query, query_len, lexical_keys, nullptr, nullptr, nullptr,
                                  nullptr, topk, out_node_ids, out_cap, out_count);
}

extern "C" int grm_store_route_filtered(grm_store_handle* h, const float* query, uint64_t query_len,
                                        const char* lexical_keys, const char* kind_filters,
                                        const char* scope_filters, const char* durability_filters,
                                        const char* mutability_filters, uint64_t topk,
                                        uint64_t* out_node_ids, uint64_t out_cap,
                                        uint64_t* out_count) {
  if (!h || !query) return grm::fail(-1, "invalid route arguments");
  GRM_CHECK_RC(check_out(out_node_ids, out_cap, out_count));
  if (h->dialect != kMla) return grm::fail(-1, "route requires an MLA store (use route_gqa)");
  if (query_len != h->dim) return grm::fail(-1, "query length does not match the store dim");
  std::lock_guard<std::mutex> lock(h->mu);
  const Filters f = make_filters(kind_filters, scope_filters, durability_filters, mutability_filters);
  const int rc = route(h, query, 0, 0, lexical_keys, f, topk, out_node_ids, nullptr, out_cap,
                       out_count);
  if (rc == 0) grm::clear_error();
  return rc;
}

extern "C" int grm_store_route_gqa(grm_store_handle* h, const float* query, uint64_t query_heads,
                                   uint64_t query_tokens, uint64_t head_dim,
                                   const char* lexical_keys, const char* kind_filters,
                                   const char* scope_filters, const char* durability_filters,
                                   const char* mutability_filters, uint64_t topk,
                                   uint64_t* out_node_ids, uint64_t out_cap, uint64_t* out_count) {
  if (!h) return grm::fail(-1, "invalid route_gqa arguments");
  GRM_CHECK_RC(check_out(out_node_ids, out_cap, out_count));
  if (h->dialect != kGqa) return grm::fail(-1, "route_gqa requires a GQA store");
  if (head_dim != h->hd) return grm::fail(-1, "route_gqa head_dim does not match the store");
  if (query_heads == 0 || query_tokens == 0 || query_heads % h->kv != 0 ||
      query_heads > (1u << 20) || query_tokens > (1u << 20)) {
    return grm::fail(-1, "route_gqa needs heads a multiple of kv_heads and tokens > 0");
  }
  if (!query) return grm::fail(-1, "null GQA query");
  std::lock_guard<std::mutex> lock(h->mu);
  const Filters f = make_filters(kind_filters, scope_filters, durability_filters, mutability_filters);
  const int rc = route(h, query, query_heads, query_tokens, lexical_keys, f, topk, out_node_ids,
                       nullptr, out_cap, out_count);
  if (rc == 0) grm::clear_error();
  return rc;
}

// ======================================================== extensions

extern "C" int grm_hip_store_set_routes(grm_store_handle* h, uint64_t count, const uint64_t* node_ids,
                                        const float* keys, const uint64_t* key_lens,
                                        const char* const* lexical_keys,
                                        const char* const* metadata) {
  if (!h || (count > 0 && (!node_ids || !keys || !key_lens))) {
    return grm::fail(-1, "invalid set_routes arguments");
  }
  std::lock_guard<std::mutex> lock(h->mu);
  std::unordered_set<uint64_t> seen;
  uint64_t total = 0;
  for (uint64_t i = 0; i < count; ++i) {
    if (node_ids[i] == kNone || h->entries.count(node_ids[i]) || !seen.insert(node_ids[i]).second) {
      return grm::fail(-1, "set_routes takes new, distinct node ids");
    }
    if (h->dialect == kMla && key_lens[i] != h->dim) {
      return grm::fail(-1, "route key length does not match the store dim");
    }
    if (h->dialect == kGqa && key_lens[i] % (static_cast<uint64_t>(h->kv) * h->hd) != 0) {
      return grm::fail(-1, "GQA route key is not whole [kv_heads][L][head_dim] blocks");
    }
    total += key_lens[i];
  }
  if (count == 0) return 0;
  int rc;
  if (h->dialect == kMla) {
    rc = grm_mla_hip_append(h->mla, keys, GRM_DTYPE_F32, count, node_ids, nullptr);
  } else {
    std::vector<uint64_t> toks(count);
    for (uint64_t i = 0; i < count; ++i) toks[i] = key_lens[i] / (static_cast<uint64_t>(h->kv) * h->hd);
    rc = grm_gqa_hip_append(h->gqa, keys, nullptr, toks.data(), count, node_ids, nullptr);
    if (rc == -3) {
      const int crc = grm_gqa_hip_compact(h->gqa);
      if (crc != 0) return crc;
      rc = grm_gqa_hip_append(h->gqa, keys, nullptr, toks.data(), count, node_ids, nullptr);
    }
  }
  if (rc != 0) return rc;
  (void)total;
  std::vector<uint64_t> ids(node_ids, node_ids + count), bits(count);
  for (uint64_t i = 0; i < count; ++i) {
    Entry e;
    for (int c = 0; c < 4; ++c) {
      const char* v = metadata ? metadata[4 * i + c] : nullptr;
      e.meta[c] = (v && v[0]) ? v : kDefaultMeta[c];
    }
    e.lex = split_keys(lexical_keys ? lexical_keys[i] : nullptr);
    e.bits = entry_bits(e);
    for (const auto& s : e.lex) h->index[s].insert(node_ids[i]);
    bits[i] = e.bits;
    h->entries[node_ids[i]] = std::move(e);
  }
  rc = set_bits(h, ids, bits);
  if (rc == 0) grm::clear_error();
  return rc;
}

extern "C" int grm_hip_store_route_scored(grm_store_handle* h, const float* query,
                                          uint64_t query_heads, uint64_t query_tokens,
                                          const char* lexical_keys, const char* kind_filters,
                                          const char* scope_filters,
                                          const char* durability_filters,
                                          const char* mutability_filters, uint64_t topk,
                                          uint64_t* out_node_ids, float* out_scores,
                                          uint64_t out_cap, uint64_t* out_count) {
  if (!h || !query) return grm::fail(-1, "invalid route arguments");
  GRM_CHECK_RC(check_out(out_node_ids, out_cap, out_count));
  if (h->dialect == kGqa && (query_heads == 0 || query_tokens == 0 || query_heads % h->kv != 0)) {
    return grm::fail(-1, "route needs heads a multiple of kv_heads and tokens > 0");
  }
  std::lock_guard<std::mutex> lock(h->mu);
  const Filters f = make_filters(kind_filters, scope_filters, durability_filters, mutability_filters);
  const bool gqa = h->dialect == kGqa;
  const int rc = route(h, query, gqa ? query_heads : 0, gqa ? query_tokens : 0, lexical_keys, f,
                       topk, out_node_ids, out_scores, out_cap, out_count);
  if (rc == 0) grm::clear_error();
  return rc;
}

extern "C" int grm_hip_store_info(grm_store_handle* h, uint64_t* out4) {
  if (!h || !out4) return grm::fail(-1, "null argument");
  std::lock_guard<std::mutex> lock(h->mu);
  out4[0] = static_cast<uint64_t>(h->dialect);
  out4[1] = h->entries.size();
  out4[2] = h->dialect == kMla ? h->dim : h->kv;
  out4[3] = h->dialect == kMla ? 0 : h->hd;
  return 0;
}

extern "C" const char* grm_store_last_error(grm_store_handle* h) {
  (void)h;
  return grm_hip_last_error();
}
