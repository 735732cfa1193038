// gqa_kernels.hpp -- device code of the ragged GQA route (included by
// gqa_route.hip only).
//
// Law (cpp/grm_runtime.cpp:2980-3029 gqa_raw_score; core/graft_arena.py:2888-2900):
//   score(node) = float( (sum_h best_h) / H )                 h ascending, fp64
//   best_h      = max over (query token qi, key token t) of |dot| / sqrt(hd)
//   dot         = sum_d (double)q[h][qi][d] * (double)k[h/R][t][d], d ascending
// A node with zero key tokens scores 0.0; any non-finite query or key value
// makes the score NaN (never ranked).
//
// Two kernel families produce the per-(node, head) maxima best_h, both
// exactly as the law defines them; the maxima combine with a 64-bit
// atomicMax on the bit pattern (non-negative doubles order like their
// bits, so the result does not depend on scheduling):
//  * exact           -- the law itself in fp64 for every key token, one
//                       lane per token, d in order (fp32 banks, other
//                       head sizes);
//  * screen + refine -- |q.k| for every key token on the matrix cores (bf16
//                       or fp16 MFMA 16x16x32, fp32 accumulate) with a
//                       rigorous error bound; only the tokens the bound
//                       cannot exclude from a maximum are recomputed in the
//                       law's fp64 order.
// A finalize kernel sums the maxima over heads in order.
#pragma once

#include "grm_common.hpp"

#include <hip/hip_fp16.h>

namespace grm {
namespace gqa {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kUnitWaves = 4;     // wavefronts per work-item block
constexpr int kFinWaves = 4;      // wavefronts per finalize block
constexpr int kMaxRQ = 32;        // query columns per kv head of one exact pass

// Query passes.  A route's query has H = kv * R heads of Qt tokens; the
// kernels below read one pass of it: heads g*R + r0 + rr (rr < Rc) of every
// kv head g and tokens t0 + tt (tt < Qc).  The host hands a pass over as a
// query pointer advanced by (r0 * Qt + t0) * hd values and a maxima pointer
// advanced by r0 * cap, so the kernels index with the full R and Qt as
// strides and with Rc and Qc as counts: the value (rr, tt, d) of kv head g
// is element ((g*R + rr) * Qt + tt) * hd + d, and its head's maximum is at
// (g*R + rr) * cap.  best_h is a maximum over (query token, key token), so
// passes over disjoint parts of the query fold into one maximum with the
// same atomicMax, in any order.
constexpr uint32_t kMaxHeadDim = 512;

// Key chunk planes.  A key row of head_dim values is C 16-byte pieces
// (epc values each); S consecutive pieces (S = 4 when the row is a
// multiple of 64 bytes, else 2 or 1) form a chunk.  The block of (slot,
// kv head g) -- the slot's key tokens, in L rows (the token count rounded
// up to kTokAlign) -- is stored as C/S planes of L chunks: piece p of
// token t is piece index
//     row0 * C + (p / S) * L * S + t * S + p % S
// of the key arena, with row0 = tok_off * kv + g * L.  INT8 scales are
// planes per group: scale of group j of token t is element
// row0 * G + j * L + t (G = head_dim / group_size).  Sixteen consecutive
// tokens' chunk is one contiguous run (1 KiB with S = 4), a token's row is
// C/S whole chunks, every run of kTokAlign tokens starts a 128-byte line
// (no two streams share a line), and a slot's blocks stay contiguous
// (tok_off * kv * head_dim values), so whole nodes move as one copy.  Rows
// past the token count are never read.
constexpr uint32_t kTokAlign = 8;

// Piece p of token t of a block whose piece 0 is at `kb` (S = 1 << sS).
__device__ inline const u32x4* piece_ptr(const u32x4* kb, uint64_t L, int sS, uint32_t t,
                                         int p) {
  return kb + (static_cast<uint64_t>(p >> sS) * L << sS) + (static_cast<uint64_t>(t) << sS) +
         (p & ((1 << sS) - 1));
}

// Work item: `count` consecutive key tokens, from t0, of one slot (all kv
// heads).  `base` = tok_off[slot] * kv, so row0 of kv head g is
// base + g * len, `len` being the slot's padded row count.  `q` is the
// query an item of a candidate list belongs to (0 elsewhere).
struct Item {
  uint64_t base;  // tok_off[slot] * kv
  uint32_t slot;
  uint32_t t0;
  uint32_t count;
  uint32_t len;
  uint32_t q;
  uint32_t pad;
};
static_assert(sizeof(Item) == 32, "Item layout");

__device__ inline float load_scale(const unsigned char* __restrict__ scales,
                                   int scale_dtype, uint64_t idx) {
  if (scale_dtype == kF16) {
    return __half2float(reinterpret_cast<const __half*>(scales)[idx]);
  }
  return reinterpret_cast<const float*>(scales)[idx];
}

// INT8 dequant law: fp16(float(code) * scale) (core/graft_quant.py:136-144):
// the product rounds to fp32, then to fp16.  The empty asm keeps the fp32
// product a value of its own; without it the compiler fuses multiply and
// conversion into v_fma_mixlo_f16, which rounds the exact product to fp16
// once and differs from the law when the fp32 rounding crosses an fp16
// rounding boundary.
__device__ inline _Float16 dequant_i8(int code, float scale) {
  float p = static_cast<float>(code) * scale;
  asm volatile("" : "+v"(p));
  return static_cast<_Float16>(p);
}

// The bank stores an INT8 code c as the byte c ^ 0x80 (c + 128 read as an
// unsigned byte); gqa_place_kernel applies it on upload.  The screens'
// conversion of codes to f16 then starts from the unsigned byte directly.
__device__ inline int stored_code(uint32_t w, int b) {
  return static_cast<int>((w >> (8 * b)) & 0xffu) - 128;
}
__device__ inline u32x4 to_stored_codes(u32x4 v) {
  v.x ^= 0x80808080u;
  v.y ^= 0x80808080u;
  v.z ^= 0x80808080u;
  v.w ^= 0x80808080u;
  return v;
}

template <int KDT>
struct KeyTraits {
  static constexpr int kEsize = KDT == kF32 ? 4 : (KDT == kI8 ? 1 : 2);
  static constexpr int kEpc = 16 / kEsize;  // elements per 16-byte chunk
};

// Decode one 16-byte chunk of the bank into floats (law-level values);
// `scale` is the chunk's INT8 group scale (ignored for the other types),
// INT8 codes in their stored form (stored_code).
template <int KDT>
__device__ inline void decode_chunk(u32x4 v, float scale, float* out) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  if constexpr (KDT == kF32) {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(w[i]);
  } else if constexpr (KDT == kBF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = __uint_as_float(w[i] << 16);
      out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  } else if constexpr (KDT == kF16) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      out[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(w[i] & 0xffffu)));
      out[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(w[i] >> 16)));
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        out[4 * i + b] = static_cast<float>(dequant_i8(stored_code(w[i], b), scale));
      }
    }
  }
}

// ----------------------------------------------------------------- exact

// Query rows of one pass as doubles for the exact kernels:
// q64[((qb * kv + g) * hd + d) * RQP + j] = value (j / Qc, j % Qc, d) of kv
// head g for j < Rc*Qc, 0 for the padding rows j < RQP.  The d-major order
// lets a wave read the RQP values of one d as one wave-uniform (scalar)
// load.  qflags[qb * kv + g] = 1 when a value of query qb read by kv head g
// is non-finite; the first pass (flags_or = 0) writes 0 otherwise, later
// passes leave the flag as it is.  grid (kv, Qb).
__global__ __launch_bounds__(1024) void gqa_q64_kernel(
    const void* __restrict__ query, int q_dtype, size_t q_elems, int Qt, int Qc,
    int hd, int kv, int R, int Rc, int RQP, double* __restrict__ q64,
    unsigned* __restrict__ qflags, int flags_or) {
  const int g = blockIdx.x;
  const int qb = blockIdx.y;
  const int rq = Rc * Qc;
  bool bad = false;
  for (int idx = threadIdx.x; idx < RQP * hd; idx += blockDim.x) {
    const int d = idx / RQP;
    const int j = idx - d * RQP;
    double v = 0.0;
    if (j < rq) {
      const uint64_t src = static_cast<uint64_t>(qb) * q_elems +
                           (static_cast<uint64_t>(g * R + j / Qc) * Qt + j % Qc) * hd + d;
      const float f = q_dtype == kBF16
                          ? bf16_to_f32(static_cast<const uint16_t*>(query)[src])
                          : static_cast<const float*>(query)[src];
      bad = bad || !isfinite(f);
      v = static_cast<double>(f);
    }
    q64[(static_cast<size_t>(qb * kv + g) * hd + d) * RQP + idx % RQP] = v;
  }
  bad = __syncthreads_or(bad);
  if (threadIdx.x == 0 && (bad || !flags_or)) qflags[qb * kv + g] = bad ? 1u : 0u;
}

// Chunks per stage of the pipelined exact kernel (two stages live in
// registers): at most 8, and at most 64 (RQ <= 8) or 32 decoded values.
template <int KDT, int RQ>
constexpr int exact_stage_chunks() {
  constexpr int epc = KeyTraits<KDT>::kEpc;
  constexpr int cap = (RQ <= 8 ? 64 : 32) / epc;
  return cap < 1 ? 1 : (cap > 8 ? 8 : cap);
}

// Exact maxima for every (kv head, item) pair against query it.q of the
// item (q64 of gqa_q64_kernel; maxima at hmax + q*hstride), as a software
// pipeline (the item count is *n_items_dev when that is given, for lists
// built on the device): wavefront w of W walks
// pairs p = w, w+W, ... (p = g * n_items + item, so neighbouring waves
// share a kv head and its query rows stay in the scalar cache) as one
// stream of stages -- NB chunks of one 64-token tile -- and loads the next
// stage while it folds the current one, so every wave keeps HBM reads in
// flight while its fp64 work runs.  Lane l owns token t+l of the tile; a
// stage's chunks are the law's d order, so the dot products stay
// sequential in d.  hmax is head-major: hmax[h * cap + slot].
template <int KDT, int RQ, int NB>
__global__ __launch_bounds__(kUnitWaves * kWave) void gqa_exact_kernel(
    const unsigned char* __restrict__ keys,
    const unsigned char* __restrict__ scales, int scale_dtype, int group_size,
    const Item* __restrict__ items, uint32_t n_items, const uint32_t* __restrict__ n_items_dev,
    int kv, int hd, int sS, int R, int Rc, int Qc, const double* __restrict__ q64, double denom,
    unsigned long long* __restrict__ hmax, size_t hstride, size_t cap) {
  using T = KeyTraits<KDT>;
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t W = gridDim.x * kUnitWaves;
  if (n_items_dev) n_items = *n_items_dev;
  const uint32_t n_pairs = n_items * static_cast<uint32_t>(kv);
  uint32_t p_cur = blockIdx.x * kUnitWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  if (p_cur >= n_pairs) return;
  const int C = hd / T::kEpc;
  const int nb = (C + NB - 1) / NB;  // stages per tile
  const int G = KDT == kI8 ? hd / group_size : 1;
  const int cpg = KDT == kI8 ? group_size / T::kEpc : 1;
  const int ses = scale_dtype == kF16 ? 2 : 4;

  // Loads are unconditional (no branch around them, so the compiler can
  // count outstanding loads instead of draining them): lanes past the
  // item's end read its last token and chunks past C read chunk C-1; those
  // values are never folded (see `fold` and the tile end).
  auto load = [&](u32x4 (&v)[NB], float (&sc)[NB], const Item& it, int g, uint32_t t, int b) {
    const uint64_t row0 = it.base + static_cast<uint64_t>(g) * it.len;
    const uint32_t tl = min(t + lane, it.t0 + it.count - 1);
    const u32x4* kb = reinterpret_cast<const u32x4*>(keys) + row0 * C;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int c = min(b * NB + j, C - 1);
      v[j] = __builtin_nontemporal_load(piece_ptr(kb, it.len, sS, tl, c));
      sc[j] = 0.0f;
      if constexpr (KDT == kI8) {
        sc[j] = load_scale(scales + (row0 * G + tl) * ses, scale_dtype,
                           static_cast<uint64_t>(c / cpg) * it.len);
      }
    }
  };
  double acc[RQ], best[RQ];
#pragma unroll
  for (int j = 0; j < RQ; ++j) {
    acc[j] = 0.0;
    best[j] = 0.0;
  }
  auto fold = [&](const u32x4 (&v)[NB], const float (&sc)[NB], uint32_t q, int g, int b) {
    const double* __restrict__ qg = q64 + (static_cast<size_t>(q) * kv + g) * hd * RQ;
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int c = b * NB + j;
      if (c < C) {
        float f[T::kEpc];
        decode_chunk<KDT>(v[j], sc[j], f);
        const double* qc = qg + static_cast<size_t>(c) * T::kEpc * RQ;
#pragma unroll
        for (int e = 0; e < T::kEpc; ++e) {
          const double kd = static_cast<double>(f[e]);
#pragma unroll
          for (int r = 0; r < RQ; ++r) acc[r] = fma(kd, qc[e * RQ + r], acc[r]);
        }
      }
    }
  };
  auto emit = [&](const Item& it, int g) {
    const int rq_used = Rc * Qc;
    for (int r = 0; r < Rc; ++r) {
      double m = 0.0;
#pragma unroll
      for (int j = 0; j < RQ; ++j) {
        if (j / Qc == r && j < rq_used) m = (best[j] > m || isnan(best[j])) ? best[j] : m;
      }
      // max(|dot|)/denom equals the law's max(|dot|/denom): division by a
      // positive constant is monotone under rounding to nearest
      unsigned long long bits = __double_as_longlong(m / denom);
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        const unsigned long long o = __shfl_xor(bits, off);
        bits = o > bits ? o : bits;
      }
      if (lane == 0) {
        atomicMax(hmax + it.q * hstride + static_cast<size_t>(g * R + r) * cap + it.slot, bits);
      }
    }
#pragma unroll
    for (int j = 0; j < RQ; ++j) best[j] = 0.0;
  };

  int g_cur = static_cast<int>(p_cur / n_items);
  Item cur = items[p_cur - static_cast<uint32_t>(g_cur) * n_items];
  uint32_t p_nxt = p_cur + W;
  int g_nxt = static_cast<int>(min(p_nxt, n_pairs - 1) / n_items);
  Item nxt = items[min(p_nxt, n_pairs - 1) - static_cast<uint32_t>(g_nxt) * n_items];
  uint32_t t = cur.t0;
  int b = 0;
  u32x4 v0[NB], v1[NB];
  float s0[NB], s1[NB];
  load(v0, s0, cur, g_cur, t, 0);
  // One stage: fold `now` while the next stage loads into `later` (the
  // stream's last stage reloads itself, harmlessly, to keep the load
  // unconditional).  Returns false when the wave's stream is exhausted.
  auto step = [&](u32x4 (&now)[NB], float (&snow)[NB], u32x4 (&later)[NB],
                  float (&slater)[NB]) -> bool {
    const bool last_b = b + 1 == nb;
    const bool last_t = t + kWave >= cur.t0 + cur.count;
    const bool item_end = last_b && last_t;
    const bool more = !item_end || p_nxt < n_pairs;
    const bool jump = item_end && more;
    const Item& nit = jump ? nxt : cur;
    const int ng = jump ? g_nxt : g_cur;
    const uint32_t nt = !more ? t : (item_end ? nxt.t0 : (last_b ? t + kWave : t));
    const int nbb = (!more || !last_b) ? (more ? b + 1 : b) : 0;
    load(later, slater, nit, ng, nt, nbb);
    fold(now, snow, cur.q, g_cur, b);
    if (!last_b) {
      ++b;
      return true;
    }
    // tile done: fold |dot| of the lane's token (if inside the item) into
    // the item maxima
    const bool in_item = t + lane < cur.t0 + cur.count;
#pragma unroll
    for (int j = 0; j < RQ; ++j) {
      const double a = fabs(acc[j]);
      if (in_item) best[j] = (a > best[j] || isnan(a)) ? a : best[j];
      acc[j] = 0.0;
    }
    b = 0;
    if (!last_t) {
      t += kWave;
      return true;
    }
    emit(cur, g_cur);
    if (p_nxt >= n_pairs) return false;
    p_cur = p_nxt;
    g_cur = g_nxt;
    cur = nxt;
    t = cur.t0;
    p_nxt = p_cur + W;
    g_nxt = static_cast<int>(min(p_nxt, n_pairs - 1) / n_items);
    nxt = items[min(p_nxt, n_pairs - 1) - static_cast<uint32_t>(g_nxt) * n_items];
    return true;
  };
  while (step(v0, s0, v1, s1) && step(v1, s1, v0, s0)) {
  }
}

// Exact scores of every live slot -- or, with slot_list, of the slots
// slot_list[qb*list_stride ..) (list_count[qb] of them) -- from the
// head-major maxima (h in order, fp64); grid (blocks, queries), grid-stride
// over groups of 64 slots.
// Query qb's maxima are hmax[qb*hstride + h*cap + slot].  All waves of the
// block stage the group's maxima in LDS -- every load of a group is in
// flight at once, since the atomics that produced them leave them outside
// the cache; wave 0 sums each slot's heads in order, keeps the block's k
// best and writes them to block_out[(qb*gridDim.x + blockIdx.x)*k ..).
// qbad[qb*kv + g] are the query's non-finite flags.  With done
// (host-mapped memory) the entries carry route_tag(seq) in their slot
// field (store_entry) and wave 0 then stores seq at done[qb*gridDim.x +
// blockIdx.x] once its list is complete (after its end tick at the same
// index of stamps, when given), so a host that sees every flag of a launch
// holds its lists without waiting for the stream; the maxima are re-zeroed
// last.
constexpr int kFinSlots = 64;    // slots per finalize group (one per lane)
constexpr int kFinHeads = 128;   // heads staged per pass

__global__ __launch_bounds__(kFinWaves * kWave) void gqa_finalize_kernel(
    unsigned long long* __restrict__ hmax, size_t hstride, size_t cap, int H, uint32_t n_slots,
    const uint32_t* __restrict__ lens, const uint32_t* __restrict__ flags,
    const uint64_t* __restrict__ ids, const unsigned* __restrict__ qbad, int kv,
    int k, Cand* __restrict__ block_out, const uint32_t* __restrict__ slot_list,
    const uint32_t* __restrict__ list_count, size_t list_stride, unsigned* __restrict__ done,
    unsigned seq, unsigned long long* __restrict__ stamps) {
  __shared__ double s_h[kFinHeads][kFinSlots];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int qb = blockIdx.y;
  hmax += qb * hstride;
  if (slot_list) {
    slot_list += qb * list_stride;
    n_slots = list_count[qb];
  }
  // Every load a group needs is issued before any result is used: slot
  // metadata, ids and the query flags ride along with the maxima.
  unsigned qbad_lane = 0u;
  for (int g0 = 0; g0 < kv; g0 += kWave) {
    if (g0 + lane < kv) qbad_lane |= qbad[qb * kv + g0 + lane];
  }
  WaveList L;
  wl_init(L);
  bool q_bad = false;
  bool q_bad_known = false;
  for (uint32_t base = blockIdx.x * kFinSlots; base < n_slots; base += gridDim.x * kFinSlots) {
    const bool in = base + lane < n_slots;
    const uint32_t slot = slot_list ? (in ? slot_list[base + lane] : 0u) : base + lane;
    uint32_t f = 0u, len = 0u;
    uint64_t id = kNoId;
    if (wave == 0 && in) {
      f = flags[slot];
      len = lens[slot];
      id = ids[slot];
    }
    double total = 0.0;
    for (int h0 = 0; h0 < H; h0 += kFinHeads) {
      const int nh = min(kFinHeads, H - h0);
      constexpr int kPer = kFinHeads / kFinWaves;
      double v[kPer];
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int h = wave + kFinWaves * i;
        v[i] = (in && h < nh) ? __longlong_as_double(hmax[(h0 + h) * cap + slot]) : 0.0;
      }
#pragma unroll
      for (int i = 0; i < kPer; ++i) {
        const int h = wave + kFinWaves * i;
        if (h < nh) s_h[h][lane] = v[i];
      }
      __syncthreads();
      if (wave == 0) {
        // h ascending; LDS reads go out 16 at a time ahead of the adds
        int h = 0;
        for (; h + 16 <= nh; h += 16) {
          double x[16];
#pragma unroll
          for (int j = 0; j < 16; ++j) x[j] = s_h[h + j][lane];
#pragma unroll
          for (int j = 0; j < 16; ++j) total += x[j];
        }
        for (; h < nh; ++h) total += s_h[h][lane];
      }
      __syncthreads();
    }
    if (!q_bad_known) {
      q_bad = __ballot(qbad_lane != 0u) != 0ull;
      q_bad_known = true;
    }
    if (wave == 0) {
      float sc = __builtin_nanf("");
      if (f & 1u) {
        if (len == 0) {
          sc = 0.0f;
        } else if ((f & 2u) && !q_bad) {  // all key and query values finite
          sc = static_cast<float>(total / static_cast<double>(H));
        }
      }
      const bool need = isfinite(sc) && sc >= L.th_s;
      wl_consume(L, k, sc, id, slot, need);
    }
  }
  if (wave == 0 && lane < k) {
    store_entry(block_out + (static_cast<size_t>(qb) * gridDim.x + blockIdx.x) * k + lane, wl_entry(L),
                done ? route_tag(seq) : kNoSlot);
  }
  if (done && wave == 0) {
    // wave 0's list stores are complete before the end tick and the flag
    const size_t fi = static_cast<size_t>(qb) * gridDim.x + blockIdx.x;
    if (stamps && lane == 0) stamps[fi] = wall_clock64();
    __threadfence_system();
    if (lane == 0) done[fi] = seq;
  }
  // The maxima go back to zero for the next route after the flag, so the
  // host does not wait for these stores; the next route's kernels follow
  // this one on the stream.
  for (uint32_t base = blockIdx.x * kFinSlots; base < n_slots; base += gridDim.x * kFinSlots) {
    const bool in = base + lane < n_slots;
    const uint32_t slot = slot_list ? (in ? slot_list[base + lane] : 0u) : base + lane;
    if (in) {
      for (int h = wave; h < H; h += kFinWaves) hmax[h * cap + slot] = 0ull;
    }
  }
}

// ------------------------------------------------------- screen and refine
//
// For bf16, fp16 and INT8 banks every key token is screened on the matrix
// cores: s~ = |q~ . k| with the key as stored (bf16, fp16, or the law's
// fp16 dequantisation of INT8) and the query column rounded to the MFMA
// type (bf16 or fp16), fp32 accumulation.  For every query column and key
// token of a node the screen obeys |s~ - |s|| <= E = coef(column) * kmax +
// eabs(column) (see gqa_sr_prep_kernel), s the law's fp64 dot and kmax the
// node's largest key norm.  Within one work item, with
// M~ the largest screened value of a column, a token with s~ < M~ - 2E
// cannot hold the item's largest |s| (its |s| < M~ - E <= |s| of the token
// that gave M~), so the exact item maximum is the largest exact |s| over
// the candidates s~ >= M~ - 2E, recomputed in the law's fp64 order.  The
// result per (node, head) is therefore the law's value for every node --
// no shortlist, no certificate, no second route.

// MFMA operand type of a key storage type: bf16 keys run bf16 MFMA; fp16
// and int8 (dequantised to fp16 by the law) run fp16 MFMA.
template <int KDT>
struct ScreenTraits {
  static constexpr int kMfma = KDT == kBF16 ? kBF16 : kF16;
};

template <int MT>
__device__ inline f32x4 mfma16x16x32(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (MT == kBF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

__device__ inline uint32_t pack_f16x2(_Float16 lo, _Float16 hi) {
  return static_cast<uint32_t>(__builtin_bit_cast(unsigned short, lo)) |
         (static_cast<uint32_t>(__builtin_bit_cast(unsigned short, hi)) << 16);
}

constexpr int kMaxCols = 64;  // query columns (Qb * R * Qt) per screen pass
constexpr int kMaxSmaxCols = 128;  // per screen-only pass (gqa_smax_kernel, NT up to 8)


// ------------------------------------------------------- query columns
//
// A screen pass reads kv head g's query columns: column cg = (qb*Rc + rr)*Qc
// + tt (cg < cols) is query qb's row of head g*R + rr at query token tt of
// the pass (strides R and Qt, see "Query passes"), q_elems values after
// query qb-1's.

// Block-wide: stage the columns in s_q[cg][QS] (values at [0, HD), rows
// QS >= HD floats apart) as fp32 (exact: queries are fp32 or bf16) and
// derive each column's screen parameters
//  * scale(cg) = 2^-e, the power of two that brings max|q| of the column
//    under 2^emax (the MFMA type's safe range), 1 for ordinary values;
//  * the column's bound per unit of key norm, and its absolute part, in the
//    scaled units the screen works in (rounded up):
//      coef = ((gamma + delta + gamma*delta + rho) * ||q||
//              + sigma_q * (1 + gamma) * sqrt(hd) / scale + 2^-40 * ||q||) * scale
//      eabs = (sigma_k * sqrt(hd) * ||q|| + sigma_p * hd / scale) * scale
//    gamma bounds the fp32 accumulation, delta the query's rounding to
//    the MFMA type, rho the factoring of INT8 row scales out of the dot
//    product (0 elsewhere), sigma_q a scaled query value flushed or rounded
//    near zero, sigma_k a key value flushed near zero, sigma_p a product
//    lost to underflow, and 2^-40 the law's own fp64 rounding;
// With a rounded key plane (fp32 banks screened through an fp16 copy of
// their keys, k~ = k rounded with |k - k~| <= eps_rel |k| + eps_abs per
// value) the bound above holds for k~, whose norm is at most
// (1 + eps_rel) K + eps_abs sqrt(hd), and |q.(k - k~)| adds at most
// ||q|| (eps_rel K + eps_abs sqrt(hd)), so (before scaling)
//      coef' = coef (1 + eps_rel) + eps_rel ||q||
//      eabs' = eabs + (coef + ||q||) eps_abs sqrt(hd)
// (eps_rel = eps_abs = 0 for banks screened in their own values);
// into s_ec[cg] = {coef, eabs, scale, kcap} and s_bad[cg] = 1 when the
// column holds a non-finite value.  kcap = 2^127 / (scale * ||q|| *
// (1 + 2^-6)), rounded down: for a node whose key norm bound K stays below
// it, every product and partial sum of the screen's fp32 accumulation stays
// below 2^127 in magnitude (Cauchy-Schwarz; 1 + 2^-6 covers the roundings
// of query, key and sums), so no screened value overflows; for K >= kcap
// the bound is not established and the screen's users take E = +inf.
// Ends with a barrier.
template <int HD, int QS = HD>
__device__ inline void stage_columns(float* __restrict__ s_q, float4* __restrict__ s_ec,
                                     unsigned* __restrict__ s_bad, const void* __restrict__ query,
                                     int q_dtype, size_t q_elems, int cols, int R, int Qt, int Rc,
                                     int Qc, int g, int emax, double gamma, double delta,
                                     double rho, double sigma_q, double sigma_k, double sigma_p,
                                     double eps_rel, double eps_abs) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nwaves = blockDim.x / kWave;
  const int RQc = Rc * Qc;
  {
    // thread t stages value t % HD of columns t / HD, t / HD + per, ...
    const int per = static_cast<int>(blockDim.x) / HD;
    const int d = static_cast<int>(threadIdx.x) % HD;
    const int first = static_cast<int>(threadIdx.x) / HD;
    for (int cg = first; cg < cols && first < per; cg += per) {
      const int qb = cg / RQc;
      const int r = (cg % RQc) / Qc;
      const uint64_t src = static_cast<uint64_t>(qb) * q_elems +
                           (static_cast<uint64_t>(g * R + r) * Qt + cg % Qc) * HD + d;
      s_q[cg * QS + d] = q_dtype == kBF16 ? bf16_to_f32(static_cast<const uint16_t*>(query)[src])
                                          : static_cast<const float*>(query)[src];
    }
  }
  __syncthreads();
  // 16 lanes per column, four columns per wave at a time; the first lane
  // of each column derives its parameters
  const int sub = lane >> 4;
  const int sl = lane & 15;
  for (int c0 = wave * 4; c0 < cols; c0 += nwaves * 4) {
    const int cg = c0 + sub;
    double ss = 0.0;
    float mx = 0.0f;
    unsigned bad = 0u;
    if (cg < cols) {
      for (int d = sl; d < HD; d += 16) {
        const float f = s_q[cg * QS + d];
        bad |= isfinite(f) ? 0u : 1u;
        mx = fmaxf(mx, fabsf(f));
        ss = fma(static_cast<double>(f), static_cast<double>(f), ss);
      }
    }
#pragma unroll
    for (int off = 1; off < 16; off <<= 1) {
      ss += __shfl_xor(ss, off);
      mx = fmaxf(mx, __shfl_xor(mx, off));
      bad |= __shfl_xor(bad, off);
    }
    if (sl == 0 && cg < cols) {
      int e = 0;
      if (isfinite(mx) && mx > 0.0f) {
        const int ex = ilogbf(mx);  // mx in [2^ex, 2^(ex+1))
        if (ex >= emax) e = ex - emax + 1;
      }
      const float scale = ldexpf(1.0f, -e);
      const double norm = sqrt(ss) * (1.0 + 0x1p-40);
      const double sq = sqrt(static_cast<double>(HD));
      double c = (gamma + delta + gamma * delta + rho) * norm + sigma_q * (1.0 + gamma) * sq / scale +
                 0x1p-40 * norm;
      double ea = sigma_k * sq * norm + sigma_p * HD / scale;
      ea += (c + norm) * eps_abs * sq;
      c = c * (1.0 + eps_rel) + eps_rel * norm;
      const double up = 1.0 + 0x1p-20;
      c *= up * scale * up;
      ea *= up * scale * up;
      const double kcap = 0x1p127 / (static_cast<double>(scale) * norm * (1.0 + 0x1p-6)) * (1.0 - 0x1p-20);
      s_ec[cg] = make_float4(isfinite(c) ? static_cast<float>(c) * 1.000001f : INFINITY,
                             isfinite(ea) ? static_cast<float>(ea) * 1.000001f : INFINITY, scale,
                             kcap < 0x1p127 ? static_cast<float>(kcap) : INFINITY);
      s_bad[cg] = bad;
    }
  }
  __syncthreads();
}

// Dimension of position j (< 8) of lane quarter `quarter`'s part of MFMA
// k-block ks.  Natural order: ks*32 + quarter*8 + j, so a bf16/f16
// fragment is one 16-byte piece of a key row.  PERM (INT8 streams): a
// lane's k-blocks 2i and 2i+1 are the 16 consecutive dims i*64 +
// quarter*16 .. +16, one 16-byte piece of codes, so a wave's key load of
// 16 tokens is one contiguous 1 KiB run.  A dot product does not depend on
// the order of its terms, and the screen's bound holds for any order.
template <bool PERM>
__device__ inline int frag_dim(int ks, int quarter, int j) {
  if constexpr (PERM) return (ks >> 1) * 64 + quarter * 16 + (ks & 1) * 8 + j;
  return ks * 32 + quarter * 8 + j;
}

// Query fragments of the staged columns: fragment (nt, ks) of lane l holds
// column nt*16 + l%16 at dims frag_dim(ks, l/16, j), j < 8, of q * scale
// rounded to nearest even in the MFMA type (columns >= cols are zero).
// split (one column block, cols <= 8): column slots [cols, 2 cols) hold
// the remainders of columns [0, cols), q * scale minus its rounding,
// themselves rounded to the MFMA type, so that a column's screened value
// is the sum of its slot and the slot cols lanes up: the query's rounding
// error drops from u |q| to u^2 |q| per value (u the type's unit
// roundoff); the remainder is exact in fp32 (Sterbenz: within u of q).
template <int MT, bool PERM, int KS, int NT, int QS = 32 * KS>
__device__ inline void query_frags(u32x4 (&bq)[NT][KS], const float* __restrict__ s_q,
                                   const float4* __restrict__ s_ec, int cols, int r16,
                                   int quarter, bool split = false) {
  auto rne = [](float f) -> uint32_t {  // bf16 bits, round to nearest even (finite inputs)
    const uint32_t u = __float_as_uint(f);
    return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
  };
  auto rounded = [&](float f) -> float {  // f in the MFMA type, as fp32
    if constexpr (MT == kBF16) {
      return __uint_as_float(rne(f) << 16);
    } else {
      return static_cast<float>(static_cast<_Float16>(f));
    }
  };
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int cg = nt * 16 + r16;
    const bool lo = split && cg >= cols && cg < 2 * cols;
    const int src = lo ? cg - cols : cg;
    const bool has = src < cols;
    const float sc = has ? s_ec[src].z : 0.0f;
    const float* qc = s_q + min(src, cols - 1) * QS;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      uint32_t w[4];
#pragma unroll
      for (int j = 0; j < 8; j += 2) {
        const int d = frag_dim<PERM>(ks, quarter, j);
        float f0 = has ? qc[d] * sc : 0.0f;
        float f1 = has ? qc[d + 1] * sc : 0.0f;
        if (lo) {
          f0 -= rounded(f0);
          f1 -= rounded(f1);
        }
        if constexpr (MT == kBF16) {
          w[j / 2] = rne(f0) | (rne(f1) << 16);
        } else {
          w[j / 2] = pack_f16x2(static_cast<_Float16>(f0), static_cast<_Float16>(f1));
        }
      }
      bq[nt][ks].x = w[0];
      bq[nt][ks].y = w[1];
      bq[nt][ks].z = w[2];
      bq[nt][ks].w = w[3];
    }
  }
}

// Exact |dot| of one lane's (key token, query column) pair in the law's
// order: the token's pieces come from the planes (piece c at
// kp + (c/S)*L*S + c%S, kp the token's piece 0; chunks of S = 2^SS pieces),
// up to 8 pieces in flight at once, the column's values from qrow (LDS,
// fp32, exact, 16-byte aligned, read 4 values at a time).  Only lanes with
// `active` set read memory (the others return 0): the candidates are a few
// lanes of the wave, and their rows are all that is read again.
template <int KDT, int HD, int SS = 2>
__device__ __forceinline__ double exact_pair(bool active, const u32x4* __restrict__ kp,
                                             uint64_t L, const unsigned char* __restrict__ sp,
                                             int scale_dtype, int cpg, const float* qrow) {
  using T = KeyTraits<KDT>;
  constexpr int C = HD / T::kEpc;
  // pieces (16 bytes) per batch: 8, or 64 values when fewer
  constexpr int kB = C < 64 / T::kEpc ? C : (64 / T::kEpc < 8 ? 64 / T::kEpc : 8);
  double acc = 0.0;
  if (!active) return 0.0;
  for (int c0 = 0; c0 < C; c0 += kB) {
    u32x4 v[kB];
    float sc[kB];
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      v[b] = kp[(static_cast<uint64_t>((c0 + b) >> SS) * L << SS) + ((c0 + b) & ((1 << SS) - 1))];
      sc[b] = 0.0f;
      if constexpr (KDT == kI8) {
        sc[b] = load_scale(sp, scale_dtype, static_cast<uint64_t>((c0 + b) / cpg) * L);
      }
    }
#pragma unroll
    for (int b = 0; b < kB; ++b) {
      float f[T::kEpc];
      decode_chunk<KDT>(v[b], sc[b], f);
      const float4* q4 = reinterpret_cast<const float4*>(qrow + (c0 + b) * T::kEpc);
#pragma unroll
      for (int i = 0; i < T::kEpc / 4; ++i) {
        const float4 q = q4[i];
        acc = fma(static_cast<double>(f[4 * i]), static_cast<double>(q.x), acc);
        acc = fma(static_cast<double>(f[4 * i + 1]), static_cast<double>(q.y), acc);
        acc = fma(static_cast<double>(f[4 * i + 2]), static_cast<double>(q.z), acc);
        acc = fma(static_cast<double>(f[4 * i + 3]), static_cast<double>(q.w), acc);
      }
    }
  }
  return fabs(acc);
}

// Exact |dot| of the wavefront's candidate pairs (the lanes with `active`
// set: key token tok of the wavefront's plane, plane + tok*S + (c/S)*L*S +
// c%S holding its piece c, chunks of S = 2^SS pieces; query column values
// at qrow, LDS, fp32, 16-byte aligned),
// each in the law's order as in exact_pair, with the candidates' rows read
// once for the whole wavefront: in rounds of up to kRows candidates (about
// 4 KiB of rows) every lane loads 4 of the round's 16-byte pieces -- one
// memory round trip per round instead of a dependent batch per 64 values
// of one lane's row -- the pieces go to the wavefront's LDS rows s_rows
// (rows C + 1 pieces apart, so the candidates' reads of one piece spread
// over the banks), and each candidate lane runs its dot product from
// there.  s_tok holds the round's tokens.  Called by the whole
// wavefront (plane and L wave-uniform); inactive lanes return 0.
template <int RKDT, int HD>
struct GatherShape {
  static constexpr int kC = HD / KeyTraits<RKDT>::kEpc;  // pieces per row
  static constexpr int kRows = 4096 / (kC * 16) < 1 ? 1 : (4096 / (kC * 16) > 64 ? 64 : 4096 / (kC * 16));
  static constexpr int kStride = kC + 1;  // LDS row stride in pieces
  static constexpr int kPieces = kRows * kStride;
};

__device__ inline void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int RKDT, int HD, int SS = 2>
__device__ __forceinline__ double exact_gathered(bool active, const u32x4* __restrict__ plane,
                                                 uint32_t tok, uint64_t L, const float* qrow,
                                                 u32x4* s_rows, uint32_t* s_tok) {
  using T = KeyTraits<RKDT>;
  using GS = GatherShape<RKDT, HD>;
  constexpr int C = GS::kC;
  constexpr int kPer = (GS::kRows * C + kWave - 1) / kWave;  // pieces per lane per round
  const int lane = threadIdx.x & (kWave - 1);
  const uint64_t m = __ballot(active);
  const int n = __popcll(m);
  const int rank = __popcll(m & ((1ull << lane) - 1ull));
  double out = 0.0;
  for (int r0 = 0; r0 < n; r0 += GS::kRows) {
    const int nr = min(GS::kRows, n - r0);
    const bool mine = active && rank >= r0 && rank < r0 + nr;
    if (mine) s_tok[rank - r0] = tok;
    wave_lds_sync();
    u32x4 v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int pc = lane + kWave * i;
      if (pc < nr * C) {
        const int j = pc % C;
        v[i] = plane[(static_cast<uint64_t>(s_tok[pc / C]) << SS) +
                     (static_cast<uint64_t>(j >> SS) * L << SS) + (j & ((1 << SS) - 1))];
      }
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int pc = lane + kWave * i;
      if (pc < nr * C) s_rows[(pc / C) * GS::kStride + pc % C] = v[i];
    }
    wave_lds_sync();
    if (mine) {
      const u32x4* row = s_rows + (rank - r0) * GS::kStride;
      double acc = 0.0;
#pragma unroll
      for (int j = 0; j < C; ++j) {
        float f[T::kEpc];
        decode_chunk<RKDT>(row[j], 0.0f, f);
        const float4* q4 = reinterpret_cast<const float4*>(qrow + j * T::kEpc);
#pragma unroll
        for (int i = 0; i < T::kEpc / 4; ++i) {
          const float4 q = q4[i];
          acc = fma(static_cast<double>(f[4 * i]), static_cast<double>(q.x), acc);
          acc = fma(static_cast<double>(f[4 * i + 1]), static_cast<double>(q.y), acc);
          acc = fma(static_cast<double>(f[4 * i + 2]), static_cast<double>(q.z), acc);
          acc = fma(static_cast<double>(f[4 * i + 3]), static_cast<double>(q.w), acc);
        }
      }
      out = fabs(acc);
    }
    // the next round writes the same rows and addresses
    wave_lds_sync();
  }
  return out;
}

// Screen and refine; grid (kv heads, ceil(items / 4)) -- or, past the
// grid's y limit, (ceil(items / 4), kv heads) -- one wavefront per
// (item, kv head g).
//
// Each block first stages kv head g's query columns of the Qb queries for
// the pass (stage_columns: fp32 values for the screen fragments and the
// exact recomputation, scale and error-bound parameters per column); the
// blocks of item block 0 write qflags[qb*kv + g] = 1 when a value of query
// qb read by kv head g is non-finite (0 otherwise on the first pass,
// flags_or = 0; later passes only raise it).
// Columns with a non-finite value take no part in the screen (every score
// of that query is NaN).  The item's tokens stream in 16-token tiles, two
// tiles ahead of the one being screened.  Lane l sees column
// nt*16 + l%16 of tokens (l/16)*4 + i of every tile; it keeps the two
// largest screened values with their tokens and the third largest value.
// At the item's end: M~ per column (over the four lanes of the column),
// threshold M~ - 2E; if no lane's third value reaches the threshold the
// candidates are among the kept two and are recomputed exactly, otherwise
// the item is screened again tile by tile and every token at or above the
// threshold is recomputed.  The per-column exact maxima, divided by
// sqrt(hd) (monotone), fold into hmax[qb*hstride + (g*R + rr)*cap + slot]
// (double bits, atomicMax).
//
// XF32: the keys are an fp32 bank's fp16 copy (same rows, chunks of 4
// pieces); the exact recomputation reads the fp32 rows from xkeys (also
// chunks of 4 pieces), and eps_rel / eps_abs carry the copy's rounding
// into the bound (stage_columns).
//
// Waves per SIMD asked of the compiler: 4 (at most 128 VGPRs) for the fp32
// bank's single column block at head_dim 128, which otherwise takes a few
// registers more for its exact recomputation and loses a wave of the
// stream; 2 or 1 elsewhere.
template <int KDT, int KS, int NT, bool XF32>
constexpr int sr_waves_per_simd() {
  return XF32 && NT == 1 && KS == 4 ? 4 : ((NT * KS <= 16 && KS <= 4 && (KDT != kI8 || KS == 4 || NT == 1)) ? 2 : 1);
}

template <int KDT, int KS, int NT, bool XF32 = false>
__global__ __launch_bounds__(kUnitWaves * kWave, (sr_waves_per_simd<KDT, KS, NT, XF32>())) void gqa_sr_kernel(
    const unsigned char* __restrict__ keys, const unsigned char* __restrict__ xkeys,
    const unsigned char* __restrict__ scales, int scale_dtype, int group_size,
    const Item* __restrict__ items, uint32_t n_items, int kv, int R, int Qt, int Rc, int Qc,
    const void* __restrict__ query, int q_dtype, size_t q_elems, int Qb, int emax,
    double gamma, double delta, double sigma_q, double sigma_k, double sigma_p,
    double eps_rel, double eps_abs, unsigned* __restrict__ qflags, int flags_or, const float* __restrict__ kmax, double denom,
    unsigned long long* __restrict__ hmax, size_t hstride, size_t cap, int g_fast, int split,
    RouteStamps stamps, unsigned seq) {
  route_start_stamp(stamps, seq);
  using KT = KeyTraits<KDT>;
  constexpr int MT = ScreenTraits<KDT>::kMfma;
  constexpr int HD = 32 * KS;
  constexpr int C = HD / KT::kEpc;  // chunks per key row
  // [cols][QS]: the block's query columns; rows padded by 4 floats, so the
  // exact recomputations of 16 columns (one lane each, 16-byte reads at
  // the same offset) fall in distinct banks
  constexpr int QS = HD + 4;
  extern __shared__ __align__(16) float s_q[];
  __shared__ float4 s_ec[kMaxCols];  // {coef, eabs, scale, kcap} per column
  __shared__ unsigned s_bad[kMaxCols];
  // each wavefront's gathered candidate rows: an fp32 bank's exact
  // recomputations read fp32 rows, 512 bytes at head_dim 128, which a
  // lane alone would fetch in four dependent batches (exact_gathered: one
  // round trip for the wave); rows of the screened keys themselves take
  // one or two batches and are recomputed lane by lane (exact_pair), which
  // measured faster for them
  using GS = GatherShape<kF32, HD>;
  __shared__ u32x4 s_rows[kUnitWaves][XF32 ? GS::kPieces : 1];
  __shared__ uint32_t s_tok[kUnitWaves][XF32 ? GS::kRows : 1];
  const int lane = threadIdx.x & (kWave - 1);
  // g_fast: grid (kv, item blocks), so consecutive blocks read one node's
  // neighbouring kv-head blocks; else grid (item blocks, kv)
  const int g = g_fast ? blockIdx.x : blockIdx.y;
  const uint32_t item_block = g_fast ? blockIdx.y : blockIdx.x;
  const int RQc = Rc * Qc;
  const int cols = Qb * RQc;
  // The wave's first tiles are requested before the block prepares its
  // query columns, so the two overlap; a wave without an item issues no
  // loads but joins the block's barriers.
  const uint32_t item_raw = item_block * kUnitWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const bool has_item = item_raw < n_items;
  const Item it = items[has_item ? item_raw : n_items - 1];
  const uint64_t L = it.len;
  const uint64_t row0 = it.base + static_cast<uint64_t>(g) * L;
  const int G = KDT == kI8 ? HD / group_size : 1;
  const int cpg = KDT == kI8 ? group_size / KT::kEpc : 1;
  const int ses = scale_dtype == kF16 ? 2 : 4;
  const u32x4* kplane = reinterpret_cast<const u32x4*>(keys) + row0 * C;
  const unsigned char* splane = KDT == kI8 ? scales + row0 * G * ses : nullptr;
  const int quarter = lane >> 4;
  const int r16 = lane & 15;
  const uint32_t last = it.t0 + it.count - 1;  // last token of the item
  const int ntiles = static_cast<int>((it.count + 15) / 16);

  // Raw data of tile `tile` for this lane: token min(t0 + 16*tile + l%16,
  // last), dims ks*32 + (l/16)*8 .. +8 (loads are unconditional; rows past
  // the item are masked when folded).  INT8 tiles keep codes and scales
  // and are dequantised when folded, so no load is waited for early.
  typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
  struct Tile {
    u32x4 v[KDT == kI8 ? 1 : KS];
    u32x2 c[KDT == kI8 ? KS : 1];
    float s[KDT == kI8 ? KS : 1];
  };
  auto load_tile = [&](Tile& b, int tile) {
    const uint32_t t = min(it.t0 + static_cast<uint32_t>(tile) * 16 + r16, last);
    // chunks of 4 pieces: piece p of token t at kplane + (p/4)*L*4 + t*4 + p%4
    if constexpr (KDT != kI8) {
      // piece ks*4 + quarter: one 1 KiB run per load over the 16 tokens
      const u32x4* p = kplane + static_cast<uint64_t>(t) * 4 + quarter;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) b.v[ks] = __builtin_nontemporal_load(p + ks * 4 * L);
    } else {
      // half (quarter & 1) of piece ks*2 + quarter/2
      const u32x2* p = reinterpret_cast<const u32x2*>(kplane + static_cast<uint64_t>(t) * 4 + (quarter >> 1)) +
                       (quarter & 1);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        b.c[ks] = __builtin_nontemporal_load(p + 2 * ((ks >> 1) * 4 * L + 2 * (ks & 1)));
        b.s[ks] = load_scale(splane, scale_dtype,
                             static_cast<uint64_t>((ks * 32 + quarter * 8) / group_size) * L + t);
      }
    }
  };
  Tile x0, x1, x2, x3, x4;
  if (has_item) {
    load_tile(x0, 0);
    load_tile(x1, 1);
    load_tile(x2, 2);
    load_tile(x3, 3);
  }
  stage_columns<HD, QS>(s_q, s_ec, s_bad, query, q_dtype, q_elems, cols, R, Qt, Rc, Qc, g, emax,
                        gamma, delta, 0.0, sigma_q, sigma_k, sigma_p, eps_rel, eps_abs);
  __syncthreads();
  if (item_block == 0 && threadIdx.x < static_cast<unsigned>(Qb)) {
    unsigned bad = 0u;
    for (int j = 0; j < RQc; ++j) bad |= s_bad[threadIdx.x * RQc + j];
    if (bad || !flags_or) qflags[threadIdx.x * kv + g] = bad;
  }
  if (!has_item) return;

  // B fragments from the staged columns: fragment (nt, ks) lane l holds
  // column nt*16 + l%16 at dims ks*32 + (l/16)*8 + j, j < 8.
  u32x4 bq[NT][KS];
  // split (fp32 queries, at most 8 columns): remainders in the idle slots
  const bool sp = NT == 1 && split != 0;
  query_frags<MT, false, KS, NT, QS>(bq, s_q, s_ec, cols, r16, quarter, sp);

  auto frag = [&](const Tile& b, int ks) -> u32x4 {
    if constexpr (KDT != kI8) {
      return b.v[ks];
    } else {
      const uint32_t w[2] = {b.c[ks].x, b.c[ks].y};
      const float sc = b.s[ks];
      uint32_t o[4];
#pragma unroll
      for (int i = 0; i < 2; ++i) {
        o[2 * i] = pack_f16x2(dequant_i8(stored_code(w[i], 0), sc), dequant_i8(stored_code(w[i], 1), sc));
        o[2 * i + 1] = pack_f16x2(dequant_i8(stored_code(w[i], 2), sc), dequant_i8(stored_code(w[i], 3), sc));
      }
      u32x4 a;
      a.x = o[0];
      a.y = o[1];
      a.z = o[2];
      a.w = o[3];
      return a;
    }
  };
  // Screened |s~| of the lane's 4 rows of `tile` for column block nt;
  // rows past the item read -inf.
  auto screen = [&](const Tile& b, int tile, int nt, float (&v)[4]) {
    f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) c = mfma16x16x32<MT>(frag(b, ks), bq[nt][ks], c);
    const uint32_t tb = static_cast<uint32_t>(tile) * 16 + quarter * 4;  // item-relative
    float cv[4] = {c.x, c.y, c.z, c.w};
    if (sp) {
      // the remainder slot of column r16 (< cols) is cols lanes up, in
      // the same quarter; lanes of other slots are not live
#pragma unroll
      for (int i = 0; i < 4; ++i) cv[i] += __shfl(cv[i], lane + cols);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = tb + i < it.count ? fabsf(cv[i]) : -INFINITY;
  };

  float b1[NT], b2[NT], b3[NT];
  uint32_t t1[NT], t2[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    b1[nt] = b2[nt] = b3[nt] = -INFINITY;
    t1[nt] = t2[nt] = 0u;
  }
  auto fold = [&](const Tile& b, int tile) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float v[4];
      screen(b, tile, nt, v);
      const uint32_t tb = static_cast<uint32_t>(tile) * 16 + quarter * 4;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        // NaN compares false everywhere and is never kept
        const bool gt1 = v[i] > b1[nt];
        const bool gt2 = v[i] > b2[nt];
        const bool gt3 = v[i] > b3[nt];
        b3[nt] = gt2 ? b2[nt] : (gt3 ? v[i] : b3[nt]);
        const float nb2 = gt1 ? b1[nt] : (gt2 ? v[i] : b2[nt]);
        const uint32_t nt2 = gt1 ? t1[nt] : (gt2 ? tb + i : t2[nt]);
        b2[nt] = nb2;
        t2[nt] = nt2;
        if (gt1) {
          b1[nt] = v[i];
          t1[nt] = tb + i;
        }
      }
    }
  };

  // stream: five tile buffers, four tiles in flight ahead of the fold.
  // The exits between steps let the compiler move a step's load into the
  // path that continues, behind the fold, so the wave drains its loads
  // every few tiles; a single exit (as in gqa_smax_kernel) would fold up
  // to four reloaded tiles past every item's end instead, which measured
  // slower here, where items are short and a fold tracks three values.
  int tile = 0;
  auto step = [&](Tile& now, Tile& free) -> bool {
    load_tile(free, tile + 4);  // past the end: reloads the last token
    fold(now, tile);
    return ++tile < ntiles;
  };
  while (step(x0, x4) && step(x1, x0) && step(x2, x1) && step(x3, x2) && step(x4, x3)) {
  }

  // thresholds and candidates
  const float km = kmax[it.slot];
  double thr[NT];
  bool live[NT];
  bool amb = false;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    float m = b1[nt];
    m = fmaxf(m, __shfl_xor(m, 16));
    m = fmaxf(m, __shfl_xor(m, 32));
    const int cg = nt * 16 + r16;
    live[nt] = cg < cols && s_bad[min(cg, cols - 1)] == 0u;
    const float4 ec = s_ec[min(cg, cols - 1)];
    const double e = km < ec.w ? static_cast<double>(ec.x) * static_cast<double>(km) + static_cast<double>(ec.y)
                               : static_cast<double>(INFINITY);
    thr[nt] = static_cast<double>(m) - 2.0 * e;
    if (live[nt]) {
      amb = amb || !(thr[nt] > -INFINITY) || !isfinite(e) ||
            static_cast<double>(b3[nt]) >= thr[nt];
    }
  }
  const bool enumerate = __ballot(amb) != 0ull;

  const int wv = threadIdx.x / kWave;
  auto pair = [&](bool active, uint32_t t, int cg) -> double {
    const uint32_t tt = min(it.t0 + t, last);
    if constexpr (XF32) {
      const u32x4* xplane = reinterpret_cast<const u32x4*>(xkeys) + row0 * (HD / 4);
      return exact_gathered<kF32, HD>(active, xplane, tt, L, s_q + min(cg, cols - 1) * QS,
                                      s_rows[wv], s_tok[wv]);
    } else {
      return exact_pair<KDT, HD>(active, kplane + static_cast<uint64_t>(tt) * 4, L,
                                 KDT == kI8 ? splane + static_cast<size_t>(tt) * ses : nullptr,
                                 scale_dtype, cpg, s_q + min(cg, cols - 1) * QS);
    }
  };
  double best[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) best[nt] = -1.0;
  if (!enumerate) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int cg = nt * 16 + r16;
      const bool c1 = live[nt] && static_cast<double>(b1[nt]) >= thr[nt];
      const bool c2 = live[nt] && static_cast<double>(b2[nt]) >= thr[nt];
      if (__ballot(c1) != 0ull) {
        const double x = pair(c1, t1[nt], cg);
        if (c1) best[nt] = x;
      }
      if (__ballot(c2) != 0ull) {
        const double x = pair(c2, t2[nt], cg);
        if (c2) best[nt] = (x > best[nt] || isnan(x)) ? x : best[nt];
      }
    }
  } else {
    for (int tl = 0; tl < ntiles; ++tl) {
      Tile a;
      load_tile(a, tl);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float v[4];
        screen(a, tl, nt, v);
        const int cg = nt * 16 + r16;
        const uint32_t tb = static_cast<uint32_t>(tl) * 16 + quarter * 4;
        for (int i = 0; i < 4; ++i) {
          // a NaN screen value (non-finite keys) is recomputed too
          const bool c = live[nt] && (static_cast<double>(v[i]) >= thr[nt] || isnan(v[i]) ||
                                      !(thr[nt] > -INFINITY));
          if (__ballot(c) != 0ull) {
            const double x = pair(c, tb + i, cg);
            if (c) best[nt] = (x > best[nt] || isnan(x)) ? x : best[nt];
          }
        }
      }
    }
  }
  // per column over its four lanes, then one atomic per valid column
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    unsigned long long bits = best[nt] >= 0.0 || isnan(best[nt])
                                  ? __double_as_longlong(best[nt] / denom)
                                  : 0ull;
#pragma unroll
    for (int off = 16; off < kWave; off <<= 1) {
      const unsigned long long o = __shfl_xor(bits, off);
      bits = o > bits ? o : bits;
    }
    const int cg = nt * 16 + lane;
    if (lane < 16 && cg < cols && bits != 0ull) {
      const int qb = cg / RQc;
      const int r = (cg % RQc) / Qc;
      atomicMax(hmax + qb * hstride + static_cast<size_t>(g * R + r) * cap + it.slot, bits);
    }
  }
}

// ------------------------------------------------------ bound and verify
//
// Routes with many query columns per kv head (batched queries) take the
// bound-and-verify path: a screen-only pass keeps, per (query column,
// node), the largest screened |q~.k| over the node's tokens; the screen's
// error bound turns those maxima into an interval [lb, ub] holding each
// node's score; every node whose ub reaches the k-th largest lb of its
// query is a candidate; the law runs exactly (fp64, gqa_exact_kernel) on the
// candidates only, and the top-k is taken over their exact scores.  At
// least k nodes score >= tau (the k-th largest lb) and every other node
// scores < tau, in float as well (lb rounded down, ub rounded up), so the
// top-k of the candidates is the law's top-k, ties included.

// Maximum over the 16 lanes of a DPP row (lanes 16j .. 16j + 15), in every
// lane of the row: quad_perm [1,0,3,2] and [2,3,0,1] give each lane its
// quad's maximum, row_half_mirror (lane i of 8 reads lane 7 - i) the other
// quad's, row_mirror (lane i of 16 reads lane 15 - i) the other half's.
__device__ inline uint32_t row_max16(uint32_t x) {
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0xB1, 0xF, 0xF, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x4E, 0xF, 0xF, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x141, 0xF, 0xF, false)));
  x = max(x, static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(x), 0x140, 0xF, 0xF, false)));
  return x;
}

// Four stored int8 codes (one dword) as four exact f16 values (two dwords,
// codes 0,1 then 2,3): the stored byte u = code + 128 goes under the
// exponent of 1024 (f16 bits 0x6400 | u = 1024 + u), then 1152 comes off.
// Exact: every value involved is an integer below 2048.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
__device__ inline void codes_to_f16(uint32_t u, uint32_t& lo, uint32_t& hi) {
  const f16x2 bias = {static_cast<_Float16>(1152.0f), static_cast<_Float16>(1152.0f)};
  lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) - bias);
  hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) - bias);
}

// Query passes of one screen-only launch (see gqa_smax_kernel): pass p is
// heads r0[p] .. + rc[p] of each kv head, tokens t0[p] .. + qc[p].
struct SmaxPasses {
  int r0[4], rc[4], t0[4], qc[4];
};

// Screen-only pass; grid (P, kv heads), persistent: wave w of block b walks
// the work items b*4 + w, b*4 + w + 4P, ... -- one item per live node with
// key tokens, all of its tokens, so each (node, kv head) has one writer --
// as one stream of 16-token tiles,
// four tiles in flight ahead of the one being screened, across item
// boundaries.  The block stages kv head g's query columns once
// (stage_columns); blocks with blockIdx.x == 0 write colinfo[g*cols + cg]
// = {coef, eabs, scale, kcap} for the bounds kernel.
//
// The MFMA runs with the query columns as the row operand, so lane l holds
// columns nt*16 + (l/16)*4 + v (v < 4) of token l%16, the token whose key
// piece it loaded.  Each lane keeps a running max of |s~| per column;
// loads of tokens past an item's end are clamped to its last token, whose
// value a max already holds.  FACT (INT8 rows with one scale each): the
// codes enter the MFMA as exact f16 integers and the lane's row scale
// multiplies its results, s~ = scale_t * |q~ . c|; the difference to the
// law's fp16(code * scale) keys is in the bound (rho, and a norm bound
// that covers c * scale).  At a node's end the maxima of the 16 lanes of
// each column combine and are stored at
// hmaxf[(slot*kv + g)*colstride + gc] (float bits, scaled units): one
// (node, kv head)'s columns are one contiguous run, written by one
// coalesced store.
//
// Query passes: the launch reads pass (r0, Rc, t0, Qc) of Qb queries
// (query advanced to the pass's first value, see "Query passes"); its
// column cg = qb*Rc*Qc + rr*Qc + tt is column
// gc = qb*R*Qt + (r0 + rr)*Qt + t0 + tt of the query's full set, so passes
// over disjoint parts of a query fill disjoint cells of the same rows, and
// colinfo[g*colstride + gc] holds each column's bound parameters.
//
// NP > 1 (a single wide query): a block is 8 wavefronts, wavefront w
// screening pass w % NP for walker blockIdx.x * (8/NP) + w / NP, so the NP
// wavefronts of a walker read the same tiles at about the same time and
// the bank is streamed from HBM once for NP passes (the tiles come again
// from L2; the loads are not marked nontemporal).  Each pass's columns are
// staged in their own LDS region.
template <int KDT, int KS, int NT, bool FACT, bool SF16, int NP = 1>
__global__ __launch_bounds__((NP == 1 ? kUnitWaves : 8) * kWave,
                              (NT * KS <= 16 && (KS <= 4 || NT == 1)) ? 2 : 1) void gqa_smax_kernel(
    const unsigned char* __restrict__ keys, const unsigned char* __restrict__ scales,
    int scale_dtype, int group_size, const Item* __restrict__ items, uint32_t n_items, int kv,
    int R, int Qt, SmaxPasses ps, const void* __restrict__ query, int q_dtype,
    size_t q_elems, int Qb, int emax,
    double gamma, double delta, double rho, double sigma_q, double sigma_k, double sigma_p,
    double eps_rel, double eps_abs, float4* __restrict__ colinfo, unsigned* __restrict__ hmaxf,
    int colstride) {
  using KT = KeyTraits<KDT>;
  constexpr int MT = ScreenTraits<KDT>::kMfma;
  constexpr bool PERM = KDT == kI8;
  constexpr int HD = 32 * KS;
  constexpr int C = HD / KT::kEpc;            // 16-byte pieces per key row
  constexpr int NL = PERM ? KS / 2 : KS;       // 16-byte key loads per lane per 16 tokens
  // INT8 rows are half as wide: a tile is 32 tokens (two halves of 16, lane
  // l holding tokens l%16 and 16 + l%16) at head dims up to 128, so a tile
  // is 4 KiB as for 16-bit keys
  constexpr int NH = (KDT == kI8 && KS <= 4) ? 2 : 1;
  constexpr uint32_t TT = 16 * NH;              // tokens per tile
  static_assert(!FACT || KDT == kI8, "row-scale factoring is for INT8 banks");
  constexpr uint32_t kEnd = 0x80000000u;
  static_assert(NP == 1 || NP == 2 || NP == 4, "1, 2 or 4 passes per launch");
  static_assert(NP == 1 || NT <= 4, "split passes hold at most 64 columns each");
  constexpr int WPB = NP == 1 ? kUnitWaves : 8 / NP;  // walkers per block
  constexpr int kPassCols = NP == 1 ? kMaxSmaxCols : kMaxCols;
  extern __shared__ float s_q[];                    // [NP][NT*16][HD]
  __shared__ float4 s_ec[NP * kPassCols];
  __shared__ unsigned s_bad[NP * kPassCols];
  const int lane = threadIdx.x & (kWave - 1);
  const int g = blockIdx.y;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int pi = NP == 1 ? 0 : wave % NP;           // this wavefront's pass
  // the query's full column index of column cg of pass p
  auto full_col_of = [&](int p, int cg) {
    const int RQp = ps.rc[p] * ps.qc[p];
    const int qb = cg / RQp;
    const int rem = cg - qb * RQp;
    return qb * R * Qt + (ps.r0[p] + rem / ps.qc[p]) * Qt + ps.t0[p] + rem % ps.qc[p];
  };
  const int cols = Qb * ps.rc[pi] * ps.qc[pi];
  auto full_col = [&](int cg) { return full_col_of(pi, cg); };
  const int quarter = lane >> 4;
  const int r16 = lane & 15;
  const uint32_t stride = gridDim.x * WPB;
  uint32_t li = blockIdx.x * WPB + (NP == 1 ? wave : wave / NP);
  const bool has_item = li < n_items;
  const int G = KDT == kI8 ? HD / group_size : 1;
  const int ses = scale_dtype == kF16 ? 2 : 4;

  // Loader: the item being loaded, its next tile, the next item's
  // descriptor (fetched one item ahead).
  struct Src {
    const u32x4* kp;           // piece 0 of the (slot, g) block
    const unsigned char* sp;   // its scales (INT8)
    uint64_t L;                // padded rows of the block
    uint32_t t0, last, ntiles, slot;
  };
  auto source = [&](const Item& it) {
    Src d;
    const uint64_t row0 = it.base + static_cast<uint64_t>(g) * it.len;
    d.kp = reinterpret_cast<const u32x4*>(keys) + row0 * C;
    d.sp = KDT == kI8 ? scales + row0 * G * ses : nullptr;
    d.L = it.len;
    d.t0 = it.t0;
    d.last = it.t0 + it.count - 1;
    d.ntiles = (it.count + TT - 1) / TT;
    d.slot = it.slot;
    return d;
  };
  // INT8 scales stay raw bits until the tile is folded: a conversion next
  // to the load would make the wave wait for every load in flight
  struct Tile {
    u32x4 v[NH][NL];
    uint32_t s[NH][KDT == kI8 ? (FACT ? 1 : NL) : 1];
    uint32_t fin;  // slot | kEnd on an item's last tile, else kNoSlot
  };
  auto scale_raw = [](const unsigned char* sp, uint64_t idx) -> uint32_t {
    if constexpr (SF16) {
      return reinterpret_cast<const unsigned short*>(sp)[idx];
    } else {
      return reinterpret_cast<const uint32_t*>(sp)[idx];
    }
  };
  auto scale_of = [](uint32_t raw) -> float {
    if constexpr (SF16) {
      return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<unsigned short>(raw)));
    } else {
      return __uint_as_float(raw);
    }
  };
  Src ld = source(items[has_item ? li : 0]);
  uint32_t lt = 0;
  uint32_t lnext = li + stride;
  Item nx = items[min(lnext, n_items - 1)];
  bool ldone = false;
  auto load_tile = [&](Tile& b, uint32_t tile) {
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      const uint32_t t = min(ld.t0 + tile * TT + h * 16 + r16, ld.last);
      // piece p of token t at kp + (p/4)*L*4 + t*4 + p%4 (chunks of 4
      // pieces); load i reads piece i*4 + quarter: 16 tokens x 4 pieces,
      // 1 KiB
      const u32x4* p = ld.kp + static_cast<uint64_t>(t) * 4 + quarter;
#pragma unroll
      for (int i = 0; i < NL; ++i) {
        if constexpr (NP == 1) {
          b.v[h][i] = __builtin_nontemporal_load(p + i * 4 * ld.L);
        } else {
          b.v[h][i] = p[i * 4 * ld.L];
        }
      }
      if constexpr (KDT == kI8) {
        if constexpr (FACT) {
          b.s[h][0] = scale_raw(ld.sp, t);
        } else {
#pragma unroll
          for (int i = 0; i < NL; ++i) {
            b.s[h][i] = scale_raw(ld.sp, static_cast<uint64_t>((i * 64 + quarter * 16) / group_size) * ld.L + t);
          }
        }
      }
    }
  };
  // Load the stream's next tile into b (past the stream's end: the last
  // tile again, marked kNoSlot).
  auto load_next = [&](Tile& b) {
    load_tile(b, ldone ? ld.ntiles - 1 : lt);
    b.fin = kNoSlot;
    if (ldone) return;
    if (lt + 1 < ld.ntiles) {
      ++lt;
      return;
    }
    const bool end = lnext >= n_items;
    b.fin = ld.slot | (end ? kEnd : 0u);
    if (end) {
      ldone = true;
      return;
    }
    ld = source(nx);
    lt = 0;
    lnext += stride;
    nx = items[min(lnext, n_items - 1)];
  };
  Tile x0, x1, x2, x3, x4;
  if (has_item) {
    load_next(x0);
    load_next(x1);
    load_next(x2);
    load_next(x3);
  }
  // every pass's columns, each in its own LDS region (the query advanced
  // to the pass's first value, see "Query passes")
  const size_t esz = q_dtype == kBF16 ? 2 : 4;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const unsigned char* qp = static_cast<const unsigned char*>(query) +
                              static_cast<size_t>(ps.r0[p] * Qt + ps.t0[p]) * HD * esz;
    const int cols_p = Qb * ps.rc[p] * ps.qc[p];
    stage_columns<HD>(s_q + static_cast<size_t>(p) * NT * 16 * HD, s_ec + p * kPassCols,
                      s_bad + p * kPassCols, qp, q_dtype, q_elems, cols_p, R, Qt, ps.rc[p],
                      ps.qc[p], g, emax, gamma, delta, rho, sigma_q, sigma_k, sigma_p, eps_rel,
                      eps_abs);
    if (blockIdx.x == 0) {
      for (int cg = threadIdx.x; cg < cols_p; cg += blockDim.x) {
        colinfo[static_cast<size_t>(g) * colstride + full_col_of(p, cg)] = s_ec[p * kPassCols + cg];
      }
    }
  }
  if (!has_item) return;

  u32x4 bq[NT][KS];
  query_frags<MT, PERM, KS, NT>(bq, s_q + static_cast<size_t>(pi) * NT * 16 * HD,
                                s_ec + pi * kPassCols, cols, r16, quarter);

  // key fragment ks of half h of a tile: 8 values of the lane's token in
  // the MFMA type
  auto key_frags = [&](const Tile& b, int h, u32x4 (&bk)[KS]) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      if constexpr (KDT != kI8) {
        bk[ks] = b.v[h][ks];
      } else {
        const u32x4 v = b.v[h][ks >> 1];
        const uint32_t w0 = (ks & 1) ? v.z : v.x;
        const uint32_t w1 = (ks & 1) ? v.w : v.y;
        if constexpr (FACT) {
          uint32_t o[4];
          codes_to_f16(w0, o[0], o[1]);
          codes_to_f16(w1, o[2], o[3]);
          bk[ks].x = o[0];
          bk[ks].y = o[1];
          bk[ks].z = o[2];
          bk[ks].w = o[3];
        } else {
          const float sc = scale_of(b.s[h][ks >> 1]);
          const uint32_t w[2] = {w0, w1};
          uint32_t o[4];
#pragma unroll
          for (int i = 0; i < 2; ++i) {
            o[2 * i] = pack_f16x2(dequant_i8(stored_code(w[i], 0), sc), dequant_i8(stored_code(w[i], 1), sc));
            o[2 * i + 1] = pack_f16x2(dequant_i8(stored_code(w[i], 2), sc), dequant_i8(stored_code(w[i], 3), sc));
          }
          bk[ks].x = o[0];
          bk[ks].y = o[1];
          bk[ks].z = o[2];
          bk[ks].w = o[3];
        }
      }
    }
  };
  // running maxima as float bits: the values are non-negative, so their
  // bit patterns order like the values (a NaN, possible only from
  // non-finite keys or query values, wins; such a node or query is never
  // ranked, by its flags)
  uint32_t m[NT][4];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int v = 0; v < 4; ++v) m[nt][v] = 0u;
  }
  auto fold = [&](const Tile& b) {
    f32x4 c[NH][NT];
    float sc[NH];
#pragma unroll
    for (int h = 0; h < NH; ++h) {
      u32x4 bk[KS];
      key_frags(b, h, bk);
      sc[h] = 1.0f;
      if constexpr (FACT) sc[h] = scale_of(b.s[h][0]);
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        c[h][nt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) c[h][nt] = mfma16x16x32<MT>(bq[nt][ks], bk[ks], c[h][nt]);
      }
    }
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float x0 = FACT ? fabsf(c[0][nt][v]) * sc[0] : fabsf(c[0][nt][v]);
        if constexpr (NH == 2) {
          const float x1 = FACT ? fabsf(c[1][nt][v]) * sc[1] : fabsf(c[1][nt][v]);
          m[nt][v] = max(max(m[nt][v], __float_as_uint(x0)), __float_as_uint(x1));  // v_max3_u32
        } else {
          m[nt][v] = max(m[nt][v], __float_as_uint(x0));
        }
      }
    }
  };
  // node end: the column maxima over the 16 lanes of each quarter; lane
  // (quarter, r16) then stores column nt*16 + quarter*4 + v for
  // nt = r16/4 + 4*i, v = r16%4: one (node, kv head)'s columns are one
  // contiguous run, written by coalesced stores
  constexpr int kStores = (NT + 3) / 4;
  int my_gc[kStores];
  bool my_col[kStores];
#pragma unroll
  for (int i = 0; i < kStores; ++i) {
    const int cg = ((r16 >> 2) + 4 * i) * 16 + quarter * 4 + (r16 & 3);
    my_col[i] = (r16 >> 2) + 4 * i < NT && cg < cols;
    my_gc[i] = my_col[i] ? full_col(cg) : 0;
  }
  auto emit = [&](uint32_t slot) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        m[nt][v] = row_max16(m[nt][v]);
      }
    }
    uint32_t mine[kStores];
#pragma unroll
    for (int i = 0; i < kStores; ++i) mine[i] = 0u;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        if (r16 == (nt % 4) * 4 + v) mine[nt / 4] = m[nt][v];
        m[nt][v] = 0u;
      }
    }
#pragma unroll
    for (int i = 0; i < kStores; ++i) {
      if (my_col[i]) hmaxf[(static_cast<size_t>(slot) * kv + g) * colstride + my_gc[i]] = mine[i];
    }
  };
  // Groups of five steps with one exit, at the bottom: steps after the
  // stream's last tile fold reloaded tiles marked kNoSlot, which emit
  // nothing (an exit between steps would leave the compiler unable to keep
  // the rotating tile buffers in place, and it would drain the loads).
  bool done = false;
  auto step = [&](Tile& now, Tile& free) {
    load_next(free);
    __builtin_amdgcn_sched_barrier(0);
    fold(now);
    if (now.fin != kNoSlot && !done) {
      emit(now.fin & ~kEnd);
      done = (now.fin & kEnd) != 0u;
    }
  };
  do {
    step(x0, x4);
    step(x1, x0);
    step(x2, x1);
    step(x3, x2);
    step(x4, x3);
  } while (!done);
}

// Norm bound K of a node's keys as the screen used them: its largest key
// norm kmax, or with FACT (INT8 rows with one scale each, screened as
// scale * codes) the bound on ||code * scale||,
// (kmax + 2^-25 sqrt(hd)) / (1 - 2^-10).
__host__ __device__ inline double screen_key_norm(float kmax, bool fact, int hd) {
  return fact ? (static_cast<double>(kmax) + 0x1p-25 * sqrt(static_cast<double>(hd))) / (1.0 - 0x1p-10)
              : static_cast<double>(kmax);
}

// Node-score bounds; grid (queries, blocks), 4 wavefronts, lane = slot,
// grid-stride over groups of 64 slots.  For query qb and slot s, each
// column's screened maximum m (hmaxf[(s*kv + g)*colstride + cg], cg the
// column of head h = g*R + r and query token qi; scaled units) bounds the
// law's
// max_t |dot| / sqrt(hd) of its head and query token from below by
// max(0, m - E) / scale / denom and from above by (m + E) / scale / denom,
// E = coef * K + eabs (colinfo), K = screen_key_norm(kmax[s]), and
// E = +inf where K >= kcap (the screen may have overflowed).
// best_h is the max over the head's query tokens, so its bounds are the
// max of theirs; the score (sum_h best_h) / H lies in [lb, ub] with
// lb = sum_h lo_h / H, ub = sum_h hi_h / H, widened by 2^-40 for the fp64
// arithmetic on both sides and rounded outward to float.  Writes
// lbub[qb*cap + s] = (lb, ub): (0, 0) for a live node without key tokens,
// NaN for slots that are not ranked (free, non-finite keys, non-finite
// query; their cells are never read) or certainly unranked (a lower bound
// past the float range: the law's score is +inf); the block's k best
// lower bounds among nodes with a finite upper bound (tie law) go to
// block_out[(qb*blocks + block)*k ..).  Also
// zeroes the candidates kernel's counters: counters[qb] (query qb's
// candidates) and counters[n_counters - 1] (work items).  cols is the
// stride of colinfo's kv-head rows.  kStaged: the query's H*Qt column
// parameters are staged in LDS (else read from colinfo, for queries of
// many tokens).
template <bool kStaged>
__global__ __launch_bounds__(kFinWaves * kWave) void gqa_bounds_kernel(
    const unsigned* __restrict__ hmaxf, int colstride, size_t cap, int H, int Qt, int R, int cols,
    int kv, uint32_t n_slots, const uint32_t* __restrict__ lens,
    const uint32_t* __restrict__ flags, const uint64_t* __restrict__ ids,
    const unsigned* __restrict__ kmax, const float4* __restrict__ colinfo,
    const unsigned* __restrict__ qbad, int fact, int hd, int k, float2* __restrict__ lbub,
    Cand* __restrict__ block_out, uint32_t* __restrict__ counters, int n_counters, int nq) {
  __shared__ Cand s_lists[kFinWaves][kMaxTopK];
  extern __shared__ float4 s_ci[];  // [H*Qt]: query qb's {coef, eabs, 1/scale, kcap}, (h, qi) order
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  // 1-D grid of nq * nsblk blocks (nsblk a multiple of 8).  Blocks go to
  // the 8 XCDs in turn (block b to XCD b % 8), each with its own L2, and a
  // slot's maxima for all queries share cache lines: block b takes slot
  // block ((b/8) / nq) * 8 + b % 8 of query (b/8) % nq, so the nq blocks
  // of one slot block run on one XCD, one after another in dispatch order.
  const uint32_t nsblk = gridDim.x / static_cast<uint32_t>(nq);
  const uint32_t bj = blockIdx.x / 8u;
  const int qb = static_cast<int>(bj % static_cast<uint32_t>(nq));
  const uint32_t sblk = (bj / static_cast<uint32_t>(nq)) * 8u + blockIdx.x % 8u;
  if (sblk == 0 && threadIdx.x == 0) {
    counters[qb] = 0u;
    if (qb == 0) counters[n_counters - 1] = 0u;
  }
  const double denom = sqrt(static_cast<double>(hd));
  const int HQ = H * Qt;
  const int RQ = R * Qt;
  const bool vec4 = RQ % 4 == 0 && colstride % 4 == 0;
  // column parameters of (h, qi), with 1/scale (the scale is a power of
  // two: its inverse is exact)
  auto col_params = [&](int i) {
    const int h = i / Qt;
    float4 ci = colinfo[static_cast<size_t>(h / R) * cols + (qb * R + h % R) * Qt + i % Qt];
    ci.z = 1.0f / ci.z;
    return ci;
  };
  if constexpr (kStaged) {
    for (int i = threadIdx.x; i < HQ; i += blockDim.x) s_ci[i] = col_params(i);
    __syncthreads();
  }
  bool q_bad = false;
  for (int g0 = 0; g0 < kv; g0 += kWave) {
    q_bad = q_bad || (g0 + lane < kv && qbad[qb * kv + g0 + lane] != 0u);
  }
  q_bad = __ballot(q_bad) != 0ull;
  WaveList Lw;
  wl_init(Lw);
  const uint32_t gstride = nsblk * kFinWaves * kWave;
  for (uint32_t base = (sblk * kFinWaves + wave) * kWave; base < n_slots; base += gstride) {
    const uint32_t slot = base + lane;
    const bool in = slot < n_slots;
    const uint32_t f = in ? flags[slot] : 0u;
    const uint32_t len = in ? lens[slot] : 0u;
    const uint64_t id = in ? ids[slot] : kNoId;
    const float kmf = in ? __uint_as_float(kmax[slot]) : 0.0f;
    const double K = screen_key_norm(kmf, fact != 0, hd);
    // only ranked nodes with key tokens have screened maxima
    const bool screened = in && (f & 3u) == 3u && len != 0u && !q_bad;
    const unsigned* cells = hmaxf + static_cast<size_t>(screened ? slot : 0u) * kv * colstride;
    // (h, qi) in ascending order, the cells of 16 of them loaded ahead.
    // (h, qi) = (g*R + r, qi) is cell g*colstride + qb*RQ + r*Qt + qi: a
    // query's cells of one kv head are one run of RQ, loaded 4 at a time
    // when runs and rows are multiples of 4 cells (16-byte aligned)
    constexpr int kAhead = 16;
    double lo_sum = 0.0, hi_sum = 0.0, lo_h = 0.0, hi_h = 0.0;
    for (int j0 = 0; j0 < HQ; j0 += kAhead) {
      float mv[kAhead];
      if (vec4) {
#pragma unroll
        for (int j = 0; j < kAhead; j += 4) {
          const int hq = j0 + j;
          uint4 w = make_uint4(0u, 0u, 0u, 0u);
          if (screened && hq < HQ) {
            w = *reinterpret_cast<const uint4*>(cells + (hq / RQ) * colstride + qb * RQ + hq % RQ);
          }
          mv[j] = __uint_as_float(w.x);
          mv[j + 1] = __uint_as_float(w.y);
          mv[j + 2] = __uint_as_float(w.z);
          mv[j + 3] = __uint_as_float(w.w);
        }
      } else {
#pragma unroll
        for (int j = 0; j < kAhead; ++j) {
          const int hq = j0 + j;
          mv[j] = 0.0f;
          if (screened && hq < HQ) mv[j] = __uint_as_float(cells[(hq / RQ) * colstride + qb * RQ + hq % RQ]);
        }
      }
#pragma unroll
      for (int j = 0; j < kAhead; ++j) {
        const int hq = j0 + j;
        if (hq < HQ) {
          const float4 ci = kStaged ? s_ci[hq] : col_params(hq);
          const double e = K < static_cast<double>(ci.w)
                               ? (static_cast<double>(ci.x) * K + static_cast<double>(ci.y)) * (1.0 + 0x1p-50)
                               : static_cast<double>(INFINITY);
          const double m = static_cast<double>(mv[j]);
          const double inv = static_cast<double>(ci.z);
          const double lo = fmax(0.0, m - e) * inv;
          const double hi = (m + e) * inv;
          lo_h = fmax(lo_h, lo);
          hi_h = (hi > hi_h || isnan(hi)) ? hi : hi_h;
          if (hq % Qt == Qt - 1) {  // the head's last query token
            lo_sum += lo_h;
            hi_sum += hi_h;
            lo_h = hi_h = 0.0;
          }
        }
      }
    }
    const double lb = lo_sum / denom / static_cast<double>(H) * (1.0 - 0x1p-40);
    const double ub = hi_sum / denom / static_cast<double>(H) * (1.0 + 0x1p-40);
    float lbf = __builtin_nanf(""), ubf = __builtin_nanf("");
    if (in && (f & 1u)) {
      if (len == 0) {
        lbf = ubf = 0.0f;
      } else if ((f & 2u) && !q_bad && !isinf(static_cast<float>(lb))) {
        // (a lower bound that rounds to +inf means the law's float score
        // is +inf too: the node is certainly not ranked and stays NaN)
        lbf = static_cast<float>(lb);
        if (static_cast<double>(lbf) > lb) lbf = nextafterf(lbf, -INFINITY);
        ubf = static_cast<float>(ub);
        if (static_cast<double>(ubf) < ub || isnan(ub)) ubf = isnan(ub) ? INFINITY : nextafterf(ubf, INFINITY);
      }
    }
    if (in) lbub[static_cast<size_t>(qb) * cap + slot] = make_float2(lbf, ubf);
    // a lower bound counts towards the k best only when the node's score
    // is certainly finite (ub below the float range), as only finite
    // scores are ranked
    wl_consume(Lw, k, lbf, id, slot, isfinite(lbf) && isfinite(ubf) && lbf >= Lw.th_s);
  }
  if (lane < kMaxTopK) s_lists[wave][lane] = wl_entry(Lw);
  __syncthreads();
  if (wave == 0) {
    WaveList B;
    block_merge<kFinWaves>(s_lists, k, B);
    if (lane < k) block_out[(static_cast<size_t>(qb) * nsblk + sblk) * k + lane] = wl_entry(B);
  }
}

// The same bounds for queries of many tokens (H*Qt cells per node): one
// wavefront per node at a time, its lanes over heads -- lane l takes heads
// l, l + 64, ..., each the max over its Qt query tokens' bounds -- and the
// heads' sums formed by a reduction across the wavefront (a different
// order than the sequential sum, which the 2^-40 widening covers many
// times over: the fp64 sum of H non-negative terms is within H * 2^-53 of
// exact).  grid (queries, blocks), kFinWaves wavefronts; wavefront w of
// block b takes nodes (b * kFinWaves + w) + i * blocks * kFinWaves.
// Outputs as gqa_bounds_kernel.
__global__ __launch_bounds__(kFinWaves * kWave) void gqa_bounds_wide_kernel(
    const unsigned* __restrict__ hmaxf, int colstride, size_t cap, int H, int Qt, int R, int cols,
    int kv, uint32_t n_slots, const uint32_t* __restrict__ lens,
    const uint32_t* __restrict__ flags, const uint64_t* __restrict__ ids,
    const unsigned* __restrict__ kmax, const float4* __restrict__ colinfo,
    const unsigned* __restrict__ qbad, int fact, int hd, int k, float2* __restrict__ lbub,
    Cand* __restrict__ block_out, uint32_t* __restrict__ counters, int n_counters) {
  __shared__ Cand s_lists[kFinWaves][kMaxTopK];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int qb = blockIdx.x;
  const uint32_t sblk = blockIdx.y, nsblk = gridDim.y;
  if (sblk == 0 && threadIdx.x == 0) {
    counters[qb] = 0u;
    if (qb == 0) counters[n_counters - 1] = 0u;
  }
  const double denom = sqrt(static_cast<double>(hd));
  bool q_bad = false;
  for (int g0 = 0; g0 < kv; g0 += kWave) {
    q_bad = q_bad || (g0 + lane < kv && qbad[qb * kv + g0 + lane] != 0u);
  }
  q_bad = __ballot(q_bad) != 0ull;
  WaveList Lw;
  wl_init(Lw);
  for (uint32_t slot = sblk * kFinWaves + wave; slot < n_slots; slot += nsblk * kFinWaves) {
    const uint32_t f = flags[slot];
    const uint32_t len = lens[slot];
    const uint64_t id = ids[slot];
    const double K = screen_key_norm(__uint_as_float(kmax[slot]), fact != 0, hd);
    const bool screened = (f & 3u) == 3u && len != 0u && !q_bad;
    double lo_sum = 0.0, hi_sum = 0.0;
    if (screened) {
      const unsigned* cells = hmaxf + static_cast<size_t>(slot) * kv * colstride;
      for (int h = lane; h < H; h += kWave) {
        const size_t c0 = static_cast<size_t>(h / R) * colstride + (qb * R + h % R) * Qt;
        const size_t i0 = static_cast<size_t>(h / R) * cols + (qb * R + h % R) * Qt;
        double lo_h = 0.0, hi_h = 0.0;
        // the head's Qt cells and column parameters, 8 loaded before any
        // is used
        constexpr int kB = 8;
        for (int t0 = 0; t0 < Qt; t0 += kB) {
          float4 ci[kB];
          float mv[kB];
#pragma unroll
          for (int j = 0; j < kB; ++j) {
            const int t = min(t0 + j, Qt - 1);
            ci[j] = colinfo[i0 + t];
            mv[j] = __uint_as_float(cells[c0 + t]);
          }
#pragma unroll
          for (int j = 0; j < kB; ++j) {
            if (t0 + j >= Qt) break;
            const double e = K < static_cast<double>(ci[j].w)
                                 ? (static_cast<double>(ci[j].x) * K + static_cast<double>(ci[j].y)) * (1.0 + 0x1p-50)
                                 : static_cast<double>(INFINITY);
            const double m = static_cast<double>(mv[j]);
            const double inv = 1.0 / static_cast<double>(ci[j].z);  // a power of two: exact
            const double lo = fmax(0.0, m - e) * inv;
            const double hi = (m + e) * inv;
            lo_h = fmax(lo_h, lo);
            hi_h = (hi > hi_h || isnan(hi)) ? hi : hi_h;
          }
        }
        lo_sum += lo_h;
        hi_sum += hi_h;
      }
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) {
        lo_sum += __shfl_xor(lo_sum, off);
        const double o = __shfl_xor(hi_sum, off);
        hi_sum = isnan(o) ? o : hi_sum + o;
      }
    }
    const double lb = lo_sum / denom / static_cast<double>(H) * (1.0 - 0x1p-40);
    const double ub = hi_sum / denom / static_cast<double>(H) * (1.0 + 0x1p-40);
    float lbf = __builtin_nanf(""), ubf = __builtin_nanf("");
    if (f & 1u) {
      if (len == 0) {
        lbf = ubf = 0.0f;
      } else if ((f & 2u) && !q_bad && !isinf(static_cast<float>(lb))) {
        lbf = static_cast<float>(lb);
        if (static_cast<double>(lbf) > lb) lbf = nextafterf(lbf, -INFINITY);
        ubf = static_cast<float>(ub);
        if (static_cast<double>(ubf) < ub || isnan(ub)) ubf = isnan(ub) ? INFINITY : nextafterf(ubf, INFINITY);
      }
    }
    if (lane == 0) lbub[static_cast<size_t>(qb) * cap + slot] = make_float2(lbf, ubf);
    wl_consume(Lw, k, lbf, id, slot, lane == 0 && isfinite(lbf) && isfinite(ubf) && lbf >= Lw.th_s);
  }
  if (lane < kMaxTopK) s_lists[wave][lane] = wl_entry(Lw);
  __syncthreads();
  if (wave == 0) {
    WaveList B;
    block_merge<kFinWaves>(s_lists, k, B);
    if (lane < k) block_out[(static_cast<size_t>(qb) * nsblk + sblk) * k + lane] = wl_entry(B);
  }
}

// The law on the candidates of a query of many tokens (one query, every
// column screened by gqa_smax_kernel): per (candidate, kv head g) pair a
// wavefront first finds, for each of g's heads r, the columns (query
// tokens) whose screened maximum can still hold the head's maximum -- the
// screen bounds each column's law maximum in [max(0, m - E), m + E] / scale
// (gqa_bounds_kernel), so a column whose upper bound lies below the largest
// lower bound of its head's columns cannot -- and evaluates the law (fp64,
// d ascending, |dot| / sqrt(hd)) only on those columns, over all of the
// node's tokens, folding the per-column maxima into hmax[(g*R + r)*cap +
// slot] with the 64-bit atomicMax.  The head's maximum over its columns is
// unchanged: the column that holds it has an upper bound at or above every
// column's lower bound.  A NaN bound keeps its column.  q64 holds the query
// columns as doubles, value d of column gc at q64[(g*hd + d)*rqp + gc].
// Wavefronts walk pairs p = w, w + W, ... (p = candidate * kv + g).
constexpr int kSparseCols = 4;  // columns evaluated per read of a pair's key rows
template <int KDT>
__global__ __launch_bounds__(kUnitWaves * kWave) void gqa_exact_sparse_kernel(
    const unsigned char* __restrict__ keys, const unsigned char* __restrict__ scales,
    int scale_dtype, int group_size, int sS, const uint32_t* __restrict__ cand_slots,
    const uint32_t* __restrict__ cand_count, int kv, int R, int Qt, int hd, int colstride,
    const unsigned* __restrict__ hmaxf, const float4* __restrict__ colinfo,
    const unsigned* __restrict__ kmax, int fact, const uint64_t* __restrict__ tok_off,
    const uint32_t* __restrict__ lens, const double* __restrict__ q64, int rqp, double denom,
    unsigned long long* __restrict__ hmax, size_t cap) {
  using T = KeyTraits<KDT>;
  extern __shared__ double s_qv[];  // [kUnitWaves][kSparseCols][hd]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const uint32_t W = gridDim.x * kUnitWaves;
  const uint32_t n_pairs = cand_count[0] * static_cast<uint32_t>(kv);
  const int C = hd / T::kEpc;
  const int G = KDT == kI8 ? hd / group_size : 1;
  const int cpg = KDT == kI8 ? group_size / T::kEpc : 1;
  const int ses = scale_dtype == kF16 ? 2 : 4;
  for (uint32_t pr = blockIdx.x * kUnitWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
       pr < n_pairs; pr += W) {
    const uint32_t slot = cand_slots[pr / kv];
    const int g = static_cast<int>(pr % kv);
    const uint32_t L = lens[slot];
    if (L == 0u) continue;
    const double K = screen_key_norm(__uint_as_float(kmax[slot]), fact != 0, hd);
    const unsigned* cells = hmaxf + (static_cast<size_t>(slot) * kv + g) * colstride;
    const float4* cinf = colinfo + static_cast<size_t>(g) * colstride;
    const uint64_t Lp = (L + kTokAlign - 1) & ~(kTokAlign - 1);
    const uint64_t row0 = tok_off[slot] * static_cast<uint64_t>(kv) + static_cast<uint64_t>(g) * Lp;
    const u32x4* kb = reinterpret_cast<const u32x4*>(keys) + row0 * C;
    // the screen's bounds of column c of head r (unscaled)
    auto bounds = [&](int c, double& lo, double& hi) {
      const float4 ci = cinf[c];
      const double e = K < static_cast<double>(ci.w)
                           ? (static_cast<double>(ci.x) * K + static_cast<double>(ci.y)) * (1.0 + 0x1p-50)
                           : static_cast<double>(INFINITY);
      const double m = static_cast<double>(__uint_as_float(cells[c]));
      const double inv = 1.0 / static_cast<double>(ci.z);  // a power of two: exact
      lo = fmax(0.0, m - e) * inv;
      hi = (m + e) * inv;
    };
    // kept columns in (head, token) order, kSparseCols at a time: their
    // query rows go to this wavefront's LDS rows, and each lane reads its
    // token's key row once per group, one fp64 sum per column
    double* qv = s_qv + static_cast<size_t>(wave) * kSparseCols * hd;
    int r = 0, q0 = 0;
    uint64_t mask = 0ull;
    bool run_loaded = false;
    double lo_max = 0.0;
    auto next_col = [&]() -> int {
      while (r < R) {
        if (!run_loaded) {
          if (q0 == 0) {
            double m = 0.0;
            for (int x0 = 0; x0 < Qt; x0 += kWave) {
              if (x0 + lane < Qt) {
                double lo, hi;
                bounds(r * Qt + x0 + lane, lo, hi);
                m = fmax(m, lo);
              }
            }
#pragma unroll
            for (int off = 1; off < kWave; off <<= 1) m = fmax(m, __shfl_xor(m, off));
            lo_max = m;
          }
          bool keep = false;
          if (q0 + lane < Qt) {
            double lo, hi;
            bounds(r * Qt + q0 + lane, lo, hi);
            keep = !(hi < lo_max);
          }
          mask = __ballot(keep);
          run_loaded = true;
        }
        if (mask != 0ull) {
          const int bit = __ffsll(static_cast<long long>(mask)) - 1;
          mask &= mask - 1ull;
          return r * Qt + q0 + bit;
        }
        run_loaded = false;
        q0 += kWave;
        if (q0 >= Qt) {
          q0 = 0;
          ++r;
        }
      }
      return -1;
    };
    const double* qb0 = q64 + static_cast<size_t>(g) * hd * rqp;
    for (;;) {
      int gcs[kSparseCols];
      int n = 0;
      for (int j = 0; j < kSparseCols; ++j) {
        gcs[j] = n == j ? next_col() : -1;
        if (gcs[j] >= 0) ++n;
      }
      if (n == 0) break;
      // stage the group's query rows (unused rows zero)
      for (int idx = lane; idx < kSparseCols * hd; idx += kWave) {
        const int j = idx / hd;
        const int d = idx - j * hd;
        qv[idx] = j < n ? qb0[static_cast<size_t>(d) * rqp + gcs[j]] : 0.0;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      double best[kSparseCols];
#pragma unroll
      for (int j = 0; j < kSparseCols; ++j) best[j] = 0.0;
      for (uint32_t t0 = 0; t0 < L; t0 += kWave) {
        const uint32_t t = min(t0 + static_cast<uint32_t>(lane), L - 1u);
        double acc[kSparseCols];
#pragma unroll
        for (int j = 0; j < kSparseCols; ++j) acc[j] = 0.0;
        for (int c = 0; c < C; ++c) {
          const u32x4 v = piece_ptr(kb, Lp, sS, t, c)[0];
          float sc = 0.0f;
          if constexpr (KDT == kI8) {
            sc = load_scale(scales + (row0 * G + t) * ses, scale_dtype,
                            static_cast<uint64_t>(c / cpg) * Lp);
          }
          float f[T::kEpc];
          decode_chunk<KDT>(v, sc, f);
#pragma unroll
          for (int e = 0; e < T::kEpc; ++e) {
            const double fe = static_cast<double>(f[e]);
            const int d = c * T::kEpc + e;
#pragma unroll
            for (int j = 0; j < kSparseCols; ++j) acc[j] = fma(fe, qv[j * hd + d], acc[j]);
          }
        }
        if (t0 + lane < L) {
#pragma unroll
          for (int j = 0; j < kSparseCols; ++j) {
            const double x = fabs(acc[j]);
            best[j] = (x > best[j] || isnan(x)) ? x : best[j];
          }
        }
      }
      // the group's LDS rows are read before the next group writes them
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // max(|dot|)/denom equals the law's max(|dot|/denom) (division by a
      // positive constant is monotone under rounding to nearest)
      for (int j = 0; j < n; ++j) {
        unsigned long long bits = __double_as_longlong(best[j] / denom);
#pragma unroll
        for (int off = 1; off < kWave; off <<= 1) {
          const unsigned long long o = __shfl_xor(bits, off);
          bits = o > bits ? o : bits;
        }
        const int hr = gcs[j] / Qt;
        if (lane == 0 && bits != 0ull) atomicMax(hmax + static_cast<size_t>(g * R + hr) * cap + slot, bits);
      }
    }
  }
}

// Candidates; grid (queries, slot blocks), kCandWaves wavefronts per
// block.  tau = the k-th best lower bound of query qb (merged from the
// bounds kernel's block lists, by every block; -inf when fewer than k
// nodes are ranked); every slot with ub >= tau is a candidate: its slot
// goes to cand_slots[qb*cap ..) (count in cand_count[qb]) and its key
// tokens, in items of `chunk` tokens, to the shared list citems (count in
// *n_citems) with q = qb, for the exact kernel.  Both counts are zeroed
// before the launch (by the bounds kernel); each wavefront with candidates
// reserves its places with one atomicAdd on each.
constexpr int kCandWaves = 16;
__global__ __launch_bounds__(kCandWaves * kWave) void gqa_cands_kernel(
    const Cand* __restrict__ lists, uint32_t n_lists, int k, const float2* __restrict__ lbub,
    size_t cap, uint32_t n_slots, const uint64_t* __restrict__ tok_off,
    const uint32_t* __restrict__ lens, int kv, uint32_t chunk, uint32_t* __restrict__ cand_slots,
    uint32_t* __restrict__ cand_count, Item* __restrict__ citems, uint32_t* __restrict__ n_citems) {
  __shared__ Cand s_lists[kCandWaves][kMaxTopK];
  __shared__ float s_tau;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int qb = blockIdx.x;
  WaveList G;
  wl_init(G);
  wl_consume_global(G, k, lists + static_cast<size_t>(qb) * n_lists * k, n_lists * k,
                    static_cast<uint32_t>(wave), kCandWaves);
  if (lane < kMaxTopK) s_lists[wave][lane] = wl_entry(G);
  __syncthreads();
  if (wave == 0) {
    WaveList B;
    block_merge<kCandWaves>(s_lists, k, B);
    const float t = lane_f32(B.s, k - 1);
    if (lane == 0) s_tau = isfinite(t) ? t : -INFINITY;
  }
  __syncthreads();
  const float tau = s_tau;
  const float2* lq = lbub + static_cast<size_t>(qb) * cap;
  const uint32_t gstride = gridDim.y * kCandWaves * kWave;
  for (uint32_t base = (blockIdx.y * kCandWaves + wave) * kWave; base < n_slots; base += gstride) {
    const uint32_t slot = base + lane;
    bool c = false;
    uint32_t len = 0u;
    if (slot < n_slots) {
      const float ub = lq[slot].y;
      c = ub >= tau;  // NaN (not ranked) compares false
      if (c) len = lens[slot];
    }
    const uint64_t cm = __ballot(c);
    if (cm == 0ull) continue;
    const uint32_t n_items = c ? (len + chunk - 1) / chunk : 0u;
    // wave prefix sums of candidates and of their items
    uint32_t pre_items = n_items;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const uint32_t o = __shfl_up(pre_items, off);
      if (lane >= off) pre_items += o;
    }
    const uint32_t tot_items = __shfl(pre_items, kWave - 1);
    pre_items -= n_items;
    uint32_t cbase = 0u, ibase = 0u;
    if (lane == 0) {
      cbase = atomicAdd(cand_count + qb, static_cast<uint32_t>(__popcll(cm)));
      if (tot_items) ibase = atomicAdd(n_citems, tot_items);
    }
    cbase = __shfl(cbase, 0);
    ibase = __shfl(ibase, 0);
    if (c) {
      const uint32_t rank = static_cast<uint32_t>(__popcll(cm & ((1ull << lane) - 1ull)));
      cand_slots[static_cast<size_t>(qb) * cap + cbase + rank] = slot;
      const uint64_t b0 = tok_off[slot] * static_cast<uint64_t>(kv);
      const uint32_t Lp = (len + kTokAlign - 1) & ~(kTokAlign - 1);
      for (uint32_t j = 0; j < n_items; ++j) {
        Item it;
        it.base = b0;
        it.slot = slot;
        it.t0 = j * chunk;
        it.count = min(chunk, len - j * chunk);
        it.len = Lp;
        it.q = static_cast<uint32_t>(qb);
        it.pad = 0u;
        citems[ibase + pre_items + j] = it;
      }
    }
  }
}

// ----------------------------------------------------------- bank upkeep

// Placement of new slots: copy their key rows (and INT8 scales) from the
// staging layout -- per slot [kv][len][head_dim] values, rows of
// [kv][len][G] scales, slot blocks back to back from staged token 0 -- into
// the chunk planes, and gather key statistics on the way: nonfinite[slot]
// set when a decoded value is not finite; kmax[slot] = max over kv heads
// and tokens of ||k||_2, rounded up (float bits, atomicMax).  Items carry
// the destination base; the staged row of (item, g, t) is
// base - src_base + g*len + t.  grid (ceil(items / 4), kv).
//
// INT8 codes are written in their stored form (stored_code).
//
// With `skeys` (fp32 banks only) each row is also written, rounded to
// fp16 (nearest even), to the bank's fp16 copy: the same rows as chunk
// planes of 4 pieces, which the matrix-core screens read.  A slot with a
// finite value whose fp16 rounding is not finite (|value| >= 65520) gets
// kmax = +inf: its screen bound is then infinite and every one of its
// tokens is recomputed exactly.
template <int KDT>
__global__ __launch_bounds__(kUnitWaves * kWave) void gqa_place_kernel(
    const u32x4* __restrict__ src_keys, const unsigned char* __restrict__ src_scales,
    uint64_t src_base, unsigned char* __restrict__ keys,
    unsigned char* __restrict__ scales, int scale_dtype, int group_size,
    const Item* __restrict__ items, uint32_t n_items, int hd, int sS,
    uint32_t* __restrict__ nonfinite, unsigned* __restrict__ kmax,
    unsigned char* __restrict__ skeys) {
  using T = KeyTraits<KDT>;
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t item_i = blockIdx.x * kUnitWaves + threadIdx.x / kWave;
  if (item_i >= n_items) return;
  const int g = blockIdx.y;
  const Item it = items[item_i];
  const int C = hd / T::kEpc;
  const int G = KDT == kI8 ? hd / group_size : 1;
  const int cpg = KDT == kI8 ? group_size / T::kEpc : 1;
  const size_t ses = scale_dtype == kF16 ? 2 : 4;
  const uint64_t row0 = it.base + static_cast<uint64_t>(g) * it.len;
  const uint64_t srow0 = row0 - src_base;
  u32x4* dst = reinterpret_cast<u32x4*>(keys) + row0 * C;
  const int S = 1 << sS;
  bool bad = false, sbad = false;
  double mx = 0.0;
  for (uint32_t t = it.t0 + lane; t < it.t0 + it.count; t += kWave) {
    const u32x4* src = src_keys + (srow0 + t) * C;
    double acc = 0.0;
    for (int c = 0; c < C; ++c) {
      u32x4 v = src[c];
      if constexpr (KDT == kI8) v = to_stored_codes(v);
      dst[(static_cast<uint64_t>(c >> sS) * it.len << sS) + (static_cast<uint64_t>(t) << sS) + (c & (S - 1))] = v;
      if constexpr (KDT == kF32) {
        if (skeys) {
          // fp16 piece c/2 of the copy (8 values), half c%2 of it
          const float f[4] = {__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z),
                              __uint_as_float(v.w)};
          _Float16 h[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            h[e] = static_cast<_Float16>(f[e]);
            sbad = sbad || (isfinite(f[e]) && !isfinite(static_cast<float>(h[e])));
          }
          const int p = c >> 1;
          u32x4* sdst = reinterpret_cast<u32x4*>(skeys) + row0 * (C / 2) +
                        (static_cast<uint64_t>(p >> 2) * it.len << 2) + (static_cast<uint64_t>(t) << 2) + (p & 3);
          typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
          u32x2 w;
          w.x = pack_f16x2(h[0], h[1]);
          w.y = pack_f16x2(h[2], h[3]);
          reinterpret_cast<u32x2*>(sdst)[c & 1] = w;
        }
      }
      float sc = 0.0f;
      if constexpr (KDT == kI8) {
        const int j = c / cpg;
        const unsigned char* s_in = src_scales + ((srow0 + t) * G + j) * ses;
        unsigned char* s_out = scales + ((row0 * G) + static_cast<uint64_t>(j) * it.len + t) * ses;
        if (c % cpg == 0) {
          if (ses == 2) {
            *reinterpret_cast<uint16_t*>(s_out) = *reinterpret_cast<const uint16_t*>(s_in);
          } else {
            *reinterpret_cast<uint32_t*>(s_out) = *reinterpret_cast<const uint32_t*>(s_in);
          }
        }
        sc = load_scale(src_scales, scale_dtype, (srow0 + t) * G + j);
      }
      float f[T::kEpc];
      decode_chunk<KDT>(v, sc, f);
#pragma unroll
      for (int e = 0; e < T::kEpc; ++e) {
        bad = bad || !isfinite(f[e]);
        acc = fma(static_cast<double>(f[e]), static_cast<double>(f[e]), acc);
      }
    }
    mx = fmax(mx, acc);
  }
  if (__ballot(bad) != 0ull && lane == 0) atomicOr(nonfinite + it.slot, 1u);
  float nrm = static_cast<float>(sqrt(mx) * (1.0 + 1e-6));
  if (!isfinite(nrm)) nrm = 3.0e38f;
  if (sbad) nrm = INFINITY;
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) nrm = fmaxf(nrm, __shfl_xor(nrm, off));
  if (lane == 0) atomicMax(kmax + it.slot, __float_as_uint(nrm));
}

// Slot metadata for placed nodes; meta = [count slots][count tok_off]
// [count lens][count ids].  flags are committed after the statistics.
__global__ void gqa_set_slots_kernel(const uint64_t* __restrict__ meta,
                                     uint64_t count,
                                     uint64_t* __restrict__ tok_off,
                                     uint32_t* __restrict__ lens,
                                     uint64_t* __restrict__ ids,
                                     uint32_t* __restrict__ flags,
                                     uint32_t* __restrict__ nonfinite,
                                     unsigned* __restrict__ kmax) {
  for (uint64_t i = blockIdx.x * static_cast<uint64_t>(blockDim.x) + threadIdx.x;
       i < count; i += static_cast<uint64_t>(gridDim.x) * blockDim.x) {
    const uint64_t s = meta[i];
    tok_off[s] = meta[count + i];
    lens[s] = static_cast<uint32_t>(meta[2 * count + i]);
    ids[s] = meta[3 * count + i];
    flags[s] = 0u;
    nonfinite[s] = 0u;
    kmax[s] = 0u;
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

__global__ void gqa_clear_flags_kernel(unsigned* __restrict__ flags, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) flags[i] = 0u;
}

// Route filters (cpp/grm_runtime.cpp:3074-3104; bits as route_filter_bits,
// :2793-2838): slot i passes when, for each category c with filters (bit c
// of cats), its bits meet that category's 16-bit mask at shift 16c.  A
// failing slot loses its live bit in the route's copy of the flags, which
// every score path reads, so it scores NaN and never ranks.
__global__ void gqa_filter_flags_kernel(const uint32_t* __restrict__ flags,
                                        const uint64_t* __restrict__ fbits, uint64_t n,
                                        uint64_t fmask, uint32_t cats,
                                        uint32_t* __restrict__ out) {
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += stride) {
    const uint64_t hit = fbits[i] & fmask;
    bool ok = true;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if ((cats >> c) & 1u) ok = ok && ((hit >> (16 * c)) & 0xffffull) != 0;
    }
    out[i] = ok ? flags[i] : (flags[i] & ~1u);
  }
}

// Scores of listed slots from their per-head maxima (query 0; the exact
// kernel filled them): the finalize kernel's law -- heads summed in order
// in fp64, / H, 0.0 for a slot without key tokens, NaN for a slot that is
// not live, holds a non-finite key value, or meets a non-finite query
// value -- one thread per listed slot, which then re-zeroes its maxima.
__global__ void gqa_slot_scores_kernel(unsigned long long* __restrict__ hmax, size_t cap, int H,
                                       const uint32_t* __restrict__ slots, uint64_t n,
                                       const uint32_t* __restrict__ lens,
                                       const uint32_t* __restrict__ flags,
                                       const unsigned* __restrict__ qbad, int kv,
                                       float* __restrict__ out) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  bool q_bad = false;
  for (int g = 0; g < kv; ++g) q_bad = q_bad || qbad[g] != 0u;
  const uint32_t slot = slots[i];
  double total = 0.0;
  for (int h = 0; h < H; ++h) {
    total += __longlong_as_double(hmax[static_cast<size_t>(h) * cap + slot]);
    hmax[static_cast<size_t>(h) * cap + slot] = 0ull;
  }
  const uint32_t f = flags[slot];
  float sc = __builtin_nanf("");
  if (f & 1u) {
    if (lens[slot] == 0) {
      sc = 0.0f;
    } else if ((f & 2u) && !q_bad) {
      sc = static_cast<float>(total / static_cast<double>(H));
    }
  }
  out[i] = sc;
}

}  // namespace gqa
}  // namespace grm
