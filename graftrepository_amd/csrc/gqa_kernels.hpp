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
// Two kernel families:
//  * exact  -- the law itself in fp64, one lane per key token, d in order;
//              per-(node, head) maxima combine with a 64-bit atomicMax on
//              the bit pattern (non-negative doubles order like their bits,
//              so the result does not depend on scheduling);
//  * screen -- |q.k| for every key token on the matrix cores (bf16 or fp16
//              MFMA 16x16x32, fp32 accumulate), reduced to a screened node
//              score with a rigorous error bound; a select/shortlist pass
//              keeps the nodes that can still reach the top-k and certifies
//              the shortlist; the exact family then rescores only those.
#pragma once

#include "grm_common.hpp"

#include <hip/hip_fp16.h>

namespace grm {
namespace gqa {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kUnitWaves = 4;     // wavefronts per exact/stats/screen block
constexpr int kFinWaves = 4;      // wavefronts per finalize/select block
constexpr int kMaxRQ = 32;        // R * Qt supported by the exact kernels
constexpr int kMaxShort = 64;     // shortlist capacity + 1 (one wave list)
constexpr uint32_t kMaxHeadDim = 512;

constexpr int kRowBatch = 8;      // 16-byte chunks of a key row loaded at once

// Work item: `count` consecutive key tokens, from t0, of one slot (all kv
// heads).  Token t of kv head g is key row base + g*len + t (rows of
// head_dim values).
struct Item {
  uint64_t base;  // tok_off[slot] * kv
  uint32_t slot;
  uint32_t t0;
  uint32_t count;
  uint32_t len;
};
static_assert(sizeof(Item) == 24, "Item layout");

__device__ inline float load_scale(const unsigned char* __restrict__ scales,
                                   int scale_dtype, uint64_t idx) {
  if (scale_dtype == kF16) {
    return __half2float(reinterpret_cast<const __half*>(scales)[idx]);
  }
  return reinterpret_cast<const float*>(scales)[idx];
}

// INT8 dequant law: fp16(float(code) * scale) (core/graft_quant.py:136-144).
__device__ inline _Float16 dequant_i8(int code, float scale) {
  return static_cast<_Float16>(static_cast<float>(code) * scale);
}

template <int KDT>
struct KeyTraits {
  static constexpr int kEsize = KDT == kF32 ? 4 : (KDT == kI8 ? 1 : 2);
  static constexpr int kEpc = 16 / kEsize;  // elements per 16-byte chunk
};

// Decode one 16-byte chunk of a key row into floats (law-level values).
template <int KDT>
__device__ inline void decode_chunk(u32x4 v, const unsigned char* __restrict__ scales,
                                    int scale_dtype, uint64_t scale_idx,
                                    float* out) {
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
    const float s = load_scale(scales, scale_dtype, scale_idx);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int code = static_cast<int>(static_cast<int8_t>((w[i] >> (8 * b)) & 0xffu));
        out[4 * i + b] = static_cast<float>(dequant_i8(code, s));
      }
    }
  }
}

// ----------------------------------------------------------------- exact

// Stage the R*Qt query rows of kv head g (rows >= R*Qt are zero) as doubles.
// Returns true when this lane saw a non-finite value.
__device__ inline bool stage_group_query(double* __restrict__ q, int RQ,
                                         const void* __restrict__ query,
                                         int q_dtype, int g, int R, int Qt,
                                         int hd, bool active, int lane,
                                         int nthreads) {
  bool bad = false;
  const int rq_used = R * Qt;
  for (int i = lane; i < RQ * hd; i += nthreads) {
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
  return bad;
}

// Exact maxima of one (slot, kv head g, token range): lane t walks tokens
// t0+lane, t0+lane+64, ...; for every query row the dot product runs in the
// law's d order in fp64.  Folds max|dot|/denom per query head r into
// target[(g*R + r) * tstride] (double bits, atomicMax).  row0 = key row of
// token 0 of (slot, g).  Row chunks load kRowBatch at a time.
template <int KDT, int RQ>
__device__ inline void exact_unit(const unsigned char* __restrict__ keys,
                                  const unsigned char* __restrict__ scales,
                                  int scale_dtype, int group_size,
                                  uint64_t row0, uint32_t t0, uint32_t count,
                                  const double* __restrict__ q, int g, int R,
                                  int Qt, int hd, double denom,
                                  unsigned long long* __restrict__ target,
                                  size_t tstride) {
  using T = KeyTraits<KDT>;
  const int lane = threadIdx.x & (kWave - 1);
  const int rq_used = R * Qt;
  const int nch = hd / T::kEpc;
  double best[RQ];
#pragma unroll
  for (int j = 0; j < RQ; ++j) best[j] = 0.0;
  const int groups = KDT == kI8 ? hd / group_size : 1;
  for (uint32_t t = t0 + lane; t < t0 + count; t += kWave) {
    double acc[RQ];
#pragma unroll
    for (int j = 0; j < RQ; ++j) acc[j] = 0.0;
    const uint64_t row = row0 + t;
    const u32x4* p = reinterpret_cast<const u32x4*>(keys + row * hd * T::kEsize);
    for (int c0 = 0; c0 < nch; c0 += kRowBatch) {
      u32x4 v[kRowBatch];
#pragma unroll
      for (int b = 0; b < kRowBatch; ++b) {
        if (c0 + b < nch) v[b] = p[c0 + b];
      }
#pragma unroll
      for (int b = 0; b < kRowBatch; ++b) {
        if (c0 + b >= nch) break;
        float f[T::kEpc];
        const int e0 = (c0 + b) * T::kEpc;
        decode_chunk<KDT>(v[b], scales, scale_dtype,
                          KDT == kI8 ? row * groups + e0 / group_size : 0, f);
#pragma unroll
        for (int e = 0; e < T::kEpc; ++e) {
          const double kd = static_cast<double>(f[e]);
#pragma unroll
          for (int j = 0; j < RQ; ++j) acc[j] = fma(kd, q[j * hd + e0 + e], acc[j]);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < RQ; ++j) {
      const double v = fabs(acc[j]);
      best[j] = (v > best[j] || isnan(v)) ? v : best[j];
    }
  }
  // Division by the positive constant sqrt(hd) is monotone under rounding to
  // nearest, so max(|dot|)/denom equals the law's max(|dot|/denom).
  for (int r = 0; r < R; ++r) {
    double m = 0.0;
#pragma unroll
    for (int j = 0; j < RQ; ++j) {
      if (j / Qt == r && j < rq_used) m = (best[j] > m || isnan(best[j])) ? best[j] : m;
    }
    unsigned long long bits = __double_as_longlong(m / denom);
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
      const unsigned long long o = __shfl_xor(bits, off);
      bits = o > bits ? o : bits;
    }
    if (lane == 0) atomicMax(target + static_cast<size_t>(g * R + r) * tstride, bits);
  }
}

// Exact maxima for every item; grid (ceil(items / 4), kv heads).  All
// waves of a block share kv head blockIdx.y and its staged query rows.
// hmax is head-major: hmax[h * cap + slot].
template <int KDT, int RQ>
__global__ __launch_bounds__(kUnitWaves * kWave) void gqa_exact_heads_kernel(
    const unsigned char* __restrict__ keys,
    const unsigned char* __restrict__ scales, int scale_dtype, int group_size,
    const Item* __restrict__ items, uint32_t n_items, int hd, int R, int Qt,
    const void* __restrict__ query, int q_dtype, double denom,
    unsigned long long* __restrict__ hmax, size_t cap,
    unsigned* __restrict__ qbad) {
  extern __shared__ double qs[];  // [RQ][hd]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int g = blockIdx.y;
  const uint32_t item_i = blockIdx.x * kUnitWaves + wave;
  const bool bad = stage_group_query(qs, RQ, query, q_dtype, g, R, Qt, hd,
                                     true, threadIdx.x, blockDim.x);
  if (__ballot(bad) != 0ull && lane == 0) atomicOr(qbad, 1u);
  __syncthreads();
  if (item_i >= n_items) return;
  const Item it = items[item_i];
  exact_unit<KDT, RQ>(keys, scales, scale_dtype, group_size,
                      it.base + static_cast<uint64_t>(g) * it.len, it.t0, it.count,
                      qs, g, R, Qt, hd, denom, hmax + it.slot, cap);
}

// Exact scores of every live slot from the head-major maxima (h in order,
// fp64); each block writes its k best entries (block_topk_write).
// Re-zeroes the maxima it read.
__global__ __launch_bounds__(kFinWaves * kWave) void gqa_finalize_kernel(
    unsigned long long* __restrict__ hmax, size_t cap, int H, uint32_t n_slots,
    const uint32_t* __restrict__ lens, const uint32_t* __restrict__ flags,
    const uint64_t* __restrict__ ids, const unsigned* __restrict__ qbad, int k,
    Cand* __restrict__ block_out) {
  constexpr int kHB = 16;  // head maxima loaded at once
  __shared__ Cand s_lists[kFinWaves][kMaxTopK];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const bool q_bad = *qbad != 0u;
  WaveList L;
  wl_init(L);
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t base = blockIdx.x * blockDim.x + wave * kWave; base < n_slots;
       base += stride) {
    const uint32_t slot = base + lane;
    const bool in = slot < n_slots;
    const uint32_t f = in ? flags[slot] : 0u;
    const uint32_t len = in ? lens[slot] : 0u;
    const bool scored = (f & 1u) && len > 0;
    double total = 0.0;
    for (int h0 = 0; h0 < H; h0 += kHB) {
      double v[kHB];
#pragma unroll
      for (int j = 0; j < kHB; ++j) {
        v[j] = (scored && h0 + j < H) ? __longlong_as_double(hmax[(h0 + j) * cap + slot]) : 0.0;
      }
#pragma unroll
      for (int j = 0; j < kHB; ++j) total += v[j];  // h ascending
#pragma unroll
      for (int j = 0; j < kHB; ++j) {
        if (scored && h0 + j < H) hmax[(h0 + j) * cap + slot] = 0ull;
      }
    }
    float s = __builtin_nanf("");
    if (f & 1u) {
      if (len == 0) {
        s = 0.0f;
      } else if ((f & 2u) && !q_bad) {  // all key and query values finite
        s = static_cast<float>(total / static_cast<double>(H));
      }
    }
    const bool need = isfinite(s) && s >= L.th_s;
    uint64_t id = kNoId;
    if (need) id = ids[slot];
    wl_consume(L, k, s, id, slot, need);
  }
  block_topk_write<kFinWaves>(L, k, s_lists, block_out);
}

// ---------------------------------------------------------------- screen

// MFMA operand type of a key storage type: bf16 keys run bf16 MFMA; fp16
// and int8 (dequantised to fp16 by the law) run fp16 MFMA.
template <int KDT>
struct ScreenTraits {
  static constexpr int kMfma = KDT == kBF16 ? kBF16 : kF16;
  static constexpr int kEsize = KDT == kI8 ? 1 : 2;
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

// Query preparation, one launch per batch of Qb queries:
//  blocks [0, kv): B fragments of the screen MFMAs.  Fragment (g, nt, ks)
//    lane l holds column c = l%16 of N-tile nt -- batch column
//    cg = nt*16 + c = (qb*R + r)*Qt + qi -- at dims
//    d = ks*32 + (l/16)*8 + j, j < 8, converted to the MFMA type with
//    round to nearest even; flags[qb] bit 0: non-finite value, bit 1:
//    value outside the fp16 range.
//  blocks [kv, kv+Qb): coef[qb], the screen error coefficient (see
//    gqa_select_kernel): ((g + d + g*d)*Qsum + s*(1+g)*sqrt(hd)) / sqrt(hd)
//    with g = gamma, d = delta, s = sigma and Qsum the mean over heads of
//    max over query tokens of ||q||_2, rounded up.
template <int MT>
__global__ __launch_bounds__(256) void gqa_query_prep_kernel(
    const void* __restrict__ query, int q_dtype, int Qb, int H, int Qt, int hd,
    int kv, int R, int NT, int KS, u32x4* __restrict__ bfrag,
    unsigned* __restrict__ qflags, float* __restrict__ coef, double gamma,
    double delta, double sigma) {
  auto qval = [&](uint64_t idx) -> float {
    return q_dtype == kBF16 ? bf16_to_f32(static_cast<const uint16_t*>(query)[idx])
                            : static_cast<const float*>(query)[idx];
  };
  if (blockIdx.x < static_cast<unsigned>(kv)) {
    const int g = blockIdx.x;
    const int cols = Qb * R * Qt;
    for (int idx = threadIdx.x; idx < NT * KS * kWave; idx += blockDim.x) {
      const int lane = idx % kWave;
      const int ks = (idx / kWave) % KS;
      const int nt = idx / (kWave * KS);
      const int cg = nt * 16 + (lane & 15);
      uint32_t w[4] = {0u, 0u, 0u, 0u};
      if (cg < cols) {
        const int qb = cg / (R * Qt);
        const int r = (cg % (R * Qt)) / Qt;
        const int qi = cg % Qt;
        const uint64_t base =
            ((static_cast<uint64_t>(qb) * H + g * R + r) * Qt + qi) * hd +
            ks * 32 + (lane >> 4) * 8;
        unsigned bad = 0u;
        for (int j = 0; j < 8; j += 2) {
          const float f0 = qval(base + j), f1 = qval(base + j + 1);
          if (!isfinite(f0) || !isfinite(f1)) bad |= 1u;
          uint32_t packed;
          if constexpr (MT == kBF16) {
            // round to nearest even; inputs are finite here or flagged
            auto rne = [](float f) {
              uint32_t u = __float_as_uint(f);
              return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
            };
            packed = rne(f0) | (rne(f1) << 16);
          } else {
            const _Float16 h0 = static_cast<_Float16>(f0);
            const _Float16 h1 = static_cast<_Float16>(f1);
            if (isfinite(f0) && !isfinite(static_cast<float>(h0))) bad |= 2u;
            if (isfinite(f1) && !isfinite(static_cast<float>(h1))) bad |= 2u;
            packed = pack_f16x2(h0, h1);
          }
          w[j / 2] = packed;
        }
        if (bad) atomicOr(qflags + qb, bad);
      }
      u32x4 v;
      v.x = w[0];
      v.y = w[1];
      v.z = w[2];
      v.w = w[3];
      bfrag[(static_cast<size_t>(g * NT + nt) * KS + ks) * kWave + lane] = v;
    }
    return;
  }
  // norms block for query qb: one wave per (head, query token) row, lanes
  // over d (order is free: the norm only bounds the screen error)
  __shared__ double s_row[kMaxRQ * 128];  // per (h, qi) row: ||q||_2
  __shared__ double s_sum[256];
  const int qb = blockIdx.x - kv;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int nw = blockDim.x / kWave;
  const int rows = H * Qt;
  double part = 0.0;
  const int chunk_rows = (kMaxRQ * 128 / Qt) * Qt;  // whole heads per chunk
  for (int r0 = 0; r0 < rows; r0 += chunk_rows) {
    const int nrow = min(rows - r0, chunk_rows);
    for (int r = wave; r < nrow; r += nw) {
      const uint64_t base = (static_cast<uint64_t>(qb) * rows + r0 + r) * hd;
      double acc = 0.0;
      for (int d = lane; d < hd; d += kWave) {
        const double v = static_cast<double>(qval(base + d));
        acc = fma(v, v, acc);
      }
#pragma unroll
      for (int off = 1; off < kWave; off <<= 1) acc += __shfl_xor(acc, off);
      if (lane == 0) s_row[r] = sqrt(acc);
    }
    __syncthreads();
    // max over query tokens of each head, summed over heads
    for (int hh = threadIdx.x; hh * Qt < nrow; hh += blockDim.x) {
      double mx = 0.0;
      for (int qi = 0; qi < Qt; ++qi) mx = fmax(mx, s_row[hh * Qt + qi]);
      part += mx;
    }
    __syncthreads();
  }
  s_sum[threadIdx.x] = part;
  __syncthreads();
  for (int off = blockDim.x / 2; off > 0; off >>= 1) {
    if (threadIdx.x < static_cast<unsigned>(off)) s_sum[threadIdx.x] += s_sum[threadIdx.x + off];
    __syncthreads();
  }
  if (threadIdx.x == 0) {
    const double qsum = s_sum[0] / H;
    const double sq = sqrt(static_cast<double>(hd));
    const double c = ((gamma + delta + gamma * delta) * qsum + sigma * (1.0 + gamma) * sq) / sq;
    coef[qb] = static_cast<float>(c * (1.0 + 1e-6));
  }
}

// Screen: |q.k| on the matrix cores for every key token, for all batch
// columns at once; grid (blocks, kv).  Each wavefront walks the items
// w, w+W, ... of kv head blockIdx.y as one stream of 16-token steps with
// the next step's loads in flight while the current one is folded.  The
// per-(query, node, head) maxima land in head-major hms
// [qb][h][slot] (fp32 bits, atomicMax; non-negative floats order like their
// bits).  K-step ks of lane l covers dims ks*32 + (l/16)*8 .. +8 of key
// token l%16 (matching the B fragments), so one load instruction reads 64
// contiguous bytes of each of 16 key rows.  Tokens past an item read as
// zero, and |0| never raises a maximum.
template <int KDT, int KS, int NT>
__global__ __launch_bounds__(kUnitWaves * kWave) void gqa_screen_kernel(
    const unsigned char* __restrict__ keys,
    const unsigned char* __restrict__ scales, int scale_dtype, int group_size,
    const Item* __restrict__ items, uint32_t n_items, int R, int Qt, int cols,
    const u32x4* __restrict__ bfrag, unsigned* __restrict__ hms,
    size_t hms_qstride, size_t cap) {
  using ST = ScreenTraits<KDT>;
  constexpr int HD = 32 * KS;
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t W = gridDim.x * kUnitWaves;
  uint32_t i_cur = blockIdx.x * kUnitWaves + threadIdx.x / kWave;
  if (i_cur >= n_items) return;
  const int g = blockIdx.y;
  u32x4 bq[NT][KS];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bq[nt][ks] = bfrag[(static_cast<size_t>(g * NT + nt) * KS + ks) * kWave + lane];
    }
  }
  const int quarter = lane >> 4;
  const int r16 = lane & 15;
  const int groups = KDT == kI8 ? HD / group_size : 1;
  const u32x4 zero = {0u, 0u, 0u, 0u};

  auto load_step = [&](u32x4 (&a)[KS], const Item& it, uint32_t s) {
    const uint32_t tl = s * 16 + r16;
    const bool ok = tl < it.count;
    const uint64_t row = it.base + static_cast<uint64_t>(g) * it.len + it.t0 + tl;
    if constexpr (KDT != kI8) {
      const u32x4* p = reinterpret_cast<const u32x4*>(keys + (row * HD + quarter * 8) * ST::kEsize);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) a[ks] = ok ? p[ks * 4] : zero;  // +64 bytes per K-step
    } else {
      typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
      const u32x2* p = reinterpret_cast<const u32x2*>(keys + row * HD + quarter * 8);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x2 v = ok ? p[ks * 4] : u32x2{0u, 0u};  // +32 bytes per K-step
        const float sc = ok ? load_scale(scales, scale_dtype,
                                         row * groups + (ks * 32 + quarter * 8) / group_size)
                            : 0.0f;
        const uint32_t w[2] = {v.x, v.y};
        uint32_t o[4];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          o[2 * i] = pack_f16x2(dequant_i8(static_cast<int8_t>(w[i] & 0xffu), sc),
                                dequant_i8(static_cast<int8_t>((w[i] >> 8) & 0xffu), sc));
          o[2 * i + 1] = pack_f16x2(dequant_i8(static_cast<int8_t>((w[i] >> 16) & 0xffu), sc),
                                    dequant_i8(static_cast<int8_t>(w[i] >> 24), sc));
        }
        a[ks].x = o[0];
        a[ks].y = o[1];
        a[ks].z = o[2];
        a[ks].w = o[3];
      }
    }
  };
  float m[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) m[nt] = 0.0f;
  auto fold = [&](const u32x4 (&a)[KS]) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      f32x4 c = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) c = mfma16x16x32<ST::kMfma>(a[ks], bq[nt][ks], c);
      m[nt] = fmaxf(m[nt], fmaxf(fmaxf(fabsf(c.x), fabsf(c.y)), fmaxf(fabsf(c.z), fabsf(c.w))));
    }
  };
  auto emit = [&](const Item& it) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      float v = fmaxf(m[nt], __shfl_xor(m[nt], 16));
      v = fmaxf(v, __shfl_xor(v, 32));
      const int cg = nt * 16 + lane;
      if (lane < 16 && cg < cols) {
        const int qb = cg / (R * Qt);
        const int r = (cg % (R * Qt)) / Qt;
        atomicMax(hms + qb * hms_qstride + static_cast<size_t>(g * R + r) * cap + it.slot,
                  __float_as_uint(v));
      }
      m[nt] = 0.0f;
    }
  };

  Item cur = items[i_cur];
  uint32_t i_nxt = i_cur + W;
  Item nxt = items[i_nxt < n_items ? i_nxt : i_cur];
  uint32_t s = 0;
  uint32_t nsteps = (cur.count + 15) / 16;
  u32x4 a0[KS], a1[KS];
  load_step(a0, cur, 0);
  // One step: fold `now` while the following step loads into `later`.
  // Returns false when the wave's stream is exhausted.
  auto step = [&](u32x4 (&now)[KS], u32x4 (&later)[KS]) -> bool {
    const bool last_of_item = s + 1 == nsteps;
    if (!last_of_item) {
      load_step(later, cur, s + 1);
    } else if (i_nxt < n_items) {
      load_step(later, nxt, 0);
    }
    fold(now);
    if (!last_of_item) {
      ++s;
      return true;
    }
    emit(cur);
    if (i_nxt >= n_items) return false;
    i_cur = i_nxt;
    cur = nxt;
    i_nxt = i_cur + W;
    nxt = items[i_nxt < n_items ? i_nxt : i_cur];
    s = 0;
    nsteps = (cur.count + 15) / 16;
    return true;
  };
  while (step(a0, a1) && step(a1, a0)) {
  }
}

// Select: per (query, live slot) the screened score S~ = sum_h m_h /
// (H sqrt(hd)) and its bound B = coef*kmax + slack*|S~| (|S~ - S| <= B for
// the law's score S); keeps the best mU slots by U = S~ + B and the best k
// by Lo = S~ - B (ties to the lower node id).  grid (blocks, Qb).  Reads the
// head-major maxima coalesced and re-zeroes them.
__global__ __launch_bounds__(kFinWaves * kWave) void gqa_select_kernel(
    unsigned* __restrict__ hms, size_t hms_qstride, size_t cap, int H,
    uint32_t n_slots, const uint32_t* __restrict__ lens,
    const uint32_t* __restrict__ flags, const uint64_t* __restrict__ ids,
    const float* __restrict__ kmax, const float* __restrict__ coef,
    float inv_scale, float slack_rel, int mU, int k, Cand* __restrict__ bu,
    Cand* __restrict__ bl) {
  constexpr int kHB = 32;  // head maxima loaded at once
  __shared__ Cand s_u[kFinWaves][kMaxShort];
  __shared__ Cand s_l[kFinWaves][kMaxTopK];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int qb = blockIdx.y;
  const float cq = coef[qb];
  unsigned* hq = hms + qb * hms_qstride;
  WaveList WU, WL;
  wl_init(WU);
  wl_init(WL);
  const uint32_t stride = gridDim.x * blockDim.x;
  for (uint32_t base = blockIdx.x * blockDim.x + wave * kWave; base < n_slots;
       base += stride) {
    const uint32_t slot = base + lane;
    const bool in = slot < n_slots;
    const uint32_t f = in ? flags[slot] : 0u;
    const uint32_t len = in ? lens[slot] : 0u;
    const bool scored = (f & 1u) && len > 0;
    float sum = 0.0f;
    for (int h0 = 0; h0 < H; h0 += kHB) {
      float v[kHB];
#pragma unroll
      for (int j = 0; j < kHB; ++j) {
        v[j] = (scored && h0 + j < H) ? __uint_as_float(hq[(h0 + j) * cap + slot]) : 0.0f;
      }
#pragma unroll
      for (int j = 0; j < kHB; ++j) sum += v[j];
#pragma unroll
      for (int j = 0; j < kHB; ++j) {
        if (scored && h0 + j < H) hq[(h0 + j) * cap + slot] = 0u;
      }
    }
    bool valid = false;
    float u = 0.0f, lo = 0.0f;
    if (f & 1u) {
      if (len == 0) {
        valid = true;  // exact score 0.0
      } else if (f & 2u) {
        valid = true;
        const float sc = sum * inv_scale;
        const float b = cq * kmax[slot] + slack_rel * fabsf(sc);
        u = sc + b;
        lo = sc - b;
        if (!isfinite(u) || !isfinite(lo)) {
          u = 3.0e38f;  // unbounded screen value: always shortlisted
          lo = -3.0e38f;
        }
      }
    }
    const uint64_t id = valid ? ids[slot] : kNoId;
    wl_consume(WU, mU, u, id, slot, valid);
    wl_consume(WL, k, lo, id, slot, valid);
  }
  Cand* bu_q = bu + (static_cast<size_t>(qb) * gridDim.x) * mU;
  Cand* bl_q = bl + (static_cast<size_t>(qb) * gridDim.x) * k;
  block_topk_write<kFinWaves>(WU, mU, s_u, bu_q);
  __syncthreads();
  block_topk_write<kFinWaves>(WL, k, s_l, bl_q);
}

// Shortlist: merge the select blocks of query blockIdx.x; shortlist the best
// M slots by U and certify: every node outside it has U <= U_(M+1), every
// node's law score lies in [Lo, U], so if U_(M+1) < Lo_(k) (k-th best Lo)
// the law's top-k lies inside the shortlist.  Writes status[q] = 1 when
// certified and copies the query's prep flags to out_flags[q] (both host
// mapped).
__global__ __launch_bounds__(kFinWaves * kWave) void gqa_shortlist_kernel(
    const Cand* __restrict__ bu, const Cand* __restrict__ bl, uint32_t nblk,
    int mU, int k, int M, uint32_t* __restrict__ shortlist,
    const unsigned* __restrict__ qflags, unsigned* __restrict__ out_flags,
    unsigned* __restrict__ status) {
  __shared__ Cand s_u[kFinWaves][kMaxShort];
  __shared__ Cand s_l[kFinWaves][kMaxTopK];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int qb = blockIdx.x;
  WaveList WU, WL;
  wl_init(WU);
  wl_init(WL);
  wl_consume_global(WU, mU, bu + static_cast<size_t>(qb) * nblk * mU, nblk * mU,
                    static_cast<uint32_t>(wave), kFinWaves);
  wl_consume_global(WL, k, bl + static_cast<size_t>(qb) * nblk * k, nblk * k,
                    static_cast<uint32_t>(wave), kFinWaves);
  if (lane < kMaxShort) s_u[wave][lane] = wl_entry(WU);
  if (lane < kMaxTopK) s_l[wave][lane] = wl_entry(WL);
  __syncthreads();
  if (wave == 0) {
    WaveList BU, BL;
    block_merge<kFinWaves>(s_u, mU, BU);
    block_merge<kFinWaves>(s_l, k, BL);
    const bool filled = lane < mU && BU.id != kNoId;
    const int count = __popcll(__ballot(filled));
    const float u_next = __shfl(BU.s, M);
    const float tau = __shfl(BL.s, k - 1);  // -inf when fewer than k nodes
    if (lane < M) shortlist[static_cast<size_t>(qb) * M + lane] = lane < count ? BU.slot : kNoSlot;
    if (lane == 0) {
      status[qb] = (count <= M || u_next < tau) ? 1u : 0u;
      out_flags[qb] = qflags[qb];
    }
  }
}

// Exact rescore of the shortlisted slots; grid (ceil(units / 4), kv) with
// units = Qb * M * max_chunks (64-token chunks).  hex[h * QM + (qb*M + m)]
// (QM = Qb*M) receives the exact maxima (double bits, atomicMax).
template <int KDT, int RQ>
__global__ __launch_bounds__(kUnitWaves * kWave) void gqa_rescore_kernel(
    const unsigned char* __restrict__ keys,
    const unsigned char* __restrict__ scales, int scale_dtype, int group_size,
    const uint64_t* __restrict__ tok_off, const uint32_t* __restrict__ lens,
    const uint32_t* __restrict__ shortlist, int M, int Qb, uint32_t max_chunks,
    int kv, int hd, int R, int Qt, const void* __restrict__ query, int q_dtype,
    size_t q_stride, double denom, unsigned long long* __restrict__ hex) {
  extern __shared__ double qs[];  // [kUnitWaves][RQ][hd]
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int g = blockIdx.y;
  const uint64_t unit = static_cast<uint64_t>(blockIdx.x) * kUnitWaves + wave;
  const uint64_t units = static_cast<uint64_t>(Qb) * M * max_chunks;
  const bool in_range = unit < units;
  const uint32_t qm = in_range ? static_cast<uint32_t>(unit / max_chunks) : 0;
  const uint32_t chunk = in_range ? static_cast<uint32_t>(unit % max_chunks) : 0;
  const int qb = static_cast<int>(qm / M);
  const uint32_t slot = in_range ? shortlist[qm] : kNoSlot;
  const uint32_t L = slot != kNoSlot ? lens[slot] : 0u;
  const uint32_t t0 = chunk * kWave;
  const bool active = slot != kNoSlot && t0 < L;
  double* q = qs + static_cast<size_t>(wave) * RQ * hd;
  const unsigned char* qptr = static_cast<const unsigned char*>(query) +
                              static_cast<size_t>(qb) * q_stride * (q_dtype == kBF16 ? 2 : 4);
  stage_group_query(q, RQ, qptr, q_dtype, g, R, Qt, hd, active, lane, kWave);
  __syncthreads();
  if (!active) return;
  exact_unit<KDT, RQ>(keys, scales, scale_dtype, group_size,
                      tok_off[slot] * kv + static_cast<uint64_t>(g) * L, t0,
                      min(static_cast<uint32_t>(kWave), L - t0), q, g, R, Qt, hd,
                      denom, hex + qm, static_cast<size_t>(Qb) * M);
}

// Exact scores of the shortlist entries into out[qb*M + m] (host mapped),
// h in order in fp64, re-zeroing the maxima.  One thread per entry.
__global__ void gqa_rescore_finalize_kernel(
    unsigned long long* __restrict__ hex, int H,
    const uint32_t* __restrict__ shortlist, uint32_t total,
    const uint32_t* __restrict__ lens, const uint64_t* __restrict__ ids,
    Cand* __restrict__ out) {
  constexpr int kHB = 16;
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= total) return;
  const uint32_t slot = shortlist[i];
  double sum = 0.0;
  for (int h0 = 0; h0 < H; h0 += kHB) {
    double v[kHB];
#pragma unroll
    for (int j = 0; j < kHB; ++j) {
      v[j] = h0 + j < H ? __longlong_as_double(hex[static_cast<size_t>(h0 + j) * total + i]) : 0.0;
    }
#pragma unroll
    for (int j = 0; j < kHB; ++j) sum += v[j];  // h ascending
#pragma unroll
    for (int j = 0; j < kHB; ++j) {
      if (h0 + j < H) hex[static_cast<size_t>(h0 + j) * total + i] = 0ull;
    }
  }
  Cand c;
  c.score = __builtin_nanf("");
  c.slot = kNoSlot;
  c.id = kNoId;
  if (slot != kNoSlot) {
    c.score = lens[slot] == 0 ? 0.0f : static_cast<float>(sum / static_cast<double>(H));
    c.slot = slot;
    c.id = ids[slot];
  }
  out[i] = c;
}

// ----------------------------------------------------------- bank upkeep

// Key statistics of new slots: nonfinite[slot] set when a decoded value is
// not finite; kmax[slot] = max over kv heads and tokens of ||k||_2, rounded
// up (float bits, atomicMax).  grid (ceil(items / 4), kv).
template <int KDT>
__global__ __launch_bounds__(kUnitWaves * kWave) void gqa_key_stats_kernel(
    const unsigned char* __restrict__ keys,
    const unsigned char* __restrict__ scales, int scale_dtype, int group_size,
    const Item* __restrict__ items, uint32_t n_items, int hd,
    uint32_t* __restrict__ nonfinite, unsigned* __restrict__ kmax) {
  using T = KeyTraits<KDT>;
  const int lane = threadIdx.x & (kWave - 1);
  const uint32_t item_i = blockIdx.x * kUnitWaves + threadIdx.x / kWave;
  if (item_i >= n_items) return;
  const int g = blockIdx.y;
  const Item it = items[item_i];
  const int groups = KDT == kI8 ? hd / group_size : 1;
  bool bad = false;
  double mx = 0.0;
  for (uint32_t t = it.t0 + lane; t < it.t0 + it.count; t += kWave) {
    const uint64_t row = it.base + static_cast<uint64_t>(g) * it.len + t;
    const u32x4* p = reinterpret_cast<const u32x4*>(keys + row * hd * T::kEsize);
    double acc = 0.0;
    for (int c = 0; c < hd / T::kEpc; ++c) {
      float f[T::kEpc];
      const int e0 = c * T::kEpc;
      decode_chunk<KDT>(p[c], scales, scale_dtype,
                        KDT == kI8 ? row * groups + e0 / group_size : 0, f);
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

}  // namespace gqa
}  // namespace grm
