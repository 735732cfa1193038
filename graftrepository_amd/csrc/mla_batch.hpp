// mla_batch.hpp -- batched MLA route on the matrix cores (included by
// mla_route.hip only).
//
// Q queries against a bf16 bank, law as the single-query route
// (cpp/grm_runtime.cpp:3518-3545):
//   score = float( dot / (qnorm * (double)norm_f + 1e-8) ),  dot in fp64, d ascending.
// The scores of all Q x N pairs form a dense contraction.  It runs as bf16
// MFMA 32x32x16 with fp32 accumulation, reduced on the fly: the score
// matrix never leaves registers.
//
//  * screen  -- every node tile (32 slots) against every query of a pass
//               (up to 256, staged in LDS).  The screened score
//               s~ = acc * (1/norm_f) * (1/qnorm) obeys |s~ - score| <= B,
//               B a per-query constant (see mla_batch_merge_kernel).
//               Each lane follows one query over half of every tile its
//               wavefront walks -- a sub-stream -- and keeps the two best
//               (s~, slot) and the largest s~ it did not keep.
//  * merge   -- one block per query: the kept entries of all sub-streams,
//               their top-32 by s~, and the certificate: with t = (k-th
//               best s~) - 2B, if every sub-stream's largest dropped s~ and
//               the 32nd kept s~ lie below t, the law's top-k is among the
//               kept entries at or above t (any other node's score is below
//               the k-th best's).  Those are scored with the law in fp64
//               and ranked (score desc, node id asc).  A query without a
//               certificate is routed again on the exact single-query path.
#pragma once

#include "grm_common.hpp"

namespace grm {
namespace mla {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBatchWaves = 8;       // wavefronts per screen block (one block per CU)
constexpr int kBatchMaxCols = 256;   // queries per screen pass
constexpr int kBatchKeep = 32;       // entries the merge ranks by s~

// Per (wavefront, query, lane half) result of the screen.
struct BatchEntry {
  float s1, s2, nk;  // two best s~ kept, largest s~ not kept
  uint32_t i1, i2;   // their slots
};
static_assert(sizeof(BatchEntry) == 20, "BatchEntry layout");

// Screen; grid = one block of kBatchWaves wavefronts per CU, LDS holds the
// pass's queries: qpad[QP][stride] bf16 (row d of query j at j*stride + d,
// stride = dim_pad + 8 so the 16-byte reads of 32 rows hit distinct
// banks).  Wavefront w walks 32-slot tiles [w*T/W, (w+1)*T/W).  For K-step
// ks the A fragment of lane l is chunk 2*ks + l/32 (8 values) of slot
// tile*32 + l%32 -- two 512-byte runs per load -- and the B fragment is
// query ct*32 + l%32 at dims 16*ks + 8*(l/32) .. +8; result register r of
// lane l is slot tile*32 + 8*(r/4) + 4*(l/32) + r%4 against that query.
template <int KS, int CT>
__global__ __launch_bounds__(kBatchWaves * kWave) void mla_batch_screen_kernel(
    const u32x4* __restrict__ tiles, const float* __restrict__ norms, uint64_t cap,
    uint32_t chunks, uint32_t n_tiles32, const uint16_t* __restrict__ qpad, int stride,
    const float* __restrict__ inv_qn, BatchEntry* __restrict__ out) {
  constexpr int QP = 32 * CT;
  extern __shared__ uint16_t s_qb[];  // [QP][stride]
  {
    const u32x4* src = reinterpret_cast<const u32x4*>(qpad);
    u32x4* dst = reinterpret_cast<u32x4*>(s_qb);
    const int n16 = QP * stride / 8;
    for (int i = threadIdx.x; i < n16; i += blockDim.x) dst[i] = src[i];
  }
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int half = lane >> 5;
  const int col = lane & 31;
  const uint32_t W = gridDim.x * kBatchWaves;
  const uint32_t w = blockIdx.x * kBatchWaves + __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const uint32_t t_begin = static_cast<uint32_t>(static_cast<uint64_t>(w) * n_tiles32 / W);
  const uint32_t t_end = static_cast<uint32_t>(static_cast<uint64_t>(w + 1) * n_tiles32 / W);
  float iq[CT], b1[CT], b2[CT], nk[CT];
  uint32_t i1[CT], i2[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    iq[ct] = inv_qn[ct * 32 + col];
    b1[ct] = b2[ct] = nk[ct] = -INFINITY;
    i1[ct] = i2[ct] = 0u;
  }
  const u32x4 zero = {0u, 0u, 0u, 0u};
  auto load_a = [&](u32x4 (&a)[KS], uint32_t t) {
    const uint64_t slot = static_cast<uint64_t>(t) * 32 + col;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const uint32_t c = 2 * ks + half;
      a[ks] = c < chunks ? __builtin_nontemporal_load(tiles + c * cap + slot) : zero;
    }
  };
  const uint16_t* qrow = s_qb + col * stride + 8 * half;
  auto fold = [&](const u32x4 (&a)[KS], uint32_t t) {
    // inverse row norms of the lane's 16 result rows: NaN for a tombstone
    // (never kept), 0 for an all-zero row (score 0, exact)
    float wr[16];
    const uint32_t sbase = t * 32 + 4 * half;  // slot of result register r: sbase + 8*(r/4) + r%4
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float nf = norms[sbase + 8 * (r / 4) + (r % 4)];
      wr[r] = nf == 0.0f ? 0.0f : __builtin_amdgcn_rcpf(nf);
    }
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const u32x4 b = *reinterpret_cast<const u32x4*>(qrow + ct * 32 * stride + 16 * ks);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[ks]),
                                                      __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float v = acc[r] * wr[r] * iq[ct];  // NaN compares false: never kept
        const uint32_t slot = sbase + 8 * (r / 4) + (r % 4);
        const bool gt1 = v > b1[ct];
        const bool gt2 = v > b2[ct];
        nk[ct] = fmaxf(nk[ct], gt2 ? b2[ct] : v);
        const float nb2 = gt1 ? b1[ct] : v;
        const uint32_t ni2 = gt1 ? i1[ct] : slot;
        b2[ct] = gt2 ? nb2 : b2[ct];
        i2[ct] = gt2 ? ni2 : i2[ct];
        b1[ct] = gt1 ? v : b1[ct];
        i1[ct] = gt1 ? slot : i1[ct];
      }
      // column tiles one after another: their accumulators and fragments
      // are never live together
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // One tile buffer per wavefront (the two wavefronts of a SIMD take turns
  // waiting for their tiles and running the matrix cores).
  for (uint32_t t = t_begin; t < t_end; ++t) {
    u32x4 a[KS];
    load_a(a, t);
    fold(a, t);
  }
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    BatchEntry e;
    e.s1 = b1[ct];
    e.s2 = b2[ct];
    e.nk = nk[ct];
    e.i1 = i1[ct];
    e.i2 = i2[ct];
    out[(static_cast<size_t>(w) * QP + ct * 32 + col) * 2 + half] = e;
  }
}

// Query rows of one pass for the screen: qpad[j][0, stride) = query j's
// values rounded to bf16 (nearest even; bf16 queries are copied), zero past
// dim; inv_qn[j] = 1 / ||q_j|| rounded to fp32.  Rows j >= qc are zero with
// inv_qn NaN (nothing is kept for them).  grid = QP blocks.
__global__ __launch_bounds__(kWave) void mla_batch_qprep_kernel(
    const void* __restrict__ query, int q_dtype, int qc, uint32_t dim, int stride,
    uint16_t* __restrict__ qpad, float* __restrict__ inv_qn) {
  const int j = blockIdx.x;
  const int lane = threadIdx.x;
  double ss = 0.0;
  for (int d = lane; d < stride; d += kWave) {
    uint16_t bits = 0;
    if (j < qc && static_cast<uint32_t>(d) < dim) {
      const size_t idx = static_cast<size_t>(j) * dim + d;
      float f;
      if (q_dtype == kBF16) {
        bits = static_cast<const uint16_t*>(query)[idx];
        f = bf16_to_f32(bits);
      } else {
        f = static_cast<const float*>(query)[idx];
        const uint32_t u = __float_as_uint(f);
        bits = static_cast<uint16_t>((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
      }
      ss = fma(static_cast<double>(f), static_cast<double>(f), ss);
    }
    qpad[static_cast<size_t>(j) * stride + d] = bits;
  }
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) ss += __shfl_xor(ss, off);
  if (lane == 0) inv_qn[j] = j < qc ? static_cast<float>(1.0 / sqrt(ss)) : __builtin_nanf("");
}

// Merge, certificate and exact rescore; grid = one block of kMergeWavesB
// wavefronts per query of the pass.  entries: [W][QP][2] from the screen;
// query qi (pass column) has its `dim` values at query + qi*qstride
// elements (F32 or BF16).  The screen bound for the query (|s~ - score|):
//   B = (gamma + delta) * (1 + 2^-20) + 8 * 2^-24
//       + 1.01e-8 / (qn * nmin) + sqrt(dim) * 2^-125 * (1/qn + 1/nmin)
//       + dim * 2^-125 / (qn * nmin),
// gamma bounding the fp32 accumulation, delta the rounding of an fp32
// query to bf16, 8 * 2^-24 the reciprocals and products of the screened
// score and the score's own rounding, the 1e-8 term the law's
// denominator, the last terms bf16 values or products flushed near zero;
// qn is the law's query norm and nmin the smallest positive row norm.
// Writes out[qi*k ..) (the law's top-k, host mapped) and status[qi] = 1
// when certified (0: route qi again on the exact path).
constexpr int kMergeWavesB = 4;

__global__ __launch_bounds__(kMergeWavesB * kWave) void mla_batch_merge_kernel(
    const BatchEntry* __restrict__ entries, uint32_t W, int QP, const u32x4* __restrict__ tiles,
    const float* __restrict__ norms, const uint64_t* __restrict__ ids, uint64_t cap,
    uint32_t dim, const void* __restrict__ query, int q_dtype, size_t qstride, double gamma,
    double delta, const unsigned* __restrict__ min_norm, int k, Cand* __restrict__ out,
    unsigned* __restrict__ status) {
  __shared__ Cand s_lists[kMergeWavesB][kBatchKeep];
  __shared__ float s_nk[kMergeWavesB];
  __shared__ double s_qn;
  __shared__ int s_ok;
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
  const int qi = blockIdx.x;
  const unsigned char* qbase = static_cast<const unsigned char*>(query) +
                               static_cast<size_t>(qi) * qstride * (q_dtype == kBF16 ? 2 : 4);
  auto qval = [&](uint32_t d) -> double {
    return q_dtype == kBF16
               ? static_cast<double>(bf16_to_f32(reinterpret_cast<const uint16_t*>(qbase)[d]))
               : static_cast<double>(reinterpret_cast<const float*>(qbase)[d]);
  };
  if (threadIdx.x == 0) {  // the law's query norm, d ascending
    double acc = 0.0;
    for (uint32_t d = 0; d < dim; ++d) {
      const double v = qval(d);
      acc = fma(v, v, acc);
    }
    s_qn = sqrt(acc);
  }
  // kept entries by s~ and the largest dropped s~
  WaveList L;
  wl_init(L);
  float nk = -INFINITY;
  const uint32_t n_sub = W * 2;
  for (uint32_t base = wave * kWave; base < n_sub; base += kMergeWavesB * kWave) {
    const uint32_t i = base + lane;
    BatchEntry e;
    e.s1 = e.s2 = e.nk = -INFINITY;
    e.i1 = e.i2 = 0u;
    if (i < n_sub) e = entries[(static_cast<size_t>(i / 2) * QP + qi) * 2 + (i & 1)];
    nk = fmaxf(nk, e.nk);
    wl_consume(L, kBatchKeep, e.s1, e.i1, e.i1, i < n_sub && isfinite(e.s1));
    wl_consume(L, kBatchKeep, e.s2, e.i2, e.i2, i < n_sub && isfinite(e.s2));
  }
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) nk = fmaxf(nk, __shfl_xor(nk, off));
  if (lane < kBatchKeep) s_lists[wave][lane] = wl_entry(L);
  if (lane == 0) s_nk[wave] = nk;
  __syncthreads();
  if (wave == 0) {
    WaveList B;
    block_merge<kMergeWavesB>(s_lists, kBatchKeep, B);
    float nk_all = -INFINITY;
    for (int j = 0; j < kMergeWavesB; ++j) nk_all = fmaxf(nk_all, s_nk[j]);
    const bool filled = B.id != kNoId && isfinite(B.s);
    const int count = __popcll(__ballot(lane < kBatchKeep && filled));
    const float sk = __shfl(B.s, k - 1);
    const float s_last = __shfl(B.s, kBatchKeep - 1);
    const double qn = s_qn;
    const double nmin = static_cast<double>(__uint_as_float(*min_norm));
    const double sd = sqrt(static_cast<double>(dim));
    const double bound = (gamma + delta) * (1.0 + 0x1p-20) + 8.0 * 0x1p-24 + 1.01e-8 / (qn * nmin) +
                         sd * 0x1p-125 * (1.0 / qn + 1.0 / nmin) + dim * 0x1p-125 / (qn * nmin);
    const double t = static_cast<double>(sk) - 2.0 * bound;
    const bool ok = count >= k && static_cast<double>(nk_all) < t &&
                    (count < kBatchKeep || static_cast<double>(s_last) < t);
    // exact law score of every kept entry at or above t
    Cand c;
    c.score = __builtin_nanf("");
    c.slot = kNoSlot;
    c.id = kNoId;
    const bool mine = ok && lane < count && static_cast<double>(B.s) >= t;
    if (mine) {
      const uint64_t slot = B.slot;
      double dot = 0.0;
      uint32_t d = 0;
      const uint32_t chunks = (dim + 7) / 8;
      for (uint32_t ch = 0; ch < chunks; ++ch) {
        const u32x4 v = tiles[ch * cap + slot];
        const uint32_t wv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          if (d < dim) {
            const float f = bf16_to_f32((wv[e / 2] >> (16 * (e & 1))) & 0xffffu);
            dot = fma(static_cast<double>(f), qval(d), dot);
          }
          ++d;
        }
      }
      const float sc = static_cast<float>(dot / (s_qn * static_cast<double>(norms[slot]) + 1e-8));
      if (isfinite(sc)) {
        c.score = sc;
        c.slot = static_cast<uint32_t>(slot);
        c.id = ids[slot];
      }
    }
    WaveList F;
    wl_init(F);
    wl_consume(F, k, c.score, c.id, c.slot, isfinite(c.score));
    if (lane < k) out[static_cast<size_t>(qi) * k + lane] = wl_entry(F);
    if (lane == 0) s_ok = ok ? 1 : 0;
  }
  __syncthreads();
  if (threadIdx.x == 0) status[qi] = static_cast<unsigned>(s_ok);
}

}  // namespace mla
}  // namespace grm
