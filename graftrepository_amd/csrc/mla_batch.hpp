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
//               wavefront walks and keeps the two best (s~, slot) and the
//               largest s~ it did not keep; the two halves of a query are
//               merged at the end, one sub-stream per (wavefront, query).
//  * merge   -- one block per query over the sub-streams' kept entries:
//               v_k = the k-th best kept s~, t = v_k - 2B.  A node whose
//               s~ lies below t scores below v_k - B, so if every
//               sub-stream's largest dropped s~ lies below t, the law's
//               top-k is among the kept entries at or above t.  Those are
//               scored with the law in fp64 and ranked (score desc, node id
//               asc); the k-th exact score must reach v_k - B (which fails
//               only where a law score is not finite).  A query without
//               this certificate is routed again on the exact single-query
//               path.
#pragma once

#include "grm_common.hpp"

namespace grm {
namespace mla {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kBatchWaves = 8;       // wavefronts per screen block (one block per CU)
constexpr int kBatchMaxCols = 256;   // queries per screen pass
constexpr int kEntryPlanes = 5;      // s1, s2, nk, i1, i2

// Screen results, one row of n_sub values per (plane, query): plane p of
// query q at planes + (p*QP + q)*n_sub, sub-stream i = the wavefront:
//   s1, s2  the two best s~ a sub-stream kept (float bits), i1, i2 their
//   slots, nk the largest s~ it did not keep.
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
    const float* __restrict__ inv_qn, uint32_t* __restrict__ planes) {
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
  // Lanes track u = acc * (1/norm_f); s~ = u * (1/qnorm) is formed at the
  // end (rounding is monotone, so the two best and the largest dropped u
  // give the two best and the largest dropped s~).
  // Per (lane, column tile): the two best u = acc * (1/norm_f) with their
  // slots and the largest u not kept.
  auto update = [&](float accv, float w, int ct, uint32_t slot) {
    const float v = accv * w;  // NaN compares false: never kept
    const bool gt1 = v > b1[ct];
    const bool gt2 = v > b2[ct];
    nk[ct] = fmaxf(nk[ct], gt2 ? b2[ct] : v);
    const float nb2 = gt1 ? b1[ct] : v;
    const uint32_t ni2 = gt1 ? i1[ct] : slot;
    b2[ct] = gt2 ? nb2 : b2[ct];
    i2[ct] = gt2 ? ni2 : i2[ct];
    b1[ct] = gt1 ? v : b1[ct];
    i1[ct] = gt1 ? slot : i1[ct];
  };
  // Column tile ct's matrix-core chain runs while the vector units reduce
  // column tile ct-1: after step ks of the chain come the updates of result
  // registers [ks*kUp, ks*kUp + kUp) of the previous accumulator, in that
  // order (a scheduling barrier per step), so the matrix cores and the
  // vector units work at once.  Query fragments are read kPre steps ahead.
  constexpr int kPre = 4;
  constexpr int kUp = (16 + KS - 1) / KS;  // updates per chain step
  auto fold = [&](const u32x4 (&a)[KS], const float (&wr)[16], uint32_t t) {
    const uint32_t sbase = t * 32 + 4 * half;  // slot of result register r: sbase + 8*(r/4) + r%4
    f32x16 prev;
#pragma unroll
    for (int ct = 0; ct <= CT; ++ct) {
      f32x16 acc;
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
      u32x4 bw[kPre];
      const uint16_t* qc = qrow + (ct < CT ? ct : 0) * 32 * stride;
      if (ct < CT) {
#pragma unroll
        for (int j = 0; j < kPre; ++j) bw[j] = *reinterpret_cast<const u32x4*>(qc + 16 * j);
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        if (ct < CT) {
          const u32x4 b = bw[ks % kPre];
          if (ks + kPre < KS) bw[ks % kPre] = *reinterpret_cast<const u32x4*>(qc + 16 * (ks + kPre));
          acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[ks]),
                                                        __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < kUp; ++j) {
          const int r = ks * kUp + j;
          if (ct > 0 && r < 16) update(prev[r], wr[r], ct - 1, sbase + 8 * (r / 4) + (r % 4));
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      prev = acc;
    }
  };
  // Row norms of a tile are wave-uniform loads, fetched one tile ahead.
  // 1/norm_f: NaN for a tombstone or an unused slot (never kept), 0 for an
  // all-zero row (score 0, exact).
  float ns[32];
  auto load_norms = [&](uint32_t t) {
#pragma unroll
    for (int j = 0; j < 32; ++j) ns[j] = norms[static_cast<size_t>(t) * 32 + j];
  };
  if (t_begin < t_end) load_norms(t_begin);
  // One tile buffer per wavefront (the two wavefronts of a SIMD take turns
  // waiting for their tiles and running the matrix cores).
  for (uint32_t t = t_begin; t < t_end; ++t) {
    u32x4 a[KS];
    load_a(a, t);
    float wr[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int j = 8 * (r / 4) + (r % 4);
      const float n0 = ns[j];
      const float n1 = ns[j + 4];
      const float nf = __builtin_bit_cast(float, half ? __float_as_uint(n1) : __float_as_uint(n0));
      wr[r] = nf == 0.0f ? 0.0f : __builtin_amdgcn_rcpf(nf);
    }
    if (t + 1 < t_end) load_norms(t + 1);
    fold(a, wr, t);
  }
  // The two lane halves of a column hold disjoint slots: merge their lists
  // (top two of four, the third joins the dropped maximum), then the
  // block's 8 sub-streams per query go out through LDS so that every
  // (plane, query) row receives one 32-byte run.
  __syncthreads();  // every wavefront is done with the staged queries
  uint32_t* s_out = reinterpret_cast<uint32_t*>(s_qb);  // [kEntryPlanes][QP][kBatchWaves]
  const int wv = threadIdx.x / kWave;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const float o1 = __shfl_xor(b1[ct], 32);
    const float o2 = __shfl_xor(b2[ct], 32);
    const float onk = __shfl_xor(nk[ct], 32);
    const uint32_t oi1 = __shfl_xor(i1[ct], 32);
    const uint32_t oi2 = __shfl_xor(i2[ct], 32);
    const bool mine = b1[ct] >= o1;
    const float w1 = mine ? b1[ct] : o1, w2 = mine ? b2[ct] : o2;
    const float l1 = mine ? o1 : b1[ct], l2 = mine ? o2 : b2[ct];
    const uint32_t wi1 = mine ? i1[ct] : oi1, wi2 = mine ? i2[ct] : oi2;
    const uint32_t li1 = mine ? oi1 : i1[ct];
    const bool keep_w2 = w2 >= l1;
    const float s2 = keep_w2 ? w2 : l1;
    const uint32_t si2 = keep_w2 ? wi2 : li1;
    const float third = keep_w2 ? l1 : fmaxf(w2, l2);
    const float nkm = fmaxf(fmaxf(nk[ct], onk), third);
    if (half == 0) {
      const int q = ct * 32 + col;
      s_out[(0 * QP + q) * kBatchWaves + wv] = __float_as_uint(w1 * iq[ct]);
      s_out[(1 * QP + q) * kBatchWaves + wv] = __float_as_uint(s2 * iq[ct]);
      s_out[(2 * QP + q) * kBatchWaves + wv] = __float_as_uint(nkm * iq[ct]);
      s_out[(3 * QP + q) * kBatchWaves + wv] = wi1;
      s_out[(4 * QP + q) * kBatchWaves + wv] = si2;
    }
  }
  __syncthreads();
  const size_t n_sub = static_cast<size_t>(gridDim.x) * kBatchWaves;
  for (int x = threadIdx.x; x < kEntryPlanes * QP * 2; x += blockDim.x) {
    const int pq = x >> 1;
    const u32x4 v = reinterpret_cast<const u32x4*>(s_out)[x];
    *reinterpret_cast<u32x4*>(planes + pq * n_sub + blockIdx.x * kBatchWaves + (x & 1) * 4) = v;
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

// Descending bitonic sort of one value per lane across the wavefront
// (values must not be NaN).
__device__ inline float wave_sort_desc(float v) {
  const int lane = __lane_id();
#pragma unroll
  for (int size = 2; size <= kWave; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const float o = __shfl_xor(v, stride);
      const bool desc = (lane & size) == 0;  // run direction; the last run (size 64) descends
      const bool low = (lane & stride) == 0;
      v = (low == desc) ? fmaxf(v, o) : fminf(v, o);
    }
  }
  return v;
}

// Merge, certificate and exact rescore; grid = one block of kMergeThreads
// per query of the pass.  planes: the screen's rows (n_sub sub-streams,
// QP queries); query qi (pass column) has its `dim` values at query +
// qi*qstride elements (F32 or BF16).  The screen bound for the query
// (|s~ - score|):
//   B = (gamma + delta) * (1 + 2^-20) + 8 * 2^-24
//       + 1.01e-8 / (qn * nmin) + sqrt(dim) * 2^-125 * (1/qn + 1/nmin)
//       + dim * 2^-125 / (qn * nmin),
// gamma bounding the fp32 accumulation, delta the rounding of an fp32
// query to bf16, 8 * 2^-24 the reciprocals and products of the screened
// score and the score's own rounding, the 1e-8 term the law's
// denominator, the last terms bf16 values or products flushed near zero;
// qn is the law's query norm and nmin the smallest positive row norm.
//
// Steps: the last wavefront stages the query and one of its lanes forms
// the law's qnorm while the others load the sub-streams' entries.  Each
// of those wavefronts sorts its lanes' largest kept s~; the largest k-th
// of those, L, is a lower bound on v_k, so every kept entry at or above t
// lies at or above L - 2B.  Those entries (at most kSurvMax, else no
// certificate) are collected in LDS, one thread each: it ranks its entry
// by (s~ desc, sub-stream asc) and counts the entries above s~ + 2B.
// Fewer than k such entries holds for every entry at or above t (those
// above it then lie above v_k), so the entries passing that count -- a
// prefix of the ranking -- form the law's dot products of their rows and
// are ranked by law score (score desc, node id asc).  Rescoring entries
// below t as well changes nothing: they are real nodes with law scores.
// Writes out[qi*k ..) (the law's top-k, host mapped) and status[qi] = 1
// when certified (0: route qi again on the exact path).
constexpr int kMergeThreads = 512;
constexpr int kMergeWavesB = kMergeThreads / kWave;
constexpr int kMergeLoaders = kMergeThreads - kWave;  // threads of the entry-loading wavefronts
constexpr int kMergePer = 8;       // sub-streams per loading thread: n_sub <= 3584
constexpr int kSurvMax = kMergeThreads;
constexpr uint32_t kBatchMaxDim = 288;

__global__ __launch_bounds__(kMergeThreads) void mla_batch_merge_kernel(
    const uint32_t* __restrict__ planes, uint32_t n_sub, int QP, const u32x4* __restrict__ tiles,
    const float* __restrict__ norms, const uint64_t* __restrict__ ids, uint64_t cap,
    uint32_t dim, const void* __restrict__ query, int q_dtype, size_t qstride, double gamma,
    double delta, const unsigned* __restrict__ min_norm, int k, Cand* __restrict__ out,
    unsigned* __restrict__ status) {
  __shared__ double s_q[kBatchMaxDim];      // the query, zero past dim
  __shared__ float s_lw[kMergeWavesB];      // per wavefront: k-th largest lane maximum
  __shared__ float s_nk[kMergeWavesB];      // per wavefront: largest dropped s~
  __shared__ __align__(16) float s_sv[kSurvMax];       // survivors: s~
  __shared__ __align__(16) uint32_t s_key[kSurvMax];   //   2 * sub-stream + (second kept entry)
  __shared__ uint32_t s_slot[kSurvMax];
  __shared__ uint16_t s_byrank[kSurvMax];   // survivor holding each s~ rank
  __shared__ float s_es[kSurvMax];          // law scores of the ranked prefix (NaN: not finite)
  __shared__ uint64_t s_eid[kSurvMax];
  __shared__ uint32_t s_eslot[kSurvMax];
  __shared__ double s_qn;
  __shared__ float s_ek;
  __shared__ unsigned s_count;
  const int tid = threadIdx.x;
  const int lane = tid & (kWave - 1);
  const int wave = tid / kWave;
  const int qi = blockIdx.x;
  const size_t plane = static_cast<size_t>(QP) * n_sub;
  const size_t row = static_cast<size_t>(qi) * n_sub;
  const float* p_s1 = reinterpret_cast<const float*>(planes) + row;
  const float* p_s2 = p_s1 + plane;
  const float* p_nk = p_s2 + plane;
  const uint32_t* p_i1 = planes + 3 * plane + row;
  const uint32_t* p_i2 = p_i1 + plane;

  float v1[kMergePer], v2[kMergePer];
  uint32_t j1[kMergePer], j2[kMergePer];
  float nk = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMergePer; ++j) {
    const uint32_t i = static_cast<uint32_t>(j * kMergeLoaders + tid);
    v1[j] = v2[j] = -INFINITY;
    j1[j] = j2[j] = 0u;
    if (tid < kMergeLoaders && i < n_sub) {
      v1[j] = p_s1[i];
      v2[j] = p_s2[i];
      j1[j] = p_i1[i];
      j2[j] = p_i2[i];
      nk = fmaxf(nk, p_nk[i]);
    }
  }
  if (wave == kMergeWavesB - 1) {
    // the last wavefront stages the query; its lane 0 forms the law's
    // qnorm (d ascending; zero past dim adds exact zeros)
    const unsigned char* qbase = static_cast<const unsigned char*>(query) +
                                 static_cast<size_t>(qi) * qstride * (q_dtype == kBF16 ? 2 : 4);
    for (uint32_t d = lane; d < kBatchMaxDim; d += kWave) {
      double x = 0.0;
      if (d < dim) {
        x = q_dtype == kBF16
                ? static_cast<double>(bf16_to_f32(reinterpret_cast<const uint16_t*>(qbase)[d]))
                : static_cast<double>(reinterpret_cast<const float*>(qbase)[d]);
      }
      s_q[d] = x;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if (lane == 0) {
      double acc = 0.0;
#pragma unroll
      for (uint32_t d = 0; d < kBatchMaxDim; ++d) acc = fma(s_q[d], s_q[d], acc);
      s_qn = sqrt(acc);
    }
  }
  if (tid == 0) s_count = 0u;
  // largest finite kept s~ of the thread; a +inf s~ voids the certificate
  float m = -INFINITY;
  bool pinf = false;
#pragma unroll
  for (int j = 0; j < kMergePer; ++j) {
    if (isfinite(v1[j])) m = fmaxf(m, v1[j]);
    if (isfinite(v2[j])) m = fmaxf(m, v2[j]);
    pinf = pinf || v1[j] == INFINITY || v2[j] == INFINITY;
  }
  const float ms = wave_sort_desc(m);
#pragma unroll
  for (int off = 1; off < kWave; off <<= 1) nk = fmaxf(nk, __shfl_xor(nk, off));
  if (lane == k - 1) s_lw[wave] = ms;
  if (lane == 0) s_nk[wave] = nk;
  const int any_pinf = __syncthreads_or(pinf ? 1 : 0);

  const double qn = s_qn;
  const double nmin = static_cast<double>(__uint_as_float(*min_norm));
  const double bound = (gamma + delta) * (1.0 + 0x1p-20) + 8.0 * 0x1p-24 +
                       1.01e-8 / (qn * nmin) +
                       sqrt(static_cast<double>(dim)) * 0x1p-125 * (1.0 / qn + 1.0 / nmin) +
                       dim * 0x1p-125 / (qn * nmin);
  float L = -INFINITY, nk_all = -INFINITY;
#pragma unroll
  for (int w = 0; w < kMergeWavesB - 1; ++w) {
    L = fmaxf(L, s_lw[w]);
    nk_all = fmaxf(nk_all, s_nk[w]);
  }
  const double floor_s = static_cast<double>(L) - 2.0 * bound - 0x1p-40;
  auto offer = [&](float v, uint32_t key, uint32_t slot) {
    if (isfinite(v) && static_cast<double>(v) >= floor_s) {
      const unsigned at = atomicAdd(&s_count, 1u);
      if (at < static_cast<unsigned>(kSurvMax)) {
        s_sv[at] = v;
        s_key[at] = key;
        s_slot[at] = slot;
      }
    }
  };
#pragma unroll
  for (int j = 0; j < kMergePer; ++j) {
    const uint32_t i = static_cast<uint32_t>(j * kMergeLoaders + tid);
    offer(v1[j], 2u * i, j1[j]);
    offer(v2[j], 2u * i + 1u, j2[j]);
  }
  __syncthreads();
  const unsigned count = s_count;
  const int n = static_cast<int>(count < static_cast<unsigned>(kSurvMax) ? count : kSurvMax);
  int my_rank = 0;
  bool sup = false;
  double dot = 0.0;
  float nf = 0.0f;
  uint64_t eid = kNoId;
  uint32_t slot = 0u;
  if (tid < n) {
    const float sv = s_sv[tid];
    const uint32_t key = s_key[tid];
    const double hi = static_cast<double>(sv) + 2.0 * bound + 0x1p-40;
    int above = 0;
    int i = 0;
    for (; i + 4 <= n; i += 4) {
      const float4 o = *reinterpret_cast<const float4*>(&s_sv[i]);
      const uint4 kk = *reinterpret_cast<const uint4*>(&s_key[i]);
      my_rank += (o.x > sv || (o.x == sv && kk.x < key)) ? 1 : 0;
      my_rank += (o.y > sv || (o.y == sv && kk.y < key)) ? 1 : 0;
      my_rank += (o.z > sv || (o.z == sv && kk.z < key)) ? 1 : 0;
      my_rank += (o.w > sv || (o.w == sv && kk.w < key)) ? 1 : 0;
      above += (static_cast<double>(o.x) > hi) + (static_cast<double>(o.y) > hi) +
               (static_cast<double>(o.z) > hi) + (static_cast<double>(o.w) > hi);
    }
    for (; i < n; ++i) {
      const float o = s_sv[i];
      my_rank += (o > sv || (o == sv && s_key[i] < key)) ? 1 : 0;
      above += static_cast<double>(o) > hi ? 1 : 0;
    }
    s_byrank[my_rank] = static_cast<uint16_t>(tid);
    sup = above < k;
    if (sup) {
      // the law's dot product of the row, d ascending (rows and the
      // staged query are zero past dim: exact zeros)
      constexpr int kC = kBatchMaxDim / 8;
      slot = s_slot[tid];
      const uint32_t chunks = (dim + 7) / 8;
      u32x4 rv[kC];
#pragma unroll
      for (int j = 0; j < kC; ++j) {
        const u32x4 zero = {0u, 0u, 0u, 0u};
        rv[j] = static_cast<uint32_t>(j) < chunks ? tiles[static_cast<size_t>(j) * cap + slot] : zero;
      }
      nf = norms[slot];
      eid = ids[slot];
#pragma unroll
      for (int j = 0; j < kC; ++j) {
        const uint32_t w4[4] = {rv[j].x, rv[j].y, rv[j].z, rv[j].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float f = bf16_to_f32((w4[e >> 1] >> (16 * (e & 1))) & 0xffffu);
          dot = fma(static_cast<double>(f), s_q[j * 8 + e], dot);
        }
      }
    }
  }
  const int n_el = __syncthreads_count(sup ? 1 : 0);
  const float vk = n >= k ? s_sv[s_byrank[k - 1]] : -INFINITY;
  const double t = static_cast<double>(vk) - 2.0 * bound - 0x1p-40;
  const bool pre = any_pinf == 0 && count <= static_cast<unsigned>(kSurvMax) && n >= k &&
                   static_cast<double>(nk_all) < t;
  // the rescored prefix: ranks [0, n_el)
  if (sup) {
    const float sc = static_cast<float>(dot / (qn * static_cast<double>(nf) + 1e-8));
    const bool fin = isfinite(sc);
    s_es[my_rank] = fin ? sc : __builtin_nanf("");
    s_eid[my_rank] = fin ? eid : kNoId;
    s_eslot[my_rank] = slot;
  }
  __syncthreads();
  // rank the prefix by (law score desc, node id asc)
  const bool fin = pre && tid < n_el && isfinite(s_es[tid]);
  if (fin) {
    const float es = s_es[tid];
    const uint64_t id = s_eid[tid];
    int rank = 0;
    for (int i = 0; i < n_el; ++i) rank += better(s_es[i], s_eid[i], es, id) ? 1 : 0;
    if (rank < k) {
      Cand c;
      c.score = es;
      c.slot = s_eslot[tid];
      c.id = id;
      out[static_cast<size_t>(qi) * k + rank] = c;
    }
    if (rank == k - 1) s_ek = es;
  }
  const int n_fin = __syncthreads_count(fin ? 1 : 0);
  if (tid == 0) {
    // every node outside the prefix scores below v_k - B
    const bool ok = pre && n_fin >= k &&
                    static_cast<double>(s_ek) >= static_cast<double>(vk) - bound;
    status[qi] = ok ? 1u : 0u;
  }
}

}  // namespace mla
}  // namespace grm
