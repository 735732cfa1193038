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
//               s~ = u * (1/qnorm), u = acc * (1/norm_f) with the slot's
//               index written into the low `ibits` mantissa bits of u,
//               obeys |s~ - score| <= B, B a per-query constant (see
//               mla_batch_merge_kernel).  Each lane follows one query over
//               half of every tile its wavefront walks and keeps the three
//               largest u: the two best (each carrying its slot) and the
//               largest it did not keep; the two halves of a query are
//               merged at the end, one sub-stream per (wavefront, query).
//               "Largest" is the order of u's bits as a signed integer,
//               which is the float order on values >= +0 and puts every
//               negative value (and -0) below them; the merge certifies a
//               query only when its threshold t is positive, so only
//               positive values decide.
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

// v_med3_i32 and v_and_or_b32: the compiler forms neither from the
// equivalent min/max and and/or expressions, and the screen's per-score
// work is these two instructions and a maximum.
// b = med3(a, b, c), in place
__device__ __forceinline__ void med3_i32_into(int a, int& b, int c) {
  asm("v_med3_i32 %0, %1, %0, %2" : "+v"(b) : "v"(a), "v"(c));
}
__device__ __forceinline__ uint32_t and_or_b32(uint32_t a, uint32_t b, uint32_t c) {
  uint32_t r;
  asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

constexpr int kBatchWaves = 8;       // wavefronts per screen block (one block per CU)
constexpr int kBatchMaxCols = 256;   // queries per screen pass
constexpr int kEntryPlanes = 3;      // u1, u2, nk

// Screen results, one row of n_sub values per (plane, query): plane p of
// query q at planes + (p*QP + q)*n_sub, sub-stream i = the wavefront:
//   u1, u2  the two best u a sub-stream kept (float bits, slot code in
//   the low ibits bits), nk the largest u it did not keep.
//
// Slot code of a value: (half << (ibits - 1)) | ((t - t_begin) << 4) | r
// for result register r of lane half `half` in tile t of a wavefront
// whose tiles start at t_begin; ibits - 5 bits hold the tile offset, so
// the host picks ibits from the longest run of tiles a wavefront walks.
// Writing the code moves u by less than 2^(ibits-23) |u| (2^(ibits-149)
// near zero), which the merge adds to B.
// Screen; grid = one block of kBatchWaves wavefronts per CU, LDS holds the
// pass's queries: qpad[QP][stride] bf16 (row d of query j at j*stride + d,
// stride = 16*KS + 8 so the 16-byte reads of 32 rows hit distinct
// banks).  Wavefront w walks 32-slot tiles [w*T/W, (w+1)*T/W).  For K-step
// ks the A fragment of lane l is chunk 2*ks + l/32 (8 values) of slot
// tile*32 + l%32 -- two 512-byte runs per load -- and the B fragment is
// query ct*32 + l%32 at dims 16*ks + 8*(l/32) .. +8; result register r of
// lane l is slot tile*32 + 8*(r/4) + 4*(l/32) + r%4 against that query.
//
// kProbe (tests of the screen bound only): every coded u goes to
// planes[q*cap + slot] instead of the lists, and nothing else is written.
template <int KS, int CT, bool kProbe = false>
__global__ __launch_bounds__(kBatchWaves * kWave) void mla_batch_screen_kernel(
    const u32x4* __restrict__ tiles, const float* __restrict__ norms, uint64_t cap,
    uint32_t chunks, uint32_t n_tiles32, const uint16_t* __restrict__ qpad, int stride_arg,
    int ibits, uint32_t* __restrict__ planes) {
  constexpr int QP = 32 * CT;
  constexpr int stride = 16 * KS + 8;  // the host's row stride (stride_arg)
  (void)stride_arg;
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
  // per column tile: the three largest coded u as signed-integer bits
  // (b1 >= b2 >= b3)
  int b1[CT], b2[CT], b3[CT];
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) b1[ct] = b2[ct] = b3[ct] = INT32_MIN;
  const uint32_t keep_mask = ~((1u << ibits) - 1u);
  // A fragment ks of tile t: chunk 2*ks + half of slot t*32 + col (the
  // bank holds 2*KS planes, zero past its chunks)
  const u32x4* lane_base = tiles + static_cast<uint64_t>(half) * cap + col;
  auto load_frag = [&](u32x4 (&a)[KS], uint32_t t, int ks) {
    a[ks] = __builtin_nontemporal_load(lane_base + static_cast<uint64_t>(2 * ks) * cap +
                                       static_cast<uint64_t>(t) * 32);
  };
  const uint16_t* qrow = s_qb + col * stride + 8 * half;
  // Lanes track u = acc * (1/norm_f); s~ = u * (1/qnorm) is formed by the
  // merge (rounding is monotone, so the largest u give the largest s~).
  // A slot that never ranks (tombstone, unused slot, non-finite row: the
  // bank stores its row as zeros) has 1/norm_f = -0, so u is a zero and
  // never outranks a positive value.  The accumulation cannot overflow
  // where the merge certifies (it checks ||q|| * max norm_f), so a u that
  // is not finite comes from a non-finite query, which the merge never
  // certifies.  u's low bits take the slot code, and the three largest
  // move by two medians and a maximum of the integer bits:
  // b3 = med3(b2, b3, v), b2 = med3(b1, b2, v), b1 = max(b1, v) keep
  // b1 >= b2 >= b3 the three largest values seen.
  auto update = [&](float accv, float w, int ct, uint32_t code) {
    const int v = static_cast<int>(and_or_b32(__float_as_uint(accv * w), keep_mask, code));
    med3_i32_into(b2[ct], b3[ct], v);
    med3_i32_into(b1[ct], b2[ct], v);
    b1[ct] = max(b1[ct], v);
  };
  // Matrix-core chains: the column tiles advance in groups of kG
  // independent accumulation chains -- step ks issues the kG MFMAs of a[ks]
  // with the group's kG query fragments -- and the group's 16*kG results
  // are reduced once its chains end.  With two wavefronts per SIMD, two
  // chains keep the matrix core as busy as four (the other wavefront
  // fills the gaps) and halve the stretch of MFMAs between reductions,
  // which the other wavefront's reductions then overlap more evenly: 1M x
  // 288 x 256 queries screened in 152 us with kG = 2 against 161 us with
  // kG = 4.  Query fragments stream from LDS kPre fragments ahead, across
  // step and group boundaries.  In the tile's last
  // group each a[ks] is reloaded with the next tile's fragment as soon as
  // its last MFMA has issued, so the next tile's loads are in flight
  // during the rest of the group and the reductions (no second tile
  // buffer is needed).  The reload is unconditional: after a wavefront's
  // last tile it reads that tile again (cached, and never folded).
  constexpr int kG = CT < 2 ? CT : 2;
  constexpr int kGroups = CT / kG;
  constexpr int kPre = 4;
  constexpr int kSteps = CT * KS;  // fragment stream: (group, ks, chain)
  auto bfrag = [&](int step) -> u32x4 {
    const int g = step / (KS * kG);
    const int ks = (step / kG) % KS;
    const int ct = g * kG + step % kG;
    return *reinterpret_cast<const u32x4*>(qrow + ct * 32 * stride + 16 * ks);
  };
  auto fold = [&](u32x4 (&a)[KS], const float (&wr)[16], uint32_t t, uint32_t t_next) {
    // code of result register r (slot t*32 + 8*(r/4) + 4*half + r%4): tcode | r
    const uint32_t tcode = (static_cast<uint32_t>(half) << (ibits - 1)) | ((t - t_begin) << 4);
    u32x4 bw[kPre];
#pragma unroll
    for (int j = 0; j < kPre; ++j) bw[j] = bfrag(j);
#pragma unroll
    for (int g = 0; g < kGroups; ++g) {
      f32x16 acc[kG];
#pragma unroll
      for (int c = 0; c < kG; ++c) {
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[c][r] = 0.0f;
      }
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
#pragma unroll
        for (int c = 0; c < kG; ++c) {
          const int step = (g * KS + ks) * kG + c;
          const u32x4 b = bw[step % kPre];
          if (step + kPre < kSteps) bw[step % kPre] = bfrag(step + kPre);
          acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[ks]),
                                                           __builtin_bit_cast(bf16x8, b), acc[c],
                                                           0, 0, 0);
        }
        if (g == kGroups - 1) load_frag(a, t_next, ks);
        __builtin_amdgcn_sched_barrier(0);
      }
#pragma unroll
      for (int c = 0; c < kG; ++c) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          if constexpr (kProbe) {
            const uint32_t slot = t * 32u + 8u * (r / 4) + 4u * half + (r % 4);
            const uint32_t q = (g * kG + c) * 32u + col;
            planes[static_cast<size_t>(q) * cap + slot] =
                and_or_b32(__float_as_uint(acc[c][r] * wr[r]), keep_mask, tcode | static_cast<uint32_t>(r));
          } else {
            update(acc[c][r], wr[r], g * kG + c, tcode | static_cast<uint32_t>(r));
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  // Row norms of a tile are wave-uniform loads, fetched one tile ahead.
  // 1/norm_f: -0 for a slot that never ranks (norm NaN: tombstone, unused
  // slot, non-finite row) and for a norm that overflowed (its law score is
  // a zero), 0 for an all-zero row (score 0, exact).
  float ns[32];
  auto load_norms = [&](uint32_t t) {
#pragma unroll
    for (int j = 0; j < 32; ++j) ns[j] = norms[static_cast<size_t>(t) * 32 + j];
  };
  // One tile buffer per wavefront, refilled for the next tile during the
  // current tile's last group (see fold).
  u32x4 a[KS];
  if (t_begin < t_end) {
    load_norms(t_begin);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) load_frag(a, t_begin, ks);
  }
  for (uint32_t t = t_begin; t < t_end; ++t) {
    float wr[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int j = 8 * (r / 4) + (r % 4);
      const float n0 = ns[j];
      const float n1 = ns[j + 4];
      const float nf = __builtin_bit_cast(float, half ? __float_as_uint(n1) : __float_as_uint(n0));
      wr[r] = nf == 0.0f ? 0.0f : (nf < INFINITY ? __builtin_amdgcn_rcpf(nf) : -0.0f);
    }
    if (t + 1 < t_end) load_norms(t + 1);
    fold(a, wr, t, t + 1 < t_end ? t + 1 : t);
  }
  if constexpr (kProbe) return;
  // The two lane halves of a column hold disjoint slots: merge their lists
  // (each half's three values go through the same update as a score), then
  // the block's 8 sub-streams per query go out through LDS so that every
  // (plane, query) row receives one 32-byte run.
  __syncthreads();  // every wavefront is done with the staged queries
  uint32_t* s_out = reinterpret_cast<uint32_t*>(s_qb);  // [kEntryPlanes][QP][kBatchWaves]
  const int wv = threadIdx.x / kWave;
#pragma unroll
  for (int ct = 0; ct < CT; ++ct) {
    const int o1 = __shfl_xor(b1[ct], 32);
    const int o2 = __shfl_xor(b2[ct], 32);
    const int o3 = __shfl_xor(b3[ct], 32);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int v = j == 0 ? o1 : (j == 1 ? o2 : o3);
      med3_i32_into(b2[ct], b3[ct], v);
      med3_i32_into(b1[ct], b2[ct], v);
      b1[ct] = max(b1[ct], v);
    }
    if (half == 0) {
      const int q = ct * 32 + col;
      s_out[(0 * QP + q) * kBatchWaves + wv] = static_cast<uint32_t>(b1[ct]);
      s_out[(1 * QP + q) * kBatchWaves + wv] = static_cast<uint32_t>(b2[ct]);
      s_out[(2 * QP + q) * kBatchWaves + wv] = static_cast<uint32_t>(b3[ct]);
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

// ------------------------------------------------------------ ring screen
//
// The same screen for a full pass of 256 queries, with the roles of LDS
// and registers swapped: each wavefront holds 64 queries' B fragments in
// registers for the whole bank, and the bank's 32-slot tiles stream into
// LDS, so every A fragment read from LDS feeds two MFMAs (the query
// fragments of mla_batch_screen_kernel cost one 1 KiB LDS read per MFMA).
//
//  * One block of four wavefronts per CU; wavefront w holds queries
//    [64 w, 64 w + 64) and has SIMD w to itself, so its 512 registers hold
//    the queries, two sets of accumulators and A fragments four K-steps
//    ahead.  The MFMAs of tile s and the reductions of tile s - 1 form one
//    straight-line region, each MFMA followed by its share of the
//    reductions and a scheduling barrier: the matrix core and the VALU work
//    side by side within the wavefront.
//  * Block b is sub-stream b of W = blocks and walks tiles
//    [b * n_tiles32 / W, (b + 1) * n_tiles32 / W), one per step, so the
//    merge decodes its slot codes as for the wavefront sub-streams of
//    mla_batch_screen_kernel.
//  * A ring of kRing tiles in LDS (2 KS chunk planes of 512 bytes each,
//    chunk c of the tile at c * 512) with their 32 slot weights.  Direct
//    loads (global_load_lds_dwordx4) fill it without registers.  A step is
//    KS tile loads of 1 KiB (two chunk planes each) and one weight load,
//    spread so that every wavefront issues the same number
//    (kLoadsPerWave); wavefronts without a tile load left for their last
//    issue all bring the weights (8 lanes carry the 128 bytes, the rest
//    repeat them into the pad of a 1 KiB weight area).  kRing - 1 tiles are
//    in flight while one is screened.
//  * Step s: each wavefront waits for its own loads of tile s (vmcnt) and
//    its LDS reads of tile s - 1 (lgkmcnt); the block barrier then makes
//    the whole tile visible and says every wavefront is done with tile
//    s - 1, whose slot the loads of tile s + kRing - 1 then refill.  Loads
//    past the block's last tile re-read that tile (never screened), so
//    every step has the same load count.
//  * The slot weights 1/norm_f come from mla_batch_weights_kernel, the
//    values mla_batch_screen_kernel forms per tile (same reciprocal).
template <int KS>
struct RingShape {
  static constexpr int kRing = 8;                         // tiles in LDS
  static constexpr int kTileU4 = 2 * KS * 32;             // u32x4 per tile
  static constexpr int kTileLoads = KS;                   // 1 KiB loads per tile
  static constexpr int kLoadsPerWave = kTileLoads / 4 + 1;  // every wavefront, every step
  static constexpr size_t kWeightOffset = static_cast<size_t>(kRing) * kTileU4 * 16;
  static constexpr size_t kWeightArea = 1024;             // bytes per tile (128 used)
  static constexpr size_t kLds = kWeightOffset + static_cast<size_t>(kRing) * kWeightArea;
};

constexpr int kRingWaves = 4;      // wavefronts per block, one block per CU
constexpr int kRingQueries = 256;  // queries per ring pass

// s_waitcnt vmcnt(n) lgkmcnt(0) (gfx9 encoding; expcnt left alone): the
// wavefront's loads but the last n are done, and so are its LDS reads.
template <int N>
__device__ __forceinline__ void wait_vmcnt_lds() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0070);
}

// The slot weights the screens multiply by: 1/norm_f (v_rcp_f32), 0 for
// an all-zero row, -0 for a slot that never ranks (NaN norm: tombstone,
// unused slot, non-finite row) and for a norm that overflowed.
__global__ void mla_batch_weights_kernel(const float* __restrict__ norms, uint64_t n,
                                         float* __restrict__ winv) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const float nf = norms[i];
  winv[i] = nf == 0.0f ? 0.0f : (nf < INFINITY ? __builtin_amdgcn_rcpf(nf) : -0.0f);
}

template <int KS, bool kProbe = false>
__global__ __launch_bounds__(kRingWaves * kWave, 1) void mla_batch_ring_kernel(
    const u32x4* __restrict__ tiles, const float* __restrict__ winv, uint64_t cap,
    uint32_t n_tiles32, const uint16_t* __restrict__ qpad, int ibits, uint32_t* __restrict__ planes) {
  using RS = RingShape<KS>;
  constexpr int stride = 16 * KS + 8;  // qpad row stride (bf16 elements)
  constexpr int QP = kRingQueries;
  constexpr int kPre = 4;              // A fragments in flight ahead of their MFMAs
  extern __shared__ u32x4 s_ring[];   // [kRing][2 KS][32 slots], then the weights
  unsigned char* s_w = reinterpret_cast<unsigned char*>(s_ring) + RS::kWeightOffset;
  const int lane = threadIdx.x & (kWave - 1);
  const int half = lane >> 5;
  const int col = lane & 31;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // query group
  const uint32_t W = gridDim.x;
  const uint32_t t_begin = static_cast<uint32_t>(static_cast<uint64_t>(blockIdx.x) * n_tiles32 / W);
  const uint32_t t_end = static_cast<uint32_t>(static_cast<uint64_t>(blockIdx.x + 1) * n_tiles32 / W);
  const uint32_t steps = t_end - t_begin;

  // B fragments of the wavefront's 64 queries: column tile c, K-step ks:
  // query 64 wv + 32 c + col at dims 16 ks + 8 half .. +8
  u32x4 bq[2][KS];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const uint16_t* row = qpad + static_cast<size_t>(64 * wv + 32 * c + col) * stride + 8 * half;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) bq[c][ks] = *reinterpret_cast<const u32x4*>(row + 16 * ks);
  }
  // The fragments are in registers before the ring's loads start, so the
  // only loads a step waits for are the ring's own (the empty asm uses
  // each value, which keeps its load ahead of the ring's).  They live in
  // AGPRs (the MFMAs read their B operand there), which leaves the VGPRs
  // to the accumulators, so the reductions read them without copies
  // (mla_route.hip is built with the MFMA VGPR-accumulator form).
#pragma unroll
  for (int c = 0; c < 2; ++c) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) asm volatile("" : "+a"(bq[c][ks]));
  }
  asm volatile("" ::: "memory");

  // The wavefront's loads of a step: tile loads m = wv + 4 j while
  // m < KS (load m: chunk planes 2 m and 2 m + 1), and for its last
  // issue, when no tile load is left, the step's weights.  Branch-free:
  // every issue is one 16-byte direct load whose addresses are selected.
  constexpr int kPer = RS::kLoadsPerWave;
  const u32x4* w16 = reinterpret_cast<const u32x4*>(winv);
  auto issue_step = [&](uint32_t s) {
    const int slot = static_cast<int>(s % RS::kRing);
    const uint32_t t = min(t_begin + s, t_end - 1);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int m = wv + kRingWaves * j;
      const bool tile_load = m < RS::kTileLoads;
      const u32x4* src_t = tiles + static_cast<uint64_t>(2 * m + half) * cap +
                           static_cast<uint64_t>(t) * 32 + col;
      const u32x4* src_w = w16 + static_cast<uint64_t>(t) * 8 + (lane & 7);
      u32x4* dst_t = s_ring + slot * RS::kTileU4 + m * 64;
      u32x4* dst_w = reinterpret_cast<u32x4*>(s_w + slot * RS::kWeightArea);
      __builtin_amdgcn_global_load_lds(tile_load ? src_t : src_w,
                                       (__attribute__((address_space(3))) void*)(tile_load ? dst_t : dst_w),
                                       16, 0, 0);
    }
  };
  // Wait for tile s, pass the barrier, refill the slot of tile s - 1.
  auto enter_step = [&](uint32_t s) {
    asm volatile("" ::: "memory");
    wait_vmcnt_lds<(RS::kRing - 2) * kPer>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    issue_step(s + RS::kRing - 1);
  };

  // per column tile: the three largest coded u as signed-integer bits
  int b1[2], b2[2], b3[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) b1[c] = b2[c] = b3[c] = INT32_MIN;
  const uint32_t keep_mask = ~((1u << ibits) - 1u);

  // One tile's screen results: accumulators, the weights of the lane's
  // result rows 8 (r / 4) + 4 half + r % 4, and the tile.
  struct Res {
    f32x16 acc[2];
    float w[16];
    uint32_t t;
    uint32_t tcode;
  };
  // Reduction of value v = 16 c + r of a finished tile.
  auto reduce_one = [&](const Res& R, int v) {
    const int c = v >> 4;
    const int r = v & 15;
    const uint32_t code = R.tcode | static_cast<uint32_t>(r);
    if constexpr (kProbe) {
      const uint32_t slot_id = R.t * 32u + 8u * (r / 4) + 4u * half + (r % 4);
      const uint32_t q = 64u * wv + 32u * c + col;
      planes[static_cast<size_t>(q) * cap + slot_id] =
          and_or_b32(__float_as_uint(R.acc[c][r] * R.w[r]), keep_mask, code);
    } else {
      const int u = static_cast<int>(and_or_b32(__float_as_uint(R.acc[c][r] * R.w[r]),
                                                keep_mask, code));
      med3_i32_into(b2[c], b3[c], u);
      med3_i32_into(b1[c], b2[c], u);
      b1[c] = max(b1[c], u);
    }
  };
  // Tile s into R: its reads and MFMAs, with the 32 reductions of the
  // previous tile P (when there is one) spread over its MFMAs, each MFMA
  // and its share fenced (sched_barrier) so that the share runs on the
  // VALU while its MFMA executes.  The weights are read as integers: the compiler then
  // does not order them after the ring's pending loads.
  auto step_tile = [&](uint32_t s, Res& R, const Res& P, auto has_prev) {
    const int slot = static_cast<int>(s % RS::kRing);
    const u32x4* tile = s_ring + slot * RS::kTileU4;
    const uint32_t* wt = reinterpret_cast<const uint32_t*>(s_w + slot * RS::kWeightArea);
    u32x4 af[kPre];
#pragma unroll
    for (int j = 0; j < kPre; ++j) af[j] = tile[(2 * j + half) * 32 + col];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const u32x4 w4 = *reinterpret_cast<const u32x4*>(wt + 8 * i + 4 * half);
      R.w[4 * i] = __uint_as_float(w4.x);
      R.w[4 * i + 1] = __uint_as_float(w4.y);
      R.w[4 * i + 2] = __uint_as_float(w4.z);
      R.w[4 * i + 3] = __uint_as_float(w4.w);
    }
    R.t = t_begin + s;
    R.tcode = (static_cast<uint32_t>(half) << (ibits - 1)) | (s << 4);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const u32x4 a = af[ks % kPre];
      if (ks + kPre < KS) af[ks % kPre] = tile[(2 * (ks + kPre) + half) * 32 + col];
#pragma unroll
      for (int c = 0; c < 2; ++c) {
        R.acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
            __builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, bq[c][ks]),
            ks == 0 ? f32x16{} : R.acc[c], 0, 0, 0);
        // the 32 reductions spread over the tile's 2 KS MFMAs (one each,
        // about 6 VALU issues, at KS = 16 or 18; two at KS = 8): they
        // issue while the MFMA runs, before the next MFMA (issue is in order)
        if constexpr (decltype(has_prev)::value) {
          constexpr int kM = 2 * KS;
          const int m = 2 * ks + c;
#pragma unroll
          for (int v = m * 32 / kM; v < (m + 1) * 32 / kM; ++v) reduce_one(P, v);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
  };
  auto reduce_tile = [&](const Res& R) {
#pragma unroll
    for (int v = 0; v < 32; ++v) reduce_one(R, v);
  };

  Res RA, RB;
  if (steps > 0) {
#pragma unroll
    for (int s = 0; s < RS::kRing - 1; ++s) issue_step(static_cast<uint32_t>(s));
    enter_step(0);
    step_tile(0, RA, RB, std::false_type{});
  }
  uint32_t s = 1;
  for (; s + 1 < steps; s += 2) {
    enter_step(s);
    step_tile(s, RB, RA, std::true_type{});
    enter_step(s + 1);
    step_tile(s + 1, RA, RB, std::true_type{});
  }
  if (s < steps) {
    enter_step(s);
    step_tile(s, RB, RA, std::true_type{});
    reduce_tile(RB);
  } else if (steps > 0) {
    reduce_tile(RA);
  }
  // no load may still be writing LDS when the block ends
  asm volatile("" ::: "memory");
  wait_vmcnt_lds<0>();
  if constexpr (kProbe) return;
  // merge the two lane halves (disjoint slots of one query), then one
  // value per (plane, query, sub-stream)
  const size_t n_sub = W;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int o1 = __shfl_xor(b1[c], 32);
    const int o2 = __shfl_xor(b2[c], 32);
    const int o3 = __shfl_xor(b3[c], 32);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const int v = j == 0 ? o1 : (j == 1 ? o2 : o3);
      med3_i32_into(b2[c], b3[c], v);
      med3_i32_into(b1[c], b2[c], v);
      b1[c] = max(b1[c], v);
    }
    if (half == 0) {
      const size_t q = static_cast<size_t>(64 * wv + 32 * c + col);
      planes[(0 * QP + q) * n_sub + blockIdx.x] = static_cast<uint32_t>(b1[c]);
      planes[(1 * QP + q) * n_sub + blockIdx.x] = static_cast<uint32_t>(b2[c]);
      planes[(2 * QP + q) * n_sub + blockIdx.x] = static_cast<uint32_t>(b3[c]);
    }
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
// per query of the pass.  planes: the screen's rows (n_sub sub-streams =
// the screen's wavefronts, QP queries; wavefront i walked tiles from
// i * n_tiles32 / n_sub); query qi (pass column) has its `dim` values at
// query + qi*qstride elements (F32 or BF16) and 1/||q|| at inv_qn[qi].
// The screened score of a kept value u is s~ = u * inv_qn[qi], its slot
// the code in u's low ibits bits.  The screen bound for the query
// (|s~ - score|):
//   B0 = (gamma + delta) * (1 + 2^-20) + 8 * 2^-24
//        + 1.01e-8 / (qn * nmin) + sqrt(dim) * 2^-125 * (1/qn + 1/nmin)
//        + dim * 2^-125 / (qn * nmin),
//   B  = B0 + 2^(ibits-23) * (1 + B0) * (1 + 2^-20) + 2^(ibits-148) / qn,
// gamma bounding the fp32 accumulation, delta the rounding of an fp32
// query to bf16, 8 * 2^-24 the reciprocals and products of the screened
// score and the score's own rounding, the 1e-8 term the law's
// denominator, the next terms bf16 values or products flushed near zero;
// the last two the slot code written into u (relative to |u|, with
// |score| <= 1, and absolute near zero).  qn is the law's query norm and
// nmin the smallest positive row norm.
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
constexpr uint32_t kBatchMaxDim = 288;

// The law's query norm (d ascending, fp64): one wavefront stages query qi
// (`dim` values, F32 or BF16, qstride elements apart) as doubles in
// s_q[kBatchMaxDim], zero past dim; its lane 0 sums the squares and
// returns the norm (other lanes return 0).
__device__ inline double stage_query_norm(double* __restrict__ s_q, const void* __restrict__ query,
                                          int q_dtype, size_t qstride, int qi, uint32_t dim,
                                          int lane) {
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
  double acc = 0.0;
  if (lane == 0) {
#pragma unroll
    for (uint32_t d = 0; d < kBatchMaxDim; ++d) acc = fma(s_q[d], s_q[d], acc);
  }
  return sqrt(acc);
}

// The screen bound B of a query (|s~ - score|, see mla_batch_merge_kernel)
// from the law's query norm qn and the smallest positive row norm nmin;
// it holds where qn * nmax < 2^125 (nmax the largest row norm).
__device__ inline double batch_screen_bound(double gamma, double delta, double qn, double nmin,
                                            uint32_t dim, int ibits) {
  const double bound0 = (gamma + delta) * (1.0 + 0x1p-20) + 8.0 * 0x1p-24 + 1.01e-8 / (qn * nmin) +
                        sqrt(static_cast<double>(dim)) * 0x1p-125 * (1.0 / qn + 1.0 / nmin) +
                        dim * 0x1p-125 / (qn * nmin);
  return bound0 + ldexp(1.0 + bound0, ibits - 23) * (1.0 + 0x1p-20) + ldexp(1.0, ibits - 148) / qn;
}

constexpr int kMergeThreads = 512;
constexpr int kMergeWavesB = kMergeThreads / kWave;
constexpr int kMergeLoaders = kMergeThreads - kWave;  // threads of the entry-loading wavefronts
constexpr int kMergePer = 8;       // sub-streams per loading thread: n_sub <= 3584
constexpr int kSurvMax = kMergeThreads;

__global__ __launch_bounds__(kMergeThreads) void mla_batch_merge_kernel(
    const uint32_t* __restrict__ planes, uint32_t n_sub, int QP, uint32_t n_tiles32, int ibits,
    const float* __restrict__ inv_qn, const u32x4* __restrict__ tiles,
    const float* __restrict__ norms, const uint64_t* __restrict__ ids, uint64_t cap,
    uint32_t dim, const void* __restrict__ query, int q_dtype, size_t qstride, double gamma,
    double delta, const unsigned* __restrict__ norm_range, int k, Cand* __restrict__ out,
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
  const float* p_u1 = reinterpret_cast<const float*>(planes) + row;
  const float* p_u2 = p_u1 + plane;
  const float* p_nk = p_u2 + plane;
  const float iq = inv_qn[qi];
  const uint32_t cmask = (1u << ibits) - 1u;
  // slot of coded value u kept by sub-stream i (see the screen's slot code)
  auto slot_of = [&](float u, uint32_t i) -> uint32_t {
    const uint32_t c = __float_as_uint(u) & cmask;
    const uint32_t t_begin = static_cast<uint32_t>(static_cast<uint64_t>(i) * n_tiles32 / n_sub);
    const uint32_t r = c & 15u;
    const uint32_t t = t_begin + ((c >> 4) & ((1u << (ibits - 5)) - 1u));
    const uint32_t slot = t * 32u + 8u * (r >> 2) + 4u * (c >> (ibits - 1)) + (r & 3u);
    // every code the screen writes names a slot of a tile it walked; the
    // clamp only keeps a corrupted value from reading past the bank
    return slot < cap ? slot : static_cast<uint32_t>(cap - 1);
  };

  float v1[kMergePer], v2[kMergePer];
  uint32_t j1[kMergePer], j2[kMergePer];
  float nk = -INFINITY;
#pragma unroll
  for (int j = 0; j < kMergePer; ++j) {
    const uint32_t i = static_cast<uint32_t>(j * kMergeLoaders + tid);
    v1[j] = v2[j] = -INFINITY;
    j1[j] = j2[j] = 0u;
    if (tid < kMergeLoaders && i < n_sub) {
      const float u1 = p_u1[i], u2 = p_u2[i];
      v1[j] = u1 * iq;
      v2[j] = u2 * iq;
      j1[j] = slot_of(u1, i);
      j2[j] = slot_of(u2, i);
      nk = fmaxf(nk, p_nk[i] * iq);
    }
  }
  if (wave == kMergeWavesB - 1) {
    // the last wavefront stages the query and forms the law's qnorm
    const double qn = stage_query_norm(s_q, query, q_dtype, qstride, qi, dim, lane);
    if (lane == 0) s_qn = qn;
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
  const double nmin = static_cast<double>(__uint_as_float(norm_range[0]));
  const double nmax = static_cast<double>(__uint_as_float(norm_range[1]));
  const double bound = batch_screen_bound(gamma, delta, qn, nmin, dim, ibits);
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
  // t > 0: the screen kept its values by their integer bits, the float
  // order only from +0 up.  qn * nmax < 2^125: no product or partial sum
  // of the bf16 query (norm at most qn * (1 + 2^-8)) and a row can reach
  // the fp32 overflow threshold (Cauchy-Schwarz, with the accumulation's
  // rounding), so the bound B holds for every screened value.
  const bool pre = any_pinf == 0 && count <= static_cast<unsigned>(kSurvMax) && n >= k &&
                   static_cast<double>(nk_all) < t && t > 0.0 && qn * nmax < 0x1p125;
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

// Tests of the screen bound: the screened scores s~ = u * (1/||q||) of a
// probe screen (planes[q*cap + slot], coded u bits) for slots [0, n),
// out_values[qi*n + slot], and the query's bound B, out_bounds[qi] (+inf
// where qn * nmax >= 2^125: B is not established there).  grid = queries
// of the pass, one wavefront each.
__global__ __launch_bounds__(kWave) void mla_batch_probe_finish_kernel(
    const uint32_t* __restrict__ planes, uint64_t cap, uint32_t n, const float* __restrict__ inv_qn,
    const void* __restrict__ query, int q_dtype, size_t qstride, uint32_t dim, double gamma,
    double delta, const unsigned* __restrict__ norm_range, int ibits, float* __restrict__ out_values,
    double* __restrict__ out_bounds) {
  __shared__ double s_q[kBatchMaxDim];
  const int qi = blockIdx.x;
  const int lane = threadIdx.x;
  const double qn = stage_query_norm(s_q, query, q_dtype, qstride, qi, dim, lane);
  if (lane == 0) {
    const double nmin = static_cast<double>(__uint_as_float(norm_range[0]));
    const double nmax = static_cast<double>(__uint_as_float(norm_range[1]));
    out_bounds[qi] = qn * nmax < 0x1p125 ? batch_screen_bound(gamma, delta, qn, nmin, dim, ibits)
                                         : static_cast<double>(INFINITY);
  }
  const float iq = inv_qn[qi];
  for (uint32_t s = lane; s < n; s += kWave) {
    out_values[static_cast<size_t>(qi) * n + s] =
        __uint_as_float(planes[static_cast<size_t>(qi) * cap + s]) * iq;
  }
}

}  // namespace mla
}  // namespace grm
