// synth.hip -- host-side generator of synthetic INT8 key rows.
//
// The large ragged GQA workload stores tens of GB of keys as INT8 codes
// with one fp16 scale per row (the packed graft format with group size =
// row length, core/graft_quant.py:93-131).  Its keys are N(0, 1) values
// quantised by that law.  Drawing them with numpy takes minutes at that
// size, so the draw and the quantiser run here, on host threads.  No
// device code; nothing on the route path calls this.
//
// Row r holds dim values.  Its dim / 4 64-bit words are
//   w = splitmix64_finalise(key + (r * dim / 4 + i) * 0x9E3779B97F4A7C15),
// and value 4 i + j is table[(w >> 16 j) & 0xffff], where the caller's
// table holds the 65536 normal quantiles Phi^-1((u + 0.5) / 65536).  The
// row is then quantised:
//   scale = max_j |x_j| / 127 (fp32; 0 -> 1), s = fp16(scale) (round to
//   nearest even; 0 -> 1), code_j = clamp(rint(x_j / float(s)), -128, 127).

#include "grm_common.hpp"

#include <thread>
#include <vector>

namespace {

inline uint64_t splitmix_finalise(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

void synth_rows(uint64_t key, uint64_t r_begin, uint64_t r_end, int dim, const float* table,
                int8_t* codes, uint16_t* scales) {
  const uint64_t wpr = static_cast<uint64_t>(dim) / 4;
  std::vector<float> x(static_cast<size_t>(dim));
  for (uint64_t r = r_begin; r < r_end; ++r) {
    float m = 0.0f;
    for (uint64_t i = 0; i < wpr; ++i) {
      const uint64_t w = splitmix_finalise(key + (r * wpr + i) * 0x9E3779B97F4A7C15ull);
      for (int j = 0; j < 4; ++j) {
        const float v = table[(w >> (16 * j)) & 0xffffu];
        x[4 * i + j] = v;
        const float a = v < 0.0f ? -v : v;
        m = a > m ? a : m;
      }
    }
    float scale = m / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    _Float16 s = static_cast<_Float16>(scale);
    if (s == static_cast<_Float16>(0.0f)) s = static_cast<_Float16>(1.0f);
    const float sf = static_cast<float>(s);
    int8_t* out = codes + (r - r_begin) * static_cast<uint64_t>(dim);
    for (int j = 0; j < dim; ++j) {
      // round half to even: adding and removing 1.5 * 2^23 rounds y to an
      // integer exactly for |y| < 2^22; any larger |y| gives a value of at
      // least 2^22 in magnitude, which the clamp maps to the code rint
      // would give after clamping
      const float y = x[j] / sf;
      float c = (y + 12582912.0f) - 12582912.0f;
      c = c < -128.0f ? -128.0f : (c > 127.0f ? 127.0f : c);
      out[j] = static_cast<int8_t>(c);
    }
    scales[r - r_begin] = __builtin_bit_cast(uint16_t, s);
  }
}

}  // namespace

extern "C" int grm_hip_synth_int8_rows(uint64_t key, uint64_t row0, uint64_t rows, int dim,
                                       const float* normal_table, int threads, int8_t* codes,
                                       uint16_t* scales_f16) {
  if (!normal_table || (rows && (!codes || !scales_f16))) return grm::fail(-1, "null argument");
  if (dim <= 0 || dim % 4) return grm::fail(-1, "dim must be a positive multiple of 4");
  const int nt = threads < 1 ? 1 : (threads > 256 ? 256 : threads);
  const uint64_t per = (rows + nt - 1) / nt;
  std::vector<std::thread> pool;
  for (int t = 0; t < nt; ++t) {
    const uint64_t a = per * t;
    const uint64_t b = a + per < rows ? a + per : rows;
    if (a >= b) break;
    pool.emplace_back(synth_rows, key, row0 + a, row0 + b, dim, normal_table,
                      codes + a * static_cast<uint64_t>(dim), scales_f16 + a);
  }
  for (auto& th : pool) th.join();
  grm::clear_error();
  return 0;
}
