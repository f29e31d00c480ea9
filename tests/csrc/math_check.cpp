// Host build of gaudi-kernels_amd/csrc/gk_fp8_math.h (the arithmetic the
// gfx950 kernels run), exposed with a C ABI so tests can sweep it against
// the CPU oracle.  Built by tests/test_math_host.py with g++.
#include <math.h>
#include <stdint.h>
#include <string.h>

#include <thread>
#include <vector>

#include "gk_fp8_math.h"

namespace {

float bf16_bits_to_f32(uint32_t h) { return gk::bits_f32(h << 16); }

// Mismatching e4m3 codes between gk::act_quotient and IEEE division, for
// amax over the bf16 magnitudes amax_lo <= a < amax_hi (step `step`), every
// finite bf16 x with |x| <= a and every reciprocal r within one ulp of
// fp32(1/s).
int64_t div_mismatches_range(uint32_t a_first, uint32_t a_step, uint32_t a_end) {
  int64_t bad = 0;
  for (uint32_t ah = a_first; ah < a_end; ah += a_step) {
    const float s = gk::act_scale(bf16_bits_to_f32(ah));
    volatile float one = 1.0f;
    const float rn = one / s;
    // the correctly rounded reciprocal and its two neighbours: any r within
    // one ulp of fp32(1/s), which covers every faithful reciprocal
    const float rs[3] = {nextafterf(rn, 0.0f), rn, nextafterf(rn, INFINITY)};
    for (uint32_t xh = 0; xh < 0x10000u; ++xh) {
      if ((xh & 0x7fffu) > ah) continue;
      const float x = bf16_bits_to_f32(xh);
      volatile float vx = x;
      const uint32_t want = gk::e4m3_rne(vx / s);
      for (float r : rs)
        if (gk::e4m3_rne(gk::act_quotient(x, s, r)) != want) ++bad;
    }
  }
  return bad;
}

}  // namespace

extern "C" {

void mc_e4m3_rne(const float* v, uint8_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = static_cast<uint8_t>(gk::e4m3_rne(v[i]));
}

void mc_e4m3_value(const uint8_t* c, float* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = gk::e4m3_value(c[i]);
}

void mc_bf16_rne(const float* v, uint16_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) out[i] = gk::bf16_rne(v[i]);
}

// op: 0 codec_half4, 1 ocp_nan4, 2 codec_rounded4, 3 codec_double4, 4 half_invalid4
void mc_swar(int op, const uint32_t* x, uint32_t* out, int64_t n) {
  for (int64_t i = 0; i < n; ++i) {
    switch (op) {
      case 0: out[i] = gk::codec_half4(x[i]); break;
      case 1: out[i] = gk::ocp_nan4(x[i]); break;
      case 2: out[i] = gk::codec_rounded4(x[i]); break;
      case 3: out[i] = gk::codec_double4(x[i]); break;
      default: out[i] = gk::half_invalid4(x[i]); break;
    }
  }
}

// Exhaustive check of the quantizer's division (gk::act_quotient): every
// finite positive bf16 amax (and zero, which the 1e-10 clamp covers) and
// every finite bf16 x with |x| <= amax.  Returns the number of mismatching
// E4M3 codes against IEEE fp32 division followed by the same encoder.
int64_t mc_div_mismatches(int threads) {
  if (threads < 1) threads = 1;
  std::vector<int64_t> bad(threads, 0);
  std::vector<std::thread> pool;
  for (int t = 0; t < threads; ++t)
    pool.emplace_back([t, threads, &bad] { bad[t] = div_mismatches_range(t, threads, 0x7f80u); });
  for (auto& th : pool) th.join();
  int64_t total = 0;
  for (int64_t b : bad) total += b;
  return total;
}

}  // extern "C"
