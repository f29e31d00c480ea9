// Host build of gaudi-kernels_amd/csrc/gk_fp8_math.h (the arithmetic the
// gfx950 kernels run), exposed with a C ABI so tests can sweep it against
// the CPU oracle.  Built by tests/test_math_host.py with g++.
#include <stdint.h>

#include "gk_fp8_math.h"

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

}  // extern "C"
