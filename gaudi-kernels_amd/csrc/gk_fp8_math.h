// E4M3 / bf16 bit arithmetic shared by the gfx950 kernels.  Every function is
// __host__ __device__ and the header also compiles with a plain C++ compiler,
// so the exact code the kernels run is checked on the CPU
// (tests/csrc/math_check.cpp, tests/test_math_host.py).
//
// OCP E4M3FN: magnitude m = code & 0x7f, e = m >> 3, f = m & 7,
// value = (1 + f/8) * 2^(e-7) (e > 0) or f * 2^-9 (e == 0); 0x7f is NaN.
// Gaudi2 half-range E4M3 shares the value of every magnitude <= 0x77.
#pragma once

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#else  // host-only build of the same arithmetic (CPU self-checks)
#include <cmath>
#ifndef __host__
#define __host__
#endif
#ifndef __device__
#define __device__
#endif
#endif
#include <stdint.h>

namespace gk {

__host__ __device__ inline uint32_t f32_bits(float v) {
  union { float f; uint32_t u; } c;
  c.f = v;
  return c.u;
}

__host__ __device__ inline float bits_f32(uint32_t u) {
  union { float f; uint32_t u; } c;
  c.u = u;
  return c.f;
}

// Round-to-nearest-even encode of a finite fp32 to OCP E4M3FN.  Callers clamp
// to [-448, 448] first (block_fp8_oracle.py:28 does the same before its cast),
// so the "rounds past 448" branch only maps to the NaN code like torch does.
__host__ __device__ inline uint32_t e4m3_rne(float v) {
  const uint32_t b = f32_bits(v);
  const uint32_t sign = (b >> 24) & 0x80u;
  const uint32_t mb = b & 0x7fffffffu;
  uint32_t code;
  if (mb < 0x3c800000u) {                  // |v| < 2^-6: subnormal grid 2^-9
    const float q = rintf(bits_f32(mb) * 512.0f);  // exact scale, RNE
    code = static_cast<uint32_t>(q);       // 0..8 (8 == 2^-6 == code 0x08)
  } else {
    const uint32_t r = (mb + 0x7ffffu + ((mb >> 20) & 1u)) & 0xfff00000u;
    const int e = static_cast<int>(r >> 23) - 127;
    code = (static_cast<uint32_t>(e + 7) << 3) | ((r >> 20) & 7u);
    if (code > 0x7eu) code = 0x7fu;
  }
  return sign | code;
}

// Activation scale of one 1x128 group, block_fp8_oracle.py:27 of the reference:
// fp32(max(amax, 1e-10)) * fp32(1/448), one fp32 multiply.
__host__ __device__ inline float act_scale(float amax) { return fmaxf(amax, 1e-10f) * (1.0f / 448.0f); }

// fp32 quotient x / s for the activation quantizer, given r within one ulp of
// fp32(1 / s).  q0 = x*r is refined by one residual step,
// q = q0 + (x - s*q0) * r, computed as fma(-fma(s, q0, -x), r, q0): the
// residual is formed with the opposite sign and negated, which keeps -0 for
// x = -0 (fma(-s, q0, x) would give +0 there) and costs only source
// negations.  For every finite bf16 x and every scale s =
// act_scale(a) over all bf16 magnitudes a >= |x|, e4m3_rne(q) equals
// e4m3_rne(x / s) with IEEE division; the only quotients that differ are
// fp32 subnormals, which encode to zero either way.  The exhaustive check
// is tests/csrc/math_check.cpp:mc_div_mismatches.
__host__ __device__ inline float act_quotient(float x, float s, float r) {
  const float q0 = x * r;
  return fmaf(-fmaf(s, q0, -x), r, q0);
}

// OCP E4M3FN code -> fp32 value (finite codes; 0x7f decodes to 480, never used).
__host__ __device__ inline float e4m3_value(uint32_t code) {
  const uint32_t m = code & 0x7fu;
  const uint32_t e = m >> 3, f = m & 7u;
  const float mag = e ? bits_f32(((e + 120u) << 23) | (f << 20)) : static_cast<float>(f) * (1.0f / 512.0f);
  return (code & 0x80u) ? -mag : mag;
}

// fp32 -> bf16 bits, round to nearest even (NaN -> canonical quiet NaN).
// Separately rounded fp32 multiply and add.  hipcc contracts a * b + c into
// one fma by default (and __fmul_rn / __fadd_rn are plain operators in this
// toolchain); operations emitted under contract(off) are never fused.
__host__ __device__ inline float mul_rn(float a, float b) {
#pragma clang fp contract(off)
  return a * b;
}

__host__ __device__ inline float add_rn(float a, float b) {
#pragma clang fp contract(off)
  return a + b;
}

// SiLU of the reference's fused SiLU-and-mul (csrc/tpc/generic_dense/
// silu_and_mul_bf16.c:4-15): g / (1 + e^-g) in fp32; g <= -88 gives 0; NaN
// passes through; g = +inf gives NaN there (its Newton-refined quotient
// computes -inf + inf), and so here.  The quotient is the IEEE one.
__host__ __device__ inline float silu_ref(float g) {
  // The quotient is evaluated for every g and the special cases are selected
  // afterwards (same values as early returns, but no branches, so the GPU
  // overlaps the exp and division latencies of consecutive elements).
  const float q = g / (1.0f + expf(-g));
  float r = g <= -88.0f ? 0.0f : q;
  r = g == __builtin_huge_valf() ? __builtin_nanf("") : r;
  return g != g ? g : r;
}

// GELU of the reference's gk_gelu_and_mul_bf16_v1 (csrc/tpc/generic_dense/
// gelu_and_mul_bf16.c:4-49): approximate = 0 is the exact GELU
// x * erfc(-x / sqrt(2)) / 2, approximate = 1 the tanh form
// x * sigmoid(2 sqrt(2/pi) (x + 0.044715 x^3)), both in fp32 from the
// device library's erfcf / expf (the reference evaluates its own polynomials;
// its test bounds both against fp64, tests/track_a_device_verify.cpp:274-286).
// As there: +inf -> +inf, -inf -> 0, NaN -> NaN, and the tanh form is 0 for
// x <= -15 (tpc_math_safe.h:149), where the fp64 value is below the fp32
// range anyway.
__host__ __device__ inline float gelu_erf_ref(float x) {
  if (x != x) return x;
  if (x == __builtin_huge_valf()) return x;
  if (x == -__builtin_huge_valf()) return 0.0f;
  return 0.5f * x * erfcf(-x * 0.70710678118654752f);
}

__host__ __device__ inline float gelu_tanh_ref(float x) {
  if (x != x) return x;
  if (x == __builtin_huge_valf()) return x;
  if (x <= -15.0f) return 0.0f;
  const float u = 1.5957691216057308f * (x + 0.044715f * x * x * x);
  if (u >= 0.0f) return x / (1.0f + expf(-u));
  const float e = expf(u);
  return x * (e / (1.0f + e));
}

__host__ __device__ inline uint16_t bf16_rne(float v) {
  const uint32_t b = f32_bits(v);
  if ((b & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  return static_cast<uint16_t>((b + 0x7fffu + ((b >> 16) & 1u)) >> 16);
}

__host__ __device__ inline float bf16_value(uint16_t h) { return bits_f32(static_cast<uint32_t>(h) << 16); }

// ---- codec on four packed codes (SWAR) -------------------------------------
// Forward (OCP -> half range, value / 2, RNE), per byte:
//   m >= 16 : m - 8
//   m <  16 : (m >> 1) + (m & (m >> 1) & 1)      (ties to even on the 2^-9 grid)
// Closed form of python/gaudi_kernels/fp8_codec.py:36-40.
__host__ __device__ inline uint32_t codec_half4(uint32_t x) {
  const uint32_t sign = x & 0x80808080u;
  const uint32_t m = x & 0x7f7f7f7fu;
  const uint32_t ge16 = ((m + 0x70707070u) & 0x80808080u) >> 7;      // 1 per byte if m >= 16
  const uint32_t mask_ge = ge16 * 0xffu;
  const uint32_t big = ((m | 0x80808080u) - 0x08080808u) & 0x7f7f7f7fu; // m - 8, no borrow
  const uint32_t sh = (m >> 1) & 0x3f3f3f3fu;
  const uint32_t small = sh + (m & sh & 0x01010101u);
  return sign | (big & mask_ge) | (small & ~mask_ge);
}

// Bytes of x whose OCP magnitude is the NaN code 0x7f: 0x80 in each such byte.
__host__ __device__ inline uint32_t ocp_nan4(uint32_t x) {
  return ((x & 0x7f7f7f7fu) + 0x01010101u) & 0x80808080u;
}

// Number of bytes the forward codec rounds: magnitude < 16 and odd.
__host__ __device__ inline uint32_t codec_rounded4(uint32_t x) {
  const uint32_t m = x & 0x7f7f7f7fu;
  const uint32_t lt16 = (~(m + 0x70707070u) & 0x80808080u) >> 7;
  const uint32_t odd = m & 0x01010101u;
  const uint32_t hits = lt16 & odd;
  return (hits & 1u) + ((hits >> 8) & 1u) + ((hits >> 16) & 1u) + (hits >> 24);
}

// Inverse (half range -> OCP, value * 2, exact), per byte:
//   m <= 7 : 2m       8 <= m <= 0x76 : m + 8       m >= 0x77 : no image (flagged)
__host__ __device__ inline uint32_t codec_double4(uint32_t x) {
  const uint32_t sign = x & 0x80808080u;
  const uint32_t m = x & 0x7f7f7f7fu;
  const uint32_t ge8 = ((m + 0x78787878u) & 0x80808080u) >> 7;
  const uint32_t mask_ge = ge8 * 0xffu;
  const uint32_t plus8 = m + 0x08080808u;
  const uint32_t dbl = m << 1;
  return sign | ((plus8 & mask_ge) | (dbl & ~mask_ge));
}

// Bytes with magnitude >= 0x77 (no OCP image at twice the value): 0x80 each.
__host__ __device__ inline uint32_t half_invalid4(uint32_t x) {
  return ((x & 0x7f7f7f7fu) + 0x09090909u) & 0x80808080u;
}

}  // namespace gk
