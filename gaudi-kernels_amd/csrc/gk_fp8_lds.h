// Device helpers of the kernels that stage operand tiles in LDS with
// direct-to-LDS buffer loads and read MFMA fragments from it with inline-asm
// ds_read (gk_fp8_prefill.hip).
#pragma once

#include <type_traits>
#include <utility>

#include "gk_fp8_tile.h"

namespace gk {

// Word 3 of a raw buffer resource on gfx9-family parts (data format 32; the
// format is not used by the dword loads here, but must be valid).
constexpr int kBufferWord3 = 0x00020000;

__device__ inline __attribute__((address_space(3))) void* lds_ptr(uint8_t* p) {
  return reinterpret_cast<__attribute__((address_space(3))) void*>(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)));
}

// ds_read_b128 at a per-lane base address plus an immediate offset (the
// instruction's 16-bit offset field): the block offsets of a step cost no
// address arithmetic.  Inline asm: the compiler does not treat these reads as
// aliasing the direct-to-LDS loads in flight, so it adds no waits for those;
// each caller waits for its reads itself (s_waitcnt lgkmcnt tied to the
// result registers).
template <int OFF>
__device__ inline u32x4 lds_read16_at(uint32_t base) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(r) : "v"(base), "n"(OFF));
  return r;
}

template <int OFF>
__device__ inline v8i lds_frag_at(uint32_t base0, uint32_t base1) {
  const u32x4 lo = lds_read16_at<OFF>(base0), hi = lds_read16_at<OFF>(base1);
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

// f(integral_constant<int, J>) for J = 0, 1, ...: a loop whose index is a
// compile-time constant in the body (immediate offsets, register arrays).
template <typename F, int... J>
__device__ inline void unroll_each(F&& f, std::integer_sequence<int, J...>) {
  (f(std::integral_constant<int, J>{}), ...);
}

__device__ inline v8i half_codes(v8i v) {  // native_half: OCP codes -> value / 2 (codec_half4)
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = static_cast<int>(codec_half4(static_cast<uint32_t>(v[i])));
  return v;
}

__device__ inline void promote4(v4f& acc, const v4f& t, float f) {
#pragma unroll
  for (int r = 0; r < 4; ++r) acc[r] = fmaf(t[r], f, acc[r]);
}

}  // namespace gk
