// Measurement probe for bench.py and the tests (tests/csrc/libgk_probe.so, declared in gk_probe.h beside
// this file, built by tests/csrc/build_probe.py):
// a plain streaming read of device memory, the ceiling any weight-streaming
// kernel can reach on this GPU for a given footprint.  Not part of the GEMM
// library.  Each lane reads 16-byte pieces with non-temporal loads (as the
// decode kernel reads weights), four pieces in flight per lane per loop
// step, and folds them into one word that is stored only if it takes a value
// the data never produces (so the loads cannot be removed).
//
// Also checks of the two hardware conversions the library relies on, against
// the software roundings of gk_fp8_math.h: the kernels' bf16x2_rne
// (gk_fp8_internal.h: v_cvt_pk_bf16_f32 with a NaN fix-up) against bf16_rne
// over every float bit pattern, and the E4M3 encode of quant_group8
// (v_cvt_pk_fp8_f32, both halves of the packed word) against e4m3_rne over
// every fp32 with |v| <= 464.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gk_probe.h"
#include "gk_fp8_internal.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(256) void stream_read_kernel(const u32x4* __restrict__ src, int64_t n16,
                                                          uint32_t* __restrict__ sink) {
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  u32x4 acc = {0u, 0u, 0u, 0u};
  for (; i + 3 * step < n16; i += 4 * step) {
    const u32x4 a = __builtin_nontemporal_load(src + i);
    const u32x4 b = __builtin_nontemporal_load(src + i + step);
    const u32x4 c = __builtin_nontemporal_load(src + i + 2 * step);
    const u32x4 d = __builtin_nontemporal_load(src + i + 3 * step);
    acc ^= a ^ b ^ c ^ d;
  }
  for (; i < n16; i += step) acc ^= __builtin_nontemporal_load(src + i);
  const uint32_t v = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
  if (v == 0x9E3779B9u) sink[0] = v;
}

// Input i goes through bf16x2_rne as the low value beside input i ^ 2^31 as
// the high one, so every bit pattern takes both positions.
__global__ __launch_bounds__(256) void bf16x2_check_kernel(unsigned long long* __restrict__ counts) {
  const uint64_t n = 1ull << 32, step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  unsigned long long bad = 0, seen = 0;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step) {
    const uint32_t a = static_cast<uint32_t>(i), b = a ^ 0x80000000u;
    const uint32_t h = gk::bf16x2_rne(gk::bits_f32(a), gk::bits_f32(b));
    bad += (h & 0xffffu) != gk::bf16_rne(gk::bits_f32(a));
    bad += (h >> 16) != gk::bf16_rne(gk::bits_f32(b));
    seen += 2;
  }
  atomicAdd(&counts[0], bad);
  atomicAdd(&counts[1], seen);
}

// Bit patterns 0 .. 0x43E80000 (464.0) with either sign: value i in the low
// half of the word (word_sel false) beside its negation, and again in the
// high half (word_sel true), as quant_group8 packs its eight codes.
__global__ __launch_bounds__(256) void e4m3_check_kernel(unsigned long long* __restrict__ counts) {
  const uint64_t n = 0x43E80001ull, step = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  unsigned long long bad = 0, seen = 0;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += step) {
    const float p = gk::bits_f32(static_cast<uint32_t>(i)), m = -p;
    int w = __builtin_amdgcn_cvt_pk_fp8_f32(p, m, 0, false);
    w = __builtin_amdgcn_cvt_pk_fp8_f32(m, p, w, true);
    const uint32_t cp = gk::e4m3_rne(p), cm = gk::e4m3_rne(m), u = static_cast<uint32_t>(w);
    bad += (u & 0xffu) != cp;
    bad += ((u >> 8) & 0xffu) != cm;
    bad += ((u >> 16) & 0xffu) != cm;
    bad += (u >> 24) != cp;
    seen += 2;
  }
  atomicAdd(&counts[0], bad);
  atomicAdd(&counts[1], seen);
}

}  // namespace

extern "C" int gk_probe_e4m3_check(void* counts, void* stream) {
  if (!counts || (reinterpret_cast<uintptr_t>(counts) & 7)) return 1;
  e4m3_check_kernel<<<4096, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<unsigned long long*>(counts));
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

extern "C" int gk_probe_bf16x2_check(void* counts, void* stream) {
  if (!counts || (reinterpret_cast<uintptr_t>(counts) & 7)) return 1;
  bf16x2_check_kernel<<<4096, 256, 0, static_cast<hipStream_t>(stream)>>>(static_cast<unsigned long long*>(counts));
  return hipGetLastError() == hipSuccess ? 0 : 2;
}

extern "C" int gk_probe_stream_read(const void* src, size_t bytes, void* sink, int workgroups, void* stream) {
  if (!src || !sink || bytes < 16 || (bytes & 15) || (reinterpret_cast<uintptr_t>(src) & 15) || workgroups < 1)
    return 1;
  stream_read_kernel<<<workgroups, 256, 0, static_cast<hipStream_t>(stream)>>>(
      static_cast<const u32x4*>(src), static_cast<int64_t>(bytes / 16), static_cast<uint32_t*>(sink));
  return hipGetLastError() == hipSuccess ? 0 : 2;
}
