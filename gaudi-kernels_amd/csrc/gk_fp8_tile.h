// Device helpers shared by the GEMM kernels: MFMA wrappers, fragment packing,
// streaming loads and the bf16 output tile store.
#pragma once

#include "gk_fp8_internal.h"

namespace gk {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Chunk key of tile row r: the 16-byte chunk c of row r sits at slot
// c ^ lds_key(r) of its 128-byte LDS row.  Bits 3, 1, 2 of r give bits 2, 1,
// 0 of the key, so a fragment read (16 consecutive rows, chunk 2q + h for the
// lanes of quad q) lands on distinct 16-byte slots both within each 16-lane
// quarter over a 256-byte window and within each 32-lane half over a
// 512-byte window: conflict-free on gfx950, which serves a 128-bit LDS read
// 32 lanes at a time (measured: the (r >> 1) & 7 key, distinct only over 256
// bytes, read as 64 bank-conflict cycles per wave-step of the 256 x 256 kernel).
__host__ __device__ constexpr int lds_key(int r) { return ((r >> 1) & 4) | (r & 2) | ((r >> 2) & 1); }

// 16-byte streaming load (weights are read once per call: non-temporal hint).
__device__ inline uint4 load_stream16(const uint8_t* p) {
  const u32x4 v = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
  return make_uint4(v[0], v[1], v[2], v[3]);
}

__device__ inline v8i pack8(uint4 lo, uint4 hi) {
  v8i r;
  r[0] = lo.x; r[1] = lo.y; r[2] = lo.z; r[3] = lo.w;
  r[4] = hi.x; r[5] = hi.y; r[6] = hi.z; r[7] = hi.w;
  return r;
}

template <bool HALF_W>
__device__ inline v8i weight_frag(uint4 lo, uint4 hi) {
  if (HALF_W) {
    lo.x = codec_half4(lo.x); lo.y = codec_half4(lo.y); lo.z = codec_half4(lo.z); lo.w = codec_half4(lo.w);
    hi.x = codec_half4(hi.x); hi.y = codec_half4(hi.y); hi.z = codec_half4(hi.z); hi.w = codec_half4(hi.w);
  }
  return pack8(lo, hi);
}

// v_mfma_f32_32x32x64_f8f6f4 (E4M3 x E4M3), accumulating into c.  Output
// layout: lane l, register r holds D[8 (r/4) + 4 (l/32) + r%4][l%32].
__device__ inline v16f mfma32_f8(v8i a, v8i b, v16f c) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

__device__ inline v4f mfma_f8(v8i a, v8i b) {
  const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // cbsz = blgp = 0 selects E4M3 for both operands; zero scale operands select
  // the unscaled v_mfma_f32_16x16x128_f8f6f4.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
}

// Accumulating form (C = acc): the per-token / per-channel GEMM sums over all K
// inside the matrix core (its scales do not vary along K).
__device__ inline v4f mfma_f8_acc(v8i a, v8i b, v4f c) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
}

// Per-token / per-channel epilogue of the reference's channel finish
// (csrc/tpc/block_fp8_framework/channel_finish.c:9-15): y = bf16(fma(p * sa[m],
// sw[n], bias[n])) with the product p * sa rounded to fp32 first.
__device__ inline uint16_t channel_out(float p, float sam, float swn, float bn) {
  return bf16_rne(fmaf(mul_rn(p, sam), swn, bn));
}

// Writes C[n0 + 4*quad + r][m] (r = 0..3) of one 16x16 tile as bf16 with bias.
__device__ inline void store_tile(uint16_t* __restrict__ y, int64_t ldy, const float* __restrict__ bias, int M,
                                  int N, int m, int n, v4f acc) {
  if (m >= M) return;
  float b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (bias) {
#pragma unroll
    for (int r = 0; r < 4; ++r) b[r] = (n + r < N) ? bias[n + r] : 0.0f;
  }
  uint16_t* row = y + static_cast<int64_t>(m) * ldy + n;
  const uint32_t h01 = bf16x2_rne(acc[0] + b[0], acc[1] + b[1]);
  const uint32_t h23 = bf16x2_rne(acc[2] + b[2], acc[3] + b[3]);
  if (n + 3 < N && ((reinterpret_cast<uintptr_t>(row) & 7) == 0)) {
    *reinterpret_cast<uint2*>(row) = make_uint2(h01, h23);
  } else {
    if (n < N) row[0] = static_cast<uint16_t>(h01);
    if (n + 1 < N) row[1] = static_cast<uint16_t>(h01 >> 16);
    if (n + 2 < N) row[2] = static_cast<uint16_t>(h23);
    if (n + 3 < N) row[3] = static_cast<uint16_t>(h23 >> 16);
  }
}

}  // namespace gk
