// Row-parallel (K-sharded) completion of the block-FP8 GEMM on gfx950: the
// ordered rank sum of gathered slices and the fp32-partial finish.
//
// rank_sum: the reference's gk_rank_sum_f32_v1 / gk_rank_sum_bf16_v1
// (csrc/tpc/generic_dense/rank_sum.c:4-42).  `gathered` holds world
// contiguous slices of elems values, slice r at r * elems (what an all-gather
// of each rank's partial leaves); dst[i] = ((s0[i] + s1[i]) + s2[i]) + ...
// in fp32, in rank order, so every process that sums the same gathered
// buffer gets the same bits.  The bf16 form widens each slice to fp32, sums
// the same way and rounds once to bf16 (nearest even).
//
// partial finish: y = bf16(p + bias), the last step of the decode reduce
// (csrc/tpc/block_fp8_framework/reduce_bias.c:42-57) applied to an fp32
// partial [rows][width] -- a K-range GEMM's output, or the rank sum of the
// shards' partials.
//
// Both are HBM-bound streaming kernels: each lane owns four consecutive
// values (one 16-byte load per slice when the buffers allow it).

#include "gk_fp8_internal.h"

namespace gk {

namespace {

template <bool BF16>
__device__ inline void load4(const void* base, int64_t i, bool vec, int n, float v[4]) {
  if (BF16) {
    const uint16_t* p = static_cast<const uint16_t*>(base) + i;
    if (vec) {
      const uint2 u = *reinterpret_cast<const uint2*>(p);
      v[0] = bits_f32(u.x << 16); v[1] = bits_f32(u.x & 0xffff0000u);
      v[2] = bits_f32(u.y << 16); v[3] = bits_f32(u.y & 0xffff0000u);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = e < n ? bf16_value(p[e]) : 0.0f;
    }
  } else {
    const float* p = static_cast<const float*>(base) + i;
    if (vec) {
      const v4f u = *reinterpret_cast<const v4f*>(p);
      v[0] = u[0]; v[1] = u[1]; v[2] = u[2]; v[3] = u[3];
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = e < n ? p[e] : 0.0f;
    }
  }
}

// VEC: elems % 4 == 0 and both buffers aligned for 4-value loads and stores.
template <bool BF16, bool VEC>
__global__ __launch_bounds__(256) void rank_sum_kernel(const void* __restrict__ gathered, void* __restrict__ dst,
                                                       int64_t elems, int world) {
  const int64_t quads = (elems + 3) / 4;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t qi = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; qi < quads; qi += step) {
    const int64_t i = qi * 4;
    const int n = static_cast<int>(min<int64_t>(4, elems - i));
    float acc[4];
    load4<BF16>(gathered, i, VEC, n, acc);
    for (int r = 1; r < world; ++r) {
      float v[4];
      load4<BF16>(gathered, static_cast<int64_t>(r) * elems + i, VEC, n, v);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = add_rn(acc[e], v[e]);
    }
    if (BF16) {
      uint16_t* out = static_cast<uint16_t*>(dst) + i;
      if (VEC) {
        *reinterpret_cast<uint2*>(out) =
            make_uint2(bf16x2_rne(acc[0], acc[1]), bf16x2_rne(acc[2], acc[3]));
      } else {
        for (int e = 0; e < n; ++e) out[e] = bf16_rne(acc[e]);
      }
    } else {
      float* out = static_cast<float*>(dst) + i;
      if (VEC) {
        *reinterpret_cast<v4f*>(out) = v4f{acc[0], acc[1], acc[2], acc[3]};
      } else {
        for (int e = 0; e < n; ++e) out[e] = acc[e];
      }
    }
  }
}

__global__ __launch_bounds__(256) void partial_finish_kernel(const float* __restrict__ p, int64_t ldp, int rows,
                                                             int width, const float* __restrict__ bias,
                                                             uint16_t* __restrict__ y, int64_t ldy) {
  const int64_t total = static_cast<int64_t>(rows) * width;
  const int64_t step = static_cast<int64_t>(gridDim.x) * blockDim.x;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += step) {
    const int64_t r = i / width, c = i - r * width;
    const float b = bias ? bias[c] : 0.0f;
    y[r * ldy + c] = bf16_rne(add_rn(p[r * ldp + c], b));
  }
}

unsigned grid_for(int64_t items) {
  // enough workgroups to cover the items once, at most 8 per CU
  const int64_t wgs = (items + 255) / 256;
  return static_cast<unsigned>(wgs < 2048 ? (wgs > 0 ? wgs : 1) : 2048);
}

}  // namespace

hipError_t launch_rank_sum(const void* gathered, void* dst, int64_t elems, int world, bool bf16,
                           hipStream_t stream) {
  const unsigned grid = grid_for((elems + 3) / 4);
  const uintptr_t align = bf16 ? 7 : 15;
  const bool vec = elems % 4 == 0 && ((reinterpret_cast<uintptr_t>(gathered) | reinterpret_cast<uintptr_t>(dst)) &
                                      align) == 0;
  if (bf16) {
    if (vec) rank_sum_kernel<true, true><<<grid, 256, 0, stream>>>(gathered, dst, elems, world);
    else rank_sum_kernel<true, false><<<grid, 256, 0, stream>>>(gathered, dst, elems, world);
  } else {
    if (vec) rank_sum_kernel<false, true><<<grid, 256, 0, stream>>>(gathered, dst, elems, world);
    else rank_sum_kernel<false, false><<<grid, 256, 0, stream>>>(gathered, dst, elems, world);
  }
  return hipGetLastError();
}

hipError_t launch_partial_finish(const float* p, int64_t ldp, int rows, int width, const float* bias, uint16_t* y,
                                 int64_t ldy, hipStream_t stream) {
  partial_finish_kernel<<<grid_for(static_cast<int64_t>(rows) * width), 256, 0, stream>>>(p, ldp, rows, width, bias,
                                                                                          y, ldy);
  return hipGetLastError();
}

}  // namespace gk
