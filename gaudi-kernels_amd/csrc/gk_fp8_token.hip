// Per-token activation quantization and the per-channel epilogue of the
// reference's per-token / per-channel W8A8 path, on gfx950.
//
// token quant (csrc/tpc/block_fp8_framework/activation_token.c:4-26, helpers
// activation_quant_common.h:3-30): one scale per row,
//   m     = max |x| over the row (1 where the row is all zero),
//   s     = fp8_activation_scale(m) = fma(fma(-s0, 448, m), 1/448, s0), s0 = m * (1/448),
//   z     = fma(fma(-q0, s, x), r, q0), q0 = x * r, r = 1/s   (the refined quotient),
//   code  = E4M3 round-to-nearest-even of min(|z|, 448) with x's sign, then halved
//           into the Gaudi2 half range (codec_half4: value / 2, RNE on its grid),
//   scale = 2 s stored per row.
// The reciprocal here is the IEEE one (the TPC reciprocal instruction's exact
// rounding is not documented in the reference).  On gfx950 the encode is
// v_cvt_pk_fp8_f32 (equal to the software RNE encoder for |v| <= 464).
//
// channel finish (channel_finish.c:2-18): y[r][c] = bf16(fma(p[r][c] * a[r], w[c], b[c])).

#include "gk_fp8_tile.h"

namespace gk {

namespace {

constexpr int kTokThreads = 256;

__device__ inline uint4 token_load8(const uint16_t* xr, int c, int vec_ok) {
  if (vec_ok) return *reinterpret_cast<const uint4*>(xr + c);
  uint32_t h[8];
  for (int j = 0; j < 8; ++j) h[j] = xr[c + j];
  return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
}

// One workgroup per row.  Rows of up to kTokKeep * 2048 elements stay in
// registers between the max and the quantization (one read of x); wider
// rows are read again for the second pass.
constexpr int kTokKeep = 4;

__global__ __launch_bounds__(kTokThreads) void token_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                                  int width, uint8_t* __restrict__ q, int64_t ldq,
                                                                  float* __restrict__ scales, int vec_ok) {
  __shared__ float wmax[kTokThreads / 64];
  const int row = blockIdx.x, tid = threadIdx.x;
  const uint16_t* xr = x + static_cast<int64_t>(row) * ldx;
  constexpr int kStep = kTokThreads * 8;
  const bool keep = width <= kTokKeep * kStep;
  uint4 held[kTokKeep];
  float m = 0.0f;
  if (keep) {
#pragma unroll
    for (int p = 0; p < kTokKeep; ++p) {
      const int c = tid * 8 + p * kStep;
      held[p] = make_uint4(0u, 0u, 0u, 0u);
      if (c < width) {
        held[p] = token_load8(xr, c, vec_ok);
        m = abs_max8(m, held[p]);
      }
    }
  } else {
    for (int c = tid * 8; c < width; c += kStep) m = abs_max8(m, token_load8(xr, c, vec_ok));
  }
  // |x| are non-negative: the maximum over 16 lanes in DPP steps, then across the 4 rows of 16 and the waves
  m = __uint_as_float(row_max16_bits(m));
  m = fmaxf(m, __shfl_xor(m, 16, 64));
  m = fmaxf(m, __shfl_xor(m, 32, 64));
  if ((tid & 63) == 0) wmax[tid >> 6] = m;
  __syncthreads();
  m = wmax[0];
#pragma unroll
  for (int i = 1; i < kTokThreads / 64; ++i) m = fmaxf(m, wmax[i]);
  if (m == 0.0f) m = 1.0f;  // only an all-zero token needs a substitute denominator (activation_token.c:16)
  const float s = token_scale(m);
  const float r = 1.0f / s;
  uint8_t* qr = q + static_cast<int64_t>(row) * ldq;
  if (keep) {
#pragma unroll
    for (int p = 0; p < kTokKeep; ++p) {
      const int c = tid * 8 + p * kStep;
      if (c < width) *reinterpret_cast<uint2*>(qr + c) = token_codes8(held[p], s, r);
    }
  } else {
    for (int c = tid * 8; c < width; c += kStep)
      *reinterpret_cast<uint2*>(qr + c) = token_codes8(token_load8(xr, c, vec_ok), s, r);
  }
  if (tid == 0) scales[row] = 2.0f * s;
}

__global__ __launch_bounds__(256) void channel_finish_kernel(const float* __restrict__ p, int64_t ldp, int rows,
                                                             int width, const float* __restrict__ a,
                                                             const float* __restrict__ w, const float* __restrict__ b,
                                                             uint16_t* __restrict__ y, int64_t ldy) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(rows) * width) return;
  const int64_t r = i / width;
  const int c = static_cast<int>(i - r * width);
  y[r * ldy + c] = channel_out(p[r * ldp + c], a[r], w[c], b ? b[c] : 0.0f);
}

}  // namespace

hipError_t launch_token_quant(const uint16_t* x, int64_t ldx, int rows, int width, uint8_t* q, int64_t ldq,
                              float* scales, hipStream_t stream) {
  const int vec_ok = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && ldx % 8 == 0;
  token_quant_kernel<<<rows, kTokThreads, 0, stream>>>(x, ldx, width, q, ldq, scales, vec_ok);
  return hipGetLastError();
}

hipError_t launch_channel_finish(const float* partial, int64_t ldp, int rows, int width, const float* act_scales,
                                 const float* w_scales, const float* bias, uint16_t* y, int64_t ldy,
                                 hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(rows) * width;
  channel_finish_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, stream>>>(partial, ldp, rows, width,
                                                                                     act_scales, w_scales, bias, y,
                                                                                     ldy);
  return hipGetLastError();
}

}  // namespace gk
