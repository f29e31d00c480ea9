// RMSNorm on gfx950: the reference ops gk_rms_norm_bf16_v1
// (csrc/tpc/generic_dense/rms_norm_bf16.c:4-53) and
// gk_fused_add_rms_norm_bf16_v1 (fused_add_rms_norm_bf16.c:4-63), bf16 out,
// and both fused with the 1x128 activation quantizer (codes + scales ready
// for the block-FP8 GEMM that consumes the normalized rows).
//
// Per row (one workgroup of 256 threads; thread t holds the 8-element chunks
// t, t + 256, ... in registers, at most four for width <= 8192):
//   add        r = bf16_rne(fp32(x) + fp32(residual))  (fused form; residual_out = r)
//   sum        ss = fp32 of the fp64 sum of r*r: each square is exact in
//              fp64; thread t adds its chunks' squares in element order; each
//              wave folds its 64 partial sums pairwise (lane l += lane l + s,
//              s = 32 .. 1, by butterfly shuffles), and the four wave sums are
//              folded the same way (s = 2, 1).
//   inverse    inv = fp32(1 / sqrt(fp64(ss * fp32(1/width) + eps))), the
//              multiply and the add in fp32 as the reference's expression
//              (rms_norm_bf16.c:24-25), then an fp64 square root and division
//              rounded once; an argument of +inf gives 0 (norm_math.h:22).
//   normalize  bf16_rne((r * inv) * (gamma + weight_offset)), fp32, no FMA.
// The reference joins fp32 lane sums with a compensated reduction and
// refines a hardware rsqrt (norm_math.h:5-23); both target the correctly
// rounded values that the fp64 steps here give.  The CPU restatement
// (oracle/norm.py) follows the same order, so the outputs are compared bit
// for bit, and against the reference test's own gate (2 bf16 ulps of an
// fp64 evaluation, tests/track_a_device_verify.cpp:490-540).
//
// QUANT: the normalized bf16 values are quantized per 1x128 group by
// quant_group8 -- the 16 lanes of a DPP row hold chunks 16j .. 16j + 15 of
// the row, i.e. exactly one group -- into the standard layout q [G][Mpad][128]
// / sa [G][Mpad] or the decode fragment layout, so the codes equal
// act_quant(norm_out) bit for bit.  Rows in [rows, Mpad) and columns past
// the width are written as zero, as the standalone quantizer does.

#include "gk_fp8_internal.h"

namespace gk {

namespace {

constexpr int kNormThreads = 256;
constexpr int kNormPasses = kNormMaxWidth / (8 * kNormThreads);  // 4

__device__ inline float lo_bf16(uint32_t w) { return bits_f32(w << 16); }
__device__ inline float hi_bf16(uint32_t w) { return bits_f32(w & 0xffff0000u); }

// 8 bf16 values of a row starting at column c (columns >= width read as 0).
template <bool VEC>
__device__ inline uint4 load8(const uint16_t* row, int c, int width) {
  if (VEC && c + 8 <= width) return *reinterpret_cast<const uint4*>(row + c);
  uint32_t h[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) h[j] = (c + j < width) ? row[c + j] : 0u;
  return make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
}

template <bool VEC>
__device__ inline void store8(uint16_t* row, int c, int width, uint4 v) {
  if (VEC && c + 8 <= width) {
    *reinterpret_cast<uint4*>(row + c) = v;
    return;
  }
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int j = 0; j < 8; ++j)
    if (c + j < width) row[c + j] = static_cast<uint16_t>(j & 1 ? w[j >> 1] >> 16 : w[j >> 1] & 0xffffu);
}

__device__ inline uint32_t add_pair(uint32_t a, uint32_t b) {
  return bf16x2_rne(add_rn(lo_bf16(a), lo_bf16(b)), add_rn(hi_bf16(a), hi_bf16(b)));
}

__device__ inline uint32_t norm_pair(uint32_t v, uint32_t g, float inv, float off) {
  const float n0 = mul_rn(mul_rn(lo_bf16(v), inv), add_rn(lo_bf16(g), off));
  const float n1 = mul_rn(mul_rn(hi_bf16(v), inv), add_rn(hi_bf16(g), off));
  return bf16x2_rne(n0, n1);
}

template <bool ADD, bool QUANT, bool HALF, bool PACKED, bool VEC>
__global__ __launch_bounds__(kNormThreads) void rms_norm_kernel(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ res, int64_t ld_in, const uint16_t* __restrict__ gamma,
    int rows, int width, float eps, float off, uint16_t* __restrict__ res_out, uint16_t* __restrict__ norm_out,
    int64_t ld_out, uint8_t* __restrict__ q, float* __restrict__ sa, int Mpad) {
  __shared__ double wsum[kNormThreads / 64];
  const int t = threadIdx.x;
  const int row = blockIdx.x;
  const int G = (width + 127) >> 7;
  const bool live = row < rows;  // QUANT grids cover Mpad rows; rows past `rows` write zeros
  uint4 v[kNormPasses], gv[kNormPasses];
  double acc = 0.0;
#pragma unroll
  for (int p = 0; p < kNormPasses; ++p) {
    const int c = 8 * (t + kNormThreads * p);
    v[p] = make_uint4(0u, 0u, 0u, 0u);
    gv[p] = make_uint4(0u, 0u, 0u, 0u);
    if (live && c < width) {
      gv[p] = load8<VEC>(gamma, c, width);  // issued with the row loads: no second round trip later
      const uint16_t* xr = x + static_cast<int64_t>(row) * ld_in;
      uint4 a = load8<VEC>(xr, c, width);
      if (ADD) {
        const uint4 b = load8<VEC>(res + static_cast<int64_t>(row) * ld_in, c, width);
        a = make_uint4(add_pair(a.x, b.x), add_pair(a.y, b.y), add_pair(a.z, b.z), add_pair(a.w, b.w));
        if (res_out) store8<VEC>(res_out + static_cast<int64_t>(row) * ld_out, c, width, a);
      }
      v[p] = a;
      // element order within the chunk: 0, 1, ..., 7 (a bf16 square is exact
      // in fp64, so a contracted fma gives the same sums)
      acc += static_cast<double>(lo_bf16(a.x)) * lo_bf16(a.x);
      acc += static_cast<double>(hi_bf16(a.x)) * hi_bf16(a.x);
      acc += static_cast<double>(lo_bf16(a.y)) * lo_bf16(a.y);
      acc += static_cast<double>(hi_bf16(a.y)) * hi_bf16(a.y);
      acc += static_cast<double>(lo_bf16(a.z)) * lo_bf16(a.z);
      acc += static_cast<double>(hi_bf16(a.z)) * hi_bf16(a.z);
      acc += static_cast<double>(lo_bf16(a.w)) * lo_bf16(a.w);
      acc += static_cast<double>(hi_bf16(a.w)) * hi_bf16(a.w);
    }
  }
  // lane l takes acc(l) + acc(l ^ s): on lane 0 this is the pairwise fold
#pragma unroll
  for (int s = 32; s >= 1; s >>= 1) acc = acc + __shfl_xor(acc, s, 64);
  if ((t & 63) == 0) wsum[t >> 6] = acc;
  __syncthreads();
  const float ss = static_cast<float>((wsum[0] + wsum[2]) + (wsum[1] + wsum[3]));
  const float arg = add_rn(mul_rn(ss, 1.0f / static_cast<float>(width)), eps);
  const float inv = arg == __builtin_inff() ? 0.0f : static_cast<float>(1.0 / sqrt(static_cast<double>(arg)));

#pragma unroll
  for (int p = 0; p < kNormPasses; ++p) {
    const int chunk = t + kNormThreads * p;
    const int c = 8 * chunk;
    uint4 n = make_uint4(0u, 0u, 0u, 0u);
    if (live && c < width) {
      const uint4 g = gv[p];
      n = make_uint4(norm_pair(v[p].x, g.x, inv, off), norm_pair(v[p].y, g.y, inv, off),
                     norm_pair(v[p].z, g.z, inv, off), norm_pair(v[p].w, g.w, inv, off));
      if (norm_out) store8<VEC>(norm_out + static_cast<int64_t>(row) * ld_out, c, width, n);
      if (c + 8 > width) {  // columns past the width are zero for the quantizer
        const int keep = width - c;
        uint32_t w[4] = {n.x, n.y, n.z, n.w};
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (j >= keep) w[j >> 1] &= (j & 1) ? 0x0000ffffu : 0xffff0000u;
        n = make_uint4(w[0], w[1], w[2], w[3]);
      }
    }
    if (QUANT && 8 * kNormThreads * p < width) {
      // The 16 lanes of this DPP row hold one 128-column group; groups past
      // the last are not stored.  quant_group8 runs on every lane of the
      // workgroup (the condition is uniform).
      const int g = chunk >> 4, sub = chunk & 15;
      float s;
      const uint2 codes = quant_group8(n, live, HALF, &s);
      if (g < G) {
        const int64_t slot = static_cast<int64_t>(g) * Mpad + row;
        const int64_t at = PACKED ? decode_layout_offset(g, row, 8 * sub, Mpad) : slot * 128 + sub * 8;
        *reinterpret_cast<uint2*>(q + at) = live ? codes : make_uint2(0u, 0u);
        if (sub == 0) sa[slot] = live ? s : 0.0f;
      }
    }
  }
}

}  // namespace

hipError_t launch_rms_norm(const uint16_t* x, const uint16_t* res, int64_t ld_in, const uint16_t* gamma, int rows,
                           int width, float eps, float off, uint16_t* res_out, uint16_t* norm_out, int64_t ld_out,
                           uint8_t* q, float* sa, int Mpad, bool half, bool packed, hipStream_t stream) {
  if (width < 1 || width > kNormMaxWidth || rows < 1) return hipErrorInvalidValue;
  const bool quant = q != nullptr;
  if (quant && (Mpad < rows || (packed && Mpad != 16 && Mpad != 32 && Mpad != 64))) return hipErrorInvalidValue;
  auto al16 = [](const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; };
  const bool vec = al16(x) && (!res || al16(res)) && al16(gamma) && (!res_out || al16(res_out)) &&
                   (!norm_out || al16(norm_out)) && ld_in % 8 == 0 && ld_out % 8 == 0;
  const unsigned grid = static_cast<unsigned>(quant ? Mpad : rows);
#define GK_NORM(A, Q, H, P, V)                                                                             \
  rms_norm_kernel<A, Q, H, P, V><<<grid, kNormThreads, 0, stream>>>(x, res, ld_in, gamma, rows, width, eps, off, \
                                                                     res_out, norm_out, ld_out, q, sa, Mpad)
#define GK_NORM_V(A, Q, H, P) \
  if (vec) GK_NORM(A, Q, H, P, true); else GK_NORM(A, Q, H, P, false)
#define GK_NORM_Q(A)                                       \
  if (!quant) { GK_NORM_V(A, false, false, false); }       \
  else if (half) { if (packed) { GK_NORM_V(A, true, true, true); } else { GK_NORM_V(A, true, true, false); } } \
  else { if (packed) { GK_NORM_V(A, true, false, true); } else { GK_NORM_V(A, true, false, false); } }
  if (res) {
    GK_NORM_Q(true);
  } else {
    GK_NORM_Q(false);
  }
#undef GK_NORM_Q
#undef GK_NORM_V
#undef GK_NORM
  return hipGetLastError();
}

}  // namespace gk
