// SiLU- and GELU-and-mul on gfx950, plain (bf16 out) and fused with the 1x128
// activation quantizer (codes + scales ready for the down projection).
//
// Semantics of the reference ops gk_silu_and_mul_bf16_v1
// (csrc/tpc/generic_dense/silu_and_mul_bf16.c:16-89, glue
// csrc/host/generic_dense_glue.cpp:196-236) and gk_gelu_and_mul_bf16_v1
// (gelu_and_mul_bf16.c:4-49, glue generic_dense_glue.cpp:424-458): gate_up is
// bf16 [rows, 2W], gate in columns [0, W), up in [W, 2W); out[r, c] =
// bf16(act(g) * u) with the product computed in fp32 and rounded once
// (silu_ref, gelu_erf_ref, gelu_tanh_ref in gk_fp8_math.h).
//
// The fused ops quantize those bf16 products per 1x128 group exactly as the
// activation quantizer does (quant_group8), so their codes equal
// act_quant(act_and_mul(gate_up)) bit for bit; columns past W are zero.

#include "gk_fp8_internal.h"

namespace gk {

namespace {

// Gated activations: out = bf16(act(gate) * up), the product in fp32 (act_mul_pair).
template <int ACT>
__device__ inline uint16_t act_mul_one(uint16_t g, uint16_t u) {
  return bf16_rne(mul_rn(act_ref<ACT>(bf16_value(g)), bf16_value(u)));
}

// One thread per 8 output columns; the vector path needs 16-byte aligned rows.
template <int ACT>
__global__ __launch_bounds__(256) void act_and_mul_kernel(const uint16_t* __restrict__ in, int64_t ldi, int rows,
                                                           int width, uint16_t* __restrict__ out, int64_t ldo,
                                                           int vec_ok) {
  const int per_row = (width + 7) / 8;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(rows) * per_row) return;
  const int64_t r = i / per_row;
  const int c = static_cast<int>(i - r * per_row) * 8;
  const uint16_t* g = in + r * ldi + c;
  const uint16_t* u = g + width;
  uint16_t* o = out + r * ldo + c;
  if (vec_ok && c + 8 <= width) {
    const uint4 gv = *reinterpret_cast<const uint4*>(g), uv = *reinterpret_cast<const uint4*>(u);
    *reinterpret_cast<uint4*>(o) = make_uint4(act_mul_pair<ACT>(gv.x, uv.x), act_mul_pair<ACT>(gv.y, uv.y),
                                              act_mul_pair<ACT>(gv.z, uv.z), act_mul_pair<ACT>(gv.w, uv.w));
  } else {
    for (int j = 0; j < 8 && c + j < width; ++j) o[j] = act_mul_one<ACT>(g[j], u[j]);
  }
}

// Fused: 16 lanes per (row, 128-column group), 8 columns per lane.  Output as
// act_quant_kernel: group-major q [G][Mpad][128] / sa [G][Mpad] (rows >= rows
// zero) or, PACKED, the decode fragment layout (Mpad = 16, 32 or 64).
template <int ACT, bool HALF, bool PACKED>
__global__ __launch_bounds__(256) void act_mul_quant_kernel(const uint16_t* __restrict__ in, int64_t ldi, int rows,
                                                             int width, int G, int Mpad, uint8_t* __restrict__ q,
                                                             float* __restrict__ sa, int vec_ok) {
  const int64_t gid = static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 4) + (threadIdx.x >> 4);
  const int sub = threadIdx.x & 15;
  const int64_t total = static_cast<int64_t>(Mpad) * G;
  const bool active = gid < total;
  const int64_t row = active ? gid / G : 0;
  const int g = active ? static_cast<int>(gid - row * G) : 0;
  const int col = g * 128 + sub * 8;
  const bool live = active && row < rows;
  uint4 raw = make_uint4(0u, 0u, 0u, 0u);
  if (live) {
    const uint16_t* gp = in + row * ldi + col;
    const uint16_t* up = gp + width;
    if (vec_ok && col + 8 <= width) {
      const uint4 gv = *reinterpret_cast<const uint4*>(gp), uv = *reinterpret_cast<const uint4*>(up);
      raw = make_uint4(act_mul_pair<ACT>(gv.x, uv.x), act_mul_pair<ACT>(gv.y, uv.y),
                       act_mul_pair<ACT>(gv.z, uv.z), act_mul_pair<ACT>(gv.w, uv.w));
    } else {
      uint32_t h[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) h[j] = (col + j < width) ? act_mul_one<ACT>(gp[j], up[j]) : 0u;
      raw = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
    }
  }
  float s;
  const uint2 codes = quant_group8(raw, live, HALF, &s);  // all 16 lanes of a group take part
  if (active) {
    const int64_t slot = static_cast<int64_t>(g) * Mpad + row;
    const int64_t at = PACKED ? decode_layout_offset(g, row, 8 * sub, Mpad) : slot * 128 + sub * 8;
    *reinterpret_cast<uint2*>(q + at) = live ? codes : make_uint2(0u, 0u);
    if (sub == 0) sa[slot] = live ? s : 0.0f;
  }
}

}  // namespace

namespace {

template <int ACT>
hipError_t launch_act_and_mul(const uint16_t* in, int64_t ldi, int rows, int width, uint16_t* out, int64_t ldo,
                              hipStream_t stream) {
  const int vec_ok = (((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0) &&
                     ldi % 8 == 0 && ldo % 8 == 0 && width % 8 == 0;
  const int64_t n = static_cast<int64_t>(rows) * ((width + 7) / 8);
  act_and_mul_kernel<ACT><<<static_cast<unsigned>((n + 255) / 256), 256, 0, stream>>>(in, ldi, rows, width, out,
                                                                                       ldo, vec_ok);
  return hipGetLastError();
}

template <int ACT>
hipError_t launch_act_mul_quant(const uint16_t* in, int64_t ldi, int rows, int width, int Mpad, uint8_t* q,
                                float* sa, bool half, bool packed, hipStream_t stream) {
  if (packed && Mpad != 16 && Mpad != 32 && Mpad != 64) return hipErrorInvalidValue;
  const int G = (width + 127) / 128;
  const int64_t groups = static_cast<int64_t>(Mpad) * G;
  const unsigned blocks = static_cast<unsigned>((groups + 15) / 16);
  const int vec_ok = ((reinterpret_cast<uintptr_t>(in) & 15) == 0) && ldi % 8 == 0 && width % 8 == 0;
#define GK_AMQ(H, P) \
  act_mul_quant_kernel<ACT, H, P><<<blocks, 256, 0, stream>>>(in, ldi, rows, width, G, Mpad, q, sa, vec_ok)
  if (half) {
    if (packed) GK_AMQ(true, true); else GK_AMQ(true, false);
  } else {
    if (packed) GK_AMQ(false, true); else GK_AMQ(false, false);
  }
#undef GK_AMQ
  return hipGetLastError();
}

}  // namespace

hipError_t launch_silu_and_mul(const uint16_t* in, int64_t ldi, int rows, int width, uint16_t* out, int64_t ldo,
                               hipStream_t stream) {
  return launch_act_and_mul<kSilu>(in, ldi, rows, width, out, ldo, stream);
}

hipError_t launch_silu_mul_act_quant(const uint16_t* in, int64_t ldi, int rows, int width, int Mpad, uint8_t* q,
                                     float* sa, bool half, bool packed, hipStream_t stream) {
  return launch_act_mul_quant<kSilu>(in, ldi, rows, width, Mpad, q, sa, half, packed, stream);
}

hipError_t launch_gelu_and_mul(const uint16_t* in, int64_t ldi, int rows, int width, uint16_t* out, int64_t ldo,
                               bool approximate, hipStream_t stream) {
  return approximate ? launch_act_and_mul<kGeluTanh>(in, ldi, rows, width, out, ldo, stream)
                     : launch_act_and_mul<kGeluErf>(in, ldi, rows, width, out, ldo, stream);
}

hipError_t launch_gelu_mul_act_quant(const uint16_t* in, int64_t ldi, int rows, int width, bool approximate,
                                     int Mpad, uint8_t* q, float* sa, bool half, bool packed, hipStream_t stream) {
  return approximate ? launch_act_mul_quant<kGeluTanh>(in, ldi, rows, width, Mpad, q, sa, half, packed, stream)
                     : launch_act_mul_quant<kGeluErf>(in, ldi, rows, width, Mpad, q, sa, half, packed, stream);
}

}  // namespace gk
