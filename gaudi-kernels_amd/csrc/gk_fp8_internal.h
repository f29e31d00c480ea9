// Internal declarations shared by the kernel translation units and the C-ABI
// layer.  Not part of the public interface (that is include/gk_fp8.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gk_fp8_math.h"
#include "gk_fp8_plan.h"

namespace gk {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// bf16_rne(a) | bf16_rne(b) << 16 with gfx950's v_cvt_pk_bf16_f32: it rounds
// to nearest even and keeps denormals, equal to bf16_rne for every non-NaN
// float (all 2^32 inputs: gk_probe_bf16x2_check), but keeps NaN payloads, so
// NaN inputs get bf16_rne's canonical 0x7fc0 afterwards, on the integer
// result (a select on the float inputs could be folded away: fptrunc does not
// define NaN payloads).  About 2.5 instructions a value instead of 6.
__device__ inline uint32_t bf16x2_rne(float a, float b) {
  const f32x2 v = {a, b};
  uint32_t h = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  h = a != a ? (h & 0xffff0000u) | 0x7fc0u : h;
  h = b != b ? (h & 0x0000ffffu) | 0x7fc00000u : h;
  return h;
}

// Gated activations: bf16(act(gate) * up) on two packed bf16 pairs, the
// product in fp32 -- the reference's fused SiLU-and-mul
// (csrc/tpc/generic_dense/silu_and_mul_bf16.c:4-15), whose only rounding is
// the final product, and its GELU forms.  Shared by the separate gated
// activation kernels and the grouped GEMM's fused SiLU-and-mul epilogue, so
// both give the same bits.
enum Act { kSilu = 0, kGeluErf = 1, kGeluTanh = 2 };

template <int ACT>
__device__ inline float act_ref(float g) {
  return ACT == kSilu ? silu_ref(g) : ACT == kGeluErf ? gelu_erf_ref(g) : gelu_tanh_ref(g);
}

template <int ACT>
__device__ inline uint32_t act_mul_pair(uint32_t g2, uint32_t u2) {
  const float g0 = bits_f32(g2 << 16), g1 = bits_f32(g2 & 0xffff0000u);
  const float u0 = bits_f32(u2 << 16), u1 = bits_f32(u2 & 0xffff0000u);
  return bf16x2_rne(mul_rn(act_ref<ACT>(g0), u0), mul_rn(act_ref<ACT>(g1), u1));
}

// Row padding of the quantized-activation workspace.
constexpr int kDecodeMaxRows = 16;   // one MFMA column tile of tokens (the fused quantizer, per-channel decode)
constexpr int kDecodeMaxTokens = 64;  // decode variant: M <= 64 in 1, 2 or 4 column tiles (Mpad = 16, 32, 64)
// Token tiles of the decode variant for M tokens (Mpad = 16 * decode_tiles(M)).
inline int decode_tiles(int64_t M) { return M <= 16 ? 1 : M <= 32 ? 2 : 4; }
// Offset of codes byte `e` (0..127) of token `row` in group g of the decode fragment layout with Mpad rows:
// block (g, row / 16) of 2 KB, piece (h, l) = ((e / 16) & 1, 16 (e / 32) + row % 16), byte e % 16.
__host__ __device__ inline int64_t decode_layout_offset(int g, int64_t row, int e, int Mpad) {
  return (static_cast<int64_t>(g) * (Mpad >> 4) + (row >> 4)) * 2048 + ((e >> 4) & 1) * 1024 +
         (16 * (e >> 5) + (row & 15)) * 16 + (e & 15);
}
constexpr int kPrefillRowTile = 256; // prefill variant: M padded to the token tile

// Maximum over the 16 lanes of a DPP row (lanes 16r .. 16r+15) of
// non-negative floats, in VALU data-parallel moves: xor 1 and xor 2
// (quad_perm), then the half-row and row mirrors pair quads 0-1 / 2-3 and the
// two halves.  Non-negative floats order as their bit patterns, so each step
// is one unsigned max with a DPP operand (v_max_u32_dpp: no separate move and
// no NaN canonicalization, which an fmaxf on a moved value costs).  An
// inactive source lane reads as 0 (bound_ctrl), the identity of the maximum.
// The maximum does not depend on the order.  Returns the bit pattern.
template <int CTRL>
__device__ inline uint32_t dpp_umax(uint32_t v) {
  const uint32_t o =
      static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xf, 0xf, true));
  return v > o ? v : o;
}
__device__ inline uint32_t row_max16_bits(float v) {  // v >= +0
  uint32_t b = __float_as_uint(v);
  b = dpp_umax<0xB1>(b);   // quad_perm [1,0,3,2]
  b = dpp_umax<0x4E>(b);   // quad_perm [2,3,0,1]
  b = dpp_umax<0x141>(b);  // row_half_mirror
  return dpp_umax<0x140>(b);  // row_mirror
}

// ---- 1x128 activation quantizer (block_fp8_oracle.py:25-28, :32,:34) -------
// Sixteen consecutive lanes own one 128-element group, 8 bf16 each (one
// 16-byte load).  Returns the lane's 8 OCP E4M3 codes (byte i = element i)
// and writes the group's scale (x2 in native_half mode).  amax is reduced
// over the 16 lanes (one DPP row, row_max16_bits); the fp32 quotient is act_quotient
// (exact E4M3 codes of the IEEE quotient); the encode is the gfx950
// v_cvt_pk_fp8_f32 (round to nearest even, OCP E4M3FN), which equals
// e4m3_rne for every |v| <= 464 (checked on all of them by
// gk_probe_e4m3_check) -- and |x / s| < 464 always holds because
// s >= amax/448 up to two fp32 roundings.
__device__ inline uint2 quant_group8(uint4 raw, bool live, bool half, float* scale_out) {
  float v[8];
  const uint32_t w4[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = live ? bits_f32(w4[i] << 16) : 0.0f;
    v[2 * i + 1] = live ? bits_f32(w4[i] & 0xffff0000u) : 0.0f;
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  // act_scale(amax) with the 1e-10 floor taken on the bit pattern (amax >= +0)
  const uint32_t amax_bits = row_max16_bits(amax);
  const float s = __uint_as_float(max(amax_bits, __float_as_uint(1e-10f))) * (1.0f / 448.0f);
  // 1/s: the hardware reciprocal (1 ulp) refined by one Newton step, which
  // leaves r within one ulp of fp32(1/s); act_quotient is exact for any such r
  const float r0 = __builtin_amdgcn_rcpf(s);
  const float r = fmaf(fmaf(-s, r0, 1.0f), r0, r0);
  float q[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) q[i] = act_quotient(v[i], s, r);
  int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
  lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
  int hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
  hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
  uint2 codes = make_uint2(static_cast<uint32_t>(lo), static_cast<uint32_t>(hi));
  if (half) {  // block_fp8_oracle.py:32,34: e4m3fn(qa * 0.5), sa * 2
    codes.x = codec_half4(codes.x);
    codes.y = codec_half4(codes.y);
  }
  *scale_out = half ? s * 2.0f : s;
  return codes;
}

hipError_t launch_codec(bool forward, const uint8_t* src, uint8_t* dst, int64_t n, const float* scales,
                        float* scales_out, int64_t n_scales, uint32_t* flags, unsigned long long* rounded,
                        hipStream_t stream);

// Fragment-packed weights: for 16-row tile t and group g a 2 KB block at
// (t * G + g) * 2048; piece (h, l) at h*1024 + 16 l = bytes [128 g + 32 (l/16)
// + 16 h, +16) of row 16 t + l%16, zeros past N.  K % 128 == 0.
// Per-token quantizer arithmetic (activation_token.c:4-26, activation_quant_common.h:3-30),
// shared by the token quantizer and the decode kernel's fused per-token form.
__device__ inline float token_scale(float m) {  // activation_quant_common.h:3-7
  const float inv448 = 1.0f / 448.0f;
  const float s0 = mul_rn(m, inv448);
  const float res = fmaf(-s0, 448.0f, m);
  return fmaf(res, inv448, s0);
}

// 8 bf16 values -> 8 half-range codes (as two packed dwords).
__device__ inline uint2 token_codes8(uint4 raw, float s, float r) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
  uint32_t out[2] = {0u, 0u};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float z[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float x = bits_f32(h ? (w[i] & 0xffff0000u) : (w[i] << 16));
      const float q0 = mul_rn(x, r);
      const float zz = fmaf(fmaf(-q0, s, x), r, q0);
      z[h] = copysignf(fminf(fabsf(zz), 448.0f), x);
    }
    const uint32_t two = __builtin_amdgcn_cvt_pk_fp8_f32(z[0], z[1], 0, false) & 0xffffu;
    out[i >> 1] |= two << ((i & 1) * 16);
  }
  return make_uint2(codec_half4(out[0]), codec_half4(out[1]));
}

__device__ inline float abs_max8(float m, uint4 v) {
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) m = fmaxf(m, fmaxf(fabsf(bits_f32(w[i] << 16)), fabsf(bits_f32(w[i] & 0xffff0000u))));
  return m;
}

inline int64_t packed_weight_bytes(int64_t N, int64_t K) { return (N + 15) / 16 * 16 * K; }
hipError_t launch_pack_weight(const uint8_t* w, int N, int K, uint8_t* packed, hipStream_t stream);
hipError_t launch_pack_experts(const uint8_t* w, int E, int N, int K, uint8_t* packed, hipStream_t stream);

// packed: the decode fragment layout (Mpad = 16, 32 or 64): the 2 KB block
// (group g, token tile t) at (g * Mpad/16 + t) * 2048 holds, in its 16-byte
// piece (h, l) at h*1024 + 16 l, bytes [32 (l/16) + 16 h, +16) of row
// 16 t + l%16 (decode_layout_offset).  sa stays [G][Mpad].
hipError_t launch_act_quant(const uint16_t* x, int64_t ldx, int M, int K, int Mpad, uint8_t* q, float* sa,
                            bool half, bool packed, hipStream_t stream);

// RMSNorm of bf16 rows (width <= kNormMaxWidth), optionally fused with a
// residual add (res != nullptr; residual_out written when res_out != nullptr)
// and with the 1x128 quantizer (q != nullptr: codes and scales in the layout
// of launch_act_quant, Mpad rows; norm_out may then be nullptr).
constexpr int kNormMaxWidth = 8192;  // generic_dense_glue.cpp:153
hipError_t launch_rms_norm(const uint16_t* x, const uint16_t* res, int64_t ld_in, const uint16_t* gamma, int rows,
                           int width, float eps, float off, uint16_t* res_out, uint16_t* norm_out, int64_t ld_out,
                           uint8_t* q, float* sa, int Mpad, bool half, bool packed, hipStream_t stream);

// Quantized activations qa [G][Mpad][128] / sa [G][Mpad] (launch_act_quant)
// times weight codes w [N, K] with block scales sw [ceil(N/128), G].
struct GemmArgs {
  const uint8_t* qa;
  const float* sa;
  const uint8_t* w;
  const float* sw;
  const float* bias;  // [N] or nullptr
  uint16_t* y;        // bf16 [M, ldy]
  int64_t ldy;
  int M, N, K, G;
  int Mpad;           // 16 for the decode variant
  bool half_w;        // native_half: half-range codec on weight codes in-kernel, weight scales x2
  DecodeShape dec;    // decode variant only
  bool qpack = false; // decode variant only: qa in the packed decode layout (launch_act_quant packed)
  // Per-token / per-channel scaling (launch_gemm_channel): qa row-major [M][ldq]
  // codes, sa [M] per token, sw [N] per output channel, no per-group promotion.
  bool channel = false;
  int64_t ldq = 0;
  // Weights in the fragment-packed layout of launch_pack_weight (decode and
  // 256 x 256 kernels only).
  bool wpack = false;
  // Decode variant only: qa is the bf16 activation x [M][ldq] (16-byte
  // aligned rows, ldq % 8 == 0), quantized inside the GEMM (sa unused).
  bool xq = false;
  // K range of a larger weight (decode and 256 x 256 kernels, block scaling):
  // w and sw already point at the range's first group, G counts its groups,
  // K stays the weight row stride and gs the groups of the whole row (the
  // scale-grid row stride and, for packed weights, the 16-row tile stride in
  // 2 KB blocks).  0: the whole row (gs = G).
  int gs = 0;
  int gstride() const { return gs > 0 ? gs : G; }
  // fp32 output instead of bf16 y: yp [M][ldyp] = the sum over the K range
  // (+ yp when accumulate), no bias.
  float* yp = nullptr;
  int64_t ldyp = 0;
  bool accumulate = false;
  // Grouped 256 x 256 kernel only: SiLU-and-mul + 1x128 quantization fused into
  // the epilogue.  The weights hold N = 2 * inter rows (gate rows, then up
  // rows); instead of y the kernel writes the codes of bf16(silu(gate) * up)
  // to swiglu_q [inter/128][Mpad][128] and their scales to swiglu_s
  // [inter/128][Mpad] (the layout of launch_act_quant), live rows only.
  uint8_t* swiglu_q = nullptr;
  float* swiglu_s = nullptr;
};

hipError_t launch_gemm_decode(const GemmArgs& a, hipStream_t stream);
hipError_t launch_gemm_prefill(const GemmArgs& a, hipStream_t stream);     // dispatches by M
hipError_t launch_gemm_prefill256(const GemmArgs& a, hipStream_t stream);  // 256 x 256 tiles, Mpad % 256 == 0
// The 256 x 256 kernels address a 256-row weight panel and the whole
// group-major activation array with 32-bit byte offsets.
inline bool prefill256_fits(const GemmArgs& a) {
  return static_cast<int64_t>(a.Mpad) * a.G * 128 <= int64_t{0xffffffff} &&
         static_cast<int64_t>(256) * a.K <= int64_t{0xffffffff};
}
// Grouped (MoE) 256 x 256 GEMM over expert row segments; see gk_fp8_prefill.hip.
// Grouped (MoE) 256 x 256 GEMM over expert row segments (gk_fp8_prefill.hip):
// segment e starts at group_off[e] (multiple of 256) and holds group_cnt[e]
// live rows; 32-row blocks past the live rows are skipped.  yp == nullptr:
// bf16 y; otherwise fp32 planes yp[part][M][N] (a.y unused), one per K part
// (kparts = 1 or 2; 2 splits the groups in halves).  a.swiglu_q: the fused
// SiLU-and-mul quantizer output instead (kparts = 1, no yp, N % 256 == 0).
hipError_t launch_gemm_grouped256(const GemmArgs& a, const int32_t* group_off, const int32_t* group_cnt,
                                  int n_groups, int kparts, float* yp, hipStream_t stream);
hipError_t launch_gemm_generic(const GemmArgs& a, hipStream_t stream);
// Per-token / per-channel GEMM (a.channel): M <= 16 streams weights (decode
// shapes), larger M runs the 256 x 256 kernel in its channel form.
hipError_t launch_gemm_channel(const GemmArgs& a, hipStream_t stream);
// Per-token quantizer fused into the per-channel decode: a.qa = bf16 x [M][a.ldq], M <= 16.
hipError_t launch_gemm_token_channel(const GemmArgs& a, hipStream_t stream);
hipError_t launch_gemm_channel256(const GemmArgs& a, hipStream_t stream);  // gk_fp8_prefill.hip

// ---- row-parallel completion (gk_fp8_reduce.hip) -------------------------------------
// rank_sum.c:4-42: dst[i] = sum over r < world of gathered[r * elems + i] in
// fp32, rank order (bf16: slices widened, one final bf16 rounding).
hipError_t launch_rank_sum(const void* gathered, void* dst, int64_t elems, int world, bool bf16, hipStream_t stream);
// y = bf16(p + bias) on an fp32 partial [rows][width] (bias may be null).
hipError_t launch_partial_finish(const float* p, int64_t ldp, int rows, int width, const float* bias, uint16_t* y,
                                 int64_t ldy, hipStream_t stream);

// ---- per-token activation quantization (gk_fp8_token.hip) ------------------------
// activation_token.c:4-26: q [rows][width] Gaudi2 half-range codes (row-major,
// row stride ldq), scales [rows] = 2 * fp8_activation_scale(row max |x|).
hipError_t launch_token_quant(const uint16_t* x, int64_t ldx, int rows, int width, uint8_t* q, int64_t ldq,
                              float* scales, hipStream_t stream);
// channel_finish.c:2-18 on an fp32 partial [rows][width].
hipError_t launch_channel_finish(const float* partial, int64_t ldp, int rows, int width, const float* act_scales,
                                 const float* w_scales, const float* bias, uint16_t* y, int64_t ldy,
                                 hipStream_t stream);

// ---- SiLU- and GELU-and-mul (gk_fp8_act.hip) ---------------------------------
// in: bf16 [rows, 2*width] (gate | up), row stride ldi; out bf16 [rows, width].
hipError_t launch_silu_and_mul(const uint16_t* in, int64_t ldi, int rows, int width, uint16_t* out, int64_t ldo,
                               hipStream_t stream);
// Fused with the 1x128 quantizer: outputs as launch_act_quant (group-major or packed).
hipError_t launch_silu_mul_act_quant(const uint16_t* in, int64_t ldi, int rows, int width, int Mpad, uint8_t* q,
                                     float* sa, bool half, bool packed, hipStream_t stream);
// GELU-and-mul (approximate: the tanh form), plain and fused, same layouts.
hipError_t launch_gelu_and_mul(const uint16_t* in, int64_t ldi, int rows, int width, uint16_t* out, int64_t ldo,
                               bool approximate, hipStream_t stream);
hipError_t launch_gelu_mul_act_quant(const uint16_t* in, int64_t ldi, int rows, int width, bool approximate,
                                     int Mpad, uint8_t* q, float* sa, bool half, bool packed, hipStream_t stream);

// ---- MoE (gk_fp8_moe.hip) ------------------------------------------------------
// Workspace pieces of one MoE layer call (device pointers).
struct MoeRouting {
  int32_t* ids;        // [T, k] expert of each slot
  float* wts;          // [T, k] combine weight
  int32_t* row_of;     // [T, k] padded row of each slot
  int32_t* row_token;  // [rows_max] token of each padded row, -1 for padding
  int32_t* off;        // [E + 1] padded expert starts (multiples of kMoeRowAlign)
  int32_t* cnt;        // [E] live rows of each expert
};
constexpr int kMoeRowAlign = 256;
constexpr int kMoeMaxExperts = 256;

hipError_t launch_moe_route(const float* logits, int T, int E, int64_t ld_logits, int top_k, int rows_max,
                            const MoeRouting& r, hipStream_t stream);
hipError_t launch_act_quant_rows(const uint16_t* x, int64_t ldx, int K, const int32_t* row_of, int T, int top_k,
                                 int rows, uint8_t* q, float* sa, bool half, hipStream_t stream);
// z: kparts fp32 planes [kparts][rows][H] of the down GEMM; y[t] = bf16(sum_k w_k bf16(sum_p z_p[row])).
hipError_t launch_moe_combine(const float* z, int kparts, int64_t plane, int H, const int32_t* row_of,
                              const float* wts, int T, int top_k, uint16_t* y, int64_t ldy, hipStream_t stream);

}  // namespace gk
