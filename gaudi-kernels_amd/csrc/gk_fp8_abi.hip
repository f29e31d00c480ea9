// C ABI of libgk_fp8.so (declared in include/gk_fp8.h).
//
// Host-side validation, planning and dispatch.  The op table and status
// codes mirror the Synapse provider of the reference
// (csrc/host/generic_dense_glue.cpp:897-1013, generic_fp8_glue.hpp): a static
// name table with a count query, int status codes, no exceptions, and the
// same rejection classes (scale grid mismatch -> INCOMPATIBLE_INPUT_SIZE,
// bad parameters -> UNSUPPORTED_LAYER_CONFIGURATION).  Unlike the glue, which
// runs at graph-compile time, these entry points launch the kernels directly
// on the caller's stream.

#include <hip/hip_runtime.h>

#include <cmath>
#include <cstring>
#include <mutex>

#include "../../include/gk_fp8.h"
#include <algorithm>

#include "gk_fp8_internal.h"

namespace {

constexpr const char* kOps[] = {
    "gk_fp8_codec_ocp_to_half_v1",  // fp8_codec.py:14-53
    "gk_fp8_codec_half_to_ocp_v1",  // inverse codec (build-defined)
    "gk_fp8_act_quant_bf16_v1",     // activation_native.c:9-30 with block_fp8_oracle.py:25-28 numerics
    "gk_fp8_block_gemm_bf16_v1",    // quant -> MME -> reduce_bias.c / prefill chain, fused
    "gk_fp8_block_gemm_q_bf16_v1",  // GEMM on pre-quantized activations
    "gk_fp8_check_inputs_v1",       // block_fp8_oracle.py:22-24
    "gk_fp8_token_quant_bf16_v1",   // activation_token.c:4-26, glue generic_fp8_glue.hpp:31-50
    "gk_fp8_channel_finish_bf16_v1",  // channel_finish.c:2-18, glue generic_fp8_glue.hpp:52-82
    "gk_fp8_channel_gemm_bf16_v1",  // MME + channel finish, fused (build-defined)
    "gk_fp8_token_channel_gemm_bf16_v1",  // token quant + MME + channel finish, fused, M <= 16 (build-defined)
    "gk_silu_and_mul_bf16_v1",      // silu_and_mul_bf16.c, glue generic_dense_glue.cpp:196-236
    "gk_fp8_silu_mul_quant_bf16_v1",  // SiLU-and-mul fused with the 1x128 quantizer (build-defined)
    "gk_gelu_and_mul_bf16_v1",      // gelu_and_mul_bf16.c, glue generic_dense_glue.cpp:424-458
    "gk_fp8_gelu_mul_quant_bf16_v1",  // GELU-and-mul fused with the 1x128 quantizer (build-defined)
    "gk_fp8_moe_route_v1",          // MoE routing + expert-sorted layout (build-defined)
    "gk_fp8_moe_bf16_v2",           // block-FP8 MoE layer (build-defined); v2: packed
                                    // experts are gk_fp8_pack_experts' panel-major layout
    "gk_fp8_pack_weight_v1",        // load-time layout packing (fp8_codec.py:19 "a separate step")
    "gk_fp8_pack_experts_v1",       // the same for the MoE layer's expert weights, panel-major
    "gk_rms_norm_bf16_v1",          // rms_norm_bf16.c, glue generic_dense_glue.cpp:135-190
    "gk_fused_add_rms_norm_bf16_v1",  // fused_add_rms_norm_bf16.c, same glue
    "gk_fp8_rms_norm_quant_bf16_v1",  // (fused add +) RMSNorm fused with the 1x128 quantizer (build-defined)
    "gk_fp8_block_gemm_kslice_f32_v1",  // K range -> fp32 partial (quant_act_fp16_1k col_offset contract)
    "gk_rank_sum_f32_v1",           // rank_sum.c, glue generic_dense_glue.cpp:568-600, 871-895
    "gk_rank_sum_bf16_v1",          // same, bf16 slices
    "gk_fp8_partial_finish_bf16_v1",  // fp32 partial + bias -> bf16 (reduce_bias.c:42-57 final step)
};
constexpr uint32_t kNumOps = sizeof(kOps) / sizeof(kOps[0]);

constexpr uint32_t kKnownFlags = GK_FLAG_NATIVE_HALF | GK_FLAG_FORCE_DECODE | GK_FLAG_FORCE_PREFILL |
                                  GK_FLAG_FORCE_GENERIC | GK_FLAG_WEIGHT_PACKED;
constexpr uint32_t kKsliceFlags = GK_FLAG_NATIVE_HALF | GK_FLAG_FORCE_DECODE | GK_FLAG_FORCE_PREFILL |
                                  GK_FLAG_WEIGHT_PACKED | GK_FLAG_ACCUMULATE;
constexpr size_t kStatusBytes = 256;
constexpr int64_t kMaxDim = (int64_t{1} << 31) - 1;

int64_t round_up(int64_t v, int64_t a) { return (v + a - 1) / a * a; }
size_t align256(size_t v) { return (v + 255) & ~size_t{255}; }

gk_status from_hip(hipError_t e) { return e == hipSuccess ? GK_SUCCESS : GK_DEVICE_ERROR; }

// Per-device gfx950 gate, evaluated once per device.
constexpr int kMaxDevices = 64;
std::once_flag g_dev_once[kMaxDevices];
bool g_dev_ok[kMaxDevices];

bool device_ok(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return false;
  std::call_once(g_dev_once[dev], [dev] {
    hipDeviceProp_t prop;
    g_dev_ok[dev] = hipGetDeviceProperties(&prop, dev) == hipSuccess &&
                    std::strncmp(prop.gcnArchName, "gfx950", 6) == 0;
  });
  return g_dev_ok[dev];
}

gk_status current_device_ok() {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return GK_DEVICE_ERROR;
  return device_ok(dev) ? GK_SUCCESS : GK_UNSUPPORTED_DEVICE;
}

__global__ void zero_words_kernel(uint32_t* p, int n) {
  if (static_cast<int>(threadIdx.x) < n) p[threadIdx.x] = 0u;
}

// Status block in the caller's workspace: word 0 = flags, words 2..3 = 64-bit count.
struct Status {
  uint32_t flags;
  uint32_t pad;
  unsigned long long count;
};

gk_status read_status(void* ws, Status* st, hipStream_t stream) {
  if (hipMemcpyAsync(st, ws, sizeof(Status), hipMemcpyDeviceToHost, stream) != hipSuccess) return GK_DEVICE_ERROR;
  return from_hip(hipStreamSynchronize(stream));
}

__global__ __launch_bounds__(256) void check_inputs_kernel(const uint16_t* __restrict__ x, int64_t m, int64_t k,
                                                           int64_t ldx, const uint8_t* __restrict__ w,
                                                           int64_t nw, const float* __restrict__ s, int64_t ns,
                                                           uint32_t* __restrict__ flags) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t bad = 0;
  for (int64_t i = tid; i < m * k; i += stride) {
    const int64_t r = i / k, c = i - r * k;
    bad |= (x[r * ldx + c] & 0x7f80u) == 0x7f80u;
  }
  for (int64_t i = tid; i < nw; i += stride) bad |= (w[i] & 0x7fu) == 0x7fu;
  for (int64_t i = tid; i < ns; i += stride) {
    const float v = s[i];
    bad |= !(v >= 0.0f) || (gk::f32_bits(v) & 0x7f800000u) == 0x7f800000u;
  }
  if (bad) atomicOr(flags, 1u);
}

struct Plan {
  int variant;
  int64_t m_pad;
  size_t q_bytes = 0, sa_bytes = 0;  // quantized activations [G][m_pad][128] and scales [G][m_pad]
  gk::DecodeShape dec{0, 0, 0};
};

gk_status make_plan(int64_t m, int64_t n, int64_t k, uint32_t flags, const void* w, Plan* p) {
  if (m < 1 || n < 1 || k < 1 || m > kMaxDim || n > kMaxDim || k > kMaxDim) return GK_INCOMPATIBLE_INPUT_SIZE;
  if (flags & ~kKnownFlags) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  const uint32_t force = flags & (GK_FLAG_FORCE_DECODE | GK_FLAG_FORCE_PREFILL | GK_FLAG_FORCE_GENERIC);
  if (force & (force - 1)) return GK_UNSUPPORTED_LAYER_CONFIGURATION;  // more than one forced variant
  const bool tiled_ok = (k % 128 == 0) && ((reinterpret_cast<uintptr_t>(w) & 15) == 0);
  const bool wpack = (flags & GK_FLAG_WEIGHT_PACKED) != 0;
  if (wpack && (!tiled_ok || force == GK_FLAG_FORCE_GENERIC)) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  const int64_t g = (k + 127) / 128;
  int variant;
  if (force == GK_FLAG_FORCE_GENERIC || (!force && !tiled_ok)) {
    variant = GK_VARIANT_GENERIC;
  } else if (!tiled_ok) {
    return GK_UNSUPPORTED_LAYER_CONFIGURATION;  // decode/prefill need K % 128 == 0 and 16-byte aligned weights
  } else if (force == GK_FLAG_FORCE_PREFILL) {
    variant = GK_VARIANT_PREFILL;
  } else if (force == GK_FLAG_FORCE_DECODE) {
    if (m > gk::kDecodeMaxTokens) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
    variant = GK_VARIANT_DECODE;
  } else {
    variant = m <= gk::kDecodeMaxTokens ? GK_VARIANT_DECODE : GK_VARIANT_PREFILL;
  }
  *p = Plan();
  p->variant = variant;
  p->m_pad = variant == GK_VARIANT_DECODE    ? 16 * gk::decode_tiles(m)
             : variant == GK_VARIANT_PREFILL ? round_up(m, gk::kPrefillRowTile)
                                             : m;
  p->q_bytes = align256(static_cast<size_t>(p->m_pad) * static_cast<size_t>(g) * 128);
  p->sa_bytes = align256(static_cast<size_t>(p->m_pad) * static_cast<size_t>(g) * 4);
  if (variant == GK_VARIANT_DECODE)
    p->dec = gk::fit_group_step(
        gk::plan_decode_shape(static_cast<int>(n), static_cast<int>(g), wpack, gk::decode_tiles(m)),
        static_cast<int>(g));
  // The prefill variant (256 x 256 kernel) addresses its panels with 32-bit
  // offsets: larger shapes run the generic variant (packed weights: rejected).
  if (variant == GK_VARIANT_PREFILL && (p->m_pad * g * 128 > int64_t{0xffffffff} || 256 * k > int64_t{0xffffffff})) {
    if (wpack || force == GK_FLAG_FORCE_PREFILL) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
    p->variant = GK_VARIANT_GENERIC;
    p->m_pad = m;
    p->q_bytes = align256(static_cast<size_t>(m) * static_cast<size_t>(g) * 128);
    p->sa_bytes = align256(static_cast<size_t>(m) * static_cast<size_t>(g) * 4);
  }
  return GK_SUCCESS;
}

// Decode GEMM with the quantizer fused: every workgroup quantizes the
// ceil(M/4) token rows of 4 it needs over its K range.  That redundant work,
// relative to one workgroup per CU over K = 4096 with all 16 rows, is
// (workgroups / 256) * (K / 4096) * ceil(M/4) / 4.  Measured on MI355X with
// the fused kernel's own load step (fused_quant_shape) over eight N x K
// shapes and M = 1..16, fusing saves up to 2 us (the separate quantizer
// launch) while this stays <= 1.2 -- N = 6144, K = 4096 at every M <= 16,
// 7168 x 7168 at M <= 12, 28672 x 4096 and 4096 x 14336 at M <= 4 -- and
// costs up to 6 us beyond it.  Near the bound either choice is within 1 us.
bool fused_quant_pays(int64_t m, int64_t n, int64_t k, const gk::DecodeShape& d) {
  const double wgs = static_cast<double>((n + 16 * d.r - 1) / (16 * d.r));
  const double rows4 = static_cast<double>((std::min<int64_t>(m, 16) + 3) / 4);
  return (wgs / 256.0) * (static_cast<double>(k) / 4096.0) * (rows4 / 4.0) <= 1.2;
}

gk_status check_gemm_common(int64_t k, const void* w, int64_t n, const float* scales, int64_t scale_rows,
                            int64_t scale_cols, const float* bias, const void* y, int64_t ldy) {
  if (!w || !scales || !y) return GK_INVALID_ARGUMENT;
  if (scale_rows != (n + 127) / 128 || scale_cols != (k + 127) / 128) return GK_INCOMPATIBLE_INPUT_SIZE;
  if (ldy < n) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (((reinterpret_cast<uintptr_t>(scales) | reinterpret_cast<uintptr_t>(bias)) & 3) ||
      (reinterpret_cast<uintptr_t>(y) & 1))
    return GK_INCOMPATIBLE_DATA_TYPE;
  return GK_SUCCESS;
}

// xq_ldx > 0: q is the bf16 activation x (row stride xq_ldx elements), quantized inside the decode kernel.
gk_status run_gemm(const Plan& p, const uint8_t* q, const float* sa, int64_t m, int64_t k, const void* w,
                   int64_t n, const float* scales, const float* bias, void* y, int64_t ldy, uint32_t flags,
                   bool qpack, hipStream_t stream, int64_t xq_ldx = 0) {
  gk::GemmArgs a;
  a.qa = q;
  a.sa = sa;
  a.w = static_cast<const uint8_t*>(w);
  a.sw = scales;
  a.bias = bias;
  a.y = static_cast<uint16_t*>(y);
  a.ldy = ldy;
  a.M = static_cast<int>(m);
  a.N = static_cast<int>(n);
  a.K = static_cast<int>(k);
  a.G = static_cast<int>((k + 127) / 128);
  a.Mpad = static_cast<int>(p.m_pad);
  a.half_w = (flags & GK_FLAG_NATIVE_HALF) != 0;
  a.dec = p.dec;
  a.qpack = qpack;
  a.wpack = (flags & GK_FLAG_WEIGHT_PACKED) != 0;
  a.xq = xq_ldx > 0;
  a.ldq = xq_ldx;
  hipError_t e;
  switch (p.variant) {
    case GK_VARIANT_DECODE: e = gk::launch_gemm_decode(a, stream); break;
    case GK_VARIANT_PREFILL: e = gk::launch_gemm_prefill(a, stream); break;
    default: e = gk::launch_gemm_generic(a, stream); break;
  }
  return from_hip(e);
}

gk_status codec_common(bool forward, const void* src, void* dst, int64_t n, const float* scales, float* scales_out,
                       int64_t n_scales, int64_t* rounded, void* ws, size_t wsb, void* stream) {
  if (!src || !dst || !scales || !scales_out || !ws) return GK_INVALID_ARGUMENT;
  if (n < 1) return GK_INCOMPATIBLE_INPUT_SIZE;         // "expected a nonempty ... weight"
  if (n_scales < 1) return GK_INVALID_SCALE;            // "expected nonempty ... scales"
  if (wsb < kStatusBytes) return GK_INSUFFICIENT_BUFFER;
  if (reinterpret_cast<uintptr_t>(ws) & 7) return GK_INCOMPATIBLE_DATA_TYPE;
  if (reinterpret_cast<uintptr_t>(scales) & 3 || reinterpret_cast<uintptr_t>(scales_out) & 3)
    return GK_INCOMPATIBLE_DATA_TYPE;
  gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* words = static_cast<uint32_t*>(ws);
  zero_words_kernel<<<1, 64, 0, s>>>(words, 4);
  if (hipGetLastError() != hipSuccess) return GK_DEVICE_ERROR;
  const hipError_t e = gk::launch_codec(forward, static_cast<const uint8_t*>(src), static_cast<uint8_t*>(dst), n,
                                        scales, scales_out, n_scales, words,
                                        reinterpret_cast<unsigned long long*>(words + 2), s);
  if (e != hipSuccess) return GK_DEVICE_ERROR;
  Status stat;
  st = read_status(ws, &stat, s);
  if (st != GK_SUCCESS) return st;
  if (forward) {
    if (stat.flags & 2u) return GK_INVALID_SCALE;
    if (stat.flags & 4u) return GK_SCALE_OVERFLOW;
    if (stat.flags & 1u) return GK_NONFINITE_CODE;
    if (rounded) *rounded = static_cast<int64_t>(stat.count);
  } else {
    if (stat.flags & 2u) return GK_INVALID_SCALE;
    if (stat.flags & 8u) return GK_NONFINITE_CODE;
    if (stat.flags & 16u) return GK_INEXACT_SCALE;
  }
  return GK_SUCCESS;
}

}  // namespace

extern "C" {

uint64_t gk_lib_version(void) { return 1; }

gk_status gk_list_ops(uint32_t* count, const char** names) {
  if (!count) return GK_INVALID_ARGUMENT;
  const uint32_t capacity = *count;
  *count = kNumOps;
  if (!names || capacity == 0) return GK_SUCCESS;
  const uint32_t emit = capacity < kNumOps ? capacity : kNumOps;
  for (uint32_t i = 0; i < emit; ++i) names[i] = kOps[i];
  return capacity < kNumOps ? GK_INSUFFICIENT_BUFFER : GK_SUCCESS;
}

gk_status gk_device_supported(int device) {
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess) return GK_DEVICE_ERROR;
  if (device < 0 || device >= count) return GK_UNSUPPORTED_DEVICE;
  return device_ok(device) ? GK_SUCCESS : GK_UNSUPPORTED_DEVICE;
}

gk_status gk_fp8_codec_workspace_bytes(size_t* bytes) {
  if (!bytes) return GK_INVALID_ARGUMENT;
  *bytes = kStatusBytes;
  return GK_SUCCESS;
}

gk_status gk_fp8_codec_ocp_to_half(const void* src, void* dst, int64_t n, const float* scales, float* scales_out,
                                   int64_t n_scales, int64_t* rounded, void* workspace, size_t workspace_bytes,
                                   void* stream) {
  return codec_common(true, src, dst, n, scales, scales_out, n_scales, rounded, workspace, workspace_bytes, stream);
}

gk_status gk_fp8_codec_half_to_ocp(const void* src, void* dst, int64_t n, const float* scales, float* scales_out,
                                   int64_t n_scales, void* workspace, size_t workspace_bytes, void* stream) {
  return codec_common(false, src, dst, n, scales, scales_out, n_scales, nullptr, workspace, workspace_bytes,
                      stream);
}

gk_status gk_fp8_act_quant_bf16(const void* x, int64_t m, int64_t k, int64_t ldx, void* q, float* sa, int64_t m_pad,
                                uint32_t flags, void* stream) {
  if (!x || !q || !sa) return GK_INVALID_ARGUMENT;
  if (m < 1 || k < 1 || m > kMaxDim || k > kMaxDim || ldx < k) return GK_INCOMPATIBLE_INPUT_SIZE;
  if (m_pad < m || m_pad > kMaxDim) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (flags & ~uint32_t{GK_FLAG_NATIVE_HALF | GK_FLAG_DECODE_LAYOUT}) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  const bool packed = (flags & GK_FLAG_DECODE_LAYOUT) != 0;
  if (packed && m_pad != 16 && m_pad != 32 && m_pad != 64) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if ((reinterpret_cast<uintptr_t>(x) & 1) || (reinterpret_cast<uintptr_t>(q) & 7) ||
      (reinterpret_cast<uintptr_t>(sa) & 3))
    return GK_INCOMPATIBLE_DATA_TYPE;
  gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_act_quant(static_cast<const uint16_t*>(x), ldx, static_cast<int>(m),
                                       static_cast<int>(k), static_cast<int>(m_pad), static_cast<uint8_t*>(q), sa,
                                       (flags & GK_FLAG_NATIVE_HALF) != 0, packed, static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_packed_weight_bytes(int64_t n, int64_t k, size_t* bytes) {
  if (!bytes) return GK_INVALID_ARGUMENT;
  if (n < 1 || k < 128 || k % 128 != 0 || n > kMaxDim || k > kMaxDim) return GK_INCOMPATIBLE_INPUT_SIZE;
  *bytes = static_cast<size_t>(gk::packed_weight_bytes(n, k));
  return GK_SUCCESS;
}

gk_status gk_fp8_pack_weight(const void* w, int64_t n, int64_t k, void* packed, size_t packed_bytes, void* stream) {
  if (!w || !packed) return GK_INVALID_ARGUMENT;
  size_t need = 0;
  gk_status st = gk_fp8_packed_weight_bytes(n, k, &need);
  if (st != GK_SUCCESS) return st;
  if (packed_bytes < need) return GK_INSUFFICIENT_BUFFER;
  if ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(packed)) & 15) return GK_INCOMPATIBLE_DATA_TYPE;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_pack_weight(static_cast<const uint8_t*>(w), static_cast<int>(n), static_cast<int>(k),
                                         static_cast<uint8_t*>(packed), static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_pack_experts(const void* w, int64_t e, int64_t n, int64_t k, void* packed, size_t packed_bytes,
                              void* stream) {
  if (!w || !packed) return GK_INVALID_ARGUMENT;
  if (e < 1 || e > gk::kMoeMaxExperts) return GK_INCOMPATIBLE_INPUT_SIZE;
  size_t per = 0;
  gk_status st = gk_fp8_packed_weight_bytes(n, k, &per);
  if (st != GK_SUCCESS) return st;
  if (packed_bytes / per < static_cast<size_t>(e)) return GK_INSUFFICIENT_BUFFER;
  if ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(packed)) & 15) return GK_INCOMPATIBLE_DATA_TYPE;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_pack_experts(static_cast<const uint8_t*>(w), static_cast<int>(e), static_cast<int>(n),
                                          static_cast<int>(k), static_cast<uint8_t*>(packed),
                                          static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_block_gemm_plan(int64_t m, int64_t n, int64_t k, uint32_t flags, const void* w, int* variant,
                                 int64_t* m_pad, size_t* workspace_bytes) {
  Plan p;
  const gk_status st = make_plan(m, n, k, flags, w, &p);
  if (st != GK_SUCCESS) return st;
  if (variant) *variant = p.variant;
  if (m_pad) *m_pad = p.m_pad;
  if (workspace_bytes) *workspace_bytes = p.q_bytes + p.sa_bytes;
  return GK_SUCCESS;
}

gk_status gk_fp8_block_gemm_bf16(const void* x, int64_t m, int64_t k, int64_t ldx, const void* w, int64_t n,
                                 const float* scales, int64_t scale_rows, int64_t scale_cols, const float* bias,
                                 void* y, int64_t ldy, uint32_t flags, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  if (!x || !workspace) return GK_INVALID_ARGUMENT;
  Plan p;
  gk_status st = make_plan(m, n, k, flags, w, &p);
  if (st != GK_SUCCESS) return st;
  if (ldx < k) return GK_INCOMPATIBLE_INPUT_SIZE;
  st = check_gemm_common(k, w, n, scales, scale_rows, scale_cols, bias, y, ldy);
  if (st != GK_SUCCESS) return st;
  if (workspace_bytes < p.q_bytes + p.sa_bytes) return GK_INSUFFICIENT_BUFFER;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) || (reinterpret_cast<uintptr_t>(x) & 1))
    return GK_INCOMPATIBLE_DATA_TYPE;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  // Decode variant with 16-byte aligned activation rows and little redundant
  // quantization work: the GEMM quantizes x itself (one launch, the same
  // codes and scales as the quantizer below).
  if (p.variant == GK_VARIANT_DECODE && p.dec.mt == 1 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
      ldx % 8 == 0 && fused_quant_pays(m, n, k, p.dec)) {
    Plan fused = p;
    fused.dec = gk::fused_quant_shape(p.dec, static_cast<int>((k + 127) / 128));
    return run_gemm(fused, static_cast<const uint8_t*>(x), nullptr, m, k, w, n, scales, bias, y, ldy, flags, false,
                    s, ldx);
  }
  uint8_t* q = static_cast<uint8_t*>(workspace);
  float* sa = reinterpret_cast<float*>(q + p.q_bytes);
  // The decode variant takes its activations in the packed fragment layout.
  const bool packed = p.variant == GK_VARIANT_DECODE;
  hipError_t e = gk::launch_act_quant(static_cast<const uint16_t*>(x), ldx, static_cast<int>(m), static_cast<int>(k),
                                      static_cast<int>(p.m_pad), q, sa, (flags & GK_FLAG_NATIVE_HALF) != 0, packed,
                                      s);
  if (e != hipSuccess) return GK_DEVICE_ERROR;
  return run_gemm(p, q, sa, m, k, w, n, scales, bias, y, ldy, flags, packed, s);
}

// ---- allocation-free GEMM entry -----------------------------------------------------------
// The quantized-activation scratch of gk_fp8_block_gemm_bf16_noalloc lives in
// this file-scope device array (one copy per GPU, held until the process
// ends).  Host code never passes `scratch` itself to a kernel: its device
// address, per device, comes from hipGetSymbolAddress on the first call on
// that device and is what the kernels receive.
namespace {

static_assert(GK_NOALLOC_SCRATCH_BYTES % 256 == 0, "scratch is used as a 256-byte aligned workspace");
static __device__ __align__(256) uint8_t scratch[GK_NOALLOC_SCRATCH_BYTES];

std::once_flag g_scratch_once[kMaxDevices];
void* g_scratch_ptr[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices];

// Device address of `scratch` on the current device (nullptr on failure).
void* scratch_address(int dev) {
  if (dev < 0 || dev >= kMaxDevices) return nullptr;
  std::call_once(g_scratch_once[dev], [dev] {
    void* ptr = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    g_scratch_ptr[dev] = g_scratch_err[dev] == hipSuccess ? ptr : nullptr;
  });
  return g_scratch_ptr[dev];
}

}  // namespace

gk_status gk_fp8_block_gemm_bf16_noalloc(const void* x, int64_t m, int64_t k, int64_t ldx, const void* w, int64_t n,
                                         const float* scales, int64_t scale_rows, int64_t scale_cols,
                                         const float* bias, void* y, int64_t ldy, uint32_t flags, void* stream) {
  if (!x) return GK_INVALID_ARGUMENT;
  Plan p;
  gk_status st = make_plan(m, n, k, flags, w, &p);
  if (st != GK_SUCCESS) return st;
  if (p.q_bytes + p.sa_bytes > size_t{GK_NOALLOC_SCRATCH_BYTES}) return GK_INSUFFICIENT_BUFFER;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess) return GK_DEVICE_ERROR;
  void* ws = scratch_address(dev);
  if (!ws) return GK_DEVICE_ERROR;
  // The quantizer rewrites every byte of the scratch the GEMM reads (padding rows included), so nothing left
  // by an earlier call is read.
  return gk_fp8_block_gemm_bf16(x, m, k, ldx, w, n, scales, scale_rows, scale_cols, bias, y, ldy, flags, ws,
                                GK_NOALLOC_SCRATCH_BYTES, stream);
}

gk_status gk_fp8_block_gemm_q_bf16(const void* q, const float* sa, int64_t m, int64_t m_pad, int64_t k,
                                   const void* w, int64_t n, const float* scales, int64_t scale_rows,
                                   int64_t scale_cols, const float* bias, void* y, int64_t ldy, uint32_t flags,
                                   void* stream) {
  if (!q || !sa) return GK_INVALID_ARGUMENT;
  const bool packed = (flags & GK_FLAG_DECODE_LAYOUT) != 0;
  Plan p;
  gk_status st = make_plan(m, n, k, flags & ~uint32_t{GK_FLAG_DECODE_LAYOUT}, w, &p);
  if (st != GK_SUCCESS) return st;
  if (packed && p.variant != GK_VARIANT_DECODE) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  if (m_pad != p.m_pad) return GK_INCOMPATIBLE_INPUT_SIZE;
  st = check_gemm_common(k, w, n, scales, scale_rows, scale_cols, bias, y, ldy);
  if (st != GK_SUCCESS) return st;
  if ((reinterpret_cast<uintptr_t>(q) & 15) || (reinterpret_cast<uintptr_t>(sa) & 3))
    return GK_INCOMPATIBLE_DATA_TYPE;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return run_gemm(p, static_cast<const uint8_t*>(q), sa, m, k, w, n, scales, bias, y, ldy, flags, packed,
                  static_cast<hipStream_t>(stream));
}

gk_status gk_fp8_block_gemm_kslice_f32(const void* x, int64_t m, int64_t k, int64_t ldx, int64_t k_offset,
                                       int64_t k_len, const void* w, int64_t n, const float* scales,
                                       int64_t scale_rows, int64_t scale_cols, float* partial, int64_t ldp,
                                       uint32_t flags, void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !w || !scales || !partial || !workspace) return GK_INVALID_ARGUMENT;
  if (flags & ~kKsliceFlags) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  // col_offset rules of generic_fp8_glue.hpp:169-176 (offset >= 0, a multiple of 128) and :245-252 (widths
  // nonzero multiples of 128, offset + width within the input)
  if (k_offset < 0 || k_offset % 128) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  if (m < 1 || n < 1 || k < 128 || k % 128 || k_len < 128 || k_len % 128 || m > kMaxDim || n > kMaxDim ||
      k > kMaxDim || k_len > k || k_offset > k - k_len || ldx < k)
    return GK_INCOMPATIBLE_INPUT_SIZE;
  if (scale_rows != (n + 127) / 128 || scale_cols != k / 128) return GK_INCOMPATIBLE_INPUT_SIZE;
  if (ldp < n) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if ((reinterpret_cast<uintptr_t>(x) & 1) || ((reinterpret_cast<uintptr_t>(scales) |
                                                 reinterpret_cast<uintptr_t>(partial)) & 3) ||
      (reinterpret_cast<uintptr_t>(workspace) & 255))
    return GK_INCOMPATIBLE_DATA_TYPE;
  const bool wpack = (flags & GK_FLAG_WEIGHT_PACKED) != 0;
  const int64_t g0 = k_offset / 128, gl = k_len / 128;
  const uint8_t* wb = static_cast<const uint8_t*>(w) + (wpack ? g0 * 2048 : k_offset);
  Plan p;
  gk_status st = make_plan(m, n, k_len, flags & ~uint32_t{GK_FLAG_ACCUMULATE}, wb, &p);
  if (st != GK_SUCCESS) return st;
  // the tiled kernels only (the prefill kernel addresses a weight panel of the whole row with 32-bit offsets)
  if (p.variant == GK_VARIANT_GENERIC || (p.variant == GK_VARIANT_PREFILL && 256 * k > int64_t{0xffffffff}))
    return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  if (workspace_bytes < p.q_bytes + p.sa_bytes) return GK_INSUFFICIENT_BUFFER;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint16_t* xs = static_cast<const uint16_t*>(x) + k_offset;
  gk::GemmArgs a{};
  a.w = wb;
  a.sw = scales + g0;
  a.bias = nullptr;
  a.y = nullptr;
  a.M = static_cast<int>(m);
  a.N = static_cast<int>(n);
  a.K = static_cast<int>(k);  // row stride of the row-major weights
  a.G = static_cast<int>(gl);
  a.gs = static_cast<int>(k / 128);
  a.Mpad = static_cast<int>(p.m_pad);
  a.half_w = (flags & GK_FLAG_NATIVE_HALF) != 0;
  a.dec = p.dec;
  a.wpack = wpack;
  a.yp = partial;
  a.ldyp = ldp;
  a.accumulate = (flags & GK_FLAG_ACCUMULATE) != 0;
  if (p.variant == GK_VARIANT_DECODE && p.dec.mt == 1 && (reinterpret_cast<uintptr_t>(xs) & 15) == 0 &&
      ldx % 8 == 0 && fused_quant_pays(m, n, k_len, p.dec)) {
    a.dec = gk::fused_quant_shape(p.dec, static_cast<int>(gl));
    a.qa = reinterpret_cast<const uint8_t*>(xs);
    a.xq = true;
    a.ldq = ldx;
    return from_hip(gk::launch_gemm_decode(a, s));
  }
  uint8_t* q = static_cast<uint8_t*>(workspace);
  float* sa = reinterpret_cast<float*>(q + p.q_bytes);
  const bool packed = p.variant == GK_VARIANT_DECODE;
  hipError_t e = gk::launch_act_quant(xs, ldx, static_cast<int>(m), static_cast<int>(k_len),
                                      static_cast<int>(p.m_pad), q, sa, a.half_w, packed, s);
  if (e != hipSuccess) return GK_DEVICE_ERROR;
  a.qa = q;
  a.sa = sa;
  a.qpack = packed;
  return from_hip(p.variant == GK_VARIANT_DECODE ? gk::launch_gemm_decode(a, s) : gk::launch_gemm_prefill(a, s));
}

// ---- row-parallel completion ------------------------------------------------------------
// infer_rank_sum (generic_dense_glue.cpp:871-895): world_size in [2, 8], the
// gathered length a nonzero multiple of it.
gk_status gk_rank_sum_infer(int64_t gathered_elems, int world_size, int64_t* elems) {
  if (!elems) return GK_INVALID_ARGUMENT;
  if (world_size < 2 || world_size > 8) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  if (gathered_elems < world_size || gathered_elems % world_size) return GK_INCOMPATIBLE_INPUT_SIZE;
  *elems = gathered_elems / world_size;
  return GK_SUCCESS;
}

namespace {

// instantiate_rank_sum (generic_dense_glue.cpp:568-600), in its order:
// world_size, data type (here: alignment), output size, gathered size.
gk_status rank_sum_common(const void* gathered, int64_t gathered_elems, int world_size, void* dst, int64_t elems,
                          bool bf16, void* stream) {
  if (!gathered || !dst) return GK_INVALID_ARGUMENT;
  if (world_size < 2 || world_size > 8) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  if (((reinterpret_cast<uintptr_t>(gathered) | reinterpret_cast<uintptr_t>(dst)) & (bf16 ? 1 : 3)) != 0)
    return GK_INCOMPATIBLE_DATA_TYPE;
  if (elems < 1 || elems > kMaxDim / world_size) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (gathered_elems != elems * world_size) return GK_INCOMPATIBLE_INPUT_SIZE;
  const gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_rank_sum(gathered, dst, elems, world_size, bf16, static_cast<hipStream_t>(stream)));
}

}  // namespace

gk_status gk_rank_sum_f32(const float* gathered, int64_t gathered_elems, int world_size, float* dst, int64_t elems,
                          void* stream) {
  return rank_sum_common(gathered, gathered_elems, world_size, dst, elems, false, stream);
}

gk_status gk_rank_sum_bf16(const void* gathered, int64_t gathered_elems, int world_size, void* dst, int64_t elems,
                           void* stream) {
  return rank_sum_common(gathered, gathered_elems, world_size, dst, elems, true, stream);
}

gk_status gk_fp8_partial_finish_bf16(const float* partial, int64_t rows, int64_t width, int64_t ldp,
                                     const float* bias, void* y, int64_t ldy, void* stream) {
  if (!partial || !y) return GK_INVALID_ARGUMENT;
  if (rows < 1 || width < 1 || rows > kMaxDim || width > kMaxDim || ldp < width) return GK_INCOMPATIBLE_INPUT_SIZE;
  if (ldy < width) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (((reinterpret_cast<uintptr_t>(partial) | reinterpret_cast<uintptr_t>(bias)) & 3) ||
      (reinterpret_cast<uintptr_t>(y) & 1))
    return GK_INCOMPATIBLE_DATA_TYPE;
  const gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_partial_finish(partial, ldp, static_cast<int>(rows), static_cast<int>(width), bias,
                                            static_cast<uint16_t*>(y), ldy, static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_check_inputs(const void* x, int64_t m, int64_t k, int64_t ldx, const void* w, int64_t n,
                              const float* scales, int64_t n_scales, void* workspace, size_t workspace_bytes,
                              void* stream) {
  if (!x || !w || !scales || !workspace) return GK_INVALID_ARGUMENT;
  if (m < 1 || k < 1 || n < 1 || ldx < k || n_scales < 1) return GK_INCOMPATIBLE_INPUT_SIZE;
  if (workspace_bytes < kStatusBytes) return GK_INSUFFICIENT_BUFFER;
  if ((reinterpret_cast<uintptr_t>(x) & 1) || (reinterpret_cast<uintptr_t>(scales) & 3) ||
      (reinterpret_cast<uintptr_t>(workspace) & 7))
    return GK_INCOMPATIBLE_DATA_TYPE;
  gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint32_t* words = static_cast<uint32_t*>(workspace);
  zero_words_kernel<<<1, 64, 0, s>>>(words, 4);
  check_inputs_kernel<<<1024, 256, 0, s>>>(static_cast<const uint16_t*>(x), m, k, ldx,
                                           static_cast<const uint8_t*>(w), n * k, scales, n_scales, words);
  if (hipGetLastError() != hipSuccess) return GK_DEVICE_ERROR;
  Status stat;
  st = read_status(workspace, &stat, s);
  if (st != GK_SUCCESS) return st;
  return stat.flags ? GK_NONFINITE_INPUT : GK_SUCCESS;
}

// ---- per-token / per-channel ----------------------------------------------------------
gk_status gk_fp8_token_quant_bf16(const void* x, int64_t rows, int64_t width, int64_t ldx, void* q, int64_t ldq,
                                  float* scales, void* stream) {
  if (!x || !q || !scales) return GK_INVALID_ARGUMENT;
  // generic_fp8_glue.hpp:39-44: nonzero width, multiple of 128; rows >= 1
  if (rows < 1 || width < 128 || width % 128 || rows > kMaxDim || width > kMaxDim || ldx < width)
    return GK_INCOMPATIBLE_INPUT_SIZE;
  if (ldq < width || ldq % 8) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if ((reinterpret_cast<uintptr_t>(x) & 1) || (reinterpret_cast<uintptr_t>(q) & 7) ||
      (reinterpret_cast<uintptr_t>(scales) & 3))
    return GK_INCOMPATIBLE_DATA_TYPE;
  const gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_token_quant(static_cast<const uint16_t*>(x), ldx, static_cast<int>(rows),
                                         static_cast<int>(width), static_cast<uint8_t*>(q), ldq, scales,
                                         static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_channel_finish_bf16(const float* partial, int64_t rows, int64_t width, int64_t ldp,
                                     const float* act_scales, const float* w_scales, const float* bias, void* y,
                                     int64_t ldy, void* stream) {
  if (!partial || !act_scales || !w_scales || !y) return GK_INVALID_ARGUMENT;
  // generic_fp8_glue.hpp:61-66: width a nonzero multiple of 128
  if (rows < 1 || width < 128 || width % 128 || rows > kMaxDim || width > kMaxDim || ldp < width)
    return GK_INCOMPATIBLE_INPUT_SIZE;
  if (ldy < width) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (((reinterpret_cast<uintptr_t>(partial) | reinterpret_cast<uintptr_t>(act_scales) |
        reinterpret_cast<uintptr_t>(w_scales) | reinterpret_cast<uintptr_t>(bias)) & 3) ||
      (reinterpret_cast<uintptr_t>(y) & 1))
    return GK_INCOMPATIBLE_DATA_TYPE;
  const gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_channel_finish(partial, ldp, static_cast<int>(rows), static_cast<int>(width),
                                            act_scales, w_scales, bias, static_cast<uint16_t*>(y), ldy,
                                            static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_channel_gemm_bf16(const void* q, int64_t ldq, const float* sa, int64_t m, int64_t k, const void* w,
                                   int64_t n, const float* sw, const float* bias, void* y, int64_t ldy,
                                   uint32_t flags, void* stream) {
  if (!q || !sa || !w || !sw || !y) return GK_INVALID_ARGUMENT;
  if (flags) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  if (m < 1 || n < 1 || k < 128 || k % 128 || m > kMaxDim || n > kMaxDim || k > kMaxDim || ldq < k)
    return GK_INCOMPATIBLE_INPUT_SIZE;
  if (ldy < n) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(w)) & 15) || ldq % 16 ||
      ((reinterpret_cast<uintptr_t>(sa) | reinterpret_cast<uintptr_t>(sw) | reinterpret_cast<uintptr_t>(bias)) & 3) ||
      (reinterpret_cast<uintptr_t>(y) & 1))
    return GK_INCOMPATIBLE_DATA_TYPE;
  if (int64_t{256} * ldq > int64_t{0xffffffff} || int64_t{256} * k > int64_t{0xffffffff})
    return GK_INCOMPATIBLE_INPUT_SIZE;
  const gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  gk::GemmArgs a{};
  a.qa = static_cast<const uint8_t*>(q); a.sa = sa; a.w = static_cast<const uint8_t*>(w); a.sw = sw; a.bias = bias;
  a.y = static_cast<uint16_t*>(y); a.ldy = ldy; a.M = static_cast<int>(m); a.N = static_cast<int>(n);
  a.K = static_cast<int>(k); a.G = static_cast<int>(k / 128); a.Mpad = static_cast<int>(m); a.half_w = false;
  a.channel = true; a.ldq = ldq;
  return from_hip(gk::launch_gemm_channel(a, static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_token_channel_gemm_bf16(const void* x, int64_t ldx, int64_t m, int64_t k, const void* w, int64_t n,
                                         const float* sw, const float* bias, void* y, int64_t ldy, uint32_t flags,
                                         void* stream) {
  if (!x || !w || !sw || !y) return GK_INVALID_ARGUMENT;
  if (flags) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  // the token quantizer's width rule (generic_fp8_glue.hpp:39-44) and the fused form's M <= 16
  if (m < 1 || m > 16 || n < 1 || k < 128 || k % 128 || n > kMaxDim || k > kMaxDim || ldx < k)
    return GK_INCOMPATIBLE_INPUT_SIZE;
  if (ldy < n) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if ((reinterpret_cast<uintptr_t>(x) & 15) || ldx % 8 || (reinterpret_cast<uintptr_t>(w) & 15) ||
      ((reinterpret_cast<uintptr_t>(sw) | reinterpret_cast<uintptr_t>(bias)) & 3) ||
      (reinterpret_cast<uintptr_t>(y) & 1))
    return GK_INCOMPATIBLE_DATA_TYPE;
  const gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  gk::GemmArgs a{};
  a.qa = static_cast<const uint8_t*>(x); a.sa = nullptr; a.w = static_cast<const uint8_t*>(w); a.sw = sw;
  a.bias = bias; a.y = static_cast<uint16_t*>(y); a.ldy = ldy; a.M = static_cast<int>(m);
  a.N = static_cast<int>(n); a.K = static_cast<int>(k); a.G = static_cast<int>(k / 128);
  a.Mpad = static_cast<int>(m); a.half_w = false; a.channel = true; a.ldq = ldx;
  return from_hip(gk::launch_gemm_token_channel(a, static_cast<hipStream_t>(stream)));
}

// ---- SiLU-and-mul ----------------------------------------------------------------------
gk_status gk_silu_and_mul_bf16(const void* gate_up, int64_t rows, int64_t width, int64_t ld_in, void* out,
                               int64_t ld_out, void* stream) {
  if (!gate_up || !out) return GK_INVALID_ARGUMENT;
  // generic_dense_glue.cpp:203-210: nonzero sizes within int, input width even (= 2 * width)
  if (rows < 1 || width < 1 || rows > kMaxDim || width > kMaxDim / 2 || ld_in < 2 * width)
    return GK_INCOMPATIBLE_INPUT_SIZE;
  if (ld_out < width) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if ((reinterpret_cast<uintptr_t>(gate_up) | reinterpret_cast<uintptr_t>(out)) & 1) return GK_INCOMPATIBLE_DATA_TYPE;
  const gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_silu_and_mul(static_cast<const uint16_t*>(gate_up), ld_in, static_cast<int>(rows),
                                          static_cast<int>(width), static_cast<uint16_t*>(out), ld_out,
                                          static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_silu_mul_quant_bf16(const void* gate_up, int64_t rows, int64_t width, int64_t ld_in, void* q,
                                     float* sa, int64_t m_pad, uint32_t flags, void* stream) {
  if (!gate_up || !q || !sa) return GK_INVALID_ARGUMENT;
  if (rows < 1 || width < 1 || rows > kMaxDim || width > kMaxDim / 2 || ld_in < 2 * width)
    return GK_INCOMPATIBLE_INPUT_SIZE;
  if (m_pad < rows || m_pad > kMaxDim) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (flags & ~uint32_t{GK_FLAG_NATIVE_HALF | GK_FLAG_DECODE_LAYOUT}) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  const bool packed = (flags & GK_FLAG_DECODE_LAYOUT) != 0;
  if (packed && m_pad != 16 && m_pad != 32 && m_pad != 64) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if ((reinterpret_cast<uintptr_t>(gate_up) & 1) || (reinterpret_cast<uintptr_t>(q) & 7) ||
      (reinterpret_cast<uintptr_t>(sa) & 3))
    return GK_INCOMPATIBLE_DATA_TYPE;
  const gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_silu_mul_act_quant(static_cast<const uint16_t*>(gate_up), ld_in, static_cast<int>(rows),
                                                static_cast<int>(width), static_cast<int>(m_pad),
                                                static_cast<uint8_t*>(q), sa, (flags & GK_FLAG_NATIVE_HALF) != 0,
                                                packed, static_cast<hipStream_t>(stream)));
}

// generic_dense_glue.cpp:424-431: approximate is 0 (exact GELU) or 1 (tanh form).
gk_status gk_gelu_and_mul_bf16(const void* gate_up, int64_t rows, int64_t width, int64_t ld_in, void* out,
                               int64_t ld_out, int approximate, void* stream) {
  if (approximate != 0 && approximate != 1) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  if (!gate_up || !out) return GK_INVALID_ARGUMENT;
  if (rows < 1 || width < 1 || rows > kMaxDim || width > kMaxDim / 2 || ld_in < 2 * width)
    return GK_INCOMPATIBLE_INPUT_SIZE;
  if (ld_out < width) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if ((reinterpret_cast<uintptr_t>(gate_up) | reinterpret_cast<uintptr_t>(out)) & 1) return GK_INCOMPATIBLE_DATA_TYPE;
  const gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_gelu_and_mul(static_cast<const uint16_t*>(gate_up), ld_in, static_cast<int>(rows),
                                          static_cast<int>(width), static_cast<uint16_t*>(out), ld_out,
                                          approximate != 0, static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_gelu_mul_quant_bf16(const void* gate_up, int64_t rows, int64_t width, int64_t ld_in,
                                     int approximate, void* q, float* sa, int64_t m_pad, uint32_t flags,
                                     void* stream) {
  if (approximate != 0 && approximate != 1) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  if (!gate_up || !q || !sa) return GK_INVALID_ARGUMENT;
  if (rows < 1 || width < 1 || rows > kMaxDim || width > kMaxDim / 2 || ld_in < 2 * width)
    return GK_INCOMPATIBLE_INPUT_SIZE;
  if (m_pad < rows || m_pad > kMaxDim) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (flags & ~uint32_t{GK_FLAG_NATIVE_HALF | GK_FLAG_DECODE_LAYOUT}) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  const bool packed = (flags & GK_FLAG_DECODE_LAYOUT) != 0;
  if (packed && m_pad != 16 && m_pad != 32 && m_pad != 64) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if ((reinterpret_cast<uintptr_t>(gate_up) & 1) || (reinterpret_cast<uintptr_t>(q) & 7) ||
      (reinterpret_cast<uintptr_t>(sa) & 3))
    return GK_INCOMPATIBLE_DATA_TYPE;
  const gk_status st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_gelu_mul_act_quant(static_cast<const uint16_t*>(gate_up), ld_in, static_cast<int>(rows),
                                                static_cast<int>(width), approximate != 0, static_cast<int>(m_pad),
                                                static_cast<uint8_t*>(q), sa, (flags & GK_FLAG_NATIVE_HALF) != 0,
                                                packed, static_cast<hipStream_t>(stream)));
}

// ---- RMSNorm ----------------------------------------------------------------------------
namespace {

// generic_dense_glue.cpp:146-160: epsilon finite and > 0 and weight_offset
// finite (else the layer configuration is unsupported), then 1 <= width <=
// 8192 and rows >= 1 (input size), then bf16 (2-byte aligned) tensors.
gk_status check_norm(const void* x, int64_t rows, int64_t width, int64_t ld_in, const void* gamma, float eps,
                     float off) {
  if (!x || !gamma) return GK_INVALID_ARGUMENT;
  if (!std::isfinite(eps) || eps <= 0.0f || !std::isfinite(off)) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  if (rows < 1 || rows > kMaxDim || width < 1 || width > gk::kNormMaxWidth || ld_in < width)
    return GK_INCOMPATIBLE_INPUT_SIZE;
  if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(gamma)) & 1) return GK_INCOMPATIBLE_DATA_TYPE;
  return GK_SUCCESS;
}

bool odd(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 1) != 0; }

}  // namespace

gk_status gk_rms_norm_bf16(const void* x, int64_t rows, int64_t width, int64_t ld_in, const void* gamma,
                           float epsilon, float weight_offset, void* out, int64_t ld_out, void* stream) {
  gk_status st = check_norm(x, rows, width, ld_in, gamma, epsilon, weight_offset);
  if (st != GK_SUCCESS) return st;
  if (!out) return GK_INVALID_ARGUMENT;
  if (ld_out < width) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (odd(out)) return GK_INCOMPATIBLE_DATA_TYPE;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_rms_norm(static_cast<const uint16_t*>(x), nullptr, ld_in,
                                      static_cast<const uint16_t*>(gamma), static_cast<int>(rows),
                                      static_cast<int>(width), epsilon, weight_offset, nullptr,
                                      static_cast<uint16_t*>(out), ld_out, nullptr, nullptr, 0, false, false,
                                      static_cast<hipStream_t>(stream)));
}

gk_status gk_fused_add_rms_norm_bf16(const void* x, const void* residual, int64_t rows, int64_t width,
                                     int64_t ld_in, const void* gamma, float epsilon, float weight_offset,
                                     void* residual_out, void* norm_out, int64_t ld_out, void* stream) {
  gk_status st = check_norm(x, rows, width, ld_in, gamma, epsilon, weight_offset);
  if (st != GK_SUCCESS) return st;
  if (!residual || !residual_out || !norm_out) return GK_INVALID_ARGUMENT;
  if (ld_out < width) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (odd(residual) || odd(residual_out) || odd(norm_out)) return GK_INCOMPATIBLE_DATA_TYPE;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_rms_norm(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(residual), ld_in,
                                      static_cast<const uint16_t*>(gamma), static_cast<int>(rows),
                                      static_cast<int>(width), epsilon, weight_offset,
                                      static_cast<uint16_t*>(residual_out), static_cast<uint16_t*>(norm_out), ld_out,
                                      nullptr, nullptr, 0, false, false, static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_rms_norm_quant_bf16(const void* x, const void* residual, int64_t rows, int64_t width,
                                     int64_t ld_in, const void* gamma, float epsilon, float weight_offset,
                                     void* residual_out, int64_t ld_out, void* q, float* sa, int64_t m_pad,
                                     uint32_t flags, void* stream) {
  gk_status st = check_norm(x, rows, width, ld_in, gamma, epsilon, weight_offset);
  if (st != GK_SUCCESS) return st;
  if (!q || !sa || (residual_out && !residual)) return GK_INVALID_ARGUMENT;
  if (flags & ~uint32_t{GK_FLAG_NATIVE_HALF | GK_FLAG_DECODE_LAYOUT}) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  const bool packed = (flags & GK_FLAG_DECODE_LAYOUT) != 0;
  if (m_pad < rows || m_pad > kMaxDim || (residual_out && ld_out < width)) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (packed && m_pad != 16 && m_pad != 32 && m_pad != 64) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (odd(residual) || odd(residual_out) || (reinterpret_cast<uintptr_t>(q) & 7) ||
      (reinterpret_cast<uintptr_t>(sa) & 3))
    return GK_INCOMPATIBLE_DATA_TYPE;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  return from_hip(gk::launch_rms_norm(static_cast<const uint16_t*>(x), static_cast<const uint16_t*>(residual), ld_in,
                                      static_cast<const uint16_t*>(gamma), static_cast<int>(rows),
                                      static_cast<int>(width), epsilon, weight_offset,
                                      static_cast<uint16_t*>(residual_out), nullptr, residual_out ? ld_out : 0,
                                      static_cast<uint8_t*>(q), sa, static_cast<int>(m_pad),
                                      (flags & GK_FLAG_NATIVE_HALF) != 0, packed, static_cast<hipStream_t>(stream)));
}

// ---- MoE ------------------------------------------------------------------------------
namespace {

struct MoeLayout {
  int64_t rows;  // padded rows (multiple of 256)
  int kparts;    // K split of the down GEMM (fp32 partial planes of z)
  size_t ids, wts, row_of, row_token, off, cnt, q1, sa1, q2, sa2, z, total;  // byte offsets
};

gk_status moe_rows(int64_t T, int64_t E, int top_k, int64_t* rows) {
  if (T < 1 || E < 1 || E > gk::kMoeMaxExperts || top_k < 1 || top_k > 2 || top_k > E || T > (int64_t{1} << 24))
    return GK_INCOMPATIBLE_INPUT_SIZE;
  *rows = round_up(T * top_k + (gk::kMoeRowAlign - 1) * E, gk::kMoeRowAlign);
  return GK_SUCCESS;
}

gk_status moe_layout(int64_t T, int64_t H, int64_t I, int64_t E, int top_k, MoeLayout* L) {
  if (H < 128 || I < 128 || H % 128 || I % 128 || H > kMaxDim || I > kMaxDim / 2) return GK_INCOMPATIBLE_INPUT_SIZE;
  // the gather quantizer takes one grid row (gridDim.y <= 65535) per 128-column group
  if (H / 128 > 65535 || I / 128 > 65535) return GK_INCOMPATIBLE_INPUT_SIZE;
  gk_status st = moe_rows(T, E, top_k, &L->rows);
  if (st != GK_SUCCESS) return st;
  // the grouped GEMMs address the gathered activations with 32-bit offsets
  if (L->rows * (H > I ? H : I) > int64_t{0xffffffff}) return GK_INCOMPATIBLE_INPUT_SIZE;
  const size_t R = static_cast<size_t>(L->rows), tk = static_cast<size_t>(T * top_k);
  size_t o = 0;
  auto take = [&o](size_t bytes) { const size_t at = o; o += align256(bytes); return at; };
  L->ids = take(tk * 4);
  L->wts = take(tk * 4);
  L->row_of = take(tk * 4);
  L->row_token = take(R * 4);
  L->off = take(static_cast<size_t>(E + 1) * 4);
  L->cnt = take(static_cast<size_t>(E) * 4);
  L->q1 = take(R * static_cast<size_t>(H));
  L->sa1 = take(R * static_cast<size_t>(H / 128) * 4);
  L->q2 = take(R * static_cast<size_t>(I));
  L->sa2 = take(R * static_cast<size_t>(I / 128) * 4);
  // The down GEMM has (rows / 256) * ceil(H / 256) workgroups at most: below two
  // per CU it splits K in two halves (fp32 partial planes summed by the combine).
  L->kparts = (L->rows / 256) * ((H + 255) / 256) < 512 ? 2 : 1;
  L->z = take(static_cast<size_t>(L->kparts) * R * static_cast<size_t>(H) * 4);
  L->total = o;
  return GK_SUCCESS;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace

gk_status gk_fp8_moe_rows_max(int64_t T, int64_t E, int top_k, int64_t* rows_max) {
  if (!rows_max) return GK_INVALID_ARGUMENT;
  return moe_rows(T, E, top_k, rows_max);
}

gk_status gk_fp8_moe_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int top_k, size_t* bytes) {
  if (!bytes) return GK_INVALID_ARGUMENT;
  MoeLayout L;
  const gk_status st = moe_layout(T, H, I, E, top_k, &L);
  if (st != GK_SUCCESS) return st;
  *bytes = L.total;
  return GK_SUCCESS;
}

gk_status gk_fp8_moe_route(const float* logits, int64_t T, int64_t E, int64_t ld_logits, int top_k, int32_t* ids,
                           float* wts, int32_t* row_of, int32_t* row_token, int64_t rows_max, int32_t* offsets,
                           void* stream) {
  if (!logits || !ids || !wts || !row_of || !row_token || !offsets) return GK_INVALID_ARGUMENT;
  int64_t rows = 0;
  gk_status st = moe_rows(T, E, top_k, &rows);
  if (st != GK_SUCCESS) return st;
  if (ld_logits < E) return GK_INCOMPATIBLE_INPUT_SIZE;
  if (rows_max < rows) return GK_INSUFFICIENT_BUFFER;
  if (rows_max > kMaxDim) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if ((reinterpret_cast<uintptr_t>(logits) | reinterpret_cast<uintptr_t>(ids) | reinterpret_cast<uintptr_t>(wts) |
       reinterpret_cast<uintptr_t>(row_of) | reinterpret_cast<uintptr_t>(row_token) |
       reinterpret_cast<uintptr_t>(offsets)) & 3)
    return GK_INCOMPATIBLE_DATA_TYPE;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  const gk::MoeRouting r{ids, wts, row_of, row_token, offsets, nullptr};
  // every entry of the caller's row_token buffer is defined: padding rows and
  // rows past the layout read -1
  return from_hip(gk::launch_moe_route(logits, static_cast<int>(T), static_cast<int>(E), ld_logits, top_k,
                                       static_cast<int>(rows_max), r, static_cast<hipStream_t>(stream)));
}

gk_status gk_fp8_moe_bf16(const void* x, int64_t T, int64_t H, int64_t ldx, const float* logits, int64_t E,
                          int64_t ld_logits, int top_k, const void* w_gu, const float* s_gu, int64_t I,
                          const void* w_dn, const float* s_dn, void* y, int64_t ldy, uint32_t flags,
                          void* workspace, size_t workspace_bytes, void* stream) {
  if (!x || !logits || !w_gu || !s_gu || !w_dn || !s_dn || !y || !workspace) return GK_INVALID_ARGUMENT;
  if (flags & ~uint32_t{GK_FLAG_NATIVE_HALF | GK_FLAG_WEIGHT_PACKED}) return GK_UNSUPPORTED_LAYER_CONFIGURATION;
  const bool wpack = (flags & GK_FLAG_WEIGHT_PACKED) != 0;
  MoeLayout L;
  gk_status st = moe_layout(T, H, I, E, top_k, &L);
  if (st != GK_SUCCESS) return st;
  if (ldx < H || ld_logits < E) return GK_INCOMPATIBLE_INPUT_SIZE;
  if (ldy < H) return GK_INCOMPATIBLE_OUTPUT_SIZE;
  if (workspace_bytes < L.total) return GK_INSUFFICIENT_BUFFER;
  if ((reinterpret_cast<uintptr_t>(workspace) & 255) || !aligned16(x) || !aligned16(y) || !aligned16(w_gu) ||
      !aligned16(w_dn) || ldx % 8 || ldy % 8 || (reinterpret_cast<uintptr_t>(s_gu) & 3) ||
      (reinterpret_cast<uintptr_t>(s_dn) & 3) || (reinterpret_cast<uintptr_t>(logits) & 3))
    return GK_INCOMPATIBLE_DATA_TYPE;
  st = current_device_ok();
  if (st != GK_SUCCESS) return st;
  hipStream_t s = static_cast<hipStream_t>(stream);
  uint8_t* ws = static_cast<uint8_t*>(workspace);
  const bool half = (flags & GK_FLAG_NATIVE_HALF) != 0;
  const int R = static_cast<int>(L.rows);
  const gk::MoeRouting r{reinterpret_cast<int32_t*>(ws + L.ids), reinterpret_cast<float*>(ws + L.wts),
                         reinterpret_cast<int32_t*>(ws + L.row_of), reinterpret_cast<int32_t*>(ws + L.row_token),
                         reinterpret_cast<int32_t*>(ws + L.off), reinterpret_cast<int32_t*>(ws + L.cnt)};
  hipError_t e = gk::launch_moe_route(logits, static_cast<int>(T), static_cast<int>(E), ld_logits, top_k, R, r, s);
  if (e != hipSuccess) return GK_DEVICE_ERROR;
  uint8_t* q1 = ws + L.q1;
  float* sa1 = reinterpret_cast<float*>(ws + L.sa1);
  e = gk::launch_act_quant_rows(static_cast<const uint16_t*>(x), ldx, static_cast<int>(H), r.row_of,
                                static_cast<int>(T), top_k, R, q1, sa1, half, s);
  if (e != hipSuccess) return GK_DEVICE_ERROR;
  // gate_up GEMM with the SiLU-and-mul and the 1x128 quantizer in its
  // epilogue: the down GEMM's codes and scales, no bf16 intermediate
  uint8_t* q2 = ws + L.q2;
  float* sa2 = reinterpret_cast<float*>(ws + L.sa2);
  gk::GemmArgs a{};
  a.qa = q1; a.sa = sa1; a.w = static_cast<const uint8_t*>(w_gu); a.sw = s_gu; a.bias = nullptr;
  a.y = nullptr; a.ldy = 0; a.M = R; a.N = static_cast<int>(2 * I); a.K = static_cast<int>(H);
  a.G = static_cast<int>(H / 128); a.Mpad = R; a.half_w = half; a.wpack = wpack;
  a.swiglu_q = q2; a.swiglu_s = sa2;
  e = gk::launch_gemm_grouped256(a, r.off, r.cnt, static_cast<int>(E), 1, nullptr, s);
  if (e != hipSuccess) return GK_DEVICE_ERROR;
  float* z = reinterpret_cast<float*>(ws + L.z);
  gk::GemmArgs d{};
  d.qa = q2; d.sa = sa2; d.w = static_cast<const uint8_t*>(w_dn); d.sw = s_dn; d.bias = nullptr;
  d.y = nullptr; d.ldy = H; d.M = R; d.N = static_cast<int>(H); d.K = static_cast<int>(I);
  d.G = static_cast<int>(I / 128); d.Mpad = R; d.half_w = half; d.wpack = wpack;
  e = gk::launch_gemm_grouped256(d, r.off, r.cnt, static_cast<int>(E), L.kparts, z, s);
  if (e != hipSuccess) return GK_DEVICE_ERROR;
  return from_hip(gk::launch_moe_combine(z, L.kparts, static_cast<int64_t>(R) * H, static_cast<int>(H), r.row_of,
                                         r.wts, static_cast<int>(T), top_k,
                                         static_cast<uint16_t*>(y), ldy, s));
}

}  // extern "C"
