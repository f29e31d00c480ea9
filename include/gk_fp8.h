/* gk_fp8.h -- C ABI of the MI355X (gfx950) block-FP8 library, libgk_fp8.so.
 *
 * This library replaces, for the block-FP8 W8A8 path of tracycam/gaudi-kernels,
 *   - the Synapse provider exports of csrc/host/generic_dense_glue.cpp:966-1013
 *     (GetKernelGuids / InstantiateTpcKernel / GetLibVersion) and the FP8 glue
 *     of csrc/host/generic_fp8_glue.hpp:31-349, and
 *   - the CPU-only Python helpers python/gaudi_kernels/block_fp8_oracle.py:11-46
 *     and python/gaudi_kernels/fp8_codec.py:14-53, whose numerics the kernels
 *     implement on the GPU.
 *
 * Conventions
 *   - Every buffer is caller-owned device memory (HIP); the library never
 *     allocates.  Scratch space is passed as a workspace whose size is asked
 *     for first (two-phase protocol, as the glue's ELF-size query in
 *     csrc/host/generic_attention_glue.hpp:84-90).  A GEMM workspace is
 *     256-byte aligned; calls that share a workspace must be ordered (one
 *     stream).
 *   - `stream` is a hipStream_t passed as void* (NULL = default stream).  All
 *     entry points are stream-ordered and asynchronous, except the codec and
 *     gk_fp8_check_inputs, which read a status word back and synchronize the
 *     stream (the reference raises ValueError synchronously there).
 *   - Return values are gk_status codes; the library never throws.  The
 *     rejection classes follow the glue's GLUE_* codes.
 *   - Layouts are row-major: activations x bf16 [M, K] (row stride ldx
 *     elements), weights E4M3 codes [N, K] (row stride K bytes), block scales
 *     fp32 [ceil(N/128), ceil(K/128)], bias fp32 [N], output bf16 [M, N] (row
 *     stride ldy elements).
 */
#ifndef GK_FP8_H
#define GK_FP8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum gk_status {
  GK_SUCCESS = 0,                          /* GLUE_SUCCESS */
  GK_INCOMPATIBLE_INPUT_SIZE = 1,          /* GLUE_INCOMPATIBLE_INPUT_SIZE (shapes, scale grid) */
  GK_INCOMPATIBLE_OUTPUT_SIZE = 2,         /* GLUE_INCOMPATIBLE_OUTPUT_SIZE */
  GK_INCOMPATIBLE_DATA_TYPE = 3,           /* GLUE_INCOMPATIBLE_DATA_TYPE (alignment of typed buffers) */
  GK_UNSUPPORTED_LAYER_CONFIGURATION = 4,  /* GLUE_UNSUPPORTED_LAYER_CONFIGURATION (flags) */
  GK_INSUFFICIENT_BUFFER = 5,              /* GLUE_INSUFFICIENT_ELF_BUFFER (workspace or name array too small) */
  GK_NODE_NOT_FOUND = 6,                   /* GLUE_NODE_NOT_FOUND (unknown op name) */
  GK_INVALID_ARGUMENT = 7,                 /* NULL pointer where a buffer is required */
  GK_NONFINITE_CODE = 8,                   /* OCP NaN code (fp8_codec.py:48-49) / half code without OCP image */
  GK_INVALID_SCALE = 9,                    /* negative or nonfinite scale (fp8_codec.py:26-29) */
  GK_SCALE_OVERFLOW = 10,                  /* doubling a scale overflows fp32 (fp8_codec.py:30-32) */
  GK_INEXACT_SCALE = 11,                   /* halving a scale is inexact (inverse codec) */
  GK_NONFINITE_INPUT = 12,                 /* nonfinite activation / weight (block_fp8_oracle.py:22-24) */
  GK_UNSUPPORTED_DEVICE = 13,              /* device is not gfx950 (DEVICE_ID_GAUDI2 gate, generic_dense_glue.cpp:969) */
  GK_DEVICE_ERROR = 14                     /* HIP runtime error */
} gk_status;

/* GEMM flags. */
#define GK_FLAG_NATIVE_HALF 1u     /* block_fp8_oracle.py:31-35: half-range activations and weights, scales x2 */
#define GK_FLAG_FORCE_DECODE 2u    /* force the M <= 16 weight-streaming variant (requires M <= 16) */
#define GK_FLAG_FORCE_PREFILL 4u   /* force the LDS-tiled MFMA variant */
#define GK_FLAG_FORCE_GENERIC 8u   /* force the any-shape variant */

/* Variants reported by gk_fp8_block_gemm_plan. */
#define GK_VARIANT_DECODE 1
#define GK_VARIANT_PREFILL 2
#define GK_VARIANT_GENERIC 3

/* ---- provider surface ------------------------------------------------------ */

/* Library ABI version.  Replaces GetLibVersion (generic_dense_glue.cpp:1013). */
uint64_t gk_lib_version(void);

/* Op names, count-query idiom of GetKernelGuids (generic_dense_glue.cpp:966-981):
 * *count is the capacity of `names` on entry and the number of ops on return;
 * names == NULL (or capacity 0) only queries the count.  Names are static. */
gk_status gk_list_ops(uint32_t* count, const char** names);

/* GK_SUCCESS if `device` is a gfx950 GPU, GK_UNSUPPORTED_DEVICE otherwise.
 * Replaces the DEVICE_ID_GAUDI2 gate of GetKernelGuids (generic_dense_glue.cpp:969). */
gk_status gk_device_supported(int device);

/* ---- load-time codec (fp8_codec.py:14-53) ------------------------------------ */

/* Workspace bytes for the two codec entry points (status word + rounded count). */
gk_status gk_fp8_codec_workspace_bytes(size_t* bytes);

/* OCP E4M3FN codes -> Gaudi2 half-range codes (value / 2, RNE), scales x2.
 * Replaces reencode_e4m3fn_half (fp8_codec.py:14-53): src/dst n codes,
 * scales/scales_out n_scales fp32, *rounded = number of rounded codes.
 * Errors (checked in this order, as the reference does): GK_INVALID_SCALE,
 * GK_SCALE_OVERFLOW, GK_NONFINITE_CODE.  src and scales are never modified;
 * dst / scales_out are unspecified on error.  Synchronizes `stream`. */
gk_status gk_fp8_codec_ocp_to_half(const void* src, void* dst, int64_t n, const float* scales,
                                   float* scales_out, int64_t n_scales, int64_t* rounded, void* workspace,
                                   size_t workspace_bytes, void* stream);

/* Inverse codec (no reference function; SURVEY a2'): half-range codes ->
 * OCP E4M3FN (value x2, exact), scales / 2.  Magnitudes >= 0x77 have no OCP
 * image -> GK_NONFINITE_CODE; a scale whose half is an inexact fp32
 * subnormal -> GK_INEXACT_SCALE.  Synchronizes `stream`. */
gk_status gk_fp8_codec_half_to_ocp(const void* src, void* dst, int64_t n, const float* scales,
                                   float* scales_out, int64_t n_scales, void* workspace, size_t workspace_bytes,
                                   void* stream);

/* ---- activation quantization ------------------------------------------------ */

/* Per-row 1x128 E4M3 quantization with the oracle's scale rule
 * (block_fp8_oracle.py:25-28; native_half adds :32,:34).  Replaces the
 * gk_fp8_block_quant_bf16_v1 op (activation_native.c:9-30, glue
 * generic_fp8_glue.hpp:84-109) in that op's group-major layout ({128, R, G}
 * FCD-first): q codes [G][m_pad][128] (G = ceil(k/128)), sa fp32 [G][m_pad];
 * rows >= m and columns >= k are written as zero.  m_pad >= m. */
gk_status gk_fp8_act_quant_bf16(const void* x, int64_t m, int64_t k, int64_t ldx, void* q, float* sa,
                                int64_t m_pad, uint32_t flags, void* stream);

/* ---- block-FP8 GEMM ------------------------------------------------------------ */

/* Plan query: which variant runs for (m, n, k, flags, weight pointer
 * alignment), the row padding of its quantized activations and the workspace
 * bytes gk_fp8_block_gemm_bf16 needs.  Any output pointer may be NULL. */
gk_status gk_fp8_block_gemm_plan(int64_t m, int64_t n, int64_t k, uint32_t flags, const void* w, int* variant,
                                 int64_t* m_pad, size_t* workspace_bytes);

/* y = bf16( sum_g P_g * sa * sw + bias ), block_fp8_oracle.py:11-46 on the
 * GPU for any M >= 1.  Replaces the Gaudi2 decode chain quant -> MME ->
 * gk_fp8_block_reduce_bf16_v1 (reduce_bias.c:204-258) and the prefill chain
 * act_row_scale -> quant_act_fp16_1k -> dequant_weight_fp16_1k -> MME ->
 * epilogue(_bias) (fp8_hybrid_tpcsim_test.cpp:180-324).  Dispatch by M:
 * M <= 16 streams weights (decode), larger M runs the LDS-tiled MFMA kernel
 * (prefill).  The activations are quantized into the workspace first.  scale_rows x scale_cols must equal ceil(n/128) x ceil(k/128)
 * (GK_INCOMPATIBLE_INPUT_SIZE otherwise, as generic_fp8_glue_test.cpp:98-100).
 * bias may be NULL.  Inputs are not checked for NaN (see gk_fp8_check_inputs). */
gk_status gk_fp8_block_gemm_bf16(const void* x, int64_t m, int64_t k, int64_t ldx, const void* w, int64_t n,
                                 const float* scales, int64_t scale_rows, int64_t scale_cols, const float* bias,
                                 void* y, int64_t ldy, uint32_t flags, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* The same GEMM on activations already quantized by gk_fp8_act_quant_bf16
 * (q [G][m_pad][128], sa [G][m_pad]); m_pad must equal the plan's m_pad for
 * these flags.  No workspace.  (The second half of the Gaudi2 decode chain:
 * MME partials + reduce_bias.c, fused.) */
gk_status gk_fp8_block_gemm_q_bf16(const void* q, const float* sa, int64_t m, int64_t m_pad, int64_t k,
                                   const void* w, int64_t n, const float* scales, int64_t scale_rows,
                                   int64_t scale_cols, const float* bias, void* y, int64_t ldy, uint32_t flags,
                                   void* stream);

/* Finite-input check of block_fp8_oracle.py:22-24 on device buffers: every
 * activation finite, no OCP NaN weight code, every scale finite and >= 0.
 * Returns GK_NONFINITE_INPUT / GK_SUCCESS.  Uses the codec workspace.
 * Synchronizes `stream`. */
gk_status gk_fp8_check_inputs(const void* x, int64_t m, int64_t k, int64_t ldx, const void* w, int64_t n,
                              const float* scales, int64_t n_scales, void* workspace, size_t workspace_bytes,
                              void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GK_FP8_H */
