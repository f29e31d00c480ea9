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
#define GK_FLAG_FORCE_DECODE 2u    /* force the weight-streaming variant (requires M <= 64) */
#define GK_FLAG_FORCE_PREFILL 4u   /* force the LDS-tiled MFMA variant */
#define GK_FLAG_FORCE_GENERIC 8u   /* force the any-shape variant */
#define GK_FLAG_DECODE_LAYOUT 16u  /* act_quant / q GEMM only: quantized activations in the decode fragment layout */
#define GK_FLAG_WEIGHT_PACKED 32u  /* block GEMMs: weights packed by gk_fp8_pack_weight (not the generic variant);
                                      MoE layer: experts packed by gk_fp8_pack_experts (op gk_fp8_moe_bf16_v2) */
#define GK_FLAG_ACCUMULATE 64u     /* K-slice GEMM only: add into the fp32 partial instead of overwriting it */

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

/* Inverse codec (no reference function): half-range codes ->
 * OCP E4M3FN (value x2, exact), scales / 2.  Magnitudes >= 0x77 have no OCP
 * image -> GK_NONFINITE_CODE; a scale whose half is an inexact fp32
 * subnormal -> GK_INEXACT_SCALE.  Synchronizes `stream`. */
gk_status gk_fp8_codec_half_to_ocp(const void* src, void* dst, int64_t n, const float* scales,
                                   float* scales_out, int64_t n_scales, void* workspace, size_t workspace_bytes,
                                   void* stream);

/* ---- load-time weight packing ------------------------------------------------------ */

/* The layout packing step that fp8_codec.py:19 leaves to the loader ("layout
 * packing is a separate step"; the Gaudi2 runtime packs to [G, N, 128]).
 * Here the packed layout is the fragment order of the gfx950 FP8 matrix
 * instructions: for each 16-row tile t < ceil(n/16) and 128-K group g < k/128
 * a 2 KB block at (t * G + g) * 2048 whose 16-byte piece (h, l), h < 2,
 * l < 64, at h*1024 + 16 l holds bytes [128 g + 32 (l/16) + 16 h, +16) of
 * row 16 t + l%16 (zeros for rows >= n).  Each wave of the GEMM kernels then
 * reads a tile's group as two contiguous 1 KB loads.  Requires k % 128 == 0.
 * Block scales are not packed.  Codes are copied unchanged (OCP or half
 * range alike). */
gk_status gk_fp8_packed_weight_bytes(int64_t n, int64_t k, size_t* bytes);

/* w E4M3 codes [n, k] (row stride k) -> packed (packed_bytes >= the size
 * above, 16-byte aligned).  Stream-ordered, no synchronization. */
gk_status gk_fp8_pack_weight(const void* w, int64_t n, int64_t k, void* packed, size_t packed_bytes,
                             void* stream);

/* Expert weights for the MoE layer (gk_fp8_moe_bf16 with GK_FLAG_WEIGHT_PACKED):
 * w E4M3 codes [e, n, k] (contiguous) -> packed, expert i at byte
 * i * gk_fp8_packed_weight_bytes(n, k) (packed_bytes >= e times that, 16-byte
 * aligned).  The same 2 KB blocks as gk_fp8_pack_weight in panel-major order:
 * tiles in panels of 16 (256 rows), panel p's blocks starting at block
 * 16 * G * p, group by group, each group's nbp = min(16, T - 16 p) tiles side
 * by side (block 16 G p + g nbp + t % 16, T = ceil(n/16), G = k/128), so the
 * grouped GEMM reads each step's 256-row weight tile as one contiguous run.
 * No reference function: the reference has no MoE code (pack_weight's
 * fp8_codec.py:19 note applies).  Stream-ordered, no synchronization. */
gk_status gk_fp8_pack_experts(const void* w, int64_t e, int64_t n, int64_t k, void* packed, size_t packed_bytes,
                              void* stream);

/* ---- activation quantization ------------------------------------------------ */

/* Per-row 1x128 E4M3 quantization with the oracle's scale rule
 * (block_fp8_oracle.py:25-28; native_half adds :32,:34).  Replaces the
 * gk_fp8_block_quant_bf16_v1 op (activation_native.c:9-30, glue
 * generic_fp8_glue.hpp:84-109) in that op's group-major layout ({128, R, G}
 * FCD-first): q codes [G][m_pad][128] (G = ceil(k/128)), sa fp32 [G][m_pad];
 * rows >= m and columns >= k are written as zero.  m_pad >= m.
 * flags: GK_FLAG_NATIVE_HALF; GK_FLAG_DECODE_LAYOUT (m_pad must be 16, 32 or
 * 64: 16 tokens per tile, T = m_pad/16 tiles) writes q in the decode fragment
 * layout the M <= 64 GEMM reads with coalesced loads: the 2 KB block of group
 * g and token tile t sits at (g*T + t)*2048, and its 16-byte piece (h, l),
 * h < 2, l < 64, at + h*1024 + 16 l holds bytes [32 (l/16) + 16 h, +16) of
 * row 16 t + l%16.  sa keeps its [G][m_pad] layout. */
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
 * M <= 64 streams weights (decode: one to four 16-token tiles share each
 * weight fragment), larger M runs the LDS-tiled MFMA kernel (prefill).  The activations are quantized into the workspace first.  scale_rows x scale_cols must equal ceil(n/128) x ceil(k/128)
 * (GK_INCOMPATIBLE_INPUT_SIZE otherwise, as generic_fp8_glue_test.cpp:98-100).
 * bias may be NULL.  Inputs are not checked for NaN (see gk_fp8_check_inputs).
 * GK_FLAG_WEIGHT_PACKED: w is gk_fp8_pack_weight's output for (n, k); the
 * results are bit-identical to those on the row-major weights. */
gk_status gk_fp8_block_gemm_bf16(const void* x, int64_t m, int64_t k, int64_t ldx, const void* w, int64_t n,
                                 const float* scales, int64_t scale_rows, int64_t scale_cols, const float* bias,
                                 void* y, int64_t ldy, uint32_t flags, void* workspace, size_t workspace_bytes,
                                 void* stream);

/* Scratch of gk_fp8_block_gemm_bf16_noalloc (bytes, per GPU): enough for
 * the quantized activations of config 4's M = 4096, K = 7168.  The array is
 * part of the library's code object, so loading the library reserves these
 * 32 MiB of device memory on every GPU the process runs the library's
 * kernels on, whether or not this entry point is ever called. */
#define GK_NOALLOC_SCRATCH_BYTES (32u << 20)

/* gk_fp8_block_gemm_bf16 without a workspace argument and without any
 * allocation.  No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).  The quantized activations go to
 * a fixed scratch array of GK_NOALLOC_SCRATCH_BYTES in the library's code
 * object, one per GPU, held until the process ends; plans needing more
 * (gk_fp8_block_gemm_plan's workspace_bytes) -> GK_INSUFFICIENT_BUFFER before
 * any device work.  Results are those of gk_fp8_block_gemm_bf16 bit for bit.
 * Every call on one GPU shares that GPU's scratch: calls that overlap in time
 * on one GPU (different streams, or several host threads) race and must be
 * ordered by the caller. */
gk_status gk_fp8_block_gemm_bf16_noalloc(const void* x, int64_t m, int64_t k, int64_t ldx, const void* w, int64_t n,
                                         const float* scales, int64_t scale_rows, int64_t scale_cols,
                                         const float* bias, void* y, int64_t ldy, uint32_t flags, void* stream);

/* The same GEMM on activations already quantized by gk_fp8_act_quant_bf16
 * (q [G][m_pad][128], sa [G][m_pad]); m_pad must equal the plan's m_pad for
 * these flags.  GK_FLAG_DECODE_LAYOUT: q is in the decode fragment layout
 * (the plan must be the decode variant).  No workspace.  (The second half of the Gaudi2 decode chain:
 * MME partials + reduce_bias.c, fused.) */
gk_status gk_fp8_block_gemm_q_bf16(const void* q, const float* sa, int64_t m, int64_t m_pad, int64_t k,
                                   const void* w, int64_t n, const float* scales, int64_t scale_rows,
                                   int64_t scale_cols, const float* bias, void* y, int64_t ldy, uint32_t flags,
                                   void* stream);

/* One K range of the block-FP8 GEMM, as an fp32 partial: the chunked-K form
 * of the reference's prefill chain, whose activation quantizer takes a
 * col_offset (gk_fp8_quant_act_fp16_1k_v1, generic_fp8_glue.hpp:233-273;
 * fp8_hybrid_tpcsim_test.cpp:253-302 accumulates c0 over K chunks), and the
 * per-shard GEMM of a row-parallel (K-sharded) linear layer.
 *   partial[i][j] (+)= sum over groups g in [k_offset/128, (k_offset+k_len)/128)
 *                      of P_g[i][j] * sa[i][g] * sw[j/128][g]
 * x bf16 [m, k] (row stride ldx; only columns [k_offset, k_offset + k_len)
 * are read), w codes [n, k] (row-major, or packed for (n, k) with
 * GK_FLAG_WEIGHT_PACKED), scales the whole [ceil(n/128), k/128] grid,
 * partial fp32 [m, n] (row stride ldp).  The activation groups of the range
 * are quantized exactly as in gk_fp8_block_gemm_bf16.  GK_FLAG_ACCUMULATE adds
 * the range's sum to what partial holds.  No bias; finish with
 * gk_fp8_partial_finish_bf16 (directly, or after gk_rank_sum_f32 over the
 * shards' partials).
 * Rules (the col_offset rules of generic_fp8_glue.hpp:169-176, :245-252):
 * k_offset < 0 or not a multiple of 128 -> GK_UNSUPPORTED_LAYER_CONFIGURATION;
 * k or k_len not a nonzero multiple of 128, or k_offset + k_len > k (e.g.
 * offset 384 + 256 > 512, generic_fp8_glue_test.cpp:216-218) ->
 * GK_INCOMPATIBLE_INPUT_SIZE.  The workspace is gk_fp8_block_gemm_plan(m, n,
 * k_len, flags, w) bytes; the variant is that plan's (decode for m <= 64, the
 * LDS-tiled kernel above; the generic variant is not offered here).  On the
 * LDS-tiled kernel the sums start from partial when accumulating, so
 * consecutive ranges accumulated over several calls give the bits of one call
 * over their union; the decode kernel splits each range over its waves, so
 * there the bits depend on the ranges (each call within the GEMM gate). */
gk_status gk_fp8_block_gemm_kslice_f32(const void* x, int64_t m, int64_t k, int64_t ldx, int64_t k_offset,
                                       int64_t k_len, const void* w, int64_t n, const float* scales,
                                       int64_t scale_rows, int64_t scale_cols, float* partial, int64_t ldp,
                                       uint32_t flags, void* workspace, size_t workspace_bytes, void* stream);

/* y[i][j] = bf16(partial[i][j] + bias[j]) (one fp32 addition, one rounding to
 * nearest even; bias may be NULL): the final step of the decode reduce
 * (csrc/tpc/block_fp8_framework/reduce_bias.c:42-57) on an fp32 partial
 * [rows, width] (row stride ldp) -> bf16 [rows, width] (row stride ldy). */
gk_status gk_fp8_partial_finish_bf16(const float* partial, int64_t rows, int64_t width, int64_t ldp,
                                     const float* bias, void* y, int64_t ldy, void* stream);

/* ---- row-parallel rank sum ------------------------------------------------------ */

/* The reference's gk_rank_sum_f32_v1 / gk_rank_sum_bf16_v1
 * (csrc/tpc/generic_dense/rank_sum.c:4-42, glue generic_dense_glue.cpp:568-600):
 * gathered holds world_size contiguous slices of `elems` values (slice r at
 * r * elems, as an all-gather leaves them); dst[i] = ((s_0[i] + s_1[i]) +
 * s_2[i]) + ... in fp32, in rank order.  The bf16 form widens each slice,
 * sums the same way and rounds once to bf16 (nearest even).  Checks, in the
 * glue's order: world_size outside [2, 8] ->
 * GK_UNSUPPORTED_LAYER_CONFIGURATION; misaligned buffers ->
 * GK_INCOMPATIBLE_DATA_TYPE; elems < 1 or elems * world_size beyond int32 ->
 * GK_INCOMPATIBLE_OUTPUT_SIZE; gathered_elems != elems * world_size ->
 * GK_INCOMPATIBLE_INPUT_SIZE.  Stream-ordered. */
gk_status gk_rank_sum_f32(const float* gathered, int64_t gathered_elems, int world_size, float* dst, int64_t elems,
                          void* stream);
gk_status gk_rank_sum_bf16(const void* gathered, int64_t gathered_elems, int world_size, void* dst, int64_t elems,
                           void* stream);

/* Shape inference of the rank sum (infer_rank_sum, generic_dense_glue.cpp:871-895):
 * *elems = gathered_elems / world_size; world_size outside [2, 8] ->
 * GK_UNSUPPORTED_LAYER_CONFIGURATION; gathered_elems < world_size or not a
 * multiple of it -> GK_INCOMPATIBLE_INPUT_SIZE. */
gk_status gk_rank_sum_infer(int64_t gathered_elems, int world_size, int64_t* elems);

/* Finite-input check of block_fp8_oracle.py:22-24 on device buffers: every
 * activation finite, no OCP NaN weight code, every scale finite and >= 0.
 * Returns GK_NONFINITE_INPUT / GK_SUCCESS.  Uses the codec workspace.
 * Synchronizes `stream`. */
gk_status gk_fp8_check_inputs(const void* x, int64_t m, int64_t k, int64_t ldx, const void* w, int64_t n,
                              const float* scales, int64_t n_scales, void* workspace, size_t workspace_bytes,
                              void* stream);

/* ---- per-token / per-channel W8A8 -------------------------------------------------- */

/* The reference's gk_fp8_token_quant_bf16_v1 (csrc/tpc/block_fp8_framework/
 * activation_token.c:4-26, glue generic_fp8_glue.hpp:31-50): x bf16 [rows,
 * width] (width a multiple of 128, row stride ldx) -> q [rows, width]
 * Gaudi2 half-range E4M3 codes (row stride ldq, a multiple of 8) and one fp32
 * scale per row, scales[r] = 2 * s_r with s_r = max|x_r| / 448 (FMA-refined;
 * 1 / 448 for an all-zero row).  Each code is the E4M3 round-to-nearest-even
 * of min(|x / s_r|, 448), halved into the half range (codec rule). */
gk_status gk_fp8_token_quant_bf16(const void* x, int64_t rows, int64_t width, int64_t ldx, void* q, int64_t ldq,
                                  float* scales, void* stream);

/* The reference's gk_fp8_channel_finish_bf16_v1 (channel_finish.c:2-18, glue
 * generic_fp8_glue.hpp:52-82): fp32 partial [rows, width] (width a multiple
 * of 128) -> y[r][c] = bf16(fma(partial[r][c] * act_scales[r], w_scales[c],
 * bias[c])), the product rounded to fp32 first; bias may be NULL (zero). */
gk_status gk_fp8_channel_finish_bf16(const float* partial, int64_t rows, int64_t width, int64_t ldp,
                                     const float* act_scales, const float* w_scales, const float* bias, void* y,
                                     int64_t ldy, void* stream);

/* The per-token / per-channel GEMM: the MME product of the reference chain
 * (token quant -> MME -> channel finish) fused with the channel finish.
 * q: E4M3 codes [m, k] (row stride ldq, a multiple of 16; half-range codes
 * from gk_fp8_token_quant_bf16 are read as the OCP codes of half their value,
 * which the doubled scales restore), sa [m]; w: codes [n, k] (16-byte
 * aligned, k a multiple of 128), sw [n] per output channel; bias [n] or NULL.
 * y[i][j] = bf16(fma(P[i][j] * sa[i], sw[j], bias[j])), P the fp32 sum of the
 * code products over k.  M <= 16 streams the weights; larger M runs the
 * 256 x 256 MFMA kernel.  flags must be 0. */
gk_status gk_fp8_channel_gemm_bf16(const void* q, int64_t ldq, const float* sa, int64_t m, int64_t k, const void* w,
                                   int64_t n, const float* sw, const float* bias, void* y, int64_t ldy,
                                   uint32_t flags, void* stream);

/* The per-token quantizer fused into the per-channel GEMM for decode batches
 * (build-defined; the reference chains three ops: activation_token.c:4-26,
 * the MME, channel_finish.c:2-18).  x bf16 [m, k] (16-byte aligned, row
 * stride ldx a multiple of 8, m <= 16, k a multiple of 128); w, sw, bias, y
 * as gk_fp8_channel_gemm_bf16.  y equals gk_fp8_token_quant_bf16 followed by
 * gk_fp8_channel_gemm_bf16 bit for bit, in one launch that streams the
 * weights once.  m > 16 -> GK_INCOMPATIBLE_INPUT_SIZE (call the two ops).
 * flags must be 0. */
gk_status gk_fp8_token_channel_gemm_bf16(const void* x, int64_t ldx, int64_t m, int64_t k, const void* w, int64_t n,
                                         const float* sw, const float* bias, void* y, int64_t ldy, uint32_t flags,
                                         void* stream);

/* ---- SiLU-and-mul ------------------------------------------------------------ */

/* The reference's gk_silu_and_mul_bf16_v1 (csrc/tpc/generic_dense/
 * silu_and_mul_bf16.c, glue generic_dense_glue.cpp:196-236): gate_up bf16
 * [rows, 2*width] (gate = columns [0, width), up = [width, 2*width), row
 * stride ld_in >= 2*width) -> out bf16 [rows, width] (row stride ld_out),
 * out = bf16(silu(gate) * up) in fp32, silu(g) = g / (1 + e^-g), g <= -88 ->
 * 0, NaN -> NaN, +inf -> NaN. */
gk_status gk_silu_and_mul_bf16(const void* gate_up, int64_t rows, int64_t width, int64_t ld_in, void* out,
                               int64_t ld_out, void* stream);

/* The same products quantized per 1x128 group for the next block-FP8 GEMM
 * (no reference op; saves the bf16 round trip of the products): codes and scales exactly as gk_fp8_act_quant_bf16 would write
 * for the bf16 output of gk_silu_and_mul_bf16 (q [G][m_pad][128], sa
 * [G][m_pad], G = ceil(width/128); flags GK_FLAG_NATIVE_HALF,
 * GK_FLAG_DECODE_LAYOUT with m_pad = 16, 32 or 64 as there). */
gk_status gk_fp8_silu_mul_quant_bf16(const void* gate_up, int64_t rows, int64_t width, int64_t ld_in, void* q,
                                     float* sa, int64_t m_pad, uint32_t flags, void* stream);

/* The reference's gk_gelu_and_mul_bf16_v1 (csrc/tpc/generic_dense/
 * gelu_and_mul_bf16.c:4-49, glue generic_dense_glue.cpp:424-458): shape rules
 * of gk_silu_and_mul_bf16, out = bf16(gelu(gate) * up) with the product in
 * fp32; approximate = 0 is the exact GELU x * erfc(-x/sqrt(2)) / 2, 1 the tanh
 * form x * sigmoid(2 sqrt(2/pi) (x + 0.044715 x^3)) (0 for x <= -15); any
 * other value -> GK_UNSUPPORTED_LAYER_CONFIGURATION.  fp32 evaluation through
 * the device library's erfcf / expf; the output is within one bf16 ulp of
 * the fp64 value (the reference test's bound). */
gk_status gk_gelu_and_mul_bf16(const void* gate_up, int64_t rows, int64_t width, int64_t ld_in, void* out,
                               int64_t ld_out, int approximate, void* stream);

/* The same products quantized per 1x128 group (no reference op), as
 * gk_fp8_silu_mul_quant_bf16: codes and scales exactly as
 * gk_fp8_act_quant_bf16 would write for the output of gk_gelu_and_mul_bf16. */
gk_status gk_fp8_gelu_mul_quant_bf16(const void* gate_up, int64_t rows, int64_t width, int64_t ld_in,
                                     int approximate, void* q, float* sa, int64_t m_pad, uint32_t flags,
                                     void* stream);

/* ---- RMSNorm ------------------------------------------------------------------ */

/* The reference's gk_rms_norm_bf16_v1 (csrc/tpc/generic_dense/rms_norm_bf16.c:4-53,
 * glue csrc/host/generic_dense_glue.cpp:135-190): x bf16 [rows, width] (row
 * stride ld_in), gamma bf16 [width] -> out bf16 [rows, width] (row stride
 * ld_out), out = bf16((x * inv) * (gamma + weight_offset)) with
 * inv = 1 / sqrt(sum(x^2) * (1/width) + epsilon) per row.  The sum of squares
 * is taken exactly (fp64, fixed order) and rounded to fp32 once; inv is
 * fp32(1 / sqrt) of the fp32 argument; the products are fp32.  As the glue:
 * epsilon must be finite and > 0 and weight_offset finite
 * (GK_UNSUPPORTED_LAYER_CONFIGURATION), 1 <= width <= 8192 and rows >= 1
 * (GK_INCOMPATIBLE_INPUT_SIZE). */
gk_status gk_rms_norm_bf16(const void* x, int64_t rows, int64_t width, int64_t ld_in, const void* gamma,
                           float epsilon, float weight_offset, void* out, int64_t ld_out, void* stream);

/* The reference's gk_fused_add_rms_norm_bf16_v1 (fused_add_rms_norm_bf16.c:4-63,
 * same glue): residual_out = bf16(x + residual) (fp32 sum, one rounding),
 * norm_out = gk_rms_norm_bf16 of residual_out.  x and residual share ld_in,
 * both outputs ld_out. */
gk_status gk_fused_add_rms_norm_bf16(const void* x, const void* residual, int64_t rows, int64_t width,
                                     int64_t ld_in, const void* gamma, float epsilon, float weight_offset,
                                     void* residual_out, void* norm_out, int64_t ld_out, void* stream);

/* The same normalized rows quantized per 1x128 group for the next block-FP8
 * GEMM (no reference op; the upstream fusion of the activation quantizer into
 * the norm): codes and scales exactly as gk_fp8_act_quant_bf16 would write for
 * norm_out (q [G][m_pad][128], sa [G][m_pad], G = ceil(width/128); flags
 * GK_FLAG_NATIVE_HALF, GK_FLAG_DECODE_LAYOUT with m_pad = 16, 32 or 64).
 * residual may be NULL (plain RMSNorm); with a residual, residual_out (row
 * stride ld_out) may be NULL. */
gk_status gk_fp8_rms_norm_quant_bf16(const void* x, const void* residual, int64_t rows, int64_t width,
                                     int64_t ld_in, const void* gamma, float epsilon, float weight_offset,
                                     void* residual_out, int64_t ld_out, void* q, float* sa, int64_t m_pad,
                                     uint32_t flags, void* stream);

/* ---- block-FP8 MoE layer ------------------------------------
 * No reference function: the reference has no MoE code for this path.  The
 * layer is build-defined from the reference's pieces (oracle/moe.py restates
 * it on the CPU): top-k (k = 1 or 2) experts per token by router logit, ties
 * to the lower expert index, combine weights = softmax over the selected
 * logits; rows grouped by expert in token order, each expert's segment padded
 * to 256 rows; gate_up GEMM (block_fp8_oracle.py numerics) -> bf16 ->
 * h = bf16(silu(gate) * up) (csrc/tpc/generic_dense/silu_and_mul_bf16.c) ->
 * down GEMM -> y = bf16(sum_k w_k z_k).
 *
 * Shapes: x bf16 [T, H] (row stride ldx), logits fp32 [T, E] (row stride
 * ld_logits), w_gu E4M3 [E, 2I, H] (gate rows 0..I-1, up rows I..2I-1) with
 * scales fp32 [E, 2I/128, H/128], w_dn E4M3 [E, H, I] with scales fp32
 * [E, H/128, I/128], y bf16 [T, H] (row stride ldy).  H and I multiples of
 * 128 up to 65535 * 128, E <= 256; x, y, weights 16-byte aligned with ldx, ldy multiples of 8.
 * flags: GK_FLAG_NATIVE_HALF; GK_FLAG_WEIGHT_PACKED: w_gu and w_dn are
 * gk_fp8_pack_experts outputs (the results are bit-identical). */

/* Padded row count of the expert-sorted layout: an upper bound of
 * sum_e round_up(count_e, 256), i.e. round_up(T*top_k + 255*E, 256). */
gk_status gk_fp8_moe_rows_max(int64_t T, int64_t E, int top_k, int64_t* rows_max);

gk_status gk_fp8_moe_workspace_bytes(int64_t T, int64_t H, int64_t I, int64_t E, int top_k, size_t* bytes);

/* Routing only: ids int32 [T, k], wts fp32 [T, k], row_of int32 [T, k]
 * (padded row of each slot), row_token int32 [rows_max] (every entry is
 * written: the token of each routed row, -1 for padding rows and for rows at
 * or past offsets[E]), offsets int32 [E + 1] (padded segment starts;
 * offsets[E] = rows in use).  rows_max below gk_fp8_moe_rows_max ->
 * GK_INSUFFICIENT_BUFFER; every buffer 4-byte aligned. */
gk_status gk_fp8_moe_route(const float* logits, int64_t T, int64_t E, int64_t ld_logits, int top_k, int32_t* ids,
                           float* wts, int32_t* row_of, int32_t* row_token, int64_t rows_max, int32_t* offsets,
                           void* stream);

/* The whole layer, stream-ordered and asynchronous.  After the call the
 * workspace holds the routing and the intermediates, in this order, each
 * region starting at a 256-byte boundary (R = rows_max, G_H = H/128,
 * G_I = I/128): ids, wts, row_of [T*k] x 4 B; row_token [R] int32;
 * offsets [E+1] int32; counts [E] int32 (live rows of each expert); gathered
 * codes [G_H][R][128] u8 and scales [G_H][R] fp32; SiLU-and-mul codes
 * [G_I][R][128] u8 and scales [G_I][R] fp32 (the gate_up GEMM writes them
 * from its epilogue: its bf16 output is not stored);
 * down output fp32 [P][R][H], P = 2 partial sums over the two halves of I
 * when (R/256) * ceil(H/256) < 512, else P = 1 (the layer rounds
 * sum_p z[p] to bf16 before the combine).  Only the live rows of each
 * expert segment are defined in the intermediates. */
gk_status gk_fp8_moe_bf16(const void* x, int64_t T, int64_t H, int64_t ldx, const float* logits, int64_t E,
                          int64_t ld_logits, int top_k, const void* w_gu, const float* s_gu, int64_t I,
                          const void* w_dn, const float* s_dn, void* y, int64_t ldy, uint32_t flags,
                          void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* GK_FP8_H */
