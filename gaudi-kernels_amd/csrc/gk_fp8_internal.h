// Internal declarations shared by the kernel translation units and the C-ABI
// layer.  Not part of the public interface (that is include/gk_fp8.h).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gk_fp8_math.h"

namespace gk {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));

// Row padding of the quantized-activation workspace.
constexpr int kDecodeMaxRows = 16;   // decode variant: M <= 16, padded to one MFMA column tile
constexpr int kPrefillRowTile = 256; // prefill variant: M padded to the token tile

hipError_t launch_codec(bool forward, const uint8_t* src, uint8_t* dst, int64_t n, const float* scales,
                        float* scales_out, int64_t n_scales, uint32_t* flags, unsigned long long* rounded,
                        hipStream_t stream);

hipError_t launch_act_quant(const uint16_t* x, int64_t ldx, int M, int K, int Mpad, uint8_t* q, float* sa,
                            bool half, hipStream_t stream);

// Quantized activations qa [Mpad, G*128] / sa [Mpad, G] (from launch_act_quant)
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
  int Mpad;
  bool half_w;        // apply the half-range codec to weight codes in-kernel (native_half)
};

hipError_t launch_gemm_decode(const GemmArgs& a, hipStream_t stream);
hipError_t launch_gemm_prefill(const GemmArgs& a, hipStream_t stream);
hipError_t launch_gemm_generic(const GemmArgs& a, hipStream_t stream);

// Grouped (MoE) variant: rows of qa are sorted by expert; expert e owns rows
// [offsets[e], offsets[e+1]).  Weights/scales are stacked per expert.
struct GroupedArgs {
  const uint8_t* qa;
  const float* sa;
  const uint8_t* w;      // [E, N, K]
  const float* sw;       // [E, NB, G]
  const int32_t* offsets;  // [E + 1] device
  uint16_t* y;           // [rows, N]
  int rows, E, N, K, G;
  int rows_pad;
  int max_rows;          // host-known upper bound of rows of any expert
};

hipError_t launch_gemm_grouped(const GroupedArgs& a, hipStream_t stream);

}  // namespace gk
