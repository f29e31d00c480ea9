// gfx950 block-FP8 W8A8 GEMM kernels.
//
// y[m, n] = bf16( sum_g  P[m, n, g] * sa[m, g] * sw[n / 128, g]  + bias[n] )
// P[m, n, g] = sum_{i < 128} qa[m, 128 g + i] * w[n, 128 g + i]
//
// This is the arithmetic of python/gaudi_kernels/block_fp8_oracle.py:38-46
// (per-group partials, then the original block scales applied per 128-K
// block) and of the Gaudi2 decode reduce (csrc/tpc/block_fp8_framework/
// reduce_bias.c:13-61: fp32 partial times ws*as accumulated over g, + bias,
// bf16 RNE).  On gfx950 one v_mfma_f32_16x16x128_f8f6f4 computes exactly one
// 128-K group of a 16x16 tile, so each MFMA result is promoted into the fp32
// accumulator with one FMA per element using the group's scale product.
//
// Operand roles: the MFMA "A" operand is a 16-row slab of weights (rows n),
// "B" is a 16-column slab of quantized activations (columns m).  The 16x16
// result lands as C[n = 4*(lane/16) + r][m = lane%16], so one lane's four
// accumulators share one token m and one 128-row weight block: the promotion
// factor sa[m,g]*sw[nb,g] is a single scalar per lane.  Both operands put the
// same 32 K-bytes in a lane (K offset 32*(lane/16)); because the hardware
// pairs A and B bytes by the same (lane, byte) position, the result does not
// depend on which K indices those bytes are.

#include "gk_fp8_internal.h"

namespace gk {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

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

__device__ inline v4f mfma_f8(v8i a, v8i b) {
  const v4f zero = {0.0f, 0.0f, 0.0f, 0.0f};
  // cbsz = blgp = 0 selects E4M3 for both operands; zero scale operands select
  // the unscaled v_mfma_f32_16x16x128_f8f6f4.
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, zero, 0, 0, 0, 0, 0, 0);
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
  const uint16_t h0 = bf16_rne(acc[0] + b[0]), h1 = bf16_rne(acc[1] + b[1]);
  const uint16_t h2 = bf16_rne(acc[2] + b[2]), h3 = bf16_rne(acc[3] + b[3]);
  if (n + 3 < N && ((reinterpret_cast<uintptr_t>(row) & 7) == 0)) {
    *reinterpret_cast<uint2*>(row) = make_uint2(h0 | (static_cast<uint32_t>(h1) << 16),
                                                h2 | (static_cast<uint32_t>(h3) << 16));
  } else {
    if (n < N) row[0] = h0;
    if (n + 1 < N) row[1] = h1;
    if (n + 2 < N) row[2] = h2;
    if (n + 3 < N) row[3] = h3;
  }
}

// ---------------------------------------------------------------------------
// Decode variant (M <= 16): HBM-bound weight streaming.
// One workgroup owns 16 weight rows; its NW waves split the G groups into
// contiguous ranges and each streams its 16 x (range*128) weight slab with
// 16-byte loads, U groups in flight per wave.  qa/sa (16 padded rows) are
// L2-resident.  Wave partials are summed in LDS in fixed wave order.
template <int NW, int U, bool HALF_W>
__global__ __launch_bounds__(NW * 64) void gemm_decode_kernel(const uint8_t* __restrict__ qa,
                                                              const float* __restrict__ sa,
                                                              const uint8_t* __restrict__ w,
                                                              const float* __restrict__ sw,
                                                              const float* __restrict__ bias,
                                                              uint16_t* __restrict__ y, int64_t ldy, int M,
                                                              int N, int K, int G) {
  __shared__ v4f red[NW][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, quad = lane >> 4;
  const int n0 = blockIdx.x * 16;
  const int nrow = min(n0 + col, N - 1);  // rows past N are computed on row N-1 and discarded
  const int64_t ldq = static_cast<int64_t>(G) * 128;
  const uint8_t* wp = w + static_cast<int64_t>(nrow) * K + quad * 32;
  const uint8_t* qp = qa + col * ldq + quad * 32;
  const float* sap = sa + col * G;
  const float* swp = sw + static_cast<int64_t>(n0 >> 7) * G;
  const int gbeg = (G * wave) / NW, gend = (G * (wave + 1)) / NW;

  v4f acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int g0 = gbeg; g0 < gend; g0 += U) {
    uint4 wa[U][2], qb[U][2];
    float f[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = min(g0 + u, gend - 1);
      const uint8_t* w8 = wp + static_cast<int64_t>(g) * 128;
      const uint4* q4 = reinterpret_cast<const uint4*>(qp + static_cast<int64_t>(g) * 128);
      wa[u][0] = load_stream16(w8);
      wa[u][1] = load_stream16(w8 + 16);
      qb[u][0] = q4[0];
      qb[u][1] = q4[1];
      // native_half doubles the weight scales (block_fp8_oracle.py:35); x2 is exact.
      f[u] = (g0 + u < gend) ? sap[g] * (HALF_W ? 2.0f * swp[g] : swp[g]) : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const v4f t = mfma_f8(weight_frag<HALF_W>(wa[u][0], wa[u][1]), pack8(qb[u][0], qb[u][1]));
      acc[0] = fmaf(t[0], f[u], acc[0]);
      acc[1] = fmaf(t[1], f[u], acc[1]);
      acc[2] = fmaf(t[2], f[u], acc[2]);
      acc[3] = fmaf(t[3], f[u], acc[3]);
    }
  }
  if (NW > 1) {
    red[wave][lane] = acc;
    __syncthreads();
    if (wave != 0) return;
    acc = red[0][lane];
#pragma unroll
    for (int v = 1; v < NW; ++v) acc += red[v][lane];
  }
  store_tile(y, ldy, bias, M, N, col, n0 + 4 * quad, acc);
}

// ---------------------------------------------------------------------------
// Prefill variant: LDS-tiled, double-buffered.  Workgroup tile 128 weight rows
// x 128 tokens, K step 128 (one scale group), 4 waves in a 2x2 grid, each
// wave 64 x 64 = 4 x 4 MFMA tiles.  Tiles are stored in LDS as 128 rows x 128
// bytes with the 16-byte chunk index XOR-swizzled by (row & 7) so that the 16
// lanes reading one column chunk of 16 consecutive rows hit distinct banks.
constexpr int kPB = 128;  // tile edge (rows of W, rows of qa, K bytes)

__device__ inline int swz(int row, int chunk) { return row * kPB + ((chunk ^ (row & 7)) << 4); }

template <bool HALF_W>
__global__ __launch_bounds__(256) void gemm_prefill_kernel(const uint8_t* __restrict__ qa,
                                                           const float* __restrict__ sa,
                                                           const uint8_t* __restrict__ w,
                                                           const float* __restrict__ sw,
                                                           const float* __restrict__ bias,
                                                           uint16_t* __restrict__ y, int64_t ldy, int M, int N,
                                                           int K, int G) {
  __shared__ __attribute__((aligned(16))) uint8_t smem[2][2][kPB * kPB];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wn = wave & 1, wm = wave >> 1;
  const int n0 = blockIdx.x * kPB, m0 = blockIdx.y * kPB;
  const int64_t ldq = static_cast<int64_t>(G) * 128;

  // Global -> LDS staging: chunk c = tid + 256 i, row = c / 8, 16-byte chunk = c % 8.
  const int lrow = tid >> 3, lkc = tid & 7;
  const uint8_t* wsrc[4];
  const uint8_t* qsrc[4];
  int soff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int r = lrow + 32 * i;
    wsrc[i] = w + static_cast<int64_t>(min(n0 + r, N - 1)) * K + lkc * 16;
    qsrc[i] = qa + static_cast<int64_t>(m0 + r) * ldq + lkc * 16;
    soff[i] = swz(r, lkc);
  }
  // Fragment reads.
  const int fr = lane & 15, fk = (lane >> 4) * 2;
  int aoff[4][2], boff[4][2];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int ra = wn * 64 + i * 16 + fr, rb = wm * 64 + i * 16 + fr;
    aoff[i][0] = swz(ra, fk); aoff[i][1] = swz(ra, fk + 1);
    boff[i][0] = swz(rb, fk); boff[i][1] = swz(rb, fk + 1);
  }
  const float* sap[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sap[j] = sa + static_cast<int64_t>(m0 + wm * 64 + j * 16 + fr) * G;
  const float* swp = sw + static_cast<int64_t>(n0 >> 7) * G;

  v4f acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};

  uint4 wreg[4], qreg[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    wreg[i] = *reinterpret_cast<const uint4*>(wsrc[i]);
    qreg[i] = *reinterpret_cast<const uint4*>(qsrc[i]);
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    *reinterpret_cast<uint4*>(&smem[0][0][soff[i]]) = wreg[i];
    *reinterpret_cast<uint4*>(&smem[0][1][soff[i]]) = qreg[i];
  }
  __syncthreads();

  for (int g = 0; g < G; ++g) {
    const int buf = g & 1;
    if (g + 1 < G) {
      const int64_t koff = static_cast<int64_t>(g + 1) * 128;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        wreg[i] = *reinterpret_cast<const uint4*>(wsrc[i] + koff);
        qreg[i] = *reinterpret_cast<const uint4*>(qsrc[i] + koff);
      }
    }
    const float swg = HALF_W ? 2.0f * swp[g] : swp[g];  // native_half: scales x2
    float f[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) f[j] = sap[j][g] * swg;
    v8i bfr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      bfr[j] = pack8(*reinterpret_cast<const uint4*>(&smem[buf][1][boff[j][0]]),
                     *reinterpret_cast<const uint4*>(&smem[buf][1][boff[j][1]]));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const v8i afr = weight_frag<HALF_W>(*reinterpret_cast<const uint4*>(&smem[buf][0][aoff[i][0]]),
                                          *reinterpret_cast<const uint4*>(&smem[buf][0][aoff[i][1]]));
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const v4f t = mfma_f8(afr, bfr[j]);
        acc[i][j][0] = fmaf(t[0], f[j], acc[i][j][0]);
        acc[i][j][1] = fmaf(t[1], f[j], acc[i][j][1]);
        acc[i][j][2] = fmaf(t[2], f[j], acc[i][j][2]);
        acc[i][j][3] = fmaf(t[3], f[j], acc[i][j][3]);
      }
    }
    if (g + 1 < G) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        *reinterpret_cast<uint4*>(&smem[buf ^ 1][0][soff[i]]) = wreg[i];
        *reinterpret_cast<uint4*>(&smem[buf ^ 1][1][soff[i]]) = qreg[i];
      }
    }
    __syncthreads();
  }

  const int quad = lane >> 4;
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
      store_tile(y, ldy, bias, M, N, m0 + wm * 64 + j * 16 + fr, n0 + wn * 64 + i * 16 + 4 * quad, acc[i][j]);
}

// ---------------------------------------------------------------------------
// Generic variant for shapes the tiled kernels do not take (K % 128 != 0 or
// misaligned weights): one thread per output, byte loads with K bounds.
__global__ __launch_bounds__(256) void gemm_generic_kernel(const uint8_t* __restrict__ qa,
                                                           const float* __restrict__ sa,
                                                           const uint8_t* __restrict__ w,
                                                           const float* __restrict__ sw,
                                                           const float* __restrict__ bias,
                                                           uint16_t* __restrict__ y, int64_t ldy, int M, int N,
                                                           int K, int G, int half_w) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(M) * N) return;
  const int m = static_cast<int>(idx / N), n = static_cast<int>(idx % N);
  const int64_t ldq = static_cast<int64_t>(G) * 128;
  float acc = 0.0f;
  for (int g = 0; g < G; ++g) {
    float part = 0.0f;
    const int kend = min(128, K - g * 128);
    for (int i = 0; i < kend; ++i) {
      const int64_t k = static_cast<int64_t>(g) * 128 + i;
      uint32_t wc = w[static_cast<int64_t>(n) * K + k];
      if (half_w) wc = codec_half4(wc) & 0xffu;
      part = fmaf(e4m3_value(qa[m * ldq + k]), e4m3_value(wc), part);
    }
    const float swg = sw[static_cast<int64_t>(n >> 7) * G + g];
    acc = fmaf(part, sa[static_cast<int64_t>(m) * G + g] * (half_w ? 2.0f * swg : swg), acc);
  }
  if (bias) acc += bias[n];
  y[static_cast<int64_t>(m) * ldy + n] = bf16_rne(acc);
}

// ---------------------------------------------------------------------------
hipError_t launch_gemm_decode(const GemmArgs& a, hipStream_t stream) {
  constexpr int NW = 4, U = 8;
  const dim3 grid((a.N + 15) / 16);
  if (a.half_w)
    gemm_decode_kernel<NW, U, true><<<grid, NW * 64, 0, stream>>>(a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy,
                                                                   a.M, a.N, a.K, a.G);
  else
    gemm_decode_kernel<NW, U, false><<<grid, NW * 64, 0, stream>>>(a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy,
                                                                    a.M, a.N, a.K, a.G);
  return hipGetLastError();
}

hipError_t launch_gemm_prefill(const GemmArgs& a, hipStream_t stream) {
  const dim3 grid((a.N + kPB - 1) / kPB, (a.M + kPB - 1) / kPB);
  if (a.half_w)
    gemm_prefill_kernel<true><<<grid, 256, 0, stream>>>(a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy, a.M, a.N,
                                                        a.K, a.G);
  else
    gemm_prefill_kernel<false><<<grid, 256, 0, stream>>>(a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy, a.M, a.N,
                                                         a.K, a.G);
  return hipGetLastError();
}

hipError_t launch_gemm_generic(const GemmArgs& a, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(a.M) * a.N;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  gemm_generic_kernel<<<grid, 256, 0, stream>>>(a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy, a.M, a.N, a.K, a.G,
                                                a.half_w ? 1 : 0);
  return hipGetLastError();
}

}  // namespace gk
