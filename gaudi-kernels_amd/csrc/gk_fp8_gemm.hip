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
// same 32 K-bytes of the group in a lane; because the hardware pairs A and B
// bytes by the same (lane, byte) position, the result does not depend on
// which K indices those bytes are.
//
// Quantized activations are group-major, qa [G][Mpad][128] and sa [G][Mpad]
// (the reference quant op's {128, R, G} layout, generic_fp8_glue.hpp:84-109):
// the 16 x 128 codes of one group and 16 tokens are one contiguous 2 KB block.

#include "gk_fp8_tile.h"

namespace gk {

// ---------------------------------------------------------------------------
// Decode variant (M <= 16): HBM-bound weight streaming.
//
// Workgroup = NW waves over R 16-row weight tiles (16R rows).  The waves split
// the G groups into contiguous ranges; the NW partials are summed in LDS in
// wave order (deterministic) and rounded to bf16 with the bias.
//
// Weights are read fully coalesced: one load instruction covers 8 rows x 128
// bytes of a group, lane l reading row 2 (l/16) + (l/8)%2, 16-byte chunk l%8,
// so sixteen lanes read 256 contiguous bytes (the MFMA operand layout instead
// puts 16 different rows in 16 consecutive lanes, which the memory pipeline
// serves about 1.5-2x slower).  The tile goes through a wave-private 2 KB LDS
// buffer -- chunk c of row r at slot c ^ lds_key(r), bank-conflict free for
// both the write and the fragment read -- into the MFMA layout.
//
// K permutation (A and B alike): lane (col, quad) holds bytes [32 quad,
// 32 quad + 32) of the group.  Activations come in one of two layouts:
//   * standard  qa [G][16][128]: lane reads token col at +32 quad, +32 quad+16;
//   * packed    the decode fragment layout (launch_act_quant with packed):
//     group g is 2 KB, piece (h, l) at g*2048 + h*1024 + 16 l holds bytes
//     [32 (l/16) + 16 h, +16) of token l%16 -- the two loads of a wave read
//     1 KB each, contiguous.
// Tokens >= M read token M-1 (their results are never stored), so M < 16
// touches fewer activation lines.  Every load is unconditional (indices are
// clamped) and all loads of a step are issued before the first use: the
// compiler then waits on them one by one instead of draining the queue.
//
// WPACK: weights in the fragment-packed layout (launch_pack_weight): lane l
// of a tile's group reads pieces (0, l) and (1, l), two contiguous 1 KB loads
// per wave that land in the MFMA layout directly -- no LDS transpose.  The
// operands, and so the results, are bit-identical to the row-major path.
//
// XQ: the activations come as bf16 x [M][ldq] and are quantized inside the
// kernel by the standalone quantizer's own code (quant_group8): per group,
// load j (of 4) gives 16 lanes to each of tokens 4j..4j+3, 8 elements a lane
// (full 128-byte lines), and the codes go through a wave-private LDS buffer
// into the fragment layout.  The x loads of a step are issued before its
// weight loads, so the quantizer's arithmetic overlaps the weight fetch
// instead of costing a separate launch and memory round trip.  Every
// workgroup quantizes the activations of its K range again, so this pays
// only while that work is small (few tokens, few workgroups; the caller
// decides).  Codes and scales are the standalone quantizer's, so the results
// equal quantize-then-GEMM bit for bit.
//
// CH (per-token / per-channel scaling): activations row-major [M][ldq], one
// scale per token sa[m] and per output channel sw[n]; the MFMAs accumulate
// over all of K (no per-group promotion) and the epilogue applies
// bf16(fma(p * sa[m], sw[n], bias[n])) (channel_finish.c:9-15).
//
// CH and XQ: the per-token quantizer fused in (sa unused).  A token's scale
// needs the maximum |x| over its whole row, so each wave first takes the
// maximum over its own groups (the XQ loader's lanes), the waves combine them
// in LDS, and every lane forms s and 1/s of its four loader tokens and 2 s of
// its output token; the main loop then encodes with the token quantizer's
// token_codes8.  The maximum does not depend on the order (fmaxf drops NaN,
// |x| >= +0), so codes, scales and results equal token quant + this kernel's
// CH form bit for bit.
template <int NW, int R, int U, bool HALF, bool QPACK, bool CH = false, bool WPACK = false, bool XQ = false,
          int MT = 1>
__global__ __launch_bounds__(NW * 64) void gemm_decode_kernel(const uint8_t* __restrict__ qa,
                                                              const float* __restrict__ sa,
                                                              const uint8_t* __restrict__ w,
                                                              const float* __restrict__ sw,
                                                              const float* __restrict__ bias,
                                                              uint16_t* __restrict__ y, int64_t ldy, int M,
                                                              int N, int K, int G, int64_t ldq, int gs,
                                                              float* __restrict__ yp, int64_t ldyp, int accum) {
  static_assert(16 * R <= 128 && NW >= R, "a workgroup's rows lie in one 128-row scale block");
  static_assert(MT == 1 || (!XQ && !CH), "several token tiles take pre-quantized block-scaled activations");
  __shared__ __attribute__((aligned(16))) uint8_t tile[WPACK ? 1 : NW][2048];
  __shared__ __attribute__((aligned(16))) uint8_t xqbuf[XQ ? NW : 1][XQ ? U : 1][2048 + 64];  // codes + 16 scales
  __shared__ v4f red[NW][R][MT][64];
  __shared__ float tmax[CH && XQ ? NW : 1][16];
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
  const int col = lane & 15, quad = lane >> 4;
  const int n0 = blockIdx.x * 16 * R;
  const int lrow = 2 * (lane >> 4) + ((lane >> 3) & 1), lch = lane & 7;
  const uint8_t* wp[R];
  int64_t d8[R];  // row-major: byte distance from row lrow to row lrow + 8 (rows past N re-read row N-1)
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (WPACK) {  // tiles past the last re-read the last tile (never stored)
      const int t = min((n0 >> 4) + r, ((N + 15) >> 4) - 1);
      wp[r] = w + static_cast<int64_t>(t) * gs * 2048 + lane * 16;
      d8[r] = 1024;
    } else {
      const int a0 = min(n0 + 16 * r + lrow, N - 1), a1 = min(n0 + 16 * r + lrow + 8, N - 1);
      wp[r] = w + static_cast<int64_t>(a0) * K + lch * 16;
      d8[r] = static_cast<int64_t>(a1 - a0) * K;
    }
  }
  constexpr int kWG = WPACK ? 2048 : 128;  // weight bytes from one group to the next
  const uint32_t woff0 = lrow * 128 + ((lch ^ lds_key(lrow)) << 4);
  const uint32_t woff1 = (lrow + 8) * 128 + ((lch ^ lds_key(lrow + 8)) << 4);
  const uint32_t roff0 = col * 128 + (((2 * quad) ^ lds_key(col)) << 4);
  const uint32_t roff1 = col * 128 + (((2 * quad + 1) ^ lds_key(col)) << 4);
  // Token tile t holds tokens 16 t .. 16 t + 15; tokens >= M read token M-1.
  // Decode fragment layout: (group g, token tile tt) is the 2 KB block
  // g * MT + tt; standard layout: row tok of group g at (g * 16 MT + tok) * 128.
  const uint8_t* qpt[MT];
  const float* sapt[MT];
#pragma unroll
  for (int t = 0; t < MT; ++t) {
    const int tk = min(16 * t + col, M - 1);
    qpt[t] = CH      ? qa + tk * ldq + quad * 32
             : QPACK ? qa + (tk >> 4) * 2048 + (16 * quad + (tk & 15)) * 16
                     : qa + tk * 128 + quad * 32;
    sapt[t] = sa + tk;
  }
  // XQ loader: load j reads token 4j + lane/16 (tokens >= M re-read token
  // M-1), elements [8 (lane%16), +8) of the group; its 8 codes are bytes
  // e0 = 8 (lane%16) .. e0+7 of that token, which the fragment layout keeps
  // in piece (h, L) = ((e0/16) & 1, 16 (e0/32) + token) at byte e0 % 16.
  const uint8_t* xrow[4];
  uint32_t xwoff[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int t = 4 * j + (lane >> 4), e0 = 8 * (lane & 15);
    xrow[j] = qa + (static_cast<int64_t>(min(t, M - 1)) * ldq + e0) * 2;
    xwoff[j] = ((e0 >> 4) & 1) * 1024 + 16 * (16 * (e0 >> 5) + t) + (e0 & 15);
  }
  // Token rows 4j..4j+3 with 4j >= M are neither loaded nor quantized: their
  // fragment columns hold whatever the buffer held and are never stored.
  const int xjn = (min(M, 16) + 3) >> 2;
  constexpr int kQHi = QPACK ? 1024 : 16;
  constexpr int kQG = CH ? 128 : 2048 * MT;         // activation bytes from one group to the next
  const float* swp = sw + static_cast<int64_t>(n0 >> 7) * gs;
  const int gbeg = (G * wave) / NW, gend = (G * (wave + 1)) / NW;
  uint8_t* buf = tile[WPACK ? 0 : wave];

  // Fused per-token quantizer: s, 1/s of loader token 4 j + lane/16, 2 s of token col.
  float tsc[4] = {1.0f, 1.0f, 1.0f, 1.0f}, trc[4] = {1.0f, 1.0f, 1.0f, 1.0f}, tcol2 = 0.0f;
  if (CH && XQ) {
    float mj[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int g = gbeg; g < gend; ++g) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (j < xjn) mj[j] = abs_max8(mj[j], *reinterpret_cast<const uint4*>(xrow[j] + static_cast<int64_t>(g) * 256));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float m16 = __uint_as_float(row_max16_bits(mj[j]));  // over the 16 lanes of the token
      if ((lane & 15) == 0) tmax[wave][4 * j + (lane >> 4)] = m16;
    }
    __syncthreads();
    auto token_max = [&](int t) {
      float m = tmax[0][t];
#pragma unroll
      for (int v = 1; v < NW; ++v) m = fmaxf(m, tmax[v][t]);
      return m == 0.0f ? 1.0f : m;  // an all-zero token (activation_token.c:16)
    };
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      tsc[j] = token_scale(token_max(4 * j + (lane >> 4)));
      trc[j] = 1.0f / tsc[j];
    }
    tcol2 = 2.0f * token_scale(token_max(col));
  }

  v4f acc[R][MT];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) acc[r][t] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  for (int g0 = gbeg; g0 < gend; g0 += U) {
    uint4 wa[U][R][2], qb[U][MT][2], xb[XQ ? U : 1][4];
    float sv[U][MT], wv[U];
    if (XQ) {  // activations first: they are needed before the weights
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j >= xjn) continue;  // wave-uniform: token rows 4j.. are all >= M
#pragma unroll
        for (int u = 0; u < U; ++u)
          xb[u][j] = *reinterpret_cast<const uint4*>(xrow[j] + static_cast<int64_t>(min(g0 + u, gend - 1)) * 256);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int g = min(g0 + u, gend - 1);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const uint8_t* p = wp[r] + static_cast<int64_t>(g) * kWG;
        wa[u][r][0] = load_stream16(p);
        wa[u][r][1] = load_stream16(p + d8[r]);
      }
      if (!XQ) {
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const uint8_t* q = qpt[t] + static_cast<int64_t>(g) * kQG;
          qb[u][t][0] = *reinterpret_cast<const uint4*>(q);
          qb[u][t][1] = *reinterpret_cast<const uint4*>(q + kQHi);
        }
      }
      if (!CH) {
        if (!XQ) {
#pragma unroll
          for (int t = 0; t < MT; ++t) sv[u][t] = sapt[t][g * 16 * MT];
        }
        wv[u] = swp[g];
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load of the step is in flight before the first use
    v8i bq[XQ ? U : 1];  // XQ implies MT == 1
    if (XQ) {
      uint8_t* xq = xqbuf[wave][0];
      // One straight-line block per token quad j holds the U independent
      // quantizer chains of the step, which the scheduler interleaves.  All
      // 16 lanes of a token-group store its (equal) scale.
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j >= xjn) continue;
#pragma unroll
        for (int u = 0; u < U; ++u) {
          if (CH) {
            *reinterpret_cast<uint2*>(xq + u * (2048 + 64) + xwoff[j]) = token_codes8(xb[u][j], tsc[j], trc[j]);
          } else {
            float sc;
            const uint2 c = quant_group8(xb[u][j], true, HALF, &sc);
            *reinterpret_cast<uint2*>(xq + u * (2048 + 64) + xwoff[j]) = c;
            *reinterpret_cast<float*>(xq + u * (2048 + 64) + 2048 + 4 * (4 * j + (lane >> 4))) = sc;
          }
        }
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {  // same wave: its LDS accesses complete in order
        const uint8_t* b = xq + u * (2048 + 64);
        bq[u] = pack8(*reinterpret_cast<const uint4*>(b + 16 * lane), *reinterpret_cast<const uint4*>(b + 1024 + 16 * lane));
        if (!CH) sv[u][0] = *reinterpret_cast<const float*>(b + 2048 + 4 * col);
      }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      // native_half doubles the weight scales (block_fp8_oracle.py:35); x2 is exact.
      const float ws = HALF ? 2.0f * wv[u] : wv[u];
      const bool live = g0 + u < gend;  // the clamped repeat of the last group adds nothing
#pragma unroll
      for (int r = 0; r < R; ++r) {
        uint4 lo = wa[u][r][0], hi = wa[u][r][1];
        if (!WPACK) {
          *reinterpret_cast<uint4*>(buf + woff0) = wa[u][r][0];
          *reinterpret_cast<uint4*>(buf + woff1) = wa[u][r][1];
          lo = *reinterpret_cast<const uint4*>(buf + roff0);
          hi = *reinterpret_cast<const uint4*>(buf + roff1);
        }
        const v8i a = weight_frag<HALF>(lo, hi);
#pragma unroll
        for (int t = 0; t < MT; ++t) {
          const v8i b = XQ ? bq[u] : pack8(qb[u][t][0], qb[u][t][1]);
          if (CH) {
            if (live) acc[r][t] = mfma_f8_acc(a, b, acc[r][t]);
          } else {
            const float f = live ? sv[u][t] * ws : 0.0f;
            const v4f p = mfma_f8(a, b);
            acc[r][t][0] = fmaf(p[0], f, acc[r][t][0]);
            acc[r][t][1] = fmaf(p[1], f, acc[r][t][1]);
            acc[r][t][2] = fmaf(p[2], f, acc[r][t][2]);
            acc[r][t][3] = fmaf(p[3], f, acc[r][t][3]);
          }
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int t = 0; t < MT; ++t) red[wave][r][t][lane] = acc[r][t];
  __syncthreads();
  // wave w sums (tile, token tile) pairs w, w + NW, ... of the NW partials in wave order
  for (int pr = wave; pr < R * MT; pr += NW) {
    const int r = pr / MT, t = pr % MT;
    v4f sum = red[0][r][t][lane];
#pragma unroll
    for (int v = 1; v < NW; ++v) sum += red[v][r][t][lane];
    const int m = 16 * t + col, n = n0 + 16 * r + 4 * quad;
    if (CH) {
      if (m >= M) continue;
      const float sam = XQ ? tcol2 : sa[m];
      uint16_t* row = y + static_cast<int64_t>(m) * ldy + n;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + i < N) row[i] = channel_out(sum[i], sam, sw[n + i], bias ? bias[n + i] : 0.0f);
    } else if (yp) {  // fp32 partial of this K range (+ the partial already there)
      if (m >= M) continue;
      float* row = yp + static_cast<int64_t>(m) * ldyp + n;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (n + i < N) row[i] = accum ? row[i] + sum[i] : sum[i];
    } else {
      store_tile(y, ldy, bias, M, N, m, n, sum);
    }
  }
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
                                                           int K, int G, int Mpad, int half_w) {
  const int64_t idx = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (idx >= static_cast<int64_t>(M) * N) return;
  const int m = static_cast<int>(idx / N), n = static_cast<int>(idx % N);
  float acc = 0.0f;
  for (int g = 0; g < G; ++g) {
    float part = 0.0f;
    const int kend = min(128, K - g * 128);
    for (int i = 0; i < kend; ++i) {
      const int64_t k = static_cast<int64_t>(g) * 128 + i;
      uint32_t wc = w[static_cast<int64_t>(n) * K + k];
      if (half_w) wc = codec_half4(wc) & 0xffu;
      part = fmaf(e4m3_value(qa[(static_cast<int64_t>(g) * Mpad + m) * 128 + i]), e4m3_value(wc), part);
    }
    const float swg = sw[static_cast<int64_t>(n >> 7) * G + g];
    acc = fmaf(part, sa[static_cast<int64_t>(g) * Mpad + m] * (half_w ? 2.0f * swg : swg), acc);
  }
  if (bias) acc += bias[n];
  y[static_cast<int64_t>(m) * ldy + n] = bf16_rne(acc);
}

// ---------------------------------------------------------------------------
template <int NW, int R, int U, int MT>
static hipError_t decode_launch(const GemmArgs& a, hipStream_t stream) {
  const dim3 grid(static_cast<unsigned>((a.N + 16 * R - 1) / (16 * R)));
#define GK_DECODE_LAUNCH(H, P, WP, X)                                                                          \
  gemm_decode_kernel<NW, R, U, H, P, false, WP, X, MT><<<grid, NW * 64, 0, stream>>>(                               \
      a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy, a.M, a.N, a.K, a.G, a.ldq, a.gstride(), a.yp, a.ldyp,         \
      a.accumulate ? 1 : 0)
#define GK_DECODE_LAUNCH_P(H, P, X) \
  if (a.wpack) GK_DECODE_LAUNCH(H, P, true, X); else GK_DECODE_LAUNCH(H, P, false, X)
#define GK_DECODE_LAUNCH_A(H)                                       \
  if (MT == 1 && a.xq) { GK_DECODE_LAUNCH_P(H, false, MT == 1); }      \
  else if (a.qpack) { GK_DECODE_LAUNCH_P(H, true, false); }               \
  else { GK_DECODE_LAUNCH_P(H, false, false); }
  if (a.half_w) {
    GK_DECODE_LAUNCH_A(true)
  } else {
    GK_DECODE_LAUNCH_A(false)
  }
#undef GK_DECODE_LAUNCH_A
#undef GK_DECODE_LAUNCH_P
#undef GK_DECODE_LAUNCH
  return hipGetLastError();
}

template <int NW, int R, int U, int MT>
static hipError_t decode_channel_launch(const GemmArgs& a, hipStream_t stream) {
  static_assert(MT == 1, "the per-channel decode takes one token tile");
  const dim3 grid(static_cast<unsigned>((a.N + 16 * R - 1) / (16 * R)));
  gemm_decode_kernel<NW, R, U, false, false, true><<<grid, NW * 64, 0, stream>>>(
      a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy, a.M, a.N, a.K, a.G, a.ldq, a.G, nullptr, 0, 0);
  return hipGetLastError();
}

// Per-token quantizer fused in: a.qa = bf16 x, a.ldq its row stride (elements).
template <int NW, int R, int U, int MT>
static hipError_t decode_token_channel_launch(const GemmArgs& a, hipStream_t stream) {
  static_assert(MT == 1, "the fused per-token decode takes one token tile");
  const dim3 grid(static_cast<unsigned>((a.N + 16 * R - 1) / (16 * R)));
  gemm_decode_kernel<NW, R, U, false, false, true, false, true><<<grid, NW * 64, 0, stream>>>(
      a.qa, nullptr, a.w, a.sw, a.bias, a.y, a.ldy, a.M, a.N, a.K, a.G, a.ldq, a.G, nullptr, 0, 0);
  return hipGetLastError();
}

hipError_t launch_gemm_decode(const GemmArgs& a, hipStream_t stream) {
  switch (decode_key(a.dec.nw, a.dec.r, a.dec.u, a.dec.mt)) {
#define GK_CASE(NW, R, U, MT) \
  case decode_key(NW, R, U, MT): return decode_launch<NW, R, U, MT>(a, stream);
    GK_DECODE_SHAPES(GK_CASE)
#undef GK_CASE
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm_prefill(const GemmArgs& a, hipStream_t stream) {
  // 256 x 256 tiles (gk_fp8_prefill.hip) at every M > 16: they skip the 32-row
  // blocks past M.  (A 128 x 128 kernel measured 1.2-3x slower at 16 < M <= 128
  // on MI355X.)  The plan sends shapes whose panels exceed the kernel's 32-bit
  // offsets to the generic variant.
  if (!prefill256_fits(a)) return hipErrorInvalidValue;
  return launch_gemm_prefill256(a, stream);
}

hipError_t launch_gemm_channel(const GemmArgs& a, hipStream_t stream) {
  if (a.M > kDecodeMaxRows) return launch_gemm_channel256(a, stream);
  const DecodeShape d = plan_decode_shape(a.N, a.G, false, 1);
  switch (decode_key(d.nw, d.r, d.u, d.mt)) {
#define GK_CASE(NW, R, U, MT) \
  case decode_key(NW, R, U, MT): return decode_channel_launch<NW, R, U, MT>(a, stream);
    GK_DECODE_SHAPES1(GK_CASE)
#undef GK_CASE
    default: return hipErrorInvalidValue;
  }
}

// Fused per-token quantizer + per-channel decode, M <= 16: the shape of the
// block path's fused quantizer (fused_quant_shape on row-major weights).
hipError_t launch_gemm_token_channel(const GemmArgs& a, hipStream_t stream) {
  if (a.M < 1 || a.M > 16) return hipErrorInvalidValue;
  const DecodeShape d = fused_quant_shape(fit_group_step(plan_decode_shape(a.N, a.G, false, 1), a.G), a.G);
  switch (decode_key(d.nw, d.r, d.u, d.mt)) {
#define GK_CASE(NW, R, U, MT) \
  case decode_key(NW, R, U, MT): return decode_token_channel_launch<NW, R, U, MT>(a, stream);
    GK_DECODE_SHAPES_T1(GK_CASE)
#undef GK_CASE
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_gemm_generic(const GemmArgs& a, hipStream_t stream) {
  const int64_t total = static_cast<int64_t>(a.M) * a.N;
  const dim3 grid(static_cast<unsigned>((total + 255) / 256));
  gemm_generic_kernel<<<grid, 256, 0, stream>>>(a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy, a.M, a.N, a.K, a.G,
                                                a.Mpad, a.half_w ? 1 : 0);
  return hipGetLastError();
}

}  // namespace gk
