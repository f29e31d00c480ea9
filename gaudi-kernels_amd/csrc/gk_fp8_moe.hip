// Block-FP8 MoE layer kernels for gfx950: routing, row gather + 1x128
// quantization, weighted combine.  The expert GEMMs are the grouped 256 x 256
// kernel (gk_fp8_prefill.hip); the gate_up GEMM's epilogue applies the
// SiLU-and-mul and the 1x128 quantizer of the down GEMM's activations.
//
// The reference has no MoE code for this path; the layer follows BASELINE.json's
// config 5 and is build-defined (the CPU restatement is oracle/moe.py):
//   * route: top-k (k <= 2) experts by router logit, ties to the lower index;
//     combine weights = softmax over the k selected logits (fp32);
//   * rows: one row per (token, slot), ordered by expert then token; each
//     expert's segment starts at a multiple of kMoeRowAlign (256) so a GEMM
//     row tile never spans two experts; padding rows carry no token and are
//     never written (each GEMM output row depends on its own input row only,
//     and no later stage reads a padding row's outputs);
//   * act: h = bf16(silu(g) * u) in fp32 -- the reference's fused
//     SiLU-and-mul (csrc/tpc/generic_dense/silu_and_mul_bf16.c:4-15), whose
//     only rounding is the final product -- followed here by the same 1x128
//     quantizer as the activations (block_fp8_oracle.py:25-28);
//   * combine: y = bf16(w_0 z_0 + w_1 z_1) with each product and the sum
//     rounded to fp32 (no fused multiply-add), slot order.

#include "gk_fp8_internal.h"

namespace gk {

namespace {

// ---- routing: one workgroup of 1024 threads ---------------------------------------
// Phase 1: per token, the top-k experts (strictly greater wins; ties keep the
// lower index) and softmax weights; an LDS histogram of expert counts.
// Phase 2: padded segment starts.  Phase 3, per chunk of 1024 tokens: each
// wave ballots every expert over its 64 tokens (a token's rank among the
// wave's tokens of that expert), the per-wave counts are prefix-summed over
// the waves per expert, and a slot's row is its expert's start + the tokens of
// that expert in earlier chunks and waves + its rank in the wave: rows are in
// token order inside each expert -- stable, deterministic.
constexpr int kRouteThreads = 1024;
constexpr int kRouteWaves = kRouteThreads / 64;

__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(const float* __restrict__ logits, int T, int E,
                                                                  int64_t ld, int top_k, int rows_max,
                                                                  MoeRouting r) {
  __shared__ int counts[kMoeMaxExperts];
  __shared__ int offs[kMoeMaxExperts + 1];
  __shared__ int carry[kMoeMaxExperts];
  __shared__ int wcnt[kRouteWaves][kMoeMaxExperts];  // per chunk: wave counts, then their exclusive prefix
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int e = tid; e < E; e += kRouteThreads) counts[e] = 0;
  for (int i = tid; i < rows_max; i += kRouteThreads) r.row_token[i] = -1;
  __syncthreads();

  // ids of the first kKeep tokens of each thread stay in registers for phase 3
  // (no global write-then-read round trip); later tokens are read back from r.ids
  constexpr int kKeep = 4;
  int keep0[kKeep], keep1[kKeep];
#pragma unroll
  for (int i = 0; i < kKeep; ++i) keep0[i] = keep1[i] = -1;
  for (int t = tid, it = 0; t < T; t += kRouteThreads, ++it) {
    const float* row = logits + static_cast<int64_t>(t) * ld;
    // One pass in expert order, eight logits loaded at a time.  best0: the
    // first expert holding the maximum (strictly greater wins); best1: the
    // same over the other experts -- a new maximum hands its predecessor to
    // best1, which is then the first holder of the best value among the rest.
    int best0 = 0, best1 = -1;
    float v0 = 0.0f, v1 = 0.0f;
    for (int c = 0; c < E; c += 8) {
      float lv[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) lv[u] = c + u < E ? row[c + u] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int e = c + u;
        if (e >= E) break;
        const float v = lv[u];
        if (e == 0) {
          v0 = v;
        } else if (v > v0) {
          best1 = best0; v1 = v0;
          best0 = e; v0 = v;
        } else if (best1 < 0 || v > v1) {
          best1 = e; v1 = v;
        }
      }
    }
    r.ids[t * top_k] = best0;
    atomicAdd(&counts[best0], 1);
    int kept1 = -1;
    if (top_k == 2) {
      r.ids[t * 2 + 1] = best1;
      atomicAdd(&counts[best1], 1);
      kept1 = best1;
      // softmax over (v0, v1) with v0 >= v1: exp(0) = 1 and exp(v1 - v0), fp32
      const float e1 = expf(v1 - v0);
      const float s = 1.0f + e1;
      r.wts[t * 2] = 1.0f / s;
      r.wts[t * 2 + 1] = e1 / s;
    } else {
      r.wts[t] = 1.0f;
    }
#pragma unroll
    for (int i = 0; i < kKeep; ++i)
      if (it == i) {
        keep0[i] = best0;
        keep1[i] = kept1;
      }
  }
  __syncthreads();
  if (tid == 0) {
    int acc = 0;
    for (int e = 0; e < E; ++e) {
      offs[e] = acc;
      carry[e] = 0;
      acc += (counts[e] + kMoeRowAlign - 1) / kMoeRowAlign * kMoeRowAlign;
    }
    offs[E] = acc;
  }
  __syncthreads();
  for (int e = tid; e <= E; e += kRouteThreads) r.off[e] = offs[e];
  if (r.cnt)
    for (int e = tid; e < E; e += kRouteThreads) r.cnt[e] = counts[e];

  for (int base = 0, it = 0; base < T; base += kRouteThreads, ++it) {
    const int t = base + tid;
    const bool live = t < T;
    int e0 = -1, e1 = -1;
    if (it < kKeep) {
#pragma unroll
      for (int i = 0; i < kKeep; ++i)
        if (it == i) {
          e0 = keep0[i];
          e1 = keep1[i];
        }
    } else {
      e0 = live ? r.ids[t * top_k] : -1;
      e1 = (live && top_k == 2) ? r.ids[t * 2 + 1] : -1;
    }
    const unsigned long long below_lane = (1ull << lane) - 1ull;
    int rank0 = 0, rank1 = 0;
    for (int e = 0; e < E; ++e) {  // a token picks an expert at most once
      const unsigned long long mask = __ballot(e0 == e || e1 == e);
      if (lane == 0) wcnt[wave][e] = __popcll(mask);
      if (e0 == e) rank0 = __popcll(mask & below_lane);
      if (e1 == e) rank1 = __popcll(mask & below_lane);
    }
    __syncthreads();
    for (int e = tid; e < E; e += kRouteThreads) {  // exclusive prefix over the waves, from the carry
      int acc = carry[e];
      for (int v = 0; v < kRouteWaves; ++v) {
        const int c = wcnt[v][e];
        wcnt[v][e] = acc;
        acc += c;
      }
      carry[e] = acc;
    }
    __syncthreads();
    if (e0 >= 0) {
      const int row = offs[e0] + wcnt[wave][e0] + rank0;
      r.row_token[row] = t;
      r.row_of[t * top_k] = row;
    }
    if (e1 >= 0) {
      const int row = offs[e1] + wcnt[wave][e1] + rank1;
      r.row_token[row] = t;
      r.row_of[t * 2 + 1] = row;
    }
    __syncthreads();  // the next chunk rewrites wcnt
  }
}

// ---- gather + quantize rows: token t's groups, quantized once, go to the rows
// row_of[t * top_k + s] of its k slots (padding rows are not written: their
// GEMM outputs are never read).
template <bool HALF>
__global__ __launch_bounds__(256) void act_quant_rows_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                             const int32_t* __restrict__ row_of, int T, int top_k,
                                                             int rows, uint8_t* __restrict__ q,
                                                             float* __restrict__ sa) {
  // grid: x = 16 tokens per block, y = group (no division for the indices)
  const int t = static_cast<int>(blockIdx.x) * (blockDim.x >> 4) + (threadIdx.x >> 4);
  const int g = static_cast<int>(blockIdx.y), sub = threadIdx.x & 15;
  if (t >= T) return;  // a whole 16-lane group leaves together
  const uint4 raw = *reinterpret_cast<const uint4*>(x + t * ldx + g * 128 + sub * 8);
  float s;
  const uint2 codes = quant_group8(raw, true, HALF, &s);
  for (int k = 0; k < top_k; ++k) {
    const int64_t slot = static_cast<int64_t>(g) * rows + row_of[t * top_k + k];
    *reinterpret_cast<uint2*>(q + slot * 128 + sub * 8) = codes;
    if (sub == 0) sa[slot] = s;
  }
}

// ---- combine: y[t] = bf16(w_0 z_0 + w_1 z_1), 8 columns per thread -------------------
// z_k = bf16(sum_p zp[p][row_of[t, k]]): the down GEMM's output rounded to bf16
// once, from its kparts fp32 partial planes.
__global__ __launch_bounds__(256) void moe_combine_kernel(const float* __restrict__ z, int kparts, int64_t plane,
                                                          int H, const int32_t* __restrict__ row_of,
                                                          const float* __restrict__ wts, int T, int top_k,
                                                          uint16_t* __restrict__ y, int64_t ldy) {
  const int per_row = H / 8;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= static_cast<int64_t>(T) * per_row) return;
  const int t = static_cast<int>(i / per_row);
  const int c = static_cast<int>(i - static_cast<int64_t>(t) * per_row) * 8;
  float acc[8];
  for (int k = 0; k < top_k; ++k) {
    const float wk = wts[t * top_k + k];
    const float* zr = z + static_cast<int64_t>(row_of[t * top_k + k]) * H + c;
    float zv[8];
    const float4 a0 = *reinterpret_cast<const float4*>(zr), a1 = *reinterpret_cast<const float4*>(zr + 4);
    zv[0] = a0.x; zv[1] = a0.y; zv[2] = a0.z; zv[3] = a0.w; zv[4] = a1.x; zv[5] = a1.y; zv[6] = a1.z; zv[7] = a1.w;
    for (int p = 1; p < kparts; ++p) {
      const float4 b0 = *reinterpret_cast<const float4*>(zr + p * plane);
      const float4 b1 = *reinterpret_cast<const float4*>(zr + p * plane + 4);
      zv[0] = add_rn(zv[0], b0.x); zv[1] = add_rn(zv[1], b0.y); zv[2] = add_rn(zv[2], b0.z);
      zv[3] = add_rn(zv[3], b0.w); zv[4] = add_rn(zv[4], b1.x); zv[5] = add_rn(zv[5], b1.y);
      zv[6] = add_rn(zv[6], b1.z); zv[7] = add_rn(zv[7], b1.w);
    }
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const uint32_t zb = bf16x2_rne(zv[j], zv[j + 1]);  // z rounded to bf16, two columns at a time
      const float p0 = mul_rn(wk, bits_f32(zb << 16)), p1 = mul_rn(wk, bits_f32(zb & 0xffff0000u));
      acc[j] = k ? add_rn(acc[j], p0) : p0;
      acc[j + 1] = k ? add_rn(acc[j + 1], p1) : p1;
    }
  }
  uint32_t o[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) o[j] = bf16x2_rne(acc[2 * j], acc[2 * j + 1]);
  *reinterpret_cast<uint4*>(y + static_cast<int64_t>(t) * ldy + c) = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace

hipError_t launch_moe_route(const float* logits, int T, int E, int64_t ld_logits, int top_k, int rows_max,
                            const MoeRouting& r, hipStream_t stream) {
  if (E < 1 || E > kMoeMaxExperts || top_k < 1 || top_k > 2 || top_k > E) return hipErrorInvalidValue;
  moe_route_kernel<<<1, kRouteThreads, 0, stream>>>(logits, T, E, ld_logits, top_k, rows_max, r);
  return hipGetLastError();
}

hipError_t launch_act_quant_rows(const uint16_t* x, int64_t ldx, int K, const int32_t* row_of, int T, int top_k,
                                 int rows, uint8_t* q, float* sa, bool half, hipStream_t stream) {
  const dim3 grid((T + 15) / 16, K / 128);
  if (half)
    act_quant_rows_kernel<true><<<grid, 256, 0, stream>>>(x, ldx, row_of, T, top_k, rows, q, sa);
  else
    act_quant_rows_kernel<false><<<grid, 256, 0, stream>>>(x, ldx, row_of, T, top_k, rows, q, sa);
  return hipGetLastError();
}

hipError_t launch_moe_combine(const float* z, int kparts, int64_t plane, int H, const int32_t* row_of,
                              const float* wts, int T, int top_k, uint16_t* y, int64_t ldy, hipStream_t stream) {
  const int64_t n = static_cast<int64_t>(T) * (H / 8);
  moe_combine_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, stream>>>(z, kparts, plane, H, row_of, wts,
                                                                                   T, top_k, y, ldy);
  return hipGetLastError();
}

}  // namespace gk
