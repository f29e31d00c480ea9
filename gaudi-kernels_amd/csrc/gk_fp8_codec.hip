// gfx950 kernels for the load-time E4M3 codec and the 1x128 activation quantizer.
//
// Codec (forward, OCP E4M3FN -> Gaudi2 half range) restates
// python/gaudi_kernels/fp8_codec.py:14-53 of the reference: a per-byte table
// (evaluated here as 4-byte SWAR arithmetic, gk_fp8_math.h), scales x2, a count
// of rounded codes, rejection of the OCP NaN code and of scales that are
// negative, nonfinite or overflow when doubled.  The inverse (half -> OCP) is
// build-defined: value x2 (exact), scales / 2.
//
// Both are HBM-streaming byte kernels: four 16-byte loads, then four 16-byte
// stores per lane per step, grid-stride, with the rounded count reduced in
// registers and one 64-bit atomic per workgroup.
//
// The activation quantizer restates block_fp8_oracle.py:25-28 (and :31-34 for
// native_half): per row and 128-column group, sa = fp32(max(amax, 1e-10)) *
// fp32(1/448), q = e4m3_rne(clamp(fp32(x / sa), +-448)) -- the exact codes of
// the IEEE quotient (quant_group8 in gk_fp8_internal.h).  Sixteen lanes own
// one group (8 bf16 each, one 16-byte load per lane).

#include "gk_fp8_internal.h"

namespace gk {

// Status flags written by the codec kernels (bit OR into flags[0]).
enum : uint32_t {
  kFlagNanCode = 1u,       // OCP NaN code in the forward input
  kFlagBadScale = 2u,      // negative or nonfinite scale
  kFlagScaleOverflow = 4u, // doubling overflows fp32
  kFlagInvalidHalf = 8u,   // half-range magnitude >= 0x77 in the inverse input
  kFlagInexactHalve = 16u, // halving a scale is inexact (fp32 subnormal result)
};

__device__ inline uint32_t wave_sum_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ inline uint32_t wave_or_u32(uint32_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v |= __shfl_xor(v, off, 64);
  return v;
}

// Folds the block's rounded count and flags into the status block: one
// atomic of each kind per workgroup (a per-wave atomic on one address
// serialized to ~2 ns each and dominated the kernel at 51 M codes).
__device__ inline void block_status(uint32_t count, uint32_t bad, uint32_t flag_bit, uint32_t* flags,
                                    unsigned long long* rounded) {
  __shared__ uint32_t wc[4], wb[4];
  count = wave_sum_u32(count);
  bad = wave_or_u32(bad);
  if ((threadIdx.x & 63) == 0) {
    wc[threadIdx.x >> 6] = count;
    wb[threadIdx.x >> 6] = bad;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint32_t c = wc[0] + wc[1] + wc[2] + wc[3];
    if (c) atomicAdd(rounded, static_cast<unsigned long long>(c));
    if (wb[0] | wb[1] | wb[2] | wb[3]) atomicOr(flags, flag_bit);
  }
}

template <bool FORWARD>
__global__ __launch_bounds__(256) void codec_bytes_kernel(const uint8_t* __restrict__ src,
                                                          uint8_t* __restrict__ dst, int64_t n,
                                                          uint32_t* __restrict__ flags,
                                                          unsigned long long* __restrict__ rounded) {
  const int64_t nvec = n >> 4;
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  const int64_t tid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  uint32_t bad = 0, count = 0;
  const uint4* s4 = reinterpret_cast<const uint4*>(src);
  uint4* d4 = reinterpret_cast<uint4*>(dst);
  auto convert = [&](const uint4& v) {
    uint4 o;
    if (FORWARD) {
      bad |= ocp_nan4(v.x) | ocp_nan4(v.y) | ocp_nan4(v.z) | ocp_nan4(v.w);
      count += codec_rounded4(v.x) + codec_rounded4(v.y) + codec_rounded4(v.z) + codec_rounded4(v.w);
      o.x = codec_half4(v.x); o.y = codec_half4(v.y); o.z = codec_half4(v.z); o.w = codec_half4(v.w);
    } else {
      bad |= half_invalid4(v.x) | half_invalid4(v.y) | half_invalid4(v.z) | half_invalid4(v.w);
      o.x = codec_double4(v.x); o.y = codec_double4(v.y); o.z = codec_double4(v.z); o.w = codec_double4(v.w);
    }
    return o;
  };
  // Four 16-byte loads in flight per lane before the first conversion (one
  // at a time left the kernel latency-bound: 51 M codes at 1.3 TB/s).
  int64_t i = tid;
  for (; i + 3 * stride < nvec; i += 4 * stride) {
    uint4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = s4[i + u * stride];
#pragma unroll
    for (int u = 0; u < 4; ++u) d4[i + u * stride] = convert(v[u]);
  }
  for (; i < nvec; i += stride) d4[i] = convert(s4[i]);
  // Tail bytes (n % 16): one byte per thread of the first block.
  if (blockIdx.x == 0) {
    for (int64_t j = (nvec << 4) + threadIdx.x; j < n; j += blockDim.x) {
      const uint32_t v = src[j];
      if (FORWARD) {
        bad |= ocp_nan4(v) & 0x80u;
        count += codec_rounded4(v) & 1u;
        dst[j] = static_cast<uint8_t>(codec_half4(v));
      } else {
        bad |= half_invalid4(v) & 0x80u;
        dst[j] = static_cast<uint8_t>(codec_double4(v));
      }
    }
  }
  block_status(count, bad, FORWARD ? kFlagNanCode : kFlagInvalidHalf, flags, rounded);
}

// Byte-granular variant for buffers that are not 16-byte aligned.
template <bool FORWARD>
__global__ __launch_bounds__(256) void codec_unaligned_kernel(const uint8_t* __restrict__ src,
                                                              uint8_t* __restrict__ dst, int64_t n,
                                                              uint32_t* __restrict__ flags,
                                                              unsigned long long* __restrict__ rounded) {
  const int64_t stride = static_cast<int64_t>(gridDim.x) * blockDim.x;
  uint32_t bad = 0, count = 0;
  for (int64_t j = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; j < n; j += stride) {
    const uint32_t v = src[j];
    if (FORWARD) {
      bad |= ocp_nan4(v) & 0x80u;
      count += codec_rounded4(v) & 1u;
      dst[j] = static_cast<uint8_t>(codec_half4(v));
    } else {
      bad |= half_invalid4(v) & 0x80u;
      dst[j] = static_cast<uint8_t>(codec_double4(v));
    }
  }
  block_status(count, bad, FORWARD ? kFlagNanCode : kFlagInvalidHalf, flags, rounded);
}

// Scales: forward doubles, inverse halves; both validate (finite, >= 0).
template <bool FORWARD>
__global__ __launch_bounds__(256) void codec_scales_kernel(const float* __restrict__ s, float* __restrict__ out,
                                                           int64_t n, uint32_t* __restrict__ flags) {
  uint32_t f = 0;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < n;
       i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const float v = s[i];
    const uint32_t b = f32_bits(v);
    if (!(v >= 0.0f) || (b & 0x7f800000u) == 0x7f800000u) f |= kFlagBadScale;  // NaN, inf, negative
    if (FORWARD) {
      const float d = v * 2.0f;
      if ((f32_bits(d) & 0x7f800000u) == 0x7f800000u) f |= kFlagScaleOverflow;
      out[i] = d;
    } else {
      if ((b & 0x7f800000u) <= 0x00800000u && (b & 1u)) f |= kFlagInexactHalve;
      out[i] = v * 0.5f;
    }
  }
  f = wave_or_u32(f);
  if ((threadIdx.x & 63) == 0 && f) atomicOr(flags, f);
}

// ---- activation quantizer ----------------------------------------------------
// x: bf16 [M, K] with row stride ldx (elements).  Group-major outputs (the
// reference quant op's {128, R, G} layout): q [G][Mpad][128] codes (rows >= M
// and columns >= K are written as zero), sa [G][Mpad] fp32 (zero for rows >=
// M).  One group = 16 lanes x 8 elements (quant_group8); each 16-lane set
// takes U consecutive groups and issues their loads before quantizing any
// (bytes in flight: the kernel streams ~1.5 B per element).  PACKED writes q
// in the decode fragment layout instead (Mpad = 16, 32 or 64;
// gk_fp8_internal.h).
template <bool HALF, bool PACKED, int U>
__global__ __launch_bounds__(256) void act_quant_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                        int K, int G, int Mpad, uint8_t* __restrict__ q,
                                                        float* __restrict__ sa, int vec_ok) {
  const int64_t gid0 = (static_cast<int64_t>(blockIdx.x) * (blockDim.x >> 4) + (threadIdx.x >> 4)) * U;
  const int sub = threadIdx.x & 15;
  const int64_t total = static_cast<int64_t>(Mpad) * G;
  uint4 raw[U];
  int64_t row[U];
  int gg[U];
  bool active[U], live[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int64_t gid = gid0 + u;
    active[u] = gid < total;
    row[u] = active[u] ? gid / G : 0;
    gg[u] = active[u] ? static_cast<int>(gid - row[u] * G) : 0;
    const int col = gg[u] * 128 + sub * 8;
    live[u] = active[u] && row[u] < M;
    raw[u] = make_uint4(0u, 0u, 0u, 0u);
    if (live[u] && col + 8 <= K && vec_ok) {
      raw[u] = *reinterpret_cast<const uint4*>(x + row[u] * ldx + col);
    } else if (live[u]) {
      uint32_t h[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) h[i] = (col + i < K) ? x[row[u] * ldx + col + i] : 0u;
      raw[u] = make_uint4(h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16));
    }
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    float s;
    const uint2 codes = quant_group8(raw[u], live[u], HALF, &s);  // all 16 lanes of a group take part
    if (active[u]) {
      const int64_t slot = static_cast<int64_t>(gg[u]) * Mpad + row[u];
      // bytes [8 sub, 8 sub + 8): 16-byte chunk c = sub / 2 goes to piece (c % 2, 16 (c / 2) + row)
      const int64_t at = PACKED ? decode_layout_offset(gg[u], row[u], 8 * sub, Mpad) : slot * 128 + sub * 8;
      *reinterpret_cast<uint2*>(q + at) = live[u] ? codes : make_uint2(0u, 0u);
      if (sub == 0) sa[slot] = live[u] ? s : 0.0f;
    }
  }
}

// ---- load-time weight packing (fragment order of the FP8 matrix instructions) ----
// One thread per 16-byte piece o of the output: block b = o / 128 = (tile t,
// group g), piece (h, l) = ((o / 64) % 2, o % 64) <- bytes [128 g + 32 (l/16)
// + 16 h, +16) of row 16 t + l%16; rows >= N give zeros.  The writes are
// contiguous; each wave's reads cover 16 rows x 64 bytes.
//
// Block order: tile-major (PANELS = false: b = t G + g, launch_pack_weight)
// or, for expert weights, panel-major (launch_pack_experts): tiles in panels
// of 16 (256 rows); panel p's blocks start at p 16 G, group by group, each
// group's nbp = min(16, T - 16 p) tiles side by side (b = 16 G p + g nbp +
// t % 16).  Both orders hold the same blocks in the same T G 2 KB.  Expert e
// starts at e T G 2 KB (grid over all experts).
template <bool PANELS>
__global__ __launch_bounds__(256) void pack_weight_kernel(const uint8_t* __restrict__ w, int N, int K, int G,
                                                          uint8_t* __restrict__ out, int64_t pieces,
                                                          int64_t per_expert) {
  const int T = (N + 15) >> 4;
  for (int64_t o = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; o < pieces;
       o += static_cast<int64_t>(gridDim.x) * blockDim.x) {
    const int64_t e = o / per_expert, oe = o - e * per_expert;
    const int64_t b = oe >> 7;
    const int h = static_cast<int>((oe >> 6) & 1), l = static_cast<int>(oe & 63);
    int t, g;
    if (PANELS) {
      const int p = static_cast<int>(b / (16 * G));
      const int r = static_cast<int>(b - static_cast<int64_t>(p) * 16 * G);
      const int nbp = min(16, T - 16 * p);
      g = r / nbp;
      t = 16 * p + (r - g * nbp);
    } else {
      t = static_cast<int>(b / G);
      g = static_cast<int>(b - static_cast<int64_t>(t) * G);
    }
    const int row = 16 * t + (l & 15);
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < N)
      v = *reinterpret_cast<const uint4*>(w + (e * N + row) * static_cast<int64_t>(K) + 128 * g + 32 * (l >> 4) +
                                          16 * h);
    *reinterpret_cast<uint4*>(out + o * 16) = v;
  }
}

// ---- launchers -----------------------------------------------------------------
static int codec_grid(int64_t nvec) {
  int64_t blocks = (nvec + 255) / 256;
  if (blocks < 1) blocks = 1;
  if (blocks > 8192) blocks = 8192;  // grid-stride beyond 32 blocks per CU
  return static_cast<int>(blocks);
}

hipError_t launch_codec(bool forward, const uint8_t* src, uint8_t* dst, int64_t n, const float* scales,
                        float* scales_out, int64_t n_scales, uint32_t* flags, unsigned long long* rounded,
                        hipStream_t stream) {
  const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
  if (vec) {
    const int blocks = codec_grid(n >> 4) < 1024 ? codec_grid(n >> 4) : 1024;  // 4 per CU, grid-stride
    if (forward)
      codec_bytes_kernel<true><<<blocks, 256, 0, stream>>>(src, dst, n, flags, rounded);
    else
      codec_bytes_kernel<false><<<blocks, 256, 0, stream>>>(src, dst, n, flags, rounded);
  } else {
    const int blocks = codec_grid(n) < 1024 ? codec_grid(n) : 1024;
    if (forward)
      codec_unaligned_kernel<true><<<blocks, 256, 0, stream>>>(src, dst, n, flags, rounded);
    else
      codec_unaligned_kernel<false><<<blocks, 256, 0, stream>>>(src, dst, n, flags, rounded);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (n_scales > 0) {
    const int sblocks = codec_grid(n_scales / 16 + 1);
    if (forward)
      codec_scales_kernel<true><<<sblocks, 256, 0, stream>>>(scales, scales_out, n_scales, flags);
    else
      codec_scales_kernel<false><<<sblocks, 256, 0, stream>>>(scales, scales_out, n_scales, flags);
    e = hipGetLastError();
  }
  return e;
}

hipError_t launch_pack_weight(const uint8_t* w, int N, int K, uint8_t* packed, hipStream_t stream) {
  if (N < 1 || K < 128 || K % 128 != 0) return hipErrorInvalidValue;
  const int64_t pieces = packed_weight_bytes(N, K) / 16;
  pack_weight_kernel<false><<<codec_grid(pieces), 256, 0, stream>>>(w, N, K, K / 128, packed, pieces, pieces);
  return hipGetLastError();
}

hipError_t launch_pack_experts(const uint8_t* w, int E, int N, int K, uint8_t* packed, hipStream_t stream) {
  if (E < 1 || N < 1 || K < 128 || K % 128 != 0) return hipErrorInvalidValue;
  const int64_t per = packed_weight_bytes(N, K) / 16;
  pack_weight_kernel<true><<<codec_grid(per * E), 256, 0, stream>>>(w, N, K, K / 128, packed, per * E, per);
  return hipGetLastError();
}

hipError_t launch_act_quant(const uint16_t* x, int64_t ldx, int M, int K, int Mpad, uint8_t* q, float* sa,
                            bool half, bool packed, hipStream_t stream) {
  if (packed && Mpad != 16 && Mpad != 32 && Mpad != 64) return hipErrorInvalidValue;
  const int G = (K + 127) / 128;
  const int64_t groups = static_cast<int64_t>(Mpad) * G;
  const int vec_ok = ((reinterpret_cast<uintptr_t>(x) & 15) == 0) && (ldx % 8 == 0);
  // Four groups per 16 lanes once there are enough groups to keep every CU
  // busy with them (prefill-sized inputs); decode-sized inputs keep one.
  const bool wide = groups >= 65536;
  const int per = wide ? 64 : 16;  // groups per 256-thread block
  const int blocks = static_cast<int>((groups + per - 1) / per);
#define GK_AQ(H, P)                                                                                          \
  do {                                                                                                       \
    if (wide) act_quant_kernel<H, P, 4><<<blocks, 256, 0, stream>>>(x, ldx, M, K, G, Mpad, q, sa, vec_ok);     \
    else act_quant_kernel<H, P, 1><<<blocks, 256, 0, stream>>>(x, ldx, M, K, G, Mpad, q, sa, vec_ok);          \
  } while (0)
  if (half) {
    if (packed) GK_AQ(true, true); else GK_AQ(true, false);
  } else {
    if (packed) GK_AQ(false, true); else GK_AQ(false, false);
  }
#undef GK_AQ
  return hipGetLastError();
}

}  // namespace gk
