// Large-M prefill block-FP8 GEMM for gfx950: 256 x 256 output tile per
// workgroup, FP8 MFMA 32x32x64, per-128-K-group fp32 scale promotion.
//
// Same arithmetic as the other variants (block_fp8_oracle.py:38-46): each
// 128-K group's exact fp8 x fp8 partial (two chained MFMAs over K = 64) is
// multiplied by sa[m, g] * sw[n / 128, g] and accumulated in fp32; bias and
// bf16 rounding happen in the epilogue.
//
// Structure (one workgroup = 8 waves, 4 along N x 2 along M, 64 x 128 each):
//   * Stage = one 128-K group: the 256 x 128-byte weight tile and the 256 x
//     128-byte activation tile, copied global -> LDS with direct-to-LDS loads
//     (buffer_load_dwordx4 ... lds: each wave instruction moves 8 rows x 128 B).
//     Weights rotate through three LDS stages and are loaded two steps ahead
//     (they come from HBM); activations rotate through two and are loaded one
//     step ahead (they are re-read by every weight panel and come from L2).
//     Step g waits only for its own tiles: the weights of step g+1 and the
//     token scales stay in flight across its barrier.
//   * LDS rows are 128 bytes with the 16-byte chunk c of row r stored at slot
//     c ^ ((r >> 1) & 7): sixteen consecutive rows reading one chunk hit 16
//     distinct 16-byte bank groups (measured: zero LDS bank conflicts).
//   * Fragment reads are issued as inline-asm ds_read_b128 with explicit
//     lgkmcnt waits tied to the fragment registers.  The compiler then does
//     not treat them as reads that may alias the in-flight direct-to-LDS
//     loads of the next stage (it would otherwise wait for those loads before
//     every fragment read and serialize the pipeline).
//   * 32x32 output layout: lane l, register r -> n = 8 (r/4) + 4 (l/32) + r%4,
//     m = l % 32: one token per lane, so the promotion factor is one scalar.

#include <mutex>

#include "gk_fp8_tile.h"

namespace gk {

namespace {

constexpr int kBN = 256, kBM = 256;        // workgroup tile (weight rows x tokens)
constexpr int kTile = 256 * 128;           // one operand tile of one group in LDS
constexpr int kWStages = 3, kAStages = 2;  // weight / activation stages
constexpr int kLdsBytes = (kWStages + kAStages) * kTile;  // 160 KB: all of the LDS

// Word 3 of a raw buffer resource on gfx9-family parts (data format 32; the
// format is not used by the dword loads here, but must be valid).
constexpr int kBufferWord3 = 0x00020000;

__device__ inline __attribute__((address_space(3))) void* lds_ptr(uint8_t* p) {
  return reinterpret_cast<__attribute__((address_space(3))) void*>(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>(p)));
}

__device__ inline u32x4 lds_read16(uint32_t addr) {
  u32x4 r;
  asm volatile("ds_read_b128 %0, %1" : "=v"(r) : "v"(addr));
  return r;
}

__device__ inline v8i lds_frag(uint32_t a0, uint32_t a1) {
  const u32x4 lo = lds_read16(a0), hi = lds_read16(a1);
  v8i r;
  r[0] = lo[0]; r[1] = lo[1]; r[2] = lo[2]; r[3] = lo[3];
  r[4] = hi[0]; r[5] = hi[1]; r[6] = hi[2]; r[7] = hi[3];
  return r;
}

__device__ inline v8i half_codes(v8i v) {  // native_half: OCP codes -> value / 2 (codec_half4)
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = static_cast<int>(codec_half4(static_cast<uint32_t>(v[i])));
  return v;
}

__device__ inline void promote(v16f& acc, const v16f& t, float f) {
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = fmaf(t[r], f, acc[r]);
}

// Grouped (MoE) form: the rows of qa are expert segments starting at
// group_off[e] (multiples of 256, group_off[n_groups] = rows in use) with
// group_cnt[e] live rows; the tile's rows belong to expert e, whose weights
// are w + e * w_stride and scales sw + e * sw_stride.  Tiles past
// group_off[n_groups] exit at once.
//
// Live rows: a wave skips the MFMAs, fragment reads and stores of its 32-row
// blocks that lie past the tile's live rows (rows >= M, or past the expert's
// live rows): their outputs are never read.  The other wave of the SIMD then
// has the matrix core to itself.
//
// fp32 output (yp != nullptr): the tile stores fp32 sums to yp[part][m][n]
// (row stride ldyp, plane stride M * ldyp) instead of bf16 y (no bias).  K
// split (kparts = 2, grid doubled, needs yp): the second half of the grid
// takes the second half of the groups.  accum: the sums start from yp.
//
// K range (gs > G): w and sw point at the range's first group; gs is the
// groups of the whole weight row (scale row stride, packed tile stride in
// 2 KB blocks) while K stays the row-major weight row stride.
//
// CH (per-token / per-channel scaling): activations row-major [M][ldq] (rows
// past M re-read row M-1), sa [M], sw [N]; the MFMAs accumulate over all of
// K and the epilogue applies bf16(fma(p * sa[m], sw[n], bias[n]))
// (channel_finish.c:9-15).
//
// WPACK: weights in the fragment-packed layout (launch_pack_weight): chunk c
// of row r in group g is piece (c & 1, 16 (c >> 1) + r % 16) of the 2 KB
// block (r / 16, g).  The weight tile is kept in LDS in that packed order, so
// each loader instruction copies 1 KB of contiguous global memory (wave w:
// blocks 2w and 2w + 1), and a fragment's two chunks (fc, fc + 1) are the
// pieces h = 0, 1 of one lane slot, 1024 bytes apart.
template <bool HALF, bool GROUPED, bool CH = false, bool WPACK = false>
__global__ __launch_bounds__(512) void gemm_prefill256_kernel(const uint8_t* __restrict__ qa,
                                                              const float* __restrict__ sa,
                                                              const uint8_t* __restrict__ w,
                                                              const float* __restrict__ sw,
                                                              const float* __restrict__ bias,
                                                              uint16_t* __restrict__ y, int64_t ldy, int M, int N,
                                                              int K, int G, int Mpad,
                                                              const int32_t* __restrict__ group_off,
                                                              const int32_t* __restrict__ group_cnt, int n_groups,
                                                              int64_t w_stride, int64_t sw_stride, int kparts,
                                                              float* __restrict__ yp, int64_t ldq, int gs,
                                                              int64_t ldyp, int accum) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it are scalar
  const int wn = wave & 3, wm = wave >> 2;
  const int tiles_m = Mpad / kBM;
  const int tiles = tiles_m * ((N + kBN - 1) / kBN);
  const int part = static_cast<int>(blockIdx.x) / tiles, bid = static_cast<int>(blockIdx.x) % tiles;
  const int tn = bid / tiles_m, tm = bid % tiles_m;
  const int n0 = tn * kBN, m0 = tm * kBM;  // consecutive workgroups share the weight panel
  int live = M - m0;                       // rows of this tile whose outputs are used
  if (GROUPED) {
    if (m0 >= group_off[n_groups]) return;  // uniform across the workgroup
    int e = 0;
    while (e + 1 < n_groups && group_off[e + 1] <= m0) ++e;
    w += e * w_stride;
    sw += e * sw_stride;
    live = min(live, group_cnt[e] - (m0 - group_off[e]));
  }
  // 32-row blocks of this wave's 128 rows that hold live rows (wave-uniform)
  const int jlive = min(4, max(0, (live - wm * 128 + 31) / 32));
  const int gbeg = (G * part) / kparts, gend = (G * (part + 1)) / kparts;

  // Loader: wave w fills weight rows and activation rows [32 w, 32 w + 32) of
  // the stage, 4 + 4 instructions of 8 rows; lane -> (row r0 + 8 i, slot ls)
  // fetches chunk ls ^ key(row).  Weight rows past N re-read row N-1.
  const int lr = lane >> 3, ls = lane & 7;
  const int r0 = wave * 32 + lr;
  int lcs[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) lcs[i] = (ls ^ (((r0 + 8 * i) >> 1) & 7)) * 16;
  // Loader addresses: a wave-uniform base (scalar registers) plus a per-lane
  // 32-bit offset.  Packed weights need one lane offset (lane * 16) and the
  // group-major activations two (the chunk key of rows r0 + 8 i alternates with
  // i % 2); row-major weights and per-token activations clamp every row, so
  // they keep one offset per instruction.
  const uint8_t* asrc = w + static_cast<int64_t>(n0) * K;  // packed: tile n0/16 starts at (n0/16) * G * 2048 = n0 * K
  const uint8_t* bsrc = qa + static_cast<int64_t>(m0) * (CH ? ldq : 128);
  const int nmax = N - 1 - n0, mmax = M - 1 - m0;
  const int nblk = ((N + 15) >> 4) - 1 - (n0 >> 4);  // last 16-row block of the panel
  const uint32_t lane16 = static_cast<uint32_t>(lane) * 16u;
  const uint32_t bl0 = lr * 128 + ((ls ^ (lr >> 1)) << 4), bl1 = lr * 128 + ((ls ^ (lr >> 1) ^ 4) << 4);
  uint32_t aoff[4], boff[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    aoff[i] = static_cast<uint32_t>(min(r0 + 8 * i, nmax) * K + lcs[i]);
    boff[i] = static_cast<uint32_t>(min(r0 + 8 * i, mmax) * ldq + lcs[i]);
  }
  // Activation rows [32 wave, +32) past the tile's live rows are never read
  // (every wave skips its 32-row blocks past them): their copies are skipped.
  const bool act_live = wave * 32 < live;  // wave-uniform
  // Tile copies are buffer loads with the LDS bit (buffer_load_dwordx4 ... lds):
  // the compiler counts them exactly, so the token-scale loads issued between
  // them get partial vmcnt waits.  (With the FLAT-encoded global_load_lds it
  // waits for every load in flight before the first use of any loaded value.)
  // Offsets stay below 2^32 (prefill256_fits, launch_gemm_channel256); the
  // records field is at its maximum, so no load is range-clipped.
  const __amdgpu_buffer_rsrc_t wrsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(asrc), 0, -1, kBufferWord3);
  const __amdgpu_buffer_rsrc_t arsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(bsrc), 0, -1, kBufferWord3);
  // Exactly four load instructions each: the step's wait counts on it.
  auto issue_w = [&](int g, int ws) {
    uint8_t* base = smem + ws * kTile + wave * 32 * 128;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t vo, so;
      if (WPACK) {  // block 2 wave + i/2 of the tile (blocks past the last re-read the last one), half i % 2
        const int blk = min(2 * wave + (i >> 1), nblk);
        vo = lane16;
        so = static_cast<uint32_t>((blk * gs + g) * 2048 + (i & 1) * 1024);
      } else {
        vo = aoff[i];
        so = static_cast<uint32_t>(g) * 128u;
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(wrsrc, lds_ptr(base + i * 1024), 16, vo, so, 0, 0);
    }
  };
  auto issue_a = [&](int g, int as) {
    if (!act_live) return;
    uint8_t* base = smem + (kWStages + as) * kTile + wave * 32 * 128;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint32_t vo, so;
      if (CH) {
        vo = boff[i];
        so = static_cast<uint32_t>(g) * 128u;
      } else {  // rows r0 + 8 i of group g: (wave * 32 + 8 i) * 128 + the lane's row and chunk
        vo = (i & 1) ? bl1 : bl0;
        so = static_cast<uint32_t>(g) * static_cast<uint32_t>(Mpad * 128) + static_cast<uint32_t>((wave * 32 + 8 * i) * 128);
      }
      __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, lds_ptr(base + i * 1024), 16, vo, so, 0, 0);
    }
  };

  // Fragments: lane -> row (lane & 31) of a 32-row strip, chunks h*4 + 2 (lane >> 5) + {0, 1}.
  const int fr = lane & 31, fc = (lane >> 5) * 2, kf = (fr >> 1) & 7;
  const uint32_t xo00 = ((0 + fc) ^ kf) << 4, xo01 = ((1 + fc) ^ kf) << 4;
  const uint32_t xo10 = ((4 + fc) ^ kf) << 4, xo11 = ((5 + fc) ^ kf) << 4;
  // packed weight tile: row ra = wn*64 + fr, chunk fc + h (+4 for the second K half) ->
  // (ra/16)*2048 + h*1024 + 16*(16*((fc + 4k)/2) + ra%16)
  const uint32_t pa = ((wn * 64 + fr) >> 4) * 2048 + 16 * (16 * (lane >> 5) + (fr & 15));
  const uint32_t ya00 = WPACK ? 0u : xo00, ya01 = WPACK ? 1024u : xo01;
  const uint32_t ya10 = WPACK ? 512u : xo10, ya11 = WPACK ? 1536u : xo11;
  const uint32_t lbase = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  const uint32_t arow = WPACK ? pa : (wn * 64 + fr) * 128, brow = kWStages * kTile + (wm * 128 + fr) * 128;
  const float* sap = sa + (m0 + wm * 128 + fr);  // + 32 j + g * Mpad  (m0 + 256 <= Mpad)
  const float* swp = sw + static_cast<int64_t>(min(n0 + wn * 64, N - 1) >> 7) * gs;
  float* ypp = yp ? yp + static_cast<int64_t>(part) * M * ldyp : nullptr;

  // Accumulator element (i, j, 4 q + r) is output (m0 + wm*128 + 32 j + fr,
  // n0 + wn*64 + 32 i + 8 q + 4 (lane/32) + r).  With accum the sums start
  // from the fp32 partial in yp, so K ranges accumulated over several calls
  // give the bits of one call over their union.
  v16f acc[2][4];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
  if (accum) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int m = m0 + wm * 128 + j * 32 + fr;
        if (j >= jlive || m >= M) continue;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const int n = n0 + wn * 64 + i * 32 + 8 * q + 4 * (lane >> 5);
#pragma unroll
          for (int r = 0; r < 4; ++r)
            if (n + r < N) acc[i][j][4 * q + r] = ypp[static_cast<int64_t>(m) * ldyp + n + r];
        }
      }
  }

  // Issue order in step g: token scales of g + 1 (before the wait), then, past
  // the barrier, activations of g + 1 and weights of g + 2.  Weights are issued
  // at every step (past the last group they re-read it into a stage no later
  // step reads), so at the top of step g the loads younger than step g's
  // activations are exactly weights g + 1 and scales g + 1: vmcnt(8) (vmcnt(4)
  // in the CH form, which loads no token scales) completes step g's tiles and
  // leaves those in flight.  The compiler tracks the scale loads itself; it
  // counts the buffer loads exactly, so its waits for them are partial too.
  float sv[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // token scales of the next step
  auto load_sav = [&](int g) {
    if (!CH) {
#pragma unroll
      for (int j = 0; j < 4; ++j) sv[j] = sap[j * 32 + static_cast<int64_t>(g) * Mpad];
    }
  };
  // (An empty K range, a K-split half with no groups, stores zeros.)
  if (gbeg < gend) {
    issue_w(gbeg, 0);
    load_sav(gbeg);
    issue_a(gbeg, 0);
    issue_w(min(gbeg + 1, gend - 1), 1);
    int ws = 0, as = 0;  // stages of step g
    int g = gbeg;
    do {
      // native_half doubles the weight scales (block_fp8_oracle.py:35); x2 is exact.
      const float swg = CH ? 0.0f : (HALF ? 2.0f * swp[g] : swp[g]);
      float fj[4];  // promotion factors of step g
#pragma unroll
      for (int j = 0; j < 4; ++j) fj[j] = sv[j] * swg;
      load_sav(min(g + 1, gend - 1));
      asm volatile("" ::: "memory");  // the scale loads stay ahead of the wait, whose count includes them
      // This wave's tile loads of step g are done: vmcnt(8) or vmcnt(4), expcnt(7), lgkmcnt(15).
      if (CH)
        __builtin_amdgcn_s_waitcnt(0x0F74);
      else
        __builtin_amdgcn_s_waitcnt(0x0F78);
      // ... for every wave; all fragment reads of step g-1 are done too (each
      // step's reads end with lgkmcnt(0)).  A bare barrier: __syncthreads()'s
      // release fence would wait for the weight loads still in flight.
      __builtin_amdgcn_s_barrier();
      if (g + 1 < gend) issue_a(g + 1, as ^ 1);
      issue_w(min(g + 2, gend - 1), ws == 0 ? 2 : ws - 1);  // the stage step g-1 used
      const uint32_t A = lbase + ws * kTile + arow;
      const uint32_t B = lbase + as * kTile + brow;
      ws = ws == 2 ? 0 : ws + 1;
      as ^= 1;
      if (jlive == 0) continue;  // no live rows for this wave (it still takes part in the loads and barriers)
      v8i a00 = lds_frag(A + ya00, A + ya01), a01 = lds_frag(A + ya10, A + ya11);
      v8i a10 = lds_frag(A + 4096 + ya00, A + 4096 + ya01), a11 = lds_frag(A + 4096 + ya10, A + 4096 + ya11);
      v8i b0 = lds_frag(B + xo00, B + xo01), b1 = lds_frag(B + xo10, B + xo11);
      asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(a00), "+v"(a01), "+v"(a10), "+v"(a11), "+v"(b0), "+v"(b1));
      if (HALF) {
        a00 = half_codes(a00); a01 = half_codes(a01); a10 = half_codes(a10); a11 = half_codes(a11);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j < jlive) {  // wave-uniform; j is a constant after unrolling, so acc stays in registers
          if (j > 0) {
            b0 = lds_frag(B + j * 4096 + xo00, B + j * 4096 + xo01);
            b1 = lds_frag(B + j * 4096 + xo10, B + j * 4096 + xo11);
            asm volatile("s_waitcnt lgkmcnt(0)" : "+v"(b0), "+v"(b1));
          }
          if (CH) {
            acc[0][j] = mfma32_f8(a00, b0, acc[0][j]);
            acc[1][j] = mfma32_f8(a10, b0, acc[1][j]);
            acc[0][j] = mfma32_f8(a01, b1, acc[0][j]);
            acc[1][j] = mfma32_f8(a11, b1, acc[1][j]);
          } else {
            const float f = fj[j];
            v16f t;
#pragma unroll
            for (int r = 0; r < 16; ++r) t[r] = 0.0f;
            t = mfma32_f8(a01, b1, mfma32_f8(a00, b0, t));
            promote(acc[0][j], t, f);
#pragma unroll
            for (int r = 0; r < 16; ++r) t[r] = 0.0f;
            t = mfma32_f8(a11, b1, mfma32_f8(a10, b0, t));
            promote(acc[1][j], t, f);
          }
        }
      }
    } while (++g < gend);
  }

  __builtin_amdgcn_s_waitcnt(0);  // the re-read weight loads still in flight write LDS

  if (CH) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < jlive) {
        const int m = m0 + wm * 128 + j * 32 + fr;
        if (m < M) {
          const float sam = sa[m];
          uint16_t* row = y + static_cast<int64_t>(m) * ldy;
#pragma unroll
          for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
              const int n = n0 + wn * 64 + i * 32 + 8 * q + 4 * (lane >> 5);
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (n + r < N)
                  row[n + r] = channel_out(acc[i][j][4 * q + r], sam, sw[n + r], bias ? bias[n + r] : 0.0f);
            }
        }
      }
    }
    return;
  }
  if (yp) {
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if (j < jlive) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int m = m0 + wm * 128 + j * 32 + fr, n = n0 + wn * 64 + i * 32 + 8 * q + 4 * (lane >> 5);
            if (m >= M) continue;
            float* dst = ypp + static_cast<int64_t>(m) * ldyp + n;
            const v4f v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
            if (n + 3 < N && (reinterpret_cast<uintptr_t>(dst) & 15) == 0) {
              *reinterpret_cast<v4f*>(dst) = v;
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r)
                if (n + r < N) dst[r] = v[r];
            }
          }
        }
      }
    return;
  }
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if (j < jlive) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const v4f v = {acc[i][j][4 * q], acc[i][j][4 * q + 1], acc[i][j][4 * q + 2], acc[i][j][4 * q + 3]};
          store_tile(y, ldy, bias, M, N, m0 + wm * 128 + j * 32 + fr,
                     n0 + wn * 64 + i * 32 + 8 * q + 4 * (lane >> 5), v);
        }
      }
    }
}

// The 128 KB of dynamic LDS is above the default limit: raise it once per device.
constexpr int kMaxDevices = 64;

std::once_flag g_lds_once[kMaxDevices][16];
hipError_t g_lds_err[kMaxDevices][16];

template <bool HALF, bool GROUPED, bool CH = false, bool WPACK = false>
hipError_t ensure_lds_limit() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  constexpr int slot = (HALF ? 1 : 0) + (GROUPED ? 2 : 0) + (CH ? 4 : 0) + (WPACK ? 8 : 0);
  std::call_once(g_lds_once[dev][slot], [dev] {
    g_lds_err[dev][slot] = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_prefill256_kernel<HALF, GROUPED, CH, WPACK>),
        hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  });
  return g_lds_err[dev][slot];
}

template <bool HALF, bool GROUPED, bool WPACK = false>
hipError_t launch256(const GemmArgs& a, const int32_t* group_off, const int32_t* group_cnt, int n_groups,
                     int64_t w_stride, int64_t sw_stride, int kparts, float* yp, int64_t ldyp, hipStream_t stream) {
  hipError_t e = ensure_lds_limit<HALF, GROUPED, false, WPACK>();
  if (e != hipSuccess) return e;
  const unsigned tiles = static_cast<unsigned>(((a.N + kBN - 1) / kBN) * (a.Mpad / kBM));
  gemm_prefill256_kernel<HALF, GROUPED, false, WPACK><<<tiles * kparts, 512, kLdsBytes, stream>>>(
      a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy, a.M, a.N, a.K, a.G, a.Mpad, group_off, group_cnt, n_groups,
      w_stride, sw_stride, kparts, yp, 0, a.gstride(), ldyp, a.accumulate ? 1 : 0);
  return hipGetLastError();
}

}  // namespace

// Per-token / per-channel form: a.qa row-major [M][a.ldq], a.sa [M], a.sw [N]; any M.
hipError_t launch_gemm_channel256(const GemmArgs& a, hipStream_t stream) {
  if (static_cast<int64_t>(256) * a.ldq > int64_t{0xffffffff} || static_cast<int64_t>(256) * a.K > int64_t{0xffffffff})
    return hipErrorInvalidValue;
  hipError_t e = ensure_lds_limit<false, false, true>();
  if (e != hipSuccess) return e;
  const int mpad = (a.M + kBM - 1) / kBM * kBM;
  const unsigned tiles = static_cast<unsigned>(((a.N + kBN - 1) / kBN) * (mpad / kBM));
  gemm_prefill256_kernel<false, false, true><<<tiles, 512, kLdsBytes, stream>>>(
      a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy, a.M, a.N, a.K, a.G, mpad, nullptr, nullptr, 0, 0, 0, 1, nullptr,
      a.ldq, a.G, 0, 0);
  return hipGetLastError();
}

// Requires K % 128 == 0, 16-byte aligned weights, Mpad % 256 == 0 (qa/sa
// padded with zero rows up to Mpad).
hipError_t launch_gemm_prefill256(const GemmArgs& a, hipStream_t stream) {
  if (a.Mpad % kBM != 0 || !prefill256_fits(a)) return hipErrorInvalidValue;
  if (a.wpack)
    return a.half_w ? launch256<true, false, true>(a, nullptr, nullptr, 0, 0, 0, 1, a.yp, a.ldyp, stream)
                    : launch256<false, false, true>(a, nullptr, nullptr, 0, 0, 0, 1, a.yp, a.ldyp, stream);
  return a.half_w ? launch256<true, false>(a, nullptr, nullptr, 0, 0, 0, 1, a.yp, a.ldyp, stream)
                  : launch256<false, false>(a, nullptr, nullptr, 0, 0, 0, 1, a.yp, a.ldyp, stream);
}

// Grouped form: a.Mpad = padded rows (multiple of 256), a.M = a.Mpad; weights
// [n_groups][N][K] (a.wpack: each group's weights packed by launch_pack_weight,
// one after the other), scales [n_groups][ceil(N/128)][G]; group_off,
// group_cnt on device.
hipError_t launch_gemm_grouped256(const GemmArgs& a, const int32_t* group_off, const int32_t* group_cnt,
                                  int n_groups, int kparts, float* yp, hipStream_t stream) {
  if (a.Mpad % kBM != 0 || n_groups < 1 || kparts < 1 || kparts > 2 || (kparts > 1 && !yp) || (yp && a.N % 4) ||
      !prefill256_fits(a))
    return hipErrorInvalidValue;
  const int64_t w_stride = a.wpack ? packed_weight_bytes(a.N, a.K) : static_cast<int64_t>(a.N) * a.K;
  const int64_t sw_stride = static_cast<int64_t>((a.N + 127) / 128) * a.G;
  if (a.wpack)
    return a.half_w ? launch256<true, true, true>(a, group_off, group_cnt, n_groups, w_stride, sw_stride, kparts, yp,
                                                  a.N, stream)
                    : launch256<false, true, true>(a, group_off, group_cnt, n_groups, w_stride, sw_stride, kparts,
                                                   yp, a.N, stream);
  return a.half_w ? launch256<true, true>(a, group_off, group_cnt, n_groups, w_stride, sw_stride, kparts, yp, a.N,
                                          stream)
                  : launch256<false, true>(a, group_off, group_cnt, n_groups, w_stride, sw_stride, kparts, yp, a.N,
                                           stream);
}

}  // namespace gk
