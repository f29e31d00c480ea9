// Large-M prefill block-FP8 GEMM for gfx950: 256 x 256 output tile per
// workgroup, FP8 MFMA 16x16x128, per-128-K-group fp32 scale promotion.
//
// Same arithmetic as the other variants (block_fp8_oracle.py:38-46): each
// 128-K group's fp8 x fp8 partial (one v_mfma_f32_16x16x128_f8f6f4 per 16 x 16
// block) is multiplied by sa[m, g] * sw[n / 128, g] and accumulated in fp32;
// bias and bf16 rounding happen in the epilogue.
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
//     c ^ lds_key(r) (gk_fp8_lds.h): the fragment reads of any 16 and of any
//     32 consecutive lanes hit distinct 16-byte slots of a 256- and a
//     512-byte window.
//   * Fragment reads are issued as inline-asm ds_read_b128 with explicit
//     lgkmcnt waits tied to the fragment registers.  The compiler then does
//     not treat them as reads that may alias the in-flight direct-to-LDS
//     loads of the next stage (it would otherwise wait for those loads before
//     every fragment read and serialize the pipeline).
//   * A wave's step: four weight fragments (16 rows x 128 K each) read once,
//     then eight 16-token blocks j, each one activation fragment and four
//     MFMAs.  The fragment of block j + 1 is read while block j's MFMAs run
//     (a partial lgkmcnt wait), and block j - 1 is promoted after block j's
//     MFMAs are issued, so the promotion FMAs never wait on the MFMA they
//     follow; block 7's promotion waits for the next step's block 0 (past the
//     barrier and the first fragment reads; each output element still adds its
//     groups in order).  When all of a wave's token blocks are live the step is
//     straight-line code, which the scheduler interleaves freely.
//   * 16x16 output layout: lane l, register r -> n = 4 (l/16) + r, m = l % 16:
//     one token per lane, so the promotion factor is one scalar per block.
//   * Dense tiles: the younger wave of each SIMD runs the first half of a step
//     at raised priority (the two share the matrix core), and the bf16 tile
//     leaves through LDS as whole-row 16-byte stores.

#include <mutex>
#include <type_traits>
#include <utility>

#include "gk_fp8_lds.h"

namespace gk {

namespace {

#ifndef GK_PREFILL_SPREAD
#define GK_PREFILL_SPREAD 1  // dense: a step's tile loads are issued between its token blocks, not all at its top
#endif
#ifndef GK_PREFILL_BBUF
#define GK_PREFILL_BBUF 2  // activation fragments held per wave: reads run one block ahead
#endif
constexpr int kBN = 256, kBM = 256;        // workgroup tile (weight rows x tokens)
constexpr int kTile = 256 * 128;           // one operand tile of one group in LDS
constexpr int kWStages = 3, kAStages = 2;  // weight / activation stages
constexpr int kLdsBytes = (kWStages + kAStages) * kTile;  // 160 KB: all of the LDS

// Grouped (MoE) form: the rows of qa are expert segments starting at
// group_off[e] (multiples of 256, group_off[n_groups] = rows in use) with
// group_cnt[e] live rows; the tile's rows belong to expert e, whose weights
// are w + e * w_stride and scales sw + e * sw_stride.  Tiles past
// group_off[n_groups] exit at once.
//
// Live rows: a wave skips the stores of its 16-row blocks that lie past the
// tile's live rows (rows >= M, or past the expert's live rows), whose outputs
// are never read; in the grouped form it skips their MFMAs and fragment reads
// too, and the two waves of a SIMD take alternate blocks, so both keep a
// share of the live rows.
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
// pieces h = 0, 1 of one lane slot, 1024 bytes apart.  The grouped form reads
// the experts' panel-major order (launch_pack_experts): the same 2 KB blocks,
// each 256-row panel's blocks of one group side by side, so a step's weight
// tile is one contiguous run (measured on MI355X, config 5 gate_up: 259 ->
// 243 us; in the tile-major order a step reads 16 pieces 64 KB apart).
//
// SWI (grouped, NA = 4): SiLU-and-mul + 1x128 quantization fused into the
// epilogue of a gate_up GEMM, whose N = 2 inter weight rows are the gate rows
// then the up rows.  Tile tn loads gate rows [128 tn, +128) as its rows 0..127
// and up rows [inter + 128 tn, +128) as rows 128..255, so waves wn = 0, 1 hold
// gate columns and waves wn = 2, 3 the up columns of the same rows and
// columns, in the same lane layout.  The epilogue rounds both to bf16 (as the
// bf16 store does), meets them in LDS and quantizes h = bf16(silu(g) * u)
// with the same per-lane arithmetic as the separate fused quantizer, into
// group tn of swq [inter/128][Mpad][128] / sws [inter/128][Mpad]: h is never
// written to memory (measured on MI355X, config 5 MoE layer: the 59 MB bf16
// round trip and its 21 us kernel go).
//
// NA: 16-row weight blocks per wave; the tile is 64 NA weight rows (256, or
// 192 for the narrow tiles that fill the last round of a large GEMM).  A
// 48-row wave can straddle two 128-row scale blocks, so NA = 3 takes one
// weight scale per block.
// The workgroup body; `block` is the workgroup's index within its launch (or
// within its column range of the split launch below).
template <bool HALF, bool GROUPED, bool CH, bool WPACK, int NA, bool SWI = false>
__device__ __forceinline__ void prefill256_body(int block, const uint8_t* __restrict__ qa,
                                                const float* __restrict__ sa, const uint8_t* __restrict__ w,
                                                const float* __restrict__ sw, const float* __restrict__ bias,
                                                uint16_t* __restrict__ y, int64_t ldy, int M, int N, int K, int G,
                                                int Mpad, const int32_t* __restrict__ group_off,
                                                const int32_t* __restrict__ group_cnt, int n_groups,
                                                int64_t w_stride, int64_t sw_stride, int kparts,
                                                float* __restrict__ yp, int64_t ldq, int gs, int64_t ldyp,
                                                int accum, int xcd_cus, uint8_t* __restrict__ swq = nullptr,
                                                float* __restrict__ sws = nullptr) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: branches on it are scalar
  const int wn = wave & 3, wm = wave >> 2;
  constexpr int BN = 64 * NA;  // weight rows of the tile
  static_assert(!(GROUPED && WPACK) || NA == 4, "panel-major experts come in 256-row panels");
  static_assert(!SWI || (GROUPED && !CH && NA == 4), "the fused SiLU-and-mul epilogue is a grouped 256-row form");
  const int tiles_m = Mpad / kBM;
  const int tiles = tiles_m * ((N + BN - 1) / BN);
  const int tiles_nn = (N + BN - 1) / BN;
  int part = block / tiles, bid = block % tiles;
  if (GROUPED && xcd_cus <= 0 && block >= tiles * kparts) return;  // the grid's round-up to a multiple of 8
  if (GROUPED && xcd_cus > 0) {
    // A grouped grid whose live (tile, K part) pairs fit one round of the
    // xcd_cus CUs: pair l of the expert-major order (tile, then part, then
    // column panel) goes to workgroup 8 (l % q) + l / q, q = ceil(live / 8).
    // The hardware places workgroup b on XCD b % 8, so each XCD holds q
    // consecutive pairs -- one expert segment's workgroups share an L2 and
    // fetch its activation rows once, not once per XCD.  A bijection on the
    // live pairs wherever the workgroups run; the grid is a multiple of 8 and
    // its other workgroups exit.
    const int per = tiles_nn * kparts;
    const int pairs = (group_off[n_groups] / kBM) * per;
    if (pairs <= xcd_cus) {
      const int q = (pairs + 7) >> 3, l = (block & 7) * q + (block >> 3);
      if ((block >> 3) >= q || l >= pairs) return;
      const int t = l / per, r = l - t * per;
      part = r / tiles_nn;
      bid = t * tiles_nn + (r - part * tiles_nn);
    } else if (block >= tiles * kparts) {
      return;
    }
  }
  // Grouped: consecutive workgroups take consecutive panels of one expert
  // segment, whose activation tiles then stay in L2 (measured on MI355X,
  // config 5 MoE layer: 482 -> 456 us).  Dense: XCD-aware order.  Workgroup b
  // runs on XCD b % 8; in a launch (or column range) of a multiple of 8 tiles,
  // XCD x takes the x-th eighth of the tiles in super-block order (4 weight
  // panels x all row tiles, row tile by row tile), so the CUs of one XCD share
  // few panels and row tiles in its L2 (config 4: 4 panels x 8 row tiles per
  // XCD instead of 16 panels x 2 row tiles): dense_tile_of (gk_fp8_plan.h).
  int tn, tm;
  if (GROUPED) {
    tn = bid % tiles_nn;
    tm = bid / tiles_nn;
  } else {
    const int v = dense_tile_of(bid, tiles_m, tiles_nn, kparts);
    tn = v >> 16;
    tm = v & 0xffff;
  }
  const int n0 = tn * BN, m0 = tm * kBM;
  int live = M - m0;                       // rows of this tile whose outputs are used
  if (GROUPED) {
    if (m0 >= group_off[n_groups]) return;  // uniform across the workgroup
    int e = 0;
    while (e + 1 < n_groups && group_off[e + 1] <= m0) ++e;
    w += e * w_stride;
    sw += e * sw_stride;
    live = min(live, group_cnt[e] - (m0 - group_off[e]));
  }
  const int gbeg = (G * part) / kparts, gend = (G * (part + 1)) / kparts;

  // Loader: wave w fills weight rows [8 NA w, +8 NA) and activation rows
  // [32 w, +32) of the stage, NA + 4 instructions of 8 rows; lane -> (row
  // r + 8 i, slot ls) fetches chunk ls ^ key(row).  Weight rows past N re-read
  // row N-1.
  const int lr = lane >> 3, ls = lane & 7;
  const int r0 = wave * 32 + lr, rw0 = wave * 8 * NA + lr;
  int lcs[4], lcw[NA];
#pragma unroll
  for (int i = 0; i < 4; ++i) lcs[i] = (ls ^ lds_key(r0 + 8 * i)) * 16;
#pragma unroll
  for (int i = 0; i < NA; ++i) lcw[i] = (ls ^ lds_key(rw0 + 8 * i)) * 16;
  // Loader addresses: a wave-uniform base (scalar registers) plus a per-lane
  // 32-bit offset.  Packed weights need one lane offset (lane * 16) and the
  // group-major activations two (the chunk key of rows r0 + 8 i alternates with
  // i % 2); row-major weights and per-token activations clamp every row, so
  // they keep one offset per instruction.
  // SWI: weight row of this wave's first loaded tile row 32 wave (tile rows
  // 0..127 are gate rows 128 tn + r, rows 128..255 up rows inter + 128 tn + r - 128;
  // a wave's 32 rows lie in one 256-row panel).  Row-major weights start the
  // wave's view at tile row 0's weight row, packed ones at its panel.
  const int swrow = SWI ? (wave < 4 ? 128 * tn : (N >> 1) + 128 * tn - 128) + 32 * wave : 0;
  const int64_t wrow0 = SWI ? (WPACK ? (swrow & ~255) : swrow - 32 * wave) : n0;
  const int sblk = SWI ? (swrow & 255) >> 4 : 0;  // SWI, packed: the wave's first 16-row block in its panel
  const uint8_t* asrc = w + wrow0 * K;  // packed: tile n0/16 starts at (n0/16) * G * 2048 = n0 * K
  const uint8_t* bsrc = qa + static_cast<int64_t>(m0) * (CH ? ldq : 128);
  const int nmax = N - 1 - n0, mmax = M - 1 - m0;
  const int nblk = ((N + 15) >> 4) - 1 - (n0 >> 4);  // last 16-row block of the panel
  const uint32_t lane16 = static_cast<uint32_t>(lane) * 16u;
  // rows r0 + 8 i (r0 = 32 wave + lr): key lds_key(lr) for even i, lds_key(lr) ^ 4 for odd i
  const uint32_t bl0 = lr * 128 + ((ls ^ lds_key(lr)) << 4), bl1 = lr * 128 + ((ls ^ lds_key(lr) ^ 4) << 4);
  uint32_t aoff[NA], boff[4];
#pragma unroll
  for (int i = 0; i < NA; ++i) aoff[i] = static_cast<uint32_t>(min(rw0 + 8 * i, nmax) * K + lcw[i]);
#pragma unroll
  for (int i = 0; i < 4; ++i) boff[i] = static_cast<uint32_t>(min(r0 + 8 * i, mmax) * ldq + lcs[i]);
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
  // Exactly NA weight and four activation load instructions a step: the
  // step's wait counts on it.  Packed weights: wave w copies the 1 KB pieces
  // p = NA w + i of the tile (block p / 2, half p % 2; blocks past the last
  // re-read the last one).  Panel-major (GROUPED): block b of group g sits at
  // (g nbp + b) 2 KB in the panel, nbp = the panel's blocks.
  const int nbp = min(16, nblk + 1);
  auto issue_w_one = [&](int g, int ws, int i) {
    uint8_t* base = smem + ws * kTile + wave * 8 * NA * 128;
    uint32_t vo, so;
    if (WPACK) {
      const int p = NA * wave + i;
      const int blk = SWI ? sblk + (i >> 1) : min(p >> 1, nblk);
      vo = lane16;
      so = static_cast<uint32_t>((GROUPED ? g * nbp + blk : blk * gs + g) * 2048 + (p & 1) * 1024);
    } else {
      vo = aoff[i];
      so = static_cast<uint32_t>(g) * 128u;
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(wrsrc, lds_ptr(base + i * 1024), 16, vo, so, 0, 0);
  };
  // The dense form's spread copies are issued on every path (dead rows and the
  // last step included, clamped to rows and groups that exist), so the
  // compiler's vmcnt waits count the same loads on every path through a step:
  // with a conditional copy it waits for the minimum count over the paths,
  // which at the loop's back edge meant waiting for this step's weight copies
  // (measured on MI355X, config 4 GEMM: 197-204 -> 190-193 us with the
  // interleaved promotion below; M = 1024, N = 4096, K = 14336: 170 -> 153 us).
  auto issue_a_one = [&](int g, int as, int i) {
    uint8_t* base = smem + (kWStages + as) * kTile + wave * 32 * 128;
    uint32_t vo, so;
    if (CH) {
      vo = boff[i];
      so = static_cast<uint32_t>(g) * 128u;
    } else {
      vo = (i & 1) ? bl1 : bl0;
      so = static_cast<uint32_t>(g) * static_cast<uint32_t>(Mpad * 128) + static_cast<uint32_t>((wave * 32 + 8 * i) * 128);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(arsrc, lds_ptr(base + i * 1024), 16, vo, so, 0, 0);
  };
  auto issue_w = [&](int g, int ws) {
#pragma unroll
    for (int i = 0; i < NA; ++i) issue_w_one(g, ws, i);
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

  // Fragments (16x16x128 operand layout): lane -> row (lane & 15) of a
  // 16-row block, K bytes [32 (lane >> 4), +32) = chunks 2 (lane >> 4) + {0, 1}.
  // Row-major tiles keep chunk c of row r at slot c ^ lds_key(r); the
  // packed weight tile holds each 16-row block as 2 KB in fragment order
  // (piece h of lane l at h * 1024 + 16 l).
  const int fr = lane & 15, fq = lane >> 4, kf = lds_key(fr);
  const uint32_t xo0 = static_cast<uint32_t>(((2 * fq) ^ kf) << 4), xo1 = static_cast<uint32_t>(((2 * fq + 1) ^ kf) << 4);
  const uint32_t lbase = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(smem));
  // weight block i of this wave: rows wn*16*NA + 16 i
  const uint32_t arow = WPACK ? static_cast<uint32_t>(wn * NA * 2048 + 16 * lane)
                              : static_cast<uint32_t>((wn * 16 * NA + fr) * 128);
  const uint32_t ya0 = WPACK ? 0u : xo0, ya1 = WPACK ? 1024u : xo1;
  // activation block j of this wave: tile rows mw + kJS j.  Dense: the wave's
  // own 128 rows (mw = 128 wm, kJS = 16).  Grouped: the two waves of a SIMD
  // take alternate 16-row blocks (mw = 16 wm, kJS = 32), so an expert segment
  // that ends inside the tile leaves both with about half of its live rows
  // (a lone wave per SIMD hides none of its read and MFMA latency; measured on
  // MI355X, config 5 gate_up with the loads taken out: 191 us).  Each output
  // element's arithmetic is the same either way.
  constexpr int kJS = GROUPED ? 32 : 16, kJB = kJS * 128;  // block stride in rows and in LDS bytes
  const int mw = GROUPED ? 16 * wm : 128 * wm;
  const uint32_t brow = static_cast<uint32_t>(kWStages * kTile + (mw + fr) * 128);
  const float* sap = sa + (m0 + mw + fr);  // + kJS j + g * Mpad  (m0 + 256 <= Mpad)
  // weight scale rows of the wave's blocks (one for NA = 4: 64 rows at a multiple of 64)
  constexpr int kScales = NA == 4 ? 1 : NA;
  const float* swp[kScales];
#pragma unroll
  for (int i = 0; i < kScales; ++i)
    swp[i] = sw + static_cast<int64_t>(SWI ? (wn < 2 ? tn : (N >> 8) + tn)
                                           : min(n0 + wn * 16 * NA + 16 * i, N - 1) >> 7) * gs;
  float* ypp = yp ? yp + static_cast<int64_t>(part) * M * ldyp : nullptr;
  // the wave's blocks that hold live rows: j < jl (wave-uniform)
  const int jl = min(8, max(0, (live - mw + kJS - 1) / kJS));

  // Accumulator acc[i][j] register r is output (m0 + mw + kJS j + fr,
  // n0 + wn*16*NA + 16 i + 4 fq + r).  With accum the sums start from the fp32
  // partial in yp, so K ranges accumulated over several calls give the bits
  // of one call over their union.
  v4f acc[NA][8];
#pragma unroll
  for (int i = 0; i < NA; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = v4f{0.0f, 0.0f, 0.0f, 0.0f};
  if (accum) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int m = m0 + mw + j * kJS + fr;
      if (j >= jl || m >= M) continue;
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int n = n0 + wn * 16 * NA + i * 16 + 4 * fq;
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (n + r < N) acc[i][j][r] = ypp[static_cast<int64_t>(m) * ldyp + n + r];
      }
    }
  }

  // Issue order in step g: token scales of g + 1 (before the wait), then, past
  // the barrier, activations of g + 1 and weights of g + 2.  Weights are issued
  // at every step (past the last group they re-read it into a stage no later
  // step reads), so at the top of step g the loads younger than step g's
  // activations are exactly weights g + 1 and scales g + 1: vmcnt(12) (vmcnt(4)
  // in the CH form, which loads no token scales) completes step g's tiles and
  // leaves those in flight.  The compiler tracks the scale loads itself; it
  // counts the buffer loads exactly, so its waits for them are partial too.
  float sv[8] = {0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f, 0.0f};  // token scales of the next step
  auto load_sav = [&](int g) {
    if (!CH) {
#pragma unroll
      for (int j = 0; j < 8; ++j) sv[j] = sap[j * kJS + static_cast<int64_t>(g) * Mpad];
    }
  };
  // One token block: NA MFMAs on the weight fragments.
  auto block_mfma = [&](const v8i (&a)[NA], const v8i& b, v4f (&t)[NA]) {
#pragma unroll
    for (int i = 0; i < NA; ++i) t[i] = mfma_f8(a[i], b);
  };
  // (An empty K range, a K-split half with no groups, stores zeros.)
  if (gbeg < gend) {
    issue_w(gbeg, 0);
    load_sav(gbeg);
    issue_a(gbeg, 0);
    issue_w(min(gbeg + 1, gend - 1), 1);
    int ws = 0, as = 0;  // stages of step g
    int g = gbeg;
    v4f t[2][NA];
    float pf7[NA];  // the promotion factors of the previous step's block 7 (deferred past the barrier)
#pragma unroll
    for (int i = 0; i < NA; ++i) pf7[i] = 0.0f;
    do {
      // native_half doubles the weight scales (block_fp8_oracle.py:35); x2 is exact.
      float swg[NA];  // weight scales of step g (promotion factor of block (i, j): svg[j] * swg[i])
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const float v = CH ? 0.0f : swp[i < kScales ? i : 0][g];
        swg[i] = HALF ? 2.0f * v : v;
      }
      float svg[8];  // token scales of step g
#pragma unroll
      for (int j = 0; j < 8; ++j) svg[j] = sv[j];
      load_sav(min(g + 1, gend - 1));
      asm volatile("" ::: "memory");  // the scale loads stay ahead of the wait, whose count includes them
      // This wave's tile loads of step g are done: vmcnt(8 + NA) or vmcnt(NA), expcnt(7), lgkmcnt(15).
      __builtin_amdgcn_s_waitcnt(0x0F70 | (CH ? NA : 8 + NA));
      // ... for every wave; all fragment reads of step g-1 are done too (each
      // step's reads end with lgkmcnt(0)).  A bare barrier: __syncthreads()'s
      // release fence would wait for the weight loads still in flight.
      __builtin_amdgcn_s_barrier();
      // Dense: the two waves of a SIMD (wm = 0, 1) share its matrix core, and
      // the issue arbiter favours the older one, which then waits at the next
      // barrier while the younger one finishes alone (measured on MI355X with
      // per-step timers, config 4: about 900 of 3000 cycles a step).  The
      // younger wave runs the first half of the step (blocks 0..3) at raised
      // priority; both are back at 0 from block 4 (config 4 GEMM: -2%).
      if (!GROUPED && wm) __builtin_amdgcn_s_setprio(1);
      const int as_next = as ^ 1, ws_free = ws == 0 ? 2 : ws - 1;  // the stages step g-1 used
      // Dense GEMMs (MFMA-bound) spread the step's loads between the token
      // blocks; the grouped form (bound by the weight stream) issues them all
      // here, as early as possible (measured on MI355X, config 5 gate_up: 240
      // -> 233 us).
      constexpr bool kSpread = GK_PREFILL_SPREAD && !GROUPED;
      if (!kSpread) {
        if (g + 1 < gend) issue_a(g + 1, as_next);
        issue_w(min(g + 2, gend - 1), ws_free);
      }
      const uint32_t A = lbase + ws * kTile + arow;
      const uint32_t B = lbase + as * kTile + brow;
      ws = ws == 2 ? 0 : ws + 1;
      as ^= 1;
      // A wave with no live rows skips its MFMAs (GROUPED: every block; dense
      // GEMMs, where only the last row tile has such waves, compute them and
      // never store them), but runs the step: it copies its share of the next
      // tiles there.
      if (jl == 0 && !kSpread) continue;
      // Straight-line step.  b[j % kNB] holds block j's fragment; reads run kNB - 1
      // blocks ahead of the MFMAs, and block j - 1 is promoted after block j's
      // MFMAs are issued.  Token blocks past the live rows are computed too
      // (their rows of the tile are zeros or stale LDS contents, which only
      // reach their own outputs, never stored): one code path keeps the
      // accumulators in registers.  Block offsets are immediates of the reads.
      const uint32_t A0 = A + ya0, A1 = A + ya1, B0 = B + xo0, B1 = B + xo1;
      v8i a[NA];
      unroll_each([&](auto ic) {
        constexpr int i = decltype(ic)::value;
        a[i] = lds_frag_at<i * 2048>(A0, A1);  // 16 weight rows = 2 KB in both tile layouts
      }, std::make_integer_sequence<int, NA>{});
      constexpr int kNB = GK_PREFILL_BBUF;
      static_assert(kNB >= 2 && kNB <= 8, "activation fragment buffers");
      v8i b[kNB];
      unroll_each([&](auto uc) {
        constexpr int u = decltype(uc)::value;
        b[u] = lds_frag_at<u * kJB>(B0, B1);
      }, std::make_integer_sequence<int, kNB - 1>{});
      unroll_each([&](auto jc) {
        constexpr int j = decltype(jc)::value;
        // Expert segments (GROUPED) often end inside a wave's rows: there the
        // blocks past the live rows are skipped (a wave-uniform branch).  Dense
        // GEMMs have at most one partial row tile and keep the branch-free step.
        const bool skip = GROUPED && j >= jl;
        if constexpr (j == 4) {
          if (!GROUPED) __builtin_amdgcn_s_setprio(0);
        }
        if (kSpread) {  // this step's tile loads, spread over the first blocks
          if (j < 4) {
            issue_a_one(min(g + 1, gend - 1), as_next, j);
          } else if (j - 4 < NA) {
            issue_w_one(min(g + 2, gend - 1), ws_free, j - 4);
          }
        }
        // block j + kNB - 1's read goes out; then block j's fragment must be in,
        // with the reads of blocks j + 1 .. min(7, j + kNB - 1) still in flight
        if (j + kNB - 1 < 8) b[(j + kNB - 1) % kNB] = lds_frag_at<(j + kNB - 1) * kJB>(B0, B1);
        constexpr int later = (kNB - 1 < 7 - j) ? kNB - 1 : 7 - j;
        if (j == 0) {  // ... and the weight fragments, read before block 0's
          asm volatile("s_waitcnt lgkmcnt(%3)" : "+v"(a[0]), "+v"(a[NA - 1]), "+v"(b[0]) : "n"(2 * later));
          if (NA == 4) asm volatile("" : "+v"(a[1]), "+v"(a[2]));
          if (NA == 3) asm volatile("" : "+v"(a[1]));
          if (HALF) {
#pragma unroll
            for (int i = 0; i < NA; ++i) a[i] = half_codes(a[i]);
          }
        } else {
          asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(b[j % kNB]) : "n"(2 * later));
        }
        if (CH) {
#pragma unroll
          for (int i = 0; i < NA; ++i) acc[i][j] = mfma_f8_acc(a[i], b[j % kNB], acc[i][j]);
        } else if (GROUPED) {
          if (!skip) {
            block_mfma(a, b[j % kNB], t[0]);
#pragma unroll
            for (int i = 0; i < NA; ++i) promote4(acc[i][j], t[0][i], svg[j] * swg[i]);
          }
        } else {
          block_mfma(a, b[j % kNB], t[j & 1]);
          if constexpr (j > 0) {
#pragma unroll
            for (int i = 0; i < NA; ++i) promote4(acc[i][j - 1], t[(j - 1) & 1][i], svg[j - 1] * swg[i]);
          } else if (g > gbeg) {
#pragma unroll
            for (int i = 0; i < NA; ++i) promote4(acc[i][7], t[1][i], pf7[i]);
          }
          // One MFMA, then the four promotion FMAs of the previous block's
          // same weight fragment: the matrix core and the VALU work side by
          // side (a microbenchmark of this mix on MI355X: 85% -> 90% of the
          // FP8 peak at two waves per SIMD).
#pragma unroll
          for (int i = 0; i < NA; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 4, 0);  // VALU
          }
        }
      }, std::make_integer_sequence<int, 8>{});
      if (!CH && !GROUPED) {
#pragma unroll
        for (int i = 0; i < NA; ++i) pf7[i] = svg[7] * swg[i];
      }
    } while (++g < gend);
    if (!CH && !GROUPED) {
#pragma unroll
      for (int i = 0; i < NA; ++i) promote4(acc[i][7], t[1][i], pf7[i]);
    }
  }

  __builtin_amdgcn_s_waitcnt(0);  // the re-read weight loads still in flight write LDS

  if (SWI) {
    // gate (waves wn = 0, 1) and up (wn = 2, 3) outputs, bf16-rounded as
    // store_tile rounds them, into LDS [2][256 rows][256 B]: 16-byte chunk c
    // of row m at slot c ^ (m & 15), so the 32 lanes of a wave's 8-byte write
    // (16 rows x 2 halves of one chunk) and the 16 lanes reading one row each
    // cover a 256-byte bank window once.  (Measured on MI355X, config 5
    // gate_up: about 1.9 K bank-conflict cycles per CU over a launch remain;
    // a padded 272-byte row layout gave more, at the same time.)  Rows past
    // the live rows are never read.
    __syncthreads();  // every wave's fragment reads are done (the tile copies: waitcnt above)
    const uint32_t hbase = static_cast<uint32_t>(wn >> 1) << 16;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < jl) {
        const int ml = mw + j * kJS + fr;
#pragma unroll
        for (int i = 0; i < NA; ++i) {
          const int c = 8 * (wn & 1) + 2 * i + (fq >> 1);
          const v4f v = acc[i][j];
          *reinterpret_cast<uint2*>(smem + hbase + ml * 256 + ((c ^ (ml & 15)) << 4) + (fq & 1) * 8) =
              make_uint2(bf16x2_rne(v[0] + 0.0f, v[1] + 0.0f), bf16x2_rne(v[2] + 0.0f, v[3] + 0.0f));
        }
      }
    }
    __syncthreads();
    // 16 lanes per live row: 8 gate and 8 up values each -> 8 bf16 products
    // -> the row's 128-column group quantized (a 16-lane set leaves together)
    const int rows = min(live, kBM), sub = tid & 15;
    for (int r = tid >> 4; r < rows; r += 32) {
      const uint32_t o = static_cast<uint32_t>(r * 256 + ((sub ^ (r & 15)) << 4));
      const uint4 gv = *reinterpret_cast<const uint4*>(smem + o);
      const uint4 uv = *reinterpret_cast<const uint4*>(smem + 65536 + o);
      const uint4 h = make_uint4(act_mul_pair<kSilu>(gv.x, uv.x), act_mul_pair<kSilu>(gv.y, uv.y),
                                 act_mul_pair<kSilu>(gv.z, uv.z), act_mul_pair<kSilu>(gv.w, uv.w));
      float s;
      const uint2 codes = quant_group8(h, true, HALF, &s);
      const int64_t slot = static_cast<int64_t>(tn) * Mpad + m0 + r;
      *reinterpret_cast<uint2*>(swq + slot * 128 + sub * 8) = codes;
      if (sub == 0) sws[slot] = s;
    }
    return;
  }

  if (CH) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < jl) {
        const int m = m0 + mw + j * kJS + fr;
        if (m < M) {
          const float sam = sa[m];
          uint16_t* row = y + static_cast<int64_t>(m) * ldy;
#pragma unroll
          for (int i = 0; i < NA; ++i) {
            const int n = n0 + wn * 16 * NA + i * 16 + 4 * fq;
#pragma unroll
            for (int r = 0; r < 4; ++r)
              if (n + r < N) row[n + r] = channel_out(acc[i][j][r], sam, sw[n + r], bias ? bias[n + r] : 0.0f);
          }
        }
      }
    }
    return;
  }
  if (yp) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if (j < jl) {
        const int m = m0 + mw + j * kJS + fr;
        if (m >= M) continue;
#pragma unroll
        for (int i = 0; i < NA; ++i) {
          const int n = n0 + wn * 16 * NA + i * 16 + 4 * fq;
          float* dst = ypp + static_cast<int64_t>(m) * ldyp + n;
          const v4f v = acc[i][j];
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
  if (!GROUPED && (reinterpret_cast<uintptr_t>(y) & 15) == 0 && (ldy & 7) == 0) {
    // Dense bf16 tile through LDS (free once every wave is past its last
    // fragment read and its own copies have landed): rows of BN * 2 bytes at
    // a stride of BN * 2 + 16, then whole-row 16-byte stores.  The fragment
    // layout would store 32-byte pieces of 16 rows per instruction; every
    // workgroup of a round stores its tile at once, so the epilogue is a
    // write burst (measured on MI355X, config 4 GEMM: -1%).  Same bits as
    // store_tile: bias added in fp32, one bf16 rounding.
    constexpr int kRS = BN * 2 + 16, kCPR = BN / 8;  // LDS row stride; 16-byte chunks per row
    static_assert(kBM * kRS <= kLdsBytes, "the staged tile fits the LDS");
    __builtin_amdgcn_s_barrier();
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int i = 0; i < NA; ++i) {
        const int nl = wn * 16 * NA + i * 16 + 4 * fq, ml = mw + j * kJS + fr;
        float b[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        if (bias) {
#pragma unroll
          for (int r = 0; r < 4; ++r) b[r] = (n0 + nl + r < N) ? bias[n0 + nl + r] : 0.0f;
        }
        const uint32_t h01 = bf16x2_rne(acc[i][j][0] + b[0], acc[i][j][1] + b[1]);
        const uint32_t h23 = bf16x2_rne(acc[i][j][2] + b[2], acc[i][j][3] + b[3]);
        *reinterpret_cast<uint2*>(smem + ml * kRS + nl * 2) = make_uint2(h01, h23);
      }
    }
    __syncthreads();
    const int rows = min(live, kBM);
#pragma unroll 4
    for (int it = tid; it < kBM * kCPR; it += 512) {
      const int r = it / kCPR, c = it - r * kCPR;
      if (r >= rows) break;
      const uint4 v = *reinterpret_cast<const uint4*>(smem + r * kRS + c * 16);
      const int n = n0 + c * 8;
      uint16_t* dst = y + static_cast<int64_t>(m0 + r) * ldy + n;
      if (n + 7 < N) {
        *reinterpret_cast<uint4*>(dst) = v;
      } else {
        const uint32_t h[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if (n + e < N) dst[e] = static_cast<uint16_t>(h[e >> 1] >> (16 * (e & 1)));
      }
    }
    return;
  }
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    if (j < jl) {
#pragma unroll
      for (int i = 0; i < NA; ++i)
        store_tile(y, ldy, bias, M, N, m0 + mw + j * kJS + fr, n0 + wn * 16 * NA + i * 16 + 4 * fq, acc[i][j]);
    }
  }
}

template <bool HALF, bool GROUPED, bool CH = false, bool WPACK = false, int NA = 4, bool SWI = false>
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
                                                              int64_t ldyp, int accum, int xcd_cus,
                                                              uint8_t* __restrict__ swq, float* __restrict__ sws) {
  prefill256_body<HALF, GROUPED, CH, WPACK, NA, SWI>(static_cast<int>(blockIdx.x), qa, sa, w, sw, bias, y, ldy, M,
                                                     N, K, G, Mpad, group_off, group_cnt, n_groups, w_stride,
                                                     sw_stride, kparts, yp, ldq, gs, ldyp, accum, xcd_cus, swq, sws);
}

// A dense GEMM in two column ranges, one launch: workgroups [0, split) take
// 256-wide tiles of columns [0, wide) and the rest 192-wide tiles of [wide, N)
// (weights, scales, bias and outputs of the second range passed offset, with
// n2 = N - wide columns).  One launch instead of two: workgroups of the second
// range start on the CUs as the first range's finish, with no launch gap and
// no idle tail between the ranges.
template <bool HALF, bool WPACK>
__global__ __launch_bounds__(512) void gemm_prefill256_split_kernel(
    int split, const uint8_t* __restrict__ qa, const float* __restrict__ sa, int64_t ldy, int M, int K, int G,
    int Mpad, int gs, int64_t ldyp, int accum, const uint8_t* __restrict__ w1, const float* __restrict__ sw1,
    const float* __restrict__ bias1, uint16_t* __restrict__ y1, float* __restrict__ yp1, int n1,
    const uint8_t* __restrict__ w2, const float* __restrict__ sw2, const float* __restrict__ bias2,
    uint16_t* __restrict__ y2, float* __restrict__ yp2, int n2) {
  const int b = static_cast<int>(blockIdx.x);
  if (b < split)
    prefill256_body<HALF, false, false, WPACK, 4>(b, qa, sa, w1, sw1, bias1, y1, ldy, M, n1, K, G, Mpad, nullptr,
                                                  nullptr, 0, 0, 0, 1, yp1, 0, gs, ldyp, accum, 0);
  else
    prefill256_body<HALF, false, false, WPACK, 3>(b - split, qa, sa, w2, sw2, bias2, y2, ldy, M, n2, K, G, Mpad,
                                                  nullptr, nullptr, 0, 0, 0, 1, yp2, 0, gs, ldyp, accum, 0);
}

// The 160 KB of dynamic LDS is above the default limit: raise it once per device.
constexpr int kMaxDevices = 64;

std::once_flag g_lds_once[kMaxDevices][40];
hipError_t g_lds_err[kMaxDevices][40];

template <bool HALF, bool GROUPED, bool CH = false, bool WPACK = false, int NA = 4, bool SWI = false>
hipError_t ensure_lds_limit() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  // slots 32..35: the split kernel; 36..39: the fused SiLU-and-mul form (grouped, NA = 4)
  constexpr int slot = SWI ? 36 + (HALF ? 1 : 0) + (WPACK ? 2 : 0)
                           : (HALF ? 1 : 0) + (GROUPED ? 2 : 0) + (CH ? 4 : 0) + (WPACK ? 8 : 0) + (NA == 3 ? 16 : 0);
  std::call_once(g_lds_once[dev][slot], [dev] {
    g_lds_err[dev][slot] = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&gemm_prefill256_kernel<HALF, GROUPED, CH, WPACK, NA, SWI>),
        hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  });
  return g_lds_err[dev][slot];
}

template <bool HALF, bool WPACK>
hipError_t ensure_lds_limit_split() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  constexpr int slot = 32 + (HALF ? 1 : 0) + (WPACK ? 2 : 0);
  std::call_once(g_lds_once[dev][slot], [dev] {
    g_lds_err[dev][slot] = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_prefill256_split_kernel<HALF, WPACK>),
                                               hipFuncAttributeMaxDynamicSharedMemorySize, kLdsBytes);
  });
  return g_lds_err[dev][slot];
}

template <bool HALF, bool WPACK>
hipError_t launch_split(const GemmArgs& a, int wide, hipStream_t stream) {
  hipError_t e = ensure_lds_limit_split<HALF, WPACK>();
  if (e != hipSuccess) return e;
  const int tiles_m = a.Mpad / kBM, n2 = a.N - wide;
  const int split = tiles_m * (wide / 256);
  const unsigned blocks = static_cast<unsigned>(split + tiles_m * ((n2 + 191) / 192));
  // Columns [wide, N): weight rows from `wide` (row-major: + wide * K bytes; packed:
  // 16-row tiles of gs * 2048 = K * 16 bytes, the same offset), scale rows from wide / 128.
  gemm_prefill256_split_kernel<HALF, WPACK><<<blocks, 512, kLdsBytes, stream>>>(
      split, a.qa, a.sa, a.ldy, a.M, a.K, a.G, a.Mpad, a.gstride(), a.ldyp, a.accumulate ? 1 : 0, a.w, a.sw, a.bias,
      a.y, a.yp, wide, a.w + static_cast<int64_t>(wide) * a.K, a.sw + static_cast<int64_t>(wide / 128) * a.gstride(),
      a.bias ? a.bias + wide : nullptr, a.y ? a.y + wide : nullptr, a.yp ? a.yp + wide : nullptr, n2);
  return hipGetLastError();
}

// Compute units of the current device (cached per device; 0 if unknown).
std::once_flag g_cu_once[kMaxDevices];
int g_cus[kMaxDevices];

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  std::call_once(g_cu_once[dev], [dev] {
    int n = 0;
    g_cus[dev] = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess ? n : 0;
  });
  return g_cus[dev];
}

template <bool HALF, bool GROUPED, bool WPACK = false, int NA = 4, bool SWI = false>
hipError_t launch256(const GemmArgs& a, const int32_t* group_off, const int32_t* group_cnt, int n_groups,
                     int64_t w_stride, int64_t sw_stride, int kparts, float* yp, int64_t ldyp, hipStream_t stream) {
  hipError_t e = ensure_lds_limit<HALF, GROUPED, false, WPACK, NA, SWI>();
  if (e != hipSuccess) return e;
  constexpr int BN = 64 * NA;
  const unsigned tiles = static_cast<unsigned>(((a.N + BN - 1) / BN) * (a.Mpad / kBM));
  // grouped: the XCD placement of one-round grids (a grid of a multiple of 8)
  const int xcd_cus = GROUPED ? device_cus() : 0;
  const unsigned grid = GROUPED ? (tiles * kparts + 7) / 8 * 8 : tiles * kparts;
  gemm_prefill256_kernel<HALF, GROUPED, false, WPACK, NA, SWI><<<grid, 512, kLdsBytes, stream>>>(
      a.qa, a.sa, a.w, a.sw, a.bias, a.y, a.ldy, a.M, a.N, a.K, a.G, a.Mpad, group_off, group_cnt, n_groups,
      w_stride, sw_stride, kparts, yp, 0, a.gstride(), ldyp, a.accumulate ? 1 : 0, xcd_cus, a.swiglu_q, a.swiglu_s);
  return hipGetLastError();
}

template <int NA>
hipError_t launch_dense(const GemmArgs& a, hipStream_t stream) {
  if (a.wpack)
    return a.half_w ? launch256<true, false, true, NA>(a, nullptr, nullptr, 0, 0, 0, 1, a.yp, a.ldyp, stream)
                    : launch256<false, false, true, NA>(a, nullptr, nullptr, 0, 0, 0, 1, a.yp, a.ldyp, stream);
  return a.half_w ? launch256<true, false, false, NA>(a, nullptr, nullptr, 0, 0, 0, 1, a.yp, a.ldyp, stream)
                  : launch256<false, false, false, NA>(a, nullptr, nullptr, 0, 0, 0, 1, a.yp, a.ldyp, stream);
}


}  // namespace

// Columns [0, n_wide) in 256-wide weight tiles and the rest in 192-wide tiles,
// when that fills the CUs better than 256-wide tiles alone: a GEMM whose
// 256 x 256 tiles need more than one round over the CUs otherwise leaves CUs
// idle in its last round (config 4: 448 tiles on 256 CUs = 1.75 rounds, run
// as 256 + 256 tiles of 256 and 192 columns).  Work is counted in rounds, a
// 192-wide tile taking 0.8 of a 256-wide one (it keeps the activation
// traffic of the full tile).  Returns N (no split) when nothing gains.
int prefill_wide_columns(int Mpad, int N, int cus) {
  const int tiles_m = Mpad / kBM;
  const int nt = (N + 255) / 256;
  if (cus <= 0 || tiles_m * nt <= cus) return N;
  auto rounds = [cus](int tiles) { return (tiles + cus - 1) / cus; };
  double best = rounds(tiles_m * nt);
  int best_wide = N;
  for (int a = 1; a < nt; ++a) {
    const int n2 = N - 256 * a;
    const double est = rounds(tiles_m * a) + 0.8 * rounds(tiles_m * ((n2 + 191) / 192)) + 0.02;
    if (est < best - 1e-9) {
      best = est;
      best_wide = 256 * a;
    }
  }
  return best_wide;
}

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
      a.ldq, a.G, 0, 0, 0, nullptr, nullptr);
  return hipGetLastError();
}

// Requires K % 128 == 0, 16-byte aligned weights, Mpad % 256 == 0 (qa/sa
// padded with zero rows up to Mpad).  Large GEMMs may run in two column
// ranges of different tile widths (prefill_wide_columns), in one launch; each
// output column is computed by one workgroup either way, with the same
// per-element arithmetic.
hipError_t launch_gemm_prefill256(const GemmArgs& a, hipStream_t stream) {
  if (a.Mpad % kBM != 0 || !prefill256_fits(a)) return hipErrorInvalidValue;
  const int wide = prefill_wide_columns(a.Mpad, a.N, device_cus());
  if (wide >= a.N) return launch_dense<4>(a, stream);
  if (a.wpack) return a.half_w ? launch_split<true, true>(a, wide, stream) : launch_split<false, true>(a, wide, stream);
  return a.half_w ? launch_split<true, false>(a, wide, stream) : launch_split<false, false>(a, wide, stream);
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
  if (a.swiglu_q) {
    // the fused SiLU-and-mul form: gate | up halves of 128-row multiples, one K part, codes out
    if (!a.swiglu_s || kparts != 1 || yp || a.N % 256) return hipErrorInvalidValue;
    if (a.wpack)
      return a.half_w ? launch256<true, true, true, 4, true>(a, group_off, group_cnt, n_groups, w_stride, sw_stride,
                                                             1, nullptr, 0, stream)
                      : launch256<false, true, true, 4, true>(a, group_off, group_cnt, n_groups, w_stride,
                                                              sw_stride, 1, nullptr, 0, stream);
    return a.half_w ? launch256<true, true, false, 4, true>(a, group_off, group_cnt, n_groups, w_stride, sw_stride, 1,
                                                            nullptr, 0, stream)
                    : launch256<false, true, false, 4, true>(a, group_off, group_cnt, n_groups, w_stride, sw_stride,
                                                             1, nullptr, 0, stream);
  }
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
