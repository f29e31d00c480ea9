// Decode-variant shape planning: plain C++ (no HIP), shared by the kernels'
// dispatch (gk_fp8_gemm.hip), the C-ABI layer (gk_fp8_abi.hip) and a host test
// that checks every planned shape against the instantiated list.
#pragma once

namespace gk {

// Decode variant shape: NW waves per workgroup (splitting K), R 16-row weight
// tiles per workgroup, U groups per load step, MT 16-token column tiles.
struct DecodeShape {
  int nw, r, u, mt;
};

// Instantiated decode shapes (NW, R, U, MT).  GK_DECODE_SHAPES1: the
// per-channel decode (plan_decode_shape at MT = 1, no step fitting);
// GK_DECODE_SHAPES_T1: every MT = 1 shape (fit_group_step and
// fused_quant_shape halve U); GK_DECODE_SHAPES: all, including MT = 2, 4.
#define GK_DECODE_SHAPES1(X) X(2, 2, 4, 1) X(8, 2, 2, 1) X(8, 2, 4, 1) X(8, 1, 2, 1) X(16, 1, 2, 1)
#define GK_DECODE_SHAPES_T1(X) GK_DECODE_SHAPES1(X) \
  X(2, 2, 2, 1) X(2, 2, 1, 1) X(8, 2, 1, 1) X(8, 1, 1, 1) X(16, 1, 1, 1)
#define GK_DECODE_SHAPES(X) GK_DECODE_SHAPES_T1(X)                                             \
  X(2, 2, 2, 2) X(2, 2, 1, 2) X(8, 2, 1, 2) X(8, 2, 2, 2) X(8, 1, 1, 2) X(16, 1, 1, 2)         \
  X(2, 2, 1, 4) X(8, 2, 1, 4) X(8, 1, 1, 4) X(16, 1, 1, 4)

constexpr int decode_key(int nw, int r, int u, int mt) { return ((nw * 10 + r) * 10 + u) * 10 + mt; }

// Membership in the three lists above (list 1, T1 or all).
inline bool decode_shape_listed(const DecodeShape& d, int list) {
  const int key = decode_key(d.nw, d.r, d.u, d.mt);
  int n = 0;
  int keys[32];
#define GK_KEY(NW, R, U, MT) keys[n++] = decode_key(NW, R, U, MT);
  if (list == 1) {
    GK_DECODE_SHAPES1(GK_KEY)
  } else if (list == 2) {
    GK_DECODE_SHAPES_T1(GK_KEY)
  } else {
    GK_DECODE_SHAPES(GK_KEY)
  }
#undef GK_KEY
  for (int i = 0; i < n; ++i)
    if (keys[i] == key) return true;
  return false;
}

inline DecodeShape plan_decode_shape(int N, int G, bool packed_weights, int mt) {
  // R: 16-row tiles per workgroup.  Every workgroup reads the activations of
  // its K range once, so larger R cuts activation traffic, but the workgroup
  // count (tiles / R) must stay near or above the 256 CUs.  NW: waves
  // splitting K (the partials are summed in wave order, so NW fixes the
  // result bits; both weight layouts use the same NW for every N and give
  // identical results).  U: groups per load step, divided by the token tiles
  // mt (each group's activation fragments grow with mt).  Measured on MI355X
  // at M = 16 for N x K = 28672 x 4096, 6144 x 4096, 4096 x 14336; the packed
  // layout (no LDS transpose) gains from the deeper step at N = 6144.
  (void)G;
  const int tiles = (N + 15) / 16;
  DecodeShape d;
  if (tiles >= 1536) d = DecodeShape{2, 2, 4, 1};
  else if (tiles >= 384) d = packed_weights ? DecodeShape{8, 2, 4, 1} : DecodeShape{8, 2, 2, 1};
  else if (tiles >= 256) d = DecodeShape{8, 1, 2, 1};
  else d = DecodeShape{16, 1, 2, 1};
  d.mt = mt;
  d.u = d.u / mt > 0 ? d.u / mt : 1;
  return d;
}

inline DecodeShape fit_group_step(DecodeShape d, int G) {
  // A wave's last load step is padded with repeats of its last group (loaded
  // again, multiplied, and scaled by zero), so U is halved until it divides
  // every wave's group count (G/NW rounded either way).  Measured on MI355X:
  // 7168 x 7168 (7 groups a wave) 10.9 -> 10.0 us at M = 16 with U = 1,
  // 8192 x 2048 (2 a wave) 6.5 -> 5.0 us with U = 2.  NW, and so the result
  // bits, is unchanged.
  const int lo = G / d.nw, hi = (G + d.nw - 1) / d.nw;
  while (d.u > 1 && (lo == 0 || lo % d.u != 0 || hi % d.u != 0)) d.u /= 2;
  return d;
}

inline DecodeShape fused_quant_shape(DecodeShape d, int G) {
  // With the quantizer fused, a load step also quantizes its U groups, and a
  // padded step repeats that work for nothing.  U divides every wave's group
  // count: 4 only where each wave has exactly 4 groups, else 2 where both
  // counts are even, else 1.  More, shorter steps also keep the quantizer's
  // arithmetic beside the weight fetch.  Measured on MI355X at M = 1, 8, 16
  // for nine N x K shapes; NW (and so the result bits) is unchanged.
  const int lo = G / d.nw, hi = (G + d.nw - 1) / d.nw;
  d.u = (lo == 4 && hi == 4 && d.u == 4) ? 4 : (lo % 2 == 0 && hi % 2 == 0 && lo > 0) ? 2 : 1;
  return d;
}

// Dense 256 x 256 GEMM tile order (gk_fp8_prefill.hip).  Workgroup bid of a
// launch (or column range) of tiles_m x tiles_nn tiles and kparts K parts runs
// on XCD bid % 8 of the GPU.  With a multiple of 8 tiles and one K part, XCD
// x takes the x-th eighth of the tiles in super-block order: 4 weight panels
// (tn) by all row tiles (tm), row tile by row tile -- so the CUs of one XCD
// share few weight panels and activation row tiles in its L2.  Returns
// tn * 65536 + tm; a bijection on the tiles for every grid (plan_check.cpp).
// constexpr: callable from device code.
constexpr int dense_tile_of(int bid, int tiles_m, int tiles_nn, int kparts) {
  const int tiles = tiles_m * tiles_nn;
  const int l = (tiles % 8 == 0 && kparts == 1) ? (bid % 8) * (tiles / 8) + bid / 8 : bid;
  const int sb = l / (4 * tiles_m);
  const int left = tiles_nn - sb * 4;
  const int wsb = left < 4 ? left : 4;
  const int rem = l - sb * 4 * tiles_m;
  return (sb * 4 + rem % wsb) * 65536 + rem / wsb;
}

}  // namespace gk
