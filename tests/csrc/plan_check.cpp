// Host check of the decode-variant planner (gaudi-kernels_amd/csrc/gk_fp8_plan.h):
// every shape the C-ABI layer can plan must be one the kernels instantiate.
// Prints each planned shape that is missing from its list and exits nonzero
// if there is one.  Built and run by tests/test_plan_host.py with g++.
#include <cstdio>
#include <initializer_list>

#include "gk_fp8_plan.h"

int main() {
  using gk::DecodeShape;
  // N across every tier boundary of plan_decode_shape (tiles = ceil(N/16)).
  const int ns[] = {1, 16, 17, 128, 2048, 4080, 4095, 4096, 4097, 6144, 6145, 7168, 14336, 24560, 24575,
                    24576, 24577, 28672, 57344, 131072};
  int bad = 0, checked = 0;
  auto check = [&](const DecodeShape& d, int list, const char* path, int n, int g, int mt, int packed) {
    ++checked;
    if (!gk::decode_shape_listed(d, list)) {
      ++bad;
      std::printf("%s: N=%d G=%d mt=%d packed=%d -> (%d,%d,%d,%d) not instantiated\n", path, n, g, mt, packed,
                  d.nw, d.r, d.u, d.mt);
    }
  };
  for (int n : ns)
    for (int g = 1; g <= 256; ++g) {
      for (int mt : {1, 2, 4})
        for (int packed = 0; packed < 2; ++packed) {
          // gk_fp8_block_gemm_bf16 / _q_bf16: make_plan's decode shape
          const DecodeShape d = gk::fit_group_step(gk::plan_decode_shape(n, g, packed != 0, mt), g);
          check(d, 3, "block gemm", n, g, mt, packed);
          // the fused-quantizer form (one token tile)
          if (mt == 1) check(gk::fused_quant_shape(d, g), 3, "block gemm, fused quantizer", n, g, mt, packed);
        }
      // per-channel decode and its fused per-token form (row-major weights, one token tile)
      check(gk::plan_decode_shape(n, g, false, 1), 1, "channel gemm", n, g, 1, 0);
      check(gk::fused_quant_shape(gk::fit_group_step(gk::plan_decode_shape(n, g, false, 1), g), g), 2,
            "token-channel gemm", n, g, 1, 0);
    }
  std::printf("checked %d planned shapes, %d missing\n", checked, bad);
  // dense_tile_of: every tile of every grid exactly once
  int orders = 0, bad_orders = 0;
  static bool seen[64 * 96];
  for (int tiles_m = 1; tiles_m <= 64; ++tiles_m)
    for (int tiles_nn = 1; tiles_nn <= 96; ++tiles_nn) {
      const int tiles = tiles_m * tiles_nn;
      for (int i = 0; i < tiles; ++i) seen[i] = false;
      bool ok = true;
      for (int b = 0; b < tiles && ok; ++b) {
        const int v = gk::dense_tile_of(b, tiles_m, tiles_nn, 1);
        const int tn = v >> 16, tm = v & 0xffff;
        if (tn < 0 || tn >= tiles_nn || tm < 0 || tm >= tiles_m || seen[tn * tiles_m + tm]) ok = false;
        else seen[tn * tiles_m + tm] = true;
      }
      ++orders;
      if (!ok) {
        ++bad_orders;
        std::printf("dense_tile_of: tiles_m=%d tiles_nn=%d is not a bijection\n", tiles_m, tiles_nn);
      }
    }
  std::printf("checked %d tile orders, %d not bijective\n", orders, bad_orders);
  return (bad || bad_orders) ? 1 : 0;
}
