// Activation inputs of the reference's five 1K FP16 GEMM cases
// (tests/fp8_hybrid_tpcsim_test.cpp:187-201, cases :388-392): std::mt19937 seeded
// with k*13 + m*7 + n + (bias ? 99 : 0), std::normal_distribution<float>(0, 1), rows
// and groups in order, row 1 and group (0, 0) left zero (not tiny), envelope 12 or
// 1.5 by (g/2)%4 (tiny: 1e-12 / 1e-15 by g parity), bf16 round-to-nearest-even.
// Usage: hybrid_x m n k bias tiny > x.bin   (m*k little-endian uint16 bf16 bits)
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

static uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

int main(int argc, char** argv) {
  if (argc != 6) return 2;
  const uint64_t m = std::strtoull(argv[1], nullptr, 10), n = std::strtoull(argv[2], nullptr, 10);
  const uint64_t k = std::strtoull(argv[3], nullptr, 10);
  const bool bias = std::atoi(argv[4]) != 0, tiny = std::atoi(argv[5]) != 0;
  std::mt19937 rng(static_cast<uint32_t>(k * 13 + m * 7 + n + (bias ? 99 : 0)));
  std::normal_distribution<float> norm(0.0f, 1.0f);
  std::vector<uint16_t> x(m * k, 0);
  for (uint64_t r = 0; r < m; ++r) {
    if (!tiny && r == 1) continue;
    for (uint64_t g = 0; g < k / 128; ++g) {
      if (!tiny && r == 0 && g == 0) continue;
      const float env = tiny ? ((g & 1) ? 1.0e-15f : 1.0e-12f) : (((g / 2) % 4 == 0) ? 12.0f : 1.5f);
      for (uint64_t i = 0; i < 128; ++i) x[r * k + g * 128 + i] = to_bf16(norm(rng) * env);
    }
  }
  std::fwrite(x.data(), 2, x.size(), stdout);
  return 0;
}
