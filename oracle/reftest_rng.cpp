/*
 * hipgemm oracle -- reference-test input mode.  TEST INFRASTRUCTURE ONLY.
 *
 * Restates init_random (utils.hpp:27-34): a std::mt19937 seeded with `seed`
 * drives std::normal_distribution<float>(-1.0f, 1.0f) (mean -1, sigma 1), and
 * each draw is cast to e4m3 with the HIP constructor's rounding (RNE,
 * satfinite), here hg_f32_to_e4m3.  The random stream itself is the C++
 * standard library's (libstdc++), not reference code, so this file is C++.
 * Pinned bit-exactly against init_random compiled from the reference sources
 * (oracle/_ref) in tests/test_oracle.py.
 */
#include <random>

#include "oracle.h"

extern "C" void hg_fill_e4m3_reftest(uint8_t *out, size_t n, uint64_t seed) {
  std::mt19937 gen(static_cast<std::mt19937::result_type>(seed));
  std::normal_distribution<float> dis(-1.0f, 1.0f);
  for (size_t i = 0; i < n; ++i) out[i] = hg_f32_to_e4m3(dis(gen));
}
