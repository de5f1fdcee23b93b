/*
 * hipgemm oracle pin -- TEST INFRASTRUCTURE ONLY.
 *
 * Exhaustive comparison of the oracle's element codecs against the HIP
 * headers' host conversions, which are what the reference calls:
 *   fp8(x)         utils.hpp:32  -> __hip_fp8_e4m3(float)  (amd_hip_fp8.h)
 *   float(fp8)     test.cpp:25   -> __hip_fp8_e4m3::operator float
 *   bf16(acc)      test.cpp:27   -> __hip_bfloat16(float)  (amd_hip_bf16.h)
 * Built host-only (no device code) by oracle/Makefile.
 */
#include <hip/hip_bfloat16.h>
#include <hip/hip_fp8.h>

#include <cmath>
#include <cstdint>
#include <cstring>

#include "oracle.h"

extern "C" uint8_t hg_pin_hip_f32_to_e4m3(float x) {
  __hip_fp8_e4m3 v(x);
  return static_cast<uint8_t>(v.__x);
}

extern "C" float hg_pin_hip_e4m3_to_f32(uint8_t b) {
  __hip_fp8_e4m3 v;
  v.__x = b;
  return static_cast<float>(v);
}

extern "C" uint16_t hg_pin_hip_f32_to_bf16(float x) {
  __hip_bfloat16 v(x);
  uint16_t r;
  std::memcpy(&r, &v, 2);
  return r;
}

/* Sweep fp32 bit patterns [lo, hi) (hi <= 2^32).  Returns the number of
 * mismatches and writes up to `cap` mismatching inputs to `bad`.
 * what = 0: f32 -> e4m3 (exact byte compare)
 * what = 1: f32 -> bf16 (exact compare; NaNs must map to NaNs)
 * The HIP fp8 routine shifts by more than 63 bits (undefined in C++) for
 * inputs below 2^-69, so those are compared against the exact answer (signed
 * zero) instead and counted separately through `n_tiny`. */
extern "C" uint64_t hg_pin_sweep(int what, uint64_t lo, uint64_t hi,
                                 uint32_t *bad, uint64_t cap,
                                 uint64_t *n_tiny) {
  uint64_t nbad = 0, tiny = 0, nlist = 0;
#pragma omp parallel for schedule(static, 1 << 16) reduction(+ : nbad, tiny)
  for (uint64_t i = lo; i < hi; ++i) {
    const uint32_t u = static_cast<uint32_t>(i);
    float x;
    std::memcpy(&x, &u, 4);
    bool ok;
    if (what == 0) {
      const uint8_t mine = hg_f32_to_e4m3(x);
      if ((u & 0x7fffffffu) < 0x1d000000u) { /* |x| < 2^-69 */
        ++tiny;
        ok = mine == ((u >> 24) & 0x80);
      } else {
        ok = mine == hg_pin_hip_f32_to_e4m3(x);
      }
    } else {
      const uint16_t mine = hg_f32_to_bf16(x), ref = hg_pin_hip_f32_to_bf16(x);
      if (std::isnan(x))
        ok = (mine & 0x7fff) > 0x7f80 && (ref & 0x7fff) > 0x7f80;
      else
        ok = mine == ref;
    }
    if (!ok) {
      ++nbad;
      uint64_t slot;
#pragma omp atomic capture
      slot = nlist++;
      if (slot < cap) bad[slot] = u;
    }
  }
  if (n_tiny) *n_tiny = tiny;
  return nbad;
}
