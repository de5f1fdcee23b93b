// The 4-wave schedule with the per-tensor epilogue: 16x16x128 for every
// operand-format pair (fp6 included), 32x32x64 for e4m3 x e4m3.
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

template <bool kVec, int kMf, int kFmt, bool kLine = false>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_4wave(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg4w::kLdsBytes];
  gemm_4wave_body<kVec, kMf, false, kFmt, kActNone, kOutBf16, false, kLine>(
      g, (lds_u8*)lds);
}

}  // namespace

const void* four_wave_plain(int mf, const Key& k) {
  if (mf == 32) {
    if (k.fmt != 0) return nullptr;
    return k.vec ? (const void*)&k_fp8_gemm_4wave<true, 32, 0>
                 : (const void*)&k_fp8_gemm_4wave<false, 32, 0>;
  }
  // Line-aligned rows of C with 16-byte stores: the overlapped epilogue
  // (8-bit pairs and fp4 x fp4).
  if (k.vec && k.line && k.fmt <= kFmtPairFp4)
    return sel_fmt(k.fmt, [&](auto F) {
      return (const void*)&k_fp8_gemm_4wave<true, 16, decltype(F)::value, true>;
    });
  // The 8-bit pairs, fp4 x fp4 (kFmtPairFp4) and fp6 x fp6
  // (kFmtPairFp6 + 0..3).
  return sel_fmt_t128(k.fmt, [&](auto F) {
    return sel2(k.vec, [&](auto V) {
      return (const void*)&k_fp8_gemm_4wave<decltype(V)::value == 1, 16, decltype(F)::value>;
    });
  });
}

}  // namespace kernels
}  // namespace hipgemm
