// The 4-wave 16x16x128 schedule with the extended epilogue and bf16 output,
// for every operand-format pair and activation.
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

template <bool kVec, int kFmt, int kAct>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_4wave_ext(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg4w::kLdsBytes];
  gemm_4wave_body<kVec, 16, true, kFmt, kAct, kOutBf16>(g, (lds_u8*)lds);
}

}  // namespace

const void* four_wave_ext_bf16(const Key& k) {
  return sel_fmt_t128(k.fmt, [&](auto F) {  // 8-bit pairs, fp4 x fp4, fp6 x fp6
    return sel4(k.act, [&](auto A) {
      return sel2(k.vec, [&](auto V) {
        return (const void*)&k_fp8_gemm_4wave_ext<decltype(V)::value == 1,
                                                  decltype(F)::value,
                                                  decltype(A)::value>;
      });
    });
  });
}

}  // namespace kernels
}  // namespace hipgemm
