// The 128 x 128-tile schedule with the extended epilogue and a 2-byte output
// (bf16, fp16), for every operand-format pair (fp4 x fp4 included) and
// activation.
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

template <bool kVec, int kFmt, int kAct, int kOut>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_t128_ext(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[CfgT128::kLdsBytes];
  gemm_t128_body<kVec, true, kFmt, kAct, kOut>(g, (lds_u8*)lds);
}

}  // namespace

const void* tile128_ext_narrow(const Key& k) {
  return sel_fmt_t128(k.fmt, [&](auto F) {
    return sel4(k.act, [&](auto A) {
      return sel2(k.out, [&](auto O) {
        return sel2(k.vec, [&](auto V) {
          return (const void*)&k_fp8_gemm_t128_ext<
              decltype(V)::value == 1, decltype(F)::value, decltype(A)::value,
              decltype(O)::value>;
        });
      });
    });
  });
}

}  // namespace kernels
}  // namespace hipgemm
