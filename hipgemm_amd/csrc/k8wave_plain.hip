// The 8-wave ping-pong schedule with the per-tensor epilogue, for every
// operand-format pair.
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

template <bool kVec, int kFmt>
__global__ __launch_bounds__(512, 1) void k_fp8_gemm_8wave(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg8w::kLdsBytes];
  gemm_8wave_body<kVec, false, kFmt>(g, (lds_u8*)lds);
}

}  // namespace

const void* eight_wave_plain(const Key& k) {
  return sel4(k.fmt, [&](auto F) {
    return sel2(k.vec, [&](auto V) {
      return (const void*)&k_fp8_gemm_8wave<decltype(V)::value == 1, decltype(F)::value>;
    });
  });
}

}  // namespace kernels
}  // namespace hipgemm
