// The 128 x 128-tile schedule with the per-tensor epilogue, for every
// operand-format pair (fp4 x fp4 and fp6 x fp6 included).
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

template <bool kVec, int kFmt>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_t128(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[CfgT128::kLdsBytes];
  gemm_t128_body<kVec, false, kFmt>(g, (lds_u8*)lds);
}

// K-slices: the partial tiles, summed by the last slice to arrive at each
// quadrant (g.split.arrivals, per-tensor epilogue, kVec: 16-byte C stores)
// or by the reduce kernel (one wave per workgroup) with either epilogue.
template <bool kVec, int kFmt>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_t128_split(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[CfgT128::kLdsBytes];
  gemm_t128_body<kVec, false, kFmt, kActNone, kOutBf16, true>(g, (lds_u8*)lds);
}

template <bool kVec8, bool kExt>
__global__ __launch_bounds__(64) void k_fp8_gemm_t128_reduce(GemmArgs g) {
  gemm_t128_reduce_body<kVec8, kExt>(g);
}

}  // namespace

const void* tile128_split(const Key& k) {
  return sel_fmt_t128(k.fmt, [&](auto F) {
    return sel2(k.vec, [&](auto V) {
      return (const void*)&k_fp8_gemm_t128_split<decltype(V)::value == 1,
                                                 decltype(F)::value>;
    });
  });
}

const void* tile128_reduce(const Key& k) {
  return sel2(k.ext, [&](auto E) {
    return sel2(k.vec, [&](auto V) {
      return (const void*)&k_fp8_gemm_t128_reduce<decltype(V)::value == 1,
                                                 decltype(E)::value == 1>;
    });
  });
}

const void* tile128_plain(const Key& k) {
  return sel_fmt_t128(k.fmt, [&](auto F) {
    return sel2(k.vec, [&](auto V) {
      return (const void*)&k_fp8_gemm_t128<decltype(V)::value == 1, decltype(F)::value>;
    });
  });
}

}  // namespace kernels
}  // namespace hipgemm
