// The split-K skinny schedule (M <= 128) with the per-tensor epilogue, for
// every row-block count and operand-format pair, and the slice-reduce
// kernel for both epilogues.
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

template <int kMB, bool kVec8, int kFmt, int kF>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_skinny(SkinnyArgs g) {
  gemm_skinny_body<kMB, kVec8, false, kFmt, kF>(g);
}

template <bool kVec8, bool kExt, int kF>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_skinny_reduce(SkinnyArgs g,
                                                                    int kmb) {
  gemm_skinny_reduce_body<kVec8, kExt, kF>(g, kmb);
}

// (row blocks, B_T fragments per wave) pairs the plan uses: 4 fragments up
// to 32 rows, 2 above, and 1 as well from 65 rows.
template <class F>
const void* sel_mb(int kmb, int kf, F&& f) {
  switch (kmb * 8 + kf) {
    case 1 * 8 + 4: return f(ic<1>{}, ic<4>{});
    case 2 * 8 + 4: return f(ic<2>{}, ic<4>{});
    case 4 * 8 + 2: return f(ic<4>{}, ic<2>{});
    case 8 * 8 + 2: return f(ic<8>{}, ic<2>{});
    case 8 * 8 + 1: return f(ic<8>{}, ic<1>{});
    default: return nullptr;
  }
}

}  // namespace

const void* skinny_plain(int kmb, int kf, const Key& k) {
  return sel_mb(kmb, kf, [&](auto B, auto KF) {
    return sel4(k.fmt, [&](auto F) {
      return sel2(k.vec, [&](auto V) {
        return (const void*)&k_fp8_gemm_skinny<decltype(B)::value, decltype(V)::value == 1,
                                     decltype(F)::value, decltype(KF)::value>;
      });
    });
  });
}

const void* skinny_reduce(int kf, const Key& k) {
  return sel2(k.ext, [&](auto E) {
    return sel2(k.vec, [&](auto V) {
      if (kf == 2)
        return (const void*)&k_fp8_gemm_skinny_reduce<decltype(V)::value == 1,
                                                      decltype(E)::value == 1, 2>;
      if (kf == 4)
        return (const void*)&k_fp8_gemm_skinny_reduce<decltype(V)::value == 1,
                                                      decltype(E)::value == 1, 4>;
      if (kf == 1)
        return (const void*)&k_fp8_gemm_skinny_reduce<decltype(V)::value == 1,
                                                      decltype(E)::value == 1, 1>;
      return (const void*)nullptr;
    });
  });
}

}  // namespace kernels
}  // namespace hipgemm
