// The split-K skinny schedule with the extended epilogue (activation and
// output type chosen at run time: its epilogue is small), for every
// row-block count and operand-format pair.
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

template <int kMB, bool kVec8, int kFmt, int kF>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_skinny_ext(SkinnyArgs g) {
  gemm_skinny_body<kMB, kVec8, true, kFmt, kF>(g);
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

const void* skinny_ext(int kmb, int kf, const Key& k) {
  return sel_mb(kmb, kf, [&](auto B, auto KF) {
    return sel4(k.fmt, [&](auto F) {
      return sel2(k.vec, [&](auto V) {
        return (const void*)&k_fp8_gemm_skinny_ext<decltype(B)::value, decltype(V)::value == 1,
                                     decltype(F)::value, decltype(KF)::value>;
      });
    });
  });
}

}  // namespace kernels
}  // namespace hipgemm
