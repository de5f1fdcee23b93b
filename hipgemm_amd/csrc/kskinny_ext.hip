// The split-K skinny schedule with the extended epilogue (activation and
// output type chosen at run time: its epilogue is small), for every
// row-block count and operand-format pair.
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

template <int kMB, bool kVec8, int kFmt>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_skinny_ext(SkinnyArgs g) {
  gemm_skinny_body<kMB, kVec8, true, kFmt>(g);
}

template <class F>
const void* sel_mb(int kmb, F&& f) {
  switch (kmb) {
    case 1: return f(ic<1>{});
    case 2: return f(ic<2>{});
    case 4: return f(ic<4>{});
    case 8: return f(ic<8>{});
    default: return nullptr;
  }
}

}  // namespace

const void* skinny_ext(int kmb, const Key& k) {
  return sel_mb(kmb, [&](auto B) {
    return sel4(k.fmt, [&](auto F) {
      return sel2(k.vec, [&](auto V) {
        return (const void*)&k_fp8_gemm_skinny_ext<decltype(B)::value, decltype(V)::value == 1, decltype(F)::value>;
      });
    });
  });
}

}  // namespace kernels
}  // namespace hipgemm
