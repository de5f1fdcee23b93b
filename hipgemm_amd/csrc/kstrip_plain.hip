// The column-strip skinny schedule (M <= 128) with the per-tensor epilogue, for every
// row-block count, strip width and operand-format pair.
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

template <int kMB, int kNB, bool kVec8, int kFmt>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_strip_plain(StripArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[CfgStrip::lds_bytes(kMB, kNB)];
  gemm_strip_body<kMB, kNB, kVec8, false, kFmt>(g, (lds_u8*)lds);
}

template <class F>
const void* sel_mb(int kmb, F&& f) {
  switch (kmb) {
    case 1: return f(ic<1>{});
    case 2: return f(ic<2>{});
    case 3: return f(ic<3>{});
    case 4: return f(ic<4>{});
    case 8: return f(ic<8>{});
    default: return nullptr;
  }
}

}  // namespace

const void* strip_plain(int kmb, int knb, const Key& k) {
  if (knb != 2 && knb != 4) return nullptr;
  return sel_mb(kmb, [&](auto B) {
    return sel2(knb == 4, [&](auto W) {
      return sel4(k.fmt, [&](auto F) {
        return sel2(k.vec, [&](auto V) {
          return (const void*)&k_fp8_gemm_strip_plain<decltype(B)::value,
                                                     decltype(W)::value ? 4 : 2,
                                                     decltype(V)::value == 1,
                                                     decltype(F)::value>;
        });
      });
    });
  });
}

}  // namespace kernels
}  // namespace hipgemm
