// AUTO's column split of C (hipgemm_split_columns) as one persistent launch:
// every workgroup runs its tiles of columns [0, n1) on the 4-wave 16x16x128
// schedule, then its tiles of [n1, N) on the 128 x 128 one.  Per-tensor
// epilogue with 16-byte stores on both parts, 8-bit operand pairs.
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

static_assert(Cfg4w::kLdsBytes >= CfgT128::kLdsBytes, "one LDS array for both parts");
static_assert(Cfg4w::kThreads == CfgT128::kThreads, "one workgroup shape");

template <int kFmt, bool kLine>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_split(GemmArgs g4, GemmArgs g1) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg4w::kLdsBytes];
  gemm_4wave_body<true, 16, false, kFmt, kActNone, kOutBf16, false, kLine>(
      g4, (lds_u8*)lds);
  // The 4-wave part has waited for its own DMAs; its waves may still read
  // their epilogue stages.
  __syncthreads();
  gemm_t128_body<true, false, kFmt>(g1, (lds_u8*)lds);
}

}  // namespace

const void* split_plain(const Key& k) {
  return sel4(k.fmt, [&](auto F) {
    return sel2(k.line, [&](auto L) {
      return (const void*)&k_fp8_gemm_split<decltype(F)::value,
                                            decltype(L)::value == 1>;
    });
  });
}

}  // namespace kernels
}  // namespace hipgemm
