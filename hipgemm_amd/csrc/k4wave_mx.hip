// The schedules with MX block scales (per-tensor epilogue): the 4-wave
// 16x16x128 one and the 128 x 128 one, and the scale-packing kernel.
#include "kernels.hpp"

namespace hipgemm {
namespace kernels {
namespace {

using namespace detail;

template <bool kVec, int kFmt>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_4wave_mx(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg4w::kLdsBytes];
  gemm_4wave_body<kVec, 16, false, kFmt, kActNone, kOutBf16, true>(g, (lds_u8*)lds);
}

// The 128 x 128 schedule with MX block scales (per-tensor epilogue), for
// every operand-format pair including fp4 x fp4; whole K and K-slices.
template <bool kVec, int kFmt>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_t128_mx(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[CfgT128::kLdsBytes];
  gemm_t128_body<kVec, false, kFmt, kActNone, kOutBf16, false, true>(g, (lds_u8*)lds);
}
template <int kFmt>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_t128_split_mx(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[CfgT128::kLdsBytes];
  gemm_t128_body<true, false, kFmt, kActNone, kOutBf16, true, true>(g, (lds_u8*)lds);
}

// One thread per packed byte (layout of MxArgs): byte f of step st of lane l
// in (W, p) is the scale of row 128 W + 16 f + l % 16, K-block
// 4 (2 p + st) + l / 16; 127 (1.0) past the rows or blocks of the source.
__global__ __launch_bounds__(256) void k_mx_pack(const uint8_t* src, int rows,
                                                 int kblocks, int ld, int pairs,
                                                 uint8_t* dst, size_t n) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int f = (int)(i & 7), st = (int)((i >> 3) & 1), l = (int)((i >> 4) & 63);
  const size_t wp = i >> 10;
  const int p = (int)(wp % pairs), W = (int)(wp / pairs);
  const int row = 128 * W + 16 * f + (l & 15);
  const int blk = 4 * (2 * p + st) + (l >> 4);
  dst[i] = (row < rows && blk < kblocks) ? src[(size_t)row * ld + blk] : 127;
}

}  // namespace

const void* four_wave_mx(const Key& k) {
  // The 8-bit pairs and fp4 x fp4 (MXFP4).
  return sel_fmt(k.fmt, [&](auto F) {
    return sel2(k.vec, [&](auto V) {
      return (const void*)&k_fp8_gemm_4wave_mx<decltype(V)::value == 1,
                                               decltype(F)::value>;
    });
  });
}

const void* tile128_mx(const Key& k) {
  return sel_fmt(k.fmt, [&](auto F) {
    return sel2(k.vec, [&](auto V) {
      return (const void*)&k_fp8_gemm_t128_mx<decltype(V)::value == 1,
                                              decltype(F)::value>;
    });
  });
}

const void* tile128_split_mx(const Key& k) {
  return sel_fmt(k.fmt, [&](auto F) {
    return (const void*)&k_fp8_gemm_t128_split_mx<decltype(F)::value>;
  });
}

hipError_t mx_pack(const uint8_t* src, int rows, int K, int ld, uint8_t* dst,
                   hipStream_t stream) {
  const size_t n = mx_packed_bytes(rows, K);
  if (n == 0) return hipSuccess;
  int kblocks = (K + 31) / 32, pairs = mx_pairs(K);
  void* args[] = {&src, &rows, &kblocks, &ld, &pairs, &dst, const_cast<size_t*>(&n)};
  return hipLaunchKernel((const void*)&k_mx_pack, dim3((unsigned)((n + 255) / 256)),
                         dim3(256), args, 0, stream);
}

}  // namespace kernels
}  // namespace hipgemm
