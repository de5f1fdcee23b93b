// hipgemm -- drop-in C++ launch surface for the FP8 GEMM.
//
// Replaces the reference header fp8_4wave.hpp (nirw4nna/hipgemm) for its
// callers:
//   * global aliases `fp8` = __hip_fp8_e4m3 and `bf16` = __hip_bfloat16,
//     which the reference callers use unqualified (fp8_4wave.hpp:15-16,
//     test.cpp:19, utils.hpp:28);
//   * the kernel template
//       template <int M, int N, int K> __global__ __launch_bounds__(256, 1)
//       void fp8_gemm_4wave_256x256x128(const fp8*, const fp8*, bf16*)
//     with the reference's name, template parameters and pointer signature
//     (fp8_4wave.hpp:334-338), launched exactly as the callers do:
//       <<<(M * N) / (256 * 256), 256>>>      (test.cpp:79, bench.cpp:55/78)
//     C = A . B_T^T with A M x K row-major, B_T N x K row-major (K
//     contiguous), C M x N row-major bf16, fp32 accumulation;
//   * its sibling fp8_gemm_4wave_256x256x128_ref with the same signature
//     (fp8_4wave.hpp:594-598), launched the same way.
//
// Behavioural differences, all on inputs where the reference is wrong or
// undefined: any grid size >= 1 is correct (the first min(grid, 256)
// workgroups loop over the 256 x 256 tiles, the rest return at once), M and
// N need not be multiples of 256, and K only needs to be a multiple of 16
// (16-byte rows for the vector loads).  Output rounding is
// round-to-nearest-even (the reference kernel truncates, fp8_4wave.hpp:214;
// the reference's CPU check rounds to nearest even, test.cpp:27).
//
// Runtime shapes, leading dimensions, per-tensor scales, streams and the
// other schedules are in the C ABI, include/hipgemm.h.
#pragma once

#include <hip/hip_bfloat16.h>
#include <hip/hip_fp8.h>
#include <hip/hip_runtime.h>

#include "detail/gemm_4wave.hpp"

using fp8 = __hip_fp8_e4m3;
using bf16 = __hip_bfloat16;

static_assert(sizeof(fp8) == 1, "fp8 must be one byte");
static_assert(sizeof(bf16) == 2, "bf16 must be two bytes");

template <int M, int N, int K>
__global__ __launch_bounds__(256, 1) void fp8_gemm_4wave_256x256x128(
    const fp8* __restrict A, const fp8* __restrict B_T, bf16* __restrict C) {
  static_assert(M > 0 && N > 0 && K > 0, "shape must be positive");
  static_assert(K % 16 == 0, "K must be a multiple of 16 (16-byte rows)");
  using namespace hipgemm::detail;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg4w::kLdsBytes];
  constexpr int tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
  const GemmArgs args{reinterpret_cast<const uint8_t*>(A),
                      reinterpret_cast<const uint8_t*>(B_T),
                      reinterpret_cast<uint16_t*>(C),
                      nullptr,
                      nullptr,
                      M,
                      N,
                      K,
                      K,
                      K,
                      N,
                      default_group_m(tiles_m, tiles_n),
                      Cfg4w::kDropinWorkers,
                      EpiArgs{},
                      MxArgs{},
                      SplitArgs{}};
  // 16-byte epilogue stores: N a multiple of 8 (C itself must be 16-byte
  // aligned, as every hipMalloc'd buffer is); the overlapped epilogue where
  // rows of C are whole 128-byte lines (N a multiple of 64 and C line-
  // aligned, as hipMalloc'd buffers are; an unaligned C stays correct).
  gemm_4wave_body<N % 8 == 0, 16, false, 0, kActNone, kOutBf16, false,
                  N % 64 == 0>(args, (lds_u8*)lds);
}

// The reference header's second kernel,
//   template <int M, int N, int K> __global__ __launch_bounds__(256, 1)
//   void fp8_gemm_4wave_256x256x128_ref(const fp8*, const fp8*, bf16*)
// (fp8_4wave.hpp:594-598): its "simple" 4-wave kernel, one 256 x 256 tile per
// workgroup, launched like the main one (<<<(M * N) / 65536, 256>>>).  Same
// name, template parameters and pointer signature, so callers that name it
// compile unchanged.  Here it is the same 4-wave schedule run without the
// persistent worker cap: every workgroup of the caller's grid is a worker,
// so a grid of one workgroup per tile gives each workgroup exactly one tile
// (the reference's _ref decomposition); other grids stay correct, as for the
// main kernel.  Output rounding is round-to-nearest-even, as in the
// reference's _ref epilogue (fp8_4wave.hpp:693-696).
template <int M, int N, int K>
__global__ __launch_bounds__(256, 1) void fp8_gemm_4wave_256x256x128_ref(
    const fp8* __restrict A, const fp8* __restrict B_T, bf16* __restrict C) {
  static_assert(M > 0 && N > 0 && K > 0, "shape must be positive");
  static_assert(K % 16 == 0, "K must be a multiple of 16 (16-byte rows)");
  using namespace hipgemm::detail;
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg4w::kLdsBytes];
  constexpr int tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
  const GemmArgs args{reinterpret_cast<const uint8_t*>(A),
                      reinterpret_cast<const uint8_t*>(B_T),
                      reinterpret_cast<uint16_t*>(C),
                      nullptr,
                      nullptr,
                      M,
                      N,
                      K,
                      K,
                      K,
                      N,
                      default_group_m(tiles_m, tiles_n),
                      0,  // workers: the whole grid
                      EpiArgs{},
                      MxArgs{},
                      SplitArgs{}};
  gemm_4wave_body<N % 8 == 0, 16, false, 0, kActNone, kOutBf16, false,
                  N % 64 == 0>(args, (lds_u8*)lds);
}
