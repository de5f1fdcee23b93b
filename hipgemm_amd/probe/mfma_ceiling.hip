// hipgemm -- MFMA ceiling probe (measurement only, not part of the GEMM API).
//
// Sustained rate of v_mfma_f32_16x16x128_f8f6f4 on this GPU with nothing but
// the matrix unit at work: each wave keeps 16 operand fragments (8 "A", 8
// "B", 32 bytes per lane each) in VGPRs and 64 accumulator blocks (256
// AGPRs per lane) -- the register footprint and MFMA stream of one wave of
// the 4-wave 256 x 256 schedule in one K-step -- and repeats that step
// `iters` times with no memory, LDS or barrier traffic.  One workgroup of 4
// waves (one per SIMD) per CU, as in the tiled kernels.
//
// The matrix unit's power depends on the operand bits, so the operands are
// whatever the caller loads into `ops` (bench.py: the same normal(0,1) e4m3
// distribution as its GEMM inputs).  Under sustained load an MI355X lowers
// its clock to stay inside its power limit; this kernel's rate is therefore
// the ceiling that a GEMM reaches only if its loads, LDS traffic and
// epilogue cost neither issue cycles nor energy.
#include <hip/hip_runtime.h>

#include "hipgemm/detail/arch.hpp"

using namespace hipgemm::detail;

namespace {

constexpr int kSets = 64;           // distinct operand sets in `ops`
constexpr int kFragsPerWave = 16;   // 8 A + 8 B fragments

__global__ __launch_bounds__(256, 1) void mfma_ceiling_16x16x128(
    const i32x8* __restrict__ ops, float* __restrict__ out, int iters) {
  const int lane = threadIdx.x % kWave;
  const int wave = threadIdx.x / kWave;
  const i32x8* src =
      ops + ((blockIdx.x * 4 + wave) % kSets) * (kFragsPerWave * kWave) + lane;
  i32x8 a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = src[i * kWave];
    b[i] = src[(8 + i) * kWave];
  }
  f32x4 acc[8][8];
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 8; ++j)
        acc[i][j] = mfma_16x16x128(a[i], b[j], acc[i][j]);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i)
#pragma unroll
    for (int j = 0; j < 8; ++j)
      s += (acc[i][j][0] + acc[i][j][1]) + (acc[i][j][2] + acc[i][j][3]);
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

}  // namespace

extern "C" {

// Bytes of `ops` the kernel reads: kSets operand sets of 16 fragments x 64
// lanes x 32 bytes (2 MiB).
size_t hipgemm_probe_ops_bytes(void) {
  return (size_t)kSets * kFragsPerWave * kWave * sizeof(i32x8);
}

// One launch of `grid` workgroups x 256 threads; `out` holds grid * 256
// floats.  flop per launch = grid * 4 * iters * 64 * (2 * 16 * 16 * 128).
int hipgemm_probe_mfma_ceiling(const void* ops, float* out, int grid,
                               int iters, hipStream_t stream) {
  if (!ops || !out || grid < 1 || iters < 1) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(mfma_ceiling_16x16x128, dim3(grid), dim3(256), 0, stream,
                     static_cast<const i32x8*>(ops), out, iters);
  return (int)hipGetLastError();
}

}  // extern "C"
