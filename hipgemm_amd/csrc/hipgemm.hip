// hipgemm -- C ABI implementation (libhipgemm.so).
//
// Argument validation, variant selection and kernel launches over
// hipLaunchKernel.  The kernels are the header schedules of
// include/hipgemm/detail/, instantiated here with runtime shapes.
#include "hipgemm.h"

#include <atomic>
#include <cstdint>

#include "hipgemm/fp8_gemm.hpp"

namespace {

using namespace hipgemm::detail;

template <bool kVecStore, int kMf>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_4wave(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg4w::kLdsBytes];
  gemm_4wave_body<kVecStore, kMf>(g, (lds_u8*)lds);
}

constexpr int kMaxLd = 1 << 23;  // 256 rows * ld (bytes) must stay below 2^31

bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

hipError_t validate(const void* A, const void* B_T, void* C, int M, int N,
                    int K, int lda, int ldb, int ldc, int variant) {
  if (M < 0 || N < 0 || K < 0) return hipErrorInvalidValue;
  if (variant < 0 || variant >= HIPGEMM_VARIANT_COUNT)
    return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  if (!C || !aligned(C, 2) || ldc < N || ldc > kMaxLd)
    return hipErrorInvalidValue;
  if (K == 0) return hipSuccess;  // A and B_T are not read
  if (!A || !B_T) return hipErrorInvalidValue;
  if (K % 16 != 0) return hipErrorInvalidValue;
  if (lda < K || ldb < K || lda % 16 != 0 || ldb % 16 != 0)
    return hipErrorInvalidValue;
  if (lda > kMaxLd || ldb > kMaxLd) return hipErrorInvalidValue;
  if (!aligned(A, 16) || !aligned(B_T, 16)) return hipErrorInvalidValue;
  return hipSuccess;
}

int tiles_of(int M, int N) {
  return ((M + Cfg4w::kBM - 1) / Cfg4w::kBM) * ((N + Cfg4w::kBN - 1) / Cfg4w::kBN);
}

// Compute units of the current device, queried once per device (a lazily
// filled, thread-safe cache; concurrent first calls store the same value).
int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

template <int kMf>
hipError_t launch_4wave(GemmArgs g, hipStream_t stream) {
  // Persistent grid: one workgroup per CU at most (the kernel's 160 KiB of
  // LDS allows no more), each walking tiles w, w + grid, ...
  const int tiles = tiles_of(g.M, g.N);
  const int cus = cu_count();
  const int grid = tiles < cus ? tiles : cus;
  g.workers = grid;
  // 16-byte epilogue stores need 8-column groups that never straddle N and
  // 16-byte aligned rows.
  const bool vec = (g.N % 8 == 0) && (g.ldc % 8 == 0) && aligned(g.C, 16);
  void* args[] = {&g};
  const void* fn =
      vec ? reinterpret_cast<const void*>(&k_fp8_gemm_4wave<true, kMf>)
          : reinterpret_cast<const void*>(&k_fp8_gemm_4wave<false, kMf>);
  return hipLaunchKernel(fn, dim3(grid), dim3(Cfg4w::kThreads), args, 0,
                         stream);
}

}  // namespace

extern "C" {

int hipgemm_select_variant(int M, int N, int K) {
  (void)M;
  (void)N;
  (void)K;
  // 16x16x128 sustains a higher clock than 32x32x64 under the power limit
  // that caps long GEMMs on MI355X (same work per step).
  return HIPGEMM_VARIANT_4WAVE_MFMA16;
}

hipError_t hipgemm_fp8_gemm_bf16(const void* A, const void* B_T, void* C,
                                 int M, int N, int K, int lda, int ldb,
                                 int ldc, const float* scale_a,
                                 const float* scale_b, int variant,
                                 hipStream_t stream) {
  hipError_t e = validate(A, B_T, C, M, N, K, lda, ldb, ldc, variant);
  if (e != hipSuccess || M == 0 || N == 0) return e;
  if (variant == HIPGEMM_VARIANT_AUTO) variant = hipgemm_select_variant(M, N, K);
  if (K == 0) lda = ldb = 16;  // nothing is read; keep the offset math inert
  const int tiles_m = (M + Cfg4w::kBM - 1) / Cfg4w::kBM;
  const int tiles_n = (N + Cfg4w::kBN - 1) / Cfg4w::kBN;
  GemmArgs g{static_cast<const uint8_t*>(A),
             static_cast<const uint8_t*>(B_T),
             static_cast<uint16_t*>(C),
             scale_a,
             scale_b,
             M,
             N,
             K,
             lda,
             ldb,
             ldc,
             default_group_m(tiles_m, tiles_n),
             0};
  switch (variant) {
    case HIPGEMM_VARIANT_4WAVE_MFMA16:
      return launch_4wave<16>(g, stream);
    case HIPGEMM_VARIANT_4WAVE:
    default:
      return launch_4wave<32>(g, stream);
  }
}

hipError_t hipgemm_fp8_gemm_4wave_256x256x128(const void* A, const void* B_T,
                                              void* C, int M, int N, int K,
                                              hipStream_t stream) {
  return hipgemm_fp8_gemm_bf16(A, B_T, C, M, N, K, K, K, N, nullptr, nullptr,
                               HIPGEMM_VARIANT_4WAVE_MFMA16, stream);
}

const char* hipgemm_variant_name(int variant) {
  switch (variant) {
    case HIPGEMM_VARIANT_AUTO:
      return "auto";
    case HIPGEMM_VARIANT_4WAVE:
      return "4wave_256x256x128_mfma32";
    case HIPGEMM_VARIANT_4WAVE_MFMA16:
      return "4wave_256x256x128_mfma16";
    default:
      return nullptr;
  }
}

int hipgemm_version(void) { return HIPGEMM_VERSION; }

int hipgemm_tile_order(int grid, int tiles_m, int tiles_n, int group_m,
                       int* tile_m, int* tile_n, int cap) {
  if (grid <= 0 || tiles_m <= 0 || tiles_n <= 0 || !tile_m || !tile_n ||
      cap < 0)
    return 0;
  if (group_m <= 0) group_m = default_group_m(tiles_m, tiles_n);
  const int tiles = tiles_m * tiles_n;
  int w = 0;
  for (int b = 0; b < grid && w < cap; ++b) {
    for (int t = xcd_contiguous(b, grid); t < tiles && w < cap; t += grid) {
      const TileCoord tc = grouped_tile(t, tiles_m, tiles_n, group_m);
      tile_m[w] = tc.m;
      tile_n[w] = tc.n;
      ++w;
    }
  }
  return w;
}

int hipgemm_lds_slot(int row, int chunk) {
  if (row < 0 || chunk < 0 || chunk > 7) return -1;
  return chunk ^ slot_xor(row);
}

}  // extern "C"
