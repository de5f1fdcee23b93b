// hipgemm -- C ABI implementation (libhipgemm.so).
//
// Argument validation, variant selection and kernel launches over
// hipLaunchKernel.  The kernels are the header schedules of
// include/hipgemm/detail/, instantiated here with runtime shapes.
#include "hipgemm.h"

#include <atomic>
#include <cstdint>

#include "hipgemm/detail/gemm_8wave.hpp"
#include "hipgemm/detail/gemm_skinny.hpp"
#include "hipgemm/fp8_gemm.hpp"

namespace {

using namespace hipgemm::detail;

// kRowCol: per-row / per-column scale vectors instead of per-tensor scalars.
template <bool kVecStore, int kMf, bool kRowCol>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_4wave(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg4w::kLdsBytes];
  gemm_4wave_body<kVecStore, kMf, kRowCol>(g, (lds_u8*)lds);
}

template <bool kVecStore, bool kRowCol>
__global__ __launch_bounds__(512, 1) void k_fp8_gemm_8wave(GemmArgs g) {
  __shared__ __attribute__((aligned(1024))) uint8_t lds[Cfg8w::kLdsBytes];
  gemm_8wave_body<kVecStore, kRowCol>(g, (lds_u8*)lds);
}

template <int kMB, bool kVec8, bool kRowCol>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_skinny(SkinnyArgs g) {
  gemm_skinny_body<kMB, kVec8, kRowCol>(g);
}

template <bool kVec8, bool kRowCol>
__global__ __launch_bounds__(256, 1) void k_fp8_gemm_skinny_reduce(SkinnyArgs g,
                                                                    int kmb) {
  gemm_skinny_reduce_body<kVec8, kRowCol>(g, kmb);
}

// 32-bit buffer offsets: 256 rows of A or B_T (1-byte elements) span at most
// 2^31 bytes, 256 rows of C (2-byte elements) likewise.
constexpr int kMaxLd = 1 << 23;
constexpr int kMaxLdc = 1 << 22;

bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

hipError_t validate(const void* A, const void* B_T, void* C, int M, int N,
                    int K, int lda, int ldb, int ldc, int variant) {
  if (M < 0 || N < 0 || K < 0) return hipErrorInvalidValue;
  if (variant < 0 || variant >= HIPGEMM_VARIANT_COUNT)
    return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  if (!C || !aligned(C, 2) || ldc < N || ldc > kMaxLdc)
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

template <int kMf, bool kRowCol>
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
      vec ? reinterpret_cast<const void*>(&k_fp8_gemm_4wave<true, kMf, kRowCol>)
          : reinterpret_cast<const void*>(&k_fp8_gemm_4wave<false, kMf, kRowCol>);
  return hipLaunchKernel(fn, dim3(grid), dim3(Cfg4w::kThreads), args, 0,
                         stream);
}

template <bool kRowCol>
hipError_t launch_8wave(GemmArgs g, hipStream_t stream) {
  // Same persistent grid as the 4-wave kernel (160 KiB of LDS: one
  // workgroup per CU).
  const int tiles = tiles_of(g.M, g.N);
  const int cus = cu_count();
  const int grid = tiles < cus ? tiles : cus;
  g.workers = grid;
  const bool vec = (g.N % 8 == 0) && (g.ldc % 8 == 0) && aligned(g.C, 16);
  void* args[] = {&g};
  const void* fn =
      vec ? reinterpret_cast<const void*>(&k_fp8_gemm_8wave<true, kRowCol>)
          : reinterpret_cast<const void*>(&k_fp8_gemm_8wave<false, kRowCol>);
  return hipLaunchKernel(fn, dim3(grid), dim3(Cfg8w::kThreads), args, 0, stream);
}

// Split-K plan of the skinny schedule: 16-row blocks of M, K-slices per
// 256-column tile (enough workgroups to give every CU one), and the
// workspace it needs (arrival counters, then the partial tiles).
struct SkinnyPlan {
  int kmb, tiles_n, slices, slice_steps;
  size_t counter_bytes, ws_bytes;
};

SkinnyPlan plan_skinny(int M, int N, int K) {
  SkinnyPlan p{};
  p.kmb = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8;
  p.tiles_n = (N + CfgSkinny::kBN - 1) / CfgSkinny::kBN;
  const int steps = (K + CfgSkinny::kBK - 1) / CfgSkinny::kBK;
  const int target = cu_count();
  int slices = (target + p.tiles_n - 1) / p.tiles_n;
  if (slices > steps) slices = steps;
  if (slices < 1) slices = 1;
  p.slice_steps = steps > 0 ? (steps + slices - 1) / slices : 0;
  p.slices = p.slice_steps > 0 ? (steps + p.slice_steps - 1) / p.slice_steps : 1;
  if (p.slices > 1) {
    p.counter_bytes = ((size_t)p.tiles_n * sizeof(int) + 255) / 256 * 256;
    p.ws_bytes = p.counter_bytes + (size_t)p.tiles_n * p.slices * p.kmb * 16 *
                                       CfgSkinny::kBN * sizeof(float);
  }
  return p;
}

template <int kMB, bool kRowCol>
hipError_t launch_skinny_mb(const SkinnyArgs& g, bool vec8, int grid,
                            hipStream_t stream) {
  void* args[] = {const_cast<SkinnyArgs*>(&g)};
  const void* fn =
      vec8 ? reinterpret_cast<const void*>(&k_fp8_gemm_skinny<kMB, true, kRowCol>)
           : reinterpret_cast<const void*>(&k_fp8_gemm_skinny<kMB, false, kRowCol>);
  return hipLaunchKernel(fn, dim3(grid), dim3(CfgSkinny::kThreads), args, 0,
                         stream);
}

template <bool kRowCol>
hipError_t launch_skinny(const GemmArgs& a, const SkinnyPlan& p, void* ws,
                         hipStream_t stream) {
  // From 4 row blocks up, one workgroup per column tile summing every slice
  // (1 MiB of partials per tile at M = 128) is the long pole: a second
  // kernel sums them over tiles_n x kmb workgroups instead.
  const int reduce_pass = p.slices > 1 && p.kmb >= 4;
  SkinnyArgs g{a.A, a.B, a.C, a.scale_a, a.scale_b, a.M, a.N, a.K,
               a.lda, a.ldb, a.ldc, p.slices, p.slice_steps, nullptr, nullptr,
               reduce_pass};
  if (p.slices > 1) {
    g.arrivals = static_cast<int*>(ws);
    g.partial = reinterpret_cast<float*>(static_cast<char*>(ws) + p.counter_bytes);
  }
  const bool vec8 = (a.N % 4 == 0) && (a.ldc % 4 == 0) && aligned(a.C, 8);
  const int grid = p.tiles_n * p.slices;
  hipError_t e;
  switch (p.kmb) {
    case 1: e = launch_skinny_mb<1, kRowCol>(g, vec8, grid, stream); break;
    case 2: e = launch_skinny_mb<2, kRowCol>(g, vec8, grid, stream); break;
    case 4: e = launch_skinny_mb<4, kRowCol>(g, vec8, grid, stream); break;
    default: e = launch_skinny_mb<8, kRowCol>(g, vec8, grid, stream); break;
  }
  if (e != hipSuccess || !reduce_pass) return e;
  int kmb = p.kmb;
  void* args[] = {&g, &kmb};
  const void* fn =
      vec8 ? reinterpret_cast<const void*>(&k_fp8_gemm_skinny_reduce<true, kRowCol>)
           : reinterpret_cast<const void*>(&k_fp8_gemm_skinny_reduce<false, kRowCol>);
  return hipLaunchKernel(fn, dim3(p.tiles_n * p.kmb), dim3(CfgSkinny::kThreads),
                         args, 0, stream);
}

int resolve_variant(int variant, int M, int N, int K);

// Shared body of the GEMM entry points.  `ws` may be null when `ws_given` is
// false: a schedule that needs a workspace then takes a stream-ordered
// allocation for the call.  With `rowcol`, scale_a / scale_b are vectors of M
// / N floats (or null for all ones) applied per row of C / per column of C.
template <bool kRowCol>
hipError_t run_gemm(const void* A, const void* B_T, void* C, int M, int N,
                    int K, int lda, int ldb, int ldc, const float* scale_a,
                    const float* scale_b, int variant, bool ws_given, void* ws,
                    size_t ws_bytes, hipStream_t stream) {
  hipError_t e = validate(A, B_T, C, M, N, K, lda, ldb, ldc, variant);
  if (e != hipSuccess) return e;
  if (variant == HIPGEMM_VARIANT_SKINNY && M > CfgSkinny::kMaxM)
    return hipErrorInvalidValue;
  if (ws_given && ws_bytes > 0 && (!ws || !aligned(ws, 256)))
    return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  // Scale vectors are read with 4-byte loads; the 32x32x64 schedule has no
  // per-row/per-column epilogue.
  if (kRowCol && (!aligned(scale_a, 4) || !aligned(scale_b, 4) ||
                  variant == HIPGEMM_VARIANT_4WAVE))
    return hipErrorInvalidValue;
  variant = resolve_variant(variant, M, N, K);
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
    case HIPGEMM_VARIANT_SKINNY: {
      const SkinnyPlan p = plan_skinny(M, N, K);
      if (p.ws_bytes == 0) return launch_skinny<kRowCol>(g, p, nullptr, stream);
      if (ws_given) {
        if (ws_bytes < p.ws_bytes) return hipErrorInvalidValue;
        return launch_skinny<kRowCol>(g, p, ws, stream);
      }
      void* tmp = nullptr;
      if ((e = hipMallocAsync(&tmp, p.ws_bytes, stream)) != hipSuccess) return e;
      e = hipMemsetAsync(tmp, 0, p.counter_bytes, stream);
      if (e == hipSuccess) e = launch_skinny<kRowCol>(g, p, tmp, stream);
      const hipError_t f = hipFreeAsync(tmp, stream);
      return e != hipSuccess ? e : f;
    }
    case HIPGEMM_VARIANT_4WAVE_MFMA16:
      return launch_4wave<16, kRowCol>(g, stream);
    case HIPGEMM_VARIANT_8WAVE:
      return launch_8wave<kRowCol>(g, stream);
    case HIPGEMM_VARIANT_4WAVE:
    default:
      if constexpr (kRowCol) return hipErrorInvalidValue;  // rejected above
      else return launch_4wave<32, false>(g, stream);
  }
}

int resolve_variant(int variant, int M, int N, int K) {
  return variant == HIPGEMM_VARIANT_AUTO ? hipgemm_select_variant(M, N, K)
                                         : variant;
}

}  // namespace

extern "C" {

int hipgemm_select_variant(int M, int N, int K) {
  // Up to 128 rows the GEMM is a stream over B_T: the split-K schedule
  // spreads it over every CU.  Above, the 4-wave 16x16x128 schedule (1-2 %
  // ahead of the 8-wave one from 4096^3 up, and at 4000 x 5000 x 3584),
  // except for short K on few tiles (a fraction of one round over the CUs),
  // where the 8-wave one is 3-12 % ahead (2048^3, 512^3).  Measured on
  // MI355X, schedules compared in one process.
  if (M <= CfgSkinny::kMaxM) return HIPGEMM_VARIANT_SKINNY;
  if (K <= 2048 && tiles_of(M, N) <= 128) return HIPGEMM_VARIANT_8WAVE;
  return HIPGEMM_VARIANT_4WAVE_MFMA16;
}

hipError_t hipgemm_fp8_gemm_bf16(const void* A, const void* B_T, void* C,
                                 int M, int N, int K, int lda, int ldb,
                                 int ldc, const float* scale_a,
                                 const float* scale_b, int variant,
                                 hipStream_t stream) {
  return run_gemm<false>(A, B_T, C, M, N, K, lda, ldb, ldc, scale_a, scale_b,
                         variant, false, nullptr, 0, stream);
}

hipError_t hipgemm_fp8_gemm_bf16_ws(const void* A, const void* B_T, void* C,
                                    int M, int N, int K, int lda, int ldb,
                                    int ldc, const float* scale_a,
                                    const float* scale_b, int variant,
                                    void* workspace, size_t workspace_bytes,
                                    hipStream_t stream) {
  return run_gemm<false>(A, B_T, C, M, N, K, lda, ldb, ldc, scale_a, scale_b,
                         variant, true, workspace, workspace_bytes, stream);
}

hipError_t hipgemm_fp8_gemm_bf16_rowcol(const void* A, const void* B_T, void* C,
                                        int M, int N, int K, int lda, int ldb,
                                        int ldc, const float* scale_rows,
                                        const float* scale_cols, int variant,
                                        void* workspace, size_t workspace_bytes,
                                        hipStream_t stream) {
  // A null workspace with a zero size lets the call allocate one when the
  // split-K schedule needs it, like hipgemm_fp8_gemm_bf16.
  const bool ws_given = workspace != nullptr || workspace_bytes != 0;
  return run_gemm<true>(A, B_T, C, M, N, K, lda, ldb, ldc, scale_rows,
                        scale_cols, variant, ws_given, workspace,
                        workspace_bytes, stream);
}

size_t hipgemm_workspace_size(int M, int N, int K, int variant) {
  if (M <= 0 || N <= 0 || K < 0) return 0;
  if (resolve_variant(variant, M, N, K) != HIPGEMM_VARIANT_SKINNY) return 0;
  if (M > CfgSkinny::kMaxM) return 0;
  return plan_skinny(M, N, K).ws_bytes;
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
    case HIPGEMM_VARIANT_SKINNY:
      return "skinny_splitk_256";
    case HIPGEMM_VARIANT_8WAVE:
      return "8wave_256x256x128_mfma16";
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
    const TileWalk walk = tile_walk(b, grid, tiles);
    for (int t = walk.first; t < walk.end && w < cap; t += walk.stride) {
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
