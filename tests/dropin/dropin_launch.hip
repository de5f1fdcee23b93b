// Test launcher for the C++ drop-in header (include/fp8_4wave.hpp): launches
// fp8_gemm_4wave_256x256x128<M, N, K> and fp8_gemm_4wave_256x256x128_ref<M,
// N, K> exactly as the reference's callers do (test.cpp:79:
// <<<(M * N) / (256 * 256), 256>>>, no dynamic LDS), at a few fixed shapes,
// for the GPU parity tests.  Built by tests/dropin/Makefile (build()); test
// infrastructure only, not part of libhipgemm.so.
#include "fp8_4wave.hpp"

namespace {

template <int M, int N, int K>
hipError_t launch(int kernel, const void* A, const void* B, void* C, int grid,
                  hipStream_t s) {
  if (grid <= 0) grid = (M * N) / (256 * 256);  // the callers' formula
  if (grid <= 0) grid = 1;
  const fp8* a = static_cast<const fp8*>(A);
  const fp8* b = static_cast<const fp8*>(B);
  bf16* c = static_cast<bf16*>(C);
  if (kernel == 0)
    fp8_gemm_4wave_256x256x128<M, N, K><<<grid, 256, 0, s>>>(a, b, c);
  else
    fp8_gemm_4wave_256x256x128_ref<M, N, K><<<grid, 256, 0, s>>>(a, b, c);
  return hipGetLastError();
}

struct Shape {
  int M, N, K;
};
// The reference bench's default shape (bench.cpp:4-14) and its long-K
// LLM shape come last.
constexpr Shape kShapes[] = {{512, 512, 512},   {4096, 4096, 4096},
                             {4000, 5000, 3584}, {8192, 8192, 8192},
                             {8192, 8192, 28672}};

}  // namespace

extern "C" {

// Number of shapes, and shape i.
int dropin_shapes(void) { return (int)(sizeof(kShapes) / sizeof(kShapes[0])); }
int dropin_shape(int i, int* M, int* N, int* K) {
  if (i < 0 || i >= dropin_shapes() || !M || !N || !K) return -1;
  *M = kShapes[i].M;
  *N = kShapes[i].N;
  *K = kShapes[i].K;
  return 0;
}

// kernel 0: fp8_gemm_4wave_256x256x128, 1: ..._ref; grid <= 0: the callers'
// (M * N) / 65536.  Returns the hipError_t of the launch.
int dropin_launch(int kernel, int shape, const void* A, const void* B, void* C,
                  int grid, hipStream_t s) {
  switch (shape) {
    case 0: return (int)launch<512, 512, 512>(kernel, A, B, C, grid, s);
    case 1: return (int)launch<4096, 4096, 4096>(kernel, A, B, C, grid, s);
    case 2: return (int)launch<4000, 5000, 3584>(kernel, A, B, C, grid, s);
    case 3: return (int)launch<8192, 8192, 8192>(kernel, A, B, C, grid, s);
    case 4: return (int)launch<8192, 8192, 28672>(kernel, A, B, C, grid, s);
    default: return (int)hipErrorInvalidValue;
  }
}

}  // extern "C"
