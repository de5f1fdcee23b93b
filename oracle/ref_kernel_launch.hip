// Launchers for the reference's own GPU kernel -- MEASUREMENT INFRASTRUCTURE.
//
// Compiled (by `make -C oracle ref`) against the reference's header where it
// lies in the reference tree (-I$(REF)); nothing of it is copied here.  The
// result, oracle/_ref/libref_gpu.so, lets bench.py time the reference's
// fp8_gemm_4wave_256x256x128<M,N,K> (fp8_4wave.hpp:334-567) in the same
// harness, on the same stream and inputs, as this library's kernel.  It is
// never part of the product path.
//
// The reference kernel is a template over the shape and is only valid where
// M and N are multiples of 256 and K of 128 (and the grid is a multiple of
// 8, fp8_4wave.hpp:357-377), so only the compute-bound benchmark shapes are
// instantiated.  It has no scales: C = bf16_truncate(A . B_T^T).
#include <hip/hip_runtime.h>

#include "fp8_4wave.hpp"

namespace {

template <int M, int N, int K>
hipError_t launch(const void* A, const void* B_T, void* C, hipStream_t s) {
  fp8_gemm_4wave_256x256x128<M, N, K><<<(M * N) / (256 * 256), 256, 0, s>>>(
      static_cast<const fp8*>(A), static_cast<const fp8*>(B_T),
      static_cast<bf16*>(C));
  return hipGetLastError();
}

}  // namespace

extern "C" {

// hipSuccess, or hipErrorInvalidValue for a shape with no instantiation.
hipError_t hipgemm_reference_4wave(const void* A, const void* B_T, void* C,
                                   int M, int N, int K, hipStream_t s) {
  if (M == 4096 && N == 4096 && K == 4096) return launch<4096, 4096, 4096>(A, B_T, C, s);
  if (M == 8192 && N == 8192 && K == 8192) return launch<8192, 8192, 8192>(A, B_T, C, s);
  if (M == 8192 && N == 28672 && K == 8192) return launch<8192, 28672, 8192>(A, B_T, C, s);
  if (M == 8192 && N == 8192 && K == 28672) return launch<8192, 8192, 28672>(A, B_T, C, s);
  return hipErrorInvalidValue;
}

}  // extern "C"
