// Scratch memory of hipgemm_gemm_noalloc (include/hipgemm.h): a static device
// array, one copy per GPU, in a translation unit of its own so that it sits
// in its own code object -- the HIP runtime loads it on a GPU (and reserves
// the array there) at the first lookup below, not when any other kernel of
// the library first runs on that GPU.  No allocation call ever creates or
// frees it; it lives until the process ends.  Laid out as any workspace:
// arrival counters first (zero between calls), then partial tiles.  Host
// code never uses the array's name as an address: its per-device address
// comes from hipGetSymbolAddress (noalloc_scratch below).
#include "hipgemm.h"

#include <atomic>
#include <cstdint>
#include <mutex>

#include "kernels.hpp"

static __device__ __align__(256) uint8_t scratch[HIPGEMM_NOALLOC_SCRATCH_BYTES];

// Clears n 4-byte words (the scratch counters at first use on a device): a
// kernel, not a memset.
__global__ void clear_words(uint32_t* p, int n) {
  for (int i = blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += gridDim.x * blockDim.x)
    p[i] = 0u;
}

namespace hipgemm {
namespace kernels {

void* noalloc_scratch(hipStream_t stream, hipError_t* err) {
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> ptrs[kMaxDevices];
  static std::mutex init;
  int dev = 0;
  *err = hipGetDevice(&dev);
  if (*err != hipSuccess) return nullptr;
  if (dev < 0 || dev >= kMaxDevices) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  void* p = ptrs[dev].load(std::memory_order_acquire);
  if (p) return p;
  std::lock_guard<std::mutex> lock(init);
  p = ptrs[dev].load(std::memory_order_relaxed);
  if (p) return p;
  *err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (*err != hipSuccess || !p) {
    if (*err == hipSuccess) *err = hipErrorInvalidSymbol;
    return nullptr;
  }
  // The array is zero when its code object loads; the clear makes that
  // explicit.  Not under stream capture, where it would only be recorded
  // into the caller's graph (and run on every replay).
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  *err = hipStreamIsCapturing(stream, &cap);
  if (*err != hipSuccess) return nullptr;
  if (cap == hipStreamCaptureStatusNone) {
    const int words = (int)(HIPGEMM_WS_COUNTER_BYTES / sizeof(uint32_t));
    uint32_t* w = static_cast<uint32_t*>(p);
    void* args[] = {&w, (void*)&words};
    *err = hipLaunchKernel((const void*)clear_words, dim3(16), dim3(256), args,
                           0, stream);
    if (*err != hipSuccess) return nullptr;
  }
  ptrs[dev].store(p, std::memory_order_release);
  return p;
}

}  // namespace kernels
}  // namespace hipgemm
