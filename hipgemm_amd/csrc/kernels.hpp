// Kernel lookup across the library's translation units.  Each schedule's
// instantiations live in their own file (compiled in parallel); the C ABI
// (hipgemm.hip) asks here for the entry point of one configuration.
#pragma once

#include <hip/hip_runtime.h>

#include <type_traits>

#include "hipgemm/detail/gemm_8wave.hpp"
#include "hipgemm/detail/gemm_skinny.hpp"
#include "hipgemm/detail/gemm_strip.hpp"
#include "hipgemm/detail/gemm_t128.hpp"

namespace hipgemm {
namespace kernels {

// One configuration: operand formats (bit 0 A, bit 1 B_T), extended
// epilogue, its activation and output type, the store width (16 bytes per
// lane for the tiled schedules, 8 for the skinny one), and whether C's rows
// start on 128-byte lines (the 4-wave schedule's overlapped epilogue).
struct Key {
  int fmt = 0;
  bool ext = false;
  int act = 0;
  int out = 0;
  bool vec = true;
  bool line = false;
};

// Entry points (host handles for hipLaunchKernel), nullptr for a
// configuration that is not built.
const void* four_wave_plain(int mf, const Key& k);  // k4wave_plain.hip
const void* four_wave_ext_bf16(const Key& k);       // k4wave_ext_bf16.hip
const void* four_wave_ext_f16(const Key& k);        // k4wave_ext_f16.hip
const void* four_wave_ext_wide(const Key& k);       // k4wave_ext_wide.hip
const void* eight_wave_plain(const Key& k);         // k8wave_plain.hip
const void* eight_wave_ext_bf16(const Key& k);      // k8wave_ext_bf16.hip
const void* eight_wave_ext_f16(const Key& k);       // k8wave_ext_f16.hip
const void* skinny_plain(int kmb, int kf, const Key& k);  // kskinny_plain.hip
const void* skinny_ext(int kmb, int kf, const Key& k);    // kskinny_ext.hip
const void* skinny_reduce(int kf, const Key& k);    // kskinny_plain.hip
const void* strip_plain(int kmb, int knb, const Key& k);  // kstrip_plain.hip
const void* strip_ext(int kmb, int knb, const Key& k);    // kstrip_ext.hip
const void* four_wave_mx(const Key& k);             // k4wave_mx.hip
const void* tile128_mx(const Key& k);               // k4wave_mx.hip
const void* tile128_split_mx(const Key& k);         // k4wave_mx.hip
const void* tile128_plain(const Key& k);            // kt128_plain.hip
const void* tile128_ext_narrow(const Key& k);       // kt128_ext.hip
const void* tile128_ext_wide(const Key& k);         // kt128_ext_wide.hip
inline const void* tile128_ext(const Key& k) {
  return k.out >= detail::kOutF32 ? tile128_ext_wide(k) : tile128_ext_narrow(k);
}
const void* tile128_split(const Key& k);            // kt128_plain.hip
const void* tile128_reduce(const Key& k);           // kt128_plain.hip
const void* split_plain(const Key& k);              // ksplit_plain.hip
// hipgemm_gemm_noalloc's static scratch array on the current device
// (noalloc_scratch.hip): its address, looked up once per device (with that
// device current); at that first lookup its counter region is cleared on
// `stream` unless the stream is being captured.  nullptr with *err set on
// failure.
void* noalloc_scratch(hipStream_t stream, hipError_t* err);
// Packs [rows][ceil(K/32)] E8M0 scales (row stride ld) into MxArgs' layout.
hipError_t mx_pack(const uint8_t* src, int rows, int K, int ld, uint8_t* dst,
                   hipStream_t stream);

// Runtime value -> integral_constant, for building the lookups.
template <int I>
using ic = std::integral_constant<int, I>;
template <class F>
const void* sel2(int v, F&& f) {
  return v ? f(ic<1>{}) : f(ic<0>{});
}
// Operand-format pairs: the four 8-bit pairs and fp4 x fp4 (kFmtPairFp4).
template <class F>
const void* sel_fmt(int v, F&& f) {
  switch (v) {
    case 0: return f(ic<0>{});
    case 1: return f(ic<1>{});
    case 2: return f(ic<2>{});
    case 3: return f(ic<3>{});
    case 4: return f(ic<4>{});
    default: return nullptr;
  }
}
// The pairs of sel_fmt and fp6 x fp6 (kFmtPairFp6 + 0..3): the 128 x 128
// schedule's, and the 4-wave schedule's with the per-tensor epilogue.
template <class F>
const void* sel_fmt_t128(int v, F&& f) {
  switch (v) {
    case 8: return f(ic<8>{});
    case 9: return f(ic<9>{});
    case 10: return f(ic<10>{});
    case 11: return f(ic<11>{});
    default: return sel_fmt(v, f);
  }
}
template <class F>
const void* sel4(int v, F&& f) {
  switch (v) {
    case 0: return f(ic<0>{});
    case 1: return f(ic<1>{});
    case 2: return f(ic<2>{});
    case 3: return f(ic<3>{});
    default: return nullptr;
  }
}

}  // namespace kernels
}  // namespace hipgemm
