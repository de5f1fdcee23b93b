// hipgemm -- gfx950 (CDNA4) device primitives.
//
// Everything here is a thin, named wrapper over one hardware facility:
//   * buffer resources (V#) with hardware range checking, so out-of-range
//     lanes read zero instead of faulting (ragged tiles, K tails);
//   * direct global->LDS DMA (buffer_load_dwordx4 ... lds), 16 bytes per lane,
//     written to LDS at M0 + 16*lane;
//   * v_mfma_f32_32x32x64_f8f6f4 / v_mfma_f32_16x16x128_f8f6f4 with OCP e4m3
//     operands (cbsz = blgp = 0) and fp32 accumulators;
//   * explicit s_waitcnt / s_barrier / s_setprio placement;
//   * v_cvt_pk_bf16_f32 (round-to-nearest-even fp32 -> bf16).
//
// Reference counterparts (nirw4nna/hipgemm): fp8_4wave.hpp:53-59 (MFMA
// wrapper), :80-100 (raw.buffer.load.lds and the buffer resource), :214-217
// (bf16 conversion, truncating there; RNE here).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace hipgemm {
namespace detail {

using i32x4 = int __attribute__((ext_vector_type(4)));
using i32x8 = int __attribute__((ext_vector_type(8)));
using u32x2 = unsigned __attribute__((ext_vector_type(2)));
using f32x2 = float __attribute__((ext_vector_type(2)));
using f32x4 = float __attribute__((ext_vector_type(4)));
using f32x16 = float __attribute__((ext_vector_type(16)));
using bf16x2_t = __bf16 __attribute__((ext_vector_type(2)));

// LDS (address space 3) byte pointer.
using lds_u8 = __attribute__((address_space(3))) uint8_t;

constexpr int kWave = 64;

// Word 3 of a gfx9 buffer resource: DATA_FORMAT (bits 18:15) = 4 (32-bit),
// everything else zero -- no swizzle, no add-tid, stride 0 (raw buffer), so
// the hardware range check is a plain byte-offset test against num_records.
constexpr int kBufferWord3 = 0x00020000;

// Cache policy of the C stores: nt (streaming).  Every CU reaches its tile
// epilogue at about the same time, so a round's C (32 MiB at 8192^3) is
// written in one burst; marked non-temporal it displaces less of the A/B
// panels the next tiles read from L2 (8192^3: +1.2 %, measured).
constexpr int kStoreC = 2;
// Cache policy of the C stores that write part of a line per instruction
// (straight from the accumulators: fp32 and e4m3 outputs, and the 8-, 2- and
// 1-byte stores for N or ldc that rule out 16-byte ones): cached, so the L2
// merges a line before it goes to memory.  Non-temporal, such stores
// measured 4x slower than cached (8192 x 8192 x 128).
constexpr int kStoreCPart = 0;

// Any per-lane offset at or above this is out of range for every buffer we
// build (num_records is always < 2^31): such a lane reads zero.
constexpr uint32_t kOobOffset = 0x80000000u;

// A buffer resource over [base, base + bytes).  Both must be wave-uniform
// (every caller builds them from kernel arguments, tile coordinates, the
// workgroup index or the scalar wave index); they are read from lane 0 into
// scalar registers.  Where part of the address came out of VALU code (integer
// division has no scalar form) the compiler would otherwise treat the
// resource as divergent and wrap every buffer instruction that takes it in a
// readfirstlane loop.  readfirstlane is convergent: a select between such a
// resource and another is not speculated (in a loop it becomes a branch), so
// the resources of the K loops are built once per tile, outside them.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base,
                                                           uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint64_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)p);
  const uint64_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(p >> 32));
  return __builtin_amdgcn_make_buffer_rsrc(reinterpret_cast<void*>(lo | (hi << 32)),
                                           (short)0,
                                           __builtin_amdgcn_readfirstlane((int)bytes),
                                           kBufferWord3);
}

// 16 bytes per lane, global (rsrc + voffset + soffset) -> LDS
// (lds_wave_base + 16 * lane).  lds_wave_base must be wave-uniform.
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rsrc,
                                      lds_u8* lds_wave_base, uint32_t voffset,
                                      uint32_t soffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void*)lds_wave_base, 16,
      (int)voffset, (int)soffset, 0, 0);
}

// 4 bytes per lane, global (rsrc + voffset) -> LDS (lds_wave_base + 4 * lane);
// each lane's range check covers exactly its own 4 bytes.
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t rsrc,
                                     lds_u8* lds_wave_base, uint32_t voffset) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(
      rsrc, (__attribute__((address_space(3))) void*)lds_wave_base, 4,
      (int)voffset, 0, 0, 0);
}

__device__ __forceinline__ i32x4 lds_read16(const lds_u8* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) i32x4*>(p);
}

__device__ __forceinline__ uint32_t lds_read4(const lds_u8* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) uint32_t*>(p);
}

__device__ __forceinline__ u32x2 lds_read8(const lds_u8* p) {
  return *reinterpret_cast<const __attribute__((address_space(3))) u32x2*>(p);
}

__device__ __forceinline__ void lds_write4(lds_u8* p, uint32_t v) {
  *reinterpret_cast<__attribute__((address_space(3))) uint32_t*>(p) = v;
}

__device__ __forceinline__ void lds_write8(lds_u8* p, u32x2 v) {
  *reinterpret_cast<__attribute__((address_space(3))) u32x2*>(p) = v;
}

__device__ __forceinline__ i32x8 join(i32x4 lo, i32x4 hi) {
  return i32x8{lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
}

// Operand formats of the f8f6f4 MFMA family (its cbsz / blgp immediates):
// OCP E4M3 (fp8), OCP E5M2 (bf8), OCP E2M3 and E3M2 (fp6, four per three
// bytes) and OCP E2M1 (fp4, two per byte).
constexpr int kFmtE4M3 = 0, kFmtE5M2 = 1, kFmtFp6E2M3 = 2, kFmtFp6E3M2 = 3,
              kFmtFp4 = 4;
// A kernel's operand-format pair kFmt: 0-3, bit 0 the 8-bit format of A,
// bit 1 that of B_T (0 = e4m3 x e4m3); kFmtPairFp4, fp4 x fp4;
// kFmtPairFp6 + 0-3, fp6 x fp6, bit 0 set for E3M2 A, bit 1 for E3M2 B_T.
constexpr int kFmtPairFp4 = 4;
constexpr int kFmtPairFp6 = 8;
__host__ __device__ constexpr bool is_fp4(int f) { return f == kFmtPairFp4; }
__host__ __device__ constexpr bool is_fp6(int f) { return (f & ~3) == kFmtPairFp6; }
__host__ __device__ constexpr int fmt_a(int f) {
  return is_fp4(f) ? kFmtFp4 : is_fp6(f) ? kFmtFp6E2M3 + (f & 1) : f & 1;
}
__host__ __device__ constexpr int fmt_b(int f) {
  return is_fp4(f) ? kFmtFp4 : is_fp6(f) ? kFmtFp6E2M3 + ((f >> 1) & 1) : (f >> 1) & 1;
}

// D[32x32] += X[32x64] . Y[32x64]^T -> fp32, X in format kFx, Y in kFy.
// Lane l carries row l%32 of X (and of Y) and 32 of its 64 K-bytes.
template <int kFx = kFmtE4M3, int kFy = kFmtE4M3>
__device__ __forceinline__ f32x16 mfma_32x32x64(i32x8 x, i32x8 y, f32x16 acc) {
  return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(x, y, acc, kFx, kFy, 0,
                                                         0, 0, 0);
}

// D[16x16] += X[16x128] . Y[16x128]^T -> fp32, X in format kFx, Y in kFy.
template <int kFx = kFmtE4M3, int kFy = kFmtE4M3>
__device__ __forceinline__ f32x4 mfma_16x16x128(i32x8 x, i32x8 y, f32x4 acc) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(x, y, acc, kFx, kFy,
                                                          0, 0, 0, 0);
}

// The same with E8M0 block scales (2^(e - 127); 255 is NaN), one byte per
// lane in the low byte of sx / sy: lane l gives the scale of row l % 16 of X
// / Y for K-block l / 16 (K 32 (l / 16) .. + 31).  In the instruction's K
// order, lane l carries K 16 (l / 16) .. + 15 in registers 0-3 and
// 64 + 16 (l / 16) .. + 15 in registers 4-7, so K-block b is held by lane
// groups 2b % 4 and 2b % 4 + 1, in registers 0-3 for b < 2 and 4-7 for
// b >= 2.
// kOx / kOy (op_sel) pick the byte of sx / sy that holds the scale.
template <int kFx, int kFy, int kOx, int kOy>
__device__ __forceinline__ f32x4 mfma_16x16x128_mx(i32x8 x, i32x8 y, f32x4 acc,
                                                   uint32_t sx, uint32_t sy) {
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
      x, y, acc, kFx, kFy, kOx, (int)sx, kOy, (int)sy);
}
// The same with the bytes ox, oy (0..3) given as values: in unrolled code,
// where they are constants, the switch folds to the one instruction (no
// shifts of the scale words).
template <int kFx = kFmtE4M3, int kFy = kFmtE4M3>
__device__ __forceinline__ f32x4 mfma_16x16x128_mx(i32x8 x, i32x8 y, f32x4 acc,
                                                   uint32_t sx, uint32_t sy,
                                                   int ox, int oy) {
#define HIPGEMM_MX_CASE(X, Y) \
  case 4 * X + Y:             \
    return mfma_16x16x128_mx<kFx, kFy, X, Y>(x, y, acc, sx, sy);
  switch (4 * ox + oy) {
    HIPGEMM_MX_CASE(0, 0) HIPGEMM_MX_CASE(0, 1) HIPGEMM_MX_CASE(0, 2)
    HIPGEMM_MX_CASE(0, 3) HIPGEMM_MX_CASE(1, 0) HIPGEMM_MX_CASE(1, 1)
    HIPGEMM_MX_CASE(1, 2) HIPGEMM_MX_CASE(1, 3) HIPGEMM_MX_CASE(2, 0)
    HIPGEMM_MX_CASE(2, 1) HIPGEMM_MX_CASE(2, 2) HIPGEMM_MX_CASE(2, 3)
    HIPGEMM_MX_CASE(3, 0) HIPGEMM_MX_CASE(3, 1) HIPGEMM_MX_CASE(3, 2)
    default: return mfma_16x16x128_mx<kFx, kFy, 3, 3>(x, y, acc, sx, sy);
  }
#undef HIPGEMM_MX_CASE
}

// One accumulator element (AGPR) -> VGPR at this point of the program.  The
// compiler otherwise copies every live accumulator to VGPRs at the end of the
// K loop in one burst, which needs 256 VGPRs on top of the live ones.
__device__ __forceinline__ float acc_read(float a) {
  float v;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(v) : "a"(a));
  return v;
}
// 128-bit buffer store followed by two wait states.  A v_accvgpr_read (the
// inline asm of acc_read, which the compiler's hazard check does not pad)
// that overwrites a data VGPR of the store in the very next cycle has been
// measured on gfx950 to replace that dword in some lanes with the new value.
// The nop is volatile asm, which the compiler keeps in order with every
// memory access and every other volatile asm, so each acc_read that follows
// the store in program order also follows the nop.
template <int kAux>
__device__ __forceinline__ void store_b128(i32x4 v, __amdgpu_buffer_rsrc_t rsrc,
                                           uint32_t voff, uint32_t soff) {
  __builtin_amdgcn_raw_buffer_store_b128(v, rsrc, voff, soff, kAux);
  asm volatile("s_nop 1" ::: "memory");
}

// 32 wait states, issued in place: covers the MFMA-result-to-VALU-read
// latency ahead of the first acc_read after an MFMA.
__device__ __forceinline__ void mfma_drain() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Two fp32 -> packed bf16x2, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  bf16x2_t v = __builtin_convertvector(f32x2{lo, hi}, bf16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

// Scalar wave index (a compile-time-unknown but wave-uniform value kept in an
// SGPR, so LDS DMA destinations built from it need no readfirstlane).
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
}
__device__ __forceinline__ int lane_id() { return threadIdx.x % kWave; }

// Explicit counters.  The compiler does not order LDS reads after LDS-DMA
// writes, so every stage hand-off is an explicit vmcnt wait + barrier.  The
// waits go through __builtin_amdgcn_s_waitcnt (not inline asm) so the
// compiler's own waitcnt insertion sees them and adds no redundant waits;
// sched_barrier(0) keeps the scheduler from moving any instruction (MFMA
// included) across a wait or barrier, and the empty asm with a "memory"
// clobber keeps IR passes from moving loads and stores across.
// gfx9 s_waitcnt immediate: vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] |
// vmcnt[5:4] at [15:14]; a field at its maximum means "do not wait".
constexpr int waitcnt_imm(int vmcnt, int lgkmcnt) {
  return (vmcnt & 15) | ((vmcnt >> 4) << 14) | (7 << 4) | (lgkmcnt << 8);
}
__device__ __forceinline__ void sched_fence() {
  __builtin_amdgcn_sched_barrier(0);
}
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  compiler_fence();
  sched_fence();
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(N, 15));
  sched_fence();
  compiler_fence();
}
template <int N>
__device__ __forceinline__ void wait_lgkmcnt() {
  static_assert(N >= 0 && N < 16, "lgkmcnt range");
  compiler_fence();
  sched_fence();
  __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, N));
  sched_fence();
  compiler_fence();
}
__device__ __forceinline__ void barrier() {
  compiler_fence();
  sched_fence();
  __builtin_amdgcn_s_barrier();
  sched_fence();
  compiler_fence();
}

}  // namespace detail
}  // namespace hipgemm
