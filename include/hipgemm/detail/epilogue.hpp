// Extended epilogue: per-row / per-column scales, bias, activation and the
// output type, shared by the schedules' kExt instantiations.  For element
// (m, n) with fp32 accumulator acc:
//
//   scale = row_scale[m] * (col_scale[n] * (scale_a * scale_b))
//   v     = fma(acc, scale, bias[n])          (one rounding)
//   C     = round_to_out(activation(v))       (RNE to bf16 or fp16; fp32 as
//                                              is; e4m3 of y * out_scale,
//                                              saturating: sat_e4m3)
//
// A null scale vector is all ones, a null bias is -0.0 (so that v is exactly
// acc * scale, -0 included), scale_a / scale_b are the per-tensor scalars
// (null = 1.0).  With every option off this is the per-tensor epilogue, bit
// for bit: 1 * (1 * s) = s and fma(acc, s, -0) = acc * s.
#pragma once

#include <type_traits>

#include "arch.hpp"

namespace hipgemm {
namespace detail {

// Activation codes (the values of include/hipgemm.h's HIPGEMM_ACT_*).
constexpr int kActNone = 0, kActRelu = 1, kActGeluTanh = 2, kActSilu = 3;
constexpr int kActAny = -1;  // chosen at run time (EpiVec::pack4)
// Output types (HIPGEMM_OUT_*) and their element sizes.
constexpr int kOutBf16 = 0, kOutF16 = 1, kOutF32 = 2, kOutF8 = 3;
__host__ __device__ constexpr int out_bytes(int out) {
  return out == kOutF32 ? 4 : out == kOutF8 ? 1 : 2;
}

struct EpiArgs {
  const float* row_scale = nullptr;  // M floats (one per row of A and C)
  const float* col_scale = nullptr;  // N floats (one per row of B_T)
  const float* bias = nullptr;       // N floats, added per column of C
  int act = kActNone;
  int out = kOutBf16;
  const float* out_scale = nullptr;  // device scalar (fp8 output), null = 1
};

// exp(x) as 2^(x log2 e) on the hardware exponential (v_exp_f32).
__device__ __forceinline__ float exp_fast(float x) {
  return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// The activations, written from their definitions:
//   relu(v) = v < 0 ? 0 : v                      (NaN stays NaN)
//   silu(v) = v / (1 + e^-v)                      (Elfwing et al. 2018)
//   gelu(v) = v/2 (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3)))
//             (Hendrycks & Gimpel 2016, tanh form), with
//             tanh(u) = 1 - 2 / (1 + e^(2u)).
__device__ __forceinline__ float relu(float v) { return v < 0.0f ? 0.0f : v; }
__device__ __forceinline__ float silu(float v) {
  return v * __builtin_amdgcn_rcpf(1.0f + exp_fast(-v));
}
__device__ __forceinline__ float gelu_tanh(float v) {
  const float u = 0.7978845608028654f * (v + 0.044715f * v * v * v);
  const float t = 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + exp_fast(2.0f * u));
  return 0.5f * v * (1.0f + t);
}

// fp32 -> the input of the e4m3 conversion under the __HIP_SATFINITE rule:
// Inf and NaN become a NaN of the same sign, finite magnitudes above 448
// become 448 (the hardware conversion then rounds to nearest even).
__device__ __forceinline__ float sat_e4m3(float x) {
  const uint32_t u = __builtin_bit_cast(uint32_t, x);
  const uint32_t a = u & 0x7fffffffu, s = u & 0x80000000u;
  const uint32_t r = a >= 0x7f800000u ? (s | 0x7fc00000u)
                     : a > 0x43e00000u ? (s | 0x43e00000u)
                                       : u;
  return __builtin_bit_cast(float, r);
}
// Four fp32 -> four OCP e4m3 bytes (v_cvt_pk_fp8_f32, round to nearest
// even), element 0 in the low byte.  The instruction writes every NaN as
// 0xff (measured: +Inf and +NaN came out 0xff); a NaN keeps its sign here,
// 0x7f | sign, as the __HIP_SATFINITE conversion does.
__device__ __forceinline__ uint32_t pack_e4m3x4(f32x4 v) {
  const f32x4 x{sat_e4m3(v[0]), sat_e4m3(v[1]), sat_e4m3(v[2]), sat_e4m3(v[3])};
  int w = __builtin_amdgcn_cvt_pk_fp8_f32(x[0], x[1], 0, false);
  w = __builtin_amdgcn_cvt_pk_fp8_f32(x[2], x[3], w, true);
  const i32x4 xb = __builtin_bit_cast(i32x4, x);  // whole-vector bit_cast
  uint32_t r = (uint32_t)w;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const uint32_t u = (uint32_t)xb[e];
    const bool nan = (u & 0x7fffffffu) > 0x7f800000u;
    const uint32_t byte = ((u >> 24) & 0x80u) | 0x7fu;
    r = nan ? (r & ~(0xffu << (8 * e))) | (byte << (8 * e)) : r;
  }
  return r;
}

// Two fp32 -> packed fp16x2, round-to-nearest-even.
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  using f16x2_t = _Float16 __attribute__((ext_vector_type(2)));
  f16x2_t v = __builtin_convertvector(f32x2{lo, hi}, f16x2_t);
  return __builtin_bit_cast(uint32_t, v);
}

// The per-lane vectors of the extended epilogue for a wave's kBR x kBC
// blocks of 16 x 16 (lane l: rows 16 bi + l % 16 of the wave's rows, columns
// 16 bj + 4 (l / 16) + e of its columns, e < 4): row scales r, column scales
// already multiplied by the per-tensor scalar (cs = col_scale * s), bias b.
template <int kBR, int kBC>
struct EpiVec {
  float r[kBR];
  float cs[kBC][4];
  float b[kBC][4];
  int act, out;
  float so = 1.0f;  // fp8 output scale

  // From LDS, as staged by the 4-wave schedule: rows at base + 4 r, columns
  // at base + 512 + 4 c, bias at base + 1024 + 4 c.  (The 16-byte reads are
  // bit-cast as whole vectors: __builtin_bit_cast of one vector element,
  // v[e], yields element 0 with this compiler.)
  __device__ __forceinline__ void read_lds(const lds_u8* base, const EpiArgs& e,
                                           float s, int lane) {
    const int lr = lane & 15, lc = 4 * (lane >> 4);
    const bool has_r = e.row_scale != nullptr, has_c = e.col_scale != nullptr,
               has_b = e.bias != nullptr;
#pragma unroll
    for (int bi = 0; bi < kBR; ++bi) {
      const float x = __builtin_bit_cast(float, lds_read4(base + 4 * (16 * bi + lr)));
      r[bi] = has_r ? x : 1.0f;
    }
#pragma unroll
    for (int bj = 0; bj < kBC; ++bj) {
      const f32x4 c = __builtin_bit_cast(
          f32x4, lds_read16(base + 512 + 4 * (16 * bj + lc)));
      const f32x4 bb = __builtin_bit_cast(
          f32x4, lds_read16(base + 1024 + 4 * (16 * bj + lc)));
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        cs[bj][q] = (has_c ? c[q] : 1.0f) * s;
        b[bj][q] = has_b ? bb[q] : -0.0f;
      }
    }
    act = __builtin_amdgcn_readfirstlane(e.act);  // wave-uniform branches
    out = __builtin_amdgcn_readfirstlane(e.out);
    if (out == kOutF8 && e.out_scale) so = *e.out_scale;
    compiler_fence();
  }

  // From global memory (buffer loads, zero past M or N): row0 / col0 are
  // the wave's first row and column.  The loads count in vmcnt.
  __device__ __forceinline__ void load(const EpiArgs& e, int M, int N, int row0,
                                       int col0, float s, int lane) {
    const int lr = lane & 15, lc = 4 * (lane >> 4);
    const __amdgpu_buffer_rsrc_t rr =
        make_rsrc(e.row_scale, e.row_scale ? (uint32_t)M * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(e.col_scale, e.col_scale ? (uint32_t)N * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(e.bias, e.bias ? (uint32_t)N * 4u : 0u);
#pragma unroll
    for (int bi = 0; bi < kBR; ++bi) {
      const float x = __builtin_bit_cast(
          float, __builtin_amdgcn_raw_buffer_load_b32(
                     rr, (uint32_t)(row0 + 16 * bi + lr) * 4u, 0, 0));
      r[bi] = e.row_scale ? x : 1.0f;
    }
#pragma unroll
    for (int bj = 0; bj < kBC; ++bj)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t o = (uint32_t)(col0 + 16 * bj + lc + q) * 4u;
        const float c =
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rc, o, 0, 0));
        const float bb =
            __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rb, o, 0, 0));
        cs[bj][q] = (e.col_scale ? c : 1.0f) * s;
        b[bj][q] = e.bias ? bb : -0.0f;
      }
    act = __builtin_amdgcn_readfirstlane(e.act);
    out = __builtin_amdgcn_readfirstlane(e.out);
    if (out == kOutF8 && e.out_scale) so = *e.out_scale;
  }

  // Elements q = 0..3 of block (bi, bj), packed (4 consecutive columns).
  // kAct: the activation code, or kActAny for the one `act` names, chosen
  // per block (scalar branches on a wave-uniform code).  kOut: the output
  // type.  The tiled schedules take <kAct, kOut> as kernel template
  // parameters: with per-block branches (or a copy of the epilogue per
  // choice inside one kernel) they lost 3-8 %.
  // The four activated values of block (bi, bj), before the conversion.
  template <int kAct>
  __device__ __forceinline__ f32x4 value4(float a0, float a1, float a2, float a3,
                                          int bi, int bj) const {
    float v0 = __builtin_fmaf(a0, r[bi] * cs[bj][0], b[bj][0]);
    float v1 = __builtin_fmaf(a1, r[bi] * cs[bj][1], b[bj][1]);
    float v2 = __builtin_fmaf(a2, r[bi] * cs[bj][2], b[bj][2]);
    float v3 = __builtin_fmaf(a3, r[bi] * cs[bj][3], b[bj][3]);
    const int a = kAct == kActAny ? act : kAct;
    if (a == kActRelu) {
      v0 = relu(v0), v1 = relu(v1), v2 = relu(v2), v3 = relu(v3);
    } else if (a == kActSilu) {
      v0 = silu(v0), v1 = silu(v1), v2 = silu(v2), v3 = silu(v3);
    } else if (a == kActGeluTanh) {
      v0 = gelu_tanh(v0), v1 = gelu_tanh(v1), v2 = gelu_tanh(v2),
      v3 = gelu_tanh(v3);
    }
    return f32x4{v0, v1, v2, v3};
  }
  // Four e4m3 bytes of the activated values times the output scale.
  __device__ __forceinline__ uint32_t e4m3x4(const f32x4& v) const {
    return pack_e4m3x4(v * so);
  }
  template <int kAct, int kOut>
  __device__ __forceinline__ u32x2 pack4(float a0, float a1, float a2, float a3,
                                         int bi, int bj) const {
    const f32x4 v = value4<kAct>(a0, a1, a2, a3, bi, bj);
    if constexpr (kOut == kOutF16)
      return u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])};
    else
      return u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
  }
  // All choices at run time (per block), for the skinny schedule's small
  // epilogue.
  __device__ __forceinline__ u32x2 pack4(float a0, float a1, float a2, float a3,
                                         int bi, int bj) const {
    if (out == kOutF16) return pack4<kActAny, kOutF16>(a0, a1, a2, a3, bi, bj);
    return pack4<kActAny, kOutBf16>(a0, a1, a2, a3, bi, bj);
  }

};

// One lane's four consecutive outputs of block (bi, bj) -- columns c .. c + 3
// of one row -- with the extended epilogue and the output type chosen at run
// time (ev.act, ev.out).  off: byte offset of column c in rsrc, with the
// row's out-of-range bit; cols_left: columns of C from the offsets' column 0.
// kVec: one store of the four elements (they never straddle N), else one per
// element, each masked by its own column.
template <bool kVec, int kBR, int kBC>
__device__ __forceinline__ void store_out4(const EpiVec<kBR, kBC>& ev, float a0,
                                           float a1, float a2, float a3, int bi,
                                           int bj, __amdgpu_buffer_rsrc_t rsrc,
                                           uint32_t off, int c, int cols_left) {
  auto oob = [&](int x) -> uint32_t {
    return (uint32_t)((cols_left - 1 - x) >> 31) & kOobOffset;
  };
  const f32x4 v = ev.template value4<kActAny>(a0, a1, a2, a3, bi, bj);
  if (ev.out == kOutF32) {
    if constexpr (kVec) {
      store_b128<0>(__builtin_bit_cast(i32x4, v), rsrc, off | oob(c), 0);
    } else {
      const i32x4 vb = __builtin_bit_cast(i32x4, v);  // whole-vector bit_cast
#pragma unroll
      for (int e = 0; e < 4; ++e)
        __builtin_amdgcn_raw_buffer_store_b32((uint32_t)vb[e], rsrc,
                                              (off | oob(c + e)) + 4 * e, 0, 0);
    }
  } else if (ev.out == kOutF8) {
    const uint32_t w = ev.e4m3x4(v);
    if constexpr (kVec) {
      __builtin_amdgcn_raw_buffer_store_b32(w, rsrc, off | oob(c), 0, 0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        __builtin_amdgcn_raw_buffer_store_b8((uint8_t)(w >> (8 * e)), rsrc,
                                             (off | oob(c + e)) + e, 0, 0);
    }
  } else {
    const u32x2 pk = ev.out == kOutF16
                         ? u32x2{pack_f16x2(v[0], v[1]), pack_f16x2(v[2], v[3])}
                         : u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    if constexpr (kVec) {
      __builtin_amdgcn_raw_buffer_store_b64(pk, rsrc, off | oob(c), 0, 0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t x = (e < 2 ? pk.x : pk.y) >> (16 * (e & 1));
        __builtin_amdgcn_raw_buffer_store_b16((unsigned short)x, rsrc,
                                              (off | oob(c + e)) + 2 * e, 0, 0);
      }
    }
  }
}

}  // namespace detail
}  // namespace hipgemm
