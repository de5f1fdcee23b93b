// Extended epilogue: per-row / per-column scales, bias, activation and the
// output type, shared by the 4-wave, 8-wave and skinny schedules' kExt
// instantiations.  For element (m, n) with fp32 accumulator acc:
//
//   scale = row_scale[m] * (col_scale[n] * (scale_a * scale_b))
//   v     = fma(acc, scale, bias[n])          (one rounding)
//   C     = round_to_out(activation(v))       (RNE to bf16 or fp16)
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
// Output types (HIPGEMM_OUT_*).
constexpr int kOutBf16 = 0, kOutF16 = 1;

struct EpiArgs {
  const float* row_scale = nullptr;  // M floats (one per row of A and C)
  const float* col_scale = nullptr;  // N floats (one per row of B_T)
  const float* bias = nullptr;       // N floats, added per column of C
  int act = kActNone;
  int out = kOutBf16;
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
  }

  // Elements q = 0..3 of block (bi, bj), packed (4 consecutive columns).
  // kAct: the activation code, or kActAny for the one `act` names, chosen
  // per block (scalar branches on a wave-uniform code).  kOut: the output
  // type.  The tiled schedules take <kAct, kOut> as kernel template
  // parameters: with per-block branches (or a copy of the epilogue per
  // choice inside one kernel) they lost 3-8 %.
  template <int kAct, int kOut>
  __device__ __forceinline__ u32x2 pack4(float a0, float a1, float a2, float a3,
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
    if constexpr (kOut == kOutF16)
      return u32x2{pack_f16x2(v0, v1), pack_f16x2(v2, v3)};
    else
      return u32x2{pack_bf16x2(v0, v1), pack_bf16x2(v2, v3)};
  }
  // All choices at run time (per block), for the skinny schedule's small
  // epilogue.
  __device__ __forceinline__ u32x2 pack4(float a0, float a1, float a2, float a3,
                                         int bi, int bj) const {
    if (out == kOutF16) return pack4<kActAny, kOutF16>(a0, a1, a2, a3, bi, bj);
    return pack4<kActAny, kOutBf16>(a0, a1, a2, a3, bi, bj);
  }

};

}  // namespace detail
}  // namespace hipgemm
