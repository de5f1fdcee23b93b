// hipgemm -- column-strip FP8 GEMM for skinny M (gfx950).
//
// C[M x N] = scale_a * scale_b * A[M x K] . B_T[N x K]^T for M <= 128, where
// the work is one pass over B_T (16 x 8192 x 8192 moves 64 MiB of B_T against
// 2 GFLOP): the kernel is an HBM stream with MFMA on the side.  No reference
// counterpart: the reference kernel (fp8_4wave.hpp:334-567) is only valid for
// M a multiple of 256.
//
// Decomposition
//   * Workgroup (nt, s) of a (tiles_n x slices) grid owns the strip of
//     BN = 16 kNB columns [BN nt, BN nt + BN) of C over K-slice s
//     (`slice_steps` steps of 128 bytes).  With N / BN >= the CU count there
//     is one slice: no partial sums leave the workgroup, no workspace.
//   * The workgroup's four waves split the slice's K-steps into four
//     contiguous quarters; each wave computes the whole M x BN strip over its
//     quarter (kMB x kNB blocks of 16 x 16, v_mfma_f32_16x16x128_f8f6f4),
//     and the four partial strips are summed in LDS in wave order at the end.
//     So the main loop has no workgroup barrier at all.
//   * B_T (the HBM stream) goes global -> LDS by DMA (buffer_load_dwordx4
//     ... lds), 8 rows x 128 bytes -- whole lines -- per instruction, into a
//     ring of L + 1 stages private to the wave, with the non-temporal hint:
//     measured on a 64 MiB B_T, whole lines with nt stream at 5.4 TB/s, the
//     16-rows-by-64-bytes pattern of a direct register load at 4.5.  The
//     stage rows are 128 bytes in the plain K order with the strip_xor
//     swizzle (layout.hpp), under which the MFMA operand reads (chunks g
//     and g + 4 of 16 rows per lane group g) have no LDS bank conflict and
//     each DMA lane quad fetches one 64-byte run.  (With slot_xor, the
//     other schedules' swizzle, the same reads cost 4 conflict cycles each;
//     its conflict-free alternative, the instruction K order of layout.hpp,
//     makes each lane quad fetch two 32-byte pieces, which measured 2.5 %
//     slower on this HBM-bound kernel.)
//   * A (at most 128 rows, read by every strip, so L2-resident) goes
//     straight into registers, L steps ahead like B -- except for 32 rows
//     on 32-column strips, where it takes the same DMA path as B_T into a
//     ring of its own (CfgStrip::a_in_lds: measured faster there, slower
//     for 16 rows).
//   * K order inside a step: lane group g = l / 16 of the MFMA holds
//     K-chunks g and g + 4 of its row (the instruction's own order), for A
//     and B alike.
//
// With slices > 1 (narrow N), every workgroup stores its partial strip
// (fp32, written through to the coherent level with sc1) and bumps the
// strip's arrival counter; the workgroup that arrives last sums the slices
// in slice order (so the result does not depend on arrival order), applies
// the epilogue and resets the counter to zero.
//
// Buffer resources cover only the valid rows of A and of the strip of B_T,
// and K-chunks past the wave's K range read zero, so nothing outside A or
// B_T is addressed; C is written through a buffer resource over its window
// with out-of-range offsets for lanes outside M x N.
#pragma once

#include "arch.hpp"
#include "epilogue.hpp"
#include "layout.hpp"

namespace hipgemm {
namespace detail {

struct StripArgs {
  const uint8_t* A;      // M x K 8-bit (format by kFmt), row stride lda bytes
  const uint8_t* B;      // N x K 8-bit (B_T), row stride ldb bytes
  uint16_t* C;           // M x N, stride ldc elements of the output type
  const float* scale_a;  // device scalar, nullptr = 1.0
  const float* scale_b;  // device scalar, nullptr = 1.0
  int M, N, K;
  int lda, ldb, ldc;
  int slices;       // K-slices per strip (grid = tiles_n * slices)
  int slice_steps;  // 128-byte K-steps per slice
  float* partial;   // slices > 1: tiles_n * slices * kMB * kNB KiB
  int* arrivals;    // slices > 1: tiles_n counters, zero between calls
  EpiArgs epi;      // extended epilogue (kExt instantiations only)
};

struct CfgStrip {
  static constexpr int kThreads = 256;
  static constexpr int kBK = 128;
  static constexpr int kMaxM = 128;
  // Steps each wave keeps in flight: A occupies 8 kMB VGPRs per step in
  // flight, so 128 rows look two steps ahead, fewer rows three.
  static constexpr int lookahead(int kmb) { return kmb >= 8 ? 2 : 3; }
  // Bytes of one strip's fp32 partial (kMB x kNB blocks of 16 x 16).
  static constexpr int partial_bytes(int kmb, int knb) { return kmb * knb * 1024; }
  // A staged through LDS by DMA, as B_T is (whole lines), for 32 rows with
  // 32-column strips, where both rings fit in LDS (less 1 KiB for the
  // workgroup's other shared variables).  Measured against A in registers:
  // 32 x {8192 x 8192, 4096 x 14336, 2048 x 8192} 3 to 5 % faster; with 16
  // rows it is 1 to 22 % slower (16 x 8192 x 8192 15.2 against 12.8 us).
  static constexpr bool a_in_lds(int kmb, int knb) {
    return kmb == 2 && 4 * (lookahead(kmb) + 1) * (knb + kmb) * 16 * kBK <= 159 * 1024;
  }
  static constexpr int lds_bytes(int kmb, int knb) {
    const int rows = 16 * (knb + (a_in_lds(kmb, knb) ? kmb : 0));
    const int ring = 4 * (lookahead(kmb) + 1) * rows * kBK;
    const int red = 4 * kmb * knb * 1024;
    return ring > red ? ring : red;
  }
};

// kMB: 16-row blocks of M (M <= 16 kMB; 1, 2, 3, 4 or 8).  kNB: 16-column
// blocks per strip.
// kVec8: 8-byte C stores (N, ldc multiples of 4, C 8-byte aligned; 2-byte
// output types).  kExt: the extended epilogue of epilogue.hpp, output type
// and activation chosen at run time.
template <int kMB, int kNB, bool kVec8, bool kExt = false, int kFmt = 0>
__device__ __forceinline__ void gemm_strip_body(const StripArgs& g, lds_u8* lds) {
  using Cfg = CfgStrip;
  constexpr int L = Cfg::lookahead(kMB);
  constexpr int R = L + 1;                  // ring stages (LDS for B, VGPR or LDS for A)
  constexpr int kBN = 16 * kNB;             // strip width
  constexpr int kStageB = kBN * Cfg::kBK;   // bytes per wave per stage
  constexpr int kDmaB = kBN / 8;            // B DMA per step (8 rows each)
  constexpr bool kADma = Cfg::a_in_lds(kMB, kNB);
  constexpr int kStageA = 16 * kMB * Cfg::kBK;
  constexpr int kLdA = 2 * kMB;             // A loads (or DMA) per step
  constexpr int kOps = kDmaB + kLdA;        // vmcnt per step
  static_assert(L * kOps < 64, "vmcnt range");
  const int lane = lane_id();
  const int wave = wave_id();
  const int M = g.M, N = g.N, K = g.K;
  const int tiles_n = (N + kBN - 1) / kBN;
  const int nt = blockIdx.x % tiles_n;
  const int s = blockIdx.x / tiles_n;
  // The wave's K range in bytes, [kb0, kb1) (empty when the slice has fewer
  // than 4 q steps past it); q steps per wave, the same for every wave.
  const int q = (g.slice_steps + 3) / 4;
  const int kb0 = (s * g.slice_steps + wave * q) * Cfg::kBK;
  const int kb1 = min(min(K, (s + 1) * g.slice_steps * Cfg::kBK),
                      kb0 + q * Cfg::kBK);
  const int iters = (q + R - 1) / R * R;

  const int n0 = nt * kBN;
  const int rows_b = min(kBN, N - n0);
  const __amdgpu_buffer_rsrc_t rsrc_a = make_rsrc(g.A, (uint32_t)M * (uint32_t)g.lda);
  const __amdgpu_buffer_rsrc_t rsrc_b =
      make_rsrc(g.B + (size_t)n0 * g.ldb, (uint32_t)rows_b * (uint32_t)g.ldb);

  // DMA lane geometry: instruction j covers strip rows 8j .. 8j + 7; lane l
  // fetches row 8j + l/8, K-chunk (l%8) ^ strip_xor(row) -> LDS slot l % 8.
  const int drow = lane >> 3;
  uint32_t voff_b[kDmaB];
  int dch[kDmaB];
#pragma unroll
  for (int j = 0; j < kDmaB; ++j) {
    const int row = 8 * j + drow;
    dch[j] = (lane & 7) ^ strip_xor(row);
    voff_b[j] = (uint32_t)row * (uint32_t)g.ldb + (uint32_t)dch[j] * 16u;
  }
  // MFMA lane geometry: row r = l % 16 of a block, lane group gq = l / 16
  // holds K-chunks gq and gq + 4.
  const int r16 = lane & 15, gq = lane >> 4;
  uint32_t voff_a[kMB];
#pragma unroll
  for (int m = 0; m < kMB; ++m)
    voff_a[m] = (uint32_t)(16 * m + r16) * (uint32_t)g.lda + 16u * gq;
  // A by DMA: instruction j covers rows 8j .. 8j + 7, lanes as for B_T.
  uint32_t voff_da[kLdA];
#pragma unroll
  for (int j = 0; j < kLdA; ++j)
    voff_da[j] = (uint32_t)(8 * j + drow) * (uint32_t)g.lda + (uint32_t)dch[0] * 16u;
  const int sx = strip_xor(r16);
  lds_u8* ring = lds + wave * R * kStageB;
  lds_u8* ring_a = lds + 4 * R * kStageB + wave * R * kStageA;
  const uint32_t rd0 = (uint32_t)(r16 * Cfg::kBK + ((gq ^ sx) * 16));
  const uint32_t rd1 = (uint32_t)(r16 * Cfg::kBK + (((gq + 4) ^ sx) * 16));

  i32x4 aq[R][kMB][2];
  // Step i of the wave into ring slot d: A into registers (or LDS), B into LDS.
  auto issue = [&](int i, int d) {
    uint32_t k0 = (uint32_t)(kb0 + i * Cfg::kBK);
    asm volatile("" : "+s"(k0));
    const int lim = kb1 - (int)k0;  // bytes of this step inside the range
#pragma unroll
    for (int j = 0; j < kDmaB; ++j) {
      const uint32_t ok = (16 * dch[j] < lim) ? 0u : kOobOffset;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          rsrc_b, (__attribute__((address_space(3))) void*)(ring + d * kStageB + j * 1024),
          16, (int)(voff_b[j] | ok), (int)k0, 0, kStoreC /* nt */);
    }
    if constexpr (kADma) {
      const uint32_t ok = (16 * dch[0] < lim) ? 0u : kOobOffset;
#pragma unroll
      for (int j = 0; j < kLdA; ++j)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rsrc_a, (__attribute__((address_space(3))) void*)(ring_a + d * kStageA + j * 1024),
            16, (int)(voff_da[j] | ok), (int)k0, 0, 0);
    } else {
      const uint32_t oob0 = (16 * gq < lim) ? 0u : kOobOffset;
      const uint32_t oob1 = (64 + 16 * gq < lim) ? 0u : kOobOffset;
#pragma unroll
      for (int m = 0; m < kMB; ++m) {
        aq[d][m][0] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, voff_a[m] | oob0, k0, 0);
        aq[d][m][1] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, voff_a[m] | oob1, k0 + 64, 0);
      }
    }
  };

  f32x4 acc[kMB][kNB];
#pragma unroll
  for (int m = 0; m < kMB; ++m)
#pragma unroll
    for (int f = 0; f < kNB; ++f) acc[m][f] = f32x4{};

#pragma unroll
  for (int i = 0; i < L; ++i) issue(i, i);
  for (int i0 = 0; i0 < iters; i0 += R) {
#pragma unroll
    for (int d = 0; d < R; ++d) {
      // Ring slot (d + L) % R held step i - 1, whose LDS reads completed
      // (lgkmcnt 0) before its MFMA: refill it with step i + L.
      issue(i0 + d + L, (d + L) % R);
      wait_vmcnt<L * kOps>();  // step i's A loads and B DMA landed
      i32x8 b[kNB];
#pragma unroll
      for (int f = 0; f < kNB; ++f) {
        const lds_u8* p = ring + d * kStageB + f * 16 * Cfg::kBK;
        b[f] = join(lds_read16(p + rd0), lds_read16(p + rd1));
      }
      i32x8 al[kMB];
      if constexpr (kADma) {
#pragma unroll
        for (int m = 0; m < kMB; ++m) {
          const lds_u8* p = ring_a + d * kStageA + m * 16 * Cfg::kBK;
          al[m] = join(lds_read16(p + rd0), lds_read16(p + rd1));
        }
      }
      wait_lgkmcnt<0>();
#pragma unroll
      for (int m = 0; m < kMB; ++m) {
        const i32x8 a = kADma ? al[m] : join(aq[d][m][0], aq[d][m][1]);
#pragma unroll
        for (int f = 0; f < kNB; ++f)
          acc[m][f] = mfma_16x16x128<fmt_b(kFmt), fmt_a(kFmt)>(b[f], a, acc[m][f]);
      }
    }
  }
  // The look-ahead past the last step (zeros) still lands in LDS.
  wait_vmcnt<0>();
  mfma_drain();

  // ---- the four waves' partial strips, summed in wave order ---------------
  // Block (m, f) of wave w at ((w kMB + m) kNB + f) KiB, lane l at 16 l.  The
  // region overlaps the other waves' rings: barriers before and after.
  barrier();
#pragma unroll
  for (int m = 0; m < kMB; ++m)
#pragma unroll
    for (int f = 0; f < kNB; ++f) {
      const f32x4 v{acc_read(acc[m][f][0]), acc_read(acc[m][f][1]),
                    acc_read(acc[m][f][2]), acc_read(acc[m][f][3])};
      *reinterpret_cast<__attribute__((address_space(3))) f32x4*>(
          lds + ((wave * kMB + m) * kNB + f) * 1024 + lane * 16) = v;
    }
  wait_lgkmcnt<0>();
  barrier();
  // Wave w finishes blocks b = w, w + 4, ... of the kMB x kNB.
  constexpr int kBlocks = kMB * kNB;
  constexpr int kMine = (kBlocks + 3) / 4;
  f32x4 sum[kMine];
#pragma unroll
  for (int u = 0; u < kMine; ++u) {
    const int b = wave + 4 * u;  // wave-uniform
    sum[u] = f32x4{};
    if (b < kBlocks) {
      f32x4 p[4];
#pragma unroll
      for (int w = 0; w < 4; ++w)
        p[w] = *reinterpret_cast<const __attribute__((address_space(3))) f32x4*>(
            lds + (w * kBlocks + b) * 1024 + lane * 16);
      sum[u] = ((p[0] + p[1]) + p[2]) + p[3];
    }
  }

  // ---- slices > 1: partial strip out, arrival count, last one sums --------
  constexpr int kCoherent = 16;  // cache policy: sc1
  const int part = Cfg::partial_bytes(kMB, kNB);
  __shared__ int last;
  if (g.slices > 1) {
    const __amdgpu_buffer_rsrc_t rsrc_p = make_rsrc(
        reinterpret_cast<uint8_t*>(g.partial) + (size_t)nt * g.slices * part,
        (uint32_t)(g.slices * part));
#pragma unroll
    for (int u = 0; u < kMine; ++u) {
      const int b = wave + 4 * u;
      if (b < kBlocks)
        store_b128<kCoherent>(
            __builtin_bit_cast(i32x4, sum[u]), rsrc_p,
            (uint32_t)(b * 1024 + lane * 16), (uint32_t)(s * part));
    }
    wait_vmcnt<0>();
    barrier();
    if (threadIdx.x == 0) {
      const int before = __hip_atomic_fetch_add(g.arrivals + nt, 1, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
      last = before == g.slices - 1;
    }
    barrier();
    if (!last) return;
    // Every slice's partial, in slice order (the workgroup's own included,
    // read back, so that the order is the same whoever arrives last); slices
    // past the last load +0 out of range (no memory request) and add it.
#pragma unroll
    for (int u = 0; u < kMine; ++u) sum[u] = f32x4{};
    constexpr int kBatch = 8;
    for (int s0 = 0; s0 < g.slices; s0 += kBatch) {
      f32x4 v[kBatch][kMine];
#pragma unroll
      for (int t = 0; t < kBatch; ++t)
#pragma unroll
        for (int u = 0; u < kMine; ++u) {
          const int b = min(wave + 4 * u, kBlocks - 1);
          v[t][u] = __builtin_bit_cast(
              f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                         rsrc_p,
                         (uint32_t)(b * 1024 + lane * 16) |
                             (s0 + t < g.slices ? 0u : kOobOffset),
                         (uint32_t)(min(s0 + t, g.slices - 1) * part), kCoherent));
        }
#pragma unroll
      for (int t = 0; t < kBatch; ++t)
#pragma unroll
        for (int u = 0; u < kMine; ++u) sum[u] += v[t][u];
    }
  }

  // ---- epilogue: block (m, f), lane l -> row 16 m + l % 16, columns
  // n0 + 16 f + 4 (l / 16) .. + 3 (D = B_blk . A_blk^T) -------------------
  const float sa = g.scale_a ? *g.scale_a : 1.0f;
  const float sb = g.scale_b ? *g.scale_b : 1.0f;
  const float scale = sa * sb;
  EpiVec<kExt ? kMB : 1, kExt ? kNB : 1> ev;
  if constexpr (kExt) ev.load(g.epi, M, N, 0, n0, scale, lane);
  const int es = kExt ? out_bytes(ev.out) : 2;  // bytes per C element
  const __amdgpu_buffer_rsrc_t rsrc_c =
      make_rsrc(reinterpret_cast<uint8_t*>(g.C) + (size_t)n0 * es,
                (uint32_t)(((M - 1) * g.ldc + rows_b) * es));
  auto oob_unless = [](int x, int limit) -> uint32_t {
    return (uint32_t)((limit - 1 - x) >> 31) & kOobOffset;
  };
#pragma unroll
  for (int u = 0; u < kMine; ++u) {
    const int b = wave + 4 * u;
    if (b >= kBlocks) continue;
    const int m = b / kNB, f = b % kNB;
    const int row = 16 * m + r16;
    const int col = 16 * f + 4 * gq;
    const uint32_t base = (uint32_t)((row * g.ldc + col) * es) | oob_unless(row, M);
    const f32x4& a = sum[u];
    if constexpr (kExt) {
      store_out4<kVec8>(ev, a[0], a[1], a[2], a[3], kExt ? m : 0, kExt ? f : 0,
                        rsrc_c, base, col, rows_b);
      continue;
    }
    const uint32_t lo = pack_bf16x2(a[0] * scale, a[1] * scale);
    const uint32_t hi = pack_bf16x2(a[2] * scale, a[3] * scale);
    if constexpr (kVec8) {
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{lo, hi}, rsrc_c,
                                            base | oob_unless(col, rows_b), 0, 0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t w = (e < 2 ? lo : hi) >> (16 * (e & 1));
        __builtin_amdgcn_raw_buffer_store_b16(
            (unsigned short)w, rsrc_c, (base | oob_unless(col + e, rows_b)) + 2 * e,
            0, 0);
      }
    }
  }
  if (g.slices > 1 && threadIdx.x == 0)
    __hip_atomic_store(g.arrivals + nt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace detail
}  // namespace hipgemm
