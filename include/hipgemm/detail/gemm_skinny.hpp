// hipgemm -- split-K FP8 GEMM for skinny M (gfx950).
//
// C[M x N] (bf16) = scale_a * scale_b * A[M x K] . B_T[N x K]^T for M <= 128,
// where the work is reading B_T once from HBM (16 x 8192 x 8192 moves 64 MiB
// of B_T against 2 GFLOP).  No reference counterpart: the reference kernel
// (fp8_4wave.hpp:334-567) is only valid for M a multiple of 256.
//
// Decomposition: workgroup (n, s) of a (tiles_n x slices) grid computes the
// fp32 partial C[0:M, BN n : BN n + BN] over K-slice s (`slice_steps` steps
// of 128), BN = 64 kF columns (kF = 4 up to 32 rows, 2 above:
// CfgSkinny::frags).  Slices make the grid fill the GPU although tiles_n is
// small.
//   * Wave w owns columns 16 kF w .. + 16 kF - 1 of the tile as kF x kMB
//     blocks of 16 x 16 (v_mfma_f32_16x16x128_f8f6f4, one per block per step).
//   * Every wave streams its 16 kF B_T rows straight into registers with
//     buffer_load_dwordx4, three steps ahead; A (at most 128 rows) too for
//     M <= 32, else the workgroup stages A once per step through LDS.  A lane holds, for its row, the K-bytes
//     16g .. 16g + 15 and 64 + 16g .. 64 + 16g + 15 of each 128-byte step
//     (g = lane / 16): any K order is valid as long as A and B_T use the
//     same one, and this one makes each load instruction read 64 contiguous
//     bytes of each of 16 rows.
//   * Every slice stores its partial tile (fp32, 16 bytes per lane, whole
//     1 KiB per instruction) into the workspace, then bumps the tile's
//     arrival counter (a relaxed agent-scope atomic).  The workgroup that
//     arrives last sums the slices in slice order 0, 1, ... (so the result
//     does not depend on arrival order), applies the scales, writes bf16 C
//     and resets the counter to zero for the next call.
//
// Buffer resources cover only the valid rows of A and B_T, and K-pieces past
// the slice end read zero, so nothing outside A or B_T is addressed; C is
// written through a buffer resource over its M x N window with out-of-range
// offsets for lanes outside it.
#pragma once

#include "arch.hpp"
#include "epilogue.hpp"
#include "layout.hpp"

namespace hipgemm {
namespace detail {

struct SkinnyArgs {
  const uint8_t* A;      // M x K 8-bit (format by kFmt), row stride lda bytes
  const uint8_t* B;      // N x K 8-bit (B_T), row stride ldb bytes
  uint16_t* C;           // M x N bf16 (fp16: kExt, epi.out), stride ldc elements
  const float* scale_a;  // device scalar, nullptr = 1.0
  const float* scale_b;  // device scalar, nullptr = 1.0
  int M, N, K;
  int lda, ldb, ldc;
  int slices;       // K-slices per column tile (grid = tiles_n * slices)
  int slice_steps;  // 128-byte K-steps per slice
  float* partial;   // tiles_n * slices * kMB * 16 * 256 floats
  int* arrivals;    // tiles_n counters, zero between calls
  int reduce_pass;  // 1: a separate kernel sums the slices (no counters)
  EpiArgs epi;      // extended epilogue (kExt instantiations only)
};

struct CfgSkinny {
  static constexpr int kThreads = 256;
  static constexpr int kBK = 128;
  // B_T fragments (16 columns each) per wave, 4 waves per workgroup: 4 up to
  // 32 rows; 2 above, which halves the workgroup's column tile and so the
  // K-slices and the partial-tile traffic per output (128 x 8192 x 8192:
  // 16 instead of 32 MiB written and read back).  From 65 rows the plan
  // may take 1 instead (hipgemm.hip, plan_skinny), for two workgroups per
  // CU.
  static constexpr int frags(int kmb) { return kmb >= 4 ? 2 : 4; }
  static constexpr int bn_of(int kf) { return 4 * 16 * kf; }
  static constexpr int kMaxM = 128;
};

// Epilogue of the C elements one lane writes: rows 16 (m0 + m) + l % 16
// (m < kRows) and columns col0 + 16 f + 4 (l / 16) + i (f < kF, i < 4).  Plain:
// the product of the two per-tensor scalars; kExt: the extended epilogue of
// epilogue.hpp from g.epi (vectors zero past M or N, never stored).
template <int kRows, bool kExt, int kF>
struct SkinnyEpi {
  float s = 1.0f;
  EpiVec<kExt ? kRows : 1, kExt ? kF : 1> ev;
  __device__ __forceinline__ void load(const SkinnyArgs& g, int m0, int col0,
                                       int lane) {
    const float sa = g.scale_a ? *g.scale_a : 1.0f;
    const float sb = g.scale_b ? *g.scale_b : 1.0f;
    s = sa * sb;
    if constexpr (kExt) ev.load(g.epi, g.M, g.N, 16 * m0, col0, s, lane);
  }
  // Elements i = 0..3 of block (m, f), packed.
  __device__ __forceinline__ u32x2 pack4(const f32x4& v, int m, int f) const {
    if constexpr (kExt)
      return ev.pack4(v[0], v[1], v[2], v[3], m, f);
    else
      return u32x2{pack_bf16x2(v[0] * s, v[1] * s), pack_bf16x2(v[2] * s, v[3] * s)};
  }
};

// kMB: 16-row blocks of M (M <= 16 kMB).  kVec8: C rows allow 8-byte stores
// (N % 4 == 0, ldc % 4 == 0, C 8-byte aligned).  kExt: the extended
// epilogue (SkinnyEpi).  kF: B_T fragments per wave.
template <int kMB, bool kVec8, bool kExt = false, int kFmt = 0,
          int kF = CfgSkinny::frags(kMB)>
__device__ __forceinline__ void gemm_skinny_body(const SkinnyArgs& g) {
  using Cfg = CfgSkinny;
  constexpr int kBN = Cfg::bn_of(kF);  // columns per workgroup
  // A (at most 128 rows) is shared by the four waves: up to 32 rows each
  // wave loads its own copy into registers; above, the workgroup stages it
  // through LDS once (DMA, one barrier per step) so A costs no more HBM or
  // L2 traffic than its share.
  constexpr bool kLdsA = kMB >= 4;
  // Register sets / LDS stages: kDepth - 1 steps of loads stay in flight per
  // wave (the whole GPU's worth of in-flight loads is about half of a
  // 64 MiB B_T, so the look-ahead is as deep as the registers allow).
  // (With A in LDS, 7 steps instead of 3 measured no faster at
  // 128 x 8192 x 8192 and 24 % slower at 128 x 28672 x 8192.)
  constexpr int kDepth = kLdsA ? 4 : kMB <= 2 ? 4 : 3;
  constexpr int kDmaA = kLdsA ? kMB / 2 : 0;  // A DMA per wave per step
  constexpr int kLoads = 2 * kF + (kLdsA ? kDmaA : 2 * kMB);  // per wave per step
  static_assert((kDepth - 1) * kLoads < 64, "vmcnt range");
  const int lane = lane_id();
  const int wave = wave_id();
  const int M = g.M, N = g.N, K = g.K;
  const int tiles_n = (N + kBN - 1) / kBN;
  const int nt = blockIdx.x % tiles_n;
  const int s = blockIdx.x / tiles_n;
  const int k_begin = s * g.slice_steps * Cfg::kBK;
  const int k_end = min(K, k_begin + g.slice_steps * Cfg::kBK);
  const int steps = (k_end - k_begin + Cfg::kBK - 1) / Cfg::kBK;
  const int steps_pad = (steps + kDepth - 1) / kDepth * kDepth;

  const int n0 = nt * kBN;
  const int rows_b = min(kBN, N - n0);
  const __amdgpu_buffer_rsrc_t rsrc_a =
      make_rsrc(g.A, (uint32_t)M * (uint32_t)g.lda);
  const __amdgpu_buffer_rsrc_t rsrc_b =
      make_rsrc(g.B + (size_t)n0 * g.ldb, (uint32_t)rows_b * (uint32_t)g.ldb);

  const int r16 = lane & 15, grp = lane >> 4;
  // Lane row offsets: B_T rows 16 kF w + 16f + r16 (f < kF), A rows
  // 16m + r16.
  uint32_t voff_b[kF], voff_a[kLdsA ? 1 : kMB];
#pragma unroll
  for (int f = 0; f < kF; ++f)
    voff_b[f] = (uint32_t)(wave * 16 * kF + 16 * f + r16) * (uint32_t)g.ldb + 16 * grp;
  if constexpr (!kLdsA) {
#pragma unroll
    for (int m = 0; m < kMB; ++m)
      voff_a[m] = (uint32_t)(16 * m + r16) * (uint32_t)g.lda + 16 * grp;
  }

  // LDS A stages (kLdsA): BM rows x 128 B each, row r at 128 r, in the
  // instruction K order of layout.hpp: 16-byte slot x of the row holds
  // K-chunk kpair_chunk(x ^ slot_xor(r)), so a lane group's chunks g and
  // g + 4 sit at slots 2g and 2g + 1 (conflict-free 16-row fragment reads).
  // DMA instruction q (8 rows) belongs to wave q % 4; its lane l fetches row
  // 8q + l/8, chunk kpair_chunk((l%8) ^ slot_xor(row)) from global.
  constexpr int kStageA = kMB * 16 * Cfg::kBK;
  __shared__ __attribute__((aligned(1024))) uint8_t lds_a[kLdsA ? kDepth * kStageA : 16];
  const int drow = lane >> 3;
  uint32_t voff_dma[kDmaA > 0 ? kDmaA : 1];
  if constexpr (kLdsA) {
#pragma unroll
    for (int i = 0; i < kDmaA; ++i) {
      const int row = 8 * (4 * i + wave) + drow;
      voff_dma[i] = (uint32_t)row * (uint32_t)g.lda +
                    (uint32_t)(kpair_chunk((lane & 7) ^ slot_xor(row & 15)) * 16);
    }
  }
  const int sx16 = slot_xor(r16);

  i32x4 bq[kDepth][kF][2], aq[kLdsA ? 1 : kDepth][kMB][2];
  // Loads of step kb into register set / LDS stage d; pieces past the slice
  // end read 0.
  auto load_step = [&](int kb, int d) {
    uint32_t k0 = (uint32_t)(k_begin + kb * Cfg::kBK);
    asm volatile("" : "+s"(k0));
    const int lim = k_end - (int)k0;  // bytes of this step inside the slice
    const uint32_t oob0 = (16 * grp < lim) ? 0u : kOobOffset;
    const uint32_t oob1 = (64 + 16 * grp < lim) ? 0u : kOobOffset;
#pragma unroll
    for (int f = 0; f < kF; ++f) {
      bq[d][f][0] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_b, voff_b[f] | oob0, k0, 0);
      bq[d][f][1] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_b, voff_b[f] | oob1, k0 + 64, 0);
    }
    if constexpr (kLdsA) {
      const uint32_t oobd = (16 * kpair_chunk((lane & 7) ^ slot_xor((8 * wave + drow) & 15)) < lim)
                                ? 0u : kOobOffset;
#pragma unroll
      for (int i = 0; i < kDmaA; ++i) {
        // rows 8(4i + w) + l/8: slot_xor depends on row % 16 = 8(w % 2) + l/8
        dma16(rsrc_a,
              (lds_u8*)lds_a + d * kStageA + (4 * i + wave) * 1024,
              voff_dma[i] | oobd, k0);
      }
    } else {
#pragma unroll
      for (int m = 0; m < kMB; ++m) {
        aq[d][m][0] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, voff_a[m] | oob0, k0, 0);
        aq[d][m][1] = __builtin_amdgcn_raw_buffer_load_b128(rsrc_a, voff_a[m] | oob1, k0 + 64, 0);
      }
    }
  };

  f32x4 acc[kMB][kF];
#pragma unroll
  for (int m = 0; m < kMB; ++m)
#pragma unroll
    for (int f = 0; f < kF; ++f) acc[m][f] = f32x4{};

  auto mfma_step = [&](int d) {
#pragma unroll
    for (int m = 0; m < kMB; ++m) {
      i32x8 a;
      if constexpr (kLdsA) {
        const lds_u8* row = (const lds_u8*)lds_a + d * kStageA + (16 * m + r16) * Cfg::kBK;
        a = join(lds_read16(row + ((kpair_slot(grp) ^ sx16) * 16)),
                 lds_read16(row + ((kpair_slot(grp + 4) ^ sx16) * 16)));
      } else {
        a = join(aq[d][m][0], aq[d][m][1]);
      }
#pragma unroll
      for (int f = 0; f < kF; ++f)
        acc[m][f] = mfma_16x16x128<fmt_b(kFmt), fmt_a(kFmt)>(
            join(bq[d][f][0], bq[d][f][1]), a, acc[m][f]);
    }
  };

#pragma unroll
  for (int d = 0; d < kDepth - 1; ++d) load_step(d, d);
  for (int k0 = 0; k0 < steps_pad; k0 += kDepth) {
#pragma unroll
    for (int d = 0; d < kDepth; ++d) {
      if constexpr (kLdsA) {
        // step k0 + d landed (own part), every wave's part landed and every
        // wave done with the stage refilled below (the one step k0 + d - 1
        // read); then the refill, then this step's A from LDS.
        wait_vmcnt<(kDepth - 2) * kLoads>();
        wait_lgkmcnt<0>();
        barrier();
        load_step(k0 + d + kDepth - 1, (d + kDepth - 1) % kDepth);
      } else {
        load_step(k0 + d + kDepth - 1, (d + kDepth - 1) % kDepth);
        wait_vmcnt<(kDepth - 1) * kLoads>();  // step k0 + d landed
      }
      mfma_step(d);
    }
  }
  wait_vmcnt<0>();  // the last look-ahead loads (zeros) are done with
  mfma_drain();

  // ---- partial tile out, arrival count ------------------------------------
  // Partial tiles cross XCDs, whose L2s are not coherent with each other:
  // they are stored with sc1 (written through to the coherent level) and
  // read back with sc1 (fetched from there), which needs no L2 write-back or
  // invalidate.  The counter is a relaxed agent-scope atomic; ordering comes
  // from waiting for the stores' completion (vmcnt 0) in every wave before
  // the workgroup barrier that precedes the increment.
  constexpr int kCoherent = 16;  // cache policy: sc1
  const int tile_floats = kMB * 16 * kBN;  // floats of one slice's partial
  const __amdgpu_buffer_rsrc_t rsrc_p = make_rsrc(
      g.partial + (size_t)nt * g.slices * tile_floats,
      (uint32_t)(g.slices * tile_floats * sizeof(float)));
  // layout: float4 (m, f, wave, lane) at byte ((m*4 + f)*256 + 64 w + l)*16
  auto slot = [&](int m, int f) {
    return (uint32_t)(((m * kF + f) * Cfg::kThreads + wave * 64 + lane) * 16);
  };
  const uint32_t mine = (uint32_t)(s * tile_floats * sizeof(float));
  __shared__ int last;
  if (g.slices > 1) {
#pragma unroll
    for (int m = 0; m < kMB; ++m)
#pragma unroll
      for (int f = 0; f < kF; ++f) {
        const f32x4 v{acc_read(acc[m][f][0]), acc_read(acc[m][f][1]),
                      acc_read(acc[m][f][2]), acc_read(acc[m][f][3])};
        store_b128<kCoherent>(
            __builtin_bit_cast(i32x4, v), rsrc_p, slot(m, f), mine);
      }
    if (g.reduce_pass) return;
    wait_vmcnt<0>();
    barrier();
    if (threadIdx.x == 0) {
      const int before = __hip_atomic_fetch_add(
          g.arrivals + nt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      last = before == g.slices - 1;
    }
    barrier();
    if (!last) return;
  }

  // ---- last arrival: sum the slices in order, scale, bf16, store ----------
  SkinnyEpi<kMB, kExt, kF> scl;
  scl.load(g, 0, n0 + wave * 16 * kF, lane);
  const int es = kExt ? out_bytes(scl.ev.out) : 2;  // bytes per C element
  const __amdgpu_buffer_rsrc_t rsrc_c =
      make_rsrc(reinterpret_cast<uint8_t*>(g.C) + (size_t)n0 * es,
                (uint32_t)(((M - 1) * g.ldc + rows_b) * es));
  auto oob_unless = [](int x, int limit) -> uint32_t {
    return (uint32_t)((limit - 1 - x) >> 31) & kOobOffset;
  };
  // Sums over the slices, in slice order; the loads of kBatch slices (all
  // kMB x 4 blocks each, 32 loads) are issued before any is consumed.
  constexpr int kBatch = 8 / kMB;
  f32x4 sum[kMB][kF];
#pragma unroll
  for (int m = 0; m < kMB; ++m)
#pragma unroll
    for (int f = 0; f < kF; ++f)
      sum[m][f] = g.slices > 1
                      ? f32x4{}
                      : f32x4{acc_read(acc[m][f][0]), acc_read(acc[m][f][1]),
                              acc_read(acc[m][f][2]), acc_read(acc[m][f][3])};
  if (g.slices > 1) {
    const uint32_t stride = (uint32_t)(tile_floats * sizeof(float));
    for (int q0 = 0; q0 < g.slices; q0 += kBatch) {
      f32x4 v[kBatch][kMB][kF];
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
#pragma unroll
        for (int m = 0; m < kMB; ++m)
#pragma unroll
          for (int f = 0; f < kF; ++f)
            v[u][m][f] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                           rsrc_p, slot(m, f) | (q0 + u < g.slices ? 0u : kOobOffset),
                           (uint32_t)min(q0 + u, g.slices - 1) * stride,
                           kCoherent));
      // Slices past the last load out of range: +0, no memory request, and
      // adding it leaves every sum unchanged (a sum started at +0 is never
      // -0).  A branch here instead lets the compiler sink each load into
      // its branch and wait for it alone.
#pragma unroll
      for (int u = 0; u < kBatch; ++u)
#pragma unroll
        for (int m = 0; m < kMB; ++m)
#pragma unroll
          for (int f = 0; f < kF; ++f) sum[m][f] += v[u][m][f];
    }
  }
#pragma unroll
  for (int m = 0; m < kMB; ++m)
#pragma unroll
    for (int f = 0; f < kF; ++f) {
      // D = B_blk . A_blk^T: lane l, element i -> C row 16m + l%16,
      // column 16 kF w + 16f + 4(l/16) + i (4 consecutive columns).
      const int row = 16 * m + r16;
      const int col = wave * 16 * kF + 16 * f + 4 * grp;
      const uint32_t base = (uint32_t)((row * g.ldc + col) * es) |
                            oob_unless(row, M);
      if constexpr (kExt) {
        const f32x4& a = sum[m][f];
        store_out4<kVec8>(scl.ev, a[0], a[1], a[2], a[3], m, f, rsrc_c, base, col,
                          rows_b);
        continue;
      }
      const u32x2 pk = scl.pack4(sum[m][f], m, f);
      const uint32_t lo = pk.x, hi = pk.y;
      if constexpr (kVec8) {
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{lo, hi}, rsrc_c,
                                              base | oob_unless(col, rows_b), 0, 0);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t w = (i < 2 ? lo : hi) >> (16 * (i & 1));
          __builtin_amdgcn_raw_buffer_store_b16(
              (unsigned short)w, rsrc_c,
              (base | oob_unless(col + i, rows_b)) + 2 * i, 0, 0);
        }
      }
    }
  if (g.slices > 1 && threadIdx.x == 0)
    __hip_atomic_store(g.arrivals + nt, 0, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}

// Separate slice reduction (reduce_pass): workgroup (nt, m) sums 16-row
// block m of column tile nt over the slices in slice order, applies the
// scales and writes bf16 C -- the same arithmetic and the same C mapping as
// the in-kernel reduction, spread over tiles_n x kMB workgroups instead of
// one per tile.  Launched on the same stream right after the split kernel,
// so its partial tiles are visible without any fence.
template <bool kVec8, bool kExt, int kF>
__device__ __forceinline__ void gemm_skinny_reduce_body(const SkinnyArgs& g,
                                                        int kmb) {
  using Cfg = CfgSkinny;
  constexpr int kBN = 4 * 16 * kF;
  const int lane = lane_id();
  const int wave = wave_id();
  const int M = g.M, N = g.N;
  const int tiles_n = (N + kBN - 1) / kBN;
  const int nt = blockIdx.x % tiles_n;
  const int m = blockIdx.x / tiles_n;
  const int n0 = nt * kBN;
  const int rows_b = min(kBN, N - n0);
  const int r16 = lane & 15, grp = lane >> 4;
  const int tile_floats = kmb * 16 * kBN;
  const __amdgpu_buffer_rsrc_t rsrc_p = make_rsrc(
      g.partial + (size_t)nt * g.slices * tile_floats,
      (uint32_t)(g.slices * tile_floats * sizeof(float)));
  const uint32_t stride = (uint32_t)(tile_floats * sizeof(float));
  auto slot = [&](int f) {
    return (uint32_t)(((m * kF + f) * Cfg::kThreads + wave * 64 + lane) * 16);
  };
  // Scales first: their latency hides under the slice loads (read after the
  // loop they cost this short kernel one more memory round trip).
  SkinnyEpi<1, kExt, kF> scl;
  scl.load(g, m, n0 + wave * 16 * kF, lane);
  constexpr int kBatch = 8;  // slices whose loads are in flight together
  f32x4 sum[kF] = {};
  for (int q0 = 0; q0 < g.slices; q0 += kBatch) {
    f32x4 v[kBatch][kF];
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
#pragma unroll
      for (int f = 0; f < kF; ++f)
        v[u][f] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                       rsrc_p, slot(f) | (q0 + u < g.slices ? 0u : kOobOffset),
                       (uint32_t)min(q0 + u, g.slices - 1) * stride, 0));
    // As in gemm_skinny_body: slices past the last load +0 out of range.
#pragma unroll
    for (int u = 0; u < kBatch; ++u)
#pragma unroll
      for (int f = 0; f < kF; ++f) sum[f] += v[u][f];
  }
  const int es = kExt ? out_bytes(scl.ev.out) : 2;  // bytes per C element
  const __amdgpu_buffer_rsrc_t rsrc_c =
      make_rsrc(reinterpret_cast<uint8_t*>(g.C) + (size_t)n0 * es,
                (uint32_t)(((M - 1) * g.ldc + rows_b) * es));
  auto oob_unless = [](int x, int limit) -> uint32_t {
    return (uint32_t)((limit - 1 - x) >> 31) & kOobOffset;
  };
#pragma unroll
  for (int f = 0; f < kF; ++f) {
    const int row = 16 * m + r16;
    const int col = wave * 16 * kF + 16 * f + 4 * grp;
    const uint32_t base = (uint32_t)((row * g.ldc + col) * es) | oob_unless(row, M);
    if constexpr (kExt) {
      const f32x4& a = sum[f];
      store_out4<kVec8>(scl.ev, a[0], a[1], a[2], a[3], 0, f, rsrc_c, base, col,
                        rows_b);
      continue;
    }
    const u32x2 pk = scl.pack4(sum[f], 0, f);
    const uint32_t lo = pk.x, hi = pk.y;
    if constexpr (kVec8) {
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{lo, hi}, rsrc_c,
                                            base | oob_unless(col, rows_b), 0, 0);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t w = (i < 2 ? lo : hi) >> (16 * (i & 1));
        __builtin_amdgcn_raw_buffer_store_b16(
            (unsigned short)w, rsrc_c,
            (base | oob_unless(col + i, rows_b)) + 2 * i, 0, 0);
      }
    }
  }
}

}  // namespace detail
}  // namespace hipgemm
