// hipgemm -- 4-wave FP8 GEMM main body (gfx950).
//
// C[M x N] (bf16) = scale_a * scale_b * A[M x K] . B_T[N x K]^T, e4m3 inputs,
// fp32 accumulation.  Reference counterpart: fp8_gemm_4wave_256x256x128,
// fp8_4wave.hpp:334-567 (same interface and block shape, different design).
//
// Work decomposition
//   * One workgroup = 256 threads = 4 waves (one per SIMD) = one 256 x 256
//     output tile at a time; a grid smaller than the tile count loops over
//     tiles, so any grid size >= 1 is correct.
//   * Wave w owns the contiguous 128 x 128 quadrant (w / 2, w % 2) of the tile
//     as 4 x 4 blocks of 32 x 32 fp32 accumulators (256 AGPRs per lane).
//   * K advances 64 bytes per step: one v_mfma_f32_32x32x64_f8f6f4 per block,
//     16 per wave per step.
//
// Pipeline (STAGES = 4 LDS buffers of 256 x 64 B for A and for B, 128 KiB)
//   step kt, LDS stage s = kt % 4, register set p = kt % 2:
//     wait own DMA of step kt+1 (vmcnt), wait own LDS reads of step kt
//     (lgkmcnt), s_barrier                      -- the only barrier per step
//     DMA step kt+4 into stage s                -- 3 steps of latency slack
//     16 MFMA on register set p, interleaved with the 16 ds_read_b128 that
//     fill set p^1 with step kt+1 from stage (kt+1) % 4.
//   Steps past the end of K read zeros (every lane out of range), so the K
//   loop runs a multiple of 4 steps with no branches inside the unrolled body.
//
// Global -> LDS: buffer_load_dwordx4 ... lds, 16 rows x 64 B per instruction,
// 8 instructions per wave per step.  The buffer resource of a tile covers only
// its valid rows, so rows past M (or N) read zero; K-chunks past K are given
// an out-of-range offset.  Nothing outside A or B is ever addressed.
//
// Epilogue: acc * (scale_a * scale_b) -> bf16 (RNE), one 8-byte store of 4
// consecutive columns per lane per (block, 8-row group); per-lane masks keep
// every write inside M x N.
#pragma once

#include "arch.hpp"
#include "layout.hpp"

namespace hipgemm {
namespace detail {

struct GemmArgs {
  const uint8_t* A;      // M x K e4m3, row stride lda bytes
  const uint8_t* B;      // N x K e4m3 (B_T), row stride ldb bytes
  uint16_t* C;           // M x N bf16, row stride ldc elements
  const float* scale_a;  // device scalar, nullptr = 1.0
  const float* scale_b;  // device scalar, nullptr = 1.0
  int M, N, K;
  int lda, ldb, ldc;
  int group_m;
};

__host__ __device__ constexpr int default_group_m(int tiles_m, int tiles_n) {
  // 32 CUs per XCD: make the 32 co-resident tiles of an XCD about 4 x 8.
  const int cols = tiles_n < 8 ? tiles_n : 8;
  int g = (32 + cols - 1) / (cols > 0 ? cols : 1);
  if (g > tiles_m) g = tiles_m;
  return g < 1 ? 1 : g;
}

struct Cfg4w {
  static constexpr int kThreads = 256;
  static constexpr int kBM = 256, kBN = 256, kBK = 64, kStages = 4;
  static constexpr int kAStage = kBM * kBK;  // 16 KiB
  static constexpr int kBStage = kBN * kBK;  // 16 KiB
  static constexpr int kABase = 0;
  static constexpr int kBBase = kStages * kAStage;
  static constexpr int kLdsBytes = kStages * (kAStage + kBStage);  // 128 KiB
  static constexpr int kDmaPerStep = 8;  // per wave: 4 for A, 4 for B
};

template <bool kVecStore>
__device__ __forceinline__ void gemm_4wave_body(const GemmArgs& g,
                                                lds_u8* lds) {
  using Cfg = Cfg4w;
  constexpr int S = Cfg::kStages;
  const int lane = lane_id();
  const int wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;

  const int M = g.M, N = g.N, K = g.K;
  const int tiles_m = (M + Cfg::kBM - 1) / Cfg::kBM;
  const int tiles_n = (N + Cfg::kBN - 1) / Cfg::kBN;
  const int tiles = tiles_m * tiles_n;
  const int kt_real = (K + Cfg::kBK - 1) / Cfg::kBK;
  const int kt_pad = (kt_real + S - 1) / S * S;

  const float sa = g.scale_a ? *g.scale_a : 1.0f;
  const float sb = g.scale_b ? *g.scale_b : 1.0f;
  const float scale = sa * sb;

  // ---- DMA lane geometry: 16 rows x 4 slots per instruction -------------
  const int drow = lane >> 2;
  const int dchunk = (lane & 3) ^ slot_xor(drow);
  uint32_t voff_a[4], voff_b[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = (4 * q + wave) * 16 + drow;
    voff_a[q] = (uint32_t)row * (uint32_t)g.lda + dchunk * 16;
    voff_b[q] = (uint32_t)row * (uint32_t)g.ldb + dchunk * 16;
  }

  // ---- ds_read lane geometry: fragment row lane%32, K-half lane/32 -------
  const int rrow = lane & 31;
  const int rslot = (2 * (lane >> 5)) ^ slot_xor(rrow & 15);
  const uint32_t off_a = Cfg::kABase + (wm * 128 + rrow) * Cfg::kBK + rslot * 16;
  const uint32_t off_b = Cfg::kBBase + (wn * 128 + rrow) * Cfg::kBK + rslot * 16;
  const lds_u8* pa0 = lds + off_a;
  const lds_u8* pa1 = lds + (off_a ^ 16u);
  const lds_u8* pb0 = lds + off_b;
  const lds_u8* pb1 = lds + (off_b ^ 16u);

  const int grid = gridDim.x;
  for (int t = xcd_contiguous(blockIdx.x, grid); t < tiles; t += grid) {
    const TileCoord tc = grouped_tile(t, tiles_m, tiles_n, g.group_m);
    const int rows_a = min(Cfg::kBM, M - tc.m * Cfg::kBM);
    const int rows_b = min(Cfg::kBN, N - tc.n * Cfg::kBN);
    const __amdgpu_buffer_rsrc_t rsrc_a =
        make_rsrc(g.A + (size_t)tc.m * Cfg::kBM * g.lda,
                  (uint32_t)rows_a * (uint32_t)g.lda);
    const __amdgpu_buffer_rsrc_t rsrc_b =
        make_rsrc(g.B + (size_t)tc.n * Cfg::kBN * g.ldb,
                  (uint32_t)rows_b * (uint32_t)g.ldb);

    auto issue_dma = [&](int kb, int stage) {
      uint32_t k0 = (uint32_t)kb * Cfg::kBK;
      // Opaque to the optimiser: keeps the per-step lane masks from being
      // hoisted out of the tile loop (they would pin 32 VGPRs and spill).
      asm volatile("" : "+s"(k0));
      const bool ok = (int)(k0 + dchunk * 16) < K;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        dma16(rsrc_a,
              lds + Cfg::kABase + stage * Cfg::kAStage + (4 * q + wave) * 1024,
              ok ? voff_a[q] : kOobOffset, k0);
#pragma unroll
      for (int q = 0; q < 4; ++q)
        dma16(rsrc_b,
              lds + Cfg::kBBase + stage * Cfg::kBStage + (4 * q + wave) * 1024,
              ok ? voff_b[q] : kOobOffset, k0);
    };

    i32x8 fa[2][4], fb[2][4];
    auto read_operands = [&](int set, int stage) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int o = stage * Cfg::kAStage + i * 32 * Cfg::kBK;
        fa[set][i] = join(lds_read16(pa0 + o), lds_read16(pa1 + o));
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int o = stage * Cfg::kBStage + j * 32 * Cfg::kBK;
        fb[set][j] = join(lds_read16(pb0 + o), lds_read16(pb1 + o));
      }
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

    // Previous tile: all LDS reads done and all stores retired before the
    // stages are overwritten.
    wait_vmcnt<0>();
    barrier();

    // Prologue: steps 0..S-1 in flight, step 0 in registers.
#pragma unroll
    for (int p = 0; p < S; ++p) issue_dma(p, p);
    wait_vmcnt<(S - 1) * Cfg::kDmaPerStep>();
    barrier();
    read_operands(0, 0);

    for (int kt0 = 0; kt0 < kt_pad; kt0 += S) {
#pragma unroll
      for (int s = 0; s < S; ++s) {
        const int p = s & 1;
        wait_vmcnt<(S - 2) * Cfg::kDmaPerStep>();
        wait_lgkmcnt<0>();
        barrier();
        issue_dma(kt0 + s + S, s);
        read_operands(p ^ 1, (s + 1) % S);
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            acc[i][j] = mfma_32x32x64(fb[p][j], fa[p][i], acc[i][j]);
        // Issue order: DMA first, then one LDS read per MFMA.
#pragma unroll
        for (int x = 0; x < 8; ++x) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
#pragma unroll
        for (int x = 0; x < 16; ++x) {
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        }
      }
    }
    wait_vmcnt<0>();
    wait_lgkmcnt<0>();

    // ---- epilogue --------------------------------------------------------
    // acc[i][j] holds D = B_blk . A_blk^T, i.e. C^T for the 32x32 block:
    // lane l, register r -> C row (l % 32), C column 8*(r/4) + 4*(l/32) + r%4.
    const int m_lane = tc.m * Cfg::kBM + wm * 128 + (lane & 31);
    const int n_lane = tc.n * Cfg::kBN + wn * 128 + 4 * (lane >> 5);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int m = m_lane + 32 * i;
      if (m < M) {
        uint16_t* crow = g.C + (size_t)m * g.ldc;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int n0 = n_lane + 32 * j + 8 * q;
            const float v0 = acc[i][j][4 * q + 0] * scale;
            const float v1 = acc[i][j][4 * q + 1] * scale;
            const float v2 = acc[i][j][4 * q + 2] * scale;
            const float v3 = acc[i][j][4 * q + 3] * scale;
            const uint32_t lo = pack_bf16x2(v0, v1), hi = pack_bf16x2(v2, v3);
            if (kVecStore && n0 + 3 < N) {
              *reinterpret_cast<u32x2*>(crow + n0) = u32x2{lo, hi};
            } else {
              if (n0 + 0 < N) crow[n0 + 0] = (uint16_t)lo;
              if (n0 + 1 < N) crow[n0 + 1] = (uint16_t)(lo >> 16);
              if (n0 + 2 < N) crow[n0 + 2] = (uint16_t)hi;
              if (n0 + 3 < N) crow[n0 + 3] = (uint16_t)(hi >> 16);
            }
          }
        }
      }
    }
  }
  wait_vmcnt<0>();
}

}  // namespace detail
}  // namespace hipgemm
