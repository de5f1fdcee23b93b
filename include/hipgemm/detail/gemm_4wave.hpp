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
//   * K advances 128 bytes per step (one LDS stage); each of the 16 blocks
//     takes two v_mfma_f32_32x32x64_f8f6f4 per step (K-halves).
//
// Operand registers: four tiles of 64 rows x 128 K-bytes (32 VGPRs each):
// a_lo / a_hi = the wave's A rows 0-63 / 64-127, b_lo / b_hi likewise for B.
// A step runs four quarter-steps Q00, Q01, Q10, Q11; quarter Qij takes the
// 2 x 2 blocks (a_i, b_j), 8 MFMA.  A tile is reloaded for the next step as
// soon as its second use is over:
//   Q00(k): MFMA a_lo x b_lo | read b_hi(k)   | DMA B_lo group, step k+2
//   Q01(k): MFMA a_lo x b_hi | read a_hi(k)   | DMA B_hi group, step k+2
//   Q10(k): MFMA a_hi x b_lo | read a_lo(k+1) | DMA A_hi group, step k+2
//   Q11(k): MFMA a_hi x b_hi | read b_lo(k+1) | DMA A_lo group, step k+3
// LDS holds 2 stages (A 256 x 128 B + B 256 x 128 B each, 128 KiB).  Each
// 64-row sub-buffer group (e.g. "A_lo" = A rows 0-63 and 128-191, the a_lo
// rows of both wave rows) is read in one quarter-step and refilled in the
// next; the refill is read seven quarter-steps later (~1.75 steps, ~3.5K
// cycles of DMA latency slack).  Every quarter-step starts with: wait own
// LDS reads (the group read last quarter is free), wait own DMA up to the
// group read this quarter (vmcnt 24), s_barrier.  Inside a quarter the 8 LDS
// reads go two per MFMA in the first half and the 4 DMA one per MFMA in the
// second half, so the per-CU address unit is never offered more than about
// one 1 KiB DMA per 16 cycles.  DMA issued for steps past the end of K reads
// zeros (every lane out of range); the step count is padded to even.
//
// Global -> LDS: buffer_load_dwordx4 ... lds, 8 rows x 128 B per instruction
// (whole 128-byte lines), 16 instructions per wave per step.  The buffer
// resource of a tile covers only its valid rows, so rows past M (or N) read
// zero; K-chunks past K get an out-of-range offset.  Nothing outside A or B is
// ever addressed.
//
// Epilogue: acc * (scale_a * scale_b) -> bf16 (RNE), staged through LDS so
// that every store instruction writes whole 128-byte lines of C (16 bytes per
// lane, 4 rows x 256 B); 2-byte stores straight from the accumulators when N,
// ldc or C's alignment do not allow 16.  No branches: lanes outside M x N are
// dropped by the buffer range check.
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
  static constexpr int kBM = 256, kBN = 256, kBK = 128, kStages = 2;
  static constexpr int kAStage = kBM * kBK;  // 32 KiB
  static constexpr int kBStage = kBN * kBK;  // 32 KiB
  static constexpr int kABase = 0;
  static constexpr int kBBase = kStages * kAStage;
  static constexpr int kLdsBytes = kStages * (kAStage + kBStage);  // 128 KiB
  static constexpr int kDmaPerStep = 16;  // per wave: 8 for A, 8 for B
};

// sched_group_barrier pattern of one quarter-step: 8 MFMA (0x008); two LDS
// reads (0x100) after each of the first 4, one DMA (0x020) after each of the
// last 4.
__device__ __forceinline__ void quarter_schedule() {
  for (int x = 0; x < 4; ++x) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
  }
  for (int x = 0; x < 4; ++x) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
  }
}

template <bool kVecStore>
__device__ __forceinline__ void gemm_4wave_body(const GemmArgs& g,
                                                lds_u8* lds) {
  using Cfg = Cfg4w;
  constexpr int kDmaPerGroup = 4;  // per wave
  const int lane = lane_id();
  const int wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;

  const int M = g.M, N = g.N, K = g.K;
  const int tiles_m = (M + Cfg::kBM - 1) / Cfg::kBM;
  const int tiles_n = (N + Cfg::kBN - 1) / Cfg::kBN;
  const int tiles = tiles_m * tiles_n;
  const int kt_real = (K + Cfg::kBK - 1) / Cfg::kBK;
  const int kt_pad = (kt_real + 1) & ~1;

  const float sa = g.scale_a ? *g.scale_a : 1.0f;
  const float sb = g.scale_b ? *g.scale_b : 1.0f;
  const float scale = sa * sb;

  // ---- DMA lane geometry: instruction q of wave w covers rows
  // (4q + w) * 8 .. +8; lane l takes row +l/8, slot l%8.  q in {0,1,4,5}
  // lands in rows 0-63 and 128-191 ("lo" group), q in {2,3,6,7} in rows
  // 64-127 and 192-255 ("hi" group). ------------------------------------------
  const int drow = lane >> 3;
  const int dchunk = (lane & 7) ^ slot_xor(8 * (wave & 1) + drow);
  uint32_t voff_a[8], voff_b[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int row = (4 * q + wave) * 8 + drow;
    voff_a[q] = (uint32_t)row * (uint32_t)g.lda + dchunk * 16;
    voff_b[q] = (uint32_t)row * (uint32_t)g.ldb + dchunk * 16;
  }

  // ---- ds_read lane geometry: fragment row lane%32; K-half kh, lane group
  // g = lane/32 and sub-chunk t read K-chunk 4kh + 2g + t. -------------------
  const int rrow = lane & 31;
  const int rslot = (2 * (lane >> 5)) ^ slot_xor(rrow & 15);
  const uint32_t off_a = Cfg::kABase + (wm * 128 + rrow) * Cfg::kBK + rslot * 16;
  const uint32_t off_b = Cfg::kBBase + (wn * 128 + rrow) * Cfg::kBK + rslot * 16;
  // chunk bits (kh, g, t) sit at address bits (6, 5, 4): flip them with XOR.
  const lds_u8* pa[2][2] = {{lds + off_a, lds + (off_a ^ 16u)},
                            {lds + (off_a ^ 64u), lds + (off_a ^ 80u)}};
  const lds_u8* pb[2][2] = {{lds + off_b, lds + (off_b ^ 16u)},
                            {lds + (off_b ^ 64u), lds + (off_b ^ 80u)}};

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

    // DMA of one sub-buffer group of step kb into `stage`: operand op (0 = A,
    // 1 = B), half hi (0 = lo group, 1 = hi group).  4 instructions per wave.
    auto dma_group = [&](int kb, int stage, int op, int hi) {
      uint32_t k0 = (uint32_t)kb * Cfg::kBK;
      // Opaque to the optimiser: keeps the per-step lane masks from being
      // hoisted out of the tile loop (they would pin VGPRs and spill).
      asm volatile("" : "+s"(k0));
      const bool ok = (int)(k0 + dchunk * 16) < K;
#pragma unroll
      for (int qq = 0; qq < kDmaPerGroup; ++qq) {
        const int q = (qq & 1) + 4 * (qq >> 1) + 2 * hi;
        if (op == 0)
          dma16(rsrc_a,
                lds + Cfg::kABase + stage * Cfg::kAStage + (4 * q + wave) * 1024,
                ok ? voff_a[q] : kOobOffset, k0);
        else
          dma16(rsrc_b,
                lds + Cfg::kBBase + stage * Cfg::kBStage + (4 * q + wave) * 1024,
                ok ? voff_b[q] : kOobOffset, k0);
      }
    };

    i32x8 fa[4][2], fb[4][2];  // [32-row fragment][K-half]
    // Register tile (op, hi) of `stage`: fragments 2hi, 2hi+1, both K-halves.
    auto read_tile = [&](int op, int hi, int stage) {
#pragma unroll
      for (int f = 2 * hi; f < 2 * hi + 2; ++f)
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
          if (op == 0) {
            const int o = stage * Cfg::kAStage + f * 32 * Cfg::kBK;
            fa[f][kh] = join(lds_read16(pa[kh][0] + o), lds_read16(pa[kh][1] + o));
          } else {
            const int o = stage * Cfg::kBStage + f * 32 * Cfg::kBK;
            fb[f][kh] = join(lds_read16(pb[kh][0] + o), lds_read16(pb[kh][1] + o));
          }
        }
    };

    f32x16 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};

    // Quarter (qi, qj): blocks i in {2qi, 2qi+1} x j in {2qj, 2qj+1}, K-half
    // major so the two MFMA of one accumulator are 4 apart.
    auto quarter_mfma = [&](int qi, int qj) {
#pragma unroll
      for (int kh = 0; kh < 2; ++kh)
#pragma unroll
        for (int i = 2 * qi; i < 2 * qi + 2; ++i)
#pragma unroll
          for (int j = 2 * qj; j < 2 * qj + 2; ++j)
            acc[i][j] = mfma_32x32x64(fb[j][kh], fa[i][kh], acc[i][j]);
    };

    auto quarter_sync = [&]() {
      wait_lgkmcnt<0>();
      wait_vmcnt<6 * kDmaPerGroup>();
      barrier();
    };

    // Previous tile: all LDS reads done and all stores retired before the
    // stages are overwritten.
    wait_vmcnt<0>();
    barrier();

    // Prologue: steps 0 and 1 in group order A_lo, B_lo, B_hi, A_hi; then
    // a_lo(0), b_lo(0) into registers and the A_lo group of step 2.
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      dma_group(st, st, 0, 0);
      dma_group(st, st, 1, 0);
      dma_group(st, st, 1, 1);
      dma_group(st, st, 0, 1);
    }
    wait_vmcnt<6 * kDmaPerGroup>();
    barrier();
    read_tile(0, 0, 0);
    read_tile(1, 0, 0);
    wait_lgkmcnt<0>();
    barrier();
    dma_group(2, 0, 0, 0);

    for (int kt0 = 0; kt0 < kt_pad; kt0 += 2) {
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int kt = kt0 + s;
        quarter_sync();  // Q00
        quarter_mfma(0, 0);
        read_tile(1, 1, s);
        dma_group(kt + 2, s, 1, 0);
        quarter_schedule();
        quarter_sync();  // Q01
        quarter_mfma(0, 1);
        read_tile(0, 1, s);
        dma_group(kt + 2, s, 1, 1);
        quarter_schedule();
        quarter_sync();  // Q10
        quarter_mfma(1, 0);
        read_tile(0, 0, s ^ 1);
        dma_group(kt + 2, s, 0, 1);
        quarter_schedule();
        quarter_sync();  // Q11
        quarter_mfma(1, 1);
        read_tile(1, 0, s ^ 1);
        dma_group(kt + 3, s ^ 1, 0, 0);
        quarter_schedule();
      }
    }
    wait_vmcnt<0>();
    wait_lgkmcnt<0>();
    // The accumulators are read below by explicit v_accvgpr_read (acc_read),
    // which the compiler's hazard tracking does not see: give the last MFMA
    // its result latency here (a 16-pass XDL write needs 19 wait states
    // before a VALU read; 32 are inserted).
    mfma_drain();

    // ---- epilogue --------------------------------------------------------
    // acc[i][j] holds D = B_blk . A_blk^T, i.e. C^T for the 32x32 block:
    // lane l, register r -> C row (l % 32), C column 8*(r/4) + 4*(l/32) + r%4,
    // so each lane holds 4 consecutive bf16 (8 bytes) per (i, j, r/4).
    // Multiplying by a scale of 1.0 is exact (NaN and -0 included), so every
    // call takes the same path.
    auto cvt4 = [&](const f32x16& v, int q) {
      return u32x2{pack_bf16x2(acc_read(v[4 * q + 0]) * scale,
                               acc_read(v[4 * q + 1]) * scale),
                   pack_bf16x2(acc_read(v[4 * q + 2]) * scale,
                               acc_read(v[4 * q + 3]) * scale)};
    };
    // Out-of-range bit for "x < limit" as plain arithmetic (no lane masks,
    // which would pin scalar register pairs): kOobOffset when x >= limit.
    auto oob_unless = [](int x, int limit) -> uint32_t {
      return (uint32_t)((limit - 1 - x) >> 31) & kOobOffset;
    };
    // Every store is a buffer store over this tile's window of C; a lane
    // whose row or columns fall outside M x N gets an out-of-range offset and
    // its write is dropped by the hardware range check -- no branches.
    // Lane-derived epilogue values hang off an opaque copy of the lane id so
    // the optimiser cannot hoist them out of the tile loop, where they would
    // stay live through the K loop and spill.
    int elane = lane;
    asm volatile("" : "+v"(elane));
    const int rows_c = min(Cfg::kBM, M - tc.m * Cfg::kBM);
    const __amdgpu_buffer_rsrc_t rsrc_c = make_rsrc(
        g.C + (size_t)tc.m * Cfg::kBM * g.ldc + (size_t)tc.n * Cfg::kBN,
        (uint32_t)(((rows_c - 1) * g.ldc + Cfg::kBN) * 2));
    const int rows_left = M - tc.m * Cfg::kBM - wm * 128;  // from wave row 0
    const int cols_left = N - tc.n * Cfg::kBN - wn * 128;  // from wave col 0

    if constexpr (kVecStore) {
      // Through LDS: each wave stages its 128 x 128 bf16 quadrant (32 KiB) in
      // its own quarter of the now idle stage buffers, then stores 16 bytes
      // per lane row-major -- 4 rows x 256 B per instruction, whole 128-byte
      // lines.  Staging layout: row r at 256 r, 16-byte chunk k of the row
      // at slot k ^ (r % 16): conflict-free for the 8-byte writes (16 rows,
      // one chunk) and for the 16-byte reads (one row, 16 chunks).
      wait_vmcnt<0>();   // no DMA (real or padding) still landing in LDS
      barrier();         // every wave is done reading the stages
      lds_u8* stage_c = lds + wave * (128 * 256);
      const uint32_t wlane = (elane & 31) * 256 + 8 * (elane >> 5);
      const uint32_t xr16 = (elane & 15) * 16;
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            lds_write8(stage_c + wlane + 32 * i * 256 + (((4 * j + q) * 16) ^ xr16),
                       cvt4(acc[i][j], q));
          sched_fence();  // bound the live range: one block at a time
        }
      wait_lgkmcnt<0>();  // own quadrant only: no cross-wave hand-off
      // read: lane l takes row 4p + l/16, chunk l % 16
      const int rsub = elane >> 4, chunk = elane & 15;
      const uint32_t rlane_base = rsub * 256;
      uint32_t rx[4];
#pragma unroll
      for (int x = 0; x < 4; ++x)
        rx[x] = rlane_base + ((chunk ^ ((4 * x + rsub) & 15)) * 16);
      const uint32_t vcol = (uint32_t)((rsub * g.ldc + wn * 128 + 8 * chunk) * 2);
      const uint32_t col_oob = oob_unless(8 * chunk, cols_left);
#pragma unroll
      for (int p0 = 0; p0 < 32; p0 += 8) {
        i32x4 v[8];
#pragma unroll
        for (int p = p0; p < p0 + 8; ++p)
          v[p - p0] = lds_read16(stage_c + rx[p & 3] + 1024 * p);
#pragma unroll
        for (int p = p0; p < p0 + 8; ++p) {
          int row4 = 4 * p;
          asm volatile("" : "+s"(row4));  // recompute per store, never hoist
          const int srow =
              __builtin_amdgcn_readfirstlane((wm * 128 + row4) * g.ldc * 2);
          __builtin_amdgcn_raw_buffer_store_b128(
              v[p - p0], rsrc_c,
              vcol | col_oob | oob_unless(row4 + rsub, rows_left), srow, 0);
        }
        sched_fence();  // at most 8 rows (32 VGPRs) in flight
      }
    } else {
      // N, ldc or C's alignment rule out 16-byte stores: 2-byte stores
      // straight from the accumulators, lane masks as out-of-range offsets.
      const uint32_t vlane =
          (uint32_t)(((elane & 31) * g.ldc + wn * 128 + 4 * (elane >> 5)) * 2);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int srow =
            __builtin_amdgcn_readfirstlane((wm * 128 + 32 * i) * g.ldc * 2);
        const uint32_t vrow = vlane | oob_unless(32 * i + (elane & 31), rows_left);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const int c = 32 * j + 8 * q + 4 * (elane >> 5);
            const u32x2 v = cvt4(acc[i][j], q);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const uint32_t w = (r < 2 ? v.x : v.y) >> (16 * (r & 1));
              __builtin_amdgcn_raw_buffer_store_b16(
                  (unsigned short)w, rsrc_c,
                  (vrow | oob_unless(c + r, cols_left)) +
                      (32 * j + 8 * q + r) * 2,
                  srow, 0);
            }
          }
          sched_fence();  // bound the live range: one block at a time
        }
      }
    }
  }
  wait_vmcnt<0>();
}

}  // namespace detail
}  // namespace hipgemm
