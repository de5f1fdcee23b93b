// hipgemm -- 8-wave FP8 GEMM (gfx950): two waves per SIMD, ping-pong.
//
// Same product and tile as the 4-wave kernel (gemm_4wave.hpp): one 256 x 256
// output tile per workgroup at a time, K advancing 128 bytes per step,
// operands DMA'd (buffer_load_dwordx4 ... lds) into 128-byte LDS rows with
// the slot_xor swizzle, 16x16x128 MFMA, RNE bf16 epilogue with whole-line
// stores.  What differs is the warp-tile schedule:
//   * 512 threads = 8 waves in two groups; wave w runs on SIMD w % 4, so
//     every SIMD holds one wave of each group.  Group g = w / 4 owns rows
//     128 g .. +127 of the tile; wave w owns columns 64 (w % 4) .. +63 of
//     those: 8 x 4 blocks of 16 x 16, 128 AGPRs.  One step's operands (A 128
//     rows + B 64 rows, 96 VGPRs) fit once per wave.
//   * The groups alternate, half a step apart, between a memory phase (read
//     the step's operands from LDS, with 8 DMAs of later steps in between)
//     and a compute phase (32 MFMAs at raised wave priority, nothing else),
//     every phase closed by one workgroup barrier.  Phase 2j: group 0 reads step j while group 1
//     computes step j - 1; phase 2j + 1: group 0 computes step j while group
//     1 reads it.  Each SIMD's MFMA pipe thus alternates between its two
//     waves and never waits for an LDS read.
//   * LDS: A in 2 stages, B in 3 (160 KiB).  Each operand block is written
//     once its last reader has passed a barrier, by the group in its memory
//     phase (32 KiB per group and step):
//       A rows 128-255 of step j + 1  group 0, phase 2j      (read at 2j + 3)
//       B rows 128-255 of step j + 2  group 0, phase 2j      (read at 2j + 4)
//       A rows 0-127 of step j + 2    group 1, phase 2j + 1  (read at 2j + 4)
//       B rows 0-127 of step j + 2    group 1, phase 2j + 1  (read at 2j + 4)
//     The issuing wave waits for its own DMA (vmcnt, in issue order) at the
//     end of the phase before the first reader's.  A CU's vector memory path
//     takes ~15-25 cycles per 1 KiB DMA instruction, so a DMA issued between
//     MFMAs stalls the MFMA stream (measured: ~90 cycles each); the memory
//     phase, which waits for the other group's MFMAs anyway, absorbs them.
//   * Tiles: persistent grid, each XCD's workgroups striding through one
//     contiguous band of tiles (tile_walk).  Each tile starts with a
//     full-workgroup prologue (steps 0 and 1, B rows 0-127 of step 2) and
//     ends with both groups' epilogues; the C staging of the epilogue reuses
//     the A stages.
// No reference counterpart (the reference has only 4-wave kernels,
// fp8_4wave.hpp:334-567 and :594-708).
#pragma once

#include <type_traits>

#include "arch.hpp"
#include "gemm_4wave.hpp"
#include "layout.hpp"

namespace hipgemm {
namespace detail {

struct Cfg8w {
  static constexpr int kThreads = 512;
  static constexpr int kBM = 256, kBN = 256, kBK = 128;
  static constexpr int kAStage = kBM * kBK;  // 32 KiB
  static constexpr int kBStage = kBN * kBK;  // 32 KiB
  static constexpr int kAStages = 2, kBStages = 3;
  static constexpr int kABase = 0;
  static constexpr int kBBase = kAStages * kAStage;
  static constexpr int kLdsBytes = kBBase + kBStages * kBStage;  // 160 KiB
  static constexpr int kStoreStage = 32 * 128;  // 32 rows x 64 bf16 per wave
  static constexpr int kStoreBase = kABase;     // after the K loop only
  // DMA instructions (8 rows x 128 B each) per wave and memory phase: 4 of
  // A (one half of its rows) and 4 of B (one half).
  static constexpr int kDmaPhase = 8;
};
static_assert(Cfg8w::kLdsBytes == 160 * 1024, "LDS budget");
static_assert(8 * Cfg8w::kStoreStage <= Cfg8w::kAStages * Cfg8w::kAStage,
              "epilogue staging fits the A stages");

// kExt: the extended epilogue of epilogue.hpp (row / column scales, bias,
// activation, fp16 output) from g.epi.
// kAct / kOut (kExt only): as for gemm_4wave_body.
template <bool kVecStore, bool kExt = false, int kFmt = 0, int kAct = kActNone,
          int kOut = kOutBf16>
__device__ __forceinline__ void gemm_8wave_body(const GemmArgs& g, lds_u8* lds) {
  using Cfg = Cfg8w;
  const int lane = lane_id();
  const int wave = wave_id();  // 0..7
  const int grp = wave >> 2, wn = wave & 3;
  const int wm = grp;
  const int M = g.M, N = g.N, K = g.K;
  const int tiles_m = (M + Cfg::kBM - 1) / Cfg::kBM;
  const int tiles_n = (N + Cfg::kBN - 1) / Cfg::kBN;
  const int tiles = tiles_m * tiles_n;
  const int kt = max(1, (K + Cfg::kBK - 1) / Cfg::kBK);
  const int workers = g.workers > 0 ? min((int)gridDim.x, g.workers)
                                    : (int)gridDim.x;
  if ((int)blockIdx.x >= workers) return;

  const float sa = g.scale_a ? *g.scale_a : 1.0f;
  const float sb = g.scale_b ? *g.scale_b : 1.0f;
  const float scale = sa * sb;

  // DMA lane geometry: instruction q covers operand rows 8q .. 8q + 7; lane l
  // takes row 8q + l / 8 and LDS slot l % 8.  Every instruction a wave issues
  // has q = wave (mod 2), so the swizzled source chunk is one per lane.
  const int drow = lane >> 3;
  const int dchunk = (lane & 7) ^ slot_xor(8 * (wave & 1) + drow);
  // Per-lane part of every DMA offset; the row-group part 8 q ld is a
  // scalar added per instruction (kept opaque so that the compiler does not
  // precompute one VGPR per instruction).
  const uint32_t vbase_a = (uint32_t)drow * (uint32_t)g.lda + (uint32_t)dchunk * 16;
  const uint32_t vbase_b = (uint32_t)drow * (uint32_t)g.ldb + (uint32_t)dchunk * 16;

  // ds_read: fragment row lane%16; lane group lane/16 reads K-chunks 2g, 2g+1.
  const int r16 = lane & 15;
  const int rslot = (2 * (lane >> 4)) ^ slot_xor(r16);
  const uint32_t off_a = Cfg::kABase + (grp * 128 + r16) * Cfg::kBK + rslot * 16;
  const uint32_t off_b = Cfg::kBBase + (wn * 64 + r16) * Cfg::kBK + rslot * 16;

  i32x8 fa[8], fb[4];
  f32x4 acc[8][4];

  auto oob_unless = [](int x, int limit) -> uint32_t {
    return (uint32_t)((limit - 1 - x) >> 31) & kOobOffset;
  };

  const TileWalk walk = tile_walk(blockIdx.x, workers, tiles);
  for (int t = walk.first; t < walk.end; t += walk.stride) {
    const TileSrc src = tile_src(g, t, walk.end, tiles_m, tiles_n);
    // K-step kb's bytes of this lane's chunk exist (wave-uniform per step).
    auto k_ok = [&](int kb) {
      uint32_t k0 = (uint32_t)kb * Cfg::kBK;
      asm volatile("" : "+s"(k0));
      return (int)(k0 + dchunk * 16) < K;
    };
    // DMA instruction q of operand op (0 = A, 1 = B) for step kb.
    auto dma = [&](int op, uint32_t lds_off, int q, int kb, bool ok) {
      uint32_t ld = (uint32_t)(op == 0 ? g.lda : g.ldb);
      asm volatile("" : "+s"(ld));
      const uint32_t vo = (op == 0 ? vbase_a : vbase_b) + (uint32_t)(8 * q) * ld;
      dma16(op == 0 ? src.a : src.b, lds + lds_off + q * 1024,
            ok ? vo : kOobOffset, (uint32_t)kb * Cfg::kBK);
    };
    auto a_stage = [](int kb) { return Cfg::kABase + (kb & 1) * Cfg::kAStage; };
    auto b_stage = [](int kb) { return Cfg::kBBase + (kb % 3) * Cfg::kBStage; };

    // ---- prologue: steps 0 and 1 ------------------------------------------
    wait_lgkmcnt<0>();  // previous tile's epilogue reads of the A stages
    barrier();
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const bool ok = k_ok(kb);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int q = wave + 8 * i;
        dma(0, a_stage(kb), q, kb, ok);
        dma(1, b_stage(kb), q, kb, ok);
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{};
    wait_vmcnt<0>();
    barrier();
    if (grp == 1) barrier();  // group 1 starts half a step later

    int bs = 0;  // B stage of step j (j % 3)
    // Step j's memory phase fetches steps j + 1 and j + 2.  Up to j_edge
    // those are whole steps of the tile (below kt_full = K / 128) and the
    // DMAs take the lane offsets as they are; from there (the step K ends
    // inside, steps past the end) each lane's chunk is checked against K
    // (a VALU select per DMA, which in every step cost the 4-wave schedule
    // 2-4 %).
    const int kt_full = K / Cfg::kBK;
    const int j_edge = min(kt, max(0, kt_full - 2));
    auto step = [&](int j, auto edge) {
      constexpr bool kEdge = decltype(edge)::value;
      // ---- memory phase of step j: LDS -> registers and 8 DMAs ------------
      // Group 0: A rows 128-255 of step j + 1 (into the stage of step j - 1,
      // last read by group 1 in phase 2j - 1) and B rows 128-255 of step
      // j + 2.  Group 1: A rows 0-127 of step j + 2 (into the stage of step
      // j, read by group 0 in phase 2j) and B rows 0-127 of step j + 2.  B
      // of step j + 2 goes into the stage of step j - 1.  Steps past the end
      // are fetched as zeros (out-of-range offsets, no memory traffic), which
      // keeps every wait count exact.  One DMA after every 3 ds_reads: a
      // wave issues in order, so alternating keeps both the LDS and the
      // vector memory path busy instead of one after the other.
      const uint32_t pa = off_a + (j & 1) * Cfg::kAStage;
      const uint32_t pb = off_b + bs * Cfg::kBStage;
      const int kba = grp == 0 ? j + 1 : j + 2, kbb = j + 2;
      const bool oka = !kEdge || k_ok(kba), okb = !kEdge || k_ok(kbb);
      const uint32_t dsta = grp == 0 ? a_stage(j + 1) : a_stage(j);
      const uint32_t dstb = Cfg::kBBase + (bs == 0 ? 2 : bs - 1) * Cfg::kBStage;
      const int q0 = (grp == 0 ? 16 : 0) + wn;
      i32x4 ra[8][2], rb[4][2];
      auto rd = [&](int k) {
        if (k < 16) {
          const uint32_t p = pa + (k / 2) * 16 * Cfg::kBK;
          ra[k / 2][k % 2] = lds_read16(lds + ((k % 2) ? (p ^ 16u) : p));
        } else {
          const int kk = k - 16;
          const uint32_t p = pb + (kk / 2) * 16 * Cfg::kBK;
          rb[kk / 2][kk % 2] = lds_read16(lds + ((kk % 2) ? (p ^ 16u) : p));
        }
      };
      auto dm = [&](int s) {
        if (s < 4) dma(0, dsta, q0 + 4 * s, kba, oka);
        else dma(1, dstb, q0 + 4 * (s - 4), kbb, okb);
      };
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        rd(3 * s); rd(3 * s + 1); rd(3 * s + 2);
        dm(s);
        sched_fence();
      }
#pragma unroll
      for (int f = 0; f < 8; ++f) fa[f] = join(ra[f][0], ra[f][1]);
#pragma unroll
      for (int f = 0; f < 4; ++f) fb[f] = join(rb[f][0], rb[f][1]);
      wait_lgkmcnt<0>();
      // Group 0: its A rows of step j (issued in its previous memory phase)
      // landed for group 1's next phase; newer: B of step j + 1, then this
      // phase's 8.  Group 1: its blocks of step j + 1 landed for group 0's
      // next phase; newer: this phase's 8.
      if (grp == 0) wait_vmcnt<Cfg::kDmaPhase + 4>(); else wait_vmcnt<Cfg::kDmaPhase>();
      barrier();
      // ---- compute phase of step j: 32 MFMAs -------------------------------
      __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int m = 0; m < 32; ++m)
        acc[m / 4][m % 4] = mfma_16x16x128<fmt_b(kFmt), fmt_a(kFmt)>(
            fb[m % 4], fa[m / 4], acc[m / 4][m % 4]);
      __builtin_amdgcn_s_setprio(0);
      // Group 0: its B rows of step j + 1 landed for its own next memory
      // phase; newer: this step's 8.  At the last step, all DMAs of both
      // groups (the epilogue reuses the A stages).
      int jl = j + 1;
      asm volatile("" : "+s"(jl));  // no peeled copy of the last step
      if (jl == kt)
        wait_vmcnt<0>();
      else if (grp == 0)
        wait_vmcnt<Cfg::kDmaPhase>();
      barrier();
      bs = bs == 2 ? 0 : bs + 1;
    };
    int j = 0;
    for (; j < j_edge; ++j) step(j, std::false_type{});
    for (; j < kt; ++j) step(j, std::true_type{});
    if (grp == 0) barrier();  // group 1's last compute phase
    mfma_drain();

    // ---- epilogue: 32 rows at a time through the wave's own 4 KiB --------
    int elane = lane;
    asm volatile("" : "+v"(elane));
    const TileCoord tc = grouped_tile_u(t, tiles_m, tiles_n, g.group_m);
    const int rows_c = min(Cfg::kBM, M - tc.m * Cfg::kBM);
    const __amdgpu_buffer_rsrc_t rsrc_c = make_rsrc(
        g.C + (size_t)tc.m * Cfg::kBM * g.ldc + (size_t)tc.n * Cfg::kBN,
        (uint32_t)(((rows_c - 1) * g.ldc + Cfg::kBN) * 2));
    const int rows_left = M - tc.m * Cfg::kBM - wm * 128;
    const int cols_left = N - tc.n * Cfg::kBN - wn * 64;
    // kExt: the vectors are loaded here (there is no free LDS to stage
    // them in); waiting for them also waits for the next tile's first DMAs.
    EpiVec<8, 4> ev;
    if constexpr (kExt) {
      ev.load(g.epi, M, N, tc.m * Cfg::kBM + wm * 128, tc.n * Cfg::kBN + wn * 64,
              scale, elane);
      wait_vmcnt<0>();
    }
    // The epilogue proper.
    auto store_tile = [&]() {
    // block (bi, bj) of the wave's 8 x 4, scaled and rounded
    auto cvt = [&](int bi, int bj) {
      const f32x4& v = acc[bi][bj];
      if constexpr (kExt)
        return ev.template pack4<kAct, kOut>(acc_read(v[0]), acc_read(v[1]),
                                               acc_read(v[2]), acc_read(v[3]),
                                               bi, bj);
      else
        return u32x2{pack_bf16x2(acc_read(v[0]) * scale, acc_read(v[1]) * scale),
                     pack_bf16x2(acc_read(v[2]) * scale, acc_read(v[3]) * scale)};
    };
    if constexpr (kVecStore) {
      // Staging: row r (0..31) at 128 r; 8-byte piece x (0..15) at slot
      // x ^ (r % 16), so that the 16 lanes of one piece index (16 rows) in
      // a write instruction cover 16 distinct slots: rocprof reads no bank
      // conflict (x ^ 2((r / 2) % 8), used before, cost 4 conflict cycles
      // per write).  Chunk c of row r (pieces 2c, 2c + 1) is the 16-byte
      // unit ((2c) ^ (r % 16)) / 2, its halves swapped on odd rows.
      lds_u8* stg = lds + Cfg::kStoreBase + wave * Cfg::kStoreStage;
      const int wr = elane & 15, wg = elane >> 4;
      const int rsub = elane >> 3, chunk = elane & 7;  // store: 8 rows x 128 B
      const uint32_t vcol = (uint32_t)((rsub * g.ldc + wn * 64 + 8 * chunk) * 2);
      const uint32_t col_oob = oob_unless(8 * chunk, cols_left);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
          const int r = 16 * ii + wr;
#pragma unroll
          for (int j = 0; j < 4; ++j)
            lds_write8(stg + r * 128 + (((4 * j + wg) ^ (r & 15)) * 8),
                       cvt(2 * c + ii, j));
          sched_fence();
        }
        compiler_fence();
        i32x4 v[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const int r = 8 * p + rsub;
          v[p] = lds_read16(stg + r * 128 + ((((2 * chunk) ^ (r & 15)) >> 1) * 16));
          if (r & 1) v[p] = i32x4{v[p][2], v[p][3], v[p][0], v[p][1]};
        }
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          int row8 = 32 * c + 8 * p;
          asm volatile("" : "+s"(row8));
          const int srow =
              __builtin_amdgcn_readfirstlane((wm * 128 + row8) * g.ldc * 2);
          store_b128<kStoreC>(
              v[p], rsrc_c, vcol | col_oob | oob_unless(row8 + rsub, rows_left),
              srow);
        }
        compiler_fence();
        sched_fence();
      }
    } else {
      const uint32_t vlane =
          (uint32_t)(((elane & 15) * g.ldc + wn * 64 + 4 * (elane >> 4)) * 2);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int srow =
            __builtin_amdgcn_readfirstlane((wm * 128 + 16 * i) * g.ldc * 2);
        const uint32_t vrow = vlane | oob_unless(16 * i + (elane & 15), rows_left);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int col = 16 * j + 4 * (elane >> 4);
          const u32x2 v = cvt(i, j);
#pragma unroll
          for (int q = 0; q < 4; ++q) {
            const uint32_t w = (q < 2 ? v.x : v.y) >> (16 * (q & 1));
            __builtin_amdgcn_raw_buffer_store_b16(
                (unsigned short)w, rsrc_c,
                (vrow | oob_unless(col + q, cols_left)) + (16 * j + q) * 2, srow, kStoreCPart);
          }
          sched_fence();
        }
      }
    }
    };  // store_tile
    store_tile();
  }
  wait_vmcnt<0>();
}

}  // namespace detail
}  // namespace hipgemm
