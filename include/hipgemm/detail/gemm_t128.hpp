// hipgemm -- 128 x 128-tile FP8 GEMM (gfx950), for grids the 256 x 256
// tiles leave underfilled.
//
// C[M x N] = scale_a * scale_b * A[M x K] . B_T[N x K]^T, the same contract
// and the same GemmArgs as the 4-wave schedule (gemm_4wave.hpp).  A 256 x 256
// tile per workgroup leaves most CUs idle when M x N has few tiles (2048^3:
// 64 tiles for 256 CUs) or a short last round (4000 x 5000: 320 tiles = 1.25
// rounds); a 128 x 128 tile quarters the work per workgroup.  No reference
// counterpart: fp8_4wave.hpp:334-567 has 256 x 256 tiles only.
//
// Work decomposition
//   * One workgroup = 4 waves (one per SIMD), persistent over the tiles
//     (tile_walk / grouped_tile, layout.hpp).  Wave w owns the 64 x 64
//     quadrant (w / 2, w % 2) of a tile as 4 x 4 blocks of 16 x 16
//     (v_mfma_f32_16x16x128_f8f6f4, 16 per 128-byte K-step, 64 AGPRs).
//   * Per K-step a wave reads 4 A and 4 B fragments (8 KiB each) from LDS:
//     the 64 x 64 wave tile reads as many LDS bytes per MFMA as the LDS can
//     serve at the MFMA rate, so the fragments of step k + 1 are read while
//     the MFMA of step k run (two register sets).
//
// Pipeline: kStages LDS stages of 128 A rows + 128 B rows x 128 bytes (32
// KiB each), DMA'd (buffer_load_dwordx4 ... lds, 4 + 4 instructions per wave
// per step) kStages - 1 steps ahead.  Iteration k: wait for the wave's own
// DMA of step k + 1, barrier (every wave's part of step k + 1 landed, every
// wave done with the stage of step k - 1), DMA of step k + kStages - 1 into
// that stage, LDS reads of step k + 1, MFMA of step k.  The step sequence
// runs on across tiles: the DMA and the reads past a tile's last step are
// the next tile's first steps, so its epilogue overlaps the next tile's
// loads.  Steps per tile are padded to an even count >= kStages (padding
// steps read zeros).
//
// K order: the workgroups of XCD x (blockIdx % 8) start each unit at step
// x * steps / 8 of its range and wrap around (not with MX scales, whose
// scale words follow the plain order).  Started together at step 0, every
// workgroup's DMA of a step falls at the same offset of each operand row, and
// with row strides that are a multiple of 4096 bytes all those rows meet at
// one offset within 4 KiB -- which measured as an HBM-bound stall; one start
// per XCD keeps the workgroups of an XCD (which share operand panels in
// their L2) in step.  Same process, against starting at step 0: 40 x 28672
// x 4096 +19 %, 40 x 28672 x 8192 +27 %, 16 x 28672 x 4096 +24 %, 64 x
// 16384 x 8192 +29 %, 96 x 28672 x 4096 +15 %, 4096 x 1536 x 4096 +5 %,
// 512 x 4096 x 8192, 2048 x 2048 x 8192 and 4000 x 904 x 3584 within 1 %.
// The fp32 sums run in that rotated order (deterministic per launch shape).
//
// LDS layout: 128-byte rows with the slot_xor swizzle in the instruction K
// order (layout.hpp).  A lane reads K-chunks g and g + 4 of its row
// (g = lane / 16; lane group g of the MFMA holds K 16g .. 16g + 15 and
// 64 + 16g .. 64 + 16g + 15), stored at slots 2g and 2g + 1 before the XOR:
// conflict-free.  (Stored at slots g and g + 4 they cost 4 conflict cycles
// per ds_read_b128, measured.)
//
// Epilogue: acc * scale (or the extended epilogue, kExt) -> bf16 / fp16,
// staged through the wave's own 8 KiB of LDS (8-byte pieces, piece p of row r
// in slot p ^ (r % 16): conflict-free writes and reads), then 16-byte stores
// of whole 128-byte row segments; 2-byte stores straight from registers when
// N, ldc or C's alignment do not allow 16 (kVec false).  Lanes outside M x N
// get out-of-range offsets.  kExt: each wave DMAs its 64 row scales, 64
// column scales and 64 biases into the first 1.5 KiB of its staging area at
// the tile's first step; the K loop's own waits retire them.
#pragma once

#include <type_traits>

#include "arch.hpp"
#include "epilogue.hpp"
#include "gemm_4wave.hpp"
#include "layout.hpp"

namespace hipgemm {
namespace detail {

struct CfgT128 {
  static constexpr int kThreads = 256;
  static constexpr int kBM = 128, kBN = 128, kBK = 128;
  static constexpr int kStages = 4;
  static constexpr int kAStage = kBM * kBK;            // 16 KiB
  static constexpr int kStage = kAStage + kBN * kBK;   // 32 KiB
  static constexpr int kStoreStage = 64 * 128;         // 8 KiB per wave
  static constexpr int kStoreBase = kStages * kStage;  // 128 KiB
  static constexpr int kLdsBytes = kStoreBase + 4 * kStoreStage;  // 160 KiB
  static constexpr int kDmaPerStep = 8;  // per wave: 4 for A, 4 for B
  static constexpr int kStores = 8;      // per wave per tile, 16-byte path
};

// kSplit: work units are (tile, K-slice) pairs (g.split); each writes its
// fp32 partial tile (written through to the coherent level, sc1: the slices
// of a tile run on several XCDs, whose L2s are not coherent with each
// other).  With g.split.arrivals, each wave then waits for its own partial
// stores, counts its quadrant's arrival (a relaxed agent-scope atomic), and
// the wave that arrives last at a quadrant sums the quadrant's partials in
// slice order (its own from its accumulators, the others read back with
// sc1) and runs the epilogue on the sum: no waiting on other workgroups and
// no barrier, so waves of one workgroup may take different paths here.
// Without it, gemm_t128_reduce_body sums them in a kernel of its own; both
// add +0 + slice 0 + slice 1 + ... in fp32, so their outputs are the same.
// kMx: MX block scales from g.mx (the packed layout of MxArgs; per-tensor
// epilogue).  Each step also loads, for the next step, each operand's 16
// scale bytes of the lane into registers (one buffer load per operand).
template <bool kVec, bool kExt = false, int kFmt = 0, int kAct = kActNone,
          int kOut = kOutBf16, bool kSplit = false, bool kMx = false>
__device__ __forceinline__ void gemm_t128_body(const GemmArgs& g, lds_u8* lds) {
  using Cfg = CfgT128;
  constexpr int S = Cfg::kStages;
  // fp6 operands: a step is 128 elements, 96 bytes of a row (one MFMA per
  // block), held in LDS slots 0-5 of the 128-byte row (slots 6 and 7 stay
  // unfetched).  Other formats: 128 bytes.
  constexpr bool k6 = is_fp6(kFmt);
  constexpr int kStepBytes = k6 ? 96 : Cfg::kBK;
  static_assert(!(k6 && kMx), "MX: 8-bit and fp4 operands");
  constexpr int kDma = Cfg::kDmaPerStep;       // DMA per wave per step
  constexpr int kD = kDma + (kMx ? 2 : 0);     // memory operations per step
  static_assert(!(kMx && kExt), "MX: per-tensor epilogue");
  constexpr int kScaleDma = kExt ? 3 : 0;
  // Stores per wave per tile: 8 x 16 bytes of C (2-byte types, staged),
  // 16 x 16 bytes of partial, or 16 straight from the accumulators (fp32 /
  // e4m3 output, one per block).
  constexpr int kStores = kSplit || (kExt && kOut >= kOutF32) ? 16 : Cfg::kStores;
  static_assert(!(kSplit && kExt), "the split kernels take the plain epilogue");
  static_assert(S >= 3, "pipeline depth");
  static_assert((S - 3) * kD + kStores + kScaleDma + kD < 64, "vmcnt range");
  const int lane = lane_id();
  const int wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;
  const int M = g.M, N = g.N, K = g.K;
  const int tiles_m = (M + Cfg::kBM - 1) / Cfg::kBM;
  const int tiles_n = (N + Cfg::kBN - 1) / Cfg::kBN;
  const int tiles = tiles_m * tiles_n;
  const int units = kSplit ? tiles * g.split.slices : tiles;
  const int steps = kSplit ? g.split.slice_steps : (K + kStepBytes - 1) / kStepBytes;
  const int steps_pad = max(S, (steps + 1) & ~1);
  const int workers = g.workers > 0 ? min((int)gridDim.x, g.workers)
                                    : (int)gridDim.x;
  if ((int)blockIdx.x >= workers) return;
  // Work unit u: tile u % tiles, K-slice u / tiles (one slice unless kSplit),
  // so that units running together share A rows or B columns.
  const TileWalk walk = tile_walk(blockIdx.x, workers, units);
  int t = walk.first;
  if (t >= walk.end) return;

  const float sa = g.scale_a ? *g.scale_a : 1.0f;
  const float sb = g.scale_b ? *g.scale_b : 1.0f;
  const float scale = sa * sb;

  // ---- DMA lane geometry: instruction q (0..3) of wave w covers rows
  // (4q + w) * 8 .. + 8 of A (or B); lane l takes row + l / 8, 16-byte slot
  // l % 8, which holds global K-chunk kpair_chunk((l % 8) ^ slot_xor(row))
  // (the instruction K order of layout.hpp; fp6: chunk (l % 8) ^
  // slot_xor(row)). ---------------------------------------------------------
  const int drow = lane >> 3;
  const int dslot = (lane & 7) ^ slot_xor(8 * (wave & 1) + drow);
  const int dchunk = k6 ? dslot : kpair_chunk(dslot);
  uint32_t voff_a[4], voff_b[4];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int row = (4 * q + wave) * 8 + drow;
    voff_a[q] = (uint32_t)row * (uint32_t)g.lda + dchunk * 16;
    voff_b[q] = (uint32_t)row * (uint32_t)g.ldb + dchunk * 16;
  }

  // Buffer resources of a unit's A rows and B rows (rows past M / N read
  // zero) and its K range [k0, kend); a unit past the walk's end gets empty
  // ranges.
  struct Src {
    __amdgpu_buffer_rsrc_t a, b;
    uint32_t k0;
    int kend;
    int tm, tn;  // tile coordinates (kMx); tm = -1: no unit
  };
  auto src_of = [&](int unit) {
    if (unit >= walk.end)
      return Src{make_rsrc(g.A, 0u), make_rsrc(g.B, 0u), 0u, 0, -1, 0};
    const int tile = kSplit ? unit % tiles : unit;
    const int slice = kSplit ? unit / tiles : 0;
    const TileCoord c = grouped_tile_u(tile, tiles_m, tiles_n, g.group_m);
    const int ra = min(Cfg::kBM, M - c.m * Cfg::kBM);
    const int rb = min(Cfg::kBN, N - c.n * Cfg::kBN);
    const int k0 = slice * steps * kStepBytes;
    return Src{make_rsrc(g.A + (size_t)c.m * Cfg::kBM * g.lda,
                         (uint32_t)ra * (uint32_t)g.lda),
               make_rsrc(g.B + (size_t)c.n * Cfg::kBN * g.ldb,
                         (uint32_t)rb * (uint32_t)g.ldb),
               (uint32_t)k0, min(K, k0 + steps * kStepBytes), c.m, c.n};
  };
  Src cur = src_of(t);
  Src nxt = src_of(t + walk.stride);
  // First step of this workgroup's units (K order, above).
  const int krot = kMx ? 0 : (int)((blockIdx.x & 7u) * (unsigned)steps / 8u);

  // DMA of tile-local step d (d >= steps_pad: step d - steps_pad of the next
  // tile) into `stage`, instruction n (0-3: A rows, 4-7: B rows).  K-chunks
  // past K read zero.
  auto dma_one = [&](int d, int stage, int n) {
    const bool next = d >= steps_pad;
    const Src& s = next ? nxt : cur;
    const int dd = next ? d - steps_pad : d;  // step of the unit
    int dr = dd + krot;                        // the step it loads
    if (dr >= steps) dr -= steps;
    if (dd >= steps) dr = dd;                  // padding: past the range
    uint32_t k0 = s.k0 + (uint32_t)dr * kStepBytes;
    asm volatile("" : "+s"(k0));
    const bool ok = (int)(k0 + dchunk * 16) < s.kend && (!k6 || dchunk < 6);
    lds_u8* base = lds + stage * Cfg::kStage;
    const int q = n & 3;
    if (n < 4)
      dma16(s.a, base + (4 * q + wave) * 1024, ok ? voff_a[q] : kOobOffset, k0);
    else
      dma16(s.b, base + Cfg::kAStage + (4 * q + wave) * 1024,
            ok ? voff_b[q] : kOobOffset, k0);
  };
  auto dma_step = [&](int d, int stage) {
#pragma unroll
    for (int n = 0; n < 8; ++n) dma_one(d, stage, n);
  };

  // ---- fragment reads: A rows 64 wm + 16 i + l % 16, B rows
  // 64 wn + 16 j + l % 16; K-chunks g and g + 4 (g = l / 16). -------------
  const int r16 = lane & 15, grp = lane >> 4;
  const int rslot = kpair_slot(grp) ^ slot_xor(r16);  // chunk g + 4: slot ^ 1
  const uint32_t off_a = (uint32_t)((wm * 64 + r16) * Cfg::kBK + rslot * 16);
  const uint32_t off_b =
      (uint32_t)(Cfg::kAStage + (wn * 64 + r16) * Cfg::kBK + rslot * 16);
  // fp6: lane group g holds elements 32 g .. 32 g + 31 of the step, bytes
  // 24 g .. 24 g + 23 (element boundaries fall on multiples of 3 bytes), as
  // three 8-byte LDS reads; piece p (byte b = 24 g + 8 p) of row r sits in
  // slot (b / 16) ^ slot_xor(r), half (b / 8) % 2.  Each 32-lane half of a
  // read covers 32 distinct 8-byte bank groups (the rows' slots differ per
  // parity, the two lane groups' halves differ): conflict-free.
  const uint32_t row_a = (uint32_t)((wm * 64 + r16) * Cfg::kBK);
  const uint32_t row_b = (uint32_t)(Cfg::kAStage + (wn * 64 + r16) * Cfg::kBK);
  uint32_t p6[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const int b = 24 * grp + 8 * q;
    p6[q] = (uint32_t)((((b >> 4) ^ slot_xor(r16)) << 4) + (((b >> 3) & 1) << 3));
  }
  // Row offset of fragment f of a step (0: A0, 1-4: B0-B3, 5-7: A1-A3).
  auto frag_row = [&](int f) -> uint32_t {
    return f == 0 ? row_a : f <= 4 ? row_b + (f - 1) * 16 * Cfg::kBK
                                   : row_a + (f - 4) * 16 * Cfg::kBK;
  };
  auto join6 = [](u32x2 a, u32x2 b, u32x2 c) {
    return i32x8{(int)a.x, (int)a.y, (int)b.x, (int)b.y, (int)c.x, (int)c.y, 0, 0};
  };
  i32x8 fa[2][4], fb[2][4];
  // kMx: the lane's 16 scale bytes of A and of B_T for the step of each
  // register set (see mx_load).
  i32x4 mxa[2] = {}, mxb[2] = {};
  // Scale words of tile-local step d (d >= steps_pad: the next unit's step
  // d - steps_pad) into set `set`.  The packed layout holds, per 128-row
  // group W and per pair p of 128-element MFMA steps, 16 bytes per lane
  // (step 0 of the pair, then step 1; 8 fragments of 16 rows each): for
  // fp4 a 128-byte step is one pair (its two MFMA take halves 0 and 1),
  // for 8-bit operands half of one.  W = the tile's row (A) or column (B)
  // index.  Groups past M / N, pairs past K and missing units read zero.
  auto mx_load = [&](int d, int set) {
    const bool next = d >= steps_pad;
    const Src& s = next ? nxt : cur;
    const int gs = (int)(s.k0 / Cfg::kBK) + (next ? d - steps_pad : d);  // byte-step
    const int kel = is_fp4(kFmt) ? 2 * K : K;  // K in elements
    const int P = mx_pairs(kel);
    const int p = is_fp4(kFmt) ? gs : gs / 2;
    const MxArgs mx = kernel_mx();
    const bool live = s.tm >= 0 && p < P;
    const uint32_t vo = (uint32_t)lane * 16u;
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc(mx.a, live ? (uint32_t)mx_packed_bytes(M, kel) : 0u);
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(mx.b, live ? (uint32_t)mx_packed_bytes(N, kel) : 0u);
    const int tm = live ? s.tm : 0, tn = live ? s.tn : 0;
    mxa[set] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
        ra, vo + (uint32_t)((tm * P + p) * 1024), 0, 0));
    mxb[set] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
        rb, vo + (uint32_t)((tn * P + p) * 1024), 0, 0));
  };
  auto read_step = [&](int stage, int set) {
    const lds_u8* base = lds + stage * Cfg::kStage;
    if constexpr (k6) {
#pragma unroll
      for (int f = 0; f < 8; ++f) {
        const lds_u8* r = base + frag_row(f);
        const i32x8 v = join6(lds_read8(r + p6[0]), lds_read8(r + p6[1]),
                              lds_read8(r + p6[2]));
        if (f == 0) fa[set][0] = v;
        else if (f <= 4) fb[set][f - 1] = v;
        else fa[set][f - 4] = v;
      }
      return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t o = off_a + i * 16 * Cfg::kBK;
      fa[set][i] = join(lds_read16(base + o), lds_read16(base + (o ^ 16u)));
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t o = off_b + j * 16 * Cfg::kBK;
      fb[set][j] = join(lds_read16(base + o), lds_read16(base + (o ^ 16u)));
    }
  };

  f32x4 acc[4][4];
  // One step, in an explicit order (the scheduler otherwise put the reads
  // after all the MFMA): MFMA n (block n / 4, n % 4) of register set `set`,
  // each followed by one 16-byte read for the other set -- in the order the
  // next step's MFMA use them: A0, B0..B3, A1..A3 -- and, after the first
  // eight, one DMA each.
  auto step = [&](int set, int rstage, int d, int dstage) {
    const lds_u8* rb = lds + rstage * Cfg::kStage;
    i32x4 rd[16];
    u32x2 rd6[24];
    // kMx: this wave's scale words of the step (fp4: halves 0 and 1; 8-bit:
    // half `set` of the pair), chosen once.
    uint32_t wa0 = 0, wa1 = 0, wb0 = 0, wb1 = 0;
    if constexpr (kMx) {
      const int h0 = is_fp4(kFmt) ? 0 : 2 * set;
      wa0 = (uint32_t)(wm ? mxa[set][h0 + 1] : mxa[set][h0]);
      wb0 = (uint32_t)(wn ? mxb[set][h0 + 1] : mxb[set][h0]);
      if constexpr (is_fp4(kFmt)) {
        wa1 = (uint32_t)(wm ? mxa[set][3] : mxa[set][2]);
        wb1 = (uint32_t)(wn ? mxb[set][3] : mxb[set][2]);
      }
    }
    sched_fence();
#pragma unroll
    for (int n = 0; n < 16; ++n) {
      const int i = n / 4, j = n % 4;
      if constexpr (is_fp4(kFmt)) {
        // fp4: 256 elements per 128-byte step, two MFMA per block -- the
        // fragments' low halves (K-chunk g) and high halves (chunk g + 4);
        // the instruction reads four registers of each operand.  kMx: half
        // h uses scale word 2 h + (the wave's 64-row half), byte i / j.
        const i32x8& x = fb[set][j];
        const i32x8& y = fa[set][i];
        const i32x8 xh = __builtin_shufflevector(x, x, 4, 5, 6, 7, 0, 1, 2, 3);
        const i32x8 yh = __builtin_shufflevector(y, y, 4, 5, 6, 7, 0, 1, 2, 3);
        if constexpr (kMx) {
          acc[i][j] = mfma_16x16x128_mx<kFmtFp4, kFmtFp4>(x, y, acc[i][j], wb0, wa0,
                                                          j, i);
          acc[i][j] = mfma_16x16x128_mx<kFmtFp4, kFmtFp4>(xh, yh, acc[i][j], wb1, wa1,
                                                          j, i);
        } else {
          acc[i][j] = mfma_16x16x128<kFmtFp4, kFmtFp4>(x, y, acc[i][j]);
          acc[i][j] = mfma_16x16x128<kFmtFp4, kFmtFp4>(xh, yh, acc[i][j]);
        }
      } else if constexpr (kMx) {
        // 8-bit: the step is half `set` of its pair (units start on even
        // steps and each trip takes two steps).
        acc[i][j] = mfma_16x16x128_mx<fmt_b(kFmt), fmt_a(kFmt)>(
            fb[set][j], fa[set][i], acc[i][j], wb0, wa0, j, i);
      } else {
        acc[i][j] = mfma_16x16x128<fmt_b(kFmt), fmt_a(kFmt)>(fb[set][j], fa[set][i],
                                                             acc[i][j]);
      }
      // read n: fragment f (0: A0, 1-4: B0-B3, 5-7: A1-A3), half n % 2
      // (fp6: pieces 0 and 1 for even n, piece 2 for odd n)
      const int f = n / 2;
      if constexpr (k6) {
        const lds_u8* r = rb + frag_row(f);
        if ((n & 1) == 0) {
          rd6[3 * f] = lds_read8(r + p6[0]);
          rd6[3 * f + 1] = lds_read8(r + p6[1]);
        } else {
          rd6[3 * f + 2] = lds_read8(r + p6[2]);
        }
      } else {
        const uint32_t o = f == 0   ? off_a
                           : f <= 4 ? off_b + (f - 1) * 16 * Cfg::kBK
                                    : off_a + (f - 4) * 16 * Cfg::kBK;
        rd[n] = lds_read16(rb + ((n & 1) ? (o ^ 16u) : o));
      }
      __builtin_amdgcn_sched_group_barrier(0x008, is_fp4(kFmt) ? 2 : 1, 0);
      if (k6 && (n & 1) == 0)
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      else
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      if (n < 8) {
        dma_one(d, dstage, n);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
      }
      sched_fence();
    }
    // kMx: the scales of the step after next, into this step's set (its
    // MFMA are issued): loaded two steps ahead, they retire with the DMA
    // the waits already cover instead of making the next step wait for
    // every DMA issued before them.
    if constexpr (kMx) mx_load(d - (S - 3), set);
    const int o = set ^ 1;
    if constexpr (k6) {
      fa[o][0] = join6(rd6[0], rd6[1], rd6[2]);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        fb[o][j] = join6(rd6[3 + 3 * j], rd6[4 + 3 * j], rd6[5 + 3 * j]);
#pragma unroll
      for (int i = 1; i < 4; ++i)
        fa[o][i] = join6(rd6[12 + 3 * i], rd6[13 + 3 * i], rd6[14 + 3 * i]);
      return;
    }
    fa[o][0] = join(rd[0], rd[1]);
#pragma unroll
    for (int j = 0; j < 4; ++j) fb[o][j] = join(rd[2 + 2 * j], rd[3 + 2 * j]);
#pragma unroll
    for (int i = 1; i < 4; ++i) fa[o][i] = join(rd[8 + 2 * i], rd[9 + 2 * i]);
  };

  // kExt: the wave's 64 row scales, 64 column scales and 64 biases into its
  // staging area (rows at +0, columns at +512, bias at +1024), one float per
  // lane; zero past M / N.
  lds_u8* stg = lds + Cfg::kStoreBase + wave * Cfg::kStoreStage;
  auto scale_dma = [&](int tile) {
    const TileCoord c = grouped_tile_u(tile, tiles_m, tiles_n, g.group_m);
    const EpiArgs ea = kernel_epi();
    int ln = lane;
    asm volatile("" : "+v"(ln));
    const __amdgpu_buffer_rsrc_t rr =
        make_rsrc(ea.row_scale, ea.row_scale ? (uint32_t)M * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rc =
        make_rsrc(ea.col_scale, ea.col_scale ? (uint32_t)N * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(ea.bias, ea.bias ? (uint32_t)N * 4u : 0u);
    const uint32_t ro = (uint32_t)(c.m * Cfg::kBM + wm * 64 + ln) * 4u;
    const uint32_t co = (uint32_t)(c.n * Cfg::kBN + wn * 64 + ln) * 4u;
    dma4(rr, stg, ro);
    dma4(rc, stg + 512, co);
    dma4(rb, stg + 1024, co);
  };

  // Prologue of the first tile: (kMx: the scales of step 0,) steps
  // 0 .. S - 2, then the reads of step 0.
  if constexpr (kMx) {
    mx_load(0, 0);
    mx_load(1, 1);
  }
#pragma unroll
  for (int d = 0; d < S - 1; ++d) dma_step(d, d);
  wait_vmcnt<(S - 2) * kDma>();
  barrier();
  read_step(0, 0);

  int base = 0;          // stage of the tile's step 0
  bool stores = false;   // the previous tile's C stores are in flight
  bool first = true;     // the first tile (its first steps' DMA: prologue)
  for (;;) {
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{};

    // Two steps per trip (register set 0, then 1); steps_pad is even.
    for (int k = 0; k < steps_pad; k += 2) {
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const int kk = k + h;
        // Step kk + 1 landed: newer than it are steps kk + 2 .. kk + S - 2
        // (kD operations each; in the prologue kDma), and, during the first
        // S - 2 steps of a tile after the first, the previous tile's stores
        // (issued after this tile's first S - 1 steps' DMA); kExt's three
        // scale loads only make this wait longer.
        if (stores && kk < S - 2)
          wait_vmcnt<(S - 3) * kD + kStores>();
        else if (first && kk < S - 2)
          wait_vmcnt<(S - 3) * kDma>();
        else
          wait_vmcnt<(S - 3) * kD>();
        barrier();
        if constexpr (kExt)
          if (kk == 0) scale_dma(t);
        // The reads past the last step are the next tile's step 0, whose
        // stage is (base + steps_pad) % S.
        step(h, (base + kk + 1) % S, kk + S - 1, (base + kk + S - 1) % S);
      }
    }

    // ---- epilogue ---------------------------------------------------------
    bool write_c = !kSplit;
    if constexpr (kSplit) {
      // The unit's fp32 partial: wave w's 16 blocks at ((t * 4 + w) * 16 +
      // 4 i + j) KiB of g.split.partial, lane l's 16 bytes at + 16 l (unit
      // t = slice * tiles + tile).
      constexpr int kCoherent = 16;  // cache policy: sc1
      const int slices = g.split.slices;
      const __amdgpu_buffer_rsrc_t rp = make_rsrc(
          g.split.partial, (uint32_t)tiles * (uint32_t)slices * 65536u);
      const uint32_t lo = (uint32_t)lane * 16u;
      // Wave-uniform offsets in scalar registers (t's division ran on the
      // VALU): a buffer instruction whose scalar operand sits in a VGPR is
      // wrapped in a readfirstlane loop.
      const uint32_t own_off =
          (uint32_t)__builtin_amdgcn_readfirstlane((t * 4 + wave) * 16384);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j)
          store_b128<kCoherent>(__builtin_bit_cast(i32x4, acc[i][j]), rp,
                                lo + (uint32_t)((4 * i + j) * 1024), own_off);
      if (g.split.arrivals) {
        const int tile = __builtin_amdgcn_readfirstlane(t % tiles);
        const int own = __builtin_amdgcn_readfirstlane(t / tiles);
        int* const ctr = g.split.arrivals + tile * 4 + wave;
        // This wave's partial stores (and every other operation of it) are
        // complete before its arrival is counted.
        wait_vmcnt<0>();
        int before = 0;
        if (lane == 0)
          before = __hip_atomic_fetch_add(ctr, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);
        before = __builtin_amdgcn_readfirstlane(before);
        if (before == slices - 1) {
          // Last arrival: +0 + slice 0 + slice 1 + ..., two slices' loads
          // in flight at a time; the own slice comes from the accumulators,
          // slices past the last read zero (offset out of range: +0, which
          // leaves every sum unchanged).
          f32x4 sum[4][4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) sum[i][j] = f32x4{};
          for (int q0 = 0; q0 < slices; q0 += 2) {
            f32x4 v[2][4][4];
#pragma unroll
            for (int b = 0; b < 2; ++b) {
              const int q = q0 + b;
              const uint32_t so =
                  (uint32_t)(((q < slices ? q : 0) * tiles + tile) * 4 + wave) * 16384u;
              const uint32_t oob = q < slices && q != own ? 0u : kOobOffset;
#pragma unroll
              for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                  v[b][i][j] = __builtin_bit_cast(
                      f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                 rp, (lo + (uint32_t)((4 * i + j) * 1024)) | oob, so,
                                 kCoherent));
            }
#pragma unroll
            for (int b = 0; b < 2; ++b) {
              const bool is_own = q0 + b == own;
#pragma unroll
              for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                  sum[i][j] += is_own ? acc[i][j] : v[b][i][j];
            }
          }
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[i][j] = sum[i][j];
          // Every lane stores the same zero: no branch on the lane.
          __hip_atomic_store(ctr, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          write_c = true;
        }
      }
    }
    if (write_c) {
    const TileCoord tc =
        grouped_tile_u(kSplit ? t % tiles : t, tiles_m, tiles_n, g.group_m);
    const int rows_left = M - tc.m * Cfg::kBM - wm * 64;  // from wave row 0
    const int cols_left = N - tc.n * Cfg::kBN - wn * 64;  // from wave col 0
    auto oob_unless = [](int x, int limit) -> uint32_t {
      return (uint32_t)((limit - 1 - x) >> 31) & kOobOffset;
    };
    int elane = lane;
    asm volatile("" : "+v"(elane));
    const int er16 = elane & 15, egrp = elane >> 4;
    EpiVec<4, 4> ev;
    if constexpr (kExt) ev.read_lds(stg, kernel_epi(), scale, elane);
    auto pack = [&](const f32x4& a, int i, int j) -> u32x2 {
      if constexpr (kExt)
        return ev.template pack4<kAct, kOut>(a[0], a[1], a[2], a[3], i, j);
      else
        return u32x2{pack_bf16x2(a[0] * scale, a[1] * scale),
                     pack_bf16x2(a[2] * scale, a[3] * scale)};
    };
    // C window of this wave: rows tc.m*128 + 64 wm .., columns tc.n*128 +
    // 64 wn ..; the range ends at its last valid element.
    constexpr int es = kExt ? out_bytes(kOut) : 2;  // bytes per C element
    const int wrows = min(64, rows_left), wcols = min(64, cols_left);
    uint8_t* cw = reinterpret_cast<uint8_t*>(g.C) +
                  ((size_t)(tc.m * Cfg::kBM + wm * 64) * g.ldc + tc.n * Cfg::kBN +
                   wn * 64) * es;
    const bool any = wrows > 0 && wcols > 0;
    const __amdgpu_buffer_rsrc_t rsrc_c = make_rsrc(
        cw, any ? (uint32_t)(((wrows - 1) * g.ldc + wcols) * es) : 0u);
    if constexpr (kExt && kOut >= kOutF32) {
      // fp32 / e4m3 output: straight from the accumulators (4 consecutive
      // elements per lane and block: one 16- or 4-byte store, or one per
      // element when kVec is false).
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 16 * i + er16, col = 16 * j + 4 * egrp;
          const uint32_t off = (uint32_t)((r * g.ldc + col) * es) |
                               oob_unless(r, rows_left);
          const f32x4& a = acc[i][j];
          const f32x4 v = ev.template value4<kAct>(a[0], a[1], a[2], a[3], i, j);
          if constexpr (kOut == kOutF32) {
            if constexpr (kVec) {
              store_b128<kStoreCPart>(
                  __builtin_bit_cast(i32x4, v), rsrc_c,
                  off | oob_unless(col, cols_left), 0);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                __builtin_amdgcn_raw_buffer_store_b32(
                    (uint32_t)__builtin_bit_cast(i32x4, v)[e], rsrc_c,
                    (off | oob_unless(col + e, cols_left)) + 4 * e, 0, kStoreCPart);
            }
          } else {
            const uint32_t w = ev.e4m3x4(v);
            if constexpr (kVec) {
              __builtin_amdgcn_raw_buffer_store_b32(
                  w, rsrc_c, off | oob_unless(col, cols_left), 0, kStoreCPart);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                __builtin_amdgcn_raw_buffer_store_b8(
                    (uint8_t)(w >> (8 * e)), rsrc_c,
                    (off | oob_unless(col + e, cols_left)) + e, 0, kStoreCPart);
            }
          }
        }
    } else if constexpr (kVec) {
      // Stage: 8-byte piece p (columns 4p .. 4p + 3) of row r at slot
      // p ^ (r % 16) of the row's 128 bytes.
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int r = 16 * i + er16, p = 4 * j + egrp;
          lds_write8(stg + r * 128 + ((p ^ (r & 15)) * 8), pack(acc[i][j], i, j));
        }
      // Read back: store q covers rows 8q + l / 8, 16-byte chunk l % 8
      // (pieces 2c, 2c + 1: one 16-byte unit, halves swapped on odd rows).
      const int c = elane & 7, rsub = elane >> 3;
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        const int r = 8 * q + rsub;
        const int u = ((2 * c) ^ (r & 15)) >> 1;
        i32x4 v = lds_read16(stg + r * 128 + u * 16);
        if (r & 1) v = i32x4{v[2], v[3], v[0], v[1]};
        const uint32_t off = (uint32_t)((r * g.ldc + 8 * c) * 2) |
                             oob_unless(r, rows_left) | oob_unless(8 * c, cols_left);
        store_b128<kStoreC>(v, rsrc_c, off, 0);
      }
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const u32x2 pk = pack(acc[i][j], i, j);
          const int r = 16 * i + er16, col = 16 * j + 4 * egrp;
          const uint32_t rb = (uint32_t)((r * g.ldc + col) * 2) | oob_unless(r, rows_left);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const uint32_t w = (e < 2 ? pk.x : pk.y) >> (16 * (e & 1));
            __builtin_amdgcn_raw_buffer_store_b16(
                (unsigned short)w, rsrc_c,
                (rb | oob_unless(col + e, cols_left)) + 2 * e, 0, kStoreCPart);
          }
        }
    }

    }  // write_c

    t += walk.stride;
    if (t >= walk.end) break;
    base += steps_pad;
    base %= S;
    cur = nxt;
    nxt = src_of(t + walk.stride);
    stores = kSplit || kVec;
    first = false;
  }
  // The last tile's look-ahead DMA (empty ranges) still count in vmcnt.
  wait_vmcnt<0>();
}

// Sum of the K-slice partials of gemm_t128_body<..., kSplit = true>, in
// slice order 0, 1, ... (the result does not depend on which unit finished
// first), then the epilogue (per-tensor, or the extended one with the
// activation and output type chosen at run time) and the C stores.  One
// wave per workgroup, 16 x tiles workgroups: workgroup b takes rows
// 16 (b % 4) .. + 15 of quadrant (b / 4) % 4 of tile b / 16 (one row of
// four 16 x 16 blocks).  Its loads go out kBatch slices at a time (4 KiB per
// slice and wave), so that a wave has 32 KiB in flight instead of one
// slice: the partials come back from the device-level cache, and with one
// slice in flight per wave (4 waves per tile) the sum of 128 x 8192 x 8192's
// 16 MiB of partials took 11.1 us.  Slices past the last read as +0 (out of
// range), which leaves every sum unchanged (a sum that starts at +0 is never
// -0).  Launched right after the split kernel on the same stream, which makes
// its partials visible.  kVec8: one store per lane and block (N and ldc
// multiples of 4, C aligned to four elements), else one per element.
template <bool kVec8, bool kExt>
__device__ __forceinline__ void gemm_t128_reduce_body(const GemmArgs& g) {
  using Cfg = CfgT128;
  constexpr int kBatch = 8;
  const int lane = lane_id();
  const int M = g.M, N = g.N;
  const int tiles_m = (M + Cfg::kBM - 1) / Cfg::kBM;
  const int tiles_n = (N + Cfg::kBN - 1) / Cfg::kBN;
  const int tiles = tiles_m * tiles_n;
  const int w = (blockIdx.x >> 2) & 3, i = blockIdx.x & 3, t = blockIdx.x >> 4;
  if (t >= tiles) return;
  const int wm = w >> 1, wn = w & 1;
  const TileCoord tc = grouped_tile_u(t, tiles_m, tiles_n, g.group_m);
  const int row0 = tc.m * Cfg::kBM + wm * 64, col0 = tc.n * Cfg::kBN + wn * 64;
  const float s = (g.scale_a ? *g.scale_a : 1.0f) * (g.scale_b ? *g.scale_b : 1.0f);
  EpiVec<4, 4> ev;
  if constexpr (kExt) ev.load(g.epi, M, N, row0, col0, s, lane);
  const int slices = g.split.slices;
  const __amdgpu_buffer_rsrc_t rp = make_rsrc(
      g.split.partial, (uint32_t)tiles * (uint32_t)slices * 65536u);
  f32x4 sum[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) sum[j] = f32x4{};
  for (int q0 = 0; q0 < slices; q0 += kBatch) {
    f32x4 v[kBatch][4];
#pragma unroll
    for (int b = 0; b < kBatch; ++b) {
      const int q = q0 + b;
      const uint32_t base =
          q < slices ? (uint32_t)(((q * tiles + t) * 4 + w) * 16384 + 4 * i * 1024 +
                                  lane * 16)
                     : kOobOffset;
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v[b][j] = __builtin_bit_cast(
            f32x4, __builtin_amdgcn_raw_buffer_load_b128(rp, base + j * 1024, 0, 0));
    }
#pragma unroll
    for (int b = 0; b < kBatch; ++b)
#pragma unroll
      for (int j = 0; j < 4; ++j) sum[j] += v[b][j];
  }
  const int rows_left = M - row0, cols_left = N - col0;
  auto oob_unless = [](int x, int limit) -> uint32_t {
    return (uint32_t)((limit - 1 - x) >> 31) & kOobOffset;
  };
  const int es = kExt ? out_bytes(ev.out) : 2;  // bytes per C element
  const int wrows = min(64, rows_left), wcols = min(64, cols_left);
  const __amdgpu_buffer_rsrc_t rc = make_rsrc(
      reinterpret_cast<uint8_t*>(g.C) + ((size_t)row0 * g.ldc + col0) * es,
      wrows > 0 && wcols > 0 ? (uint32_t)(((wrows - 1) * g.ldc + wcols) * es) : 0u);
  const int r16 = lane & 15, grp = lane >> 4;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const f32x4 a = sum[j];
    const int r = 16 * i + r16, col = 16 * j + 4 * grp;
    const uint32_t rb = (uint32_t)((r * g.ldc + col) * es) | oob_unless(r, rows_left);
    if constexpr (kExt) {
      store_out4<kVec8>(ev, a[0], a[1], a[2], a[3], i, j, rc, rb, col, cols_left);
      continue;
    }
    const u32x2 pk = u32x2{pack_bf16x2(a[0] * s, a[1] * s), pack_bf16x2(a[2] * s, a[3] * s)};
    if constexpr (kVec8) {
      __builtin_amdgcn_raw_buffer_store_b64(pk, rc, rb | oob_unless(col, cols_left),
                                            0, 0);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t x = (e < 2 ? pk.x : pk.y) >> (16 * (e & 1));
        __builtin_amdgcn_raw_buffer_store_b16(
            (unsigned short)x, rc, (rb | oob_unless(col + e, cols_left)) + 2 * e, 0, 0);
      }
    }
  }
}

}  // namespace detail
}  // namespace hipgemm
