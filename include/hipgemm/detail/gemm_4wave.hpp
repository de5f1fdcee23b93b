// hipgemm -- 4-wave FP8 GEMM main body (gfx950).
//
// C[M x N] (bf16) = scale_a * scale_b * A[M x K] . B_T[N x K]^T, e4m3 inputs,
// fp32 accumulation.  Reference counterpart: fp8_gemm_4wave_256x256x128,
// fp8_4wave.hpp:334-567 (same interface and block shape, different design).
//
// Work decomposition
//   * One workgroup = 256 threads = 4 waves (one per SIMD).  The grid is
//     persistent: `workers` workgroups (at most one per CU) walk the 256 x 256
//     output tiles, the workgroups of each XCD striding through one
//     contiguous band of tile indices (tile_walk, layout.hpp).  Workgroups
//     with blockIdx.x >= workers return at once, so any launch grid >= 1 is
//     correct.
//   * Wave w owns the contiguous 128 x 128 quadrant (w / 2, w % 2) of a tile
//     as 4 x 4 blocks of 32 x 32 fp32 accumulators (256 AGPRs per lane).
//   * K advances 128 bytes per step (one LDS stage); each of the 16 blocks
//     takes two v_mfma_f32_32x32x64_f8f6f4 per step (K-halves).  The step
//     count per tile is padded to an even number >= 4 (padding steps read
//     zeros).
//
// Operand registers: four tiles of 64 rows x 128 K-bytes (32 VGPRs each):
// a_lo / a_hi = the wave's A rows 0-63 / 64-127, b_lo / b_hi likewise for B.
// A step runs four quarter-steps Q00, Q01, Q10, Q11; quarter Qij takes the
// 2 x 2 blocks (a_i, b_j).  A tile is reloaded for the next step as soon as
// its second use is over:
//   Q00(k): MFMA a_lo x b_lo | read b_hi(k)   | DMA A_lo group, step k+2
//   Q01(k): MFMA a_lo x b_hi | read a_hi(k)   | DMA B_lo group, step k+2
//   Q10(k): MFMA a_hi x b_lo | read a_lo(k+1) | DMA B_hi group, step k+2
//   Q11(k): MFMA a_hi x b_hi | read b_lo(k+1) | DMA A_hi group, step k+2
// LDS holds 2 stages (A 256 x 128 B + B 256 x 128 B each, 128 KiB).  Each
// 64-row sub-buffer group (e.g. "A_lo" = A rows 0-63 and 128-191, the a_lo
// rows of both wave rows) is refilled at least two quarter-steps after its
// last read, so only Q00 and Q10 start with s_barrier (after waiting for the
// wave's own LDS reads and its own DMA up to the groups read next); Q01 and
// Q11 wait for the wave's own LDS reads only.  Each refill lands 5-6
// quarter-steps before its first read.  Inside a quarter the 8 LDS reads go
// one per MFMA in the first half and the 4 DMA one per MFMA in the second.
// Against one barrier per quarter-step: 8192^3 0.97 -> 0.99 of the reference
// kernel, 4096^3 0.99 -> 1.04 (same process).
//
// Across tiles the pipeline does not drain: "step k+2" of the last two steps
// of a tile is step 0 or 1 of the workgroup's next tile (all-zero reads when
// there is none), so the next tile's operands are in LDS, and its a_lo /
// b_lo in registers, when the epilogue runs.  The epilogue stages through a
// separate 32 KiB LDS region and issues its 32 stores per wave without
// waiting for them; the next tile's first three barriers wait with vmcnt
// 16 + 32 (the stores sit between the DMA groups each needs and the newer
// DMAs), later ones with vmcnt 16.  vmcnt retires memory operations in issue
// order, loads and stores alike.  The first tile of a workgroup has no stores
// in flight: its prologue waits for step 0 only and its barriers use the
// steady vmcnt 16.
//
// Global -> LDS: buffer_load_dwordx4 ... lds, 8 rows x 128 B per instruction
// (whole 128-byte lines), 16 instructions per wave per step.  The buffer
// resource of a tile covers only its valid rows, so rows past M (or N) read
// zero; K-chunks past K get an out-of-range offset.  Nothing outside A or B is
// ever addressed.
//
// Epilogue: acc * (scale_a * scale_b) -> bf16 (RNE), staged 32 rows at a time
// through the wave's own 8 KiB of LDS so that every store instruction writes
// whole 128-byte lines of C (16 bytes per lane, 4 rows x 256 B); 2-byte stores
// straight from the accumulators when N, ldc or C's alignment do not allow
// 16.  No branches: lanes outside M x N are dropped by the buffer range check.
#pragma once

#include <type_traits>

#include "arch.hpp"
#include "epilogue.hpp"
#include "layout.hpp"

namespace hipgemm {
namespace detail {

// MX block scales (E8M0, one per 32 K-elements of a row), packed by
// hipgemm_mx_pack_scales: for each group of 128 rows W and each pair of
// 128-byte K-steps p, 1 KiB holding, for lane l, 16 bytes: step 0 then step
// 1, each the scales of rows 128 W + 16 f + l % 16 (f = 0..7) for K-block
// l / 16 of that step -- what one wave's 16x16x128 MFMA need, in one 16-byte
// load per operand per step pair.  W-groups of P = ceil(ceil(K / 128) / 2)
// pairs.  Null: no MX scaling.
struct MxArgs {
  const uint8_t* a = nullptr;
  const uint8_t* b = nullptr;
};

__host__ __device__ constexpr int mx_pairs(int K) { return ((K + 127) / 128 + 1) / 2; }
__host__ __device__ constexpr size_t mx_packed_bytes(int rows, int K) {
  return (size_t)((rows + 127) / 128) * mx_pairs(K) * 1024;
}

// K-slices of the 128 x 128 schedule (gemm_t128.hpp, kSplit): work unit u
// of tiles x slices is tile u % tiles over K-steps [s S, s S + S) of 128
// bytes, s = u / tiles, S = slice_steps; its fp32 partial tile goes to
// `partial` (64 KiB per unit) for the reduce kernel.
struct SplitArgs {
  int slices = 1;
  int slice_steps = 0;
  float* partial = nullptr;
  // Non-null: one arrival counter per (tile, wave quadrant), zero between
  // calls; the last slice to arrive at a quadrant sums it and writes C (no
  // reduce kernel).  Null: the reduce kernel sums the partials.
  int* arrivals = nullptr;
};

struct GemmArgs {
  const uint8_t* A;      // M x K 8-bit (format by kFmt), row stride lda bytes
  const uint8_t* B;      // N x K 8-bit (B_T), row stride ldb bytes
  uint16_t* C;           // M x N bf16 (fp16: kExt, epi.out), stride ldc elements
  const float* scale_a;  // device scalar, nullptr = 1.0
  const float* scale_b;  // device scalar, nullptr = 1.0
  int M, N, K;
  int lda, ldb, ldc;
  int group_m;
  int workers;  // persistent workgroups (<= grid); 0 = the whole grid
  EpiArgs epi;  // extended epilogue (kExt instantiations only)
  MxArgs mx;    // MX block scales (kMx instantiations only)
  SplitArgs split;  // K-slices (128 x 128 schedule only)
};

// The GemmArgs of a kernel whose only argument is a GemmArgs, read again
// from the kernel-argument segment (scalar loads) at the point of use, so
// that values needed once per tile occupy no registers across the K loop.
__device__ __forceinline__ const __attribute__((address_space(4))) GemmArgs*
kernel_args() {
  auto p = (const __attribute__((address_space(4))) GemmArgs*)
      __builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(p));
  return p;
}
__device__ __forceinline__ MxArgs kernel_mx() {
  const auto* k = kernel_args();
  MxArgs m;
  m.a = k->mx.a;
  m.b = k->mx.b;
  return m;
}
__device__ __forceinline__ EpiArgs kernel_epi() {
  const auto* k = kernel_args();
  EpiArgs e;
  e.row_scale = k->epi.row_scale;
  e.col_scale = k->epi.col_scale;
  e.bias = k->epi.bias;
  e.act = k->epi.act;
  e.out = k->epi.out;
  e.out_scale = k->epi.out_scale;
  return e;
}

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
  static constexpr int kStageEnd = kStages * (kAStage + kBStage);  // 128 KiB
  static constexpr int kStoreRows = 32;                 // epilogue chunk
  static constexpr int kStoreStage = kStoreRows * 256;  // 8 KiB per wave
  static constexpr int kStoreBase = kStageEnd;
  static constexpr int kLdsBytes = kStageEnd + 4 * kStoreStage;  // 160 KiB
  static constexpr int kDmaPerStep = 16;  // per wave: 8 for A, 8 for B
  static constexpr int kStoresPerTile = 32;  // per wave, 16-byte path
  // Workers of the C++ drop-in template, whose grid the caller sizes to the
  // tile count: one per CU of an MI355X.
  static constexpr int kDropinWorkers = 256;
};

// MFMA per quarter-step, and how many of them (the "tail") are issued after
// the next quarter-step's waits (and barrier, at Q00 and Q10) instead of
// before them.  MFMA read only registers, so they may straddle the barrier;
// the tail keeps the matrix unit busy while the waves meet, which hides the
// skew between them (one MFMA; for 16x16x128 two measured 1 % slower at
// 8192^3, none 3 % slower).
template <int kMf>
struct QuarterShape {
  static constexpr int kMfma = kMf == 16 ? 16 : 8;
  static constexpr int kTail = 1;
  static constexpr int kHead = kMfma - kTail;
};

// 16x16x128: block (row, column) of a quarter's 4 x 4 blocks that its MFMA n
// updates.  Rows in order; odd rows run right to left, so that the MFMA
// after each row change shares its B fragment with the one before (within a
// row they share the A fragment).  Same process, A/B of whole kernels,
// outputs bit-identical (each block still sums K in the same order): 8192^3
// +0.7 %, 8192 x 8192 x 28672 and 8192 x 28672 x 8192 +0.5 %, 4096^3
// +0.5 %; the column-major order (B shared within a column) was level with
// row-major.  The kernel is power-bound there: fewer operand changes are
// less switching in the matrix unit.
__host__ __device__ constexpr int quarter_row16(int n) { return n / 4; }
__host__ __device__ constexpr int quarter_col16(int n) {
  return (n / 4) % 2 ? 3 - n % 4 : n % 4;
}

// Order of one quarter-step: the previous quarter's tail MFMA first, then
// this quarter's head MFMA with its LDS reads in the first half and its 4
// DMA after.  16x16x128: [M R] x 8, [M D] x 4, [M] x 3 (spreading the DMAs
// between the reads, or issuing them first, measured 9-10 % slower), written
// out in `quarter`.  32x32x64: [M R R] x 4, [M D] x 2, [M D D], as a
// sched_group_barrier pattern (0x008 MFMA, 0x100 LDS read, 0x020 DMA) over
// the whole quarter.
__device__ __forceinline__ void quarter_schedule_32(bool tail) {
  if (tail)
    __builtin_amdgcn_sched_group_barrier(0x008, QuarterShape<32>::kTail, 0);
  for (int x = 0; x < 4; ++x) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
  }
  for (int x = 0; x < 2; ++x) {
    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
  }
  __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
  __builtin_amdgcn_sched_group_barrier(0x020, 2, 0);
}

// Operand windows of one output tile: buffer resources over the tile's valid
// rows of A and B_T (none at all past the last tile, so every read is zero),
// and its coordinates (0 past the last tile).
struct TileSrc {
  __amdgpu_buffer_rsrc_t a, b;
  int tm, tn;
};

// `end`: one past the last tile index the caller may visit.
__device__ __forceinline__ TileSrc tile_src(const GemmArgs& g, int t,
                                            int end, int tiles_m,
                                            int tiles_n) {
  if (t >= end) return TileSrc{make_rsrc(g.A, 0), make_rsrc(g.B, 0), 0, 0};
  const TileCoord tc = grouped_tile_u(t, tiles_m, tiles_n, g.group_m);
  const int rows_a = min(Cfg4w::kBM, g.M - tc.m * Cfg4w::kBM);
  const int rows_b = min(Cfg4w::kBN, g.N - tc.n * Cfg4w::kBN);
  return TileSrc{make_rsrc(g.A + (size_t)tc.m * Cfg4w::kBM * g.lda,
                           (uint32_t)rows_a * (uint32_t)g.lda),
                 make_rsrc(g.B + (size_t)tc.n * Cfg4w::kBN * g.ldb,
                           (uint32_t)rows_b * (uint32_t)g.ldb),
                 tc.m, tc.n};
}

// kMf selects the MFMA: 32 = v_mfma_f32_32x32x64_f8f6f4 (4 x 4 blocks of
// 32 x 32 per wave, two MFMA per block per step), 16 =
// v_mfma_f32_16x16x128_f8f6f4 (8 x 8 blocks of 16 x 16, one per block per
// step).  Same data flow and the same 2048 MFMA cycles per step either way.
// kExt: the extended epilogue of epilogue.hpp (row / column scales, bias,
// activation, fp16 output) from g.epi; 16x16x128 only.
// kAct / kOut (kExt only): the activation and the output type
// (epilogue.hpp) -- template parameters, so that each instantiation has one
// straight-line epilogue.
// kMx: MX block scales from g.mx (16x16x128, per-tensor epilogue).
// kLine: C's rows start on 128-byte lines (ldc a multiple of 64 elements, C
// 128-byte aligned): the plain 16x16x128 epilogue with 16-byte stores then
// runs inside the MFMA stream of the tile boundary (the overlapped epilogue
// below), whose stores write 128 bytes of a row each -- whole lines only
// when rows are line-aligned (with a 10000-byte row stride, 11 % slower than
// the epilogue after the K loop, whose stores write 256 bytes of a row).
template <bool kVecStore, int kMf = 32, bool kExt = false, int kFmt = 0,
          int kAct = kActNone, int kOut = kOutBf16, bool kMx = false,
          bool kLine = false>
__device__ __forceinline__ void gemm_4wave_body(const GemmArgs& g,
                                                lds_u8* lds) {
  using Cfg = Cfg4w;
  static_assert(kMf == 32 || kMf == 16, "MFMA shape");
  static_assert(!kExt || kMf == 16, "extended epilogue: 16x16x128 only");
  static_assert(!kMx || (kMf == 16 && !kExt), "MX: 16x16x128, plain epilogue");
  // fp4 x fp4: a 128-byte step holds 256 elements, so each 16x16 block takes
  // two MFMA per step, on the low and the high 16 bytes of its fragments
  // (the instruction reads four registers of each operand).  A and B_T share
  // the K order, which is all a plain product needs; kMx stores the
  // instruction K order (the fragment halves are then K-chunks g and g + 4,
  // the two halves of one MX scale pair).  Per-tensor epilogue.
  constexpr bool k4 = is_fp4(kFmt);
  static_assert(!k4 || kMf == 16, "fp4: 16x16x128");
  // fp6 (four elements per three bytes): a step is 128 elements, 96 bytes of
  // a row -- one MFMA per block, whose operands are six registers.  The
  // 96 bytes sit in slots 0-5 of the 128-byte LDS row (slots 6 and 7 stay
  // zero); each lane group reads its 24 bytes as three 8-byte pieces.
  constexpr bool k6 = is_fp6(kFmt);
  static_assert(!k6 || (kMf == 16 && !kMx), "fp6: 16x16x128, no MX");
  constexpr int kStep = k6 ? 96 : Cfg::kBK;  // bytes of a row per step
  constexpr int kMfmaPerBlock = k4 ? 2 : 1;
  // kMx scale words per step and MFMA: 8-bit steps take words 2s, 2s + 1 of
  // their pair's load; an fp4 step is a whole pair (its halves h take words
  // 2h, 2h + 1), so it loads its own words one step ahead and passes eight
  // per step.  Those loads are waited for by the next step's first barrier,
  // which must then retire everything but the 16 newest DMAs: the relaxed
  // waits past a tile's epilogue stores are not used.
  constexpr bool k4Mx = k4 && kMx;
  constexpr int kMxW = k4Mx ? 8 : 4;  // scale words per step
  constexpr bool k16 = kMf == 16;
  constexpr int kDmaPerGroup = 4;  // per wave
  constexpr int kWaitSteady = 4 * kDmaPerGroup;
  constexpr int kWaitAfterStores = kWaitSteady + Cfg::kStoresPerTile;
  static_assert(kWaitAfterStores < 64, "vmcnt range");
  const int lane = lane_id();
  const int wave = wave_id();
  const int wm = wave >> 1, wn = wave & 1;

  const int M = g.M, N = g.N, K = g.K;
  const int tiles_m = (M + Cfg::kBM - 1) / Cfg::kBM;
  const int tiles_n = (N + Cfg::kBN - 1) / Cfg::kBN;
  const int tiles = tiles_m * tiles_n;
  const int kt_real = (K + kStep - 1) / kStep;
  const int kt_pad = max(4, (kt_real + 1) & ~1);
  // Pair kt0 fetches steps kt0 + 2 and kt0 + 3.  The first pair whose DMAs
  // can reach a step that is not a whole step of the tile (index kt_full
  // and up: the step K ends inside, padding, the next tile's steps): the
  // smallest even kt0 >= kt_full - 3.
  const int kt_full = K / kStep;
  const int kt_edge = max(2, (kt_full - 2) & ~1);
  const int workers = g.workers > 0 ? min((int)gridDim.x, g.workers)
                                    : (int)gridDim.x;
  if ((int)blockIdx.x >= workers) return;
  const TileWalk walk = tile_walk(blockIdx.x, workers, tiles);
  int t = walk.first;
  if (t >= walk.end) return;

  // Per-tensor scales.
  const float sa = g.scale_a ? *g.scale_a : 1.0f;
  const float sb = g.scale_b ? *g.scale_b : 1.0f;
  const float scale = sa * sb;
  // Unit scale (no scales given, or their product exactly 1.0): the plain
  // epilogue skips its 256 multiplies per lane and tile.  x * 1.0f is x,
  // bit for bit, for every accumulator value (NaN and -0 included; a
  // subnormal fares the same in the multiply and in the conversion, which
  // share the denormal mode), so both paths write the same C.
  const bool unit_scale =
      __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, scale)) == 0x3f800000;

  // ---- DMA lane geometry: instruction q of wave w covers rows
  // (4q + w) * 8 .. +8; lane l takes row +l/8, slot l%8.  q in {0,1,4,5}
  // lands in rows 0-63 and 128-191 ("lo" group), q in {2,3,6,7} in rows
  // 64-127 and 192-255 ("hi" group).  kMx stores the instruction K order of
  // layout.hpp: slot l%8 holds K-chunk kpair_chunk((l%8) ^ slot_xor(row)).
  const int drow = lane >> 3;
  const int dslot = (lane & 7) ^ slot_xor(8 * (wave & 1) + drow);
  const int dchunk = kMx ? kpair_chunk(dslot) : dslot;
  // fp6: the lanes of slots 6 and 7 always read zero.
  const uint32_t pad6 = k6 && dchunk >= 6 ? kOobOffset : 0u;
  uint32_t voff_a[8], voff_b[8];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const int row = (4 * q + wave) * 8 + drow;
    voff_a[q] = ((uint32_t)row * (uint32_t)g.lda + dchunk * 16) | pad6;
    voff_b[q] = ((uint32_t)row * (uint32_t)g.ldb + dchunk * 16) | pad6;
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
  // 16x16x128: fragment row lane%16; lane group g = lane/16 reads slots 2g
  // and 2g + 1 (before the XOR; 32 bytes).  Any K order serves a plain
  // product as long as A and B share it: those slots hold K-chunks 2g and
  // 2g + 1.  Block scales need the instruction's own order -- lane group g
  // holds K 16g .. 16g + 15 in the first four registers and 64 + 16g ..
  // 64 + 16g + 15 in the last four -- which kMx gets from the DMA side (the
  // same slots then hold K-chunks g and g + 4).  Reading chunks g and g + 4
  // from slots g and g + 4 instead cost 4 LDS conflict cycles per read.
  const int rrow16 = lane & 15;
  const int rslot16 = (2 * (lane >> 4)) ^ slot_xor(rrow16);
  constexpr uint32_t kHalf16 = 16u;  // slot 2g -> 2g + 1
  const uint32_t off16_a =
      Cfg::kABase + (wm * 128 + rrow16) * Cfg::kBK + rslot16 * 16;
  const uint32_t off16_b =
      Cfg::kBBase + (wn * 128 + rrow16) * Cfg::kBK + rslot16 * 16;
  const lds_u8* pa16[2] = {lds + off16_a, lds + (off16_a ^ kHalf16)};
  const lds_u8* pb16[2] = {lds + off16_b, lds + (off16_b ^ kHalf16)};
  // fp6: lane group g = lane/16 holds bytes 24g .. 24g + 23 of the step
  // (element boundaries fall on 3-byte multiples), read as three 8-byte
  // pieces: piece p (byte b = 24g + 8p) of row r sits in slot
  // (b / 16) ^ slot_xor(r), half (b / 8) % 2.  Each 32-lane half of a read
  // covers 32 distinct 8-byte bank pairs.
  uint32_t p6[3];
#pragma unroll
  for (int q = 0; q < 3; ++q) {
    const int b = 24 * (lane >> 4) + 8 * q;
    p6[q] = (uint32_t)((((b >> 4) ^ slot_xor(rrow16)) << 4) + (((b >> 3) & 1) << 3));
  }
  const uint32_t row6_a = Cfg::kABase + (wm * 128 + rrow16) * Cfg::kBK;
  const uint32_t row6_b = Cfg::kBBase + (wn * 128 + rrow16) * Cfg::kBK;

  // K direction: where every step is whole (K a multiple of two steps, no
  // MX scales), every second tile of a workgroup walks K backwards.  Each
  // XCD's consecutive rounds share their A row panels (tile_walk), so a
  // round then starts on the K range the previous one ended on, which the
  // L2 and the 256 MB MALL still hold: 8192 x 8192 x 28672 (448 MiB of
  // operands) +1.6 %, 8192^3 and 8192 x 28672 x 8192 level (same process).
  // The fp32 sums run in the other order on those tiles (deterministic).
  const bool rev_ok = !kMx && K % (2 * kStep) == 0;
  bool rev_cur = false;
  TileSrc cur = tile_src(g, t, walk.end, tiles_m, tiles_n);
  TileSrc nxt = tile_src(g, t + walk.stride, walk.end, tiles_m, tiles_n);

  // DMA of one sub-buffer group of pipeline step kb into `stage`: operand op
  // (0 = A, 1 = B), half hi (0 = lo group, 1 = hi group).  Steps kb >= kt_pad
  // are steps kb - kt_pad of the next tile.  4 instructions per wave.
  // `edge` (std::true_type) DMAs may fetch the next tile's steps, a padding
  // step, or the step K ends inside (K not a multiple of 128): lanes whose
  // chunk lies at or past K get an out-of-range offset and read zero, one
  // VALU select per instruction.  The other DMAs (steady pairs, kt_edge)
  // fetch whole steps of the current tile and take the lane offsets as they
  // are: a select on every DMA was 24 VALU per wave-step and cost 2-4 % at
  // 4096^3 .. 8192x8192x28672.
  struct DmaSrc {
    __amdgpu_buffer_rsrc_t src;
    uint32_t k0;
    bool ok;  // this lane's chunk is below K (read by edge DMAs only)
  };
  auto dma_src = [&](int kb, int op, auto edge) {
    constexpr bool kEdge = decltype(edge)::value;
    const bool next = kEdge && kb >= kt_pad;  // wave-uniform
    const int ks = next ? kb - kt_pad : kb;
    const bool rv = next ? (rev_ok && !rev_cur) : rev_cur;
    uint32_t k0 = (uint32_t)(rv ? kt_pad - 1 - ks : ks) * kStep;
    // Opaque to the optimiser: keeps the per-step lane masks from being
    // hoisted out of the tile loop (they would pin VGPRs and spill).
    asm volatile("" : "+s"(k0));
    return DmaSrc{op == 0 ? (next ? nxt.a : cur.a) : (next ? nxt.b : cur.b), k0,
                  (int)(k0 + dchunk * 16) < K};
  };
  // Instruction qq (0..3) of the group.
  auto dma_one = [&](const DmaSrc& d, int stage, int op, int hi, int qq,
                     auto edge) {
    constexpr bool kEdge = decltype(edge)::value;
    const int q = (qq & 1) + 4 * (qq >> 1) + 2 * hi;
    const uint32_t va = kEdge ? (d.ok ? voff_a[q] : kOobOffset) : voff_a[q];
    const uint32_t vb = kEdge ? (d.ok ? voff_b[q] : kOobOffset) : voff_b[q];
    if (op == 0)
      dma16(d.src, lds + Cfg::kABase + stage * Cfg::kAStage + (4 * q + wave) * 1024,
            va, d.k0);
    else
      dma16(d.src, lds + Cfg::kBBase + stage * Cfg::kBStage + (4 * q + wave) * 1024,
            vb, d.k0);
  };
  auto dma_group = [&](int kb, int stage, int op, int hi, auto edge) {
    const DmaSrc d = dma_src(kb, op, edge);
#pragma unroll
    for (int qq = 0; qq < kDmaPerGroup; ++qq) dma_one(d, stage, op, hi, qq, edge);
  };

  // kExt: the wave's 128 row scales, 128 column scales and 128 biases of
  // tile t, by DMA into the first 1.5 KiB of its epilogue stage (rows at +0,
  // columns at +512, bias at +1024), one float per lane (6 loads; rows past
  // M or columns past N read zero).  Issued at the tile's first barrier,
  // when the previous epilogue's LDS reads are done; retired by the K loop's
  // own vmcnt waits, so the epilogue only reads LDS (a load issued there
  // would retire behind the next tile's prefetch).  A null vector gets an
  // empty range (every lane reads zero); the epilogue substitutes 1.0 or
  // -0.0 for it.  The vectors' addresses are reloaded from the kernel
  // arguments (the kernel's only argument is the GemmArgs) and the lane
  // index goes through an opaque copy, so that nothing here is hoisted out
  // of the tile loop.
  auto scale_dma = [&](int tile) {
    const TileCoord sc = grouped_tile_u(tile, tiles_m, tiles_n, g.group_m);
    const EpiArgs ea = kernel_epi();
    const float* pr = ea.row_scale;
    const float* pc = ea.col_scale;
    const float* pbias = ea.bias;
    int ln = lane;
    asm volatile("" : "+v"(ln));
    lds_u8* dst = lds + Cfg::kStoreBase + wave * Cfg::kStoreStage;
    const __amdgpu_buffer_rsrc_t rr = make_rsrc(pr, pr ? (uint32_t)M * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rc = make_rsrc(pc, pc ? (uint32_t)N * 4u : 0u);
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(pbias, pbias ? (uint32_t)N * 4u : 0u);
    const uint32_t ro = (uint32_t)(sc.m * Cfg::kBM + wm * 128 + ln) * 4u;
    const uint32_t co = (uint32_t)(sc.n * Cfg::kBN + wn * 128 + ln) * 4u;
    dma4(rr, dst, ro);
    dma4(rr, dst + 256, ro + 256);
    dma4(rc, dst + 512, co);
    dma4(rc, dst + 768, co + 256);
    dma4(rb, dst + 1024, co);
    dma4(rb, dst + 1280, co + 256);
  };

  i32x8 fa[4][2], fb[4][2];  // 32x32x64: [32-row fragment][K-half]
  i32x8 fa16[8], fb16[8];    // 16x16x128: [16-row fragment]
  // Register tile (op, hi) of `stage`: rows 64hi .. 64hi + 63 of the wave's
  // 128 A (op 0) or B (op 1) rows, all 128 K-bytes.
  // 16x16x128: read n (0..7) of register tile (op, hi): fragment
  // 4 hi + n / 2, K-half n % 2.
  auto read16_one = [&](int op, int hi, int stage, int n) -> i32x4 {
    const int f = 4 * hi + n / 2;
    if (op == 0)
      return lds_read16(pa16[n % 2] + stage * Cfg::kAStage + f * 16 * Cfg::kBK);
    return lds_read16(pb16[n % 2] + stage * Cfg::kBStage + f * 16 * Cfg::kBK);
  };
  // fp6: read n (0..11) of register tile (op, hi): fragment 4 hi + n / 3,
  // piece n % 3.
  auto read6_one = [&](int op, int hi, int stage, int n) -> u32x2 {
    const int f = 4 * hi + n / 3;
    if (op == 0)
      return lds_read8(lds + row6_a + stage * Cfg::kAStage + f * 16 * Cfg::kBK + p6[n % 3]);
    return lds_read8(lds + row6_b + stage * Cfg::kBStage + f * 16 * Cfg::kBK + p6[n % 3]);
  };
  // The six registers of an fp6 operand (the MFMA reads no more).
  auto join6 = [](u32x2 a, u32x2 b, u32x2 c) {
    return i32x8{(int)a.x, (int)a.y, (int)b.x, (int)b.y, (int)c.x, (int)c.y, 0, 0};
  };
  auto read_tile = [&](int op, int hi, int stage) {
    if constexpr (k6) {
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        const i32x8 v = join6(read6_one(op, hi, stage, 3 * f),
                              read6_one(op, hi, stage, 3 * f + 1),
                              read6_one(op, hi, stage, 3 * f + 2));
        if (op == 0) fa16[4 * hi + f] = v;
        else fb16[4 * hi + f] = v;
      }
      return;
    }
    if constexpr (k16) {
#pragma unroll
      for (int f = 4 * hi; f < 4 * hi + 4; ++f) {
        if (op == 0) {
          const int o = stage * Cfg::kAStage + f * 16 * Cfg::kBK;
          fa16[f] = join(lds_read16(pa16[0] + o), lds_read16(pa16[1] + o));
        } else {
          const int o = stage * Cfg::kBStage + f * 16 * Cfg::kBK;
          fb16[f] = join(lds_read16(pb16[0] + o), lds_read16(pb16[1] + o));
        }
      }
      return;
    }
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

  f32x16 acc[4][4];   // 32x32x64 accumulators
  f32x4 acc16[8][8];  // 16x16x128 accumulators

  // Quarter (qi, qj): the wave's rows 64qi.. x columns 64qj.. (32x32x64:
  // blocks i in {2qi, 2qi+1} x j in {2qj, 2qj+1}, K-half major so the two
  // MFMA of one accumulator are 4 apart; 16x16x128: 4 x 4 blocks).
  // kMx: the scale words of the step the MFMA belong to, w = {A frags 0-3,
  // A frags 4-7, B frags 0-3, B frags 4-7} (one byte per fragment).
  // zc: the MFMA are the first of their blocks in a tile (accumulator
  // input zero; the overlapped epilogue, 16x16x128 without MX only).
  auto quarter_mfma = [&](int qi, int qj, int from, int to,
                          const uint32_t* w = nullptr, bool zc = false) {
    if constexpr (k16) {
#pragma unroll
      for (int n = from; n < to; ++n) {
        const int i = 4 * qi + quarter_row16(n), j = 4 * qj + quarter_col16(n);
        const f32x4 c0 = zc ? f32x4{} : acc16[i][j];
        if constexpr (k4Mx) {
          const i32x8& x = fb16[j];
          const i32x8& y = fa16[i];
          acc16[i][j] = mfma_16x16x128_mx<kFmtFp4, kFmtFp4>(
              x, y, acc16[i][j], w[2 + j / 4], w[i / 4], j % 4, i % 4);
          acc16[i][j] = mfma_16x16x128_mx<kFmtFp4, kFmtFp4>(
              __builtin_shufflevector(x, x, 4, 5, 6, 7, 0, 1, 2, 3),
              __builtin_shufflevector(y, y, 4, 5, 6, 7, 0, 1, 2, 3), acc16[i][j],
              w[6 + j / 4], w[4 + i / 4], j % 4, i % 4);
        } else if constexpr (kMx) {
          acc16[i][j] = mfma_16x16x128_mx<fmt_b(kFmt), fmt_a(kFmt)>(
              fb16[j], fa16[i], acc16[i][j], w[2 + j / 4], w[i / 4], j % 4,
              i % 4);
        } else if constexpr (k4) {
          const i32x8& x = fb16[j];
          const i32x8& y = fa16[i];
          acc16[i][j] = mfma_16x16x128<kFmtFp4, kFmtFp4>(x, y, c0);
          acc16[i][j] = mfma_16x16x128<kFmtFp4, kFmtFp4>(
              __builtin_shufflevector(x, x, 4, 5, 6, 7, 0, 1, 2, 3),
              __builtin_shufflevector(y, y, 4, 5, 6, 7, 0, 1, 2, 3), acc16[i][j]);
        } else {
          acc16[i][j] = mfma_16x16x128<fmt_b(kFmt), fmt_a(kFmt)>(
              fb16[j], fa16[i], c0);
        }
      }
      return;
    }
#pragma unroll
    for (int n = from; n < to; ++n) {
      const int kh = n / 4, i = 2 * qi + (n / 2) % 2, j = 2 * qj + n % 2;
      acc[i][j] = mfma_32x32x64<fmt_b(kFmt), fmt_a(kFmt)>(fb[j][kh], fa[i][kh],
                                                           acc[i][j]);
    }
  };
  using QS = QuarterShape<kMf>;
  // kMx: scale words of the current step pair (mxc: A words 0-3, B words
  // 4-7, as loaded), of the next pair (mxn, in flight), and of the previous
  // step (mxp, for the tail MFMA that crosses into the next step).
  uint32_t mxc[8] = {}, mxn[8] = {}, mxp[kMxW] = {};
  // Loads the scale words of the step pair starting at step kb2 (fp4: of
  // step kb2, a pair by itself; steps kb2 >= kt_pad: the next tile's) into
  // dst: two 16-byte loads per lane,
  // counted in vmcnt.  The whole offset is in the range-checked VGPR
  // offset: tiles past the last, 128-row groups past M / N and the padding
  // steps past the last pair read zero (scale 2^-127 on zero data).
  auto mx_load = [&](int kb2, uint32_t (&dst)[8]) {
    const bool next = kb2 >= kt_pad;
    const int tt = next ? t + walk.stride : t;
    const int p = (next ? kb2 - kt_pad : kb2) / (k4 ? 1 : 2);
    const MxArgs mx = kernel_mx();
    const int kel = k4 ? 2 * K : K;  // K in elements (K counts bytes of a row)
    const int P = mx_pairs(kel);
    const bool live = tt < walk.end && p < P;
    // Tile coordinates from the tile's operand windows (no integer division
    // in the K loop).
    const TileCoord c{next ? nxt.tm : cur.tm, next ? nxt.tn : cur.tn};
    const __amdgpu_buffer_rsrc_t ra =
        make_rsrc(mx.a, live ? (uint32_t)mx_packed_bytes(M, kel) : 0u);
    const __amdgpu_buffer_rsrc_t rb =
        make_rsrc(mx.b, live ? (uint32_t)mx_packed_bytes(N, kel) : 0u);
    const uint32_t vo = (uint32_t)lane * 16u;
    const i32x4 va = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
        ra, vo + (uint32_t)(((c.m * 2 + wm) * P + p) * 1024), 0, 0));
    const i32x4 vb = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(
        rb, vo + (uint32_t)(((c.n * 2 + wn) * P + p) * 1024), 0, 0));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      dst[q] = (uint32_t)va[q];
      dst[4 + q] = (uint32_t)vb[q];
    }
  };

  // The last quarter-step's tail (issued after the K loop, before the
  // epilogue reads the accumulators).
  auto last_tail = [&]() { quarter_mfma(1, 1, QS::kHead, QS::kMfma, mxp); };

  // One quarter-step: the previous quarter's tail MFMA (quarter tq) if
  // `tail`, the head MFMA of quarter q, the LDS reads of register tile
  // (rop, rhi) of stage rst, and DMA group (dop, dhi) of step kb into stage
  // dst, in the order of quarter_schedule_32.  For 16x16x128 the order is
  // written out, one scheduling region per pair: given only the
  // sched_group_barrier pattern, the scheduler clustered the DMAs (DDDD) and
  // the reads in some quarters of some instantiations, and which ones moved
  // with unrelated changes elsewhere in the kernel (3-7 % slower when it
  // hit the default instantiation; tests/test_isa_schedule.py checks the
  // built loops).
  // kMx: w / wt are the scale words of this quarter's step and of the
  // tail's.
  // ep(n): epilogue work woven into slot n (0..14, after head MFMA n) and
  // n = 15 (after the last head MFMA) of a 16x16x128 quarter with 8-bit or
  // fp4 operands; see the overlapped epilogue below.  Every other caller
  // passes no_ep.
  auto no_ep = [](int) {};
  // zh / zt: the head / tail MFMA start their blocks (quarter_mfma's zc).
  auto quarter = [&](auto edge, bool tail, int tqi, int tqj, int qi, int qj,
                     int rop, int rhi, int rst, int kb, int dst, int dop, int dhi,
                     const uint32_t* w, const uint32_t* wt, auto&& ep,
                     bool zh = false, bool zt = false) {
    if constexpr (k16) {
      if (tail) quarter_mfma(tqi, tqj, QS::kHead, QS::kMfma, wt, zt);
      const DmaSrc d = dma_src(kb, dop, edge);
      sched_fence();
      if constexpr (k6) {
        // 12 eight-byte reads: [M R] x 8, [M D R] x 4, [M] x 3.
        u32x2 rd6[12];
#pragma unroll
        for (int n = 0; n < 8; ++n) {
          quarter_mfma(qi, qj, n, n + 1, w);
          rd6[n] = read6_one(rop, rhi, rst, n);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          sched_fence();
        }
#pragma unroll
        for (int n = 0; n < 4; ++n) {
          quarter_mfma(qi, qj, 8 + n, 9 + n, w);
          dma_one(d, dst, dop, dhi, n, edge);
          rd6[8 + n] = read6_one(rop, rhi, rst, 8 + n);
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          sched_fence();
        }
        quarter_mfma(qi, qj, 12, QS::kHead, w);
#pragma unroll
        for (int f = 0; f < 4; ++f) {
          const i32x8 v = join6(rd6[3 * f], rd6[3 * f + 1], rd6[3 * f + 2]);
          if (rop == 0) fa16[4 * rhi + f] = v;
          else fb16[4 * rhi + f] = v;
        }
        return;
      }
      i32x4 rd[8];
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        quarter_mfma(qi, qj, n, n + 1, w, zh);
        rd[n] = read16_one(rop, rhi, rst, n);
        ep(n);
        __builtin_amdgcn_sched_group_barrier(0x008, kMfmaPerBlock, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        sched_fence();
      }
#pragma unroll
      for (int n = 0; n < 4; ++n) {
        quarter_mfma(qi, qj, 8 + n, 9 + n, w, zh);
        dma_one(d, dst, dop, dhi, n, edge);
        ep(8 + n);
        __builtin_amdgcn_sched_group_barrier(0x008, kMfmaPerBlock, 0);
        __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
        sched_fence();
      }
#pragma unroll
      for (int n = 12; n < QS::kHead; ++n) {
        quarter_mfma(qi, qj, n, n + 1, w, zh);
        ep(n);
        sched_fence();
      }
      ep(QS::kHead);
#pragma unroll
      for (int f = 0; f < 4; ++f) {
        if (rop == 0)
          fa16[4 * rhi + f] = join(rd[2 * f], rd[2 * f + 1]);
        else
          fb16[4 * rhi + f] = join(rd[2 * f], rd[2 * f + 1]);
      }
    } else {
      if (tail) quarter_mfma(tqi, tqj, QS::kHead, QS::kMfma);
      quarter_mfma(qi, qj, 0, QS::kHead);
      read_tile(rop, rhi, rst);
      dma_group(kb, dst, dop, dhi, edge);
      quarter_schedule_32(tail);
    }
  };

  // The previous tile's epilogue stores are in flight (every tile but the
  // workgroup's first).
  bool stores_in_flight = false;
  // Two pipeline steps kt0, kt0 + 1 (stages 0, 1).  kFirst: the tile's first
  // two steps, whose first three barriers wait past the previous tile's
  // epilogue stores.
  // edge: std::true_type when one of the pair's DMAs may fetch a step that
  // K ends inside (see dma_src).
  auto step_pair = [&](int kt0, auto first, auto edge) {
    constexpr bool kFirst = decltype(first)::value;
    // One barrier per half step (before quarters 00 and 10).  Quarter q
    // refills, for step kt + 2, the LDS group whose last read was at least
    // two quarters earlier, behind one of those barriers:
    //   Q00: A lo (read at step kt - 1, Q10)   Q01: B lo (step kt - 1, Q11)
    //   Q10: B hi (step kt, Q00)               Q11: A hi (step kt, Q01)
    // and each group lands 5-6 quarters before its first read.  At a
    // barrier the group to be read next was issued 16 DMAs (4 quarters)
    // earlier, plus the previous tile's 32 stores for the first three
    // barriers of a tile.  Between the barriers only the wave's own LDS
    // reads are waited for.
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int kt = kt0 + s;
      const bool tail = !(kFirst && s == 0);
      wait_lgkmcnt<0>();
      if (kFirst && stores_in_flight && !k4Mx) wait_vmcnt<kWaitAfterStores>();
      else wait_vmcnt<kWaitSteady>();
      // After the wait (which counts only older operations): the six loads
      // at most make the tile's next two waits retire six more stores.
      if constexpr (kExt && kFirst)
        if (s == 0) scale_dma(t);
      barrier();  // Q00
      // kMx: this step's scale words; the next pair's are loaded here (after
      // the wait, like scale_dma: at most two more stores retired early).
      uint32_t w[kMxW];
      if constexpr (k4Mx) {
        // halves 0 and 1 of this step: A words 0-1, B words 0-1, then A
        // words 2-3, B words 2-3 of its load; the next step's words now.
        const uint32_t ws[8] = {mxc[0], mxc[1], mxc[4], mxc[5],
                                mxc[2], mxc[3], mxc[6], mxc[7]};
#pragma unroll
        for (int q = 0; q < 8; ++q) w[q] = ws[q];
        mx_load(kt + 1, mxn);
      } else {
        w[0] = mxc[2 * s];
        w[1] = mxc[2 * s + 1];
        w[2] = mxc[4 + 2 * s];
        w[3] = mxc[4 + 2 * s + 1];
        if constexpr (kMx)
          if (s == 0) mx_load(kt0 + 2, mxn);
      }
      quarter(edge, tail, 1, 1, 0, 0, 1, 1, s, kt + 2, s, 0, 0, w, mxp, no_ep);
      wait_lgkmcnt<0>();  // Q01
      quarter(edge, true, 0, 0, 0, 1, 0, 1, s, kt + 2, s, 1, 0, w, w, no_ep);
      wait_lgkmcnt<0>();
      if (kFirst && s == 0 && stores_in_flight && !k4Mx) wait_vmcnt<kWaitAfterStores>();
      else wait_vmcnt<kWaitSteady>();
      barrier();  // Q10
      quarter(edge, true, 0, 1, 1, 0, 0, 0, s ^ 1, kt + 2, s, 1, 1, w, w, no_ep);
      wait_lgkmcnt<0>();  // Q11
      quarter(edge, true, 1, 0, 1, 1, 1, 0, s ^ 1, kt + 2, s, 0, 1, w, w, no_ep);
      if constexpr (kMx)
#pragma unroll
        for (int q = 0; q < kMxW; ++q) mxp[q] = w[q];
      if constexpr (k4Mx)
#pragma unroll
        for (int q = 0; q < 8; ++q) mxc[q] = mxn[q];
    }
    if constexpr (kMx && !k4Mx)
#pragma unroll
      for (int q = 0; q < 8; ++q) mxc[q] = mxn[q];
  };

  // ---- Overlapped epilogue (plain bf16 output, 16-byte stores, 16x16x128,
  // 8-bit or fp4 operands) ---------------------------------------------------
  // A wave's 128 x 128 accumulators are four 64 x 64 quadrants d = 2 qi + qj
  // (rows 64 qi.., columns 64 qj..; blocks acc16[4 qi ..][4 qj ..]).  Quadrant
  // d is final once quarter-step Qd of a tile's last step (L) has issued its
  // tail MFMA -- at the start of the next quarter -- and is next written by
  // quarter Qd of the next tile's first step (0').  Its conversion and its
  // stores therefore run inside the MFMA stream of the quarters between:
  //   Q01(L): convert 0              Q10(L): store 0, convert 1
  //   Q11(L): store 1, convert 2     Q00(0'): store 2, convert 3
  //   Q01(0'): store 3
  // "Convert" is 16 blocks (acc * scale -> bf16 RNE -> the wave's 8 KiB LDS
  // stage), one block per MFMA slot, the block whose tail MFMA opened the
  // quarter last; the quarter ends by reading the quadrant back (16
  // ds_read_b64 per lane, into 32 VGPRs).  "Store" is 8 buffer_store_dwordx4
  // of whole 128-byte lines (8 rows x 128 B each), one per slot of the
  // quarter's first half, ahead of its DMAs.  The quarters after the stores
  // wait for them in vmcnt order: the barrier waits of Q00(0') / Q10(0') /
  // Q00(1') allow 32 / 48 / 32 operations (16 DMAs plus the stores issued in
  // the four quarters since the group they need), and every store has had
  // five quarter-steps when Q10(1') waits with the steady 16.  Without a
  // next tile, the rest of the epilogue runs after the K loop (drain).
  //
  // Stage layout: row r (0..63) of the quadrant at 128 r; its 8-byte piece x
  // (columns 4 x .. 4 x + 3) at slot x ^ stage_xor(r) (layout.hpp): block
  // writes and read-backs without LDS bank conflicts.
  constexpr bool kOverlap = kLine && k16 && kVecStore && !kExt && !kMx && !k6;
  struct EpiTile {
    __amdgpu_buffer_rsrc_t rsrc;  // the tile's window of C
    int rows_left, cols_left;     // rows / columns of C from the wave's origin
  };
  auto epi_tile = [&](int tile) {
    const TileCoord tc = grouped_tile_u(tile, tiles_m, tiles_n, g.group_m);
    const int rows_c = min(Cfg::kBM, M - tc.m * Cfg::kBM);
    return EpiTile{
        make_rsrc(reinterpret_cast<uint8_t*>(g.C) +
                      ((size_t)tc.m * Cfg::kBM * g.ldc + (size_t)tc.n * Cfg::kBN) * 2,
                  (uint32_t)(((rows_c - 1) * g.ldc + Cfg::kBN) * 2)),
        M - tc.m * Cfg::kBM - wm * 128, N - tc.n * Cfg::kBN - wn * 128};
  };
  lds_u8* const epi_stg = lds + Cfg::kStoreBase + wave * Cfg::kStoreStage;
  // kOobOffset when x >= limit, as plain arithmetic (no lane masks).
  auto oob_unless = [](int x, int limit) -> uint32_t {
    return (uint32_t)((limit - 1 - x) >> 31) & kOobOffset;
  };
  u32x2 epi_rd[16];  // read-back quadrant: store p, 8-byte half h at [2p + h]
  // The epilogue work of one quarter: store quadrant sq (from epi_rd) and
  // convert quadrant vq (-1: none), for tile window et.  Lane-derived
  // addresses hang off an opaque copy of the lane id (computed per quarter,
  // not hoisted into the K loop).
  auto epi_work = [&](int sq, int vq, const EpiTile& et) {
    int el = lane;
    asm volatile("" : "+v"(el));
    const int wl = el & 15, wg = el >> 4;
    // write: block (bi, bj) (rows 16 bi + wl, piece 4 bj + wg) at
    // bi * 2048 + (wbase ^ 32 bj)
    const int sw = stage_xor(wl);
    const uint32_t wbase =
        (uint32_t)(wl * 128 + (((wg ^ sw) & 3) << 3) + ((sw >> 2) << 5));
    const int rl = el >> 3, c = el & 7;
    // read-back p: pieces 2c and 2c + 1 of row 8p + rl, at p * 1024 + (rbase
    // ^ 64 (p % 2)) and that ^ 8 (stage_xor(8 + r) = 8 + stage_xor(r))
    const uint32_t rbase = (uint32_t)(rl * 128 + (((2 * c) ^ stage_xor(rl)) << 3));
    const uint32_t vst = (uint32_t)((rl * g.ldc + wn * 128 + 8 * c) * 2);
    // acc16, epi_rd and et by reference: the conversion clears the
    // accumulators and the read-back fills epi_rd for the next quarter.
    return [&, sq, vq, wbase, rbase, vst, rl, c](int slot) {
      if (sq >= 0 && slot < 8) {
        const int qi = sq >> 1, qj = sq & 1, p = slot;
        int row8 = 64 * qi + 8 * p;
        asm volatile("" : "+s"(row8));  // recompute per store, never hoist
        const int srow = __builtin_amdgcn_readfirstlane((wm * 128 + row8) * g.ldc * 2);
        const u32x2 lo = epi_rd[2 * p], hi = epi_rd[2 * p + 1];
        store_b128<kStoreC>(
            i32x4{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y}, et.rsrc,
            (vst | oob_unless(64 * qj + 8 * c, et.cols_left) |
             oob_unless(row8 + rl, et.rows_left)) + 128 * qj,
            srow);
      }
      if (vq >= 0) {
        const int qi = vq >> 1, qj = vq & 1;
        auto convert = [&](int b) {
          const int bi = b >> 2, bj = b & 3;
          const f32x4& a = acc16[4 * qi + bi][4 * qj + bj];
          lds_write8(epi_stg + bi * 2048 + (wbase ^ (uint32_t)(32 * bj)),
                     u32x2{pack_bf16x2(acc_read(a[0]) * scale, acc_read(a[1]) * scale),
                           pack_bf16x2(acc_read(a[2]) * scale, acc_read(a[3]) * scale)});
        };
        if (slot < QS::kHead) convert(slot);
        if (slot == QS::kHead - 1) convert(QS::kHead);
        if (slot == QS::kHead) {
#pragma unroll
          for (int p = 0; p < 8; ++p) {
            const uint32_t o = (uint32_t)(p * 1024) + (rbase ^ (uint32_t)((p & 1) << 6));
            epi_rd[2 * p] = lds_read8(epi_stg + o);
            epi_rd[2 * p + 1] = lds_read8(epi_stg + (o ^ 8u));
          }
        }
      }
    };
  };

  // One pipeline step pair of the overlapped schedule (kOverlap).  kMode:
  // 0 an ordinary pair; 1 the workgroup's first pair (no tail MFMA before
  // its first quarter); 2 a tile's last pair (quadrants 0-2 of this tile's
  // epilogue in its second step); 3 a tile's first pair after another tile
  // (that tile's tail MFMA, quadrant 3 and the last stores in its first
  // step).  The barrier waits count the stores (see above).
  auto step_pair_ov = [&](int kt0, auto mode, auto edge, const EpiTile& et) {
    constexpr int kMode = decltype(mode)::value;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int kt = kt0 + s;
      const bool tail = !(kMode == 1 && s == 0);
      const bool e2 = kMode == 2 && s == 1, e3 = kMode == 3 && s == 0;
      // The tile's first step: its MFMA start from zero; so does the tail
      // of its last quarter, issued in the next step's first quarter.
      const bool z = (kMode == 1 || kMode == 3) && s == 0;
      const bool z00 = (kMode == 1 || kMode == 3) && s == 1;
      wait_lgkmcnt<0>();
      if (kMode == 3) wait_vmcnt<kWaitSteady + 16>();
      else wait_vmcnt<kWaitSteady>();
      barrier();  // Q00
      if (e3) quarter(edge, tail, 1, 1, 0, 0, 1, 1, s, kt + 2, s, 0, 0, nullptr, nullptr, epi_work(2, 3, et), z, z00);
      else quarter(edge, tail, 1, 1, 0, 0, 1, 1, s, kt + 2, s, 0, 0, nullptr, nullptr, no_ep, z, z00);
      wait_lgkmcnt<0>();  // Q01
      if (e2) quarter(edge, true, 0, 0, 0, 1, 0, 1, s, kt + 2, s, 1, 0, nullptr, nullptr, epi_work(-1, 0, et), z, z);
      else if (e3) quarter(edge, true, 0, 0, 0, 1, 0, 1, s, kt + 2, s, 1, 0, nullptr, nullptr, epi_work(3, -1, et), z, z);
      else quarter(edge, true, 0, 0, 0, 1, 0, 1, s, kt + 2, s, 1, 0, nullptr, nullptr, no_ep, z, z);
      wait_lgkmcnt<0>();
      if (e3) wait_vmcnt<kWaitSteady + 32>();
      else wait_vmcnt<kWaitSteady>();
      barrier();  // Q10
      if (e2) quarter(edge, true, 0, 1, 1, 0, 0, 0, s ^ 1, kt + 2, s, 1, 1, nullptr, nullptr, epi_work(0, 1, et), z, z);
      else quarter(edge, true, 0, 1, 1, 0, 0, 0, s ^ 1, kt + 2, s, 1, 1, nullptr, nullptr, no_ep, z, z);
      wait_lgkmcnt<0>();  // Q11
      if (e2) quarter(edge, true, 1, 0, 1, 1, 1, 0, s ^ 1, kt + 2, s, 0, 1, nullptr, nullptr, epi_work(1, 2, et), z, z);
      else quarter(edge, true, 1, 0, 1, 1, 1, 0, s ^ 1, kt + 2, s, 0, 1, nullptr, nullptr, no_ep, z, z);
    }
  };

  // Prologue of the first tile: steps 0 and 1 (groups A lo, B lo, B hi,
  // A hi each), then a_lo(0), b_lo(0) into registers once step 0 landed:
  // step 1's 16 DMAs are the newest and vmcnt retires in issue order.  The
  // first tile has no epilogue stores in flight, so its waits are the
  // steady ones (stores_in_flight false), which retire step 1's groups one
  // half-step before they are read, as for any later step.  A single round
  // over the CUs thus starts after one step of DMA instead of two.  kMx
  // waits for everything: its scale loads follow the DMAs.
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    dma_group(st, st, 0, 0, std::true_type{});
    dma_group(st, st, 1, 0, std::true_type{});
    dma_group(st, st, 1, 1, std::true_type{});
    dma_group(st, st, 0, 1, std::true_type{});
  }
  if constexpr (kMx) {
    mx_load(0, mxc);
    wait_vmcnt<0>();
  } else {
    wait_vmcnt<kWaitSteady>();
  }
  barrier();
  read_tile(0, 0, 0);
  read_tile(1, 0, 0);

  if constexpr (kOverlap) {
    const EpiTile none{};
    step_pair_ov(0, std::integral_constant<int, 1>{}, std::true_type{}, none);
    for (;;) {
      int kt0 = 2;
      for (; kt0 < kt_edge; kt0 += 2)
        step_pair_ov(kt0, std::integral_constant<int, 0>{}, std::false_type{}, none);
      for (; kt0 < kt_pad - 2; kt0 += 2)
        step_pair_ov(kt0, std::integral_constant<int, 0>{}, std::true_type{}, none);
      const EpiTile et = epi_tile(t);
      step_pair_ov(kt_pad - 2, std::integral_constant<int, 2>{}, std::true_type{}, et);
      t += walk.stride;
      if (t >= walk.end) {
        // Drain: the last quarter's tail MFMA, then quadrant 3 without a
        // next tile to hide it in.
        quarter_mfma(1, 1, QS::kHead, QS::kMfma);
        asm volatile("" : "+a"(acc16[4 + quarter_row16(QS::kHead)]
                                    [4 + quarter_col16(QS::kHead)]));
        mfma_drain();
        wait_lgkmcnt<0>();
        auto ep = epi_work(2, 3, et);
#pragma unroll
        for (int n = 0; n <= QS::kHead; ++n) ep(n);
        wait_lgkmcnt<0>();
        auto ep3 = epi_work(3, -1, et);
#pragma unroll
        for (int n = 0; n < 8; ++n) ep3(n);
        break;
      }
      cur = nxt;
      rev_cur = rev_ok && !rev_cur;
      nxt = tile_src(g, t + walk.stride, walk.end, tiles_m, tiles_n);
      step_pair_ov(0, std::integral_constant<int, 3>{}, std::true_type{}, et);
    }
    // The last tile's look-ahead DMA (all zeros) still lands in LDS, and
    // the last stores are in flight.
    wait_vmcnt<0>();
    return;
  } else {
  // Lane-derived epilogue values hang off an opaque copy of the lane id so
  // the optimiser cannot hoist them out of the tile loop, where they would
  // stay live through the K loop and spill.
  for (;;) {
    if constexpr (k16) {
#pragma unroll
      for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc16[i][j] = f32x4{};
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16{};
    }

    // Edge DMAs for the first pair (one per tile) and from kt_edge on.
    step_pair(0, std::true_type{}, std::true_type{});
    int kt0 = 2;
    for (; kt0 < kt_edge; kt0 += 2)
      step_pair(kt0, std::false_type{}, std::false_type{});
    for (; kt0 < kt_pad; kt0 += 2)
      step_pair(kt0, std::false_type{}, std::true_type{});

    last_tail();
    // The tail's accumulator is read only by the epilogue's explicit
    // v_accvgpr_read, which hazard tracking does not see: an empty asm that
    // takes it ties the MFMA to this point, so that no pass sinks it into the
    // epilogue past mfma_drain() (with a branch in the epilogue, machine
    // sinking moved it next to the first read, which then read a stale
    // accumulator).
    if constexpr (k16)
      asm volatile("" : "+a"(acc16[4 + quarter_row16(QS::kHead)]
                                  [4 + quarter_col16(QS::kHead)]));
    else
      asm volatile("" : "+a"(acc[3][3]));
    sched_fence();

    // ---- epilogue --------------------------------------------------------
    // The accumulators are read by explicit v_accvgpr_read (acc_read), which
    // the compiler's hazard tracking does not see: give the last MFMA its
    // result latency first.
    mfma_drain();
    // acc[i][j] holds D = B_blk . A_blk^T, i.e. C^T for the 32x32 block:
    // lane l, register r -> C row (l % 32), C column 8*(r/4) + 4*(l/32) + r%4,
    // so each lane holds 4 consecutive bf16 (8 bytes) per (i, j, r/4).
    // Out-of-range bit for "x < limit" as plain arithmetic (no lane masks,
    // which would pin scalar register pairs): kOobOffset when x >= limit.
    int elane = lane;
    asm volatile("" : "+v"(elane));
    const TileCoord tc = grouped_tile_u(t, tiles_m, tiles_n, g.group_m);
    const int rows_c = min(Cfg::kBM, M - tc.m * Cfg::kBM);
    // Every store is a buffer store over this tile's window of C; a lane
    // whose row or columns fall outside M x N gets an out-of-range offset and
    // its write is dropped by the hardware range check -- no branches.
    constexpr int es = kExt ? out_bytes(kOut) : 2;  // bytes per C element
    const __amdgpu_buffer_rsrc_t rsrc_c = make_rsrc(
        reinterpret_cast<uint8_t*>(g.C) +
            ((size_t)tc.m * Cfg::kBM * g.ldc + (size_t)tc.n * Cfg::kBN) * es,
        (uint32_t)(((rows_c - 1) * g.ldc + Cfg::kBN) * es));
    const int rows_left = M - tc.m * Cfg::kBM - wm * 128;  // from wave row 0
    const int cols_left = N - tc.n * Cfg::kBN - wn * 128;  // from wave col 0
    // Elements of 16 x 16 block (bi, bj), packed.  kExt: the vectors come
    // from the wave's stage (scale_dma), read before the staging of C
    // overwrites them.
    EpiVec<8, 8> ev;
    if constexpr (kExt)
      ev.read_lds(lds + Cfg::kStoreBase + wave * Cfg::kStoreStage,
                  kernel_epi(), scale, elane);
    // The epilogue proper.
    // `scaled`: std::true_type multiplies by the per-tensor scale,
    // std::false_type (unit scale, plain epilogue) does not.
    auto store_tile = [&](auto scaled) {
    auto sc = [&](float x) {
      if constexpr (decltype(scaled)::value) return x * scale;
      else return x;
    };
    auto cvt4 = [&](const f32x16& v, int q) {
      return u32x2{pack_bf16x2(sc(acc_read(v[4 * q + 0])), sc(acc_read(v[4 * q + 1]))),
                   pack_bf16x2(sc(acc_read(v[4 * q + 2])), sc(acc_read(v[4 * q + 3])))};
    };
    auto pack16 = [&](const f32x4& a, int bi, int bj) -> u32x2 {
      if constexpr (kExt)
        return ev.template pack4<kAct, kOut>(acc_read(a[0]), acc_read(a[1]),
                                               acc_read(a[2]), acc_read(a[3]),
                                               bi, bj);
      else
        return u32x2{pack_bf16x2(sc(acc_read(a[0])), sc(acc_read(a[1]))),
                     pack_bf16x2(sc(acc_read(a[2])), sc(acc_read(a[3])))};
    };

    if constexpr (kExt && kOut == kOutF8 && kVecStore) {
      // e4m3 output, 16-column groups (N, ldc multiples of 16): 32 rows at a
      // time through the wave's own LDS (128 bytes per row; the 4-byte piece
      // x = 4 j + l / 16 of row r at slot x ^ 4 ((r / 2) % 8): each write
      // instruction covers 16 rows x 4 pieces, each read 8 rows x 8 lanes of
      // 16 bytes -- both conflict-free), then 16-byte stores of whole
      // 128-byte row segments (8 rows per instruction).
      lds_u8* stg = lds + Cfg::kStoreBase + wave * Cfg::kStoreStage;
      const int wr = elane & 15, wg = elane >> 4;
      const int q = elane & 7, rsub = elane >> 3;
      const uint32_t vcol = (uint32_t)(rsub * g.ldc + wn * 128 + 16 * q);
      const uint32_t col_oob = oob_unless(16 * q, cols_left);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii)
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int bi = 2 * i + ii, r = 16 * ii + wr;
            const f32x4& a = acc16[bi][j];
            const uint32_t w = ev.e4m3x4(ev.template value4<kAct>(
                acc_read(a[0]), acc_read(a[1]), acc_read(a[2]), acc_read(a[3]), bi, j));
            lds_write4(stg + r * 128 + (((4 * j + wg) ^ (4 * ((r >> 1) & 7))) * 4), w);
            sched_fence();  // bound the live range: one block at a time
          }
        compiler_fence();
        i32x4 v[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          const int r = 8 * p + rsub;
          v[p] = lds_read16(stg + r * 128 + ((q ^ ((r >> 1) & 7)) * 16));
        }
        compiler_fence();
#pragma unroll
        for (int p = 0; p < 4; ++p) {
          int row8 = 32 * i + 8 * p;
          asm volatile("" : "+s"(row8));  // recompute per store, never hoist
          const int srow = __builtin_amdgcn_readfirstlane((wm * 128 + row8) * g.ldc);
          store_b128<kStoreC>(
              v[p], rsrc_c, vcol | col_oob | oob_unless(row8 + rsub, rows_left), srow);
        }
        compiler_fence();
        sched_fence();
      }
    } else if constexpr (kExt && kOut >= kOutF32) {
      // fp32 / e4m3 output: straight from the accumulators, no staging --
      // block (i, j): lane l -> row 16 i + l % 16, columns 16 j + 4 (l / 16)
      // .. + 3, one 16-byte (fp32) or 4-byte (e4m3) store per lane, or one
      // per element when N, ldc or C's alignment rule that out.
      const uint32_t vlane =
          (uint32_t)(((elane & 15) * g.ldc + wn * 128 + 4 * (elane >> 4)) * es);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int srow =
            __builtin_amdgcn_readfirstlane((wm * 128 + 16 * i) * g.ldc * es);
        const uint32_t vrow = vlane | oob_unless(16 * i + (elane & 15), rows_left);
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int c = 16 * j + 4 * (elane >> 4);
          const f32x4& a = acc16[i][j];
          const f32x4 v = ev.template value4<kAct>(acc_read(a[0]), acc_read(a[1]),
                                                   acc_read(a[2]), acc_read(a[3]),
                                                   i, j);
          if constexpr (kOut == kOutF32) {
            if constexpr (kVecStore) {
              store_b128<kStoreCPart>(
                  __builtin_bit_cast(i32x4, v), rsrc_c,
                  (vrow | oob_unless(c, cols_left)) + 16 * j * es, srow);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                __builtin_amdgcn_raw_buffer_store_b32(
                    (uint32_t)__builtin_bit_cast(i32x4, v)[e], rsrc_c,
                    (vrow | oob_unless(c + e, cols_left)) + (16 * j + e) * es,
                    srow, kStoreCPart);
            }
          } else {
            const uint32_t w = ev.e4m3x4(v);
            if constexpr (kVecStore) {
              __builtin_amdgcn_raw_buffer_store_b32(
                  w, rsrc_c, (vrow | oob_unless(c, cols_left)) + 16 * j * es, srow,
                  kStoreCPart);
            } else {
#pragma unroll
              for (int e = 0; e < 4; ++e)
                __builtin_amdgcn_raw_buffer_store_b8(
                    (uint8_t)(w >> (8 * e)), rsrc_c,
                    (vrow | oob_unless(c + e, cols_left)) + (16 * j + e) * es,
                    srow, kStoreCPart);
            }
          }
          sched_fence();  // bound the live range: one block at a time
        }
      }
    } else if constexpr (kVecStore) {
      // 32 rows (one accumulator block row i) at a time through the wave's
      // own 8 KiB: row r at 256 r; the 8-byte piece x (0..31) of the row at
      // slot x ^ r.  Writes: lanes 0-31 (one 8-byte piece each of rows
      // 0-31) hit 32 distinct slots; reads (two 8-byte pieces per lane, 16
      // lanes per row, two rows per 32 lanes) likewise -- no bank conflicts
      // with 64 four-byte banks.  No barrier: the region is the wave's own,
      // and one wave's LDS operations complete in order.
      lds_u8* stg = lds + Cfg::kStoreBase + wave * Cfg::kStoreStage;
      // read: store p (0..7) covers rows 4p + l/16, 16-byte chunk l % 16
      const int rsub = elane >> 4, chunk = elane & 15;
      const uint32_t vcol = (uint32_t)((rsub * g.ldc + wn * 128 + 8 * chunk) * 2);
      const uint32_t col_oob = oob_unless(8 * chunk, cols_left);
      auto store_chunk = [&](int i, const i32x4 (&v)[8]) {
#pragma unroll
        for (int p = 0; p < 8; ++p) {
          int row4 = 32 * i + 4 * p;
          asm volatile("" : "+s"(row4));  // recompute per store, never hoist
          const int srow =
              __builtin_amdgcn_readfirstlane((wm * 128 + row4) * g.ldc * 2);
          store_b128<kStoreC>(
              v[p], rsrc_c, vcol | col_oob | oob_unless(row4 + rsub, rows_left),
              srow);
        }
      };
      if constexpr (k16) {
        // Blocks (2i + ii, j): lane l holds row 16 ii + l%16, 8-byte piece
        // 4j + l/16; piece x of row r at 8-byte slot x ^ (r % 16).  Each
        // write instruction's 16 lanes of one piece index (16 rows) then
        // cover 16 distinct slots modulo 16, which rocprof reads as no bank
        // conflict (the slot x ^ 2(r % 16) used before cost 4 conflict
        // cycles per write, 1024 per tile).  Chunk k of row r (pieces 2k,
        // 2k + 1) is the 16-byte unit k ^ ((r % 16) / 2), its halves swapped
        // on odd rows; each row's 16 lanes read 16 distinct units.
        //
        // Software-pipelined over the four 32-row chunks: chunk i is read
        // back, then chunk i + 1 is converted and written into the same
        // 8 KiB between chunk i's 8 stores.  One wave's LDS operations
        // complete in issue order, so the reads of chunk i return it before
        // the writes of chunk i + 1 land; the conversions overlap the
        // stores instead of waiting for them.
        const int wr = elane & 15, wg = elane >> 4;
        auto write_blk = [&](int i, int ii, int j) {
          const int bi = 2 * i + ii;
          const f32x4& a = acc16[bi][j];
          lds_write8(stg + (16 * ii + wr) * 256 + (((4 * j + wg) ^ wr) * 8),
                     pack16(a, bi, j));
        };
        auto store_one = [&](int i, int p, const i32x4& v) {
          int row4 = 32 * i + 4 * p;
          asm volatile("" : "+s"(row4));  // recompute per store, never hoist
          const int srow =
              __builtin_amdgcn_readfirstlane((wm * 128 + row4) * g.ldc * 2);
          store_b128<kStoreC>(
              v, rsrc_c, vcol | col_oob | oob_unless(row4 + rsub, rows_left),
              srow);
        };
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
#pragma unroll
          for (int j = 0; j < 8; ++j) write_blk(0, ii, j);
          sched_fence();  // bound the live range
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          compiler_fence();
          i32x4 v[8];
#pragma unroll
          for (int p = 0; p < 8; ++p) {
            const int r = 4 * p + rsub;
            v[p] = lds_read16(stg + r * 256 + ((chunk ^ ((r & 15) >> 1)) * 16));
            if (r & 1) v[p] = i32x4{v[p][2], v[p][3], v[p][0], v[p][1]};
          }
          compiler_fence();
#pragma unroll
          for (int p = 0; p < 8; ++p) {
            store_one(i, p, v[p]);
            if (i < 3) {
              write_blk(i + 1, p / 4, 2 * (p % 4));
              write_blk(i + 1, p / 4, 2 * (p % 4) + 1);
            }
            sched_fence();
          }
        }
      } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        i32x4 v[8];
        {
          // 32 rows (one accumulator block row i) through the wave's own
          // 8 KiB: row r at 256 r; the 8-byte piece x (0..31) of the row at
          // slot x ^ r.  Writes: lanes 0-31 (one 8-byte piece each of rows
          // 0-31) hit 32 distinct slots; reads (two 8-byte pieces per lane,
          // 16 lanes per row, two rows per 32 lanes) likewise -- no bank
          // conflicts with 64 four-byte banks.
          const int wr = elane & 31, wh = elane >> 5;
          const uint32_t wbase = wr * 256;
#pragma unroll
          for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q)
              lds_write8(stg + wbase + (((2 * (4 * j + q) + wh) ^ wr) * 8),
                         cvt4(acc[i][j], q));
            sched_fence();  // bound the live range: one block at a time
          }
          compiler_fence();
#pragma unroll
          for (int p = 0; p < 8; ++p) {
            const int r = 4 * p + rsub;
            const u32x2 lo = lds_read8(stg + r * 256 + (((2 * chunk) ^ r) * 8));
            const u32x2 hi = lds_read8(stg + r * 256 + (((2 * chunk + 1) ^ r) * 8));
            v[p] = i32x4{(int)lo.x, (int)lo.y, (int)hi.x, (int)hi.y};
          }
        }
        // all reads of the chunk first (above), then its 8 stores; no
        // barrier: the region is the wave's own, and one wave's LDS
        // operations complete in order
        store_chunk(i, v);
        compiler_fence();
        sched_fence();
      }
      }
    } else {
      // N, ldc or C's alignment rule out 16-byte stores: stores straight
      // from the accumulators, lane masks as out-of-range offsets -- one
      // 8-byte store of four columns per lane and block when N and ldc are
      // multiples of 4 and C is 8-byte aligned (a wave-uniform choice; at
      // 8192 x 8188 x 8192 2-byte stores ran at a third of the aligned
      // rate), else one 2-byte store per element.
      if constexpr (k16) {
        // block (i, j): lane l -> row 16 i + l%16, columns 16 j + 4(l/16) + r
        const bool four = ((g.N | g.ldc) & 3) == 0 &&
                          (reinterpret_cast<uintptr_t>(g.C) & 7) == 0;
        const uint32_t vlane =
            (uint32_t)(((elane & 15) * g.ldc + wn * 128 + 4 * (elane >> 4)) * 2);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const int srow =
              __builtin_amdgcn_readfirstlane((wm * 128 + 16 * i) * g.ldc * 2);
          const uint32_t vrow =
              vlane | oob_unless(16 * i + (elane & 15), rows_left);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            const int c = 16 * j + 4 * (elane >> 4);
            const f32x4& a = acc16[i][j];
            const u32x2 v = pack16(a, i, j);
            if (four) {
              __builtin_amdgcn_raw_buffer_store_b64(
                  v, rsrc_c, (vrow | oob_unless(c, cols_left)) + 16 * j * 2, srow,
                  kStoreCPart);
            } else {
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const uint32_t w = (r < 2 ? v.x : v.y) >> (16 * (r & 1));
                __builtin_amdgcn_raw_buffer_store_b16(
                    (unsigned short)w, rsrc_c,
                    (vrow | oob_unless(c + r, cols_left)) + (16 * j + r) * 2,
                    srow, kStoreCPart);
              }
            }
            sched_fence();  // bound the live range: one block at a time
          }
        }
      } else {
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
                    srow, kStoreCPart);
              }
            }
            sched_fence();  // bound the live range: one block at a time
          }
        }
      }
    }
    };  // store_tile
    if constexpr (kExt)
      store_tile(std::true_type{});
    else if (unit_scale)
      store_tile(std::false_type{});
    else
      store_tile(std::true_type{});
    stores_in_flight = true;

    t += walk.stride;
    if (t >= walk.end) break;
    cur = nxt;
    rev_cur = rev_ok && !rev_cur;
    nxt = tile_src(g, t + walk.stride, walk.end, tiles_m, tiles_n);
  }
  // The last tile's look-ahead DMA (all zeros) still lands in LDS: let it
  // finish before the workgroup's LDS can be handed to another workgroup.
  wait_vmcnt<0>();
  }
}

}  // namespace detail
}  // namespace hipgemm
