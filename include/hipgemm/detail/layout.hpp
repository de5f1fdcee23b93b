// hipgemm -- data layout rules shared by host and device code.
//
// 1. LDS tile layout ("128-byte rows, XOR-swizzled 16-byte slots").
//    A K-stage of an operand tile holds R rows x 128 K-bytes, row r at LDS
//    bytes [128 r, 128 r + 128) as eight 16-byte slots; slot s of row r holds
//    global K-chunk (s ^ slot_xor(r)) of that row.  The DMA writes each
//    instruction's 64 lanes x 16 B linearly (8 rows x 128 B, every global
//    request a whole 128-byte line), so the permutation is applied on the
//    global side: DMA lane l fetches chunk (l%8) ^ slot_xor(row).
//
//    slot_xor(r) = (r & 7) ^ ((r >> 3) & 1) depends on r mod 16 only.  An
//    MFMA operand fetch reads 16 consecutive rows (lane % 16) per 16-lane
//    group g.  Measured on gfx950 (SQ_LDS_BANK_CONFLICT of single
//    ds_read_b128 patterns): the groups reading slots 2g ^ slot_xor(r) -- or
//    (2g + 1) ^ slot_xor(r) -- cost no conflict cycle; slots g ^ slot_xor(r)
//    or (g + 4) ^ slot_xor(r) cost 4 per instruction, and 4 to 12 under six
//    other per-row XORs tried; under r & 7 (strip_xor, below) they cost
//    none.  In the 8 slots of a 16-row block each row parity gets 8
//    distinct slots (tests/test_layout.py checks this through the built
//    library).
//
//    Instruction K order.  The f8f6f4 MFMA's lane group g holds K-chunks g
//    and g + 4 of its row (K 16g .. 16g + 15 and 64 + 16g .. 64 + 16g + 15).
//    Kernels that need that order (block scales; fp4's two MFMA per step;
//    operands paired with register-loaded ones) store chunk c at slot
//    kpair_slot(c) ^ slot_xor(r): chunks g and g + 4 then sit at slots 2g and
//    2g + 1 (before the XOR), the measured conflict-free reads.  Their DMA
//    lane l fetches chunk kpair_chunk((l % 8) ^ slot_xor(row)).
//
// 2. Output tile order ("XCD-contiguous, grouped columns").
//    The dispatcher hands workgroup b to XCD b % 8.  tile_of_block() first
//    turns b into a logical index such that each XCD owns one contiguous run
//    of logical indices (exact for any grid size), then walks the tile grid
//    in groups of `group_m` tile rows, column by column inside a group, so
//    the workgroups resident on one XCD share A rows and B columns in its L2.
//    Bijective on [0, tiles) for every grid, tiles_m, tiles_n, group_m >= 1.
//
// Reference counterparts: fp8_4wave.hpp:136-177 (a different swizzle, row
// pairs XORed with (r >> 1) & 7) and :357-377 (a remap that is a bijection only when the
// grid is a multiple of 8).
#pragma once

#include <hip/hip_runtime.h>

namespace hipgemm {
namespace detail {

constexpr int kNumXcds = 8;

__host__ __device__ constexpr int slot_xor(int r) { return (r & 7) ^ ((r >> 3) & 1); }
// Epilogue stage of the 4-wave schedule's overlapped epilogue: 64 rows of
// 128 bytes, the 8-byte piece x (0..15) of row r at 8-byte slot
// x ^ stage_xor(r), which depends on r mod 16 only.  Its block writes
// (ds_write_b64: lane l writes one piece of row l % 16) and read-backs
// (ds_read_b64: lane l reads piece 2 (l % 8) + h of row l / 8) measured no
// SQ_LDS_BANK_CONFLICT cycle on gfx950, where a probe replaying each pattern
// measured, per instruction (write, read-back): x ^ (r mod 16) 0 and 2,
// x ^ ((r & 14) | ((r >> 1) & 1)) 4 and 0, this layout 0 and 0.  The two
// conditions that fit: the 16 rows of a block take 16 distinct slots
// (stage_xor is a permutation of r mod 16), and rows r and r + 2 opposite
// slot parities.
__host__ __device__ constexpr int stage_xor(int r) { return (r & 15) ^ ((r >> 1) & 1); }
// B_T stages of the column-strip schedule: 128-byte rows in the plain K
// order, K-chunk c of row r at slot c ^ strip_xor(r), read by lane group g at
// chunks g and g + 4 (the order of its register-loaded A).  Measured on
// gfx950 (ds_read_b128, 16 rows per lane group): this swizzle gives those
// reads no conflict cycle, where slot_xor gives 4 per instruction; its chunk
// 2g / 2g + 1 reads would cost 4.  Each DMA lane quad still fetches one
// aligned 64-byte half of a line.
__host__ __device__ constexpr int strip_xor(int r) { return r & 7; }
// Instruction K order: slot (before the XOR) of K-chunk c, and its inverse.
__host__ __device__ constexpr int kpair_slot(int c) { return ((c & 3) << 1) | (c >> 2); }
__host__ __device__ constexpr int kpair_chunk(int s) { return ((s & 1) << 2) | (s >> 1); }

struct TileCoord {
  int m, n;
};

// Tiles of persistent workgroup b among `workers`: first, first + stride,
// ... while < end.  The workgroups of XCD x (blocks b = x mod G, G =
// min(8, workers)) share one contiguous range of tile indices, sized in
// proportion to their number, and stride through it; the ranges of all XCDs
// partition [0, tiles), so every tile is visited exactly once.  Each XCD thus
// sweeps one band of consecutive tiles for the whole run (grouped_tile maps
// it to a few row panels, all columns) instead of a new band every round:
// its L2 keeps serving the same A panels.
struct TileWalk {
  int first, stride, end;
};
__host__ __device__ inline TileWalk tile_walk(int b, int workers, int tiles) {
  const int G = workers < kNumXcds ? workers : kNumXcds;
  const int x = b % G, l = b / G;
  const int per = workers / G, extra = workers % G;
  const int n = per + (x < extra ? 1 : 0);
  const int before = x * per + (x < extra ? x : extra);
  const int start = (int)((long long)tiles * before / workers);
  const int end = (int)((long long)tiles * (before + n) / workers);
  return TileWalk{start + l, n, end};
}

// Tile (m, n) for logical tile index t in [0, tiles_m * tiles_n).
__host__ __device__ inline TileCoord grouped_tile(int t, int tiles_m,
                                                  int tiles_n, int group_m) {
  const int per_group = group_m * tiles_n;
  const int g = t / per_group, r = t % per_group;
  const int m0 = g * group_m;
  const int rows = (tiles_m - m0) < group_m ? (tiles_m - m0) : group_m;
  return TileCoord{m0 + r % rows, r / rows};
}

// grouped_tile in device code, for a wave-uniform t, with both coordinates
// moved to scalar registers.  Integer division has no scalar instruction, so
// the quotients are computed by VALU; left in VGPRs, a buffer resource built
// from them counts as divergent, and every buffer instruction that takes it
// is wrapped in a readfirstlane loop (12 extra instructions and a branch per
// store in the 4-wave epilogue).
__device__ __forceinline__ TileCoord grouped_tile_u(int t, int tiles_m,
                                                    int tiles_n, int group_m) {
  const TileCoord c = grouped_tile(t, tiles_m, tiles_n, group_m);
  return TileCoord{__builtin_amdgcn_readfirstlane(c.m),
                   __builtin_amdgcn_readfirstlane(c.n)};
}

}  // namespace detail
}  // namespace hipgemm
