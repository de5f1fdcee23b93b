// hipgemm -- data layout rules shared by host and device code.
//
// 1. LDS tile layout ("64-byte rows, XOR-swizzled 16-byte slots").
//    A K-stage of an operand tile holds R rows x 64 K-bytes.  Row r occupies
//    LDS bytes [64 r, 64 r + 64) as four 16-byte slots; slot s of row r holds
//    global K-chunk (s ^ slot_xor(r)) of that row.  The DMA writes each
//    instruction's 64 lanes x 16 B linearly, so the permutation is applied on
//    the global side: DMA lane l fetches chunk (l%4) ^ slot_xor(row).
//
//    slot_xor depends on r mod 16 only and is chosen so that ds_read_b128 by
//    an MFMA operand fetch (16 consecutive rows at one K-chunk per 16-lane
//    group) touches 16 distinct 16-byte bank groups out of 256 bytes, and
//    every 8-lane half of it 8 distinct groups out of 128 bytes: bank-conflict
//    free whether the LDS serves 256 or 128 bytes per cycle.  Proof sketch for
//    r = (r3 r2 r1 r0): slot_xor = ((r3 ^ r1) << 1) | r2.
//      - 16 rows, one residue r mod 4 = (r1 r0): (r3, r2) -> slot_xor is a
//        bijection, and the row's bank offset is 64 * (r mod 4).
//      - 8 rows (r3 fixed), one parity r0: (r2, r1) -> slot_xor is a
//        bijection, and the row's offset mod 128 is 64 * r0.
//    tests/test_layout.py checks both properties exhaustively.
//
// 2. Output tile order ("XCD-contiguous, grouped columns").
//    The dispatcher hands workgroup b to XCD b % 8.  tile_of_block() first
//    turns b into a logical index such that each XCD owns one contiguous run
//    of logical indices (exact for any grid size), then walks the tile grid
//    in groups of `group_m` tile rows, column by column inside a group, so
//    the workgroups resident on one XCD share A rows and B columns in its L2.
//    Bijective on [0, tiles) for every grid, tiles_m, tiles_n, group_m >= 1.
//
// Reference counterparts: fp8_4wave.hpp:136-177 (a different swizzle over
// 128-byte rows) and :357-377 (a remap that is a bijection only when the
// grid is a multiple of 8).
#pragma once

#include <hip/hip_runtime.h>

namespace hipgemm {
namespace detail {

constexpr int kNumXcds = 8;

__host__ __device__ constexpr int slot_xor(int r) {
  return ((((r >> 3) ^ (r >> 1)) & 1) << 1) | ((r >> 2) & 1);
}

struct TileCoord {
  int m, n;
};

// Logical position of workgroup `b` once each XCD's workgroups are made
// contiguous: XCD x receives blocks x, x+8, x+16, ...; it owns logical
// indices [start(x), start(x) + count(x)).
__host__ __device__ inline int xcd_contiguous(int b, int grid) {
  const int x = b % kNumXcds, j = b / kNumXcds;
  const int per = grid / kNumXcds, extra = grid % kNumXcds;
  return x * per + (x < extra ? x : extra) + j;
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

}  // namespace detail
}  // namespace hipgemm
