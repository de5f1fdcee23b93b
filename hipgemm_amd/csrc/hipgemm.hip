// hipgemm -- C ABI implementation (libhipgemm.so).
//
// Argument validation, variant selection and kernel launches over
// hipLaunchKernel.  The kernels are the header schedules of
// include/hipgemm/detail/, instantiated with runtime shapes in the k*.hip
// files of this directory (kernels.hpp looks them up by configuration).
#include "hipgemm.h"

#include <atomic>
#include <cstdint>

#include "kernels.hpp"

namespace {

using namespace hipgemm::detail;
namespace hk = hipgemm::kernels;

static_assert(HIPGEMM_ACT_NONE == kActNone && HIPGEMM_ACT_RELU == kActRelu &&
                  HIPGEMM_ACT_GELU_TANH == kActGeluTanh &&
                  HIPGEMM_ACT_SILU == kActSilu,
              "activation codes");
static_assert(HIPGEMM_OUT_BF16 == kOutBf16 && HIPGEMM_OUT_F16 == kOutF16 &&
                  HIPGEMM_OUT_F32 == kOutF32 && HIPGEMM_OUT_FP8_E4M3 == kOutF8,
              "output codes");
static_assert(HIPGEMM_FMT_E4M3 == kFmtE4M3 && HIPGEMM_FMT_E5M2 == kFmtE5M2,
              "format codes");

// 32-bit buffer offsets: 256 rows of A or B_T (1-byte elements) span at most
// 2^31 bytes, 256 rows of C likewise (ldc * element size <= 2^23 bytes).
constexpr int kMaxLd = 1 << 23;
constexpr int kMaxLdcBytes = 1 << 23;

bool aligned(const void* p, uintptr_t a) {
  return (reinterpret_cast<uintptr_t>(p) & (a - 1)) == 0;
}

// es: bytes per element of C.
hipError_t validate(const void* A, const void* B_T, void* C, int M, int N,
                    int K, int lda, int ldb, int ldc, int variant, int es) {
  if (M < 0 || N < 0 || K < 0) return hipErrorInvalidValue;
  if (variant < 0 || variant >= HIPGEMM_VARIANT_COUNT)
    return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  if (!C || !aligned(C, es) || ldc < N || ldc > kMaxLdcBytes / es)
    return hipErrorInvalidValue;
  if (K == 0) return hipSuccess;  // A and B_T are not read
  if (!A || !B_T) return hipErrorInvalidValue;
  if (K % 16 != 0) return hipErrorInvalidValue;
  if (lda < K || ldb < K || lda % 16 != 0 || ldb % 16 != 0)
    return hipErrorInvalidValue;
  if (lda > kMaxLd || ldb > kMaxLd) return hipErrorInvalidValue;
  if (!aligned(A, 16) || !aligned(B_T, 16)) return hipErrorInvalidValue;
  return hipSuccess;
}

int tiles_of(int M, int N) {
  return ((M + Cfg4w::kBM - 1) / Cfg4w::kBM) * ((N + Cfg4w::kBN - 1) / Cfg4w::kBN);
}

// Compute units of the current device, queried once per device (a lazily
// filled, thread-safe cache; concurrent first calls store the same value).
int cu_count() {
  static std::atomic<int> cached[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) !=
            hipSuccess ||
        n <= 0)
      n = 256;
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

// One store per lane of `group` consecutive elements of C (of output type
// out): N and ldc multiples of the group, C aligned to the group's bytes.
bool vec_ok(int out, int N, int ldc, const void* C, int group) {
  const int bytes = group * out_bytes(out);
  return N % group == 0 && ldc % group == 0 && aligned(C, (uintptr_t)bytes);
}

// Rows of a 2-byte C start on 128-byte lines: the 4-wave schedule's
// overlapped epilogue (Key::line).
bool line_ok(int out, int ldc, const void* C) {
  return out_bytes(out) == 2 && ldc % 64 == 0 && aligned(C, 128);
}

// The tiled schedules (4-wave, 8-wave) on a persistent grid: one workgroup
// per CU at most (their 160 KiB of LDS allows no more), each walking tiles
// w, w + grid, ...  `key.vec` is set here: 16-byte epilogue stores need
// 8-column groups that never straddle N and 16-byte aligned rows.
hipError_t launch_tiled(int variant, GemmArgs g, hk::Key key,
                        hipStream_t stream) {
  const int bm = variant == HIPGEMM_VARIANT_TILE128 ? CfgT128::kBM : Cfg4w::kBM;
  const int bn = variant == HIPGEMM_VARIANT_TILE128 ? CfgT128::kBN : Cfg4w::kBN;
  const int tm = (g.M + bm - 1) / bm, tn = (g.N + bn - 1) / bn;
  const int tiles = tm * tn;
  g.group_m = default_group_m(tm, tn);
  const int cus = cu_count();
  const int grid = tiles < cus ? tiles : cus;
  g.workers = grid;
  // 2-byte types: 16-byte stores of 8 staged elements; fp32: one store of 4
  // elements straight from the accumulators; e4m3: 16 staged elements on
  // the 4-wave schedule, 4 from the accumulators on the 128 x 128 one.
  const bool t128 = variant == HIPGEMM_VARIANT_TILE128;
  key.vec = vec_ok(key.out, g.N, g.ldc, g.C,
                   key.out == kOutF8 ? (t128 ? 4 : 16) : key.out == kOutF32 ? 4 : 8);
  key.line = line_ok(key.out, g.ldc, g.C);
  const void* fn = nullptr;
  int threads = Cfg4w::kThreads;
  switch (variant) {
    case HIPGEMM_VARIANT_TILE128:
      fn = g.mx.a   ? hk::tile128_mx(key)
           : key.ext ? hk::tile128_ext(key)
                     : hk::tile128_plain(key);
      threads = CfgT128::kThreads;
      break;
    case HIPGEMM_VARIANT_8WAVE:
      fn = !key.ext ? hk::eight_wave_plain(key)
           : key.out == HIPGEMM_OUT_F16 ? hk::eight_wave_ext_f16(key)
                                        : hk::eight_wave_ext_bf16(key);
      threads = Cfg8w::kThreads;
      break;
    case HIPGEMM_VARIANT_4WAVE:
      fn = key.ext ? nullptr : hk::four_wave_plain(32, key);
      break;
    default:
      if (g.mx.a) {
        fn = hk::four_wave_mx(key);
        break;
      }
      fn = !key.ext ? hk::four_wave_plain(16, key)
           : key.out >= kOutF32          ? hk::four_wave_ext_wide(key)
           : key.out == HIPGEMM_OUT_F16 ? hk::four_wave_ext_f16(key)
                                        : hk::four_wave_ext_bf16(key);
      break;
  }
  if (!fn) return hipErrorInvalidValue;  // no such instantiation
  void* args[] = {&g};
  return hipLaunchKernel(fn, dim3(grid), dim3(threads), args, 0, stream);
}

// AUTO's column split (hipgemm_split_columns): g4 columns [0, n1) on the
// 4-wave 16x16x128 schedule, g1 columns [n1, N) on the 128 x 128 one.  One
// persistent launch (ksplit_plain.hip) where both take the per-tensor
// epilogue with 16-byte stores and 8-bit operands: each workgroup runs its
// 4-wave tiles, then its 128 x 128 ones, so the second part starts on every
// CU as the first finishes there, without a launch between them.  Else the
// two schedules one after the other.
hipError_t launch_split(GemmArgs g4, GemmArgs g1, hk::Key key,
                        hipStream_t stream) {
  if (!key.ext && key.fmt < 4 && !g4.mx.a &&
      vec_ok(key.out, g4.N, g4.ldc, g4.C, 8) &&
      vec_ok(key.out, g1.N, g1.ldc, g1.C, 8)) {
    const int cus = cu_count();
    auto prep = [&](GemmArgs& g, int bm, int bn) {
      const int tm = (g.M + bm - 1) / bm, tn = (g.N + bn - 1) / bn;
      g.group_m = default_group_m(tm, tn);
      g.workers = tm * tn < cus ? tm * tn : cus;
    };
    prep(g4, Cfg4w::kBM, Cfg4w::kBN);
    prep(g1, CfgT128::kBM, CfgT128::kBN);
    key.vec = true;
    key.line = line_ok(key.out, g4.ldc, g4.C);
    if (const void* fn = hk::split_plain(key)) {
      void* args[] = {&g4, &g1};
      const int grid = g4.workers > g1.workers ? g4.workers : g1.workers;
      return hipLaunchKernel(fn, dim3(grid), dim3(Cfg4w::kThreads), args, 0,
                             stream);
    }
  }
  hipError_t e = launch_tiled(HIPGEMM_VARIANT_4WAVE_MFMA16, g4, key, stream);
  if (e != hipSuccess) return e;
  return launch_tiled(HIPGEMM_VARIANT_TILE128, g1, key, stream);
}

// Split-K plan of the skinny schedule: 16-row blocks of M, column tiles of
// 64 kf columns (kf B_T fragments per wave), K-slices per column tile
// (enough workgroups to give every CU one, or two, below), and the
// workspace it needs (arrival counters, then the partial tiles).
//
// Workspace layout, shared by every schedule so that calls of different
// schedules may share one workspace: bytes [0, HIPGEMM_WS_COUNTER_BYTES)
// are arrival counters, zero between calls (a call that uses them leaves
// them zero; no call writes anything else there); partial tiles start at
// HIPGEMM_WS_COUNTER_BYTES and are fully written before they are read.
constexpr size_t kWsCounterBytes = HIPGEMM_WS_COUNTER_BYTES;
constexpr int kWsMaxCounters = (int)(kWsCounterBytes / sizeof(int));

struct SkinnyPlan {
  int kmb, kf, bn, tiles_n, slices, slice_steps;
  size_t counter_bytes, ws_bytes;
};

// Long slices: as many workgroups as two per CU hold (the kernel's LDS and
// registers allow two), when each slice keeps at least 12 steps to amortise
// its partial tile.  The second workgroup on a CU doubles the loads in
// flight there, and the per-CU miss path is this kernel's bound.  Same
// process against one workgroup per CU: 128 x 8192 x 16384 +27 %, x 28672
// +29 %, x 12288 +7 %, 128 x 4096 x 28672 +8 %; with 8 steps per slice
// (128 x 8192 x 8192) -2 %, with 4 (x 4096) -25 %.  The grid stays within
// 2 x CUs workgroups, so the workspace within 512 partial tiles.
//
// From 65 rows the column tile is 64 instead of 128 columns when only the
// narrower tile reaches two workgroups per CU: 128 x 8192 x 8192 +8 %,
// 96 x 8192 x 8192 +9 %, 128 x 4096 x 14336 +7 % (each workgroup reads all
// of A for its K-slice, so a narrower tile costs A traffic, and where the
// 128-column tile already has two workgroups per CU, or neither has,
// 64 columns measured 3-11 % slower).
// unsplit: one K-slice (no workspace), for a call under stream capture
// that brings no workspace.
SkinnyPlan plan_skinny(int M, int N, int K, bool unsplit = false) {
  const int kmb = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8;
  const int steps = (K + CfgSkinny::kBK - 1) / CfgSkinny::kBK;
  const int cus = cu_count();
  auto plan = [&](int kf, bool* two) {
    SkinnyPlan p{};
    p.kmb = kmb;
    p.kf = kf;
    p.bn = CfgSkinny::bn_of(kf);
    p.tiles_n = (N + p.bn - 1) / p.bn;
    int slices = (cus + p.tiles_n - 1) / p.tiles_n;
    const int slices2 = 2 * cus / p.tiles_n;
    *two = slices2 > slices && steps >= 12 * slices2;
    if (*two) slices = slices2;
    if (slices > steps) slices = steps;
    if (unsplit) slices = 1;
    // One counter per column tile: more tiles than the counter region holds
    // (never with slices > 1 on a GPU of at most 4096 CUs) run unsplit.
    if (slices < 1 || p.tiles_n > kWsMaxCounters) slices = 1;
    p.slice_steps = steps > 0 ? (steps + slices - 1) / slices : 0;
    p.slices = p.slice_steps > 0 ? (steps + p.slice_steps - 1) / p.slice_steps : 1;
    if (p.slices > 1) {
      p.counter_bytes = kWsCounterBytes;
      p.ws_bytes = p.counter_bytes + (size_t)p.tiles_n * p.slices * p.kmb * 16 *
                                         p.bn * sizeof(float);
    }
    return p;
  };
  bool two = false, two1 = false;
  const SkinnyPlan p = plan(CfgSkinny::frags(kmb), &two);
  if (kmb == 8 && !two) {
    const SkinnyPlan p1 = plan(1, &two1);
    if (two1) return p1;
  }
  return p;
}

hipError_t launch_skinny(const GemmArgs& a, const SkinnyPlan& p, void* ws,
                         hk::Key key, hipStream_t stream) {
  // From 4 row blocks up, one workgroup per column tile summing every slice
  // is the long pole when the tile's partials are large (1 MiB at M = 128
  // with 16 slices): a second kernel sums them over tiles_n x kmb
  // workgroups instead.  With small partials (at most 32 KiB per slice and
  // 96 KiB for the last arrival to read) the last arrival sums them itself:
  // one launch fewer.  Same process: 128 x 8192 x 8192 (64-column tiles, 4
  // slices) +3.8 %, 64 x 28672 x 4096 (2 slices of 32 KiB) +4.7 %; with 8
  // slices (128 x 4096 x 14336) or 64 KiB per slice (128 x 28672 x 8192) it
  // measured equal or 3 % slower, so those keep the second kernel.
  const size_t partial = (size_t)p.kmb * 16 * p.bn * sizeof(float);
  const bool small = partial <= (32u << 10) && (size_t)(p.slices - 1) * partial <= (96u << 10);
  const int reduce_pass = p.slices > 1 && p.kmb >= 4 && !small;
  SkinnyArgs g{a.A, a.B, a.C, a.scale_a, a.scale_b, a.M, a.N, a.K,
               a.lda, a.ldb, a.ldc, p.slices, p.slice_steps, nullptr, nullptr,
               reduce_pass, a.epi};
  if (p.slices > 1) {
    g.arrivals = static_cast<int*>(ws);
    g.partial = reinterpret_cast<float*>(static_cast<char*>(ws) + p.counter_bytes);
  }
  // One store per lane of 4 columns that never straddle N.
  key.vec = vec_ok(key.out, a.N, a.ldc, a.C, 4);
  const int grid = p.tiles_n * p.slices;
  const void* fn = key.ext ? hk::skinny_ext(p.kmb, p.kf, key)
                           : hk::skinny_plain(p.kmb, p.kf, key);
  if (!fn) return hipErrorInvalidValue;
  void* args1[] = {&g};
  hipError_t e = hipLaunchKernel(fn, dim3(grid), dim3(CfgSkinny::kThreads),
                                 args1, 0, stream);
  if (e != hipSuccess || !reduce_pass) return e;
  int kmb = p.kmb;
  void* args[] = {&g, &kmb};
  return hipLaunchKernel(hk::skinny_reduce(p.kf, key),
                         dim3(p.tiles_n * p.kmb),
                         dim3(CfgSkinny::kThreads), args, 0, stream);
}

// Plan of the column-strip schedule (gemm_strip.hpp): 16-row blocks of M,
// strips of 16 knb columns, and K-slices per strip when the strips alone
// give fewer workgroups than CUs (each wave keeps at least one step of a
// slice); the workspace holds the counters and one partial strip per
// (strip, slice).
struct StripPlan {
  int kmb, knb, tiles_n, slices, slice_steps;
  size_t ws_bytes;
};

StripPlan plan_strip(int M, int N, int K, int knb, bool unsplit = false) {
  StripPlan p{};
  // 16-row blocks: 1, 2, 3, 4 or 8.  Three for 33-48 rows instead of four
  // (A loads and MFMA for the rows that exist): same process, bit-identical,
  // 4-6 % faster (40 x 8192 x 8192 17.74 -> 16.82 us, 48 x 28672 x 4096
  // 31.69 -> 29.96, 40 x 4096 x 4096 9.68 -> 9.21).
  p.kmb = M <= 16 ? 1 : M <= 32 ? 2 : M <= 48 ? 3 : M <= 64 ? 4 : 8;
  p.knb = knb;
  const int bn = 16 * knb;
  p.tiles_n = (N + bn - 1) / bn;
  const int steps = (K + CfgStrip::kBK - 1) / CfgStrip::kBK;
  const int cus = cu_count();
  // At most one workgroup per CU: a K-slice count rounded up would put a
  // second workgroup on some CUs, which then take twice as long.
  int slices = cus / p.tiles_n;
  if (slices > steps / 4) slices = steps / 4;
  if (slices < 1 || p.tiles_n > kWsMaxCounters || unsplit) slices = 1;
  p.slice_steps = steps > 0 ? (steps + slices - 1) / slices : 0;
  p.slices = p.slice_steps > 0 ? (steps + p.slice_steps - 1) / p.slice_steps : 1;
  if (p.slices > 1)
    p.ws_bytes = kWsCounterBytes + (size_t)p.tiles_n * p.slices *
                                       CfgStrip::partial_bytes(p.kmb, p.knb);
  return p;
}

// The strip width.  Every strip reads all of A's rows over its K range
// through its CU's L1, so A's share of a CU's traffic grows with M / BN;
// narrower strips give more workgroups, fewer K-slices and smaller partial
// strips for the last arrival to sum.  32 columns, except 64 where
// 32-column strips outnumber the CUs (from 17 rows), and above 40 rows
// with K > 4096 where the 32-column plan fills at most 3/4 of the CUs, or
// fewer than all of them with K >= 12288 and the 64-column plan in at most
// 2 K-slices, or at N = 8192 above 56 rows.  Measured (one process, caller
// workspace, 32 / 64 columns, us): 40 x 14336 x 8192 32.7 / 25.4,
// 56 x 14336 x 8192 37.9 / 28.1, 32 x 28672 x 8192 50.5 / 45.2,
// 16 x 28672 x 8192 40.4 / 40.8; 64 x 3072 x 8192 14.8 / 13.4,
// 64 x 6144 x 8192 21.5 / 19.7, 60 x 7168 x 12288 31.6 / 27.0,
// 64 x 8192 x 8192 21.9 / 21.1; but 60 x 1536 x 6144 9.7 / 13.4
// (64-column strips: 10 K-slices), 44 x 3584 x 6144 12.3 / 13.3,
// 64 x 4096 x 8192 15.1 / 15.4, 40 x 8192 x 8192 17.7 / 18.9,
// 64 x 2048 x 4096 9.8 / 12.4, 64 x 1024 x 8192 10.1 / 15.1.  Over 54
// such pairs this choice is 0.2 % behind the faster on average.
int strip_knb(int M, int N, int K) {
  const int cus = cu_count();
  const int steps = (K + CfgStrip::kBK - 1) / CfgStrip::kBK;
  auto slices_of = [&](int strips) {
    const int s = cus / strips < steps / 4 ? cus / strips : steps / 4;
    return s < 1 ? 1 : s;
  };
  const int tiles = (N + 31) / 32;
  if (tiles > cus) return M > 16 ? 4 : 2;
  if (M <= 40 || K <= 4096) return 2;
  const int busy = tiles * slices_of(tiles);  // workgroups at 32 columns
  if (4 * busy <= 3 * cus) return 4;
  if (busy < cus && K >= 12288 && slices_of((N + 63) / 64) <= 2) return 4;
  return M > 56 && N >= 8192 ? 4 : 2;
}

hipError_t launch_strip(const GemmArgs& a, const StripPlan& p, void* ws,
                        hk::Key key, hipStream_t stream) {
  StripArgs g{a.A, a.B, a.C, a.scale_a, a.scale_b, a.M, a.N, a.K,
              a.lda, a.ldb, a.ldc, p.slices, p.slice_steps, nullptr, nullptr,
              a.epi};
  if (p.slices > 1) {
    g.arrivals = static_cast<int*>(ws);
    g.partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kWsCounterBytes);
  }
  // One store per lane of 4 columns that never straddle N.
  key.vec = vec_ok(key.out, a.N, a.ldc, a.C, 4);
  const void* fn = key.ext ? hk::strip_ext(p.kmb, p.knb, key)
                           : hk::strip_plain(p.kmb, p.knb, key);
  if (!fn) return hipErrorInvalidValue;
  void* args[] = {&g};
  return hipLaunchKernel(fn, dim3(p.tiles_n * p.slices), dim3(CfgStrip::kThreads),
                         args, 0, stream);
}

int resolve_variant(int variant, int M, int N, int K);
int fp4_variant(int variant, int M, int N, int Kb);

// K-split plan of the 128 x 128 schedule: when its tiles fill at most a
// quarter of the CUs and K has at least 16 steps of 128, K-slices of at
// least 8 (even) steps so that tiles x slices approaches the CU count; when
// they fill at most half of them and K has at least 64 steps, cus / tiles
// slices (2, or 3 for 65-85 tiles on 256 CUs) of at least 8 steps each.  The
// workspace holds one 64 KiB fp32 partial tile per
// (tile, slice).  Measured against no split in one process:
// 256 x 4096 x 14336 (64 tiles, 4 slices) 1.39x; 128 tiles, 2 slices, with
// the reduce kernel's batched loads: 256 x 8192 x 8192 1.18x,
// 512 x 4096 x 8192 1.18x, 384 x 4096 x 8192 (96 tiles) 1.19x,
// 256 x 8192 x 28672 1.66x, but 256 x 8192 x 4096 (16-step slices) 0.89x.
struct T128Plan {
  int slices = 1, slice_steps = 0;
  size_t ws_bytes = 0;
};

// step_bytes: bytes of a row per K-step (96 for fp6 operands, else 128).
T128Plan plan_t128(int M, int N, int K, int cus, int step_bytes = CfgT128::kBK) {
  T128Plan p;
  const int tiles = ((M + CfgT128::kBM - 1) / CfgT128::kBM) *
                    ((N + CfgT128::kBN - 1) / CfgT128::kBN);
  const int steps = (K + step_bytes - 1) / step_bytes;
  p.slice_steps = steps;
  if (tiles <= 0 || 2 * tiles > cus || steps < 16) return p;
  if (4 * tiles > cus && steps < 64) return p;
  int sl = cus / tiles < steps / 8 ? cus / tiles : steps / 8;
  if (sl < 2) return p;
  int ss = (steps + sl - 1) / sl;
  ss = (ss + 1) & ~1;
  sl = (steps + ss - 1) / ss;
  if (sl < 2) return p;
  p.slices = sl;
  p.slice_steps = ss;
  // Arrival counters (4 per tile, the per-tensor epilogue), then the
  // partial tiles.
  p.ws_bytes = kWsCounterBytes + (size_t)tiles * sl * 65536;
  return p;
}

// counters_zero: `ws` is a caller's workspace (or the no-alloc scratch),
// whose counter region is zero by contract; a workspace allocated for the
// call is not cleared for this schedule, which then sums the slices in the
// reduce kernel (a clear would be one more launch per call).
hipError_t launch_t128_split(GemmArgs g, const T128Plan& p, void* ws,
                             bool counters_zero, hk::Key key,
                             hipStream_t stream) {
  const int tm = (g.M + CfgT128::kBM - 1) / CfgT128::kBM;
  const int tn = (g.N + CfgT128::kBN - 1) / CfgT128::kBN;
  const int tiles = tm * tn, units = tiles * p.slices, cus = cu_count();
  g.group_m = default_group_m(tm, tn);
  g.workers = units < cus ? units : cus;
  g.split.slices = p.slices;
  g.split.slice_steps = p.slice_steps;
  g.split.partial = reinterpret_cast<float*>(static_cast<char*>(ws) + kWsCounterBytes);
  // Per-tensor bf16 epilogue without MX scales, at most 4 slices: the last
  // slice to arrive at each quadrant sums it in the split kernel (4
  // counters per tile in the workspace's counter region).  Else the reduce
  // kernel, which spreads the sum over 16 workgroups per tile.  Same
  // process, caller workspace, against the reduce kernel: 256 x 8192 x 8192
  // (2 slices) +12 %, 128 x 8192 x 16384 (4) +2 %, 128 x 8192 x 8192 (4)
  // level; 96 x 4096 x 28672 (8 slices, the last arrival reading 7 partial
  // quadrants) -7 %.
  const bool fused = counters_zero && !g.mx.a && !key.ext && p.slices <= 4 &&
                     4 * tiles <= kWsMaxCounters;
  g.split.arrivals = fused ? static_cast<int*>(ws) : nullptr;
  if (fused) key.vec = vec_ok(key.out, g.N, g.ldc, g.C, 8);
  const void* fn = g.mx.a ? hk::tile128_split_mx(key) : hk::tile128_split(key);
  if (!fn) return hipErrorInvalidValue;
  void* args[] = {&g};
  hipError_t e = hipLaunchKernel(fn, dim3(g.workers), dim3(CfgT128::kThreads),
                                 args, 0, stream);
  if (e != hipSuccess || fused) return e;
  key.vec = vec_ok(key.out, g.N, g.ldc, g.C, 4);
  fn = hk::tile128_reduce(key);
  if (!fn) return hipErrorInvalidValue;
  return hipLaunchKernel(fn, dim3(tiles * 16), dim3(64), args, 0, stream);
}

int ceil_div(int a, int b) { return (a + b - 1) / b; }

// AUTO's split of C's columns when the last round of 256 x 256 tiles would
// leave most CUs idle (4000 x 5000: 320 tiles = 1.25 rounds): columns
// [0, n1) on the 4-wave 16x16x128 schedule in whole rounds, the rest on the
// 128 x 128 schedule (four times as many tiles).  Costs in rounds of the
// 4-wave schedule over all CUs: a full round of the 128 x 128 schedule
// measured 0.4-0.6 of one (it moves twice the L2 and LDS bytes per flop), so
// 0.6 is charged.  Returns n1, or 0 for no split.
int split_columns(int M, int N, int cus) {
  const int tm = ceil_div(M, Cfg4w::kBM), tn = ceil_div(N, Cfg4w::kBN);
  const int tiles = tm * tn;
  if (M <= CfgSkinny::kMaxM || tiles < cus || tiles % cus == 0) return 0;
  int c = (tiles / cus) * cus / tm;  // tile columns that fill whole rounds
  if (c >= tn) c = tn - 1;
  if (c <= 0) return 0;
  const int n1 = c * Cfg4w::kBN;
  const int rounds = ceil_div(tm * c, cus);
  const int rest = ceil_div(M, CfgT128::kBM) * ceil_div(N - n1, CfgT128::kBN);
  const double split = rounds + 0.6 * ceil_div(rest, cus);
  const double plain = ceil_div(tiles, cus);
  return split + 0.25 <= plain ? n1 : 0;
}

bool valid_code(int v, int count) { return v >= 0 && v < count; }

// Shared body of the GEMM entry points.  `ws` may be null when `ws_given` is
// false: a schedule that needs a workspace then takes a stream-ordered
// allocation for the call.
// dry_run: validate only, launch nothing.
hipError_t run_gemm(const hipgemm_gemm_desc& d, bool ws_given,
                    hipStream_t stream, bool dry_run = false) {
  int M = d.M, N = d.N, K = d.K, lda = d.lda, ldb = d.ldb, variant = d.variant;
  if (!valid_code(d.out_dtype, 4)) return hipErrorInvalidValue;
  // fp4 operands: both, K a multiple of 32 elements, the 128 x 128
  // schedule or the 4-wave 16x16x128 one (fp4_variant); from here on K
  // counts bytes of a row (K / 2).  fp6 operands: both (either variant
  // each), K a multiple of 64 elements (48 bytes), the same schedules as
  // fp4 (fp4_variant on the byte shape); K counts bytes (3 K / 4).
  const bool fp4 = d.a_format == HIPGEMM_FMT_FP4_E2M1 ||
                   d.b_format == HIPGEMM_FMT_FP4_E2M1;
  auto is6 = [](int f) {
    return f == HIPGEMM_FMT_FP6_E2M3 || f == HIPGEMM_FMT_FP6_E3M2;
  };
  const bool fp6 = is6(d.a_format) || is6(d.b_format);
  if (fp4) {
    if (d.a_format != d.b_format || K % 32 != 0 ||
        (variant != HIPGEMM_VARIANT_AUTO && variant != HIPGEMM_VARIANT_TILE128 &&
         variant != HIPGEMM_VARIANT_4WAVE_MFMA16))
      return hipErrorInvalidValue;
    K /= 2;
  }
  if (fp6) {
    if (!is6(d.a_format) || !is6(d.b_format) || K % 64 != 0 ||
        (variant != HIPGEMM_VARIANT_AUTO && variant != HIPGEMM_VARIANT_TILE128 &&
         variant != HIPGEMM_VARIANT_4WAVE_MFMA16))
      return hipErrorInvalidValue;
    K = K / 4 * 3;
  }
  const int es = out_bytes(d.out_dtype);
  hipError_t e = validate(d.A, d.B_T, d.C, M, N, K, lda, ldb, d.ldc, variant, es);
  if (e != hipSuccess) return e;
  if ((variant == HIPGEMM_VARIANT_SKINNY && M > CfgSkinny::kMaxM) ||
      (variant == HIPGEMM_VARIANT_STRIP && M > CfgStrip::kMaxM))
    return hipErrorInvalidValue;
  void* ws = d.workspace;
  const size_t ws_bytes = d.workspace_bytes;
  if (ws_given && ws_bytes > 0 && (!ws || !aligned(ws, 256)))
    return hipErrorInvalidValue;
  if ((!fp4 && !fp6 && (!valid_code(d.a_format, 2) || !valid_code(d.b_format, 2))) ||
      !valid_code(d.activation, 4))
    return hipErrorInvalidValue;
  // The output scale belongs to the e4m3 output; fp32 / e4m3 outputs are not
  // built for the 8-wave schedule.
  if (d.scale_out && d.out_dtype != HIPGEMM_OUT_FP8_E4M3) return hipErrorInvalidValue;
  if (d.out_dtype >= HIPGEMM_OUT_F32 && variant == HIPGEMM_VARIANT_8WAVE)
    return hipErrorInvalidValue;
  if (M == 0 || N == 0) return hipSuccess;
  // Vectors are read with 4-byte loads.
  if (!aligned(d.scale_rows, 4) || !aligned(d.scale_cols, 4) ||
      !aligned(d.bias, 4) || !aligned(d.scale_out, 4))
    return hipErrorInvalidValue;
  const bool ext = d.scale_rows || d.scale_cols || d.bias ||
                   d.activation != HIPGEMM_ACT_NONE ||
                   d.out_dtype != HIPGEMM_OUT_BF16;
  const int fmt = fp4   ? kFmtPairFp4
                  : fp6 ? kFmtPairFp6 + (d.a_format == HIPGEMM_FMT_FP6_E3M2) +
                              2 * (d.b_format == HIPGEMM_FMT_FP6_E3M2)
                        : d.a_format | (d.b_format << 1);
  // The 32x32x64 schedule is built for e4m3 x e4m3 with the per-tensor
  // epilogue only.
  if (variant == HIPGEMM_VARIANT_4WAVE && (ext || fmt != 0))
    return hipErrorInvalidValue;
  // MX block scales: the 4-wave 16x16x128 and 128 x 128 schedules,
  // per-tensor epilogue (K in elements a multiple of 32: bytes of 16 for fp4).
  const bool mx = d.mx_scale_a || d.mx_scale_b;
  if (mx && (fp6 || !d.mx_scale_a || !d.mx_scale_b || K % (fp4 ? 16 : 32) != 0 || ext ||
             !aligned(d.mx_scale_a, 16) || !aligned(d.mx_scale_b, 16) ||
             (variant != HIPGEMM_VARIANT_AUTO &&
              variant != HIPGEMM_VARIANT_4WAVE_MFMA16 &&
              variant != HIPGEMM_VARIANT_TILE128)))
    return hipErrorInvalidValue;
  const int n1 = (variant == HIPGEMM_VARIANT_AUTO && !mx && !fp4 && !fp6 && K > 0)
                     ? split_columns(M, N, cu_count())
                     : 0;
  variant = fp6   ? fp4_variant(variant, M, N, K)
            : fp4 ? fp4_variant(variant, M, N, K)
                  : resolve_variant(variant, M, N, K);
  // MX: the 128 x 128 schedule where AUTO picks it, else the 4-wave one.
  if (mx && variant != HIPGEMM_VARIANT_TILE128) variant = HIPGEMM_VARIANT_4WAVE_MFMA16;
  if (K == 0) lda = ldb = 16;  // nothing is read; keep the offset math inert
  const int tiles_m = (M + Cfg4w::kBM - 1) / Cfg4w::kBM;
  const int tiles_n = (N + Cfg4w::kBN - 1) / Cfg4w::kBN;
  GemmArgs g{static_cast<const uint8_t*>(d.A),
             static_cast<const uint8_t*>(d.B_T),
             static_cast<uint16_t*>(d.C),
             d.scale_a,
             d.scale_b,
             M,
             N,
             K,
             lda,
             ldb,
             d.ldc,
             default_group_m(tiles_m, tiles_n),
             0,
             EpiArgs{},
             MxArgs{},
             SplitArgs{}};
  g.epi.row_scale = d.scale_rows;
  g.epi.col_scale = d.scale_cols;
  g.epi.bias = d.bias;
  g.epi.act = d.activation;
  g.epi.out = d.out_dtype;
  g.epi.out_scale = d.scale_out;
  g.mx.a = static_cast<const uint8_t*>(d.mx_scale_a);
  g.mx.b = static_cast<const uint8_t*>(d.mx_scale_b);
  hk::Key key;
  key.fmt = fmt;
  key.ext = ext;
  key.act = d.activation;
  key.out = d.out_dtype;
  if (dry_run) return hipSuccess;
  // Whether a call that brings no workspace runs under stream capture: a
  // schedule that would split K then runs unsplit, as the stream-ordered
  // allocation of its partials would only be recorded into the caller's
  // graph (the 128 x 128 schedule's K-slices from half-filled grids, the
  // split-K and strip schedules' slices).
  auto capturing = [&](bool* yes) -> hipError_t {
    *yes = false;
    if (ws_given) return hipSuccess;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    const hipError_t r = hipStreamIsCapturing(stream, &cap);
    *yes = cap != hipStreamCaptureStatusNone;
    return r;
  };
  // A schedule that needs `need` bytes of workspace (the first `zero` of
  // them zero-filled): the caller's, or a stream-ordered allocation for the
  // call.
  auto with_workspace = [&](size_t need, size_t zero, auto go) -> hipError_t {
    if (need == 0) return go(nullptr);
    if (ws_given) {
      if (ws_bytes < need) return hipErrorInvalidValue;
      return go(ws);
    }
    // No workspace given: a stream-ordered allocation (and a clear of the
    // counters) for this call -- not while the stream is being captured,
    // where they would be recorded into the caller's graph.
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    hipError_t r = hipStreamIsCapturing(stream, &cap);
    if (r != hipSuccess) return r;
    if (cap != hipStreamCaptureStatusNone) return hipErrorInvalidValue;
    void* tmp = nullptr;
    r = hipMallocAsync(&tmp, need, stream);
    if (r != hipSuccess) return r;
    if (zero > 0) r = hipMemsetAsync(tmp, 0, zero, stream);
    if (r == hipSuccess) r = go(tmp);
    const hipError_t f = hipFreeAsync(tmp, stream);
    return r != hipSuccess ? r : f;
  };
  switch (variant) {
    case HIPGEMM_VARIANT_SKINNY: {
      SkinnyPlan p = plan_skinny(M, N, K);
      if (p.ws_bytes > 0) {
        bool cap = false;
        if (const hipError_t r = capturing(&cap); r != hipSuccess) return r;
        if (cap) p = plan_skinny(M, N, K, true);
      }
      return with_workspace(p.ws_bytes, p.counter_bytes, [&](void* w) {
        return launch_skinny(g, p, w, key, stream);
      });
    }
    case HIPGEMM_VARIANT_STRIP: {
      StripPlan p = plan_strip(M, N, K, strip_knb(M, N, K));
      if (p.ws_bytes > 0) {
        bool cap = false;
        if (const hipError_t r = capturing(&cap); r != hipSuccess) return r;
        // No workspace from the caller: one K-slice where each strip then
        // streams at most 1 MiB of A and B_T, instead of a stream-ordered
        // allocation and counter clear (about 12 us of host time per call).
        // Back-to-back calls, us, allocation / one slice: 16 x 4096 x 4096
        // 22.0 / 7.0, 40 x 2048 x 2048 22.6 / 7.2, 64 x 4096 x 4096
        // 23.3 / 12.6, 64 x 2048 x 8192 21.6 / 20.7 (768 KiB per strip).
        const bool stream_one = !ws_given && (long long)(16 * p.knb + M) * K <= (1ll << 20);
        if (cap || stream_one) p = plan_strip(M, N, K, strip_knb(M, N, K), true);
      }
      return with_workspace(p.ws_bytes, p.slices > 1 ? kWsCounterBytes : 0,
                            [&](void* w) { return launch_strip(g, p, w, key, stream); });
    }
    case HIPGEMM_VARIANT_TILE128: {
      const T128Plan p = plan_t128(M, N, K, cu_count(), fp6 ? 96 : CfgT128::kBK);
      bool cap = false;
      if (p.slices > 1)
        if (const hipError_t r = capturing(&cap); r != hipSuccess) return r;
      if (p.slices == 1 || cap) return launch_tiled(variant, g, key, stream);
      return with_workspace(p.ws_bytes, 0, [&](void* w) {
        return launch_t128_split(g, p, w, ws_given, key, stream);
      });
    }
    default:
      if (n1 > 0) {
        // Columns [0, n1) on the 4-wave schedule, [n1, N) on the 128 x 128
        // one: B_T rows, C columns and the column vectors offset by n1.
        GemmArgs g2 = g;
        g.N = n1;
        g2.N = N - n1;
        g2.B += (size_t)n1 * ldb;
        g2.C = reinterpret_cast<uint16_t*>(reinterpret_cast<uint8_t*>(g.C) +
                                           (size_t)n1 * es);
        if (g2.epi.col_scale) g2.epi.col_scale += n1;
        if (g2.epi.bias) g2.epi.bias += n1;
        return launch_split(g, g2, key, stream);
      }
      return launch_tiled(variant, g, key, stream);
  }
}

hipgemm_gemm_desc base_desc(const void* A, const void* B_T, void* C, int M,
                            int N, int K, int lda, int ldb, int ldc,
                            int variant) {
  hipgemm_gemm_desc d{};
  d.size = sizeof(hipgemm_gemm_desc);
  d.A = A;
  d.B_T = B_T;
  d.C = C;
  d.M = M;
  d.N = N;
  d.K = K;
  d.lda = lda;
  d.ldb = ldb;
  d.ldc = ldc;
  d.variant = variant;
  return d;
}

int resolve_variant(int variant, int M, int N, int K) {
  return variant == HIPGEMM_VARIANT_AUTO ? hipgemm_select_variant(M, N, K)
                                         : variant;
}

// fp4 x fp4 and fp6 x fp6 (Kb: bytes of a row).  AUTO: the 4-wave 16x16x128
// schedule where it picks that one for 8-bit operands of the same byte
// shape (a 128-byte step is one MFMA's worth for 8-bit operands, two for
// fp4: the same LDS bytes per step, twice the flops; a 96-byte fp6 step is
// one MFMA of 128 elements); else the 128 x 128 one.
int fp4_variant(int variant, int M, int N, int Kb) {
  if (variant != HIPGEMM_VARIANT_AUTO) return variant;
  return hipgemm_select_variant(M, N, Kb) == HIPGEMM_VARIANT_4WAVE_MFMA16
             ? HIPGEMM_VARIANT_4WAVE_MFMA16
             : HIPGEMM_VARIANT_TILE128;
}


}  // namespace

extern "C" {

int hipgemm_select_variant(int M, int N, int K) {
  // Up to 128 rows the GEMM is a stream over B_T (times: us, caller
  // workspace, schedules compared in one process on MI355X).
  //  * Up to 64 rows the column-strip schedule (whole-line DMA of B_T, A in
  //    registers): 16 x 8192 x 8192 12.9 against 17.8 on the split-K
  //    schedule, 64 x 2048 x 4096 9.7 against 10.0 on the split-K one and
  //    14.0 on the 128 x 128 one, 40 x 14336 x 8192 25.4 / 33.1 / 33.9,
  //    64 x 8192 x 8192 21.1 / 24.6 / 21.8.  Except, from 17 rows, where
  //    even 64-column strips outnumber the CUs (N > 64 x CUs): the 128 x 128
  //    tiles, one row of them, are then ahead (28 x 20480 x 1024 8.9
  //    against 12.6, 24 x 28672 x 4096 23.4 / 24.9, 28 x 20480 x 6144
  //    30.8 / 34.5, 32 x 24576 x 8192 39.8 / 43.4, 52 x 20480 x 3072 19.1 /
  //    28.1, 64 x 28672 x 2048 14.6 / 22.0; at 16 rows the strip keeps
  //    them: 16 x 28672 x 4096 22.9 / 23.8); above 32 rows for K <= 1024
  //    unless 32-column strips fill between a quarter and all of the CUs in
  //    one K-slice (64 x 2048 x 1024 7.2 against 8.3, 56 x 14336 x 1024
  //    8.5 / 9.4, 44 x 2048 x 1024 7.3 / 7.8; but 48 x 8192 x 1024 8.1 /
  //    6.5, 40 x 3072 x 1024 8.0 / 7.5); and above 48 rows for K > 8192
  //    from N = 3072 (64 x 4096 x 14336 19.7 / 22.6, 56 x 8192 x 14336
  //    29.7 / 33.8, 62 x 11008 x 10240 34.3 / 37.6; 33-48 rows run as
  //    three 16-row blocks and keep the strip: 44 x 5120 x 12288 21.5 /
  //    18.5).  Sweeps of 584 shapes up to 128 rows and 630 from 34 to 48
  //    rows (python -m hipgemm_amd.sweep) put these rules within 0.4 % of
  //    the best schedule on average up to 64 rows.
  //  * From 65 rows the strip still for a B_T of at most 8 MiB (96 x 2048 x
  //    4096 12.0 against 13.0 on the split-K schedule and 15.1 on the
  //    128 x 128 one, 72 x 1024 x 8192 12.1 / 13.9 / 12.4, 128 x 2048 x
  //    2048 11.4 / 12.8 / 11.9; 54 shapes from 72 to 128 rows: within
  //    0.6 % of the best on average).  Above that the 128 x 128 schedule,
  //    which DMAs whole lines of A and
  //    B_T and reads A once per 128 columns: 128 x 8192 x 8192 22.6 against
  //    28.0 on the split-K schedule, 128 x 28672 x 8192 52.7 / 74.3,
  //    128 x 4096 x 28672 32.9 / 43.6.  Except
  //    where its K-split stops at its 8-step slice floor with at most half
  //    the CUs busy, in 3 slices or more, for N >= 2048: the split-K
  //    schedule, which fills every CU, is then ahead (128 x 4096 x 4096
  //    14.4 / 16.3, 128 x 2048 x 8192 14.7 / 16.2, 120 x 2560 x 4096
  //    13.9 / 15.0).  With 2 slices the 128 x 128 schedule sums the two
  //    partials in its split kernel and stays ahead (128 x 6144 x 2048 13.0
  //    / 15.6, 128 x 8192 x 2048 13.7 / 14.5), as below 2048 columns
  //    (100 x 1536 x 8192 13.9 / 15.9).
  if (M <= 16) return HIPGEMM_VARIANT_STRIP;
  if (M <= 64) {
    const int cus = cu_count();
    if (ceil_div(N, 64) > cus) return HIPGEMM_VARIANT_TILE128;
    if (M > 32 && K <= 1024) {
      const int strips = ceil_div(N, 32);
      if (strips > cus || 4 * strips <= cus) return HIPGEMM_VARIANT_TILE128;
    }
    if (M > 48 && K > 8192 && N >= 3072) return HIPGEMM_VARIANT_TILE128;
    return HIPGEMM_VARIANT_STRIP;
  }
  if (M <= CfgSkinny::kMaxM) {
    if ((long long)N * K <= (8ll << 20)) return HIPGEMM_VARIANT_STRIP;
    const int cus = cu_count();
    const T128Plan p = plan_t128(M, N, K, cus);
    const int units = ceil_div(M, CfgT128::kBM) * ceil_div(N, CfgT128::kBN) * p.slices;
    const bool half_filled = p.slices > 1 && 2 * units <= cus;
    if (half_filled && N >= 2048 && p.slices > 2) return HIPGEMM_VARIANT_SKINNY;
    return HIPGEMM_VARIANT_TILE128;
  }
  // Above 128 rows the 4-wave
  // 16x16x128 schedule (3-7 % ahead of the 8-wave one from 2048 x 4096 up),
  // except where the 128 x 128 tiles fit in one round over the CUs (the
  // 256 x 256 ones then fill at most a quarter of them; 2048^3: 1.69x the
  // 8-wave one), where its tiles fit in less than two rounds and the 256 x
  // 256 ones fill at most half the CUs (below), and for short K on at most
  // 128 tiles of 256 x 256 (half a round), where the 128 x 128 schedule is
  // level or ahead (3072 x 2048 x
  // 2048 +12 %, 2048 x 4096 x 512 +8 %, 2048 x 4096 x 2048 +1.4 %,
  // 2048 x 4096 x 1024 -0.6 %; from K = 3072, or above 128 tiles, the 4-wave
  // one leads by 3-48 %).  AUTO also splits C between the 4-wave and 128 x
  // 128 schedules for a short last round (hipgemm_split_columns); this
  // returns the 4-wave one then.
  const int cus = cu_count();
  const int t1 = ceil_div(M, CfgT128::kBM) * ceil_div(N, CfgT128::kBN);
  if (t1 <= cus) return HIPGEMM_VARIANT_TILE128;
  if (K <= 2048 && tiles_of(M, N) <= 128) return HIPGEMM_VARIANT_TILE128;
  // 256 x 256 tiles on at most half the CUs, 128 x 128 ones in less than
  // two rounds: 1536 x 4096 x 4096 35.3 us against 39.2, x 8192 64.8 /
  // 71.5, 1280 x 4096 x 8192 64.6 / 71.3, 1792 x 4096 x 4096 36.5 / 39.1,
  // 1152 x 4096 x 4096 35.4 / 37.4, 4096 x 1536 x 4096 38.6 / 39.1; in two
  // full rounds the 4-wave one stays ahead (1024 x 8192 x 4096 40.5 /
  // 41.2, 2048 x 4096 x 8192 71.3 / 74.1).  Except with a side of 8192 or
  // more and K from 4096, where the 4-wave one leads: 640 x 8192 x 8192
  // 72.5 / 67.4, x 4096 39.6 / 37.6, x 16384 134.2 / 128.4, 896 x 8192 x
  // 8192 74.0 / 67.9, 8192 x 640 x 8192 72.3 / 67.9, 768 x 8192 x 8192
  // 74.0 / 72.7 (768 x 8192 x 16384 135.0 / 140.9 the one exception seen);
  // with K = 2048 the two are level there (640 x 8192 x 2048 22.7 / 23.0).
  const bool long_side = (M >= 8192 || N >= 8192) && K >= 4096;
  if (2 * tiles_of(M, N) <= cus && t1 < 2 * cus && !long_side)
    return HIPGEMM_VARIANT_TILE128;
  return HIPGEMM_VARIANT_4WAVE_MFMA16;
}

int hipgemm_split_columns(int M, int N, int K) {
  if (M <= 0 || N <= 0 || K <= 0) return 0;
  return split_columns(M, N, cu_count());
}

hipError_t hipgemm_fp8_gemm_bf16(const void* A, const void* B_T, void* C,
                                 int M, int N, int K, int lda, int ldb,
                                 int ldc, const float* scale_a,
                                 const float* scale_b, int variant,
                                 hipStream_t stream) {
  hipgemm_gemm_desc d = base_desc(A, B_T, C, M, N, K, lda, ldb, ldc, variant);
  d.scale_a = scale_a;
  d.scale_b = scale_b;
  return run_gemm(d, false, stream);
}

hipError_t hipgemm_fp8_gemm_bf16_ws(const void* A, const void* B_T, void* C,
                                    int M, int N, int K, int lda, int ldb,
                                    int ldc, const float* scale_a,
                                    const float* scale_b, int variant,
                                    void* workspace, size_t workspace_bytes,
                                    hipStream_t stream) {
  hipgemm_gemm_desc d = base_desc(A, B_T, C, M, N, K, lda, ldb, ldc, variant);
  d.scale_a = scale_a;
  d.scale_b = scale_b;
  d.workspace = workspace;
  d.workspace_bytes = workspace_bytes;
  return run_gemm(d, true, stream);
}

hipError_t hipgemm_fp8_gemm_bf16_rowcol(const void* A, const void* B_T, void* C,
                                        int M, int N, int K, int lda, int ldb,
                                        int ldc, const float* scale_rows,
                                        const float* scale_cols, int variant,
                                        void* workspace, size_t workspace_bytes,
                                        hipStream_t stream) {
  hipgemm_gemm_desc d = base_desc(A, B_T, C, M, N, K, lda, ldb, ldc, variant);
  d.scale_rows = scale_rows;
  d.scale_cols = scale_cols;
  d.workspace = workspace;
  d.workspace_bytes = workspace_bytes;
  // A null workspace with a zero size lets the call allocate one when the
  // split-K schedule needs it, like hipgemm_fp8_gemm_bf16.
  return run_gemm(d, workspace != nullptr || workspace_bytes != 0, stream);
}

hipError_t hipgemm_gemm(const hipgemm_gemm_desc* desc, hipStream_t stream) {
  if (!desc || desc->size != sizeof(hipgemm_gemm_desc))
    return hipErrorInvalidValue;
  return run_gemm(*desc,
                  desc->workspace != nullptr || desc->workspace_bytes != 0,
                  stream);
}

size_t hipgemm_mx_scales_bytes(int rows, int K) {
  if (rows <= 0 || K <= 0) return 0;
  return mx_packed_bytes(rows, K);
}

hipError_t hipgemm_mx_pack_scales(const void* src, int rows, int K, int ld,
                                  void* dst, hipStream_t stream) {
  if (rows < 0 || K < 0 || K % 32 != 0) return hipErrorInvalidValue;
  if (rows == 0 || K == 0) return hipSuccess;
  if (!src || !dst || ld < K / 32) return hipErrorInvalidValue;
  return hk::mx_pack(static_cast<const uint8_t*>(src), rows, K, ld,
                     static_cast<uint8_t*>(dst), stream);
}

size_t hipgemm_gemm_workspace_size(const hipgemm_gemm_desc* d) {
  if (!d || d->size != sizeof(hipgemm_gemm_desc) || d->M <= 0 || d->N <= 0 ||
      d->K <= 0)
    return 0;
  const bool fp4 = d->a_format == HIPGEMM_FMT_FP4_E2M1 ||
                   d->b_format == HIPGEMM_FMT_FP4_E2M1;
  if (fp4) {
    if (fp4_variant(d->variant, d->M, d->N, d->K / 2) == HIPGEMM_VARIANT_4WAVE_MFMA16)
      return 0;
    return plan_t128(d->M, d->N, d->K / 2, cu_count()).ws_bytes;
  }
  auto is6 = [](int f) {
    return f == HIPGEMM_FMT_FP6_E2M3 || f == HIPGEMM_FMT_FP6_E3M2;
  };
  const bool fp6 = is6(d->a_format) || is6(d->b_format);
  if (fp6) {
    if (fp4_variant(d->variant, d->M, d->N, d->K / 4 * 3) ==
        HIPGEMM_VARIANT_4WAVE_MFMA16)
      return 0;
    return plan_t128(d->M, d->N, d->K / 4 * 3, cu_count(), 96).ws_bytes;
  }
  if (d->mx_scale_a || d->mx_scale_b) {  // 128 x 128 where AUTO picks it
    const int v = resolve_variant(d->variant, d->M, d->N, d->K);
    return v == HIPGEMM_VARIANT_TILE128
               ? plan_t128(d->M, d->N, d->K, cu_count()).ws_bytes
               : 0;
  }
  return hipgemm_workspace_size(d->M, d->N, d->K, d->variant);
}

hipError_t hipgemm_gemm_noalloc(const hipgemm_gemm_desc* desc,
                                hipStream_t stream) {
  if (!desc || desc->size != sizeof(hipgemm_gemm_desc) || desc->workspace ||
      desc->workspace_bytes)
    return hipErrorInvalidValue;
  const size_t need = hipgemm_gemm_workspace_size(desc);
  if (need > (size_t)HIPGEMM_NOALLOC_SCRATCH_BYTES) return hipErrorInvalidValue;
  hipgemm_gemm_desc d = *desc;
  if (need > 0) {
    // Argument errors come back before the scratch is touched.
    hipError_t e = run_gemm(d, false, stream, true);
    if (e != hipSuccess) return e;
    d.workspace = hk::noalloc_scratch(stream, &e);
    if (!d.workspace) return e;
    d.workspace_bytes = HIPGEMM_NOALLOC_SCRATCH_BYTES;
  }
  // need == 0: no schedule on this path uses a workspace (none is given,
  // so none can be allocated either).
  return run_gemm(d, true, stream);
}

size_t hipgemm_workspace_size(int M, int N, int K, int variant) {
  if (M <= 0 || N <= 0 || K < 0) return 0;
  const int v = resolve_variant(variant, M, N, K);
  if (v == HIPGEMM_VARIANT_TILE128) return plan_t128(M, N, K, cu_count()).ws_bytes;
  if (v == HIPGEMM_VARIANT_STRIP)
    return M > CfgStrip::kMaxM ? 0 : plan_strip(M, N, K, strip_knb(M, N, K)).ws_bytes;
  if (v != HIPGEMM_VARIANT_SKINNY) return 0;
  if (M > CfgSkinny::kMaxM) return 0;
  return plan_skinny(M, N, K).ws_bytes;
}

hipError_t hipgemm_fp8_gemm_4wave_256x256x128(const void* A, const void* B_T,
                                              void* C, int M, int N, int K,
                                              hipStream_t stream) {
  return hipgemm_fp8_gemm_bf16(A, B_T, C, M, N, K, K, K, N, nullptr, nullptr,
                               HIPGEMM_VARIANT_4WAVE_MFMA16, stream);
}

const char* hipgemm_variant_name(int variant) {
  switch (variant) {
    case HIPGEMM_VARIANT_AUTO:
      return "auto";
    case HIPGEMM_VARIANT_4WAVE:
      return "4wave_256x256x128_mfma32";
    case HIPGEMM_VARIANT_4WAVE_MFMA16:
      return "4wave_256x256x128_mfma16";
    case HIPGEMM_VARIANT_SKINNY:
      return "skinny_splitk_256";
    case HIPGEMM_VARIANT_8WAVE:
      return "8wave_256x256x128_mfma16";
    case HIPGEMM_VARIANT_TILE128:
      return "4wave_128x128x128_mfma16";
    case HIPGEMM_VARIANT_STRIP:
      return "strip_32_mfma16";
    default:
      return nullptr;
  }
}

int hipgemm_version(void) { return HIPGEMM_VERSION; }

int hipgemm_tile_order(int grid, int tiles_m, int tiles_n, int group_m,
                       int* tile_m, int* tile_n, int cap) {
  if (grid <= 0 || tiles_m <= 0 || tiles_n <= 0 || !tile_m || !tile_n ||
      cap < 0)
    return 0;
  if (group_m <= 0) group_m = default_group_m(tiles_m, tiles_n);
  const int tiles = tiles_m * tiles_n;
  int w = 0;
  for (int b = 0; b < grid && w < cap; ++b) {
    const TileWalk walk = tile_walk(b, grid, tiles);
    for (int t = walk.first; t < walk.end && w < cap; t += walk.stride) {
      const TileCoord tc = grouped_tile(t, tiles_m, tiles_n, group_m);
      tile_m[w] = tc.m;
      tile_n[w] = tc.n;
      ++w;
    }
  }
  return w;
}

int hipgemm_lds_slot(int row, int chunk) {
  if (row < 0 || chunk < 0 || chunk > 7) return -1;
  return chunk ^ slot_xor(row);
}

int hipgemm_lds_slot_kpair(int row, int chunk) {
  if (row < 0 || chunk < 0 || chunk > 7) return -1;
  return kpair_slot(chunk) ^ slot_xor(row);
}

int hipgemm_lds_stage_slot(int row, int piece) {
  if (row < 0 || piece < 0 || piece > 15) return -1;
  return piece ^ stage_xor(row);
}

}  // extern "C"
