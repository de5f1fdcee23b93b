/*
 * hipgemm -- C ABI of the MI355X (gfx950) FP8 GEMM.
 *
 *   C[M x N] = bf16_rne( (scale_a * scale_b) * sum_k A[m, k] * B_T[n, k] )
 *
 * A is M x K, row-major, e4m3 (OCP E4M3FN, one byte), row stride lda bytes.
 * B_T is N x K, row-major (K contiguous), e4m3, row stride ldb bytes.
 * C is M x N, row-major, bf16, row stride ldc elements.
 * (hipgemm_gemm generalises this: e5m2 operands, fp16 output, row / column
 * scales, bias and activation; see hipgemm_gemm_desc.)
 * Accumulation is fp32.  scale_a / scale_b are DEVICE pointers to one fp32
 * each (per-tensor scales), or NULL for 1.0; the product scale_a * scale_b is
 * formed in fp32 and applied to the fp32 accumulator before rounding.
 *
 * The reference (nirw4nna/hipgemm) exposes only a C++ kernel template,
 * fp8_gemm_4wave_256x256x128<M, N, K>(A, B_T, C) (fp8_4wave.hpp:334-338),
 * launched by its callers as <<<(M*N)/65536, 256>>> on the null stream
 * (test.cpp:79, bench.cpp:55, bench.cpp:78).  That surface is kept in
 * include/hipgemm/fp8_gemm.hpp; these entry points are the plain-pointer
 * boundary over it.  Plain pointers and sizes only.
 *
 * Errors: every entry point returns a hipError_t and never exits the
 * process.  Argument errors return hipErrorInvalidValue before any HIP call,
 * so they can be checked on a machine without a GPU.  Requirements:
 *   M, N, K >= 0;  C non-NULL, 2-byte aligned, N <= ldc <= 2^22;
 *   A, B_T non-NULL and 16-byte aligned;  K % 16 == 0;
 *   lda >= K, ldb >= K, lda % 16 == 0, ldb % 16 == 0, lda, ldb <= 2^23.
 * M == 0 or N == 0 is a no-op (nothing is checked or written).  K == 0
 * writes bf16(0 * scale) everywhere and neither reads nor checks A, B_T,
 * lda, ldb.
 * Nothing outside the M x N window of C is written.
 *
 * Threading: no global mutable state; calls on different streams may run
 * concurrently as long as their C windows do not overlap.
 */
#ifndef HIPGEMM_H
#define HIPGEMM_H

#include <hip/hip_runtime_api.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

#define HIPGEMM_VERSION 100 /* 1.0.0 */

/* Workspace layout (every schedule): the first HIPGEMM_WS_COUNTER_BYTES
 * bytes hold arrival counters that must be zero before a workspace's first
 * use; every call leaves them zero again and writes nothing else there.
 * Partial tiles follow; calls overwrite them before reading them.  So one
 * workspace serves calls of every shape and schedule in turn. */
#define HIPGEMM_WS_COUNTER_BYTES 16384

/* Schedules.  AUTO picks by shape (hipgemm_select_variant). */
enum {
  HIPGEMM_VARIANT_AUTO = 0,
  /* 256 threads (4 waves, one per SIMD), 256 x 256 tile, 2 LDS stages,
   * persistent grid, v_mfma_f32_32x32x64_f8f6f4. */
  HIPGEMM_VARIANT_4WAVE = 1,
  /* The same schedule on v_mfma_f32_16x16x128_f8f6f4: AUTO's choice for
   * M > 128 when the 256 x 256 tiles fill the CUs (but see TILE128 and
   * hipgemm_split_columns), and the schedule behind the drop-in
   * template. */
  HIPGEMM_VARIANT_4WAVE_MFMA16 = 2,
  /* M <= 128 only: split-K over every CU for the HBM-bound skinny shapes,
   * operands streamed straight into registers, a deterministic in-kernel
   * reduction of the K-slices.  AUTO's choice for 64 < M <= 128 only where
   * B_T exceeds 8 MiB and the 128 x 128 schedule's K-split would leave at
   * least half the CUs idle in 3 slices or more, for N >= 2048 (e.g.
   * 128 x 4096 x 4096; not 128 x 8192 x 2048).  Needs a workspace (hipgemm_workspace_size) when
   * it splits K. */
  HIPGEMM_VARIANT_SKINNY = 3,
  /* 512 threads (8 waves, two per SIMD, in two groups that alternate
   * between LDS/DMA work and MFMAs), 256 x 256 tile, each wave 128 x 64 of
   * it, persistent grid, v_mfma_f32_16x16x128_f8f6f4.  Never AUTO's
   * choice (3-7 % behind the 4-wave one from 2048 x 4096 up, behind the
   * 128 x 128 one below).  The reference's kernels are 4-wave only; no
   * reference counterpart. */
  HIPGEMM_VARIANT_8WAVE = 4,
  /* 256 threads (4 waves, one per SIMD), 128 x 128 tile, each wave 64 x 64
   * of it, 4 LDS stages, persistent grid, v_mfma_f32_16x16x128_f8f6f4: four
   * times as many tiles as the 256 x 256 schedules, for shapes whose 256 x
   * 256 tiles underfill the CUs: AUTO's choice for M > 128 when its tiles
   * fit in one round over the CUs, or in less than two where the 256 x 256
   * ones fill at most half of them (unless M or N >= 8192 and K >= 4096), or
   * for K <= 2048 on at most 128 tiles of 256 x 256, for 64 < M <= 128
   * (except as under STRIP and SKINNY), and for 16 < M <= 64 where N > 64 x
   * CUs, above 32 rows where K <= 1024 (unless N / 32 lies in (CUs / 4,
   * CUs]), or above 48 rows where K > 8192 and N >= 3072. The workgroups
   * of each XCD start their K walk at their own step (a different order of
   * the fp32 sums per XCD). Splits K into slices when its tiles fill at most a
   * quarter of the CUs and K has at least 16 steps of 128 bytes, or at most
   * half of them and K has at least 64 steps (CUs / tiles slices: 2, or 3
   * for 65-85 tiles on 256 CUs); a workspace then (hipgemm_workspace_size).
   * With a caller's workspace (or hipgemm_gemm_noalloc), the per-tensor
   * epilogue, no MX scales and at most 4 slices, the slice that finishes a
   * 64 x 64 quadrant last sums it in the same kernel (arrival counters in
   * the workspace); else a second kernel sums the slices. A call with no
   * workspace under stream capture runs unsplit (as do the split-K and strip
   * schedules' calls there). No reference counterpart (the reference has 256
   * x 256 tiles only). */
  HIPGEMM_VARIANT_TILE128 = 5,
  /* M <= 128 only: 256 threads, each workgroup a strip of 32 columns of C
   * (64 from 17 rows when 32-column strips would outnumber the CUs, and
   * for some long-K shapes above 40 rows) over all of K (over a K-slice,
   * with a workspace, when the strips alone are fewer than the CUs; at most
   * one workgroup per CU), its 4 waves each a quarter of the K-steps,
   * summed in LDS; B_T streamed by whole-line DMA into LDS, A straight into
   * registers (through LDS as well for 17-32 rows on 32-column strips).
   * AUTO's choice for M <= 64 except where TILE128 is, and for
   * 64 < M <= 128 with a B_T of at most 8 MiB.  No reference
   * counterpart. */
  HIPGEMM_VARIANT_STRIP = 6,
  HIPGEMM_VARIANT_COUNT = 7
};

/* Operand formats (OCP 8-bit floating point v1.0; OCP Microscaling v1.0
 * for E2M3, E3M2 and E2M1).  FP4_E2M1: 1 sign, 2 exponent (bias 1), 1
 * mantissa bit -- 0, 0.5, 1, 1.5, 2, 3, 4, 6 and their negatives -- two per
 * byte, element 2i in the low nibble of byte i of a row; A and B_T both
 * FP4_E2M1 (not mixed with the other formats), K (in elements) a multiple
 * of 32, lda / ldb in bytes (>= K / 2); schedules AUTO, TILE128 and
 * 4WAVE_MFMA16 (AUTO's choice where it takes that schedule for 8-bit
 * operands of the same byte shape).
 * FP6_E2M3 (1 sign, 2 exponent bits, bias 1, 3 mantissa bits; largest 7.5)
 * and FP6_E3M2 (1 sign, 3 exponent bits, bias 3, 2 mantissa bits; largest
 * 28), no inf or NaN: four per three bytes, packed LSB first -- element k
 * of a row is bits [6k, 6k + 6) of the row read as one little-endian bit
 * string; A and B_T both fp6 (either variant each), K (in elements) a
 * multiple of 64, lda / ldb in bytes (>= 3K / 4, multiples of 16),
 * schedules AUTO, TILE128 and 4WAVE_MFMA16 (AUTO's choice where it takes
 * that schedule for 8-bit operands of the same byte shape), no MX block
 * scales. */
enum {
  HIPGEMM_FMT_E4M3 = 0,     /* E4M3FN: bias 7, max 448, NaN 0x7F/0xFF, no inf */
  HIPGEMM_FMT_E5M2 = 1,     /* E5M2: bias 15, max 57344, IEEE inf and NaN     */
  HIPGEMM_FMT_FP6_E2M3 = 2, /* E2M3: max 7.5, no inf or NaN                   */
  HIPGEMM_FMT_FP6_E3M2 = 3, /* E3M2: max 28, no inf or NaN                    */
  HIPGEMM_FMT_FP4_E2M1 = 4  /* E2M1: max 6, no inf or NaN                     */
};

/* Output types of hipgemm_gemm.  BF16, F16: round to nearest even; F32: the
 * fp32 value itself; FP8_E4M3: OCP e4m3 of activation(v) * scale_out, round
 * to nearest even, finite magnitudes above 448 saturate to 448, Inf and NaN
 * become NaN (0x7f | sign) -- the __HIP_SATFINITE conversion of
 * amd_hip_fp8.h.  F32 and FP8_E4M3 run on schedules AUTO, 4WAVE_MFMA16,
 * SKINNY and TILE128. */
enum {
  HIPGEMM_OUT_BF16 = 0,
  HIPGEMM_OUT_F16 = 1,
  HIPGEMM_OUT_F32 = 2,
  HIPGEMM_OUT_FP8_E4M3 = 3
};

/* Activations of the fused epilogue, applied in fp32 after bias:
 *   RELU(v) = v < 0 ? 0 : v
 *   GELU_TANH(v) = v/2 (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3)))
 *   SILU(v) = v / (1 + exp(-v))
 * evaluated with the hardware exponential and reciprocal (a few ulp of
 * fp32 before the rounding to the output type). */
enum {
  HIPGEMM_ACT_NONE = 0,
  HIPGEMM_ACT_RELU = 1,
  HIPGEMM_ACT_GELU_TANH = 2,
  HIPGEMM_ACT_SILU = 3
};

/*
 * Full description of one GEMM for hipgemm_gemm:
 *
 *   scale[m,n] = scale_rows[m] * (scale_cols[n] * (scale_a * scale_b))
 *   v[m,n]     = fma(acc[m,n], scale[m,n], bias[n])       (one rounding)
 *   C[m,n]     = round_out(activation(v[m,n]) [* scale_out, e4m3 only])
 *
 * acc is the fp32 sum over K of A[m,k] * B_T[n,k] with A in a_format and
 * B_T in b_format.  NULL scalars and vectors are ones, a NULL bias is
 * -0.0 (v is then exactly acc * scale).  With the defaults (e4m3 x e4m3, no
 * vectors, no bias, no activation, bf16) this is hipgemm_fp8_gemm_bf16,
 * bit for bit.  Zero-initialise the struct, set `size` to
 * sizeof(hipgemm_gemm_desc) (a different size is rejected), then the
 * fields.  Shape, stride, alignment and workspace rules are those of the
 * entry points above; vectors must be 4-byte aligned; variant
 * HIPGEMM_VARIANT_4WAVE accepts only the defaults of format and epilogue.
 */
typedef struct hipgemm_gemm_desc {
  size_t size;
  const void *A;   /* M x K, row stride lda bytes */
  const void *B_T; /* N x K, row stride ldb bytes */
  void *C;         /* M x N, row stride ldc elements of out_dtype, aligned
                    * to one element */
  int M, N, K;
  int lda, ldb, ldc;
  int a_format, b_format; /* HIPGEMM_FMT_* */
  int out_dtype;          /* HIPGEMM_OUT_* */
  int activation;         /* HIPGEMM_ACT_* */
  const float *scale_a, *scale_b;       /* device scalars or NULL */
  const float *scale_rows, *scale_cols; /* device vectors of M, N or NULL */
  const float *bias;                    /* device vector of N or NULL */
  int variant;                          /* HIPGEMM_VARIANT_* */
  void *workspace; /* as for hipgemm_fp8_gemm_bf16_ws; NULL with size 0: */
  size_t workspace_bytes; /* allocate one when needed, stream-ordered    */
  /* MX block scales (OCP Microscaling v1.0): E8M0 bytes, one per 32
   * consecutive K-elements of a row of A / B_T, 2^(e - 127), 255 = NaN,
   * in the packed device layout hipgemm_mx_pack_scales writes.  Both or
   * neither; K % 32 == 0, 16-byte aligned.  Each element is multiplied by its
   * block's scale before the products are summed; the per-tensor scales
   * still apply.  Not combined with the row / column / bias / activation /
   * output-type options; schedules AUTO (the 128 x 128 one where AUTO picks
   * it, else the 4-wave one), HIPGEMM_VARIANT_4WAVE_MFMA16 and
   * HIPGEMM_VARIANT_TILE128 (which also takes fp4 operands: MXFP4). */
  const void *mx_scale_a, *mx_scale_b;
  /* Device scalar or NULL (1.0) multiplying activation(v) before the
   * conversion; FP8_E4M3 output only (NULL otherwise), 4-byte aligned. */
  const float *scale_out;
} hipgemm_gemm_desc;

/*
 * Runtime-shape GEMM with scales and a stream.
 * Replaces: fp8_gemm_4wave_256x256x128<M, N, K><<<(M*N)/65536, 256>>>(A, B_T,
 * C) (fp8_4wave.hpp:334-338, launched at test.cpp:79 and bench.cpp:78), whose
 * shapes are template constants, strides fixed at lda = ldb = K, ldc = N, with
 * no scales and the null stream.
 */
hipError_t hipgemm_fp8_gemm_bf16(const void *A, const void *B_T, void *C,
                                 int M, int N, int K, int lda, int ldb,
                                 int ldc, const float *scale_a,
                                 const float *scale_b, int variant,
                                 hipStream_t stream);

/*
 * hipgemm_fp8_gemm_bf16 with a caller-provided workspace.  A schedule that
 * needs scratch memory (hipgemm_workspace_size(M, N, K, variant) > 0: the
 * skinny split-K and column-strip schedules' K-slices and the 128 x 128
 * schedule's keep their arrival counters and fp32 partial tiles there) uses
 * `workspace` instead of taking a stream-ordered allocation
 * (hipMallocAsync, a clear of the counters, hipFreeAsync: about 12 us of
 * host time) on `stream` for the call, as hipgemm_fp8_gemm_bf16 does.  The
 * workspace must be 256-byte aligned and at least that size, and its first
 * HIPGEMM_WS_COUNTER_BYTES bytes zero before its first use (every call
 * leaves them zero: see HIPGEMM_WS_COUNTER_BYTES).  Calls that may run
 * concurrently must not share a workspace.  Returns hipErrorInvalidValue if
 * it is missing or too small when needed.
 * While `stream` is being captured into a graph, an entry point given no
 * workspace allocates none: a schedule that would split K runs with one
 * K-slice (the same result within rounding, slower on the shapes that
 * split).  Pass a workspace there to keep the split.  Without a workspace
 * the strip schedule also runs one K-slice, allocating nothing, where each
 * strip then streams at most 1 MiB of A and B_T (faster than an allocation
 * per call there; the result again within rounding of the split one).
 * Replaces: the same reference launch (the reference has no workspace and no
 * split-K path).
 */
hipError_t hipgemm_fp8_gemm_bf16_ws(const void *A, const void *B_T, void *C,
                                    int M, int N, int K, int lda, int ldb,
                                    int ldc, const float *scale_a,
                                    const float *scale_b, int variant,
                                    void *workspace, size_t workspace_bytes,
                                    hipStream_t stream);

/*
 * Per-row / per-column scaled GEMM:
 *
 *   C[m, n] = bf16_rne( (scale_rows[m] * scale_cols[n]) * sum_k A[m,k] B_T[n,k] )
 *
 * scale_rows is a DEVICE vector of M fp32 (one per row of A and C),
 * scale_cols one of N fp32 (one per row of B_T, i.e. column of C); either may
 * be NULL for all ones.  The product of the two scales is formed in fp32 and
 * applied to the fp32 accumulator before rounding, as in
 * hipgemm_fp8_gemm_bf16 (which is this call with constant vectors).  Both
 * vectors must be 4-byte aligned.  Accepts every schedule but
 * HIPGEMM_VARIANT_4WAVE, which returns hipErrorInvalidValue (SKINNY and
 * STRIP for M <= 128 only).  Workspace as in
 * hipgemm_fp8_gemm_bf16_ws, except that workspace == NULL with
 * workspace_bytes == 0 takes a stream-ordered allocation when one is needed,
 * as hipgemm_fp8_gemm_bf16 does.
 * No reference counterpart: the reference applies no scales at all
 * (store_rt, fp8_4wave.hpp:214-238, converts the accumulator straight to
 * bf16).
 */
hipError_t hipgemm_fp8_gemm_bf16_rowcol(const void *A, const void *B_T, void *C,
                                        int M, int N, int K, int lda, int ldb,
                                        int ldc, const float *scale_rows,
                                        const float *scale_cols, int variant,
                                        void *workspace, size_t workspace_bytes,
                                        hipStream_t stream);

/*
 * The general entry point: operand formats (e4m3 / e5m2, mixed), output
 * type (bf16 / fp16), per-tensor and per-row / per-column scales, bias and
 * activation, fused into the one kernel (see hipgemm_gemm_desc).
 * No reference counterpart beyond the plain launch it generalises: the
 * reference's kernel is e4m3 x e4m3 -> bf16 with no scales
 * (fp8_4wave.hpp:58 passes format codes 0, 0 and zero scales to the MFMA;
 * store_rt, :214-238, converts the accumulator straight to bf16).
 */
hipError_t hipgemm_gemm(const hipgemm_gemm_desc *desc, hipStream_t stream);

/*
 * hipgemm_gemm that allocates nothing: schedules that need scratch memory
 * (the skinny schedule's split-K counters and partial tiles, the 128 x 128
 * schedule's K-slices) use a static device array of the library,
 * HIPGEMM_NOALLOC_SCRATCH_BYTES per GPU: it belongs to the code object of
 * its own translation unit, which the HIP runtime loads on a GPU at the first
 * hipgemm_gemm_noalloc call there that needs scratch, and holds until the
 * process ends (with the runtime's deferred code-object loading; without
 * it, on every GPU where the library's code is loaded).  No call makes an
 * allocation or a memset.
 * desc->workspace must be NULL and desc->workspace_bytes 0.  Returns
 * hipErrorInvalidValue when the descriptor is invalid (as hipgemm_gemm) or
 * when the call would need more scratch than HIPGEMM_NOALLOC_SCRATCH_BYTES
 * (hipgemm_gemm_workspace_size(desc) tells; never on MI355X, whose largest
 * need is 32 MiB plus the counter region).  Every call on one GPU shares
 * that GPU's array and leaves its counters at zero: calls on one stream
 * are ordered, but calls that may overlap on one GPU (other streams,
 * threads or processes' graphs replayed concurrently) race on it.  Its
 * first call on a GPU looks the array's address up (hipGetSymbolAddress)
 * and clears its counters with a kernel on `stream`.
 * No reference counterpart (the reference's kernel needs no scratch).  For
 * callers that cannot allocate device memory: code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc.
 */
#define HIPGEMM_NOALLOC_SCRATCH_BYTES (HIPGEMM_WS_COUNTER_BYTES + (32u << 20))
hipError_t hipgemm_gemm_noalloc(const hipgemm_gemm_desc *desc,
                                hipStream_t stream);

/*
 * MX scale packing.  hipgemm_mx_scales_bytes: bytes of the packed layout for
 * an operand of `rows` rows and K columns (0 for rows or K <= 0).
 * hipgemm_mx_pack_scales: packs src, `rows` x ceil(K/32) E8M0 bytes with
 * row stride ld bytes (device), into dst (device, that many bytes),
 * stream-ordered.  The layout groups, per 128 rows and per two 128-wide
 * K-steps, what one wave's MFMA need (padding scales are 1.0).  Returns
 * hipErrorInvalidValue for K % 32 != 0, ld < K / 32 or null pointers.
 * No reference counterpart (the reference passes zero scales,
 * fp8_4wave.hpp:58).
 */
size_t hipgemm_mx_scales_bytes(int rows, int K);
hipError_t hipgemm_mx_pack_scales(const void *src, int rows, int K, int ld,
                                  void *dst, hipStream_t stream);

/* Workspace bytes hipgemm_fp8_gemm_bf16_ws needs for this shape and variant
 * on the current device (0: none).  No GPU work.  No reference counterpart. */
size_t hipgemm_workspace_size(int M, int N, int K, int variant);

/* Workspace bytes hipgemm_gemm needs for this descriptor on the current
 * device (0: none, or an invalid descriptor); it accounts for the operand
 * formats and the schedule AUTO takes for them.  No GPU work.  No reference
 * counterpart. */
size_t hipgemm_gemm_workspace_size(const hipgemm_gemm_desc *desc);

/*
 * The reference launch with runtime shapes: packed strides (lda = ldb = K,
 * ldc = N), no scales, the 4-wave schedule (16x16x128 MFMA).
 * Replaces: fp8_gemm_4wave_256x256x128<M, N, K><<<(M*N)/65536, 256>>>(A, B_T,
 * C) at test.cpp:79 and bench.cpp:55/78.
 */
hipError_t hipgemm_fp8_gemm_4wave_256x256x128(const void *A, const void *B_T,
                                              void *C, int M, int N, int K,
                                              hipStream_t stream);

/* Variant AUTO resolves to for this shape (no GPU needed). No reference
 * counterpart (the reference has one schedule). */
int hipgemm_select_variant(int M, int N, int K);

/* AUTO's column split: when the last round of 256 x 256 tiles would leave
 * most CUs idle, AUTO runs columns [0, n1) of C on the 4-wave 16x16x128
 * schedule (whole rounds) and [n1, N) on the 128 x 128 schedule, two
 * launches on the caller's stream.  Returns n1 (a multiple of 256), or 0
 * when AUTO runs one schedule.  Uses the current device's CU count (256
 * without a device).  No reference counterpart (the reference's grid is
 * M*N/65536 tiles of 256 x 256, fp8_4wave.hpp:357-377). */
int hipgemm_split_columns(int M, int N, int K);

/* Human-readable variant name, or NULL.  No reference counterpart. */
const char *hipgemm_variant_name(int variant);

/* HIPGEMM_VERSION of the built library.  No reference counterpart. */
int hipgemm_version(void);

/*
 * Host-side view of the workgroup -> output-tile order a launch of `grid`
 * workgroups uses over a tiles_m x tiles_n tile grid: fills tile_m[i],
 * tile_n[i] for the i-th tile processed (workgroup-major: the tiles of
 * workgroup b are b's first, second, ... tile).  Returns the number of
 * entries written (at most cap).  For tests of the order's bijectivity; no
 * GPU needed.  group_m <= 0 selects the library default.  Replaces the
 * in-kernel remap at fp8_4wave.hpp:357-377 (not callable there).
 */
int hipgemm_tile_order(int grid, int tiles_m, int tiles_n, int group_m,
                       int *tile_m, int *tile_n, int cap);

/*
 * Host-side view of the LDS tile layout: the 16-byte slot (0..7) at which
 * K-chunk `chunk` (0..7) of tile row `row` sits inside its 128-byte LDS row.
 * For tests of the bank-conflict-freedom of the layout; no GPU needed.
 * Returns -1 for out-of-range arguments.  Replaces the swizzle helpers at
 * fp8_4wave.hpp:136-177 (not callable there).
 */
int hipgemm_lds_slot(int row, int chunk);

/*
 * The same for the instruction K order (MX block scales on either tiled
 * schedule, every operand format of the 128x128 schedule but fp6, and the
 * skinny schedule's A): the MFMA's lane group g holds K-chunks g
 * and g + 4 of its row, stored where the plain order above keeps chunks 2g
 * and 2g + 1, so both fetch the same LDS addresses.  -1 for out-of-range
 * arguments.  No reference counterpart (its kernel has one K order).
 */
int hipgemm_lds_slot_kpair(int row, int chunk);

/*
 * The 8-byte slot (0-15) of the 8-byte piece `piece` (0-15) of row `row` of
 * the 4-wave schedule's epilogue stage (128-byte rows of bf16 C, staged
 * between the accumulators and the 16-byte stores of whole 128-byte lines).
 * -1 for out-of-range arguments.  No reference counterpart (its epilogue
 * stores from the accumulators).
 */
int hipgemm_lds_stage_slot(int row, int piece);

#ifdef __cplusplus
}
#endif

#endif /* HIPGEMM_H */
