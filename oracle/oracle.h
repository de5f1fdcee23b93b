/*
 * hipgemm oracle -- CPU restatement of the reference FP8 GEMM path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the hipgemm_amd package,
 * libhipgemm.so, include/) may include, link or call this code.  Only tests/,
 * __graft_entry__.smoke() and the cpu_baseline leg of bench.py use it, and only
 * as the checker.
 *
 * Reference being restated (nirw4nna/hipgemm):
 *   test.cpp:19-30   gemm_cpu: per output, fp32 sequential-K sum of
 *                    float(A[row*K+k]) * float(B[col*K+k]), then bf16(acc) (RNE)
 *   utils.hpp:27-34  init_random: mt19937(seed), normal_distribution<float>(-1,1),
 *                    cast to fp8 (e4m3, RNE, satfinite)
 *   fp8_4wave.hpp:15-16  fp8 = __hip_fp8_e4m3 (OCP E4M3FN), bf16 = __hip_bfloat16
 *
 * Extension the reference does not have: per-tensor fp32 scales applied as
 *   C = bf16_rne(acc * (scale_a * scale_b)), every step in fp32.
 * With scale_a = scale_b = 1 this is bit-identical to gemm_cpu.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   hg_f32_to_e4m3 / hg_e4m3_to_f32 : exhaustive 2^32 sweep against the HIP
 *       header conversion (__hip_fp8_e4m3 ctor / operator float), plus OCP
 *       closed-form values.
 *   hg_f32_to_bf16                  : exhaustive sweep against HIP's
 *       __hip_bfloat16(float) (static_cast<__bf16>), plus closed forms.
 *   hg_gemm_ref / hg_gemm_fast / hg_gemm_rows : bit-exact against the
 *       reference's own gemm_cpu compiled from its sources (oracle/_ref),
 *       brute-force fp64 on tiny shapes, one-hot / permutation / all-ones
 *       closed forms.
 *   hg_fill_e4m3 (REFTEST mode)     : bit-exact against the reference's
 *       init_random compiled from its sources (oracle/_ref).
 *   hg_fill_e4m3 (UNIFORM / NORMAL) : the build's own seeded generators (the
 *       reference has no such generator); pinned by committed golden hashes
 *       and distribution-moment checks.
 */
#ifndef HIPGEMM_ORACLE_H
#define HIPGEMM_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- element codecs ---------------------------------------------------- */
uint8_t hg_f32_to_e4m3(float x);      /* RNE, satfinite, Inf/NaN -> NaN    */
float hg_e4m3_to_f32(uint8_t v);      /* exact                              */
uint16_t hg_f32_to_bf16(float x);     /* RNE, NaN -> quiet NaN              */
float hg_bf16_to_f32(uint16_t v);     /* exact                              */

void hg_f32_to_e4m3_n(const float *x, uint8_t *out, size_t n);
void hg_e4m3_to_f32_n(const uint8_t *x, float *out, size_t n);
void hg_f32_to_bf16_n(const float *x, uint16_t *out, size_t n);
void hg_bf16_to_f32_n(const uint16_t *x, float *out, size_t n);

/* ---- seeded generators -------------------------------------------------- */
enum {
  HG_DIST_UNIFORM = 0, /* p0 + (p1 - p0) * u, u in [0,1)                     */
  HG_DIST_NORMAL = 1,  /* mean p0, std p1 (Box-Muller), clipped to +-448      */
};
uint64_t hg_rand64(uint64_t seed, uint64_t index);
/* Fill n e4m3 bytes; element i depends only on (seed, i) so the fill is
 * order-independent and parallel. */
void hg_fill_e4m3(uint8_t *out, size_t n, uint64_t seed, int dist, double p0,
                  double p1);
/* One fp32 scale drawn uniform in [lo, hi). */
float hg_draw_scale(uint64_t seed, double lo, double hi);
/* Reference-test mode: reproduces utils.hpp:27-34 (mt19937 + libstdc++
 * normal_distribution<float>(-1, 1)), implemented in reftest_rng.cpp. */
void hg_fill_e4m3_reftest(uint8_t *out, size_t n, uint64_t seed);

/* ---- GEMM --------------------------------------------------------------- */
/* C[M x N] (bf16 bits, ldc) = bf16(scale_a*scale_b * A[M x K] . B_T[N x K]^T)
 * A row-major (lda), B_T row-major N x K (ldb).  Faithful restatement of
 * test.cpp:19-30: OpenMP over outputs, scalar sequential-K fp32 sum. */
void hg_gemm_ref(const uint8_t *A, const uint8_t *B_T, uint16_t *C, int M,
                 int N, int K, int lda, int ldb, int ldc, float scale_a,
                 float scale_b);
/* Bit-identical to hg_gemm_ref (per-output sequential K order is kept; the
 * e4m3 x e4m3 products are exact in fp32, so vectorising across outputs does
 * not change any sum).  Blocked and SIMD across output columns. */
void hg_gemm_fast(const uint8_t *A, const uint8_t *B_T, uint16_t *C, int M,
                  int N, int K, int lda, int ldb, int ldc, float scale_a,
                  float scale_b);
/* Per-row / per-column scales (an extension, like the per-tensor ones):
 *   C[m, n] = bf16_rne(acc[m, n] * (scale_rows[m] * scale_cols[n]))
 * with acc the same fp32 sequential-K sum as hg_gemm_fast and the product of
 * the two scales formed in fp32 first.  Either vector may be NULL (1.0).
 * Pinned by reduction to the pinned per-tensor path: constant vectors equal
 * hg_gemm_fast with those two scalars; each row with a row scale equals
 * hg_gemm_rows with that scale_a; column scales likewise through the
 * transposed product (tests/test_oracle.py). */
void hg_gemm_rowcol(const uint8_t *A, const uint8_t *B_T, uint16_t *C, int M,
                    int N, int K, int lda, int ldb, int ldc,
                    const float *scale_rows, const float *scale_cols);

/* Same as hg_gemm_fast for the listed rows only: output row r of C_rows
 * (row-major, ld = N) is row rows[r] of the full product. */
void hg_gemm_rows(const uint8_t *A, const uint8_t *B_T, uint16_t *C_rows,
                  const int *rows, int nrows, int N, int K, int lda, int ldb,
                  float scale_a, float scale_b);
/* fp32 accumulators (before scale and rounding) for the listed rows. */
void hg_gemm_rows_acc(const uint8_t *A, const uint8_t *B_T, float *acc_rows,
                      const int *rows, int nrows, int N, int K, int lda,
                      int ldb);
/* Exact (fp64) accumulators for the listed rows; used to separate CPU and
 * GPU rounding when reporting error statistics. */
void hg_gemm_rows_f64(const uint8_t *A, const uint8_t *B_T, double *acc_rows,
                      const int *rows, int nrows, int N, int K, int lda,
                      int ldb);

/* ---- Extensions beyond the reference: other formats, fused epilogue ----- */
enum { HG_FMT_E4M3 = 0, HG_FMT_E5M2 = 1, HG_FMT_FP6_E2M3 = 2,
       HG_FMT_FP6_E3M2 = 3, HG_FMT_FP4 = 4 };
/* OCP E2M1 (FP4) decode of the low nibble of v; hg_gemm_ex takes fp4
 * operands (both) as two elements per byte, element 2i in the low nibble of
 * byte i, lda / ldb in bytes.  Pinned: the decode against the OCP MX v1.0
 * value table; the GEMM against fp64 sums of the decoded values. */
float hg_fp4_to_f32(uint8_t v);
/* OCP FP6 (MX v1.0) decodes of the low 6 bits of v: E2M3 (bias 1, largest
 * 7.5) and E3M2 (bias 3, largest 28), no Inf or NaN.  hg_gemm_ex / hg_gemm_mx
 * take fp6 operands (both fp6, either variant each) packed LSB first: element
 * k of a row at bits [6k, 6k + 6) of the row's little-endian bit string
 * (4 elements per 3 bytes), lda / ldb in bytes.  Pinned: the decodes against
 * the OCP value tables written out; the unpacking against a bit-string
 * restatement in numpy; the GEMM against fp64 sums (tests/test_oracle.py). */
float hg_fp6_e2m3_to_f32(uint8_t v);
float hg_fp6_e3m2_to_f32(uint8_t v);
enum { HG_OUT_BF16 = 0, HG_OUT_F16 = 1, HG_OUT_F32 = 2, HG_OUT_FP8 = 3 };
enum { HG_ACT_NONE = 0, HG_ACT_RELU = 1, HG_ACT_GELU_TANH = 2, HG_ACT_SILU = 3 };
/* OCP E5M2 decode (exact) and RNE encode (overflow to inf, NaN -> NaN),
 * IEEE binary16 RNE encode.  Pinned: e5m2 decode against its closed form
 * (the upper byte of a binary16, numpy float16); e5m2 encode against
 * torch's float8_e5m2 conversion and f16 encode against numpy's float16
 * conversion on large samples plus every boundary (tests/test_oracle.py). */
float hg_e5m2_to_f32(uint8_t v);
uint8_t hg_f32_to_e5m2(float x);
uint16_t hg_f32_to_f16(float x);
void hg_e5m2_to_f32_n(const uint8_t *x, float *out, size_t n);
void hg_f32_to_e5m2_n(const float *x, uint8_t *out, size_t n);
void hg_f32_to_f16_n(const float *x, uint16_t *out, size_t n);
/* The hipgemm_gemm semantics: acc = the same sequential-K fp32 sum as
 * hg_gemm_fast over A decoded as a_fmt and B_T as b_fmt (the products of two
 * 8-bit values are exact in fp32 for every pair of these formats), then
 *   scale = scale_rows[m] * (scale_cols[n] * (scale_a * scale_b))
 *   v = fmaf(acc, scale, bias[n])   (bias NULL: -0.0)
 *   y = act(v)
 *   C = bf16 / f16 bits of y (RNE), y itself (fp32), or
 *       hg_f32_to_e4m3(y * scale_out) (e4m3 output)
 * C has row stride ldc elements of the output type (2, 2, 4 or 1 bytes).
 * with the activation evaluated in double from its definition.  Pinned:
 * the defaults equal hg_gemm_fast and vectors alone equal hg_gemm_rowcol
 * bit for bit; e5m2 operands against fp64 sums of the decoded values;
 * bias against an fp64 fma; activations against scipy's expit and torch's
 * tanh-approximated gelu; f16 output against numpy. */
void hg_gemm_ex(const uint8_t *A, const uint8_t *B_T, void *C, int M,
                int N, int K, int lda, int ldb, int ldc, int a_fmt, int b_fmt,
                int out, int act, float scale_a, float scale_b,
                const float *scale_rows, const float *scale_cols,
                const float *bias, float scale_out);

/* MX block scales (OCP Microscaling v1.0): sa is M x ceil(K/32) E8M0 bytes
 * (row stride ldsa), sb N x ceil(K/32) (ldsb); element k of a row is scaled
 * by 2^(e - 127) of its block k / 32 (e = 255: NaN), then the sum runs as in
 * hg_gemm_fast and C = bf16_rne(acc * (scale_a * scale_b)).  Pinned: unit
 * scales equal hg_gemm_ex; scales constant along each row equal
 * hg_gemm_ex's row / column vectors; per-block scales on exact sums against
 * fp64; NaN scales (tests/test_oracle.py). */
void hg_gemm_mx(const uint8_t *A, const uint8_t *B_T, uint16_t *C, int M,
                int N, int K, int lda, int ldb, int ldc, int a_fmt, int b_fmt,
                const uint8_t *sa, int ldsa, const uint8_t *sb, int ldsb,
                float scale_a, float scale_b);

/* Threads OpenMP will use (for reporting cpu_baseline.cores). */
int hg_num_threads(void);

#ifdef __cplusplus
}
#endif
#endif
