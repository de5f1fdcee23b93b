/*
 * hipgemm oracle -- CPU restatement of the reference FP8 GEMM path.
 * TEST INFRASTRUCTURE ONLY (see oracle.h for the contract and what pins each
 * function).  Reference citations are file:line into nirw4nna/hipgemm.
 */
#include "oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static inline uint32_t f32_bits(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  return u;
}
static inline float bits_f32(uint32_t u) {
  float x;
  memcpy(&x, &u, 4);
  return x;
}

/* ------------------------------------------------------------------------ */
/* OCP E4M3FN ("fp8" of fp8_4wave.hpp:15).  1 sign, 4 exponent (bias 7), 3   */
/* mantissa bits; exponent field 0 is subnormal (m * 2^-9); S.1111.111 is    */
/* NaN; there is no infinity; the largest finite magnitude is 1.75*2^8=448.  */
/* ------------------------------------------------------------------------ */
float hg_e4m3_to_f32(uint8_t v) {
  const int e = (v >> 3) & 15, m = v & 7;
  float mag;
  if (e == 15 && m == 7)
    mag = NAN;
  else if (e == 0)
    mag = ldexpf((float)m, -9);
  else
    mag = ldexpf((float)(8 + m), e - 10);
  return (v & 0x80) ? -mag : mag;
}

/* Round-to-nearest-even onto the e4m3 grid with saturation to +-448, the
 * behaviour of the __hip_fp8_e4m3(float) constructor the reference uses
 * (utils.hpp:32): its default is __HIP_SATFINITE, Inf and NaN both become
 * NaN (0x7f | sign), magnitudes above 448 become 448.  Method: scale by the
 * grid quantum of x's binade (a power of two, so exact), round to an integer
 * with rintf (RNE in the default rounding mode), then re-encode the value. */
uint8_t hg_f32_to_e4m3(float x) {
  const uint32_t u = f32_bits(x);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
  const uint32_t a = u & 0x7fffffffu;
  if (a >= 0x7f800000u) return sign | 0x7f;   /* Inf, NaN -> NaN          */
  if (a > 0x43e00000u) return sign | 0x7e;    /* |x| > 448 -> 448         */
  const float ax = bits_f32(a);
  int e2;
  (void)frexpf(ax, &e2);                      /* ax = f * 2^e2, f in [.5,1) */
  int E = e2 - 1;                             /* ax in [2^E, 2^(E+1))       */
  if (a == 0 || E < -6) E = -6;               /* subnormal quantum 2^-9     */
  const int qexp = E - 3;                     /* 3 mantissa bits            */
  const float n = rintf(ldexpf(ax, -qexp));   /* integer multiple of quantum */
  if (n == 0.0f) return sign;
  const float v = ldexpf(n, qexp);            /* exact, <= 448              */
  if (v < 0.015625f)                          /* < 2^-6: subnormal          */
    return sign | (uint8_t)ldexpf(v, 9);
  int ve;
  (void)frexpf(v, &ve);
  const int Ev = ve - 1;                      /* may be E+1 after rounding  */
  const int mant = (int)ldexpf(v, 3 - Ev) - 8;
  return sign | (uint8_t)(((Ev + 7) << 3) | mant);
}

/* ------------------------------------------------------------------------ */
/* OCP E5M2 (an extension: the reference is e4m3 only).  1 sign, 5 exponent */
/* (bias 15), 2 mantissa bits -- the upper byte of an IEEE binary16:         */
/* exponent field 31 is infinity (m = 0) or NaN, field 0 is subnormal        */
/* (m * 2^-16); the largest finite magnitude is 1.75 * 2^15 = 57344.         */
/* ------------------------------------------------------------------------ */
float hg_e5m2_to_f32(uint8_t v) {
  const int e = (v >> 2) & 31, m = v & 3;
  float mag;
  if (e == 31)
    mag = m ? NAN : INFINITY;
  else if (e == 0)
    mag = ldexpf((float)m, -16);
  else
    mag = ldexpf((float)(4 + m), e - 17);
  return (v & 0x80) ? -mag : mag;
}

/* Round-to-nearest-even onto the e5m2 grid, IEEE overflow: magnitudes from
 * 61440 (halfway from 57344 to 2^16) up become infinity, NaN stays NaN
 * (0x7f | sign).  Same method as hg_f32_to_e4m3. */
uint8_t hg_f32_to_e5m2(float x) {
  const uint32_t u = f32_bits(x);
  const uint8_t sign = (uint8_t)((u >> 24) & 0x80);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7f;    /* NaN                       */
  const float ax = bits_f32(a);
  if (ax >= 61440.0f) return sign | 0x7c;     /* rounds past 57344: inf    */
  int e2;
  (void)frexpf(ax, &e2);
  int E = e2 - 1;                             /* ax in [2^E, 2^(E+1))      */
  if (a == 0 || E < -14) E = -14;             /* subnormal quantum 2^-16   */
  const int qexp = E - 2;                     /* 2 mantissa bits           */
  const float n = rintf(ldexpf(ax, -qexp));
  if (n == 0.0f) return sign;
  const float v = ldexpf(n, qexp);
  if (v < 6.103515625e-05f)                   /* < 2^-14: subnormal        */
    return sign | (uint8_t)ldexpf(v, 16);
  int ve;
  (void)frexpf(v, &ve);
  const int Ev = ve - 1;
  const int mant = (int)ldexpf(v, 2 - Ev) - 4;
  return sign | (uint8_t)(((Ev + 15) << 2) | mant);
}

/* IEEE binary16, round-to-nearest-even, overflow to infinity, NaN kept NaN
 * (quiet).  Method: as above on the 10-bit mantissa grid. */
uint16_t hg_f32_to_f16(float x) {
  const uint32_t u = f32_bits(x);
  const uint16_t sign = (uint16_t)((u >> 16) & 0x8000);
  const uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return sign | 0x7e00;
  const float ax = bits_f32(a);
  if (ax >= 65520.0f) return sign | 0x7c00;   /* halfway past 65504: inf   */
  int e2;
  (void)frexpf(ax, &e2);
  int E = e2 - 1;
  if (a == 0 || E < -14) E = -14;             /* subnormal quantum 2^-24   */
  const int qexp = E - 10;
  const float n = rintf(ldexpf(ax, -qexp));
  if (n == 0.0f) return sign;
  const float v = ldexpf(n, qexp);
  if (v < 6.103515625e-05f) return sign | (uint16_t)ldexpf(v, 24);
  int ve;
  (void)frexpf(v, &ve);
  const int Ev = ve - 1;
  const int mant = (int)ldexpf(v, 10 - Ev) - 1024;
  return sign | (uint16_t)(((Ev + 15) << 10) | mant);
}

void hg_e5m2_to_f32_n(const uint8_t *x, float *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = hg_e5m2_to_f32(x[i]);
}
void hg_f32_to_e5m2_n(const float *x, uint8_t *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = hg_f32_to_e5m2(x[i]);
}
void hg_f32_to_f16_n(const float *x, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = hg_f32_to_f16(x[i]);
}

/* bf16 = upper half of an fp32 with round-to-nearest-even on the dropped
 * half (what __hip_bfloat16(float), test.cpp:27, does on the host); NaN is
 * kept NaN with the quiet bit set. */
uint16_t hg_f32_to_bf16(float x) {
  uint32_t u = f32_bits(x);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

float hg_bf16_to_f32(uint16_t v) { return bits_f32((uint32_t)v << 16); }

void hg_f32_to_e4m3_n(const float *x, uint8_t *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = hg_f32_to_e4m3(x[i]);
}
void hg_e4m3_to_f32_n(const uint8_t *x, float *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = hg_e4m3_to_f32(x[i]);
}
void hg_f32_to_bf16_n(const float *x, uint16_t *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = hg_f32_to_bf16(x[i]);
}
void hg_bf16_to_f32_n(const uint16_t *x, float *out, size_t n) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i) out[i] = hg_bf16_to_f32(x[i]);
}

/* ------------------------------------------------------------------------ */
/* Seeded generators (the build's own; the reference only has utils.hpp's    */
/* mt19937 normal(-1,1), restated separately in reftest_rng.cpp).            */
/* Counter-based: element i = mix(mix(seed) + (i+1) * golden) with the       */
/* SplitMix64 finaliser (Steele, Lea & Flood, OOPSLA 2014).                  */
/* ------------------------------------------------------------------------ */
static inline uint64_t splitmix_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

uint64_t hg_rand64(uint64_t seed, uint64_t index) {
  return splitmix_mix(splitmix_mix(seed) + (index + 1) * 0x9e3779b97f4a7c15ull);
}

static inline double u01_open(uint32_t r) { /* (0, 1) */
  return ((double)r + 0.5) * (1.0 / 4294967296.0);
}

static inline float draw(uint64_t seed, uint64_t i, int dist, double p0,
                         double p1) {
  const uint64_t h = hg_rand64(seed, i);
  if (dist == HG_DIST_UNIFORM) {
    const double u = (double)(h >> 40) * (1.0 / 16777216.0); /* [0,1), 2^-24 */
    return (float)(p0 + (p1 - p0) * u);
  }
  /* Box-Muller, cosine branch (Box & Muller 1958). */
  const double u1 = u01_open((uint32_t)(h >> 32));
  const double u2 = (double)(uint32_t)h * (1.0 / 4294967296.0);
  const double z = sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2);
  double x = p0 + p1 * z;
  if (x > 448.0) x = 448.0;
  if (x < -448.0) x = -448.0;
  return (float)x;
}

void hg_fill_e4m3(uint8_t *out, size_t n, uint64_t seed, int dist, double p0,
                  double p1) {
#pragma omp parallel for schedule(static)
  for (size_t i = 0; i < n; ++i)
    out[i] = hg_f32_to_e4m3(draw(seed, (uint64_t)i, dist, p0, p1));
}

float hg_draw_scale(uint64_t seed, double lo, double hi) {
  return draw(seed ^ 0x5ca1e5ca1e5ca1e5ull, 0, HG_DIST_UNIFORM, lo, hi);
}

/* ------------------------------------------------------------------------ */
/* GEMM                                                                      */
/* ------------------------------------------------------------------------ */
static float g_e4m3_lut[256];
static float g_e5m2_lut[256];
static float g_fp4_lut[256];   /* indexed by a nibble value 0..15 */
static float g_e2m3_lut[256];  /* indexed by a 6-bit code 0..63 */
static float g_e3m2_lut[256];
static int g_lut_ready = 0;

static void lut_init(void) {
  if (g_lut_ready) return;
#pragma omp critical(hg_lut)
  {
    if (!g_lut_ready) {
      for (int i = 0; i < 256; ++i) {
        g_e4m3_lut[i] = hg_e4m3_to_f32((uint8_t)i);
        g_e5m2_lut[i] = hg_e5m2_to_f32((uint8_t)i);
        g_fp4_lut[i] = hg_fp4_to_f32((uint8_t)(i & 15));
        g_e2m3_lut[i] = hg_fp6_e2m3_to_f32((uint8_t)(i & 63));
        g_e3m2_lut[i] = hg_fp6_e3m2_to_f32((uint8_t)(i & 63));
      }
      g_lut_ready = 1;
    }
  }
}

static const float *lut_of(int fmt) {
  lut_init();
  return fmt == HG_FMT_E5M2        ? g_e5m2_lut
         : fmt == HG_FMT_FP4       ? g_fp4_lut
         : fmt == HG_FMT_FP6_E2M3  ? g_e2m3_lut
         : fmt == HG_FMT_FP6_E3M2  ? g_e3m2_lut
                                   : g_e4m3_lut;
}

static inline uint16_t epilogue(float acc, float s) {
  return hg_f32_to_bf16(acc * s);
}

/* test.cpp:19-30, plus the per-tensor scale extension.  Loop order, the
 * OpenMP collapse(2) over (row, col) and the scalar fp32 K sum follow the
 * reference; the e4m3 decode goes through a 256-entry table holding the same
 * values the HIP header's operator float returns. */
void hg_gemm_ref(const uint8_t *A, const uint8_t *B_T, uint16_t *C, int M,
                 int N, int K, int lda, int ldb, int ldc, float scale_a,
                 float scale_b) {
  lut_init();
  const float s = scale_a * scale_b;
#pragma omp parallel for collapse(2)
  for (int row = 0; row < M; ++row) {
    for (int col = 0; col < N; ++col) {
      float acc = 0.0f;
      for (int k = 0; k < K; ++k)
        acc += g_e4m3_lut[A[(size_t)row * lda + k]] *
               g_e4m3_lut[B_T[(size_t)col * ldb + k]];
      C[(size_t)row * ldc + col] = epilogue(acc, s);
    }
  }
}

/* B_T decoded (format fmt) and transposed to Bt[K][N] fp32. */
static float *decode_bt_fmt(const uint8_t *B_T, int N, int K, int ldb,
                            int fmt) {
  float *Bt = (float *)malloc((size_t)K * N * sizeof(float));
  if (!Bt) return NULL;
  const float *lut = lut_of(fmt);
#pragma omp parallel for schedule(static)
  for (int kb = 0; kb < K; kb += 64) {
    const int ke = kb + 64 < K ? kb + 64 : K;
    for (int n = 0; n < N; ++n)
      for (int k = kb; k < ke; ++k)
        Bt[(size_t)k * N + n] = lut[B_T[(size_t)n * ldb + k]];
  }
  return Bt;
}
static float *decode_bt(const uint8_t *B_T, int N, int K, int ldb) {
  return decode_bt_fmt(B_T, N, K, ldb, HG_FMT_E4M3);
}

#define RB 8   /* rows per block    */
#define CB 128 /* columns per block */

/* acc[r][j] for rows rows[0..nr) and columns [n0, n0+nc): per output the K
 * sum runs k = 0, 1, ..., K-1 in fp32, as in the reference. */
static void block_acc(const uint8_t *A, const float *lut_a, const float *Bt,
                      const int *rows, int nr, int n0, int nc, int N, int K,
                      int lda, float acc[RB][CB]) {
  const uint8_t *arow[RB];
  for (int r = 0; r < RB; ++r) {
    arow[r] = A + (size_t)rows[r < nr ? r : 0] * lda;
    for (int j = 0; j < CB; ++j) acc[r][j] = 0.0f;
  }
  for (int k = 0; k < K; ++k) {
    const float *b = Bt + (size_t)k * N + n0;
    for (int r = 0; r < RB; ++r) {
      const float a = lut_a[arow[r][k]];
      float *ac = acc[r];
      if (nc == CB) {
#pragma omp simd
        for (int j = 0; j < CB; ++j) ac[j] += a * b[j];
      } else {
        for (int j = 0; j < nc; ++j) ac[j] += a * b[j];
      }
    }
  }
}

/* OCP E2M1 (OCP Microscaling v1.0, FP4): 1 sign bit (3), 2 exponent bits
 * (2:1, bias 1), 1 mantissa bit (0); exponent field 0 is subnormal (m/2).
 * Values 0, 0.5, 1, 1.5, 2, 3, 4, 6.  No Inf or NaN. */
float hg_fp4_to_f32(uint8_t v) {
  const int e = (v >> 1) & 3, m = v & 1;
  const float mag = e == 0 ? 0.5f * (float)m : ldexpf(1.0f + 0.5f * (float)m, e - 1);
  return (v & 8) ? -mag : mag;
}

/* OCP FP6 (OCP Microscaling v1.0).  E2M3: 1 sign bit (5), 2 exponent bits
 * (4:3, bias 1), 3 mantissa bits (2:0); exponent field 0 is subnormal,
 * m / 8.  Largest 7.5.  E3M2: 1 sign bit (5), 3 exponent bits (4:2, bias 3),
 * 2 mantissa bits (1:0); exponent field 0 is subnormal, m / 16.  Largest 28.
 * Neither has Inf or NaN; the low 6 bits of v are the code. */
float hg_fp6_e2m3_to_f32(uint8_t v) {
  const int e = (v >> 3) & 3, m = v & 7;
  const float mag = e == 0 ? 0.125f * (float)m : ldexpf(1.0f + 0.125f * (float)m, e - 1);
  return (v & 32) ? -mag : mag;
}
float hg_fp6_e3m2_to_f32(uint8_t v) {
  const int e = (v >> 2) & 7, m = v & 3;
  const float mag = e == 0 ? 0.0625f * (float)m : ldexpf(1.0f + 0.25f * (float)m, e - 3);
  return (v & 32) ? -mag : mag;
}

/* rows x K fp6 elements packed LSB first, element k of a row at bits
 * [6k, 6k + 6) of the row's little-endian bit string (four elements in
 * three bytes: element 4j + t in bits 6t .. 6t + 5 of bytes 3j .. 3j + 2
 * read as a 24-bit little-endian word), row stride ld bytes -> rows x K
 * bytes, one 6-bit code each. */
static uint8_t *unpack_fp6(const uint8_t *X, int rows, int K, int ld) {
  uint8_t *u = (uint8_t *)malloc((size_t)(rows > 0 ? rows : 1) * (K > 0 ? K : 1));
  if (!u) abort();
  for (int r = 0; r < rows; ++r)
    for (int k = 0; k < K; ++k) {
      const size_t bit = (size_t)6 * k;
      const uint8_t *p = X + (size_t)r * ld + bit / 8;
      const unsigned w = (unsigned)p[0] | ((bit % 8) > 2 ? (unsigned)p[1] << 8 : 0u);
      u[(size_t)r * K + k] = (uint8_t)((w >> (bit % 8)) & 63u);
    }
  return u;
}

/* rows x K fp4 elements, two per byte (element 2i in the low nibble of byte
 * i of a row, row stride ld bytes) -> rows x K bytes, one nibble each. */
static uint8_t *unpack_fp4(const uint8_t *X, int rows, int K, int ld) {
  uint8_t *u = (uint8_t *)malloc((size_t)(rows > 0 ? rows : 1) * (K > 0 ? K : 1));
  if (!u) abort();
  for (int r = 0; r < rows; ++r)
    for (int k = 0; k < K; ++k) {
      const uint8_t b = X[(size_t)r * ld + k / 2];
      u[(size_t)r * K + k] = (k & 1) ? (uint8_t)(b >> 4) : (uint8_t)(b & 15);
    }
  return u;
}

/* Operand X of `rows` rows in format fmt: for fp4 and fp6 an unpacked copy,
 * one code per byte (*X and *ld updated, the copy returned for freeing);
 * NULL and no change for the 8-bit formats. */
static uint8_t *unpack_sub8(const uint8_t **X, int fmt, int rows, int K, int *ld) {
  uint8_t *u = NULL;
  if (fmt == HG_FMT_FP4)
    u = unpack_fp4(*X, rows, K, *ld);
  else if (fmt == HG_FMT_FP6_E2M3 || fmt == HG_FMT_FP6_E3M2)
    u = unpack_fp6(*X, rows, K, *ld);
  if (u) {
    *X = u;
    *ld = K;
  }
  return u;
}

/* The extended epilogue of hg_gemm_ex. */
typedef struct {
  float s;                        /* scale_a * scale_b                     */
  const float *sr, *sc, *bias;    /* NULL: ones / ones / -0.0              */
  int act, out;
  float so;                       /* e4m3 output scale                     */
} epi_t;

/* The activations from their definitions, in double (the reference for the
 * kernels' fp32 hardware-exponential evaluation). */
static float act_f(float v, int act) {
  const double x = v;
  switch (act) {
    case HG_ACT_RELU:
      return v < 0.0f ? 0.0f : v;
    case HG_ACT_SILU:
      return (float)(x / (1.0 + exp(-x)));
    case HG_ACT_GELU_TANH:
      return (float)(0.5 * x *
                     (1.0 + tanh(0.7978845608028654 * (x + 0.044715 * x * x * x))));
    default:
      return v;
  }
}

/* Element o of the output array (of e->out's type) for accumulator acc at
 * (m, n). */
static void epi_store(void *out, size_t o, float acc, int m, int n,
                      const epi_t *e) {
  const float sr = e->sr ? e->sr[m] : 1.0f;
  const float sc = e->sc ? e->sc[n] : 1.0f;
  const float scale = sr * (sc * e->s);
  const float v = fmaf(acc, scale, e->bias ? e->bias[n] : -0.0f);
  const float y = act_f(v, e->act);
  switch (e->out) {
    case HG_OUT_F16: ((uint16_t *)out)[o] = hg_f32_to_f16(y); break;
    case HG_OUT_F32: ((float *)out)[o] = y; break;
    case HG_OUT_FP8: ((uint8_t *)out)[o] = hg_f32_to_e4m3(y * e->so); break;
    default: ((uint16_t *)out)[o] = hg_f32_to_bf16(y); break;
  }
}

/* mode 0: bf16 of acc * s, or, with sa / sb given (row / column scale
 * vectors, either may be NULL = 1.0), of acc * (sa[row] * sb[col]); mode 1:
 * the fp32 acc itself; mode 2: the extended epilogue `ep`. */
static void rows_impl_lut(const uint8_t *A, const float *lut_a,
                          const float *Bt, const int *rows, int nrows, int N,
                          int K, int lda, void *out, int ldo, int mode, float s,
                          const float *sa, const float *sb, const epi_t *ep) {
  const int nrb = (nrows + RB - 1) / RB, ncb = (N + CB - 1) / CB;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int rb = 0; rb < nrb; ++rb) {
    for (int cb = 0; cb < ncb; ++cb) {
      float acc[RB][CB] __attribute__((aligned(64)));
      const int r0 = rb * RB, n0 = cb * CB;
      const int nr = nrows - r0 < RB ? nrows - r0 : RB;
      const int nc = N - n0 < CB ? N - n0 : CB;
      block_acc(A, lut_a, Bt, rows + r0, nr, n0, nc, N, K, lda, acc);
      for (int r = 0; r < nr; ++r)
        for (int j = 0; j < nc; ++j) {
          const size_t o = (size_t)(r0 + r) * ldo + n0 + j;
          if (mode == 2) {
            epi_store(out, o, acc[r][j], rows[r0 + r], n0 + j, ep);
          } else if (mode == 0 && (sa || sb)) {
            const float rs = sa ? sa[rows[r0 + r]] : 1.0f;
            const float cs = sb ? sb[n0 + j] : 1.0f;
            ((uint16_t *)out)[o] = epilogue(acc[r][j], rs * cs);
          } else if (mode == 0) {
            ((uint16_t *)out)[o] = epilogue(acc[r][j], s);
          } else {
            ((float *)out)[o] = acc[r][j];
          }
        }
    }
  }
}

static void rows_impl(const uint8_t *A, const float *Bt, const int *rows,
                      int nrows, int N, int K, int lda, void *out, int ldo,
                      int mode, float s, const float *sa, const float *sb) {
  rows_impl_lut(A, lut_of(HG_FMT_E4M3), Bt, rows, nrows, N, K, lda, out, ldo,
                mode, s, sa, sb, NULL);
}

void hg_gemm_ex(const uint8_t *A, const uint8_t *B_T, void *C, int M,
                int N, int K, int lda, int ldb, int ldc, int a_fmt, int b_fmt,
                int out, int act, float scale_a, float scale_b,
                const float *scale_rows, const float *scale_cols,
                const float *bias, float scale_out) {
  /* fp4 / fp6: one byte per element (the code), then the same path. */
  uint8_t *Au = unpack_sub8(&A, a_fmt, M, K, &lda);
  uint8_t *Bu = unpack_sub8(&B_T, b_fmt, N, K, &ldb);
  float *Bt = decode_bt_fmt(B_T, N, K, ldb, b_fmt);
  int *rows = (int *)malloc((size_t)(M > 0 ? M : 1) * sizeof(int));
  if (!Bt || !rows) abort();
  for (int i = 0; i < M; ++i) rows[i] = i;
  const epi_t ep = {scale_a * scale_b, scale_rows, scale_cols, bias, act, out,
                    scale_out};
  rows_impl_lut(A, lut_of(a_fmt), Bt, rows, M, N, K, lda, C, ldc, 2, 1.0f, NULL,
                NULL, &ep);
  free(rows);
  free(Bt);
  free(Au);
  free(Bu);
}

/* ------------------------------------------------------------------------ */
/* MX block scales (OCP Microscaling v1.0, an extension: the reference has   */
/* none).  One E8M0 scale per 32 consecutive K-elements of a row of A or     */
/* B_T: the value 2^(e - 127), e = 255 is NaN.  Each operand is decoded and  */
/* multiplied by its block scale (a power of two: exact unless it leaves     */
/* the fp32 range), then summed in the same sequential fp32 K order as       */
/* hg_gemm_fast.                                                             */
/* ------------------------------------------------------------------------ */
static inline float e8m0_value(uint8_t e) {
  return e == 255 ? NAN : ldexpf(1.0f, (int)e - 127);
}

void hg_gemm_mx(const uint8_t *A, const uint8_t *B_T, uint16_t *C, int M,
                int N, int K, int lda, int ldb, int ldc, int a_fmt, int b_fmt,
                const uint8_t *sa, int ldsa, const uint8_t *sb, int ldsb,
                float scale_a, float scale_b) {
  const float *la = lut_of(a_fmt), *lb = lut_of(b_fmt);
  /* fp4 / fp6: one byte per element (the code), as in hg_gemm_ex. */
  uint8_t *Au = unpack_sub8(&A, a_fmt, M, K, &lda);
  uint8_t *Bu = unpack_sub8(&B_T, b_fmt, N, K, &ldb);
  float *Af = (float *)malloc((size_t)(M > 0 ? M : 1) * (K > 0 ? K : 1) * sizeof(float));
  float *Bt = (float *)malloc((size_t)(N > 0 ? N : 1) * (K > 0 ? K : 1) * sizeof(float));
  if (!Af || !Bt) abort();
#pragma omp parallel for schedule(static)
  for (int m = 0; m < M; ++m)
    for (int k = 0; k < K; ++k)
      Af[(size_t)m * K + k] =
          la[A[(size_t)m * lda + k]] * e8m0_value(sa[(size_t)m * ldsa + k / 32]);
#pragma omp parallel for schedule(static)
  for (int k = 0; k < K; ++k)
    for (int n = 0; n < N; ++n)
      Bt[(size_t)k * N + n] =
          lb[B_T[(size_t)n * ldb + k]] * e8m0_value(sb[(size_t)n * ldsb + k / 32]);
  const float s = scale_a * scale_b;
  const int ncb = (N + CB - 1) / CB;
#pragma omp parallel for collapse(2) schedule(dynamic, 1)
  for (int m0 = 0; m0 < M; m0 += RB) {
    for (int cb = 0; cb < ncb; ++cb) {
      float acc[RB][CB] __attribute__((aligned(64)));
      const int n0 = cb * CB;
      const int nr = M - m0 < RB ? M - m0 : RB;
      const int nc = N - n0 < CB ? N - n0 : CB;
      for (int r = 0; r < RB; ++r)
        for (int j = 0; j < CB; ++j) acc[r][j] = 0.0f;
      for (int k = 0; k < K; ++k) {
        const float *b = Bt + (size_t)k * N + n0;
        for (int r = 0; r < nr; ++r) {
          const float a = Af[(size_t)(m0 + r) * K + k];
          for (int j = 0; j < nc; ++j) acc[r][j] += a * b[j];
        }
      }
      for (int r = 0; r < nr; ++r)
        for (int j = 0; j < nc; ++j)
          C[(size_t)(m0 + r) * ldc + n0 + j] = epilogue(acc[r][j], s);
    }
  }
  free(Af);
  free(Bt);
  free(Au);
  free(Bu);
}

void hg_gemm_fast(const uint8_t *A, const uint8_t *B_T, uint16_t *C, int M,
                  int N, int K, int lda, int ldb, int ldc, float scale_a,
                  float scale_b) {
  float *Bt = decode_bt(B_T, N, K, ldb);
  int *rows = (int *)malloc((size_t)(M > 0 ? M : 1) * sizeof(int));
  if (!Bt || !rows) abort();
  for (int i = 0; i < M; ++i) rows[i] = i;
  rows_impl(A, Bt, rows, M, N, K, lda, C, ldc, 0, scale_a * scale_b, NULL,
            NULL);
  free(rows);
  free(Bt);
}

void hg_gemm_rowcol(const uint8_t *A, const uint8_t *B_T, uint16_t *C, int M,
                    int N, int K, int lda, int ldb, int ldc,
                    const float *scale_rows, const float *scale_cols) {
  float *Bt = decode_bt(B_T, N, K, ldb);
  int *rows = (int *)malloc((size_t)(M > 0 ? M : 1) * sizeof(int));
  if (!Bt || !rows) abort();
  for (int i = 0; i < M; ++i) rows[i] = i;
  rows_impl(A, Bt, rows, M, N, K, lda, C, ldc, 0, 1.0f, scale_rows,
            scale_cols);
  free(rows);
  free(Bt);
}

void hg_gemm_rows(const uint8_t *A, const uint8_t *B_T, uint16_t *C_rows,
                  const int *rows, int nrows, int N, int K, int lda, int ldb,
                  float scale_a, float scale_b) {
  float *Bt = decode_bt(B_T, N, K, ldb);
  if (!Bt) abort();
  rows_impl(A, Bt, rows, nrows, N, K, lda, C_rows, N, 0, scale_a * scale_b,
            NULL, NULL);
  free(Bt);
}

void hg_gemm_rows_acc(const uint8_t *A, const uint8_t *B_T, float *acc_rows,
                      const int *rows, int nrows, int N, int K, int lda,
                      int ldb) {
  float *Bt = decode_bt(B_T, N, K, ldb);
  if (!Bt) abort();
  rows_impl(A, Bt, rows, nrows, N, K, lda, acc_rows, N, 1, 1.0f, NULL, NULL);
  free(Bt);
}

void hg_gemm_rows_f64(const uint8_t *A, const uint8_t *B_T, double *acc_rows,
                      const int *rows, int nrows, int N, int K, int lda,
                      int ldb) {
  lut_init();
#pragma omp parallel for collapse(2) schedule(static)
  for (int r = 0; r < nrows; ++r)
    for (int n = 0; n < N; ++n) {
      const uint8_t *a = A + (size_t)rows[r] * lda;
      const uint8_t *b = B_T + (size_t)n * ldb;
      double acc = 0.0;
      for (int k = 0; k < K; ++k)
        acc += (double)g_e4m3_lut[a[k]] * (double)g_e4m3_lut[b[k]];
      acc_rows[(size_t)r * N + n] = acc;
    }
}

int hg_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
