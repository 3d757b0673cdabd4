/*
 * oracle.c — CPU restatement of rembed's GEMM family and BERT forward.
 *
 * TEST INFRASTRUCTURE ONLY (the parity reference, never the product). See oracle.h
 * for the pinning map. Every function cites the reference file:line it
 * follows; paths are relative to the rembed source tree.
 *
 * Build: gcc -O3 -mavx2 -mfma -ffp-contract=off -fopenmp (oracle/Makefile).
 * -mavx2 -mfma only lets GCC vectorize the 16-column panel loops: each
 * output element keeps its own sequential fmaf chain, so vectorization
 * across columns cannot change a bit (the reference's 4x16/6x16/4x32
 * kernels rely on the same property, internal/tensor/pack_test.go:133-225).
 */
#include "oracle.h"
#include "oracle_int.h"

#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <immintrin.h>
#endif

/* ------------------------------------------------------------------------ */
/* quantizers                                                                */
/* ------------------------------------------------------------------------ */

/* PackB8, internal/tensor/pack8.go:25-76: float32 absmax, float32 scale
 * maxAbs/127 (1 for an all-zero channel), float64 division, RoundToEven,
 * clamp to +-127; NaN/Inf refused. */
int or_pack_b8(const float *bT, int k, int n, int8_t *q, float *scales) {
  if (n < 16 || n % 16 != 0 || k < 1) return OR_ERR_SHAPE;
  for (int j = 0; j < n; j++) {
    const float *row = bT + (size_t)j * k;
    float maxAbs = 0.0f;
    for (int p = 0; p < k; p++) {
      float v = row[p];
      if (isnan(v) || isinf(v)) return OR_ERR_NONFINITE;
      float a = fabsf(v);
      if (a > maxAbs) maxAbs = a;
    }
    float scale = maxAbs / 127.0f;
    if (scale == 0.0f) scale = 1.0f;
    scales[j] = scale;
    for (int p = 0; p < k; p++) {
      double qd = rint((double)row[p] / (double)scale);
      if (qd > 127.0) qd = 127.0;
      if (qd < -127.0) qd = -127.0;
      q[(size_t)j * k + p] = (int8_t)qd;
    }
  }
  return OR_OK;
}

/* PackB8VNNI, internal/tensor/pack_vnni.go:28-77: float64 absmax and scale,
 * q = int8(RoundToEven(w/scale)) without a clamp, colSum = sum q (int32),
 * scales stored as float32(scale). */
int or_pack_b8_vnni(const float *bT, int k, int n, int8_t *q, int32_t *colsum,
                    float *scales) {
  if (n < 16 || n % 16 != 0 || k < 1) return OR_ERR_SHAPE;
  for (int c = 0; c < n; c++) {
    const float *row = bT + (size_t)c * k;
    double maxAbs = 0.0;
    for (int p = 0; p < k; p++) {
      double v = (double)row[p];
      if (isnan(v) || isinf(v)) return OR_ERR_NONFINITE;
      double a = fabs(v);
      if (a > maxAbs) maxAbs = a;
    }
    double scale = maxAbs / 127.0;
    if (scale == 0.0) scale = 1.0;
    scales[c] = (float)scale;
    uint32_t sum = 0;
    for (int p = 0; p < k; p++) {
      int8_t qv = (int8_t)rint((double)row[p] / scale);
      sum += (uint32_t)(int32_t)qv;
      q[(size_t)c * k + p] = qv;
    }
    colsum[c] = (int32_t)sum;
  }
  return OR_OK;
}

/* QuantizeRowU8, internal/tensor/pack_vnni.go:85-117: float32 absmax,
 * s = maxAbs/127 (1 if zero), inv = 1/s in float32, u8 = clamp(
 * RoundToEven(float64(v*inv)) + 128, 0, 255), tail bytes zeroed. */
float or_quantize_row_u8(uint8_t *dst, int dstlen, const float *a, int k) {
  float maxAbs = 0.0f;
  for (int i = 0; i < k; i++) {
    float x = fabsf(a[i]);
    if (x > maxAbs) maxAbs = x;
  }
  float scale = maxAbs / 127.0f;
  if (scale == 0.0f) scale = 1.0f;
  float inv = 1.0f / scale;
  for (int i = 0; i < k; i++) {
    float prod = a[i] * inv;
    int32_t qv = (int32_t)rint((double)prod) + 128;
    if (qv < 0) qv = 0;
    else if (qv > 255) qv = 255;
    dst[i] = (uint8_t)qv;
  }
  for (int i = k; i < dstlen; i++) dst[i] = 0;
  return scale;
}

/* ------------------------------------------------------------------------ */
/* GEMMs                                                                     */
/* ------------------------------------------------------------------------ */

/* MatMulPacked (internal/tensor/pack.go:123-210) with gemm4x16's per-element
 * order (gemm_amd64.s:31-49): acc starts at +0 and takes fmaf(a[i,p],
 * b[j,p], acc) for p ascending. Columns run 16 at a time over a transposed
 * panel so GCC vectorizes across columns; the chain per element is intact. */
void or_matmul_f32(float *dst, const float *a, const float *bT, int m, int k,
                   int n) {
  float *bp = (float *)malloc(sizeof(float) * (size_t)k * 16);
  for (int j0 = 0; j0 < n; j0 += 16) {
    int w = n - j0 < 16 ? n - j0 : 16;
    for (int p = 0; p < k; p++)
      for (int c = 0; c < 16; c++)
        bp[(size_t)p * 16 + c] = c < w ? bT[(size_t)(j0 + c) * k + p] : 0.0f;
    for (int i = 0; i < m; i++) {
      const float *ar = a + (size_t)i * k;
      float acc[16];
      for (int c = 0; c < 16; c++) acc[c] = 0.0f;
      for (int p = 0; p < k; p++) {
        float av = ar[p];
        const float *b = bp + (size_t)p * 16;
        for (int c = 0; c < 16; c++) acc[c] = fmaf(av, b[c], acc[c]);
      }
      for (int c = 0; c < w; c++) dst[(size_t)i * n + j0 + c] = acc[c];
    }
  }
  free(bp);
}

/* MatMulPacked8 (internal/tensor/pack8.go:80-126) with gemm4x16i8's order
 * (gemm8_amd64.s:32-64): fmaf chain over float(q), then one multiply by the
 * column's scale. */
void or_matmul_w8(float *dst, const float *a, const int8_t *q,
                  const float *scales, int m, int k, int n) {
  float *bp = (float *)malloc(sizeof(float) * (size_t)k * 16);
  for (int j0 = 0; j0 < n; j0 += 16) {
    int w = n - j0 < 16 ? n - j0 : 16;
    for (int p = 0; p < k; p++)
      for (int c = 0; c < 16; c++)
        bp[(size_t)p * 16 + c] =
            c < w ? (float)q[(size_t)(j0 + c) * k + p] : 0.0f;
    for (int i = 0; i < m; i++) {
      const float *ar = a + (size_t)i * k;
      float acc[16];
      for (int c = 0; c < 16; c++) acc[c] = 0.0f;
      for (int p = 0; p < k; p++) {
        float av = ar[p];
        const float *b = bp + (size_t)p * 16;
        for (int c = 0; c < 16; c++) acc[c] = fmaf(av, b[c], acc[c]);
      }
      for (int c = 0; c < w; c++)
        dst[(size_t)i * n + j0 + c] = acc[c] * scales[j0 + c];
    }
  }
  free(bp);
}

/* The integer dot products of VPDPBUSD (vnni_amd64.s:45-68): u8 x s8 summed
 * into int32 with wraparound. Portable body. */
static void gemm_u8s8_portable(int32_t *acc, const uint8_t *qa, int lda,
                               const int8_t *q, int m, int k, int n) {
#pragma omp parallel for schedule(static) if ((double)m * n * k > 1e8)
  for (int i = 0; i < m; i++) {
    const uint8_t *ar = qa + (size_t)i * lda;
    for (int j = 0; j < n; j++) {
      const int8_t *br = q + (size_t)j * k;
      uint32_t s = 0;
      for (int p = 0; p < k; p++)
        s += (uint32_t)((int32_t)ar[p] * (int32_t)br[p]);
      acc[(size_t)i * n + j] = (int32_t)s;
    }
  }
}

#if defined(__x86_64__)
/* Same integers through AVX-512-VNNI VPDPBUSD (the instruction the reference
 * runs, vnni512_amd64.s:16-76): a 4x4 register block of dot products over
 * 64-byte k chunks, masked tail. Sums are exact mod 2^32 in any order. */
__attribute__((target("avx512f,avx512bw,avx512vnni"))) static void
gemm_u8s8_vnni512(int32_t *acc, const uint8_t *qa, int lda, const int8_t *q,
                  int m, int k, int n) {
  int kc = k / 64, kt = k % 64;
  __mmask64 tmask = kt ? (((__mmask64)1 << kt) - 1) : 0;
  /* Row blocks are independent; exact integer sums make the split free. */
#pragma omp parallel for schedule(static) if ((double)m * n * k > 1e8)
  for (int i0 = 0; i0 < m; i0 += 4) {
    int mr = m - i0 < 4 ? m - i0 : 4;
    for (int j0 = 0; j0 < n; j0 += 4) {
      int nr = n - j0 < 4 ? n - j0 : 4;
      __m512i c[4][4];
      for (int r = 0; r < 4; r++)
        for (int s = 0; s < 4; s++) c[r][s] = _mm512_setzero_si512();
      const uint8_t *ar[4];
      const int8_t *br[4];
      for (int r = 0; r < 4; r++)
        ar[r] = qa + (size_t)(i0 + (r < mr ? r : 0)) * lda;
      for (int s = 0; s < 4; s++)
        br[s] = q + (size_t)(j0 + (s < nr ? s : 0)) * k;
      for (int b = 0; b < kc; b++) {
        __m512i av[4], bv[4];
        for (int r = 0; r < 4; r++)
          av[r] = _mm512_loadu_si512((const void *)(ar[r] + b * 64));
        for (int s = 0; s < 4; s++)
          bv[s] = _mm512_loadu_si512((const void *)(br[s] + b * 64));
        for (int r = 0; r < 4; r++)
          for (int s = 0; s < 4; s++)
            c[r][s] = _mm512_dpbusd_epi32(c[r][s], av[r], bv[s]);
      }
      if (kt) {
        __m512i av[4], bv[4];
        for (int r = 0; r < 4; r++)
          av[r] = _mm512_maskz_loadu_epi8(tmask, ar[r] + kc * 64);
        for (int s = 0; s < 4; s++)
          bv[s] = _mm512_maskz_loadu_epi8(tmask, br[s] + kc * 64);
        for (int r = 0; r < 4; r++)
          for (int s = 0; s < 4; s++)
            c[r][s] = _mm512_dpbusd_epi32(c[r][s], av[r], bv[s]);
      }
      for (int r = 0; r < mr; r++)
        for (int s = 0; s < nr; s++)
          acc[(size_t)(i0 + r) * n + j0 + s] = _mm512_reduce_add_epi32(c[r][s]);
    }
  }
}
#endif

/* ------------------------------------------------------------------------ */
/* The reference's own full-int8 kernel shape (the CPU baseline's path)      */
/* ------------------------------------------------------------------------ */

/* PackB8VNNI's weight layout, internal/tensor/pack_vnni.go:44-72: panels of
 * 16 columns, per k-group of 4 the 16 columns' 4 bytes, zero past k:
 * pb[(c/16)*kg*64 + (p/4)*64 + (c%16)*4 + p%4] = q[c][p]. */
void or_pack_vnni_panels(const int8_t *q, int k, int n, int8_t *pb) {
  int kg = (k + 3) / 4;
  memset(pb, 0, (size_t)(n / 16) * kg * 64);
  for (int c = 0; c < n; c++) {
    size_t base = (size_t)(c / 16) * kg * 64 + (size_t)(c % 16) * 4;
    for (int p = 0; p < k; p++) pb[base + (size_t)(p / 4) * 64 + p % 4] = q[(size_t)c * k + p];
  }
}

/* gemm4x16vnni / gemm4x16vnni512 (vnni_amd64.s:22-82, vnni512_amd64.s:16-76):
 * a 4x16 int32 tile; per k-group the 64-byte panel slice is two 8-dword
 * vectors, each row's 4 activation bytes are broadcast, and eight VPDPBUSD
 * accumulate (u8 x s8, wrapping). a0..a3 are the four rows (kg*4 bytes). */
#if defined(__x86_64__)
__attribute__((target("avxvnni"))) static void tile4x16_avxvnni(
    int32_t *dst, int n, const uint8_t *const a[4], const int8_t *pb, int kg) {
  __m256i c0 = _mm256_setzero_si256(), c1 = c0, c2 = c0, c3 = c0, c4 = c0, c5 = c0,
          c6 = c0, c7 = c0;
  for (int g = 0; g < kg; g++) {
    __m256i b0 = _mm256_loadu_si256((const __m256i *)(pb + (size_t)g * 64));
    __m256i b1 = _mm256_loadu_si256((const __m256i *)(pb + (size_t)g * 64 + 32));
    int32_t w0, w1, w2, w3;
    memcpy(&w0, a[0] + 4 * g, 4);
    memcpy(&w1, a[1] + 4 * g, 4);
    memcpy(&w2, a[2] + 4 * g, 4);
    memcpy(&w3, a[3] + 4 * g, 4);
    __m256i r0 = _mm256_set1_epi32(w0), r1 = _mm256_set1_epi32(w1),
            r2 = _mm256_set1_epi32(w2), r3 = _mm256_set1_epi32(w3);
    c0 = _mm256_dpbusd_avx_epi32(c0, r0, b0);
    c1 = _mm256_dpbusd_avx_epi32(c1, r0, b1);
    c2 = _mm256_dpbusd_avx_epi32(c2, r1, b0);
    c3 = _mm256_dpbusd_avx_epi32(c3, r1, b1);
    c4 = _mm256_dpbusd_avx_epi32(c4, r2, b0);
    c5 = _mm256_dpbusd_avx_epi32(c5, r2, b1);
    c6 = _mm256_dpbusd_avx_epi32(c6, r3, b0);
    c7 = _mm256_dpbusd_avx_epi32(c7, r3, b1);
  }
  _mm256_storeu_si256((__m256i *)(dst), c0);
  _mm256_storeu_si256((__m256i *)(dst + 8), c1);
  _mm256_storeu_si256((__m256i *)(dst + n), c2);
  _mm256_storeu_si256((__m256i *)(dst + n + 8), c3);
  _mm256_storeu_si256((__m256i *)(dst + 2 * n), c4);
  _mm256_storeu_si256((__m256i *)(dst + 2 * n + 8), c5);
  _mm256_storeu_si256((__m256i *)(dst + 3 * n), c6);
  _mm256_storeu_si256((__m256i *)(dst + 3 * n + 8), c7);
}

__attribute__((target("avx512f,avx512vl,avx512vnni"))) static void tile4x16_avx512vnni(
    int32_t *dst, int n, const uint8_t *const a[4], const int8_t *pb, int kg) {
  __m256i c0 = _mm256_setzero_si256(), c1 = c0, c2 = c0, c3 = c0, c4 = c0, c5 = c0,
          c6 = c0, c7 = c0;
  for (int g = 0; g < kg; g++) {
    __m256i b0 = _mm256_loadu_si256((const __m256i *)(pb + (size_t)g * 64));
    __m256i b1 = _mm256_loadu_si256((const __m256i *)(pb + (size_t)g * 64 + 32));
    int32_t w0, w1, w2, w3;
    memcpy(&w0, a[0] + 4 * g, 4);
    memcpy(&w1, a[1] + 4 * g, 4);
    memcpy(&w2, a[2] + 4 * g, 4);
    memcpy(&w3, a[3] + 4 * g, 4);
    __m256i r0 = _mm256_set1_epi32(w0), r1 = _mm256_set1_epi32(w1),
            r2 = _mm256_set1_epi32(w2), r3 = _mm256_set1_epi32(w3);
    c0 = _mm256_dpbusd_epi32(c0, r0, b0);
    c1 = _mm256_dpbusd_epi32(c1, r0, b1);
    c2 = _mm256_dpbusd_epi32(c2, r1, b0);
    c3 = _mm256_dpbusd_epi32(c3, r1, b1);
    c4 = _mm256_dpbusd_epi32(c4, r2, b0);
    c5 = _mm256_dpbusd_epi32(c5, r2, b1);
    c6 = _mm256_dpbusd_epi32(c6, r3, b0);
    c7 = _mm256_dpbusd_epi32(c7, r3, b1);
  }
  _mm256_storeu_si256((__m256i *)(dst), c0);
  _mm256_storeu_si256((__m256i *)(dst + 8), c1);
  _mm256_storeu_si256((__m256i *)(dst + n), c2);
  _mm256_storeu_si256((__m256i *)(dst + n + 8), c3);
  _mm256_storeu_si256((__m256i *)(dst + 2 * n), c4);
  _mm256_storeu_si256((__m256i *)(dst + 2 * n + 8), c5);
  _mm256_storeu_si256((__m256i *)(dst + 3 * n), c6);
  _mm256_storeu_si256((__m256i *)(dst + 3 * n + 8), c7);
}
#endif

/* The same tile with scalar integer arithmetic (no VNNI on the host). */
static void tile4x16_portable(int32_t *dst, int n, const uint8_t *const a[4],
                              const int8_t *pb, int kg) {
  uint32_t c[4][16] = {{0}};
  for (int g = 0; g < kg; g++)
    for (int r = 0; r < 4; r++)
      for (int col = 0; col < 16; col++)
        for (int e = 0; e < 4; e++)
          c[r][col] += (uint32_t)((int32_t)a[r][4 * g + e] *
                                  (int32_t)pb[(size_t)g * 64 + col * 4 + e]);
  for (int r = 0; r < 4; r++)
    for (int col = 0; col < 16; col++) dst[(size_t)r * n + col] = (int32_t)c[r][col];
}

static int panel_kind_cached = -1;

int or_vnni_panel_kind(void) {
  if (panel_kind_cached < 0) {
    int kind = 0;
#if defined(__x86_64__)
    __builtin_cpu_init();
    if (getenv("OR_FORCE_PORTABLE") == 0) {
      /* the reference prefers the VEX form where it exists (pack_vnni.go:152-156) */
      if (__builtin_cpu_supports("avxvnni")) kind = 1;
      else if (__builtin_cpu_supports("avx512vnni") && __builtin_cpu_supports("avx512vl"))
        kind = 2;
    }
#endif
    panel_kind_cached = kind;
  }
  return panel_kind_cached;
}

/* MatMulPackedVNNI's unit loop (pack_vnni.go:142-151): one unit per 4-row x
 * 16-column tile over the row panels of qa (rows of lda >= kg*4 bytes, zero
 * past k) and the panels of pb; a partial last row panel reads zero rows, as
 * the reference's PackAPad rows are. acc[m][n] is the u8 x s8 sum. */
void or_gemm_u8s8_panels(int32_t *acc, const uint8_t *qa, int lda, const int8_t *pb, int m,
                         int k, int n) {
  int kg = (k + 3) / 4;
  int kind = or_vnni_panel_kind();
  uint8_t *zero = (uint8_t *)calloc((size_t)kg * 4, 1);
  int32_t tile[4 * 16];
  for (int rp = 0; rp < (m + 3) / 4; rp++) {
    const uint8_t *a[4];
    for (int r = 0; r < 4; r++) a[r] = rp * 4 + r < m ? qa + (size_t)(rp * 4 + r) * lda : zero;
    for (int cp = 0; cp < n / 16; cp++) {
      const int8_t *panel = pb + (size_t)cp * kg * 64;
#if defined(__x86_64__)
      if (kind == 1) tile4x16_avxvnni(tile, 16, a, panel, kg);
      else if (kind == 2) tile4x16_avx512vnni(tile, 16, a, panel, kg);
      else
#endif
        tile4x16_portable(tile, 16, a, panel, kg);
      for (int r = 0; r < 4 && rp * 4 + r < m; r++)
        memcpy(acc + (size_t)(rp * 4 + r) * n + (size_t)cp * 16, tile + r * 16, 64);
    }
  }
  free(zero);
}

static int gemm_impl = 0; /* 0: row-major dot products, 1: the reference's panels */

void or_set_gemm_impl(int impl) { gemm_impl = impl; }

static int vnni_kind_cached = -1;

int or_vnni_kind(void) {
  if (vnni_kind_cached < 0) {
    int kind = 0;
#if defined(__x86_64__)
    __builtin_cpu_init();
    if (__builtin_cpu_supports("avx512vnni") &&
        __builtin_cpu_supports("avx512bw") && getenv("OR_FORCE_PORTABLE") == 0)
      kind = 2;
#endif
    vnni_kind_cached = kind;
  }
  return vnni_kind_cached;
}

void or_gemm_u8s8_i32(int32_t *acc, const uint8_t *qa, int lda,
                      const int8_t *q, int m, int k, int n) {
#if defined(__x86_64__)
  if (or_vnni_kind() == 2) {
    gemm_u8s8_vnni512(acc, qa, lda, q, m, k, n);
    return;
  }
#endif
  gemm_u8s8_portable(acc, qa, lda, q, m, k, n);
}

/* MatMulPackedVNNI, internal/tensor/pack_vnni.go:124-176: quantize each row
 * (QuantizeRowU8), accumulate u8 x s8, then real = acc - 128*colSum (int32,
 * wrapping) and dst = float32(real) * rowScale * colScale, left to right. */
void or_matmul_vnni(float *dst, const float *a, const int8_t *q,
                    const int32_t *colsum, const float *scales, int m, int k,
                    int n, uint8_t *qa_out, float *rs_out, int32_t *acc_out) {
  uint8_t *qa = qa_out ? qa_out : (uint8_t *)malloc((size_t)m * k);
  float *rs = rs_out ? rs_out : (float *)malloc(sizeof(float) * (size_t)m);
  int32_t *acc = acc_out ? acc_out
                         : (int32_t *)malloc(sizeof(int32_t) * (size_t)m * n);
  for (int i = 0; i < m; i++)
    rs[i] = or_quantize_row_u8(qa + (size_t)i * k, k, a + (size_t)i * k, k);
  or_gemm_u8s8_i32(acc, qa, k, q, m, k, n);
  for (int i = 0; i < m; i++) {
    float r = rs[i];
    for (int j = 0; j < n; j++) {
      int32_t real =
          (int32_t)((uint32_t)acc[(size_t)i * n + j] - 128u * (uint32_t)colsum[j]);
      float t = (float)real * r;
      dst[(size_t)i * n + j] = t * scales[j];
    }
  }
  if (!qa_out) free(qa);
  if (!rs_out) free(rs);
  if (!acc_out) free(acc);
}

/* ------------------------------------------------------------------------ */
/* elementwise                                                               */
/* ------------------------------------------------------------------------ */

/* fastmath.go:17-21 */
#define EXP_LOG2E 1.44269504088896341f
#define EXP_C1 0.693359375f
#define EXP_C2 -2.12194440e-4f

static float pow2i(int32_t nexp) {
  uint32_t bits = (uint32_t)(nexp + 127) << 23;
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

/* Cephes polynomial body shared by expf32/expNonPos (fastmath.go:38-45). */
static float exp_poly(float x) {
  float z = x * x;
  float y = 1.9875691500e-4f;
  y = y * x + 1.3981999507e-3f;
  y = y * x + 8.3334519073e-3f;
  y = y * x + 4.1665795894e-2f;
  y = y * x + 1.6666665459e-1f;
  y = y * x + 5.0000001201e-1f;
  return y * z + x + 1.0f;
}

/* expf32, fastmath.go:26-55 */
float or_expf32(float x) {
  if (x > 88.72f) return INFINITY;
  if (x < -87.33f) return 0.0f;
  float half = x < 0 ? -0.5f : 0.5f;
  float nf = (float)(int32_t)(x * EXP_LOG2E + half);
  x -= nf * EXP_C1;
  x -= nf * EXP_C2;
  float y = exp_poly(x);
  int32_t n = (int32_t)nf;
  if (n >= 128) return y * pow2i(127) * 2.0f;
  return y * pow2i(n);
}

/* expNonPos, fastmath.go:93-109 (the form Softmax and GELU inline). */
float or__exp_nonpos(float x) {
  if (x < -87.33f) x = -87.33f;
  float nf = (float)(int32_t)(x * EXP_LOG2E - 0.5f);
  x -= nf * EXP_C1;
  x -= nf * EXP_C2;
  return exp_poly(x) * pow2i((int32_t)nf);
}

/* erff32, fastmath.go:69-82 (A&S 7.1.26) */
float or_erff32(float x) {
  int neg = x < 0;
  if (neg) x = -x;
  float t = 1.0f / (1.0f + 0.3275911f * x);
  float poly =
      t * (0.254829592f +
           t * (-0.284496736f +
                t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
  float r = 1.0f - poly * or_expf32(-x * x);
  return neg ? -r : r;
}

/* AddBias, tensor.go:373-380 */
void or_add_bias(float *x, const float *bias, int m, int n) {
  for (int i = 0; i < m; i++)
    for (int j = 0; j < n; j++) x[(size_t)i * n + j] += bias[j];
}

/* Add, tensor.go:383-387 */
void or_add(float *dst, const float *src, int n) {
  for (int i = 0; i < n; i++) dst[i] += src[i];
}

/* Softmax, tensor.go:391-428 */
void or_softmax(float *x, int m, int n) {
  for (int i = 0; i < m; i++) {
    float *row = x + (size_t)i * n;
    float maxv = row[0];
    for (int j = 1; j < n; j++)
      if (row[j] > maxv) maxv = row[j];
    float sum = 0.0f;
    for (int j = 0; j < n; j++) {
      float e = or__exp_nonpos(row[j] - maxv);
      row[j] = e;
      sum += e;
    }
    float inv = 1.0f / sum;
    for (int j = 0; j < n; j++) row[j] *= inv;
  }
}

/* LayerNorm, tensor.go:433-452 (biased variance, float32 sums in order) */
void or_layernorm(float *x, const float *g, const float *b, int m, int n,
                  float eps) {
  for (int i = 0; i < m; i++) {
    float *row = x + (size_t)i * n;
    float mean = 0.0f;
    for (int j = 0; j < n; j++) mean += row[j];
    mean /= (float)n;
    float var = 0.0f;
    for (int j = 0; j < n; j++) {
      float d = row[j] - mean;
      var += d * d;
    }
    var /= (float)n;
    float inv = 1.0f / (float)sqrt((double)(var + eps));
    for (int j = 0; j < n; j++) row[j] = (row[j] - mean) * inv * g[j] + b[j];
  }
}

/* RMSNorm, tensor.go:459-471 */
void or_rmsnorm(float *x, const float *g, int m, int n, float eps) {
  for (int i = 0; i < m; i++) {
    float *row = x + (size_t)i * n;
    float ss = 0.0f;
    for (int j = 0; j < n; j++) ss += row[j] * row[j];
    float inv = 1.0f / (float)sqrt((double)(ss / (float)n + eps));
    for (int j = 0; j < n; j++) row[j] = row[j] * inv * g[j];
  }
}

/* geluScalar, tensor.go:508-538 */
void or_gelu(float *x, int n) {
  const float invSqrt2 = 0.7071067811865476f;
  for (int i = 0; i < n; i++) {
    float v = x[i];
    float a = v * invSqrt2;
    float sign = 1.0f;
    if (a < 0) {
      sign = -1.0f;
      a = -a;
    }
    float t = 1.0f / (1.0f + 0.3275911f * a);
    float poly =
        t * (0.254829592f +
             t * (-0.284496736f +
                  t * (1.421413741f + t * (-1.453152027f + t * 1.061405429f))));
    float e = or__exp_nonpos(-a * a);
    float erf = sign * (1.0f - poly * e);
    x[i] = 0.5f * v * (1.0f + erf);
  }
}

/* geluAVX2's per-lane sequence (internal/tensor/gelu_amd64.s:37-123): the
 * same constants as geluScalar with FMAs where the assembly fuses (erf
 * denominator, both Horner chains, the exponent rounding, the two-part ln2
 * reduction, y*z+xe and 1-poly*e) and an exact division for t. */
float or_gelu_avx2_lane(float v) {
  float a = v * 0.7071067811865476f;
  float aa = fabsf(a);
  float t = 1.0f / fmaf(0.3275911f, aa, 1.0f);
  float h = 1.061405429f;
  h = fmaf(h, t, -1.453152027f);
  h = fmaf(h, t, 1.421413741f);
  h = fmaf(h, t, -0.284496736f);
  h = fmaf(h, t, 0.254829592f);
  float poly = h * t;
  float xe = -(aa * aa);
  if (xe < -87.33f) xe = -87.33f;
  int32_t nfi = (int32_t)fmaf(EXP_LOG2E, xe, -0.5f);
  float nf = (float)nfi;
  xe = fmaf(-(EXP_C1), nf, xe);
  xe = fmaf(-(EXP_C2), nf, xe);
  float z = xe * xe;
  float y = 1.9875691500e-4f;
  y = fmaf(y, xe, 1.3981999507e-3f);
  y = fmaf(y, xe, 8.3334519073e-3f);
  y = fmaf(y, xe, 4.1665795894e-2f);
  y = fmaf(y, xe, 1.6666665459e-1f);
  y = fmaf(y, xe, 5.0000001201e-1f);
  y = fmaf(y, z, xe);
  y = y + 1.0f;
  float e = y * pow2i(nfi);
  float val = fmaf(-poly, e, 1.0f);
  float erf = a < 0 ? -val : val; /* sign bit of a xor-ed in */
  if (a == 0 && signbit(a)) erf = -val;
  return (v * 0.5f) * (1.0f + erf);
}

/* GELU as the reference runs it on amd64 (internal/tensor/gelu_amd64.go:
 * 16-26): the AVX2 body over the first n&~7 elements, geluScalar for the
 * tail. */
void or_gelu_ref(float *x, int n) {
  int m = n & ~7;
  for (int i = 0; i < m; i++) x[i] = or_gelu_avx2_lane(x[i]);
  if (m < n) or_gelu(x + m, n - m);
}

/* GELUTanh, tensor.go:490-497 (float64 inside) */
void or_gelu_tanh(float *x, int n) {
  const double c = 0.7978845608028654;
  for (int i = 0; i < n; i++) {
    double v = (double)x[i];
    double inner = c * (v + 0.044715 * v * v * v);
    x[i] = (float)(0.5 * v * (1.0 + tanh(inner)));
  }
}

/* SiLU, tensor.go:477-481 */
void or_silu(float *x, int n) {
  for (int i = 0; i < n; i++) {
    float v = x[i];
    x[i] = v / (float)(1.0 + exp(-(double)v));
  }
}

/* L2Normalize, tensor.go:542-554 */
void or_l2normalize(float *x, int n) {
  double sum = 0.0;
  for (int i = 0; i < n; i++) sum += (double)x[i] * (double)x[i];
  if (sum == 0.0) return;
  float inv = (float)(1.0 / sqrt(sum));
  for (int i = 0; i < n; i++) x[i] *= inv;
}

/* dot4, internal/tensor/dot_amd64.s:13-94 */
void or_dot4(float *dst, const float *a, const float *b0, const float *b1,
             const float *b2, const float *b3, int k) {
  const float *bs[4] = {b0, b1, b2, b3};
  float acc[4][8];
  memset(acc, 0, sizeof(acc));
  int nb = k / 8;
  for (int blk = 0; blk < nb; blk++)
    for (int qi = 0; qi < 4; qi++)
      for (int l = 0; l < 8; l++)
        acc[qi][l] = fmaf(a[blk * 8 + l], bs[qi][blk * 8 + l], acc[qi][l]);
  for (int qi = 0; qi < 4; qi++) {
    float x[4];
    for (int l = 0; l < 4; l++) x[l] = acc[qi][l] + acc[qi][l + 4];
    for (int p = nb * 8; p < k; p++) x[0] = fmaf(a[p], bs[qi][p], x[0]);
    float h0 = x[0] + x[1], h1 = x[2] + x[3];
    dst[qi] = h0 + h1;
  }
}

/* MatMulSerial -> matMulSIMDCols, tensor.go:284-330: dot4 over column
 * quads, scalar in-order sums for the remainder columns. */
void or_matmul_serial(float *dst, const float *a, const float *bT, int m,
                      int k, int n) {
  int j;
  for (j = 0; j + 4 <= n; j += 4) {
    const float *b0 = bT + (size_t)(j + 0) * k, *b1 = bT + (size_t)(j + 1) * k;
    const float *b2 = bT + (size_t)(j + 2) * k, *b3 = bT + (size_t)(j + 3) * k;
    for (int i = 0; i < m; i++)
      or_dot4(dst + (size_t)i * n + j, a + (size_t)i * k, b0, b1, b2, b3, k);
  }
  for (; j < n; j++) {
    const float *br = bT + (size_t)j * k;
    for (int i = 0; i < m; i++) {
      const float *ar = a + (size_t)i * k;
      float s = 0.0f;
      for (int p = 0; p < k; p++) s += ar[p] * br[p];
      dst[(size_t)i * n + j] = s;
    }
  }
}

/* ------------------------------------------------------------------------ */
/* BERT-family encoder                                                       */
/* ------------------------------------------------------------------------ */

/* denseWeight, internal/model/bert.go:32-39: exactly one of the three
 * layouts is populated (newDense's fallback chain, bert.go:263-278). */

typedef struct {
  or_dense qkv, attn_out, ffn1, ffn2;
  const float *ln1_g, *ln1_b, *ln2_g, *ln2_b;
} or_layer;

struct or_bert_model {
  or_bert_config cfg;
  int quant;
  const float *word_emb, *pos_emb, *type_emb, *emb_ln_g, *emb_ln_b;
  const float *rel_bias; /* MPNet [rel_buckets][heads], or NULL */
  or_layer *layers;
};

/* relPosBucket, bert.go:123-150: n = -rel; the sign picks the table half;
 * |n| < maxExact keeps its own bucket, larger distances share buckets
 * spaced by log(|n| / maxExact) / log(128 / maxExact) (float64), clamped
 * to the half's last bucket. */
int or_rel_pos_bucket(int rel, int num_buckets) {
  int n = -rel;
  int half = num_buckets / 2;
  int ret = 0;
  if (n < 0) {
    ret = half;
    n = -n;
  }
  int max_exact = half / 2;
  if (n < max_exact) return ret + n;
  int v = max_exact + (int)(log((double)n / (double)max_exact) /
                            log(128.0 / (double)max_exact) * (double)(half - max_exact));
  return ret + (v < half - 1 ? v : half - 1);
}

void or_bert_set_rel_bias(or_bert_model *m, const float *table) { m->rel_bias = table; }

void or__dense_init(or_dense *d, const float *raw, int owned_raw,
                       const float *bias, int owned_bias, int in, int out,
                       int quant) {
  memset(d, 0, sizeof(*d));
  d->in = in;
  d->out = out;
  if (owned_bias) d->bias = (float *)bias;
  d->bias_ref = bias;
  if (quant == OR_QUANT_FULL) {
    d->q = (int8_t *)malloc((size_t)in * out);
    d->scales = (float *)malloc(sizeof(float) * out);
    d->colsum = (int32_t *)malloc(sizeof(int32_t) * out);
    if (or_pack_b8_vnni(raw, in, out, d->q, d->colsum, d->scales) == OR_OK) {
      d->kind = 2;
      d->panels = (int8_t *)malloc((size_t)(out / 16) * ((in + 3) / 4) * 64);
      or_pack_vnni_panels(d->q, in, out, d->panels);
      if (owned_raw) free((void *)raw);
      return;
    }
    free(d->q);
    free(d->scales);
    free(d->colsum);
    d->q = NULL;
    d->scales = NULL;
    d->colsum = NULL;
  }
  if (quant >= OR_QUANT_WEIGHTS) {
    d->q = (int8_t *)malloc((size_t)in * out);
    d->scales = (float *)malloc(sizeof(float) * out);
    if (or_pack_b8(raw, in, out, d->q, d->scales) == OR_OK) {
      d->kind = 1;
      if (owned_raw) free((void *)raw);
      return;
    }
    free(d->q);
    free(d->scales);
    d->q = NULL;
    d->scales = NULL;
  }
  d->kind = 0;
  d->raw = raw;
  if (owned_raw) d->rawcopy = (float *)raw;
}

void or__dense_free(or_dense *d) {
  free(d->q);
  free(d->scales);
  free(d->colsum);
  free(d->rawcopy);
  free(d->bias);
  free(d->panels);
}

/* MatMulPackedVNNI as the reference runs it (pack_vnni.go:124-176): rows
 * quantized into kg*4-byte rows (QuantizeRowU8 zeroes the tail), the 4x16
 * panel kernel, then the same dequantization as or_matmul_vnni. */
static void matmul_vnni_panels(const or_dense *d, float *dst, const float *x, int seq) {
  if (seq <= 0) return;
  int k = d->in, n = d->out, lda = ((k + 3) / 4) * 4;
  uint8_t *qa = (uint8_t *)malloc((size_t)seq * lda + 4);
  float *rs = (float *)malloc(sizeof(float) * (size_t)seq + 4);
  int32_t *acc = (int32_t *)malloc(sizeof(int32_t) * (size_t)seq * n + 4);
  for (int i = 0; i < seq; i++)
    rs[i] = or_quantize_row_u8(qa + (size_t)i * lda, lda, x + (size_t)i * k, k);
  or_gemm_u8s8_panels(acc, qa, lda, d->panels, seq, k, n);
  for (int i = 0; i < seq; i++) {
    float r = rs[i];
    for (int j = 0; j < n; j++) {
      int32_t real =
          (int32_t)((uint32_t)acc[(size_t)i * n + j] - 128u * (uint32_t)d->colsum[j]);
      float t = (float)real * r;
      dst[(size_t)i * n + j] = t * d->scales[j];
    }
  }
  free(qa);
  free(rs);
  free(acc);
}

/* applyDense, bert.go:282-301: GEMM by the mode the weight took, then a
 * separate AddBias pass. */
void or__dense_apply(const or_dense *d, float *dst, const float *x,
                        int seq) {
  if (d->kind == 2 && gemm_impl == 1 && d->panels)
    matmul_vnni_panels(d, dst, x, seq);
  else if (d->kind == 2)
    or_matmul_vnni(dst, x, d->q, d->colsum, d->scales, seq, d->in, d->out,
                   NULL, NULL, NULL);
  else if (d->kind == 1)
    or_matmul_w8(dst, x, d->q, d->scales, seq, d->in, d->out);
  else
    or_matmul_f32(dst, x, d->raw, seq, d->in, d->out);
  if (d->bias_ref) or_add_bias(dst, d->bias_ref, seq, d->out);
}

or_bert_model *or_bert_create(const or_bert_config *cfg, int quant,
                              const float *word_emb, const float *pos_emb,
                              const float *type_emb, const float *emb_ln_g,
                              const float *emb_ln_b,
                              const float *const *lt) {
  int H = cfg->hidden, I = cfg->inter;
  if (cfg->heads <= 0 || H % cfg->heads != 0) return NULL;
  or_bert_model *m = (or_bert_model *)calloc(1, sizeof(*m));
  m->cfg = *cfg;
  m->quant = quant;
  m->word_emb = word_emb;
  m->pos_emb = pos_emb;
  m->type_emb = type_emb;
  m->emb_ln_g = emb_ln_g;
  m->emb_ln_b = emb_ln_b;
  m->layers = (or_layer *)calloc((size_t)cfg->layers, sizeof(or_layer));
  for (int l = 0; l < cfg->layers; l++) {
    const float *const *t = lt + (size_t)l * OR_BERT_TENSORS_PER_LAYER;
    or_layer *L = &m->layers[l];
    /* Fuse Q|K|V into [3H][H] (bert.go:479-485). */
    float *qkvw = (float *)malloc(sizeof(float) * 3 * (size_t)H * H);
    float *qkvb = (float *)malloc(sizeof(float) * 3 * (size_t)H);
    memcpy(qkvw, t[0], sizeof(float) * (size_t)H * H);
    memcpy(qkvw + (size_t)H * H, t[2], sizeof(float) * (size_t)H * H);
    memcpy(qkvw + 2 * (size_t)H * H, t[4], sizeof(float) * (size_t)H * H);
    memcpy(qkvb, t[1], sizeof(float) * H);
    memcpy(qkvb + H, t[3], sizeof(float) * H);
    memcpy(qkvb + 2 * H, t[5], sizeof(float) * H);
    or__dense_init(&L->qkv, qkvw, 1, qkvb, 1, H, 3 * H, quant);
    or__dense_init(&L->attn_out, t[6], 0, t[7], 0, H, H, quant);
    L->ln1_g = t[8];
    L->ln1_b = t[9];
    or__dense_init(&L->ffn1, t[10], 0, t[11], 0, H, I, quant);
    or__dense_init(&L->ffn2, t[12], 0, t[13], 0, I, H, quant);
    L->ln2_g = t[14];
    L->ln2_b = t[15];
  }
  return m;
}

void or_bert_free(or_bert_model *m) {
  if (!m) return;
  for (int l = 0; l < m->cfg.layers; l++) {
    or__dense_free(&m->layers[l].qkv);
    or__dense_free(&m->layers[l].attn_out);
    or__dense_free(&m->layers[l].ffn1);
    or__dense_free(&m->layers[l].ffn2);
  }
  free(m->layers);
  free(m);
}

/* encodeWorkers, bert.go:740-923 (BERT branch; no MPNet relative bias). */
int or_bert_encode(const or_bert_model *m, const int32_t *ids, int seq,
                   float *x) {
  return or_bert_encode_layers(m, ids, seq, x, m->cfg.layers);
}

/* The same forward stopped after the first `layers` layers (the hidden
 * states that enter layer `layers`). */
int or_bert_encode_layers(const or_bert_model *m, const int32_t *ids, int seq,
                          float *x, int layers) {
  const or_bert_config *c = &m->cfg;
  if (layers < 0 || layers > c->layers) return OR_ERR_SEQ;
  int H = c->hidden, I = c->inter, heads = c->heads, dh = H / heads;
  if (seq <= 0) return OR_ERR_SEQ;
  if (seq > c->max_pos - c->pos_off) return OR_ERR_SEQ;
  for (int i = 0; i < seq; i++)
    if (ids[i] < 0 || ids[i] >= c->vocab) return OR_ERR_VOCAB;

  float *qkv = (float *)malloc(sizeof(float) * (size_t)seq * 3 * H);
  float *ctx = (float *)malloc(sizeof(float) * (size_t)seq * H);
  float *att = (float *)malloc(sizeof(float) * (size_t)seq * H);
  float *hid = (float *)malloc(sizeof(float) * (size_t)seq * I);
  float *sc = (float *)malloc(sizeof(float) * (size_t)seq * seq);
  float *qh = (float *)malloc(sizeof(float) * (size_t)seq * dh);
  float *kh = (float *)malloc(sizeof(float) * (size_t)seq * dh);
  float *vt = (float *)malloc(sizeof(float) * (size_t)seq * dh);
  float *ch = (float *)malloc(sizeof(float) * (size_t)seq * dh);

  /* Embeddings word + position + segment 0, then LayerNorm
   * (bert.go:796-814). */
  for (int i = 0; i < seq; i++) {
    const float *w = m->word_emb + (size_t)ids[i] * H;
    const float *p = m->pos_emb + (size_t)(i + c->pos_off) * H;
    float *row = x + (size_t)i * H;
    if (m->type_emb) {
      for (int j = 0; j < H; j++) row[j] = w[j] + p[j] + m->type_emb[j];
    } else {
      for (int j = 0; j < H; j++) row[j] = w[j] + p[j];
    }
  }
  or_layernorm(x, m->emb_ln_g, m->emb_ln_b, seq, H, c->eps);

  float scale = (float)(1.0 / sqrt((double)dh));
  for (int li = 0; li < layers; li++) {
    const or_layer *L = &m->layers[li];
    or__dense_apply(&L->qkv, qkv, x, seq);
    /* Per-head attention, bert.go:853-902. */
    for (int h = 0; h < heads; h++) {
      int off = h * dh;
      for (int i = 0; i < seq; i++) {
        const float *row = qkv + (size_t)i * 3 * H;
        memcpy(qh + (size_t)i * dh, row + off, sizeof(float) * dh);
        memcpy(kh + (size_t)i * dh, row + H + off, sizeof(float) * dh);
        for (int d = 0; d < dh; d++) vt[(size_t)d * seq + i] = row[2 * H + off + d];
      }
      or_matmul_serial(sc, qh, kh, seq, dh, seq);
      if (m->rel_bias) {
        /* MPNet (bert.go:876-890): scores*scale rounded, then + the bias of
         * bucket(j - i) */
        for (int i = 0; i < seq; i++)
          for (int j = 0; j < seq; j++) {
            const float s = sc[(size_t)i * seq + j] * scale;
            sc[(size_t)i * seq + j] =
                s + m->rel_bias[(size_t)or_rel_pos_bucket(j - i, c->rel_buckets) * heads + h];
          }
      } else {
        for (size_t i = 0; i < (size_t)seq * seq; i++) sc[i] *= scale;
      }
      or_softmax(sc, seq, seq);
      or_matmul_serial(ch, sc, vt, seq, seq, dh);
      for (int i = 0; i < seq; i++)
        memcpy(ctx + (size_t)i * H + off, ch + (size_t)i * dh, sizeof(float) * dh);
    }
    or__dense_apply(&L->attn_out, att, ctx, seq);
    or_add(x, att, seq * H);
    or_layernorm(x, L->ln1_g, L->ln1_b, seq, H, c->eps);
    or__dense_apply(&L->ffn1, hid, x, seq);
    for (int i = 0; i < seq; i++) or_gelu_ref(hid + (size_t)i * I, I);
    or__dense_apply(&L->ffn2, att, hid, seq);
    or_add(x, att, seq * H);
    or_layernorm(x, L->ln2_g, L->ln2_b, seq, H, c->eps);
  }
  free(qkv);
  free(ctx);
  free(att);
  free(hid);
  free(sc);
  free(qh);
  free(kh);
  free(vt);
  free(ch);
  return OR_OK;
}

/* Forward + poolMean, bert.go:649-703 */
int or_bert_forward(const or_bert_model *m, const int32_t *ids, int seq,
                    float *out) {
  int H = m->cfg.hidden;
  float *x = (float *)malloc(sizeof(float) * (size_t)(seq > 0 ? seq : 1) * H);
  int st = or_bert_encode(m, ids, seq, x);
  if (st != OR_OK) {
    free(x);
    return st;
  }
  if (m->cfg.pooling == OR_POOL_CLS) {
    memcpy(out, x, sizeof(float) * H);
  } else if (m->cfg.pooling == OR_POOL_LAST) {
    memcpy(out, x + (size_t)(seq - 1) * H, sizeof(float) * H);
  } else {
    for (int j = 0; j < H; j++) out[j] = 0.0f;
    for (int i = 0; i < seq; i++)
      for (int j = 0; j < H; j++) out[j] += x[(size_t)i * H + j];
    float inv = 1.0f / (float)seq;
    for (int j = 0; j < H; j++) out[j] *= inv;
  }
  if (m->cfg.normalize) or_l2normalize(out, H);
  free(x);
  return OR_OK;
}

/* Embed's batch path, rembed.go:309-330: texts fan out across threads, one
 * serial forward each. */
int or_bert_embed_batch(const or_bert_model *m, const int32_t *ids,
                        const int32_t *lens, int batch, int stride,
                        float *out, int threads) {
  return or_bert_embed_batch_timed(m, ids, lens, batch, stride, out, threads, NULL);
}

/* The same with each text's forward timed (wall seconds; secs may be NULL). */
int or_bert_embed_batch_timed(const or_bert_model *m, const int32_t *ids,
                        const int32_t *lens, int batch, int stride,
                        float *out, int threads, double *secs) {
  int H = m->cfg.hidden;
  int err = OR_OK;
  if (threads < 1) threads = 1;
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads)
  for (int b = 0; b < batch; b++) {
    double t0 = omp_get_wtime();
    int st = or_bert_forward(m, ids + (size_t)b * stride, lens[b], out + (size_t)b * H);
    if (secs) secs[b] = omp_get_wtime() - t0;
    if (st != OR_OK) {
#pragma omp critical
      if (err == OR_OK) err = st;
    }
  }
  return err;
}
