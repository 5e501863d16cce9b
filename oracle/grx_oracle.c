/* grx_oracle.c -- CPU oracle for the grxBLAS / grxDNN hot path.
 *
 * TEST INFRASTRUCTURE ONLY: see grx_oracle.h. Compiled with gcc
 * -ffp-contract=off so that every float operation rounds exactly as written
 * (no fused multiply-add), which the bit-exact GemmEx/dequant checks rely on.
 */
#include "grx_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0;
static int g_mutation = 0;

void oracle_set_threads(int n) {
  g_threads = n;
#ifdef _OPENMP
  if (n > 0) omp_set_num_threads(n);
#endif
}

int oracle_get_threads(void) {
#ifdef _OPENMP
  return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
  return 1;
#endif
}

void oracle_set_mutation(int which) { g_mutation = which; }

/* ---- generators ---------------------------------------------------------- */

uint32_t oracle_lcg_next(uint32_t* seed) {
  *seed = *seed * 1664525u + 1013904223u;
  return *seed;
}

/* ref tests/libs/test_grxblas.cpp:108-113 */
void oracle_fill_quarters(float* v, size_t n, uint32_t seed) {
  for (size_t i = 0; i < n; ++i) {
    const uint32_t s = oracle_lcg_next(&seed);
    v[i] = (float)((int)(s >> 16) % 17 - 8) * 0.25f;
  }
}

/* ref tests/libs/test_grxblas_ex.cpp:33-36 */
void oracle_fill_halves(float* v, size_t n, uint32_t* seed) {
  for (size_t i = 0; i < n; ++i) {
    const uint32_t s = oracle_lcg_next(seed);
    v[i] = (float)((int)((s >> 16) % 17u) - 8) * 0.5f;
  }
}

/* ---- narrow float formats ------------------------------------------------ */

static uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ref tests/common/fp16.h:21-38: normal range, RNE on the 13 dropped bits,
 * exponent underflow -> signed zero, overflow -> inf, NaN stays NaN. */
uint16_t oracle_float_to_half(float f) {
  const uint32_t x = f2u(f);
  const uint32_t sign = (x >> 16) & 0x8000u;
  const uint32_t e8 = (x >> 23) & 0xffu;
  const uint32_t frac = x & 0x7fffffu;
  if (e8 == 0xffu) return (uint16_t)(sign | 0x7c00u | (frac ? 0x200u : 0u));
  const int e5 = (int)e8 - 112;               /* rebias 127 -> 15 */
  if (e5 >= 31) return (uint16_t)(sign | 0x7c00u);
  if (e5 <= 0) return (uint16_t)sign;
  uint32_t h = sign | ((uint32_t)e5 << 10) | (frac >> 13);
  const uint32_t dropped = frac & 0x1fffu;
  if (dropped > 0x1000u || (dropped == 0x1000u && (h & 1u))) h += 1u;
  return (uint16_t)h;
}

/* ref tests/common/fp16.h:40-62 (exact, subnormals included) */
float oracle_half_to_float(uint16_t h) {
  const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  const uint32_t e5 = (h >> 10) & 0x1fu;
  uint32_t frac = h & 0x3ffu;
  if (e5 == 0x1fu) return u2f(sign | 0x7f800000u | (frac << 13));
  if (e5 != 0) return u2f(sign | ((e5 + 112u) << 23) | (frac << 13));
  if (frac == 0) return u2f(sign);
  /* subnormal: value = frac * 2^-24 */
  int e = 113;
  while (!(frac & 0x400u)) { frac <<= 1; --e; }
  return u2f(sign | ((uint32_t)e << 23) | ((frac & 0x3ffu) << 13));
}

uint16_t oracle_float_to_bf16(float f) {
  const uint32_t x = f2u(f);
  if ((x & 0x7f800000u) == 0x7f800000u && (x & 0x7fffffu))
    return (uint16_t)((x >> 16) | 0x40u);     /* quiet NaN */
  const uint32_t bias = 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)((x + bias) >> 16);
}

float oracle_bf16_to_float(uint16_t b) { return u2f((uint32_t)b << 16); }

void oracle_f32_to_bf16_array(const float* src, uint16_t* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = oracle_float_to_bf16(src[i]);
}
void oracle_bf16_to_f32_array(const uint16_t* src, float* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = oracle_bf16_to_float(src[i]);
}
void oracle_f32_to_half_array(const float* src, uint16_t* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = oracle_float_to_half(src[i]);
}
void oracle_half_to_f32_array(const uint16_t* src, float* dst, size_t n) {
  for (size_t i = 0; i < n; ++i) dst[i] = oracle_half_to_float(src[i]);
}

/* ---- GEMMs --------------------------------------------------------------- */

/* Copy op(X) out of column-major storage into a dense row-major rows x cols
 * matrix. The transpose is one swap of the storage subscripts, done here and
 * only here, so the multiply below cannot share an indexing mistake with a
 * kernel (ref tests/libs/test_grxblas.cpp:36-60). */
static float* unpack_op(const float* src, int ld, int trans, int rows, int cols) {
  float* out = (float*)malloc((size_t)(rows > 0 ? rows : 1) * (size_t)(cols > 0 ? cols : 1) * sizeof(float));
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < cols; ++c) {
      const int sr = trans ? c : r;
      const int sc = trans ? r : c;
      out[(size_t)r * (size_t)cols + (size_t)c] = src[(size_t)sr + (size_t)sc * (size_t)ld];
    }
  return out;
}

/* ref tests/libs/test_grxblas.cpp:62-80 */
void oracle_sgemm(int ta, int tb, int m, int n, int k, float alpha,
                  const float* A, int lda, const float* B, int ldb,
                  float beta, float* C, int ldc) {
  if (g_mutation == 1) ta = 0;
  if (g_mutation == 3) beta = -beta;
  const int kk = (g_mutation == 2 && k > 0) ? k - 1 : k;
  float* a = unpack_op(A, lda, ta, m, k);   /* m x k */
  float* b = unpack_op(B, ldb, tb, k, n);   /* k x n */
#pragma omp parallel for schedule(static)
  for (int j = 0; j < n; ++j) {
    for (int i = 0; i < m; ++i) {
      double acc = 0.0;
      for (int l = 0; l < kk; ++l)
        acc += (double)a[(size_t)i * (size_t)k + (size_t)l] *
               (double)b[(size_t)l * (size_t)n + (size_t)j];
      const size_t ci = (size_t)i + (size_t)j * (size_t)ldc;
      C[ci] = (beta == 0.0f) ? (float)(alpha * acc)
                             : (float)(alpha * acc + (double)beta * C[ci]);
    }
  }
  free(a);
  free(b);
}

/* ref tests/libs/test_grxblas_ex.cpp:45-63 */
void oracle_gemm_f32acc(int ta, int tb, int m, int n, int k, float alpha,
                        const float* A, int lda, const float* B, int ldb,
                        float beta, float* C, int ldc) {
  if (g_mutation == 1) ta = 0;
  if (g_mutation == 3) beta = -beta;
  const int kk = (g_mutation == 2 && k > 0) ? k - 1 : k;
#pragma omp parallel for schedule(static)
  for (int j = 0; j < n; ++j) {
    for (int i = 0; i < m; ++i) {
      float acc = 0.0f;
      for (int l = 0; l < kk; ++l) {
        /* one subscript swap per operand, as in the reference */
        const float a = ta ? A[(size_t)l + (size_t)i * lda] : A[(size_t)i + (size_t)l * lda];
        const float b = tb ? B[(size_t)j + (size_t)l * ldb] : B[(size_t)l + (size_t)j * ldb];
        acc += a * b;
      }
      const size_t ci = (size_t)i + (size_t)j * (size_t)ldc;
      C[ci] = (beta == 0.0f) ? (alpha * acc) : (alpha * acc + beta * C[ci]);
    }
  }
}

/* ref tests/libs/test_grxblas_ex.cpp:267-281. Arithmetic is done in uint32 so
 * that overflow wraps exactly like the device's 32-bit integer ALU. */
void oracle_igemm(int ta, int tb, int m, int n, int k, int32_t alpha,
                  const int8_t* A, int lda, const int8_t* B, int ldb,
                  int32_t beta, int32_t* C, int ldc) {
  if (g_mutation == 1) ta = 0;
  if (g_mutation == 3) beta = -beta;
  const int kk = (g_mutation == 2 && k > 0) ? k - 1 : k;
#pragma omp parallel for schedule(static)
  for (int j = 0; j < n; ++j) {
    for (int i = 0; i < m; ++i) {
      uint32_t acc = 0;
      for (int l = 0; l < kk; ++l) {
        const int32_t av = ta ? A[(size_t)l + (size_t)i * lda] : A[(size_t)i + (size_t)l * lda];
        const int32_t bv = tb ? B[(size_t)j + (size_t)l * ldb] : B[(size_t)l + (size_t)j * ldb];
        acc += (uint32_t)(av * bv);
      }
      const size_t ci = (size_t)i + (size_t)j * (size_t)ldc;
      uint32_t r = (uint32_t)alpha * acc;
      if (beta != 0) r += (uint32_t)beta * (uint32_t)C[ci];
      C[ci] = (int32_t)r;
    }
  }
}

void oracle_dequant(int m, int n, const int32_t* acc, int ldacc,
                    const float* scale, uint16_t* Y, int ldy) {
#pragma omp parallel for schedule(static)
  for (int j = 0; j < n; ++j) {
    for (int i = 0; i < m; ++i) {
      const float s = (g_mutation == 6) ? scale[i % n] : scale[j];
      const float a = (float)acc[(size_t)i + (size_t)j * (size_t)ldacc];
      const float v = a * s;
      Y[(size_t)i + (size_t)j * (size_t)ldy] = oracle_float_to_bf16(v);
    }
  }
}

/* ---- norms --------------------------------------------------------------- */

void oracle_rmsnorm(int rows, int hidden, int ld, const float* x,
                    const float* gamma, double eps, float* y) {
  if (g_mutation == 4) eps = 0.0;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * (size_t)ld;
    float* yr = y + (size_t)r * (size_t)ld;
    double ss = 0.0;
    for (int c = 0; c < hidden; ++c) ss += (double)xr[c] * (double)xr[c];
    const double inv = 1.0 / sqrt(ss / (double)hidden + eps);
    for (int c = 0; c < hidden; ++c)
      yr[c] = (float)((double)xr[c] * inv * (double)gamma[c]);
  }
}

void oracle_layernorm(int rows, int hidden, int ld, const float* x,
                      const float* gamma, const float* beta, double eps,
                      float* y) {
  if (g_mutation == 4) eps = 0.0;
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * (size_t)ld;
    float* yr = y + (size_t)r * (size_t)ld;
    double mean = 0.0;
    for (int c = 0; c < hidden; ++c) mean += (double)xr[c];
    mean /= (double)hidden;
    double var = 0.0;
    for (int c = 0; c < hidden; ++c) {
      const double d = (double)xr[c] - mean;
      var += d * d;
    }
    var /= (double)hidden;
    const double inv = 1.0 / sqrt(var + eps);
    for (int c = 0; c < hidden; ++c)
      yr[c] = (float)(((double)xr[c] - mean) * inv * (double)gamma[c] + (double)beta[c]);
  }
}

/* ---- attention ----------------------------------------------------------- */

void oracle_attention_head(int S, int D, int causal, double scale,
                           const float* q, const float* k, const float* v,
                           float* o, int row0, int row1) {
  if (g_mutation == 4) causal = 0;
#pragma omp parallel for schedule(dynamic, 4)
  for (int i = row0; i < row1; ++i) {
    int last = causal ? i : S - 1;            /* inclusive */
    if (g_mutation == 5 && causal && i + 1 < S) last = i + 1;
    double* p = (double*)malloc((size_t)(last + 1) * sizeof(double));
    double mx = -INFINITY;
    for (int j = 0; j <= last; ++j) {
      double s = 0.0;
      for (int d = 0; d < D; ++d)
        s += (double)q[(size_t)i * D + d] * (double)k[(size_t)j * D + d];
      p[j] = s * scale;
      if (p[j] > mx) mx = p[j];
    }
    double l = 0.0;
    for (int j = 0; j <= last; ++j) { p[j] = exp(p[j] - mx); l += p[j]; }
    for (int d = 0; d < D; ++d) {
      double acc = 0.0;
      for (int j = 0; j <= last; ++j) acc += p[j] * (double)v[(size_t)j * D + d];
      o[(size_t)i * D + d] = (float)(acc / l);
    }
    free(p);
  }
}

/* ---- softmax and GELU -------------------------------------------------- */

void oracle_softmax(int rows, int hidden, int ld, const float* x, float* y) {
#pragma omp parallel for schedule(static)
  for (int r = 0; r < rows; ++r) {
    const float* xr = x + (size_t)r * (size_t)ld;
    float* yr = y + (size_t)r * (size_t)ld;
    double mx = -INFINITY;
    for (int c = 0; c < hidden; ++c)
      if ((double)xr[c] > mx) mx = (double)xr[c];
    /* mutation 7: the last element is left out of the normaliser */
    const int terms = (g_mutation == 7 && hidden > 1) ? hidden - 1 : hidden;
    double sum = 0.0;
    for (int c = 0; c < terms; ++c) sum += exp((double)xr[c] - mx);
    for (int c = 0; c < hidden; ++c) yr[c] = (float)(exp((double)xr[c] - mx) / sum);
  }
}

/* GELU in forms without cancellation in the negative tail, where 1 + erf
 * and 1 + tanh fall below double's resolution at 1 (x < -8.3, x < -6):
 * 1/2 (1 + erf(x/sqrt 2)) = 1/2 erfc(-x/sqrt 2), and
 * 1/2 (1 + tanh z) = 1 / (1 + exp(-2z)). Same values everywhere else. */
void oracle_gelu(long n, int mode, const float* x, float* y) {
  /* mutation 8: erf(x) in place of erf(x / sqrt 2) */
  const double k = (g_mutation == 8) ? 1.0 : 1.0 / sqrt(2.0);
#pragma omp parallel for schedule(static)
  for (long i = 0; i < n; ++i) {
    const double v = (double)x[i];
    double g;
    if (mode == 1) {
      const double z = sqrt(2.0 / 3.14159265358979323846) * (v + 0.044715 * v * v * v);
      g = v / (1.0 + exp(-2.0 * z));
    } else {
      g = 0.5 * v * erfc(-v * k);
    }
    y[i] = (float)g;
  }
}
