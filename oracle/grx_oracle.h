/* grx_oracle.h -- CPU oracle for the grxBLAS / grxDNN hot path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the product (libgrxrt, libgrxblas,
 * libgrxdnn, the grxcp_amd package) includes, links or calls this. It is the
 * checker that tests/, the smoke test and the CPU-baseline leg of bench.py
 * compare the gfx950 kernels against.
 *
 * Each function restates the reference's own CPU reference where one exists
 * (file:line cited per function); where the reference has none (bf16,
 * dequant, norms, attention -- grxDNN is unimplemented upstream) the function
 * follows the mathematical definition and is pinned by the closed-form,
 * invariant and independent-library checks in tests/test_oracle.py.
 *
 * Matrices are column major with a leading dimension, as in grxBLAS.
 */
#ifndef GRX_ORACLE_H
#define GRX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Threads used by the OpenMP-parallel loops (parallel over output elements
 * only, so results do not depend on the count). 0 = OpenMP default. */
void oracle_set_threads(int n);
int  oracle_get_threads(void);

/* Planted mistakes, for tests that prove the pinning checks can fail.
 * 0 = none. 1 = ignore transa; 2 = drop the last k term; 3 = flip beta's
 * sign; 4 = norms/attention: drop eps / skip the causal mask;
 * 5 = attention: off-by-one causal mask (j <= i+1). */
void oracle_set_mutation(int which);

/* LCG of the reference's tests: seed = seed*1664525 + 1013904223
 * (ref tests/libs/test_grxblas.cpp:110, test_grxblas_ex.cpp:34). */
uint32_t oracle_lcg_next(uint32_t* seed);
/* v[i] = ((int)(s >> 16) % 17 - 8) * 0.25   (ref test_grxblas.cpp:108-113) */
void oracle_fill_quarters(float* v, size_t n, uint32_t seed);
/* v[i] = ((int)((s >> 16) % 17) - 8) * 0.5, continuing *seed
 * (ref test_grxblas_ex.cpp:33-36) */
void oracle_fill_halves(float* v, size_t n, uint32_t* seed);

/* fp16 <-> fp32, RNE, normal range only: subnormal results flush to signed
 * zero, overflow goes to inf (ref tests/common/fp16.h:21-62). */
uint16_t oracle_float_to_half(float f);
float    oracle_half_to_float(uint16_t h);
/* bf16 <-> fp32, RNE, NaN kept quiet. No reference counterpart (bf16 is
 * absent upstream). */
uint16_t oracle_float_to_bf16(float f);
float    oracle_bf16_to_float(uint16_t b);
void     oracle_f32_to_bf16_array(const float* src, uint16_t* dst, size_t n);
void     oracle_bf16_to_f32_array(const uint16_t* src, float* dst, size_t n);
void     oracle_f32_to_half_array(const float* src, uint16_t* dst, size_t n);
void     oracle_half_to_f32_array(const uint16_t* src, float* dst, size_t n);

/* fp32 SGEMM, fp64 accumulate, operands unpacked first, beta == 0 never
 * reads C (ref tests/libs/test_grxblas.cpp:45-80). */
void oracle_sgemm(int ta, int tb, int m, int n, int k, float alpha,
                  const float* A, int lda, const float* B, int ldb,
                  float beta, float* C, int ldc);

/* GemmEx reference: fp32 accumulate in k order from the float values of the
 * narrow inputs, then alpha*acc (+ beta*C) in fp32
 * (ref tests/libs/test_grxblas_ex.cpp:45-63). */
void oracle_gemm_f32acc(int ta, int tb, int m, int n, int k, float alpha,
                        const float* A, int lda, const float* B, int ldb,
                        float beta, float* C, int ldc);

/* int8 GEMM, int32 accumulate, integral alpha/beta in int32 with two's
 * complement wrap (ref tests/libs/test_grxblas_ex.cpp:267-281). */
void oracle_igemm(int ta, int tb, int m, int n, int k, int32_t alpha,
                  const int8_t* A, int lda, const int8_t* B, int ldb,
                  int32_t beta, int32_t* C, int ldc);

/* Per-output-channel dequant epilogue (no reference counterpart):
 * Y[i + j*ldy] = bf16_rne(f32((float)acc[i + j*ldacc]) * scale[j]). */
void oracle_dequant(int m, int n, const int32_t* acc, int ldacc,
                    const float* scale, uint16_t* Y, int ldy);

/* Row normalisation over `hidden`, fp64 internally, rows packed with pitch
 * `ld` (>= hidden). No reference counterpart (grxDNN is unimplemented). */
void oracle_rmsnorm(int rows, int hidden, int ld, const float* x,
                    const float* gamma, double eps, float* y);
void oracle_layernorm(int rows, int hidden, int ld, const float* x,
                      const float* gamma, const float* beta, double eps,
                      float* y);

/* One attention head, naive two-pass softmax in fp64. q,k,v,o: [S, D] row
 * major (D contiguous). Query rows [row0, row1) are computed. No reference
 * counterpart (grxDNN is unimplemented). */
void oracle_attention_head(int S, int D, int causal, double scale,
                           const float* q, const float* k, const float* v,
                           float* o, int row0, int row1);

/* Softmax over the last dimension of rows with pitch `ld`, fp64 internally:
 * y = exp(x - max) / sum(exp(x - max)). GELU element-wise, fp64:
 * mode 0 x/2 (1 + erf(x / sqrt 2)), mode 1 x/2 (1 + tanh(sqrt(2/pi)(x + 0.044715 x^3))).
 * No reference counterpart (grxDNN is unimplemented; planned by
 * ref docs/designs/grxcp_roadmap.md:864-877). */
void oracle_softmax(int rows, int hidden, int ld, const float* x, float* y);
void oracle_gelu(long n, int mode, const float* x, float* y);

#ifdef __cplusplus
}
#endif

#endif /* GRX_ORACLE_H */
