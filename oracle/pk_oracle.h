/*  pk_oracle.h - CPU oracle for the quantized weight-GEMM path.
 *
 *  TEST INFRASTRUCTURE ONLY.  Nothing in the product library links this
 *  file; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 *  leg load it, and only as the checker.
 *
 *  Each function restates one piece of the reference arithmetic
 *  (csrc/blas.c, csrc/tensor_ops.c, csrc/weights.c of
 *  eschmidbauer/parakeet-unified-en-0.6b-c) as plain scalar C with every
 *  rounding made explicit, so its results are bit-identical to the
 *  reference's AVX2 build.  How each function is pinned is listed in
 *  pk_oracle.c next to the function.
 */
#ifndef PK_ORACLE_H
#define PK_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Dequantisation, bit-exact to the reference pack step. */
float pkor_dequant_i8(int8_t q, float scale);               /* blas.c:545-555 */
int   pkor_nibble_lo(uint8_t byte);                         /* blas.c:836 */
int   pkor_nibble_hi(uint8_t byte);                         /* blas.c:837 */
/* Dequantise a whole int8 [K][N] (row stride ldb) into fp32 out[K][N]. */
void  pkor_dequant_i8_matrix(const int8_t *B, int K, int N, int ldb,
                             float scale, float *out);
/* Dequantise a packed int4 [K][N/2] matrix with scales [K][N/32] into
 * fp32 out[K][N] (blas.c:780-843; scale index blas.c:794). */
void  pkor_dequant_i4_matrix(const uint8_t *B, int K, int N, int ldb,
                             const float *scales, float *out);

/* GEMMs with the reference's exact semantics:
 *   C <- beta*C (blas.c:89-99), early exit on alpha==0 (and int8 scale==0),
 *   then for every (i, j) a sequential fmaf chain over k ascending.
 * Row-major, NoTrans/NoTrans only.  Rows are independent, so a subset of
 * rows can be checked by passing just those rows of A and C. */
void pkor_sgemm_nn(int M, int N, int K, float alpha,
                   const float *A, int lda, const float *B, int ldb,
                   float beta, float *C, int ldc);
void pkor_sgemm_qb(int M, int N, int K, float alpha,
                   const float *A, int lda, const int8_t *B, float B_scale,
                   int ldb, float beta, float *C, int ldc);
void pkor_sgemm_q4b(int M, int N, int K, float alpha,
                    const float *A, int lda, const uint8_t *B,
                    const float *scales, int ldb, float beta,
                    float *C, int ldc);

/* ---- Seeded synthetic data (identical bytes on every x86-64 host) ---- */

uint64_t pkor_splitmix64(uint64_t *state);
/* Seed for (workload, tensor name): splitmix64 of base ^ fnv1a64(name). */
uint64_t pkor_seed(uint64_t base, const char *name);
/* Normal(mean, std) as fp32, Box-Muller in double. */
void pkor_fill_normal(float *out, size_t n, float mean, float std,
                      uint64_t seed);
/* Uniform(lo, hi) as fp32. */
void pkor_fill_uniform(float *out, size_t n, float lo, float hi,
                       uint64_t seed);
/* Uniform integers in [lo, hi] (unbiased), stored as int8. */
void pkor_fill_int8(int8_t *out, size_t n, int lo, int hi, uint64_t seed);
/* Uniform bytes 0..255 (each nibble uniform 0..15). */
void pkor_fill_bytes(uint8_t *out, size_t n, uint64_t seed);

#ifdef __cplusplus
}
#endif
#endif /* PK_ORACLE_H */
