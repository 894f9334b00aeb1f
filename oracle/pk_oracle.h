/*  pk_oracle.h - CPU oracle for the quantized weight-GEMM path.
 *
 *  TEST INFRASTRUCTURE ONLY.  Nothing in the product library links this
 *  file; only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 *  leg load it, and only to check results.
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

/* ---- conformer-block operations (pk_oracle_block.c) ------------------- */

/* LayerNorm of `rows` rows of length D (tensor_ops.c:150-185).  x86_rsqrt =
 * 1 restates the compiled vrsqrtss + Newton step (x86 only, for pinning);
 * 0 takes the correctly rounded 1/sqrt(var + 1e-5f). */
void  pkor_layer_norm_rows(const float *x, const float *gamma, const float *beta,
                           float *out, int rows, int D, int x86_rsqrt);
/* pk_exp_avx2 (tensor_ops.c:98-120) per element, as the build contracts it. */
float pkor_exp_poly(float x);
/* e^x evaluated in double by fixed IEEE operations, rounded once to float
 * (the GPU's expf for GLU and softmax tails). */
float pkor_expf_ieee(float x);
void  pkor_expf_ieee_rows(const float *x, float *y, size_t n);
/* pk_swish (tensor_ops.c:367-389) per element with the source's IEEE
 * division; pkor_swish_rows applies it to n elements (y may equal x). */
float pkor_swish(float v);
void  pkor_swish_rows(const float *x, float *y, size_t n);
/* In-place softmax of `rows` rows of length len (tensor_ops.c:336-357). */
void  pkor_softmax_rows(float *x, int rows, int len);
/* One NT dot product as kernel_nt_*x16_avx2 computes it (blas.c:221-249). */
float pkor_dot8(const float *a, const float *b, int K);
/* Relative-position attention from the biased QKV rows [T][ldq] (Q | K | V,
 * D = H*Dh each) and the position projection P [2T-1][ldp] to the
 * concatenated head outputs out [T][ldo] (encoder.c:300-408). */
void  pkor_attention_core(const float *qkv, int ldq, const float *P, int ldp,
                          const float *pos_bias_u, const float *pos_bias_v,
                          float *out, int ldo, int T, int H, int Dh);
/* GLU over rows of [va | vb] (2D wide) -> rows of D (encoder.c:453-461). */
void  pkor_glu_rows(const float *in, float *out, int rows, int D);
/* Depthwise conv over time, channel-major x [C][T], w [C][K]
 * (tensor_ops.c:476-548). */
void  pkor_depthwise_conv1d(const float *x, const float *w, const float *b,
                            float *out, int C, int T, int K);

/* ---- the whole encoder (pk_oracle_encoder.c) --------------------------- */

/* The conformer blocks 0..n_blocks-1 (blocks: an array of
 * pk_gpu_block_weights, include/pk_gpu.h) over x [T][1024], chunked as
 * encode_blocks_chunked (encoder.c:514-575; chunk <= 0: one sequence), into
 * out [T][1024].  pe_table [pe_rows][1024] with centre row pe_center.
 * snapshots (optional, [n_blocks][T][1024]) receives the gathered output
 * after every block.  Returns 0, or -1 on a bad argument or no memory. */
int pkor_encoder_run(const void *blocks, int n_blocks, const float *pe_table, int pe_rows,
                     int pe_center, const float *x, int T, int chunk, int overlap, float *out,
                     float *snapshots);

#ifdef __cplusplus
}
#endif
#endif /* PK_ORACLE_H */
