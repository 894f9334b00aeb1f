/*  pk_gpu_cblas.h - exports of libpk_gpu_cblas.so, the link-level drop-in.
 *
 *  Same names and C ABI as the reference's csrc/blas.h:38-69; each forwards
 *  to libpk_gpu.so (pk_gpu.h) and aborts with the library's message if the
 *  GPU call fails (the reference functions return void).  The CBLAS enum
 *  parameters are passed as int, which is their C ABI (blas.h:11-19):
 *  CblasRowMajor = 101, CblasNoTrans = 111, CblasTrans = 112.
 *
 *  A build that links this library in place of blas.c's three definitions
 *  keeps encoder.c / tensor_ops.c unchanged; cblas_sgemv and cblas_sgemm_st
 *  (attention and decoder, blas.h:21-52) stay in the reference's blas.c.
 */
#ifndef PK_GPU_CBLAS_H
#define PK_GPU_CBLAS_H

#ifdef __cplusplus
extern "C" {
#endif

/* blas.h:38-43 -> pk_gpu_sgemm (NoTrans/NoTrans only, as its callers use). */
void cblas_sgemm(int order, int transA, int transB, int M, int N, int K,
                 float alpha, const float *A, int lda,
                 const float *B, int ldb,
                 float beta, float *C, int ldc);

/* blas.h:54-62 -> pk_gpu_gemm_i8. */
void cblas_sgemm_qb(int M, int N, int K, float alpha, const float *A, int lda,
                    const signed char *B, float B_scale, int ldb,
                    float beta, float *C, int ldc);

/* blas.h:64-69 -> pk_gpu_gemm_i4. */
void cblas_sgemm_q4b(int M, int N, int K, float alpha, const float *A, int lda,
                     const unsigned char *B, const float *scales, int ldb,
                     float beta, float *C, int ldc);

#ifdef __cplusplus
}
#endif
#endif /* PK_GPU_CBLAS_H */
