/*  pk_cblas_shim.c - libpk_gpu_cblas.so: the reference's three weight-GEMM
 *  symbols, forwarded to the MI355X library.
 *
 *  Exports cblas_sgemm, cblas_sgemm_qb and cblas_sgemm_q4b with the exact
 *  signatures of csrc/blas.h:38-69, so the reference's encoder.c and
 *  tensor_ops.c bind to them unchanged when blas.c's own three definitions
 *  are renamed out of the way (blas.c compiled with -Dcblas_sgemm=... and so
 *  on) and this library is linked.  The reference functions
 *  return void and have no error channel; a failure here prints the library
 *  message and aborts rather than computing anything on the CPU.
 *
 *  The CBLAS enums are ints on the C ABI (blas.h:11-19), so they are taken
 *  as int here: CblasRowMajor = 101, CblasNoTrans = 111.  `order` is
 *  ignored, as in blas.c:1062.
 */
#include "pk_gpu.h"
#include "pk_gpu_cblas.h"

#include <stdio.h>
#include <stdlib.h>

static void die(const char *fn, int rc)
{
    fprintf(stderr, "pk_gpu: %s failed (%d): %s\n", fn, rc, pk_gpu_last_error());
    abort();
}

void cblas_sgemm(int order, int transA, int transB, int M, int N, int K,
                 float alpha, const float *A, int lda,
                 const float *B, int ldb,
                 float beta, float *C, int ldc)
{
    (void)order;
    int rc = pk_gpu_sgemm(transA, transB, M, N, K, alpha, A, lda, B, ldb, beta, C, ldc);
    if (rc != PK_GPU_OK) die("cblas_sgemm", rc);
}

void cblas_sgemm_qb(int M, int N, int K, float alpha, const float *A, int lda,
                    const signed char *B, float B_scale, int ldb,
                    float beta, float *C, int ldc)
{
    int rc = pk_gpu_gemm_i8(M, N, K, alpha, A, lda, (const int8_t *)B, B_scale, ldb,
                            beta, C, ldc);
    if (rc != PK_GPU_OK) die("cblas_sgemm_qb", rc);
}

void cblas_sgemm_q4b(int M, int N, int K, float alpha, const float *A, int lda,
                     const unsigned char *B, const float *scales, int ldb,
                     float beta, float *C, int ldc)
{
    int rc = pk_gpu_gemm_i4(M, N, K, alpha, A, lda, (const uint8_t *)B, scales, ldb,
                            beta, C, ldc);
    if (rc != PK_GPU_OK) die("cblas_sgemm_q4b", rc);
}
