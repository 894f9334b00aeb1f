/*  pk_oracle_encoder.c - CPU oracle of the whole encoder: the 24 conformer
 *  blocks over a chunked input, composed of the oracle's pinned operations.
 *
 *  TEST INFRASTRUCTURE ONLY (see pk_oracle.h).  Built with -ffp-contract=off
 *  so every rounding happens as written; fused steps use fmaf().
 *
 *  What it composes (eschmidbauer/parakeet-unified-en-0.6b-c):
 *    conformer_block (encoder.c:479-491) = feed_forward, self_attention,
 *    conv_module, feed_forward, the output LayerNorm in place;
 *    feed_forward (encoder.c:179-217): LayerNorm, linear1 + bias, Swish,
 *      linear2 + bias, x = fma(out, 0.5, x);
 *    self_attention (encoder.c:296-425): LayerNorm, fused QKV + bias, the
 *      position projection of the chunk's positional slice (no bias,
 *      encoder.c:360), attention (pkor_attention_core), output projection +
 *      bias, x += out;
 *    conv_module (encoder.c:430-477): LayerNorm, pointwise 1 + bias
 *      (tensor_ops.c:579-590), GLU, depthwise + bias, Swish, pointwise 2 +
 *      bias, x += pw2;
 *    encode_blocks_chunked (encoder.c:514-575): chunks of `chunk` output
 *      frames with `overlap` frames of context each side, clipped to the
 *      input; every chunk through every block; each chunk's centre rows
 *      gathered; chunk <= 0 runs one sequence (encode_blocks,
 *      encoder.c:495-512).
 *
 *  Each weight GEMM is the reference's fma chain over k ascending
 *  (blas.c:187-218) on weights dequantised as fl(q*s) (blas.c:545-553,
 *  834-840), exactly as pkor_sgemm_* compute it; the pointwise
 *  convolutions compute out[t][c] = chain over k of W[c][k]*ln[t][k], the
 *  same products in the same order as the reference's sgemm with the weight
 *  as A.  Elementwise steps are the oracle's: LayerNorm with the correctly
 *  rounded 1/sqrt, Swish with the IEEE division, GLU with pkor_expf_ieee.
 *
 *  Rows and chunks are independent, so they are spread over OpenMP threads;
 *  no chain or sum is ever split, so the thread count does not change a bit.
 */
#include "pk_oracle.h"
#include "pk_gpu.h"          /* pk_gpu_block_weights: the parameter layout only */

#include <math.h>
#include <stdlib.h>
#include <string.h>

enum { D_MODEL = 1024, D_FF = 4096, N_HEADS = 8, HEAD_DIM = 128, CONV_K = 9 };
enum { EPI_NONE, EPI_SWISH, EPI_HALF_RESIDUAL, EPI_RESIDUAL };

typedef struct { int in0, len, out0, out_len; } chunk_t;

/* encoder.c:531-553 */
static int plan_chunks(int T, int C, int ov, chunk_t *ch)
{
    if (C <= 0) {
        ch[0] = (chunk_t){0, T, 0, T};
        return 1;
    }
    const int n = (T + C - 1) / C;
    for (int c = 0; c < n; c++) {
        const int o0 = c * C, o1 = o0 + C < T ? o0 + C : T;
        const int i0 = o0 - ov > 0 ? o0 - ov : 0, i1 = o1 + ov < T ? o1 + ov : T;
        ch[c] = (chunk_t){i0, i1 - i0, o0, o1 - o0};
    }
    return n;
}

/* The fp32 [K][N] values the reference's pack step produces for a weight. */
static float *weight_f32(const pk_gpu_weight *w, int K, int N)
{
    float *out = (float *)malloc((size_t)K * N * sizeof(float));
    if (!out) return NULL;
    if (w->bits == 32)
        memcpy(out, w->data, (size_t)K * N * sizeof(float));
    else if (w->bits == 8)
        pkor_dequant_i8_matrix((const int8_t *)w->data, K, N, N, w->scale, out);
    else
        pkor_dequant_i4_matrix((const uint8_t *)w->data, K, N, N / 2, w->scales, out);
    return out;
}

/* [rows][cols] -> [cols][rows] */
static float *transposed(const float *a, int rows, int cols)
{
    float *t = (float *)malloc((size_t)rows * cols * sizeof(float));
    if (!t) return NULL;
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++) t[(size_t)c * rows + r] = a[(size_t)r * cols + c];
    return t;
}

/* C[i][j] <- epilogue(chain over k of A[i][k] * W[k][j], bias[j]) for a
 * [M][K] x [K][N] product: the chain of every output starts at +0 and adds
 * fma(A[i][k], W[k][j], c) for k ascending; then v = c + bias[j] (if any)
 * and the epilogue: v, swish(v), fma(v, 0.5, C) or C + v.  Tiles of
 * MB x NB outputs keep their accumulators in a local array while k runs, so
 * the W strip is reused from cache by MB rows; every accumulator is still
 * its own sequential chain. */
#define MB 8
#define NB 128
static void gemm_chain(int M, int N, int K, const float *A, int lda, const float *W,
                       const float *bias, int epi, float *C, int ldc)
{
    const int mt = (M + MB - 1) / MB, nt = (N + NB - 1) / NB;
    #pragma omp parallel for schedule(dynamic, 1)
    for (int tile = 0; tile < mt * nt; tile++) {
        const int i0 = (tile % mt) * MB, j0 = (tile / mt) * NB;
        const int mb = M - i0 < MB ? M - i0 : MB, nb = N - j0 < NB ? N - j0 : NB;
        float acc[MB][NB];
        memset(acc, 0, sizeof(acc));
        for (int k = 0; k < K; k++) {
            const float *w = W + (size_t)k * N + j0;
            for (int r = 0; r < mb; r++) {
                const float a = A[(size_t)(i0 + r) * lda + k];
                float *c = acc[r];
                if (nb == NB) {
                    for (int j = 0; j < NB; j++) c[j] = fmaf(a, w[j], c[j]);
                } else {
                    for (int j = 0; j < nb; j++) c[j] = fmaf(a, w[j], c[j]);
                }
            }
        }
        for (int r = 0; r < mb; r++) {
            float *crow = C + (size_t)(i0 + r) * ldc + j0;
            for (int j = 0; j < nb; j++) {
                float v = acc[r][j];
                if (bias) v = v + bias[j0 + j];
                switch (epi) {
                case EPI_SWISH:         crow[j] = pkor_swish(v); break;
                case EPI_HALF_RESIDUAL: crow[j] = fmaf(v, 0.5f, crow[j]); break;
                case EPI_RESIDUAL:      crow[j] = crow[j] + v; break;
                default:                crow[j] = v; break;
                }
            }
        }
    }
}

/* One block's weights as fp32 [K][N] (pointwise convolutions transposed to
 * [Cin][Cout]). */
typedef struct {
    float *ff1_w1, *ff1_w2, *qkv, *pos, *out, *pw1t, *pw2t, *ff2_w1, *ff2_w2;
} block_f32;

static void free_block(block_f32 *b)
{
    free(b->ff1_w1); free(b->ff1_w2); free(b->qkv); free(b->pos); free(b->out);
    free(b->pw1t); free(b->pw2t); free(b->ff2_w1); free(b->ff2_w2);
}

static int load_block(const pk_gpu_block_weights *w, block_f32 *b)
{
    memset(b, 0, sizeof(*b));
    b->ff1_w1 = weight_f32(&w->ff1_linear1_w, D_MODEL, D_FF);
    b->ff1_w2 = weight_f32(&w->ff1_linear2_w, D_FF, D_MODEL);
    b->qkv = weight_f32(&w->linear_qkv_w, D_MODEL, 3 * D_MODEL);
    b->pos = weight_f32(&w->linear_pos_w, D_MODEL, D_MODEL);
    b->out = weight_f32(&w->linear_out_w, D_MODEL, D_MODEL);
    b->pw1t = transposed(w->conv_pw1_w, 2 * D_MODEL, D_MODEL);
    b->pw2t = transposed(w->conv_pw2_w, D_MODEL, D_MODEL);
    b->ff2_w1 = weight_f32(&w->ff2_linear1_w, D_MODEL, D_FF);
    b->ff2_w2 = weight_f32(&w->ff2_linear2_w, D_FF, D_MODEL);
    return b->ff1_w1 && b->ff1_w2 && b->qkv && b->pos && b->out && b->pw1t && b->pw2t &&
           b->ff2_w1 && b->ff2_w2;
}

/* feed_forward (encoder.c:179-217) over R rows of x, in place. */
static void feed_forward(const float *g, const float *be, const float *w1, const float *b1,
                         const float *w2, const float *b2, float *x, int R, float *ln, float *h)
{
    pkor_layer_norm_rows(x, g, be, ln, R, D_MODEL, 0);
    gemm_chain(R, D_FF, D_MODEL, ln, D_MODEL, w1, b1, EPI_SWISH, h, D_FF);
    gemm_chain(R, D_MODEL, D_FF, h, D_FF, w2, b2, EPI_HALF_RESIDUAL, x, D_MODEL);
}

/* encoder.c:567-569: each chunk's centre rows into dst [T][D]. */
static void gather(const chunk_t *ch, int n, const float *xs, float *dst)
{
    for (int c = 0, r = 0; c < n; r += ch[c].len, c++)
        memcpy(dst + (size_t)ch[c].out0 * D_MODEL,
               xs + (size_t)(r + ch[c].out0 - ch[c].in0) * D_MODEL,
               (size_t)ch[c].out_len * D_MODEL * sizeof(float));
}

int pkor_encoder_run(const void *blocks_v, int n_blocks, const float *pe_table, int pe_rows,
                     int pe_center, const float *x, int T, int chunk, int overlap, float *out,
                     float *snapshots)
{
    const pk_gpu_block_weights *blocks = (const pk_gpu_block_weights *)blocks_v;
    if (T <= 0 || n_blocks <= 0) return -1;
    const int max_chunks = chunk > 0 ? (T + chunk - 1) / chunk : 1;
    chunk_t *ch = (chunk_t *)malloc((size_t)max_chunks * sizeof(chunk_t));
    if (!ch) return -1;
    const int n = plan_chunks(T, chunk, overlap, ch);
    int R = 0, maxT = 0;
    for (int c = 0; c < n; c++) {
        R += ch[c].len;
        if (ch[c].len > maxT) maxT = ch[c].len;
    }
    if (pe_center - maxT + 1 < 0 || pe_center + maxT > pe_rows) { free(ch); return -1; }
    const size_t D = D_MODEL;
    float *xs = (float *)malloc((size_t)R * D * sizeof(float));           /* chunk rows */
    float *ln = (float *)malloc((size_t)R * D * sizeof(float));
    float *h = (float *)malloc((size_t)R * D_FF * sizeof(float));
    float *att = (float *)malloc((size_t)R * D * sizeof(float));
    float *P = (float *)malloc((size_t)(2 * maxT - 1) * D * sizeof(float));
    float *cm = (float *)malloc((size_t)maxT * D * sizeof(float));        /* channel-major */
    float *cm2 = (float *)malloc((size_t)maxT * D * sizeof(float));
    int rc = -1;
    if (!xs || !ln || !h || !att || !P || !cm || !cm2) goto done;
    for (int c = 0, r = 0; c < n; r += ch[c].len, c++)
        memcpy(xs + (size_t)r * D, x + (size_t)ch[c].in0 * D, (size_t)ch[c].len * D * sizeof(float));

    for (int bi = 0; bi < n_blocks; bi++) {
        const pk_gpu_block_weights *w = &blocks[bi];
        block_f32 b;
        if (!load_block(w, &b)) { free_block(&b); goto done; }

        feed_forward(w->norm_ff1_w, w->norm_ff1_b, b.ff1_w1, w->ff1_linear1_b, b.ff1_w2,
                     w->ff1_linear2_b, xs, R, ln, h);

        /* self_attention: QKV over all rows, attention per chunk */
        pkor_layer_norm_rows(xs, w->norm_sa_w, w->norm_sa_b, ln, R, D_MODEL, 0);
        gemm_chain(R, 3 * D_MODEL, D_MODEL, ln, D_MODEL, b.qkv, w->linear_qkv_b, EPI_NONE, h,
                   3 * D_MODEL);
        for (int c = 0, r = 0; c < n; r += ch[c].len, c++) {
            const int Tc = ch[c].len, L = 2 * Tc - 1;
            const float *pe = pe_table + (size_t)(pe_center - Tc + 1) * D;   /* encoder.c:220-228 */
            gemm_chain(L, D_MODEL, D_MODEL, pe, D_MODEL, b.pos, NULL, EPI_NONE, P, D_MODEL);
            pkor_attention_core(h + (size_t)r * 3 * D, 3 * D_MODEL, P, D_MODEL, w->pos_bias_u,
                                w->pos_bias_v, att + (size_t)r * D, D_MODEL, Tc, N_HEADS,
                                HEAD_DIM);
        }
        gemm_chain(R, D_MODEL, D_MODEL, att, D_MODEL, b.out, w->linear_out_b, EPI_RESIDUAL, xs,
                   D_MODEL);

        /* conv_module: pointwise 1, GLU over all rows; depthwise per chunk */
        pkor_layer_norm_rows(xs, w->norm_conv_w, w->norm_conv_b, ln, R, D_MODEL, 0);
        gemm_chain(R, 2 * D_MODEL, D_MODEL, ln, D_MODEL, b.pw1t, w->conv_pw1_b, EPI_NONE, h,
                   2 * D_MODEL);
        pkor_glu_rows(h, att, R, D_MODEL);
        for (int c = 0, r = 0; c < n; r += ch[c].len, c++) {
            const int Tc = ch[c].len;
            const float *g = att + (size_t)r * D;
            for (int t = 0; t < Tc; t++)
                for (size_t d = 0; d < D; d++) cm[d * Tc + t] = g[(size_t)t * D + d];
            pkor_depthwise_conv1d(cm, w->conv_dw_w, w->conv_dw_b, cm2, D_MODEL, Tc, CONV_K);
            pkor_swish_rows(cm2, cm2, (size_t)Tc * D);
            float *o = ln + (size_t)r * D;
            for (int t = 0; t < Tc; t++)
                for (size_t d = 0; d < D; d++) o[(size_t)t * D + d] = cm2[d * Tc + t];
        }
        gemm_chain(R, D_MODEL, D_MODEL, ln, D_MODEL, b.pw2t, w->conv_pw2_b, EPI_RESIDUAL, xs,
                   D_MODEL);

        feed_forward(w->norm_ff2_w, w->norm_ff2_b, b.ff2_w1, w->ff2_linear1_b, b.ff2_w2,
                     w->ff2_linear2_b, xs, R, ln, h);
        pkor_layer_norm_rows(xs, w->norm_out_w, w->norm_out_b, xs, R, D_MODEL, 0);
        free_block(&b);

        if (snapshots) gather(ch, n, xs, snapshots + (size_t)bi * T * D);
    }
    gather(ch, n, xs, out);
    rc = 0;
done:
    free(ch); free(xs); free(ln); free(h); free(att); free(P); free(cm); free(cm2);
    return rc;
}
