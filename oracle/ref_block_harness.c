/*  ref_block_harness.c - one conformer block of the reference, callable.
 *
 *  TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile into
 *  _ref/libpkref_block.so together with the reference's own objects (its
 *  weight GEMMs from blas.c's portable path, which decodes int4 correctly;
 *  attention GEMMs, tensor ops and thread pool from the x86 AVX2 build).
 *
 *  This translation unit includes the reference's encoder.c so that its
 *  static conformer_block (encoder.c:479-491) can be called on weights given
 *  in include/pk_gpu.h's pk_gpu_block_weights, the same struct the GPU
 *  encoder takes, so a test hands both sides identical bytes.
 */
#define _GNU_SOURCE
#include "encoder.c"

#include "pk_gpu.h"

static Weight to_weight(pk_gpu_weight w)
{
    Weight r;
    r.data = w.data;
    r.scale = w.scale;
    r.scales = w.scales;
    r.bits = w.bits;
    return r;
}

static void to_block(const pk_gpu_block_weights *w, ConformerBlock *b)
{
    memset(b, 0, sizeof *b);
    b->norm_ff1_w = w->norm_ff1_w;  b->norm_ff1_b = w->norm_ff1_b;
    b->ff1.linear1_w = to_weight(w->ff1_linear1_w);  b->ff1.linear1_b = w->ff1_linear1_b;
    b->ff1.linear2_w = to_weight(w->ff1_linear2_w);  b->ff1.linear2_b = w->ff1_linear2_b;
    b->norm_sa_w = w->norm_sa_w;    b->norm_sa_b = w->norm_sa_b;
    b->mha.linear_qkv_w = to_weight(w->linear_qkv_w);
    b->mha.linear_qkv_b = (float *)w->linear_qkv_b;
    b->mha.linear_pos_w = to_weight(w->linear_pos_w);
    b->mha.linear_out_w = to_weight(w->linear_out_w);
    b->mha.linear_out_b = w->linear_out_b;
    b->mha.pos_bias_u = w->pos_bias_u;
    b->mha.pos_bias_v = w->pos_bias_v;
    b->norm_conv_w = w->norm_conv_w; b->norm_conv_b = w->norm_conv_b;
    b->conv.pw1_w = w->conv_pw1_w;  b->conv.pw1_b = w->conv_pw1_b;
    b->conv.dw_w = w->conv_dw_w;    b->conv.dw_b = w->conv_dw_b;
    b->conv.pw2_w = w->conv_pw2_w;  b->conv.pw2_b = w->conv_pw2_b;
    b->norm_ff2_w = w->norm_ff2_w;  b->norm_ff2_b = w->norm_ff2_b;
    b->ff2.linear1_w = to_weight(w->ff2_linear1_w);  b->ff2.linear1_b = w->ff2_linear1_b;
    b->ff2.linear2_w = to_weight(w->ff2_linear2_w);  b->ff2.linear2_b = w->ff2_linear2_b;
    b->norm_out_w = w->norm_out_w;  b->norm_out_b = w->norm_out_b;
}

/* x [T][1024] in place through n_blocks blocks, each with the positional
 * slice pe_slice [2T-1][1024] (what encode_blocks does per block). */
int pkref_conformer_blocks(const pk_gpu_block_weights *w, int n_blocks, const float *pe_slice,
                           float *x, int T)
{
    CfmWS ws;
    ws.cap = conformer_ws_peak(T);
    ws.buf = (float *)malloc(ws.cap * sizeof(float));
    if (!ws.buf) return -1;
    for (int i = 0; i < n_blocks; i++) {
        ConformerBlock b;
        to_block(&w[i], &b);
        conformer_block(&b, pe_slice, x, T, &ws);
    }
    free(ws.buf);
    return 0;
}

/* pre_encode_and_scale (encoder.c:578-592): mel [128][n_frames] -> out
 * [T'][1024]; returns T' (or -1). */
int pkref_pre_encode(const pk_gpu_pre_encode_weights *w, const float *mel, int n_frames, float *out)
{
    PkModel *m = (PkModel *)calloc(1, sizeof *m);
    if (!m) return -1;
    PreEncodeWeights *p = &m->enc.pre_encode;
    p->conv0_w = w->conv0_w;  p->conv0_b = w->conv0_b;
    p->conv2_w = w->conv2_w;  p->conv2_b = w->conv2_b;
    p->conv3_w = w->conv3_w;  p->conv3_b = w->conv3_b;
    p->conv5_w = w->conv5_w;  p->conv5_b = w->conv5_b;
    p->conv6_w = w->conv6_w;  p->conv6_b = w->conv6_b;
    p->out_w = to_weight(w->out_w);
    p->out_b = w->out_b;
    float *x = NULL;
    int Tp = pre_encode_and_scale(m, mel, n_frames, &x);
    memcpy(out, x, (size_t)Tp * PK_D_MODEL * sizeof(float));
    free(x);
    free(m);
    return Tp;
}
