/*  pk_oracle_block.c - CPU oracle for the conformer-block operations that
 *  sit between the weight GEMMs (LayerNorm, relative-position attention,
 *  softmax, GLU, depthwise convolution).
 *
 *  TEST INFRASTRUCTURE ONLY (see pk_oracle.h).  Built with -ffp-contract=off
 *  so every rounding below happens as written; fused steps use fmaf().
 *
 *  What the reference computes (eschmidbauer/parakeet-unified-en-0.6b-c, x86
 *  AVX2 build: -O3 -ffast-math -march=x86-64-v3), and how each function here
 *  is pinned (tests/test_oracle_block.py):
 *
 *    LayerNorm, tensor_ops.c:150-185.  Eight interleaved partial sums
 *    (lane j adds x[j], x[j+8], ... in order), reduced as
 *    ((p0+p4)+(p2+p6)) + ((p1+p5)+(p3+p7)) (pk_hsum_avx2, tensor_ops.c:
 *    126-134); the variance the same way with fma(d, d, acc); mean and
 *    variance divided by len; out = fma(fl((x-mean)*inv), gamma, beta).
 *    The compiled reference evaluates inv = 1/sqrtf(var + 1e-5f) as
 *    vrsqrtss plus one Newton step, inv = fl(fma(fl(y*a), y, -3) * fl(y*-0.5)),
 *    whose 12-bit seed table is specific to the CPU model; mode 1 below
 *    restates exactly that (x86 only) and is compared bit-for-bit with the
 *    compiled pk_layer_norm; mode 0 takes the correctly rounded
 *    1/sqrt(var + 1e-5f), which is what the GPU path computes.
 *
 *    exp polynomial, tensor_ops.c:98-120 (pk_exp_avx2) as compiled: clamp
 *    to [-87, 87], k = rint(x*log2e), r = fma(-k, ln2, x) (the build fuses
 *    x - k*ln2), a 5-term Horner polynomial in fmas, times 2^k.
 *
 *    softmax, tensor_ops.c:336-357: max, e = exp(x - max) with the
 *    polynomial on the 8-wide part, the eight-lane sum reduced as above,
 *    1/sum by an IEEE division, x*inv.  Pinned bit-for-bit against the
 *    compiled pk_softmax for len % 8 == 0.  The scalar tail (len % 8 != 0)
 *    is left to the C library's expf in the reference, which the compiler
 *    may also vectorise; here it is pkor_expf_ieee (below), so tails agree
 *    with the reference only within tolerance (tested).
 *
 *    NT dot products of the attention scores (cblas_sgemm_st NT,
 *    blas.c:221-249): eight interleaved fma chains over k = l, l+8, ...,
 *    reduced as above, then the scalar tail; c = 0 + 1*s = s.  Pinned
 *    bit-for-bit against the compiled cblas_sgemm_st (NT).
 *
 *    attention core, encoder.c:300-408: Q_u = fl(q + pos_bias_u),
 *    Q_v = fl(q + pos_bias_v) (encoder.c:319-338), AC = Q_u K^T and
 *    BD = Q_v P^T per head (NT dot products above), the relative shift
 *    (encoder.c:230-254) reduces to BDs[i][j] = BD[i][T-1-i+j], scores
 *    fl(fl(AC + BDs) * 0x3db504f3) (encoder.c:375-393; the constant is
 *    1/sqrtf(128) as the compiler folds it), softmax per row, then
 *    scores x V as a sequential fma chain over j ascending (sgemm NN,
 *    blas.c:187-218), heads concatenated (encoder.c:401-406).  Pinned
 *    bit-for-bit (T % 8 == 0) against the compiled reference's exported
 *    cblas_sgemm_st (NT and NN) and pk_softmax_rows composed with the
 *    head gather, padded relative shift and score combine of
 *    encoder.c:315-406.
 *
 *    GLU, encoder.c:453-461: gated = va * (1 / (1 + expf(-vb))).  The
 *    compiled reference takes expf from glibc's vector library and 1/(1+e)
 *    from rcpps plus a Newton step (CPU-model specific), so no restatement
 *    can be bit-exact; here exp is pkor_expf_ieee and the division IEEE
 *    (GPU and oracle agree bit for bit; the reference within tolerance).
 *
 *    expf_ieee: e^x evaluated in double by a fixed sequence of IEEE
 *    operations and rounded once to float, so the GPU and this oracle agree
 *    bit for bit.  Pinned against the correctly rounded e^x (expl) over
 *    every float input.
 *
 *    Swish, tensor_ops.c:367-389: e = pk_exp_avx2(-v) as compiled (the
 *    build also contracts 1 + poly*2^k into one fma), s = 1/(1+e) by the
 *    IEEE division the source writes (_mm256_div_ps; the -ffast-math build
 *    turns it into rcpps plus a Newton step), y = v*s.  Pinned within a few
 *    ulp of the compiled pk_swish and against the same polynomial evaluated
 *    in double.
 *
 *    depthwise conv, tensor_ops.c:476-548: per channel, val = bias, then in
 *    the 8-wide interior (t in [pad, pad + 8*floor((T-2pad)/8))) the
 *    explicit fma chain over the K taps (tensor_ops.c:519-525).  The
 *    compiler vectorises the remaining scalar loops (left edge, interior
 *    tail, right edge) over k: products of taps 0..7 with out-of-range taps
 *    masked to +0, summed as the eight-lane reduction above and added to
 *    the bias, then fma for the taps past the last multiple of 8 (k = 8
 *    for K = 9).  This model was identified against the compiled
 *    pk_depthwise_conv1d and is pinned bit-for-bit against it for every
 *    T, including T < K.
 */
#include "pk_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#if defined(__x86_64__)
#include <xmmintrin.h>
#endif

static float hsum8(const float p[8])
{
    return ((p[0] + p[4]) + (p[2] + p[6])) + ((p[1] + p[5]) + (p[3] + p[7]));
}

static float inv_std_of(float var, int x86_rsqrt)
{
    const float a = var + 1e-5f;
#if defined(__x86_64__)
    if (x86_rsqrt) {
        const float y = _mm_cvtss_f32(_mm_rsqrt_ss(_mm_set_ss(a)));
        return fmaf(y * a, y, -3.0f) * (y * -0.5f);
    }
#else
    (void)x86_rsqrt;
#endif
    return 1.0f / sqrtf(a);
}

void pkor_layer_norm_rows(const float *x, const float *gamma, const float *beta,
                          float *out, int rows, int D, int x86_rsqrt)
{
    const int D8 = D & ~7;
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *xr = x + (size_t)r * D;
        float *o = out + (size_t)r * D;
        float p[8] = {0};
        for (int i = 0; i < D8; i += 8)
            for (int l = 0; l < 8; l++) p[l] = p[l] + xr[i + l];
        float sum = hsum8(p);
        for (int i = D8; i < D; i++) sum += xr[i];
        const float mean = sum / (float)D;
        float q[8] = {0};
        for (int i = 0; i < D8; i += 8)
            for (int l = 0; l < 8; l++) {
                const float d = xr[i + l] - mean;
                q[l] = fmaf(d, d, q[l]);
            }
        float var_sum = hsum8(q);
        for (int i = D8; i < D; i++) { const float d = xr[i] - mean; var_sum = fmaf(d, d, var_sum); }
        const float inv = inv_std_of(var_sum / (float)D, x86_rsqrt);
        for (int i = 0; i < D; i++) o[i] = fmaf((xr[i] - mean) * inv, gamma[i], beta[i]);
    }
}

float pkor_exp_poly(float x)
{
    x = fminf(fmaxf(x, -87.0f), 87.0f);
    const float kf = rintf(x * 1.44269504088896341f);
    const int ki = (int)kf;
    const float r = fmaf(-kf, 0.69314718055994529f, x);
    float y = 1.0f / 120.0f;
    y = fmaf(y, r, 1.0f / 24.0f);
    y = fmaf(y, r, 1.0f / 6.0f);
    y = fmaf(y, r, 0.5f);
    y = fmaf(y, r, 1.0f);
    y = fmaf(y, r, 1.0f);
    uint32_t bits = (uint32_t)(ki + 127) << 23;
    float p2;
    memcpy(&p2, &bits, 4);
    return y * p2;
}

/* e^x in double, rounded once to float: x = k*ln2 + r (ln2 in two parts,
 * each step one fma), the degree-12 Taylor polynomial of e^r by Horner in
 * fmas, times 2^k (exact), then the conversion to float.  Every step is one
 * IEEE double operation, so any IEEE machine gets these bits.  Pinned
 * against the correctly rounded value (expl, 64-bit significand) over all
 * float inputs in tests/test_oracle_block.py. */
float pkor_expf_ieee(float x)
{
    if (!(x > -104.0f)) return isnan(x) ? x : 0.0f;   /* e^x < 2^-150 */
    if (x > 89.0f) return INFINITY;                   /* e^89 > FLT_MAX */
    const double xd = (double)x;
    const double k = rint(xd * 0x1.71547652b82fep+0);
    double r = fma(-k, 0x1.62e42fefa39efp-1, xd);
    r = fma(-k, 0x1.abc9e3b39803fp-56, r);
    static const double inv_fact[13] = {
        1.0, 1.0, 0.5, 0x1.5555555555555p-3, 0x1.5555555555555p-5, 0x1.1111111111111p-7,
        0x1.6c16c16c16c17p-10, 0x1.a01a01a01a01ap-13, 0x1.a01a01a01a01ap-16,
        0x1.71de3a556c734p-19, 0x1.27e4fb7789f5cp-22, 0x1.ae64567f544e4p-26,
        0x1.1eed8eff8d898p-29};                       /* 1/n!, n = 0..12, rounded */
    double p = inv_fact[12];
    for (int n = 11; n >= 0; n--) p = fma(p, r, inv_fact[n]);
    const uint64_t bits = (uint64_t)((int64_t)k + 1023) << 52;
    double s;
    memcpy(&s, &bits, 8);
    return (float)(p * s);
}

void pkor_expf_ieee_rows(const float *x, float *y, size_t n)
{
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) y[i] = pkor_expf_ieee(x[i]);
}

/* pk_swish (tensor_ops.c:367-389): e = pk_exp_avx2(0 - v) with the
 * reference build's contraction of 1 + poly*2^k into one fma, then the
 * source's IEEE division s = 1/(1 + e) and y = v*s. */
float pkor_swish(float v)
{
    const float t = fminf(fmaxf(-v, -87.0f), 87.0f);
    const float kf = rintf(t * 1.44269504088896341f);
    const int ki = (int)kf;
    const float r = fmaf(-kf, 0.69314718055994529f, t);
    float q = 1.0f / 120.0f;
    q = fmaf(q, r, 1.0f / 24.0f);
    q = fmaf(q, r, 1.0f / 6.0f);
    q = fmaf(q, r, 0.5f);
    q = fmaf(q, r, 1.0f);
    q = fmaf(q, r, 1.0f);
    uint32_t bits = (uint32_t)(ki + 127) << 23;
    float p2;
    memcpy(&p2, &bits, 4);
    const float d = fmaf(q, p2, 1.0f);
    return (1.0f / d) * v;
}

void pkor_swish_rows(const float *x, float *y, size_t n)
{
    #pragma omp parallel for schedule(static)
    for (size_t i = 0; i < n; i++) y[i] = pkor_swish(x[i]);
}

void pkor_softmax_rows(float *x, int rows, int len)
{
    const int L8 = len & ~7;
    for (int r = 0; r < rows; r++) {
        float *v = x + (size_t)r * len;
        float mx = v[0];
        for (int i = 1; i < len; i++) mx = v[i] > mx ? v[i] : mx;
        float p[8] = {0};
        for (int i = 0; i < L8; i += 8)
            for (int l = 0; l < 8; l++) {
                const float e = pkor_exp_poly(v[i + l] - mx);
                v[i + l] = e;
                p[l] = p[l] + e;
            }
        float sum = hsum8(p);
        for (int i = L8; i < len; i++) { v[i] = pkor_expf_ieee(v[i] - mx); sum += v[i]; }
        const float inv = 1.0f / sum;
        for (int i = 0; i < len; i++) v[i] = v[i] * inv;
    }
}

float pkor_dot8(const float *a, const float *b, int K)
{
    const int K8 = K & ~7;
    float p[8] = {0};
    for (int k = 0; k < K8; k += 8)
        for (int l = 0; l < 8; l++) p[l] = fmaf(a[k + l], b[k + l], p[l]);
    float s = hsum8(p);
    for (int k = K8; k < K; k++) s = fmaf(a[k], b[k], s);
    return s;
}

void pkor_attention_core(const float *qkv, int ldq, const float *P, int ldp,
                         const float *pos_bias_u, const float *pos_bias_v,
                         float *out, int ldo, int T, int H, int Dh)
{
    const int D = H * Dh, L = 2 * T - 1;
    const float scale = 0.0883883461356163f;      /* 0x3db504f3 */
    #pragma omp parallel for collapse(2) schedule(dynamic, 8)
    for (int h = 0; h < H; h++) {
        for (int i = 0; i < T; i++) {
            float *qu = (float *)malloc((size_t)Dh * sizeof(float));
            float *qv = (float *)malloc((size_t)Dh * sizeof(float));
            float *s = (float *)malloc((size_t)T * sizeof(float));
            const float *q = qkv + (size_t)i * ldq + h * Dh;
            for (int d = 0; d < Dh; d++) {
                qu[d] = q[d] + pos_bias_u[h * Dh + d];
                qv[d] = q[d] + pos_bias_v[h * Dh + d];
            }
            for (int j = 0; j < T; j++) {
                const float ac = pkor_dot8(qu, qkv + (size_t)j * ldq + D + h * Dh, Dh);
                const int m = T - 1 - i + j;            /* relative shift */
                const float bd = (m >= 0 && m < L) ? pkor_dot8(qv, P + (size_t)m * ldp + h * Dh, Dh)
                                                   : 0.0f;
                s[j] = (ac + bd) * scale;
            }
            pkor_softmax_rows(s, 1, T);
            /* o[d] = fma chain over j ascending (sgemm NN); the d loop is
             * inside only so that the chains advance side by side */
            float *o = out + (size_t)i * ldo + h * Dh;
            for (int d = 0; d < Dh; d++) o[d] = 0.0f;
            for (int j = 0; j < T; j++) {
                const float *vj = qkv + (size_t)j * ldq + 2 * D + h * Dh;
                for (int d = 0; d < Dh; d++) o[d] = fmaf(s[j], vj[d], o[d]);
            }
            free(qu);
            free(qv);
            free(s);
        }
    }
}

void pkor_glu_rows(const float *in, float *out, int rows, int D)
{
    #pragma omp parallel for schedule(static)
    for (int r = 0; r < rows; r++) {
        const float *a = in + (size_t)r * 2 * D;
        for (int d = 0; d < D; d++) {
            const float e = pkor_expf_ieee(-a[D + d]);
            const float sg = 1.0f / (1.0f + e);
            out[(size_t)r * D + d] = a[d] * sg;
        }
    }
}

void pkor_depthwise_conv1d(const float *x, const float *w, const float *b, float *out,
                           int C, int T, int K)
{
    const int pad = (K - 1) / 2;
    const int t_lo = pad, t_hi = T - pad > pad ? T - pad : pad;
    const int t_vec = t_lo + (t_hi - t_lo) / 8 * 8;      /* end of the 8-wide interior */
    const int K8 = K & ~7;
    for (int c = 0; c < C; c++) {
        const float *xc = x + (size_t)c * T;
        const float *wc = w + (size_t)c * K;
        for (int t = 0; t < T; t++) {
            float val = b ? b[c] : 0.0f;
            if (t >= t_lo && t < t_vec) {                 /* tensor_ops.c:519-525 */
                for (int k = 0; k < K; k++) val = fmaf(xc[t - pad + k], wc[k], val);
            } else {                                      /* edge and tail loops, as compiled */
                for (int k0 = 0; k0 < K8; k0 += 8) {
                    float p[8];
                    for (int l = 0; l < 8; l++) {
                        const int src = t - pad + k0 + l;
                        p[l] = (src >= 0 && src < T) ? xc[src] * wc[k0 + l] : 0.0f;
                    }
                    val = val + hsum8(p);
                }
                for (int k = K8; k < K; k++) {
                    const int src = t - pad + k;
                    if (src >= 0 && src < T) val = fmaf(xc[src], wc[k], val);
                }
            }
            out[(size_t)c * T + t] = val;
        }
    }
}
