// pk_panel.hip - small-M weight GEMMs (M <= 64) on weights repacked once
// into the matrix cores' operand order (a "panel"), with the activations
// staged through LDS.
//
// These are the tolerance-path products of pk_smallm.hip (the same split
// arithmetic, within max |C - R| / max |R| <= 1e-3 of the reference's fma
// chain, blas.c:187-218, 759-771, 950-963, 1055-1072), for weights that a
// caller declared long-lived: registered host weights, the resident
// encoder's weights, or device weights passed to pk_gpu_pack_weight_dev.
// Two layouts decide their speed:
//
//   Panel.  For v_mfma_f32_16x16x32_bf16 lane l = i + 16 g takes column i of
//   a 16-column tile and the 8 consecutive k = 32 s + 8 g .. + 7 of a 32-deep
//   step s.  The panel stores, for each (tile t, step s), the 64 lanes' bytes
//   back to back, so a wave reads one step of one tile as one contiguous
//   block: int8 8 bytes a lane (the codes), int4 4 bytes (the 8 codes as
//   nibbles, low first), fp32 32 bytes (bf16 hi = bf16(w) and lo =
//   bf16(w - hi), both to nearest, so the weight split is done once here).
//   int4 scales are kept transposed, [N/32][K], so 4 consecutive k of one
//   group are one 16-byte load.  The on-disk [K][N] layout puts one
//   workgroup's 16-32 bytes of each row in a cache line of its own, which is
//   what bounds the narrow kernels of pk_smallm.hip.
//
//   Activations.  A workgroup needs every one of its M rows over its whole k
//   range, while its weights are only 16 columns wide, so activation bytes
//   dominate (8:1 for int8 at M = 32).  Read in the operand layout (16 rows
//   per load instruction, 64 bytes of each) they cost twice what the same
//   bytes cost read as whole rows (1 KB of one row per instruction), as
//   measured on MI355X.  So the rows are read whole, written to LDS with a
//   row pitch of 16 bytes beyond a multiple of 128 (the 16 rows of a
//   fragment read then fall in distinct banks), and each wave reads its
//   fragments from there and splits them as x = hi + lo + r (hi = bf16(x),
//   lo = bf16(x - hi), |r| <= 2^-16 |x|).  int4 folds its scale into the
//   activations on the way into LDS (a workgroup's columns share one
//   32-column scale group): A' = fl(A * s[k][g]), so the codes enter the
//   matrix cores exactly.
//
// Work split.  A workgroup of 8 waves owns NCT 16-column tiles, up to MB
// 16-row blocks (grid.y row groups) and a k segment (grid.z segments; each
// writes a partial tile that panel_reduce sums in segment order).  Within a segment, phases of kph k
// (as many as the LDS holds rows for) run one after the other; in a phase
// every wave issues its activation-row loads, then the weight loads of its
// own steps (s = wave + 8 q), so the weights stream from HBM while the rows
// go to LDS and are split.  The waves' partial tiles are summed in LDS in
// wave order.  Every sum has a fixed order: results are deterministic.
#include "pk_gemm_kernels.h"
#include "pk_device_math.h"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <utility>

namespace pkgpu {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kXcd = 8;
constexpr int kPW = 8;                  // waves per workgroup
constexpr int kLds = 147456;            // LDS bytes of a workgroup
constexpr int kLnChunk = 64;            // fused LayerNorms: rows of a multiple of 8 * 64

// Panel bytes per lane per (tile, step).
constexpr int unit_bytes(int wk) { return wk == W_I8 ? 8 : wk == W_I4 ? 4 : 32; }

struct PanelArgs {
    int M, N, K;
    float alpha;               // int8: alpha * scale
    float beta;
    const float* A; int lda;
    const unsigned char* P;    // codes / split weights, [T][S][64][unit]
    const float* ST;           // int4: scales [N/32][K]
    float* C; int ldc;
    const float* bias; int epi;
    float* work;               // grid.z > 1: partial tiles [grid.z][M][N]
    int kseg, kph;             // k per segment (grid.z) and per LDS phase, multiples of 32
    uint32_t a_bytes, p_bytes, s_bytes;
    const float* ln_g;         // LN kernels: A is x and the products take LayerNorm(x) with
    const float* ln_b;         //   these gamma, beta [K] (one phase holds all of K)
};

__device__ inline __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

__device__ inline v2bf to_bf2(float a, float b) { return __builtin_convertvector((v2f){a, b}, v2bf); }

__device__ inline v8bf cat(v2bf a, v2bf b, v2bf c, v2bf d)
{
    const v4bf lo = __builtin_shufflevector(a, b, 0, 1, 2, 3);
    const v4bf hi = __builtin_shufflevector(c, d, 0, 1, 2, 3);
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// x (8 fp32) -> hi = bf16(x), lo = bf16(x - hi), both to nearest.
__device__ inline void split8(const float (&x)[8], v8bf& hi, v8bf& lo)
{
    v2bf h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        h[e] = to_bf2(x[2 * e], x[2 * e + 1]);
        l[e] = to_bf2(__fsub_rn(x[2 * e], bf16_value(h[e][0])), __fsub_rn(x[2 * e + 1], bf16_value(h[e][1])));
    }
    hi = cat(h[0], h[1], h[2], h[3]);
    lo = cat(l[0], l[1], l[2], l[3]);
}

__device__ inline v4f mfma(v8bf a, v8bf b, v4f c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// The output step shared by the one-segment kernel and the segment reduce:
// C = fl(alpha * sum) (+ beta C), then bias and the fused epilogue, as the
// other small-M and exact kernels store it.
__device__ inline void store_out(const PanelArgs& p, int m, int n, float sum)
{
    float* cp = p.C + (size_t)m * p.ldc + n;
    float r = __fmul_rn(p.alpha, sum);
    if (p.beta != 0.0f) r = __fadd_rn(p.beta == 1.0f ? *cp : __fmul_rn(p.beta, *cp), r);
    if (p.bias) r = __fadd_rn(r, p.bias[n]);
    switch (p.epi) {
    case EPI_SWISH:         r = swish_f(r); break;
    case EPI_HALF_RESIDUAL: r = __fmaf_rn(r, 0.5f, *cp); break;
    case EPI_RESIDUAL:      r = __fadd_rn(*cp, r); break;
    case EPI_RELU:          r = r > 0.0f ? r : 0.0f; break;
    default:                break;
    }
    *cp = r;
}

template <int WK> struct WUnit;
template <> struct WUnit<W_I8> { typedef v2u T; };
template <> struct WUnit<W_I4> { typedef uint32_t T; };
template <> struct WUnit<W_F32> { typedef v4u T[2]; };

// Activation rows per wave and 256-k row loads per phase, as the LDS allows:
// kph is 1024 for M <= 35, at least 512 up to M = 64.  HALF: phases of 512
// k at most (segments of K split over twice as many workgroups).
template <int MB, bool HALF> struct PanelShape {
    static constexpr int RPW = (16 * MB + kPW - 1) / kPW;
    static constexpr int CPR = MB <= 3 && !HALF ? 4 : 2;
    static constexpr int SPW = CPR * 8 / kPW;            // steps per wave per phase
};

// LN: the activations are normalised on the way in (the LayerNorm that feeds
// the GEMM, fused): after the rows are in LDS, 8 lanes per row compute its
// mean and 1/sqrt(var + eps) exactly as the LayerNorm kernel does
// (ln_row_stats), and each fragment read forms fl(fl(fl(x - mean) * inv) *
// gamma + beta), the LayerNorm output bit for bit, before the int4 scale
// fold and the split.  LDS past the rows: 32 zero bytes, the rows' (mean,
// inv) pairs (64 rows' worth), gamma and beta [K], int4 scales [K].
template <int WK, int MB, int NCT, bool LN, bool HALF>
__global__ __launch_bounds__(64 * kPW) void smallm_panel(PanelArgs p)
{
    typedef PanelShape<MB, HALF> L;
    constexpr int UB = unit_bytes(WK);
    __shared__ __attribute__((aligned(16))) unsigned char smem[kLds];

    // column tiles in XCD-sized runs (workgroups reach the XCDs round-robin)
    const int x = blockIdx.x, per = gridDim.x / kXcd;
    const int tt = (x % kXcd) * per + x / kXcd;
    if (tt * 16 * NCT >= p.N) return;                    // padding workgroup (uniform)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane & 15, g = lane >> 4;
    const int m0 = 16 * MB * blockIdx.y;
    const int M = min(p.M - m0, 16 * MB), S = p.K / 32;     // this group's rows
    const int pitch = p.kph * 4 + 16;
    const int kbeg = blockIdx.z * p.kseg, kend = min(p.K, kbeg + p.kseg);
    const uint32_t grp = (uint32_t)(tt * NCT * 16) >> 5;
    const auto rA = rsrc(p.A, p.a_bytes), rP = rsrc(p.P, p.p_bytes), rS = rsrc(p.ST, p.s_bytes);

    // rows >= M read their fragments from 32 zero bytes past the last row
    if (threadIdx.x < 2) *reinterpret_cast<v4u*>(smem + M * pitch + 16 * threadIdx.x) = v4u{0, 0, 0, 0};
    float* ln_st = reinterpret_cast<float*>(smem + M * pitch + 32);      // [64][mean, inv]
    float* ln_gb = ln_st + 128;                                           // gamma [K], beta [K], scales [K]

    v4f acc[MB][NCT];
#pragma unroll
    for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int j = 0; j < NCT; ++j) acc[rb][j] = v4f{0.f, 0.f, 0.f, 0.f};

    for (int k0 = kbeg; k0 < kend; k0 += p.kph) {
        const int kn = min(p.kph, kend - k0), sph = kn / 32, s0 = k0 / 32;
        // The phase's loads, all issued before any is waited for, activation
        // rows first (256 k = 1 KB per load), then the weights of this wave's
        // steps s0 + wave + 8 q.  They are unconditional: a buffer load past
        // its operand's extent reads 0, and the lanes whose rows or steps lie
        // outside the phase are never stored or multiplied.
        v4u areg[L::RPW][L::CPR];
#pragma unroll
        for (int q = 0; q < L::RPW; ++q)
#pragma unroll
            for (int c = 0; c < L::CPR; ++c)
                areg[q][c] = __builtin_amdgcn_raw_buffer_load_b128(
                    rA, (int)(((uint32_t)(m0 + wave + kPW * q) * (uint32_t)p.lda +
                               (uint32_t)(k0 + 256 * c + 4 * lane)) * 4u), 0, 0);
        v4u sreg[L::CPR];
        if constexpr (WK == W_I4 && !LN) {
#pragma unroll
            for (int c = 0; c < L::CPR; ++c)
                sreg[c] = __builtin_amdgcn_raw_buffer_load_b128(
                    rS, (int)((grp * (uint32_t)p.K + (uint32_t)(k0 + 256 * c + 4 * lane)) * 4u), 0, 0);
        }
        // LN: gamma, beta (and the int4 group's scales), 4 k per unit, K <= 1024
        constexpr int GBU = WK == W_I4 ? 3 : 2;
        v4f gbreg[2];
        const int q4 = p.K / 4;
        if constexpr (LN) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int u = threadIdx.x + 64 * kPW * h, which = u / q4, j = u % q4;
                if (u < GBU * q4)
                    gbreg[h] = which == 0 ? *reinterpret_cast<const v4f*>(p.ln_g + 4 * j)
                             : which == 1 ? *reinterpret_cast<const v4f*>(p.ln_b + 4 * j)
                                          : *reinterpret_cast<const v4f*>(p.ST + (size_t)grp * p.K + 4 * j);
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        typename WUnit<WK>::T wreg[L::SPW][NCT];
#pragma unroll
        for (int q = 0; q < L::SPW; ++q)
#pragma unroll
            for (int j = 0; j < NCT; ++j) {
                const uint32_t off = (((uint32_t)(tt * NCT + j) * (uint32_t)S + (uint32_t)(s0 + wave + kPW * q)) * 64u +
                                      lane) * UB;
                if constexpr (WK == W_I8) {
                    wreg[q][j] = __builtin_amdgcn_raw_buffer_load_b64(rP, (int)off, 0, 0);
                } else if constexpr (WK == W_I4) {
                    wreg[q][j] = __builtin_amdgcn_raw_buffer_load_b32(rP, (int)off, 0, 0);
                } else {
                    wreg[q][j][0] = __builtin_amdgcn_raw_buffer_load_b128(rP, (int)off, 0, 0);
                    wreg[q][j][1] = __builtin_amdgcn_raw_buffer_load_b128(rP, (int)(off + 16), 0, 0);
                }
            }
        __builtin_amdgcn_sched_barrier(0);
        // the previous phase's fragment reads are done before its rows are replaced
        if (k0 != kbeg) __syncthreads();
#pragma unroll
        for (int q = 0; q < L::RPW; ++q) {
            const int r = wave + kPW * q;
#pragma unroll
            for (int c = 0; c < L::CPR; ++c) {
                const int kk = 256 * c + 4 * lane;
                v4u v = areg[q][c];
                if constexpr (WK == W_I4 && !LN) {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        v[e] = __float_as_uint(__fmul_rn(__uint_as_float(v[e]), __uint_as_float(sreg[c][e])));
                }
                if (r < M && kk < kn)
                    *static_cast<v4u*>(__builtin_assume_aligned(smem + r * pitch + kk * 4, 16)) = v;
            }
        }
        if constexpr (LN) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int u = threadIdx.x + 64 * kPW * h;
                if (u < GBU * q4) *reinterpret_cast<v4f*>(ln_gb + 4 * u) = gbreg[h];
            }
        }
        __syncthreads();
        if constexpr (LN) {
            // every row's mean and 1 / sqrt(var + eps): 8 lanes a row, one pass for 64 rows.
            // Row r starts 4 r banks into the LDS (pitch 16 mod 128 bytes): a
            // half wave takes rows 8 wave + {0, 2, 4, 6} or {1, 3, 5, 7}, whose
            // 8-float runs then fall in distinct banks.
            const int r = 8 * wave + 2 * ((lane >> 3) & 3) + (lane >> 5), l = lane & 7;
            if (r < M) {
                float mean, inv;
                ln_row_stats<kLnChunk>(reinterpret_cast<const float*>(smem + r * pitch), p.K, l, mean, inv);
                if (l == 0) {
                    ln_st[2 * r] = mean;
                    ln_st[2 * r + 1] = inv;
                }
            }
            __syncthreads();
        }
        // this wave's steps: fragments read and split, then the weights
#pragma unroll
        for (int q = 0; q < L::SPW; ++q) {
            const int st = wave + kPW * q;
            if (st >= sph) break;                         // uniform per wave
            v8bf ahi[MB], alo[MB];
            // LN: this step's 8 gammas, betas (and int4 scales) of k = 32 st + 8 g ..
            v4f lg[2], lb[2], ls[2];
            if constexpr (LN) {
                const int k = 32 * st + 8 * g;
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    lg[h] = *reinterpret_cast<const v4f*>(ln_gb + k + 4 * h);
                    lb[h] = *reinterpret_cast<const v4f*>(ln_gb + p.K + k + 4 * h);
                    if constexpr (WK == W_I4) ls[h] = *reinterpret_cast<const v4f*>(ln_gb + 2 * p.K + k + 4 * h);
                }
            }
#pragma unroll
            for (int rb = 0; rb < MB; ++rb) {
                const int r = 16 * rb + i;
                const unsigned char* f = static_cast<const unsigned char*>(__builtin_assume_aligned(
                    r < M ? smem + r * pitch + (32 * st + 8 * g) * 4 : smem + M * pitch, 16));
                const v4u a0 = *reinterpret_cast<const v4u*>(f);
                const v4u a1 = *reinterpret_cast<const v4u*>(f + 16);
                float xa[8] = {__uint_as_float(a0[0]), __uint_as_float(a0[1]), __uint_as_float(a0[2]),
                               __uint_as_float(a0[3]), __uint_as_float(a1[0]), __uint_as_float(a1[1]),
                               __uint_as_float(a1[2]), __uint_as_float(a1[3])};
                if constexpr (LN) {
                    // rows >= M (zeros, whatever they become) reach only output rows >= M
                    const float mean = r < M ? ln_st[2 * r] : 0.0f, inv = r < M ? ln_st[2 * r + 1] : 0.0f;
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        xa[e] = __fmaf_rn(__fmul_rn(__fsub_rn(xa[e], mean), inv), lg[e >> 2][e & 3], lb[e >> 2][e & 3]);
                        if constexpr (WK == W_I4) xa[e] = __fmul_rn(xa[e], ls[e >> 2][e & 3]);
                    }
                }
                split8(xa, ahi[rb], alo[rb]);
            }
            v8bf bhi[NCT], blo[NCT];
#pragma unroll
            for (int j = 0; j < NCT; ++j) {
                if constexpr (WK == W_F32) {
                    bhi[j] = __builtin_bit_cast(v8bf, wreg[q][j][0]);
                    blo[j] = __builtin_bit_cast(v8bf, wreg[q][j][1]);
                } else {
                    float wv[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        if constexpr (WK == W_I8)
                            wv[e] = (float)(int)(signed char)(wreg[q][j][e >> 2] >> (8 * (e & 3)));
                        else
                            wv[e] = (float)((int)(wreg[q][j] << (28 - 4 * e)) >> 28);
                    }
                    bhi[j] = cat(to_bf2(wv[0], wv[1]), to_bf2(wv[2], wv[3]),
                                 to_bf2(wv[4], wv[5]), to_bf2(wv[6], wv[7]));     // exact
                }
            }
#pragma unroll
            for (int rb = 0; rb < MB; ++rb)
#pragma unroll
                for (int j = 0; j < NCT; ++j) {
                    acc[rb][j] = mfma(ahi[rb], bhi[j], acc[rb][j]);
                    acc[rb][j] = mfma(alo[rb], bhi[j], acc[rb][j]);
                    if constexpr (WK == W_F32) acc[rb][j] = mfma(ahi[rb], blo[j], acc[rb][j]);
                }
        }
    }

    // fixed-order sum over the waves
    __syncthreads();                                     // every fragment read done: reuse as `red`
    v4f* red = reinterpret_cast<v4f*>(smem);             // [kPW][MB][NCT][64]
#pragma unroll
    for (int rb = 0; rb < MB; ++rb)
#pragma unroll
        for (int j = 0; j < NCT; ++j) red[((wave * MB + rb) * NCT + j) * 64 + lane] = acc[rb][j];
    __syncthreads();
    const float* rf = reinterpret_cast<const float*>(red);
    for (int o = threadIdx.x; o < MB * NCT * 256; o += 64 * kPW) {
        const int rb = o / (NCT * 256), j = (o >> 8) % NCT, l = (o >> 2) & 63, v = o & 3;
        float sum = rf[((rb * NCT + j) * 64 + l) * 4 + v];
#pragma unroll
        for (int w = 1; w < kPW; ++w) sum = __fadd_rn(sum, rf[(((w * MB + rb) * NCT + j) * 64 + l) * 4 + v]);
        const int m = 16 * rb + 4 * (l >> 4) + v, n = 16 * (tt * NCT + j) + (l & 15);
        if (m >= M || n >= p.N) continue;
        if (gridDim.z > 1) p.work[((size_t)blockIdx.z * p.M + m0 + m) * p.N + n] = sum;
        else store_out(p, m0 + m, n, sum);
    }
}

// The partials of output o over segs <= kMaxSegs segments, added in segment
// order; every load is issued before the first addition (the extra loads of
// absent segments read segment 0 and are not added).
constexpr int kMaxSegs = 16;
__device__ inline float sum_segments(const float* work, size_t o, size_t mn, int segs)
{
    float v[kMaxSegs];
#pragma unroll
    for (int z = 0; z < kMaxSegs; ++z) v[z] = work[(z < segs ? (size_t)z * mn : 0) + o];
    float sum = v[0];
#pragma unroll
    for (int z = 1; z < kMaxSegs; ++z) sum = z < segs ? __fadd_rn(sum, v[z]) : sum;
    return sum;
}

// Segment partials summed in segment order, then the output step, then,
// over each whole output row, LayerNorm with gamma, beta [N] (the block's
// LayerNorm that follows the residual add, fused): one workgroup per row,
// the row in LDS, its statistics by the first 8 lanes (ln_row_stats), then
// C = fl(fl(fl(v - mean) * inv) * gamma + beta).  N <= kReduceLnMaxN.
constexpr int kReduceLnMaxN = 2048;
// EPT outputs per thread (N <= 256 EPT): each thread's loads (partials,
// C, bias, gamma, beta of all its outputs) are issued before the first is
// used, so the row costs one memory round trip rather than EPT of them.
template <int EPT>
__global__ __launch_bounds__(256) void panel_reduce_ln(PanelArgs p, int segs, const float* gamma,
                                                       const float* beta)
{
    __shared__ float row[kReduceLnMaxN];
    __shared__ float st[2];
    const int m = blockIdx.x;
    const size_t mn = (size_t)p.M * p.N;
    float* crow = p.C + (size_t)m * p.ldc;
    float part[EPT][kMaxSegs], cv[EPT], bv[EPT], gv[EPT], be[EPT];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        // outputs past N load output N - 1's operands and are not stored
        const int n = min((int)threadIdx.x + 256 * e, p.N - 1);
        const size_t o = (size_t)m * p.N + n;
#pragma unroll
        for (int z = 0; z < kMaxSegs; ++z) part[e][z] = p.work[(z < segs ? (size_t)z * mn : 0) + o];
        cv[e] = p.beta != 0.0f || p.epi == EPI_HALF_RESIDUAL || p.epi == EPI_RESIDUAL ? crow[n] : 0.0f;
        bv[e] = p.bias ? p.bias[n] : 0.0f;
        gv[e] = gamma[n];
        be[e] = beta[n];
    }
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int n = threadIdx.x + 256 * e;
        float sum = part[e][0];
#pragma unroll
        for (int z = 1; z < kMaxSegs; ++z) sum = z < segs ? __fadd_rn(sum, part[e][z]) : sum;
        float r = __fmul_rn(p.alpha, sum);
        if (p.beta != 0.0f) r = __fadd_rn(p.beta == 1.0f ? cv[e] : __fmul_rn(p.beta, cv[e]), r);
        if (p.bias) r = __fadd_rn(r, bv[e]);
        switch (p.epi) {
        case EPI_SWISH:         r = swish_f(r); break;
        case EPI_HALF_RESIDUAL: r = __fmaf_rn(r, 0.5f, cv[e]); break;
        case EPI_RESIDUAL:      r = __fadd_rn(cv[e], r); break;
        case EPI_RELU:          r = r > 0.0f ? r : 0.0f; break;
        default:                break;
        }
        if (n < p.N) row[n] = r;
    }
    __syncthreads();
    if (threadIdx.x < 8) {
        float mean, inv;
        ln_row_stats<kLnChunk>(row, p.N, threadIdx.x, mean, inv);
        if (threadIdx.x == 0) {
            st[0] = mean;
            st[1] = inv;
        }
    }
    __syncthreads();
    const float mean = st[0], inv = st[1];
#pragma unroll
    for (int e = 0; e < EPT; ++e) {
        const int n = threadIdx.x + 256 * e;
        if (n < p.N) crow[n] = __fmaf_rn(__fmul_rn(__fsub_rn(row[n], mean), inv), gv[e], be[e]);
    }
}

// Segment partials summed in segment order, then the output step.
__global__ __launch_bounds__(256) void panel_reduce(PanelArgs p, int segs)
{
    const long long o = (long long)blockIdx.x * 256 + threadIdx.x;
    const long long mn = (long long)p.M * p.N;
    if (o >= mn) return;
    store_out(p, (int)(o / p.N), (int)(o % p.N), sum_segments(p.work, (size_t)o, (size_t)mn, segs));
}

// ---- the repack -------------------------------------------------------------
// One thread per (tile, step, lane) writes that lane's unit; columns past N
// hold code 0 (or weight 0).
template <int WK>
__global__ __launch_bounds__(256) void pack_panel(int K, int N, const void* B, int ldb, unsigned char* P)
{
    const int T = (N + 15) / 16, S = K / 32;
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long long)T * S * 64) return;
    const int l = (int)(idx % 64);
    const long long ts = idx / 64;
    const int s = (int)(ts % S), t = (int)(ts / S);
    const int i = l & 15, g = l >> 4, n = 16 * t + i;
    const size_t k0 = (size_t)(32 * s + 8 * g);
    if constexpr (WK == W_I8) {
        const signed char* b = static_cast<const signed char*>(B);
        uint32_t u[2] = {0, 0};
        if (n < N)
            for (int e = 0; e < 8; ++e) u[e >> 2] |= (uint32_t)(unsigned char)b[(k0 + e) * ldb + n] << (8 * (e & 3));
        *reinterpret_cast<v2u*>(P + idx * 8) = v2u{u[0], u[1]};
    } else if constexpr (WK == W_I4) {
        const unsigned char* b = static_cast<const unsigned char*>(B);
        uint32_t u = 0;
        if (n < N)
            for (int e = 0; e < 8; ++e) u |= (uint32_t)((b[(k0 + e) * ldb + n / 2] >> (4 * (n & 1))) & 0xF) << (4 * e);
        *reinterpret_cast<uint32_t*>(P + idx * 4) = u;
    } else {
        const float* b = static_cast<const float*>(B);
        uint32_t hi[4], lo[4];
        for (int e = 0; e < 8; e += 2) {
            const float w0 = n < N ? b[(k0 + e) * ldb + n] : 0.0f;
            const float w1 = n < N ? b[(k0 + e + 1) * ldb + n] : 0.0f;
            split_bf16x2(w0, w1, hi[e >> 1], lo[e >> 1]);
        }
        *reinterpret_cast<v4u*>(P + idx * 32) = v4u{hi[0], hi[1], hi[2], hi[3]};
        *reinterpret_cast<v4u*>(P + idx * 32 + 16) = v4u{lo[0], lo[1], lo[2], lo[3]};
    }
}

// int4 scales [K][N/32] -> [N/32][K]
__global__ __launch_bounds__(256) void pack_scales(int K, int G, const float* s, float* out)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long long)K * G) return;
    const int grp = (int)(idx / K), k = (int)(idx % K);
    out[idx] = s[(size_t)k * G + grp];
}

// The weights as the panel kernels multiply them, to out [K][N]: int8
// fl(q * scale), int4 fl(q * s[k][n/32]), fp32 hi + lo.
template <int WK>
__global__ __launch_bounds__(256) void decode_panel(int K, int N, const unsigned char* P, const float* ST,
                                                    float scale, float* out)
{
    const long long idx = (long long)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (long long)K * N) return;
    const int k = (int)(idx / N), n = (int)(idx % N);
    const int t = n / 16, i = n % 16, s = k / 32, g = (k % 32) / 8, e = k % 8;
    const long long unit = ((long long)t * (K / 32) + s) * 64 + i + 16 * g;
    float w;
    if constexpr (WK == W_I8) {
        w = __fmul_rn((float)(int)(signed char)P[unit * 8 + e], scale);
    } else if constexpr (WK == W_I4) {
        const uint32_t u = *reinterpret_cast<const uint32_t*>(P + unit * 4);
        w = __fmul_rn((float)((int)(u << (28 - 4 * e)) >> 28), ST[(size_t)(n / 32) * K + k]);
    } else {
        const unsigned short* h = reinterpret_cast<const unsigned short*>(P + unit * 32);
        w = __fadd_rn(__uint_as_float((uint32_t)h[e] << 16), __uint_as_float((uint32_t)h[8 + e] << 16));
    }
    out[idx] = w;
}

size_t codes_bytes(WeightKind kind, int K, int N)
{
    return (size_t)((N + 15) / 16) * (K / 32) * 64 * unit_bytes(kind);
}

size_t scales_offset(WeightKind kind, int K, int N)
{
    return kind == W_I4 ? (codes_bytes(kind, K, N) + 255) & ~(size_t)255 : 0;
}

// Tiles with a fused input LayerNorm: all but fp32 weights at 3-4 row blocks
// and 2 column tiles, whose registers would spill (panel_tile skips them).
constexpr bool ln_tile(int wk, int mb, int nct) { return !(wk == W_F32 && mb >= 3 && nct == 2); }

// half: phases of 512 k (MB <= 3, no fused input LayerNorm).
template <int WK, int MB, int NCT>
void launch_t(const PanelArgs& a, dim3 grid, hipStream_t st, bool half)
{
    if constexpr (ln_tile(WK, MB, NCT)) {
        if (a.ln_g) {
            hipLaunchKernelGGL((smallm_panel<WK, MB, NCT, true, false>), grid, dim3(64 * kPW), 0, st, a);
            return;
        }
    }
    if constexpr (MB <= 3) {
        if (half) {
            hipLaunchKernelGGL((smallm_panel<WK, MB, NCT, false, true>), grid, dim3(64 * kPW), 0, st, a);
            return;
        }
    }
    hipLaunchKernelGGL((smallm_panel<WK, MB, NCT, false, false>), grid, dim3(64 * kPW), 0, st, a);
}

template <int WK>
void launch_wk(int MB, int NCT, bool half, const PanelArgs& a, dim3 grid, hipStream_t st)
{
    switch (MB * 2 + NCT - 1) {
    case 2: launch_t<WK, 1, 1>(a, grid, st, half); break;
    case 3: launch_t<WK, 1, 2>(a, grid, st, half); break;
    case 4: launch_t<WK, 2, 1>(a, grid, st, half); break;
    case 5: launch_t<WK, 2, 2>(a, grid, st, half); break;
    case 6: launch_t<WK, 3, 1>(a, grid, st, half); break;
    case 7: launch_t<WK, 3, 2>(a, grid, st, half); break;
    case 8: launch_t<WK, 4, 1>(a, grid, st, half); break;
    default: launch_t<WK, 4, 2>(a, grid, st, half); break;
    }
}

thread_local int t_panel_mb = 0, t_panel_nct = 0;   // forced workgroup tile (0: the choice below)

// LDS bytes past the rows and their zero bytes: with a fused input
// LayerNorm, the rows' statistics (64 pairs), gamma and beta, and the int4
// group's scales.
size_t lds_extra(const GemmProblem& p)
{
    if (!p.ln_gamma) return 0;
    return 512 + (size_t)p.K * 4 * (p.kind == W_I4 ? 3 : 2);
}

// k per LDS phase: the longest multiple of 256 (at most 1024) whose rows, at
// a pitch of 16 bytes beyond the row, the 32 zero bytes and `extra` fit the
// LDS (0 if not even 256 do).
int phase_k(int rows, size_t extra)
{
    int kph = 1024;
    while (kph > 0 && (long long)rows * (kph * 4 + 16) + 32 + (long long)extra > kLds) kph -= 256;
    return std::min(kph, rows > 48 ? 512 : 1024);
}

// Whether a workgroup of `rows` rows can take a problem: a fused input
// LayerNorm needs all of K in one phase.
bool rows_fit(const GemmProblem& p, int rows)
{
    const int kph = phase_k(rows, lds_extra(p));
    if (kph <= 0) return false;
    return !p.ln_gamma || p.K <= kph;
}

// K segments for a workgroup of `rows` rows: one per LDS phase when K takes
// at least kMinSegs phases and the caller gave a workspace big enough for the
// partial tiles (and there is no fused input LayerNorm), else one.  With 2
// or 3 phases the phases run one after the other in one launch instead:
// measured on MI355X (graph replay, both launches of the split form), i4
// 33x1024x3072 8.1 against 9.2 us, i8 64x1024x2048 5.9 against 7.4, i4
// 64x4096x2048 11.4 against 16.4, f32 33x1024x2048 7.0 against 8.9; from 4
// phases the split wins (i4 33x1024x4096 9.55 against 10.06, i4
// 16x1024x4096 7.6 against 10.8).
// half: phases (and so segments) of at most 512 k.
constexpr int kMinSegs = 4;
int kph_of(const GemmProblem& p, int rows, bool half)
{
    const int kph = phase_k(rows, lds_extra(p));
    return half ? std::min(kph, 512) : kph;
}
int segments_for(const GemmProblem& p, int rows, bool half = false)
{
    const int kph = kph_of(p, rows, half);
    if (!p.work || p.ln_gamma || p.K <= kph) return 1;
    const int segs = (p.K + kph - 1) / kph;
    if (segs < kMinSegs) return 1;
    if (segs > kMaxSegs || (size_t)segs * p.M * p.N * 4 > p.work_bytes) return 1;
    return segs;
}

// Modelled time (us) of a workgroup tile: MB 16-row blocks (grid.y = row
// groups) and NCT 16-column tiles.  Workgroups run in rounds of 256 (one per
// CU); a round costs the busiest workgroup's split work (every one of its
// padded rows over its k), its matrix-core work (row blocks x column tiles
// x k; fp32 weights take 3 products instead of 2) and a fixed part.  Fitted
// to a sweep of every tile over the encoder's M = 33 shapes, workload 0
// (M = 32) and M = 1, 16, 64 on MI355X: it picks the fastest tile on 10 of
// 11 shapes and one within 1% on the other.
double tile_cost(const GemmProblem& p, int mb, int nct, bool half)
{
    const int rows = std::min(p.M, 16 * mb);
    const int segs = segments_for(p, rows, half);
    const double kseg = (double)p.K / segs;
    const double wgs = (double)((p.N + 16 * nct - 1) / (16 * nct)) * ((p.M + 16 * mb - 1) / (16 * mb)) * segs;
    const double rounds = std::ceil(wgs / 256.0);
    const double split = 16.0 * mb * kseg / 1024.0;
    const double mfma = mb * nct * kseg / 1024.0 * (p.kind == W_F32 ? 1.5 : 1.0);
    return rounds * (0.080 * split + 0.499 * mfma + 1.80) + 0.64;
}


}  // namespace

size_t panel_bytes(WeightKind kind, int K, int N)
{
    if (K <= 0 || N <= 0 || K % 32) return 0;
    if (kind == W_I4) return scales_offset(kind, K, N) + (size_t)(N / 32) * K * 4;
    return codes_bytes(kind, K, N);
}

hipError_t launch_pack(WeightKind kind, int K, int N, const void* B, int ldb, const float* scales,
                       void* panel, hipStream_t st)
{
    if (K <= 0 || N <= 0 || K % 32 || (kind == W_I4 && N % 32)) return hipErrorInvalidValue;
    unsigned char* P = static_cast<unsigned char*>(panel);
    const long long units = (long long)((N + 15) / 16) * (K / 32) * 64;
    const unsigned blocks = (unsigned)((units + 255) / 256);
    switch (kind) {
    case W_I8: hipLaunchKernelGGL(pack_panel<W_I8>, dim3(blocks), dim3(256), 0, st, K, N, B, ldb, P); break;
    case W_I4: hipLaunchKernelGGL(pack_panel<W_I4>, dim3(blocks), dim3(256), 0, st, K, N, B, ldb, P); break;
    default:   hipLaunchKernelGGL(pack_panel<W_F32>, dim3(blocks), dim3(256), 0, st, K, N, B, ldb, P); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || kind != W_I4) return e;
    const long long n = (long long)K * (N / 32);
    hipLaunchKernelGGL(pack_scales, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, K, N / 32, scales,
                       reinterpret_cast<float*>(P + scales_offset(kind, K, N)));
    return hipGetLastError();
}

hipError_t launch_panel_decode(WeightKind kind, int K, int N, const void* panel, float scale, float* out,
                               hipStream_t st)
{
    if (K <= 0 || N <= 0 || K % 32 || (kind == W_I4 && N % 32)) return hipErrorInvalidValue;
    const unsigned char* P = static_cast<const unsigned char*>(panel);
    const float* ST = reinterpret_cast<const float*>(P + scales_offset(kind, K, N));
    const unsigned blocks = (unsigned)(((long long)K * N + 255) / 256);
    switch (kind) {
    case W_I8: hipLaunchKernelGGL(decode_panel<W_I8>, dim3(blocks), dim3(256), 0, st, K, N, P, ST, scale, out); break;
    case W_I4: hipLaunchKernelGGL(decode_panel<W_I4>, dim3(blocks), dim3(256), 0, st, K, N, P, ST, scale, out); break;
    default:   hipLaunchKernelGGL(decode_panel<W_F32>, dim3(blocks), dim3(256), 0, st, K, N, P, ST, scale, out); break;
    }
    return hipGetLastError();
}

bool panel_force_tiles(int mb, int nct)
{
    if (mb == 0 && nct == 0) { t_panel_mb = t_panel_nct = 0; return true; }
    if (mb < 1 || mb > 4 || nct < 1 || nct > 2) return false;
    t_panel_mb = mb;
    t_panel_nct = nct;
    return true;
}

// Whether a tile may take half phases: up to 3 row blocks, no fused input
// LayerNorm, and K already split over workgroups with whole phases (where
// the phases run in one launch, a split form costs a second launch that
// tile_cost does not model).
bool half_ok(const GemmProblem& p, int mb)
{
    return mb <= 3 && !p.ln_gamma && segments_for(p, std::min(p.M, 16 * mb)) > 1;
}

// The tile of a problem, or mb = 0 if no tile holds its rows; *half: its
// phases are of 512 k (K split over twice as many workgroups where whole
// phases leave CUs idle: i4 33 x 1024 x 4096 takes 3 row blocks in one
// row group and 8 segments, 256 workgroups, instead of 2 row groups of 2
// blocks that stream the weights twice).
void panel_choice(const GemmProblem& p, int* mb, int* nct, bool* half)
{
    const int MB = (p.M + 15) / 16;
    int b = 0, c = 1;
    bool hf = false;
    double best = 1e300;
    for (int cc = 1; cc <= 2; ++cc)
        for (int bb = 1; bb <= MB; ++bb) {
            if (!rows_fit(p, std::min(p.M, 16 * bb))) continue;
            if (p.ln_gamma && !ln_tile(p.kind, bb, cc)) continue;
            for (int h = 0; h < 2; ++h) {
                if (h && !half_ok(p, bb)) continue;
                const double t = tile_cost(p, bb, cc, h != 0);
                if (t < best - 1e-9) { best = t; b = bb; c = cc; hf = h != 0; }
            }
        }
    // PK_GPU_PANEL_TILE="MB,NCT" overrides the choice (tuning sweeps)
    static const std::pair<int, int> forced = [] {
        const char* e = getenv("PK_GPU_PANEL_TILE");
        int x = 0, y = 0;
        if (e && sscanf(e, "%d,%d", &x, &y) == 2 && x >= 1 && x <= 4 && y >= 1 && y <= 2)
            return std::make_pair(x, y);
        return std::make_pair(0, 0);
    }();
    int fb = forced.first, fc = forced.second;
    if (t_panel_mb) { fb = t_panel_mb; fc = t_panel_nct; }
    if (fb && rows_fit(p, std::min(p.M, 16 * std::min(fb, MB))) &&
        (!p.ln_gamma || ln_tile(p.kind, std::min(fb, MB), fc))) {
        b = std::min(fb, MB);
        c = fc;
        hf = half_ok(p, b) && tile_cost(p, b, c, true) < tile_cost(p, b, c, false);
    }
    *mb = b;
    *nct = c;
    *half = hf;
}

void panel_tile(const GemmProblem& p, int* mb, int* nct)
{
    bool half = false;
    panel_choice(p, mb, nct, &half);
}

int panel_segments(const GemmProblem& p)
{
    int mb = 1, nct = 1;
    bool half = false;
    panel_choice(p, &mb, &nct, &half);
    return mb ? segments_for(p, std::min(p.M, 16 * mb), half) : 1;
}

bool panel_fuses_out_ln(const GemmProblem& p)
{
    return panel_supports(p) && p.N <= kReduceLnMaxN && p.N % (8 * kLnChunk) == 0 && panel_segments(p) > 1;
}

int panel_phase_k(int rows) { return phase_k(rows, 0); }

bool panel_supports(const GemmProblem& p)
{
    if (!p.panel) return false;
    if (p.M < 1 || p.M > kSmallMaxM || p.N < 1 || p.K < 32 || p.K % 32) return false;
    if (p.chain_bias || p.a_presplit) return false;
    if (p.alpha == 0.0f || (p.kind == W_I8 && p.scale == 0.0f)) return false;   // beta-only step
    if (p.lda % 4 || reinterpret_cast<uintptr_t>(p.A) % 16) return false;
    if (p.kind == W_I4 && p.N % 32) return false;
    if (p.ln_gamma && (!p.ln_beta || p.K > 1024 || p.K % (8 * kLnChunk) || reinterpret_cast<uintptr_t>(p.ln_gamma) % 16 ||
                       reinterpret_cast<uintptr_t>(p.ln_beta) % 16))
        return false;
    int mb = 0, nct = 0;
    bool half = false;
    panel_choice(p, &mb, &nct, &half);
    if (!mb) return false;
    if (p.out_ln_gamma && !(p.N <= kReduceLnMaxN && p.N % (8 * kLnChunk) == 0 && p.out_ln_beta &&
                            segments_for(p, std::min(p.M, 16 * mb), half) > 1))
        return false;
    return true;
}

hipError_t launch_panel(const GemmProblem& p, hipStream_t st)
{
    if (!panel_supports(p)) return hipErrorNotSupported;
    PanelArgs a = {};
    a.M = p.M; a.N = p.N; a.K = p.K;
    a.alpha = p.kind == W_I8 ? p.alpha * p.scale : p.alpha;
    a.beta = p.beta;
    a.A = p.A; a.lda = p.lda;
    a.P = static_cast<const unsigned char*>(p.panel);
    a.ST = p.kind == W_I4 ? reinterpret_cast<const float*>(a.P + scales_offset(p.kind, p.K, p.N)) : nullptr;
    a.C = p.C; a.ldc = p.ldc;
    a.bias = p.bias; a.epi = p.epi;
    const size_t a_ext = ((size_t)(p.M - 1) * p.lda + p.K) * 4;
    const size_t p_ext = codes_bytes(p.kind, p.K, p.N);
    const size_t s_ext = p.kind == W_I4 ? (size_t)(p.N / 32) * p.K * 4 : 0;
    const size_t lim = (size_t)1 << 31;
    if (a_ext >= lim || p_ext >= lim || s_ext >= lim) return hipErrorNotSupported;
    a.a_bytes = (uint32_t)a_ext;
    a.p_bytes = (uint32_t)p_ext;
    a.s_bytes = (uint32_t)s_ext;
    int MB = 1, NCT = 1;
    bool half = false;
    panel_choice(p, &MB, &NCT, &half);
    a.kph = kph_of(p, std::min(p.M, 16 * MB), half);
    a.ln_g = p.ln_gamma;
    a.ln_b = p.ln_beta;
    const int segs = segments_for(p, std::min(p.M, 16 * MB), half);
    a.kseg = segs > 1 ? ((p.K / 32 + segs - 1) / segs) * 32 : p.K;
    const int z = (p.K + a.kseg - 1) / a.kseg;
    a.work = z > 1 ? p.work : nullptr;
    const int groups = (p.N + 16 * NCT - 1) / (16 * NCT);
    const dim3 grid((unsigned)(((groups + kXcd - 1) / kXcd) * kXcd), (unsigned)((p.M + 16 * MB - 1) / (16 * MB)),
                    (unsigned)z);
    switch (p.kind) {
    case W_I8: launch_wk<W_I8>(MB, NCT, half, a, grid, st); break;
    case W_I4: launch_wk<W_I4>(MB, NCT, half, a, grid, st); break;
    default:   launch_wk<W_F32>(MB, NCT, half, a, grid, st); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || z == 1) return e;
    if (p.out_ln_gamma) {
        if (p.N <= 1024)
            hipLaunchKernelGGL(panel_reduce_ln<4>, dim3((unsigned)p.M), dim3(256), 0, st, a, z, p.out_ln_gamma,
                               p.out_ln_beta);
        else
            hipLaunchKernelGGL(panel_reduce_ln<8>, dim3((unsigned)p.M), dim3(256), 0, st, a, z, p.out_ln_gamma,
                               p.out_ln_beta);
        return hipGetLastError();
    }
    const long long mn = (long long)p.M * p.N;
    hipLaunchKernelGGL(panel_reduce, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, st, a, z);
    return hipGetLastError();
}

}  // namespace pkgpu
