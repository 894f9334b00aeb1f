// pk_device_math.h - the elementwise functions of the conformer block, with
// every rounding fixed so that a CPU evaluating the same IEEE operations in
// the same order gets the same bits.
//
//   exp_poly   pk_exp_avx2 (tensor_ops.c:98-120) as the reference build
//              compiles it: clamp to [-87, 87], k = rint(x*log2e),
//              r = fma(-k, ln2, x), a degree-5 Horner polynomial in fmas,
//              times 2^k.  Used by softmax (tensor_ops.c:336-357).
//   swish_f    pk_swish (tensor_ops.c:367-389): e = exp_poly(-v),
//              s = 1 / (1 + e), y = v * s.  The source's division is an IEEE
//              division (_mm256_div_ps); only the reference's -ffast-math
//              code generation turns it into vrcpps plus a Newton step,
//              whose 12-bit seed table is specific to the CPU model.  Here
//              it is the IEEE division the source writes.  As compiled, the
//              reference also contracts 1 + y*2^k into one fma; that is
//              followed (y*2^k is exact unless it is subnormal).
//   expf_ieee  e^x rounded to float for GLU's expf (encoder.c:462) and
//              softmax's scalar tail (tensor_ops.c:349): range reduction
//              x = k*ln2 + r in double (ln2 split in two), the degree-12
//              Taylor polynomial of e^r in double fmas (truncation error
//              below 6e-17 for |r| <= ln2/2), scaled by 2^k, then one
//              rounding to float.  The double result is within about 2^-51
//              of e^x, so the float is the correctly rounded one except
//              where e^x lies that close to a rounding boundary.  The
//              reference takes glibc's expf here (vectorised to its libmvec
//              form by -ffast-math), which is off the correctly rounded
//              value by up to a few ulp on about half of all inputs; no
//              fixed sequence of IEEE operations reproduces it.
//
// All HIP code is built with -ffp-contract=off: nothing below is fused
// unless written as an fma.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace pkgpu {

// The operand split of the bf16 tolerance kernels: x = hi + lo + r with
// hi = bf16(x) and lo = bf16(x - hi), both rounded to nearest (x - hi is
// exact in fp32), for two values packed as bf16 pairs.  The split GEMM
// kernels and the producers that hand them pre-split activations share it,
// so both give the same bits.  The bf16 value is read back through a
// by-value function: a bit cast applied directly to an element of a bf16
// vector gave wrong bits with this compiler.
typedef float split_v2f __attribute__((ext_vector_type(2)));
typedef __bf16 split_v2bf __attribute__((ext_vector_type(2)));

__device__ inline float bf16_value(__bf16 h)
{
    return __uint_as_float((uint32_t)__builtin_bit_cast(unsigned short, h) << 16);
}

__device__ inline void split_bf16x2(float x0, float x1, uint32_t& hi, uint32_t& lo)
{
    const split_v2bf h = __builtin_convertvector((split_v2f){x0, x1}, split_v2bf);
    hi = __builtin_bit_cast(uint32_t, h);
    const split_v2bf l = __builtin_convertvector(
        (split_v2f){__fsub_rn(x0, bf16_value(h[0])), __fsub_rn(x1, bf16_value(h[1]))}, split_v2bf);
    lo = __builtin_bit_cast(uint32_t, l);
}

// ((p0+p4)+(p2+p6)) + ((p1+p5)+(p3+p7)) across the 8 lanes of an aligned
// lane group (pk_hsum_avx2, tensor_ops.c:126-134); every lane of the group
// gets the sum.  fl(a+b) == fl(b+a), so the xor partners give the same
// association on every lane.
__device__ inline float hsum8_lanes(float p)
{
    const float a = __fadd_rn(p, __shfl_xor(p, 4));
    const float b = __fadd_rn(a, __shfl_xor(a, 2));
    return __fadd_rn(b, __shfl_xor(b, 1));
}

// LayerNorm's statistics of one row of D floats (tensor_ops.c:150-185 as
// the x86 build computes them), for lane l (0..7) of an aligned 8-lane
// group: lane l sums the elements l, l+8, ... in order (one AVX2 lane), the
// partials are added as hsum8_lanes, mean = sum / D; then the squared
// deviations fl(x - mean) the same way through an fma chain, var = sum / D,
// inv = 1 / sqrtf(var + 1e-5) (correctly rounded '/' and sqrtf).  The
// normalised value is then fl(fl(fl(x - mean) * inv) * gamma + beta) (one
// fma).  row may be LDS or global memory.  D must be a multiple of 8 * CH:
// the lane's elements are read CH at a time into registers ahead of their
// chain of additions, so the reads do not wait one by one.
template <int CH>
__device__ inline void ln_row_stats(const float* row, int D, int l, float& mean, float& inv)
{
    float p = 0.0f;
    for (int i0 = 0; i0 < D; i0 += 8 * CH) {
        float v[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) v[c] = row[i0 + 8 * c + l];
#pragma unroll
        for (int c = 0; c < CH; ++c) p = __fadd_rn(p, v[c]);
    }
    mean = __fdiv_rn(hsum8_lanes(p), (float)D);
    float q = 0.0f;
    for (int i0 = 0; i0 < D; i0 += 8 * CH) {
        float v[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) v[c] = row[i0 + 8 * c + l];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const float d = __fsub_rn(v[c], mean);
            q = __fmaf_rn(d, d, q);
        }
    }
    const float var = __fdiv_rn(hsum8_lanes(q), (float)D);
    inv = 1.0f / sqrtf(__fadd_rn(var, 1e-5f));
}

// ln_row_stats with the loops over the row's CH-element pieces kept rolled
// (fewer registers); the same operations in the same order.
template <int CH>
__device__ inline void ln_row_stats_rolled(const float* row, int D, int l, float& mean, float& inv)
{
    float p = 0.0f;
#pragma unroll 1
    for (int i0 = 0; i0 < D; i0 += 8 * CH) {
        float v[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) v[c] = row[i0 + 8 * c + l];
#pragma unroll
        for (int c = 0; c < CH; ++c) p = __fadd_rn(p, v[c]);
    }
    mean = __fdiv_rn(hsum8_lanes(p), (float)D);
    float q = 0.0f;
#pragma unroll 1
    for (int i0 = 0; i0 < D; i0 += 8 * CH) {
        float v[CH];
#pragma unroll
        for (int c = 0; c < CH; ++c) v[c] = row[i0 + 8 * c + l];
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const float d = __fsub_rn(v[c], mean);
            q = __fmaf_rn(d, d, q);
        }
    }
    const float var = __fdiv_rn(hsum8_lanes(q), (float)D);
    inv = 1.0f / sqrtf(__fadd_rn(var, 1e-5f));
}

__device__ inline float exp_poly(float x)
{
    x = fminf(fmaxf(x, -87.0f), 87.0f);
    const float kf = __builtin_rintf(__fmul_rn(x, 1.44269504088896341f));
    const int ki = (int)kf;
    const float r = __fmaf_rn(-kf, 0.69314718055994529f, x);
    float y = 1.0f / 120.0f;
    y = __fmaf_rn(y, r, 1.0f / 24.0f);
    y = __fmaf_rn(y, r, 1.0f / 6.0f);
    y = __fmaf_rn(y, r, 0.5f);
    y = __fmaf_rn(y, r, 1.0f);
    y = __fmaf_rn(y, r, 1.0f);
    return __fmul_rn(y, __int_as_float((ki + 127) << 23));
}

// d = 1 + e lies in [1, e^87], so the division never meets a subnormal or
// an infinity.
__device__ inline float swish_f(float v)
{
    const float t = fminf(fmaxf(-v, -87.0f), 87.0f);
    const float kf = __builtin_rintf(__fmul_rn(t, 1.44269504088896341f));
    const int ki = (int)kf;
    const float r = __fmaf_rn(-kf, 0.69314718055994529f, t);
    float q = 1.0f / 120.0f;
    q = __fmaf_rn(q, r, 1.0f / 24.0f);
    q = __fmaf_rn(q, r, 1.0f / 6.0f);
    q = __fmaf_rn(q, r, 0.5f);
    q = __fmaf_rn(q, r, 1.0f);
    q = __fmaf_rn(q, r, 1.0f);
    const float p2 = __int_as_float((ki + 127) << 23);
    const float d = __fmaf_rn(q, p2, 1.0f);
    return __fmul_rn(__fdiv_rn(1.0f, d), v);
}

__device__ inline float expf_ieee(float x)
{
    if (!(x > -104.0f)) return x != x ? x : 0.0f;    // NaN stays NaN; e^x < 2^-150 rounds to +0
    if (x > 89.0f) return __builtin_inff();          // e^89 > FLT_MAX
    const double xd = (double)x;
    const double k = __builtin_rint(xd * 0x1.71547652b82fep+0);          // x / ln2
    double r = __builtin_fma(-k, 0x1.62e42fefa39efp-1, xd);               // ln2, high part
    r = __builtin_fma(-k, 0x1.abc9e3b39803fp-56, r);                      // ln2, low part
    double p = 0x1.1eed8eff8d898p-29;                                     // 1/12!
    p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);                       // 1/11!
    p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);                       // 1/10!
    p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);                       // 1/9!
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);                       // 1/8!
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);                       // 1/7!
    p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);                       // 1/6!
    p = __builtin_fma(p, r, 0x1.1111111111111p-7);                        // 1/5!
    p = __builtin_fma(p, r, 0x1.5555555555555p-5);                        // 1/4!
    p = __builtin_fma(p, r, 0x1.5555555555555p-3);                        // 1/3!
    p = __builtin_fma(p, r, 0.5);
    p = __builtin_fma(p, r, 1.0);
    p = __builtin_fma(p, r, 1.0);
    // 2^k with k in [-150, 128]: a normal double, so the product is exact
    const double s = __longlong_as_double((long long)((int64_t)k + 1023) << 52);
    return (float)(p * s);
}

}  // namespace pkgpu
