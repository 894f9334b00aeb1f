// pk_smallm.hip - weight GEMMs with few rows (M <= 64), streaming the
// weights once at the HBM's pace instead of running K-long exact chains.
//
// The exact kernels (pk_gemm_tiles.h) reproduce the reference's sequential
// fma chain over k for every output, so a GEMM can finish no sooner than K
// dependent MFMA steps: about 10 us at K = 1024, whatever M is.  At M <= 64
// (the fused QKV of a 2.56 s clip has M = 33, cblas_sgemm_qb, blas.c:759-771,
// called from encoder.c:312) that floor is 5-10x the time the weights take to
// stream.  These kernels take the tolerance path instead: the products are the
// reference's (fp32 activations times the dequantised weight), summed in
// another order, within max |C - R| / max |R| <= 1e-3 of the reference (the
// measured error is about 1e-5).
//
// Arithmetic.  v_mfma_f32_16x16x32_bf16 with an fp32 accumulator.  Every
// fp32 operand x is split as x = hi + lo + r with hi = bf16(x), lo =
// bf16(x - hi), both rounded to nearest: x - hi is exact in fp32 and |r| <=
// 2^-16 |x|, and bf16 keeps fp32's exponent range, so no prescaling is needed.
//   int8: the codes q are exact in bf16; C = alpha*s * (A_hi Q + A_lo Q)
//         (2 MFMAs per tile), s the per-tensor scale.
//   int4: the codes q are exact in bf16 and a workgroup's columns share one
//         scale group, so the scale folds into the activations: A' =
//         fl(A * s[k][n/32]) (the products of blas.c:834-840's dequantised
//         weight fl(q*s) with A differ from fl(A*s)*q by one rounding of
//         2^-24), C = alpha * (A'_hi Q + A'_lo Q).
//   fp32: B = B_hi + B_lo as well; C = alpha * (A_hi B_hi + A_lo B_hi +
//         A_hi B_lo) (3 MFMAs; the dropped A_lo B_lo term is below 2^-16).
// The activations are never quantised: they stay fp32-valued to 16 bits.
//
// Work split: see the narrow-tile kernel below.  Every workgroup sums all of
// K for its tile, in a fixed order, so results are deterministic and no
// partial sums leave the workgroup.
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

struct SmArgs {
    int M, N, K;
    float alpha;               // int8: alpha * scale
    float beta;
    const float* A; int lda;
    const void* B; int ldb;    // row pitch in elements (int4: bytes)
    const float* scales; int n_groups;
    float* C; int ldc;
    const float* bias; int epi;
    uint32_t a_bytes, b_bytes, s_bytes;   // buffer extents (reads past them return 0)
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

__device__ inline float bf_to_f(__bf16 h) { return __uint_as_float((uint32_t)__builtin_bit_cast(unsigned short, h) << 16); }

// x (8 fp32) -> hi = bf16(x), lo = bf16(x - hi), both to nearest.
__device__ inline void split8(const float (&x)[8], v8bf& hi, v8bf& lo)
{
    v2bf h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        h[e] = to_bf2(x[2 * e], x[2 * e + 1]);
        l[e] = to_bf2(__fsub_rn(x[2 * e], bf_to_f(h[e][0])), __fsub_rn(x[2 * e + 1], bf_to_f(h[e][1])));
    }
    hi = cat(h[0], h[1], h[2], h[3]);
    lo = cat(l[0], l[1], l[2], l[3]);
}

__device__ inline v4f mfma(v8bf a, v8bf b, v4f c)
{
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Signed nibble j (0: low, 1: high) of byte b.
__device__ inline int q_i4(uint32_t b, int j)
{
    return (int)(b << (28 - 4 * j)) >> 28;          // low nibble = even column
}

// ---- narrow tiles: all of K per workgroup, no partials --------------------
// A workgroup of 16 waves owns NCT 16-column tiles and RB 16-row blocks and
// the whole k range: wave w takes the k steps [w*ns/16, (w+1)*ns/16) of the
// ns = K/32 steps, kChunk steps at a time.  Per chunk a wave copies the RW
// bytes of each of its rows that hold the tile's 16*NCT columns into its own
// LDS slab with U-byte loads (U = 16 where the weights are 16-byte aligned),
// and lane (i, g) then reads column 16ct + i of rows 8g .. 8g + 7 of each
// step from the slab, which is the MFMA operand layout.  Chunk row r =
// 32st + 8g + e lives in slab slot 32st + 4e + g, so the 64 lanes of one read
// touch 4 consecutive slots (distinct banks).  The next chunk's loads are
// issued before the current chunk's MFMAs.  The 16*NCT columns of an int4
// workgroup lie in one 32-column scale group, so the scale folds into the
// activations (A' = fl(A * s[k][g]), then split) and the codes enter the
// MFMA exactly.  The 16 waves' partial tiles are summed in LDS in wave order,
// then the epilogue.  Row blocks beyond RB go to more workgroups (grid.y);
// the workgroups of one column tile sit on one XCD, sharing its L2.
constexpr int kNW = 16;                 // waves per narrow workgroup
constexpr int kChunk = 2;               // k steps per chunk

template <int WK, int NCT> struct Narrow {
    static constexpr int RW = (WK == W_I8 ? 16 : WK == W_I4 ? 8 : 64) * NCT;   // row bytes
    static constexpr int SLAB = 32 * kChunk * RW;                             // bytes per wave
    static constexpr int SSLAB = WK == W_I4 ? 32 * kChunk * 4 : 0;            // scales per wave
};

template <int N> struct UnitT;
template <> struct UnitT<4> { typedef uint32_t T; };
template <> struct UnitT<8> { typedef v2u T; };
template <> struct UnitT<16> { typedef v4u T; };

template <int U>
__device__ inline typename UnitT<U>::T load_unit(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    if constexpr (U == 16) return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
    else if constexpr (U == 8) return __builtin_amdgcn_raw_buffer_load_b64(r, (int)off, 0, 0);
    else return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}

// Whether a tile's k steps get load instructions of their own (SPLIT: units
// of at most half a row, so a step's multiplies start when its own loads are
// in) or share them (units of up to a whole row: fewer, wider loads, both
// steps written to LDS after one wait), measured per format and width.
constexpr bool split_steps(int WK, int NCT) { return !(NCT == 1 && WK != W_F32); }

template <int WK, int RB, int NCT, int UB, bool SPLIT = split_steps(WK, NCT)>
__global__ __launch_bounds__(64 * kNW) void smallm_narrow(SmArgs p)
{
    typedef Narrow<WK, NCT> L;
    constexpr int RW = L::RW;
    // load unit; with SPLIT at most half a row, so units j of step st are
    // [st * NUS, (st + 1) * NUS)
    constexpr int UMAX = SPLIT ? RW / 2 : RW;
    constexpr int U = UB < UMAX ? UB : UMAX;
    constexpr int UPR = RW / U;                     // units per row
    constexpr int NU = 32 * kChunk * UPR / 64;      // units per lane per chunk
    constexpr int NUS = SPLIT ? NU / kChunk : NU;   // units written before step 0 (all without SPLIT)
    constexpr int STAGE = kNW * (L::SLAB + L::SSLAB);
    constexpr int RED = kNW * RB * NCT * 64 * 16;
    // two register sets (chunk c + 1's loads in flight while c is multiplied)
    // where the registers allow (no spills); otherwise the next chunk's loads
    // follow its multiplies
    constexpr int NB = (RB * NCT <= 2 && !(WK == W_F32 && RB > 1)) ? 2 : 1;
    typedef typename UnitT<U>::T Unit;
    static_assert(!SPLIT || (UPR % 2 == 0 && NU % kChunk == 0), "whole units per step");
    __shared__ __attribute__((aligned(16))) unsigned char smem[STAGE > RED ? STAGE : RED];

    // column tiles in XCD-sized runs (workgroups reach the XCDs round-robin)
    const int x = blockIdx.x, per = gridDim.x / kXcd;
    const int t = (x % kXcd) * per + x / kXcd;
    if (t * 16 * NCT >= p.N) return;                // padding workgroup (uniform)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane & 15, g = lane >> 4;
    const int c0 = t * 16 * NCT;
    const int m0 = 16 * RB * blockIdx.y;
    const int ns = p.K / 32, s0 = wave * ns / kNW, s1 = (wave + 1) * ns / kNW;

    const auto rA = rsrc(p.A, p.a_bytes), rB = rsrc(p.B, p.b_bytes);
    const auto rS = rsrc(p.scales, p.s_bytes);
    const uint32_t ldb_bytes = (uint32_t)p.ldb * (WK == W_F32 ? 4u : 1u);
    const uint32_t c0_bytes = WK == W_F32 ? 4u * c0 : WK == W_I8 ? (uint32_t)c0 : (uint32_t)c0 / 2;
    const uint32_t grp = (uint32_t)c0 >> 5;
    unsigned char* slab = smem + wave * L::SLAB;
    float* sslab = reinterpret_cast<float*>(smem + kNW * L::SLAB) + wave * (32 * kChunk);

    Unit wu[NB][NU];
    float sc[NB];
    v4u ar[NB][kChunk][RB][2];

    // every global load of chunk `cs` into register set b: step 0's first
    auto issue = [&](int b, int cs) {
        const int steps = min(kChunk, s1 - cs);
#pragma unroll
        for (int st = 0; st < kChunk; ++st) {
            if (st >= steps) break;                  // uniform per wave
#pragma unroll
            for (int jj = 0; jj < NUS; ++jj) {
                if (!SPLIT && st > 0) break;
                const int j = (SPLIT ? st * NUS : 0) + jj;
                const int u = lane + 64 * j, r = u / UPR, part = u % UPR;
                if (r < 32 * steps)
                    wu[b][j] = load_unit<U>(rB, (uint32_t)(32 * cs + r) * ldb_bytes + c0_bytes + (uint32_t)(part * U));
            }
            if constexpr (WK == W_I4) {
                if (st == 0 && lane < 32 * steps)
                    sc[b] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                        rS, (int)(((uint32_t)(32 * cs + lane) * (uint32_t)p.n_groups + grp) * 4u), 0, 0));
            }
            const int k0 = 32 * (cs + st);
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                // row m0 + 16rb + i, k0 + 8g .. +7: rows >= M read 0 (past the extent)
                const uint32_t off = ((uint32_t)(m0 + 16 * rb + i) * (uint32_t)p.lda + (uint32_t)(k0 + 8 * g)) * 4u;
                ar[b][st][rb][0] = __builtin_amdgcn_raw_buffer_load_b128(rA, (int)off, 0, 0);
                ar[b][st][rb][1] = __builtin_amdgcn_raw_buffer_load_b128(rA, (int)(off + 16), 0, 0);
            }
            // keep step st's loads ahead of the next step's: the wait before a
            // step's multiplies then leaves the later steps' loads in flight
            __builtin_amdgcn_sched_barrier(0);
        }
    };

    v4f acc[RB][NCT];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) acc[rb][ct] = v4f{0.f, 0.f, 0.f, 0.f};

    // multiply chunk `cs` from register set b, one step at a time: each step's
    // weights go to the slab (slot 32st + 4e + g for row 32st + 8g + e) as
    // soon as that step's loads are in
    auto process = [&](int b, int cs) {
        const int steps = min(kChunk, s1 - cs);
        if constexpr (WK == W_I4) {
            if (lane < 32 * steps) sslab[lane] = sc[b];
        }
#pragma unroll
        for (int st = 0; st < kChunk; ++st) {
            if (st >= steps) break;                  // uniform per wave
#pragma unroll
            for (int jj = 0; jj < NUS; ++jj) {
                if (!SPLIT && st > 0) break;
                const int j = (SPLIT ? st * NUS : 0) + jj;
                const int u = lane + 64 * j, r = u / UPR, part = u % UPR;
                const int slot = (r & ~31) | ((r & 7) << 2) | ((r >> 3) & 3);
                if (r < 32 * steps) *reinterpret_cast<Unit*>(slab + slot * RW + part * U) = wu[b][j];
            }
            // the wave's own LDS writes complete before its reads (LDS keeps a wave's order)
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            v8bf bhi[NCT], blo[NCT];
#pragma unroll
            for (int ct = 0; ct < NCT; ++ct) {
                float wv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const unsigned char* row = slab + (32 * st + 4 * e + g) * RW;
                    const int col = 16 * ct + i;
                    if constexpr (WK == W_I8) wv[e] = (float)(signed char)row[col];
                    else if constexpr (WK == W_I4) wv[e] = (float)q_i4(row[col >> 1], col & 1);
                    else wv[e] = reinterpret_cast<const float*>(row)[col];
                }
                if constexpr (WK == W_F32) {
                    split8(wv, bhi[ct], blo[ct]);
                } else {
                    bhi[ct] = cat(to_bf2(wv[0], wv[1]), to_bf2(wv[2], wv[3]),
                                  to_bf2(wv[4], wv[5]), to_bf2(wv[6], wv[7]));   // exact
                }
            }
            float sv[8];
            if constexpr (WK == W_I4) {
                const v4f s_lo = *reinterpret_cast<const v4f*>(sslab + 32 * st + 8 * g);
                const v4f s_hi = *reinterpret_cast<const v4f*>(sslab + 32 * st + 8 * g + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) { sv[e] = s_lo[e]; sv[4 + e] = s_hi[e]; }
            }
#pragma unroll
            for (int rb = 0; rb < RB; ++rb) {
                const v4u a0 = ar[b][st][rb][0], a1 = ar[b][st][rb][1];
                float xa[8] = {__uint_as_float(a0[0]), __uint_as_float(a0[1]), __uint_as_float(a0[2]),
                               __uint_as_float(a0[3]), __uint_as_float(a1[0]), __uint_as_float(a1[1]),
                               __uint_as_float(a1[2]), __uint_as_float(a1[3])};
                if constexpr (WK == W_I4) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) xa[e] = __fmul_rn(xa[e], sv[e]);
                }
                v8bf ahi, alo;
                split8(xa, ahi, alo);
#pragma unroll
                for (int ct = 0; ct < NCT; ++ct) {
                    acc[rb][ct] = mfma(ahi, bhi[ct], acc[rb][ct]);
                    acc[rb][ct] = mfma(alo, bhi[ct], acc[rb][ct]);
                    if constexpr (WK == W_F32) acc[rb][ct] = mfma(ahi, blo[ct], acc[rb][ct]);
                }
            }
        }
        // this chunk's slab reads are done before the next chunk overwrites it
        __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    };

    if (s0 < s1) issue(0, s0);
    if constexpr (NB == 2) {
        for (int cs = s0; cs < s1; cs += 2 * kChunk) {
            if (cs + kChunk < s1) issue(1, cs + kChunk);
            process(0, cs);
            if (cs + kChunk >= s1) break;
            if (cs + 2 * kChunk < s1) issue(0, cs + 2 * kChunk);
            process(1, cs + kChunk);
        }
    } else {
        for (int cs = s0; cs < s1; cs += kChunk) {
            process(0, cs);
            if (cs + kChunk < s1) issue(0, cs + kChunk);
        }
    }

    // fixed-order sum over the waves, one output per thread
    __syncthreads();                                 // every slab read done: reuse as `red`
    v4f* red = reinterpret_cast<v4f*>(smem);         // [kNW][RB][NCT][64]
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int ct = 0; ct < NCT; ++ct) red[((wave * RB + rb) * NCT + ct) * 64 + lane] = acc[rb][ct];
    __syncthreads();
    const int o = threadIdx.x;                       // output (rb, ct, lane l, v)
    if (o >= RB * NCT * 256) return;
    const int rb = o / (NCT * 256), ct = (o >> 8) % NCT, l = (o >> 2) & 63, v = o & 3;
    const float* rf = reinterpret_cast<const float*>(red);
    float sum = rf[((rb * NCT + ct) * 64 + l) * 4 + v];
#pragma unroll
    for (int w = 1; w < kNW; ++w) sum = __fadd_rn(sum, rf[(((w * RB + rb) * NCT + ct) * 64 + l) * 4 + v]);
    const int m = m0 + 16 * rb + 4 * (l >> 4) + v, n = c0 + 16 * ct + (l & 15);
    if (m >= p.M || n >= p.N) return;
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

template <int WK, int RB, int NCT>
hipError_t launch_narrow_t(const SmArgs& a, int ub, hipStream_t st)
{
    const int tiles = (a.N + 16 * NCT - 1) / (16 * NCT);
    const int RBs = (a.M + 15) / 16;
    const dim3 grid((unsigned)(((tiles + kXcd - 1) / kXcd) * kXcd), (unsigned)((RBs + RB - 1) / RB));
    if constexpr (WK == W_I8) {
        if (ub == 4) {
            hipLaunchKernelGGL((smallm_narrow<WK, RB, NCT, 4>), grid, dim3(64 * kNW), 0, st, a);
            return hipGetLastError();
        }
    }
    if (ub != 16) return hipErrorNotSupported;
    hipLaunchKernelGGL((smallm_narrow<WK, RB, NCT, 16>), grid, dim3(64 * kNW), 0, st, a);
    return hipGetLastError();
}

// (RB, NCT) in {1..4} x {1} and {1, 2} x {2} for int8 / int4; fp32 takes
// NCT = 1 and RB <= 3 (its 64-byte rows need the registers).
template <int WK>
hipError_t launch_narrow(int RB, int NCT, int ub, const SmArgs& a, hipStream_t st)
{
    if constexpr (WK == W_F32) {
        switch (RB) {
        case 1: return launch_narrow_t<WK, 1, 1>(a, ub, st);
        case 2: return launch_narrow_t<WK, 2, 1>(a, ub, st);
        default: return launch_narrow_t<WK, 3, 1>(a, ub, st);
        }
    } else {
        if (NCT == 2) return RB == 1 ? launch_narrow_t<WK, 1, 2>(a, ub, st) : launch_narrow_t<WK, 2, 2>(a, ub, st);
        switch (RB) {
        case 1: return launch_narrow_t<WK, 1, 1>(a, ub, st);
        case 2: return launch_narrow_t<WK, 2, 1>(a, ub, st);
        case 3: return launch_narrow_t<WK, 3, 1>(a, ub, st);
        default: return launch_narrow_t<WK, 4, 1>(a, ub, st);
        }
    }
}

}  // namespace

namespace {

// Bytes of one load unit for the weight rows: 16 where rows and base are
// 16-byte aligned, else (int8 only) 4 where they are dword aligned; 0 if
// neither.
int narrow_unit(const GemmProblem& p)
{
    const size_t pitch = (size_t)p.ldb * (p.kind == W_F32 ? 4 : 1);
    const uintptr_t pb = reinterpret_cast<uintptr_t>(p.B);
    if (pitch % 16 == 0 && pb % 16 == 0) return 16;
    if (p.kind == W_I8 && pitch % 4 == 0 && pb % 4 == 0) return 4;
    return 0;
}

// Modelled cycles of the slowest CU: the workgroups (one per CU at a time)
// run in rounds of 256 (a partial round costs 4x its fraction, at most a
// whole one: a few extra workgroups start while the first round drains, as
// measured); a workgroup's time is its L1 bytes at 64 B/clk plus its VALU
// lane operations at 64 per clock (activation split ~3 per value, weight
// conversion 1.5 (int8), 2.5 (int4), 4.5 (fp32, split too)).  It picks the
// fastest measured tile for the encoder's M = 33 shapes and for M = 1, 16,
// 32, 64 at K = 1024.
double narrow_cost(const GemmProblem& p, int RB, int NCT)
{
    const int MB = (p.M + 15) / 16;
    const int groups = (MB + RB - 1) / RB, tiles = (p.N + 16 * NCT - 1) / (16 * NCT);
    const double r = (double)groups * tiles / 256.0, whole = std::floor(r);
    const double rounds = std::max(1.0, whole + std::min(1.0, 4.0 * (r - whole)));
    const double rw = (p.kind == W_I8 ? 16.0 : p.kind == W_I4 ? 8.0 : 64.0) * NCT;
    const double bytes = RB * 16.0 * p.K * 4 + p.K * rw + (p.kind == W_I4 ? p.K * 4.0 : 0.0);
    const double conv = p.kind == W_I8 ? 1.5 : p.kind == W_I4 ? 2.5 : 4.5;
    const double valu = RB * 16.0 * p.K * (p.kind == W_I4 ? 4.0 : 3.0) + p.K * 16.0 * NCT * conv;
    return rounds * (bytes / 64.0 + valu / 64.0);
}

}  // namespace

bool smallm_supports(const GemmProblem& p)
{
    if (p.M < 1 || p.M > kSmallMaxM || p.N < 1 || p.K < 32 || p.K % 32) return false;
    if (p.chain_bias) return false;
    if (p.alpha == 0.0f || (p.kind == W_I8 && p.scale == 0.0f)) return false;   // beta-only step
    const uintptr_t pa = reinterpret_cast<uintptr_t>(p.A);
    if (p.lda % 4 || pa % 16) return false;
    if (!narrow_unit(p)) return false;
    if (p.kind == W_I4)
        return p.N % 32 == 0 && reinterpret_cast<uintptr_t>(p.scales) % 4 == 0;
    return true;
}

namespace {
thread_local int t_tile_rb = 0, t_tile_nct = 0;     // forced tile of this thread (0: none)

bool tile_ok(WeightKind kind, int rb, int nct)
{
    if (rb < 1 || rb > 4 || nct < 1 || nct > 2 || rb * nct > 4) return false;
    return kind != W_F32 || (nct == 1 && rb <= 3);
}
}  // namespace

bool smallm_force_tile(int rb, int nct)
{
    if (rb == 0 && nct == 0) { t_tile_rb = t_tile_nct = 0; return true; }
    if (!tile_ok(W_I8, rb, nct)) return false;
    t_tile_rb = rb;
    t_tile_nct = nct;
    return true;
}

void smallm_tile(const GemmProblem& p, int* rb_out, int* nct_out)
{
    // PK_GPU_SMALLM_TILE="RB,NCT" overrides the modelled choice (tuning sweeps)
    static const std::pair<int, int> forced = [] {
        const char* e = getenv("PK_GPU_SMALLM_TILE");
        int rb = 0, nct = 0;
        if (e && sscanf(e, "%d,%d", &rb, &nct) == 2) return std::make_pair(rb, nct);
        return std::make_pair(0, 0);
    }();
    const int MB = (p.M + 15) / 16;
    int best_rb = 1, best_nct = 1;
    double best = 1e300;
    for (int nct = 1; nct <= (p.kind == W_F32 ? 1 : 2); ++nct)
        for (int rb = 1; rb <= std::min(MB, nct == 2 ? 2 : p.kind == W_F32 ? 3 : 4); ++rb) {
            const double c = narrow_cost(p, rb, nct);
            if (c < best) { best = c; best_rb = rb; best_nct = nct; }
        }
    if (tile_ok(p.kind, forced.first, forced.second)) {
        best_rb = forced.first;
        best_nct = forced.second;
    }
    if (t_tile_rb) {                                 // the thread's forced tile (fp32: nct 1, rb <= 3)
        best_rb = p.kind == W_F32 ? std::min(t_tile_rb, 3) : t_tile_rb;
        best_nct = p.kind == W_F32 ? 1 : t_tile_nct;
    }
    *rb_out = best_rb;
    *nct_out = best_nct;
}

static bool smallm_args(const GemmProblem& p, SmArgs* out)
{
    SmArgs a = {};
    a.M = p.M; a.N = p.N; a.K = p.K;
    a.alpha = p.kind == W_I8 ? p.alpha * p.scale : p.alpha;
    a.beta = p.beta;
    a.A = p.A; a.lda = p.lda;
    a.B = p.B; a.ldb = p.ldb;
    a.scales = p.scales; a.n_groups = p.N / 32;
    a.C = p.C; a.ldc = p.ldc;
    a.bias = p.bias; a.epi = p.epi;
    const size_t b_row = p.kind == W_I4 ? (size_t)p.N / 2 : (size_t)p.N;
    const size_t a_ext = ((size_t)(p.M - 1) * p.lda + p.K) * 4;
    const size_t b_ext = ((size_t)(p.K - 1) * p.ldb + b_row) * (p.kind == W_F32 ? 4 : 1);
    const size_t s_ext = p.kind == W_I4 ? (size_t)p.K * (p.N / 32) * 4 : 0;
    const size_t lim = (size_t)1 << 31;
    if (a_ext >= lim || b_ext >= lim || s_ext >= lim) return false;
    a.a_bytes = (uint32_t)a_ext;
    a.b_bytes = (uint32_t)b_ext;
    a.s_bytes = (uint32_t)s_ext;
    *out = a;
    return true;
}

hipError_t launch_smallm(const GemmProblem& p, hipStream_t st)
{
    if (!smallm_supports(p)) return hipErrorNotSupported;
    SmArgs a;
    if (!smallm_args(p, &a)) return hipErrorNotSupported;
    int RB = 1, NCT = 1;
    smallm_tile(p, &RB, &NCT);
    const int ub = narrow_unit(p);
    switch (p.kind) {
    case W_I8: return launch_narrow<W_I8>(RB, NCT, ub, a, st);
    case W_I4: return launch_narrow<W_I4>(RB, NCT, ub, a, st);
    default:   return launch_narrow<W_F32>(RB, NCT, ub, a, st);
    }
}

}  // namespace pkgpu
