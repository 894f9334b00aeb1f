// pk_split.hip - weight GEMMs of any M on bf16 matrix cores with split
// operands: the fast numerics mode (PK_GPU_NUMERICS_FAST).
//
// The exact kernels (pk_gemm_tiles.h) reproduce the reference's sequential
// fma chain over k for every output (blas.c:198-208), which holds them to
// the fp32 MFMA instructions (157.3 TFLOP/s dense).  Within the GEMM
// contract max |C - R| / max |R| <= 1e-3 the same products can go through
// v_mfma_f32_32x32x16_bf16 instead (2.5 PFLOP/s dense), with every fp32
// operand x split as x = hi + lo + r, hi = bf16(x), lo = bf16(x - hi), both
// to nearest: x - hi is exact in fp32, |r| <= 2^-16 |x|, and bf16 keeps
// fp32's exponent range, so nothing is prescaled.  The accumulators are fp32.
//   int8: the codes q are exact in bf16 and the scale is per tensor:
//         C = alpha*s * (A_hi Q + A_lo Q)                    (2 MFMAs)
//   int4: each weight is first dequantised exactly as the reference's pack
//         step does, w = fl(q * s[k][n/32]) (blas.c:794, 834-840), then split:
//         C = alpha * (A_hi W_hi + A_lo W_hi + A_hi W_lo)    (3 MFMAs)
//   fp32: the weight split the same way                      (3 MFMAs)
// The dropped A_lo W_lo term and the operands' residues r are below 2^-16 of
// each product; the measured error is about 1e-5.
//
// Staging (Pipe).  K goes in 32-deep chunks.  Per chunk, every thread loads
// its share of the A rows (16-byte loads) and of the weight rows (4 or 16
// bytes per unit, two consecutive k rows per unit), splits them, and writes
// them to LDS as planes [row or column][k] of bf16 with a padded stride of
// 40, so the MFMA operands (8 consecutive k of one row or column per lane)
// are single 16-byte LDS reads.  Loads run 1-3 chunks ahead in registers.
// Each wave computes a 64 x 64 block of C as 2 x 2 MFMA blocks of 32 x 32.
//
// Launch shapes (split_shape):
//   split_gemm    workgroups of WM x WN waves own (64 WM) x (64 WN) tiles
//                 (128 x 128 or 128 x 64 where that still gives every CU a
//                 workgroup, else 64 x 64) over all of K, two LDS buffers;
//   split_gemm_k  for shapes with too few such tiles (N = 1024 at 1656 rows):
//                 64 x 64 tiles, K split over 4 waves with an LDS slab each,
//                 the 4 partial tiles summed in LDS in wave order;
//   split-K       where the caller gives a workspace (GemmProblem::work),
//                 those shapes instead run 256 x 128 or 128 x 128 tiles with
//                 K split over workgroups (split_gemm<..., SK = true>), each
//                 storing its raw partial tile, and split_reduce sums each
//                 tile's partials in segment order before the epilogue.
// Every sum has a fixed order, so results are deterministic; without a
// workspace no memory beyond the operands is used.
#include "pk_gemm_kernels.h"
#include "pk_device_math.h"

#include <algorithm>
#include <cmath>
#include <cstdlib>
#include <cstring>

namespace pkgpu {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kXcd = 8;
constexpr int KT = 32;            // k per chunk
constexpr int RS = KT + 8;        // LDS row stride of a plane, in bf16 (80 bytes)
// Lo planes start kGap bf16 (64 bytes, 16 banks) past the end of their hi
// plane, so 16-byte stores of the hi and the lo half of one row or column in
// one access phase land on distinct banks; not where those 128 bytes per
// buffer would cost a workgroup per CU (Pipe::GAP).
constexpr int kGap = 32;
constexpr int kCuLds = 163840;    // LDS bytes per CU
// Pipe's weight format for weights given pre-split (GemmProblem::b_presplit,
// int4 and fp32): per 32-deep chunk c and column n, 128 bytes at
// (c N + n) * 128: the 32 bf16 hi = bf16(w) of k = 32 c .. 32 c + 31, then
// the 32 lo = bf16(w - hi), w the weight the kernels otherwise split
// (fl(q * s) for int4), so staging a chunk is a copy.
constexpr int W_BS = 3;
// The same for int8 weights (GemmProblem::b_presplit of an int8 B): per
// chunk c and column n, 64 bytes at (c N + n) * 64, the 32 codes of k = 32 c
// .. 32 c + 31 as bf16 (exact), so the int8 GEMMs stage a chunk with 16-byte
// copies instead of 4-byte loads of 32 rows and conversions.
constexpr int W_BS8 = 4;

struct SpArgs {
    int M, N, K;
    float alpha;                  // int8: alpha * scale
    float beta;
    const float* A; int lda;
    const void* B; int ldb;       // row pitch in elements (int4: bytes)
    const float* scales; int n_groups;
    float* C; int ldc;
    const float* bias; int epi;
    uint32_t a_bytes, b_bytes, s_bytes;   // buffer extents (reads past them return 0)
    int tiles_n, tiles;           // column tiles, workgroups (tiles x segments)
    // K split over workgroups: n_seg segments of the n_tiles tiles, partial
    // tiles in work (n_seg = 1: none)
    int n_seg, n_tiles;
    float* work;
    int c_vec4;                   // C rows and the bias allow 16-byte accesses (split_reduce)
    // > 0: the partial tiles go to work row-major instead, [n_seg][work_rows][N]
    // (work_rows: the row tiles' rows), for split_reduce_ln
    int work_rows;
};

// LayerNorms formed by split_reduce_ln on the finished rows: out_g, out_b
// replace C's rows by their LayerNorm (or null); next_g, next_b write the
// LayerNorm of the rows C ends with to next_out, pre-split (or null).
struct SpLn {
    const float *out_g, *out_b;
    const float *next_g, *next_b;
    float* next_out;
};

__device__ inline __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

__device__ inline v2bf to_bf2(float a, float b) { return __builtin_convertvector((v2f){a, b}, v2bf); }

__device__ inline uint32_t bits2(v2bf v) { return __builtin_bit_cast(uint32_t, v); }

// (x0, x1) -> hi = bf16 pair, lo = bf16 pair of the residues
__device__ inline void split2(float x0, float x1, uint32_t& hi, uint32_t& lo)
{
    split_bf16x2(x0, x1, hi, lo);
}

// Signed nibble j (0: low, 1: high) of byte b.
__device__ inline int q_i4(uint32_t w, int j)
{
    return (int)(w << (28 - 4 * j)) >> 28;
}

// The A row that 8-lane group g stages: groups 2j and 2j + 1 (one 16-lane
// phase of an 8-byte LDS store) take rows 4 apart within each block of 8, so
// their 64-byte runs at the 80-byte row pitch land 16 banks apart instead of
// overlapping by 4.
__device__ inline int a_row(int g)
{
    return (g & ~7) + ((g & 1) << 2) + ((g >> 1) & 3);
}

template <int WK> struct WUnit;
template <> struct WUnit<W_I8> { uint32_t q[2]; };
template <> struct WUnit<W_I4> { uint32_t q[2]; float s[2]; };
template <> struct WUnit<W_F32> { v4u w[2]; };
template <> struct WUnit<W_BS> { v4u w; };
template <> struct WUnit<W_BS8> { v4u w; };

// Staging and multiplying one chunk of a BM x BN tile by NT threads.
// A chunk's LDS planes: A_hi, A_lo [BM][RS], then W_hi (and W_lo) [BN][RS].
// AS: A comes pre-split by its producer (GemmProblem::a_presplit: per row and
// 8 consecutive k, the 8 bf16 hi then the 8 bf16 lo, so a row takes the bytes
// and the pitch of the fp32 row), and staging it is a copy.
template <int WK, int BM, int BN, int NT, bool AS>
struct Pipe {
    static constexpr int NBP = WK == W_I8 || WK == W_BS8 ? 1 : 2;   // weight planes
    static constexpr int A_PLANE = BM * RS, B_PLANE = BN * RS;   // bf16 elements
    // two buffers per workgroup: the gaps only where they keep as many
    // workgroups per CU (the 128 x 128 tiles fill 160 KB exactly without)
    static constexpr int BYTES0 = 2 * 2 * (2 * A_PLANE + NBP * B_PLANE);
    static constexpr int GAP = kCuLds / (BYTES0 + 2 * 2 * NBP * kGap) == kCuLds / BYTES0 ? kGap : 0;
    // plane offsets in one chunk's buffer (the lo planes GAP past their hi plane)
    static constexpr int A_LO = A_PLANE + GAP, B_HI = A_LO + A_PLANE, B_LO = B_HI + B_PLANE + GAP;
    static constexpr int BUF = B_HI + NBP * B_PLANE + (NBP - 1) * GAP;   // one chunk
    // A: BM rows x 8 float4 per chunk
    static constexpr int A_ITEMS = BM * (KT / 4) / NT;
    // weight units of two consecutive k rows: 4 columns (int8, fp32) or 8
    // (int4); pre-split weights: 16-byte pieces, 8 per column (int8: 4)
    static constexpr int UC = WK == W_I4 ? 8 : 4;
    static constexpr int B_TOTAL = WK == W_BS ? 8 * BN : WK == W_BS8 ? 4 * BN : (KT / 2) * (BN / UC);
    static constexpr int B_ITEMS = (B_TOTAL + NT - 1) / NT;     // the last one partial if NT > B_TOTAL
    static_assert(A_ITEMS * NT == BM * (KT / 4) && (B_TOTAL % NT == 0 || B_TOTAL < NT), "even split");
    static_assert(B_TOTAL % 64 == 0, "whole waves per weight item");

    struct Raw {
        v4u a[A_ITEMS];
        WUnit<WK> w[B_ITEMS];
    };

    // the global loads of the chunk at k0 (rows past M, columns past the
    // operands' extents read 0; columns past N only feed unstored outputs)
    // (the same 16-byte loads with or without AS: 4 k of fp32, or the hi or
    // the lo half of 8 pre-split k)
    __device__ static void load(Raw& r, const SpArgs& p, __amdgpu_buffer_rsrc_t rA,
                                __amdgpu_buffer_rsrc_t rB, __amdgpu_buffer_rsrc_t rS, int tid,
                                int m0, int n0, int k0)
    {
#pragma unroll
        for (int i = 0; i < A_ITEMS; ++i) {
            const int idx = tid + NT * i, row = a_row(idx >> 3), kq = idx & 7;
            r.a[i] = __builtin_amdgcn_raw_buffer_load_b128(
                rA, (int)(((uint32_t)(m0 + row) * (uint32_t)p.lda + (uint32_t)(k0 + 4 * kq)) * 4u), 0, 0);
        }
        // pre-split: piece idx & 7 of column idx >> 3 (8 lanes read a column's 128 bytes)
        if constexpr (WK == W_BS) {
#pragma unroll
            for (int i = 0; i < B_ITEMS; ++i) {
                const int idx = tid + NT * i;
                if (B_TOTAL % NT != 0 && idx >= B_TOTAL) break;   // uniform per wave
                const uint32_t col = (uint32_t)(k0 / KT) * (uint32_t)p.N + (uint32_t)(n0 + (idx >> 3));
                r.w[i].w = __builtin_amdgcn_raw_buffer_load_b128(rB, (int)(col * 128u + 16u * (idx & 7)), 0, 0);
            }
        } else if constexpr (WK == W_BS8) {
            // piece idx & 3 of column idx >> 2 (4 lanes read a column's 64 bytes)
#pragma unroll
            for (int i = 0; i < B_ITEMS; ++i) {
                const int idx = tid + NT * i;
                if (B_TOTAL % NT != 0 && idx >= B_TOTAL) break;   // uniform per wave
                const uint32_t col = (uint32_t)(k0 / KT) * (uint32_t)p.N + (uint32_t)(n0 + (idx >> 2));
                r.w[i].w = __builtin_amdgcn_raw_buffer_load_b128(rB, (int)(col * 64u + 16u * (idx & 3)), 0, 0);
            }
        } else {
            load_units(r, p, rB, rS, tid, n0, k0);
        }
    }

    // the weight units of the other formats: k pairs fastest across lanes,
    // so 16 lanes write 16 consecutive LDS words
    __device__ static void load_units(Raw& r, const SpArgs& p, __amdgpu_buffer_rsrc_t rB,
                                      __amdgpu_buffer_rsrc_t rS, int tid, int n0, int k0)
    {
#pragma unroll
        for (int i = 0; i < B_ITEMS; ++i) {
            const int idx = tid + NT * i, kp = idx % (KT / 2), cu = idx / (KT / 2);
            if (B_TOTAL % NT != 0 && idx >= B_TOTAL) break;   // uniform per wave
            const int n = n0 + UC * cu;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const uint32_t k = (uint32_t)(k0 + 2 * kp + h);
                if constexpr (WK == W_I8) {
                    r.w[i].q[h] = __builtin_amdgcn_raw_buffer_load_b32(rB, (int)(k * (uint32_t)p.ldb + n), 0, 0);
                } else if constexpr (WK == W_I4) {
                    r.w[i].q[h] = __builtin_amdgcn_raw_buffer_load_b32(rB, (int)(k * (uint32_t)p.ldb + (n >> 1)), 0, 0);
                    r.w[i].s[h] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                        rS, (int)((k * (uint32_t)p.n_groups + (uint32_t)(n >> 5)) * 4u), 0, 0));
                } else {
                    r.w[i].w[h] = __builtin_amdgcn_raw_buffer_load_b128(rB, (int)((k * (uint32_t)p.ldb + n) * 4u), 0, 0);
                }
            }
        }
    }

    // split a loaded chunk into the planes at `base`
    __device__ static void store(const Raw& r, __bf16* base, int tid)
    {
        __bf16* ah = base;
        __bf16* al = base + A_LO;
        __bf16* bh = base + B_HI;
        __bf16* bl = base + B_LO;                    // int4, fp32 only
        if constexpr (AS) {
            // part kq: the hi (even) or lo (odd) half of k group kq / 2
#pragma unroll
            for (int i = 0; i < A_ITEMS; ++i) {
                const int idx = tid + NT * i, row = a_row(idx >> 3), kq = idx & 7;
                *reinterpret_cast<v4u*>((kq & 1 ? al : ah) + row * RS + 8 * (kq >> 1)) = r.a[i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < A_ITEMS; ++i) {
                const int idx = tid + NT * i, row = a_row(idx >> 3), kq = idx & 7;
                uint32_t h0, l0, h1, l1;
                split2(__uint_as_float(r.a[i][0]), __uint_as_float(r.a[i][1]), h0, l0);
                split2(__uint_as_float(r.a[i][2]), __uint_as_float(r.a[i][3]), h1, l1);
                *reinterpret_cast<v2u*>(ah + row * RS + 4 * kq) = v2u{h0, h1};
                *reinterpret_cast<v2u*>(al + row * RS + 4 * kq) = v2u{l0, l1};
            }
        }
        if constexpr (WK == W_BS) {
            // piece q = idx & 7: the hi (q < 4) or the lo half's k group q & 3
#pragma unroll
            for (int i = 0; i < B_ITEMS; ++i) {
                const int idx = tid + NT * i, q = idx & 7;
                if (B_TOTAL % NT != 0 && idx >= B_TOTAL) break;   // uniform per wave
                *reinterpret_cast<v4u*>((q < 4 ? bh : bl) + (idx >> 3) * RS + 8 * (q & 3)) = r.w[i].w;
            }
        } else if constexpr (WK == W_BS8) {
            // piece q = idx & 3: k group q of column idx >> 2
#pragma unroll
            for (int i = 0; i < B_ITEMS; ++i) {
                const int idx = tid + NT * i;
                if (B_TOTAL % NT != 0 && idx >= B_TOTAL) break;   // uniform per wave
                *reinterpret_cast<v4u*>(bh + (idx >> 2) * RS + 8 * (idx & 3)) = r.w[i].w;
            }
        } else {
            store_units(r, bh, bl, tid);
        }
    }

    // the other formats' weight units: decoded (int4: fl(q * s)), split, and
    // written to the planes
    __device__ static void store_units(const Raw& r, __bf16* bh, __bf16* bl, int tid)
    {
#pragma unroll
        for (int i = 0; i < B_ITEMS; ++i) {
            const int idx = tid + NT * i, kp = idx % (KT / 2), cu = idx / (KT / 2);
            if (B_TOTAL % NT != 0 && idx >= B_TOTAL) break;   // uniform per wave
#pragma unroll
            for (int c = 0; c < UC; ++c) {
                const int off = (UC * cu + c) * RS + 2 * kp;      // column-major plane
                if constexpr (WK == W_I8) {
                    const float q0 = (float)(int)(int8_t)(r.w[i].q[0] >> (8 * c));
                    const float q1 = (float)(int)(int8_t)(r.w[i].q[1] >> (8 * c));
                    *reinterpret_cast<uint32_t*>(bh + off) = bits2(to_bf2(q0, q1));   // exact
                } else {
                    float w0, w1;
                    if constexpr (WK == W_I4) {
                        // blas.c:834-840: fl((float)q * s), byte j = columns 2j (low), 2j+1
                        w0 = __fmul_rn((float)q_i4(r.w[i].q[0] >> (8 * (c >> 1)), c & 1), r.w[i].s[0]);
                        w1 = __fmul_rn((float)q_i4(r.w[i].q[1] >> (8 * (c >> 1)), c & 1), r.w[i].s[1]);
                    } else {
                        w0 = __uint_as_float(r.w[i].w[0][c]);
                        w1 = __uint_as_float(r.w[i].w[1][c]);
                    }
                    uint32_t hi, lo;
                    split2(w0, w1, hi, lo);
                    *reinterpret_cast<uint32_t*>(bh + off) = hi;
                    *reinterpret_cast<uint32_t*>(bl + off) = lo;
                }
            }
        }
    }

    // One wave's 64 x 64 block at rows [r0, r0 + 64), columns [c0, c0 + 64)
    // of the tile, as 2 x 2 MFMA blocks: lane (l & 31) is a row of A and a
    // column of W, k = 8 (l >> 5) .. +7 of each 16-deep step.
    __device__ static void multiply(const __bf16* base, v16f (&acc)[2][2], int lane, int r0, int c0)
    {
        const __bf16* ah = base;
        const __bf16* al = base + A_LO;
        const __bf16* bh = base + B_HI;
        const __bf16* bl = base + B_LO;
        const int r_lane = lane & 31, k_lane = 8 * (lane >> 5);
#pragma unroll
        for (int ks = 0; ks < KT / 16; ++ks) {
            v8bf a_hi[2], a_lo[2], b_hi[2], b_lo[2];
#pragma unroll
            for (int r = 0; r < 2; ++r) {
                const int o = (r0 + 32 * r + r_lane) * RS + 16 * ks + k_lane;
                a_hi[r] = *reinterpret_cast<const v8bf*>(ah + o);
                a_lo[r] = *reinterpret_cast<const v8bf*>(al + o);
            }
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const int o = (c0 + 32 * c + r_lane) * RS + 16 * ks + k_lane;
                b_hi[c] = *reinterpret_cast<const v8bf*>(bh + o);
                if constexpr (NBP == 2) b_lo[c] = *reinterpret_cast<const v8bf*>(bl + o);
            }
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    acc[r][c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_hi[r], b_hi[c], acc[r][c], 0, 0, 0);
                    acc[r][c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_lo[r], b_hi[c], acc[r][c], 0, 0, 0);
                    if constexpr (NBP == 2)
                        acc[r][c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_hi[r], b_lo[c], acc[r][c], 0, 0, 0);
                }
        }
    }
};

// The output step for one element of C: alpha, beta, bias and the epilogue
// (encoder.c:193-216, 410-424, 473-475).
__device__ inline void put(const SpArgs& p, int m, int n, float sum)
{
    float* cp = p.C + (size_t)m * p.ldc + n;
    float v = __fmul_rn(p.alpha, sum);
    if (p.beta != 0.0f) v = __fadd_rn(p.beta == 1.0f ? *cp : __fmul_rn(p.beta, *cp), v);
    if (p.bias) v = __fadd_rn(v, p.bias[n]);
    switch (p.epi) {
    case EPI_SWISH:         v = swish_f(v); break;
    case EPI_HALF_RESIDUAL: v = __fmaf_rn(v, 0.5f, *cp); break;
    case EPI_RESIDUAL:      v = __fadd_rn(*cp, v); break;
    case EPI_RELU:          v = v > 0.0f ? v : 0.0f; break;
    default:                break;
    }
    *cp = v;
}

// Tile t of the launch, in XCD-sized runs along rows of tiles (workgroups
// reach the 8 XCDs round-robin): an XCD's workgroups share A rows in its L2.
// -1 for the padding workgroups of the last run.
__device__ inline int tile_of(const SpArgs& p)
{
    const int per = gridDim.x / kXcd;
    const int t = (blockIdx.x % kXcd) * per + blockIdx.x / kXcd;
    return t < p.tiles ? t : -1;
}

__device__ inline void zero(v16f (&acc)[2][2])
{
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[r][c][e] = 0.0f;
}

// Workgroups of WM x WN waves own (64 WM) x (64 WN) tiles of C; two LDS
// buffers, loads PD chunks ahead.
// Two waves per SIMD where the registers allow it without spills (the
// others are held to one by their LDS anyway).
// SK: workgroup u takes segment u / n_tiles of K (a contiguous run of its
// chunks) for tile u % n_tiles and stores its raw sums to the tile's slot
// of that segment in work, in register order (split_reduce finishes).
template <int WK, int WM, int WN, int PD, bool SK, bool AS>
__global__ __launch_bounds__(64 * WM * WN, WK == W_I8 || WK == W_BS8 || WM * WN == 4 ? 2 : 1) void split_gemm(SpArgs p)
{
    typedef Pipe<WK, 64 * WM, 64 * WN, 64 * WM * WN, AS> L;
    __shared__ __attribute__((aligned(16))) __bf16 smem[2 * L::BUF];

    const int u = tile_of(p);
    if (u < 0) return;                               // padding workgroup (uniform)
    const int t = SK ? u % p.n_tiles : u, seg = SK ? u / p.n_tiles : 0;
    const int m0 = (t / p.tiles_n) * (64 * WM), n0 = (t % p.tiles_n) * (64 * WN);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    const auto rA = rsrc(p.A, p.a_bytes);
    const auto rB = rsrc(p.B, p.b_bytes), rS = rsrc(p.scales, p.s_bytes);

    typename L::Raw raw[PD];                         // chunk x in slot x % PD
    v16f acc[2][2];
    zero(acc);

    // Loads run PD chunks ahead: before chunk c multiplies, the slots hold
    // chunks c + 1 .. c + PD.  The loop is unrolled by PD so that every slot
    // index is a compile-time constant.  Chunks [kc, kc + nc) of K.
    const int kc = SK ? seg * (p.K / KT) / p.n_seg : 0;
    const int nc = SK ? (seg + 1) * (p.K / KT) / p.n_seg - kc : p.K / KT;
#pragma unroll
    for (int j = 0; j < PD; ++j)
        if (j < nc) L::load(raw[j], p, rA, rB, rS, tid, m0, n0, KT * (kc + j));
    L::store(raw[0], smem, tid);
    if (PD < nc) L::load(raw[0], p, rA, rB, rS, tid, m0, n0, KT * (kc + PD));
    __syncthreads();
    // Chunk c (not the last): multiply it, stage chunk c + 1 from slot
    // (j + 1) % PD (j constant once unrolled) into the other buffer, whose
    // last reader was chunk c - 1 before the barrier, and load chunk
    // c + 1 + PD into that slot.  Past the end that load fetches the last
    // chunk again, which is never staged: the body has no branch, so the
    // compiler interleaves the staging's VALU work with the multiply's MFMAs
    // (int8 QKV at 1656 rows 42.8 -> 40.8 us, fast encoder pass +0.7%).
    auto step = [&](int c, int j) {
        L::multiply(smem + (c & 1) * L::BUF, acc, lane, 64 * wm, 64 * wn);
        const int s = (j + 1) % PD;
        L::store(raw[s], smem + ((c + 1) & 1) * L::BUF, tid);
        L::load(raw[s], p, rA, rB, rS, tid, m0, n0, KT * (kc + min(c + 1 + PD, nc - 1)));
        __syncthreads();
    };
    // Whole rounds of PD chunks without an exit inside: an exit between the
    // multiplies made the compiler copy every accumulator at the end of each
    // round, after waiting for the matrix cores.  Then the chunks short of a
    // round, and the last chunk, which only multiplies.
    int c0 = 0;
    for (; c0 + PD <= nc - 1; c0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; ++j) step(c0 + j, j);
    }
#pragma unroll
    for (int j = 0; j < PD - 1; ++j)
        if (c0 + j < nc - 1) step(c0 + j, j);
    L::multiply(smem + ((nc - 1) & 1) * L::BUF, acc, lane, 64 * wm, 64 * wn);

    if constexpr (SK) {
        if (p.work_rows) {
            // row-major partials: row m of segment seg at (seg work_rows + m) N
            float* w = p.work + (size_t)seg * p.work_rows * p.N;
#pragma unroll
            for (int r = 0; r < 2; ++r)
#pragma unroll
                for (int c = 0; c < 2; ++c) {
                    const int n = n0 + 64 * wn + 32 * c + (lane & 31);
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        const int m = m0 + 64 * wm + 32 * r + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                        w[(size_t)m * p.N + n] = acc[r][c][e];
                    }
                }
            return;
        }
        // slot (seg, t): wave-major, then block, register, lane (each store
        // instruction writes 256 contiguous bytes)
        float* w = p.work + ((size_t)seg * p.n_tiles + t) * (WM * WN * 4096) + (size_t)wave * 4096;
#pragma unroll
        for (int r = 0; r < 2; ++r)
#pragma unroll
            for (int c = 0; c < 2; ++c)
#pragma unroll
                for (int e = 0; e < 16; ++e) w[((2 * r + c) * 16 + e) * 64 + lane] = acc[r][c][e];
        return;
    }

    // C[m][n]: lane (l & 31) is the column, register e the row
    // 8 (e >> 2) + 4 (l >> 5) + (e & 3) of each 32 x 32 block
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            const int n = n0 + 64 * wn + 32 * c + (lane & 31);
            if (n >= p.N) continue;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int m = m0 + 64 * wm + 32 * r + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (m < p.M) put(p, m, n, acc[r][c][e]);
            }
        }
}

// Whether the output step reads C (beta or a residual epilogue).
__device__ inline bool reads_c(const SpArgs& p)
{
    return p.beta != 0.0f || p.epi == EPI_HALF_RESIDUAL || p.epi == EPI_RESIDUAL;
}

// put's steps for four outputs of one row: alpha, beta with C's values c4,
// the bias values b4, the epilogue.
__device__ inline float4 finish4(const SpArgs& p, float4 sum, float4 c4, float4 b4)
{
    float v[4] = {__fmul_rn(p.alpha, sum.x), __fmul_rn(p.alpha, sum.y), __fmul_rn(p.alpha, sum.z),
                  __fmul_rn(p.alpha, sum.w)};
    const float c[4] = {c4.x, c4.y, c4.z, c4.w}, b[4] = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if (p.beta != 0.0f) v[i] = __fadd_rn(p.beta == 1.0f ? c[i] : __fmul_rn(p.beta, c[i]), v[i]);
        if (p.bias) v[i] = __fadd_rn(v[i], b[i]);
        switch (p.epi) {
        case EPI_SWISH:         v[i] = swish_f(v[i]); break;
        case EPI_HALF_RESIDUAL: v[i] = __fmaf_rn(v[i], 0.5f, c[i]); break;
        case EPI_RESIDUAL:      v[i] = __fadd_rn(c[i], v[i]); break;
        case EPI_RELU:          v[i] = v[i] > 0.0f ? v[i] : 0.0f; break;
        default:                break;
        }
    }
    return make_float4(v[0], v[1], v[2], v[3]);
}

// The second launch of a split-K GEMM: output i of tile t is the sum of
// its n_seg partials in segment order, then alpha, beta, bias and the
// epilogue (put).  Each thread takes outputs i .. i + 3 of a tile: four
// lanes of one register, so four consecutive columns of one row (N is a
// multiple of 32, so all four are in range or none).
template <int WM, int WN>
__global__ __launch_bounds__(256) void split_reduce(SpArgs p)
{
    constexpr int TS = WM * WN * 4096;               // floats per tile
    constexpr int PER = TS / 1024;                   // workgroups per tile
    const int t = blockIdx.x / PER, i = ((blockIdx.x % PER) * 256 + threadIdx.x) * 4;
    const int wave = i >> 12, blk = (i >> 10) & 3, e = (i >> 6) & 15, l = i & 63;
    const int m = (t / p.tiles_n) * (64 * WM) + 64 * (wave / WN) + 32 * (blk >> 1) + 8 * (e >> 2) +
                  4 * (l >> 5) + (e & 3);
    const int n = (t % p.tiles_n) * (64 * WN) + 64 * (wave % WN) + 32 * (blk & 1) + (l & 31);
    if (m >= p.M || n >= p.N) return;
    const float* w = p.work + (size_t)t * TS + i;
    float4 sum = *reinterpret_cast<const float4*>(w);
    for (int s = 1; s < p.n_seg; ++s) {
        const float4 v = *reinterpret_cast<const float4*>(w + (size_t)s * p.n_tiles * TS);
        sum.x = __fadd_rn(sum.x, v.x);
        sum.y = __fadd_rn(sum.y, v.y);
        sum.z = __fadd_rn(sum.z, v.z);
        sum.w = __fadd_rn(sum.w, v.w);
    }
    if (p.c_vec4) {
        // the same steps as put, on 16-byte accesses of C and the bias
        float4* cp = reinterpret_cast<float4*>(p.C + (size_t)m * p.ldc + n);
        const float4 c4 = reads_c(p) ? *cp : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        const float4 b4 = p.bias ? *reinterpret_cast<const float4*>(p.bias + n) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        *cp = finish4(p, sum, c4, b4);
        return;
    }
    put(p, m, n, sum.x);
    put(p, m, n + 1, sum.y);
    put(p, m, n + 2, sum.z);
    put(p, m, n + 3, sum.w);
}

// fl(fl(fl(v - mean) * inv) * g + b) per element: the LayerNorm kernels'
// output step.
__device__ inline float4 ln4(float4 v, float mean, float inv, float4 g, float4 b)
{
    return make_float4(__fmaf_rn(__fmul_rn(__fsub_rn(v.x, mean), inv), g.x, b.x),
                       __fmaf_rn(__fmul_rn(__fsub_rn(v.y, mean), inv), g.y, b.y),
                       __fmaf_rn(__fmul_rn(__fsub_rn(v.z, mean), inv), g.z, b.z),
                       __fmaf_rn(__fmul_rn(__fsub_rn(v.w, mean), inv), g.w, b.w));
}

// The statistics of the workgroup's RPW rows in buf (pitch LD) into st:
// 8 lanes per row (lanes 0-15 of the first RPW / 2 waves), with the
// LayerNorm kernels' chains (ln_row_stats_rolled).  Between two barriers.
template <int RPW, int D, int LD>
__device__ inline void rows_stats(const float* buf, float (*st)[2], int w, int lane)
{
    __syncthreads();
    if (lane < 16 && w < RPW / 2) {
        const int r = 2 * w + (lane >> 3), l = lane & 7;
        float mean, inv;
        ln_row_stats_rolled<32>(buf + r * LD, D, l, mean, inv);
        if (l == 0) {
            st[r][0] = mean;
            st[r][1] = inv;
        }
    }
    __syncthreads();
}

// Rows per workgroup of split_reduce_ln: 414 workgroups at 1656 rows, 64 KB
// of partials each in flight.  Two rows per workgroup measured 1.8% slower
// on the fast encoder pass and eight 3.5% slower (A/B on one box each, two
// runs each).
constexpr int kReduceLnRows = 4;

// The second launch of a split-K GEMM whose 1024-wide output rows feed
// LayerNorms: a workgroup of 4 waves finishes RPW whole rows, thread t the
// columns 4 t .. 4 t + 3 of each.  Each output is its partials summed in
// segment order and put's steps, as split_reduce forms it.  Then, per
// SpLn: the rows' LayerNorm replaces them in C (out_g), and/or the
// LayerNorm of what C holds is written pre-split to next_out (next_g), in
// the layout and with the arithmetic of layer_norm_split_rows: the same
// bits as split_reduce followed by the LayerNorm kernels, in one launch
// that reads the rows from memory once.
// The partials are row-major (SpArgs::work_rows), so a row of a segment is
// 4 KB in one piece.  The loads of 4 segments are issued at once
// (segments past the last repeat it and are not added): RPW x 4 16-byte
// loads per thread in flight.
template <int RPW>
__global__ __launch_bounds__(256) void split_reduce_ln(SpArgs p, SpLn q)
{
    constexpr int D = 1024, LD = D + 8;
    static_assert(RPW % 2 == 0 && RPW <= 8, "2 rows per wave's statistics lanes");
    __shared__ float buf[RPW * LD];
    __shared__ float st[RPW][2];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int row0 = blockIdx.x * RPW, nr = min(RPW, p.M - row0);
    const int n = 4 * tid;
    const size_t seg_stride = (size_t)p.work_rows * D;
    // rows past M repeat the workgroup's first row (computed, never stored)
    const float* wk[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) wk[r] = p.work + (size_t)(row0 + (r < nr ? r : 0)) * D + n;
    // C's rows and the bias first, so that they are in flight with the
    // partials (C is read whatever the epilogue: rows < M, in bounds)
    float4 c4[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
        c4[r] = *reinterpret_cast<const float4*>(p.C + (size_t)(row0 + (r < nr ? r : 0)) * p.ldc + n);
    const float4 b4 = p.bias ? *reinterpret_cast<const float4*>(p.bias + n) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const int last = p.n_seg - 1;
    float4 sum[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) sum[r] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    for (int s0 = 0; s0 <= last; s0 += 4) {
        float4 v[4][RPW];
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int r = 0; r < RPW; ++r)
                v[j][r] = *reinterpret_cast<const float4*>(wk[r] + min(s0 + j, last) * seg_stride);
        // every addition is made and the ones past the last segment are
        // dropped by a select, so no load sits inside a branch (where the
        // compiler would issue it after the previous segment's wait); the
        // first segment is taken as it is (fl(0 + x) would turn -0 to +0)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const bool first = s0 + j == 0, live = s0 + j <= last;
            // (per component: a select of whole float4 values went to scratch)
            auto acc = [&](float s, float x) { return live ? (first ? x : __fadd_rn(s, x)) : s; };
#pragma unroll
            for (int r = 0; r < RPW; ++r) {
                sum[r].x = acc(sum[r].x, v[j][r].x);
                sum[r].y = acc(sum[r].y, v[j][r].y);
                sum[r].z = acc(sum[r].z, v[j][r].z);
                sum[r].w = acc(sum[r].w, v[j][r].w);
            }
        }
    }
    const bool rc = reads_c(p);
    float4 v[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
        v[r] = finish4(p, sum[r], rc ? c4[r] : make_float4(0.0f, 0.0f, 0.0f, 0.0f), b4);

    if (q.out_g) {
        const float4 g = *reinterpret_cast<const float4*>(q.out_g + n);
        const float4 b = *reinterpret_cast<const float4*>(q.out_b + n);
#pragma unroll
        for (int r = 0; r < RPW; ++r) *reinterpret_cast<float4*>(buf + r * LD + n) = v[r];
        rows_stats<RPW, D, LD>(buf, st, w, lane);
#pragma unroll
        for (int r = 0; r < RPW; ++r) v[r] = ln4(v[r], st[r][0], st[r][1], g, b);
    }
#pragma unroll
    for (int r = 0; r < RPW; ++r)
        if (r < nr) *reinterpret_cast<float4*>(p.C + (size_t)(row0 + r) * p.ldc + n) = v[r];
    if (!q.next_g) return;

    const float4 g = *reinterpret_cast<const float4*>(q.next_g + n);
    const float4 b = *reinterpret_cast<const float4*>(q.next_b + n);
    // buf's last reads (the statistics above) are behind the barrier that
    // ended them, and so are st's (the outputs above)
#pragma unroll
    for (int r = 0; r < RPW; ++r) *reinterpret_cast<float4*>(buf + r * LD + n) = v[r];
    rows_stats<RPW, D, LD>(buf, st, w, lane);
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        if (r < nr) {
            const float4 o = ln4(v[r], st[r][0], st[r][1], g, b);
            uint32_t h0, l0, h1, l1;
            split_bf16x2(o.x, o.y, h0, l0);
            split_bf16x2(o.z, o.w, h1, l1);
            // columns 4 t .. +3: half (t & 1) of the 8-column group t / 2,
            // whose 8 hi then 8 lo bf16 values fill the group's 8 floats
            unsigned short* g8 = reinterpret_cast<unsigned short*>(q.next_out + (size_t)(row0 + r) * D + 8 * (tid >> 1));
            *reinterpret_cast<uint2*>(g8 + 4 * (tid & 1)) = make_uint2(h0, h1);
            *reinterpret_cast<uint2*>(g8 + 8 + 4 * (tid & 1)) = make_uint2(l0, l1);
        }
    }
}

// Workgroups of KS waves own 64 x 64 tiles, wave w the chunks
// [w nc / KS, (w + 1) nc / KS) of K with an LDS slab of its own (no barrier
// until the end), loads PD chunks ahead; the KS partial tiles are then
// summed in LDS in wave order.  For shapes with too few tiles to give every
// CU a workgroup otherwise (N = 1024 at 1656 rows).
template <int WK, int KS, int PD, bool AS>
__global__ __launch_bounds__(64 * KS, 2) void split_gemm_k(SpArgs p)
{
    typedef Pipe<WK, 64, 64, 64, AS> L;
    constexpr int STAGE = KS * L::BUF * 2, RED = KS * 4 * 16 * 64 * 4;   // bytes
    __shared__ __attribute__((aligned(16))) unsigned char smem[STAGE > RED ? STAGE : RED];

    const int t = tile_of(p);
    if (t < 0) return;                               // padding workgroup (uniform)
    const int m0 = (t / p.tiles_n) * 64, n0 = (t % p.tiles_n) * 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const auto rA = rsrc(p.A, p.a_bytes);
    const auto rB = rsrc(p.B, p.b_bytes), rS = rsrc(p.scales, p.s_bytes);
    __bf16* slab = reinterpret_cast<__bf16*>(smem) + wave * L::BUF;

    typename L::Raw raw[PD];
    v16f acc[2][2];
    zero(acc);
    const int nc = p.K / KT, s0 = wave * nc / KS, s1 = (wave + 1) * nc / KS;
#pragma unroll
    for (int j = 0; j < PD; ++j)
        if (s0 + j < s1) L::load(raw[j], p, rA, rB, rS, lane, m0, n0, KT * (s0 + j));
    // (here the exit inside a round costs no accumulator copies, and the
    // split_gemm form of the loop spills)
    for (int c0 = s0; c0 < s1; c0 += PD) {
#pragma unroll
        for (int j = 0; j < PD; ++j) {
            const int c = c0 + j;
            if (c >= s1) break;
            // the slab's previous reads came first: LDS keeps a wave's order
            L::store(raw[j], slab, lane);
            __asm__ volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            if (c + PD < s1) L::load(raw[j], p, rA, rB, rS, lane, m0, n0, KT * (c + PD));
            L::multiply(slab, acc, lane, 0, 0);
        }
    }

    // fixed-order sum over the waves: red[w][block][e][lane]
    __syncthreads();                                 // every slab read done: reuse as red
    float* red = reinterpret_cast<float*>(smem);
#pragma unroll
    for (int r = 0; r < 2; ++r)
#pragma unroll
        for (int c = 0; c < 2; ++c)
#pragma unroll
            for (int e = 0; e < 16; ++e) red[((wave * 4 + 2 * r + c) * 16 + e) * 64 + lane] = acc[r][c][e];
    __syncthreads();
    for (int o = threadIdx.x; o < 4 * 16 * 64; o += 64 * KS) {
        const int blk = o >> 10, e = (o >> 6) & 15, l = o & 63;
        float sum = red[o];
#pragma unroll
        for (int w = 1; w < KS; ++w) sum = __fadd_rn(sum, red[w * 4096 + o]);
        const int m = m0 + 32 * (blk >> 1) + 8 * (e >> 2) + 4 * (l >> 5) + (e & 3);
        const int n = n0 + 32 * (blk & 1) + (l & 31);
        if (m < p.M && n < p.N) put(p, m, n, sum);
    }
}

// The pre-split copy (W_BS) of an int4 or fp32 weight [K][N]: thread i
// writes 16-byte piece i, the hi (q < 4) or lo half of k group q & 3 (q =
// i & 7) of column n of chunk c, with the staging's own decode (int4:
// fl(q * s[k][n/32]), blas.c:834-840) and split (split2), so the kernels
// multiply the same bf16 values either way.
template <int WK>
__global__ __launch_bounds__(256) void split_pack(int K, int N, const void* B, int ldb, const float* scales,
                                                  unsigned char* out)
{
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long long)(K / KT) * N * 8) return;
    const int q = (int)(i & 7);
    const long long cn = i >> 3;
    const int n = (int)(cn % N), c = (int)(cn / N);
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const size_t k = (size_t)(KT * c + 8 * (q & 3) + e);
        float w0, w1;
        if constexpr (WK == W_I4) {
            const unsigned char* b = static_cast<const unsigned char*>(B);
            const size_t g = (size_t)(N / 32);
            w0 = __fmul_rn((float)q_i4(b[k * ldb + n / 2], n & 1), scales[k * g + n / 32]);
            w1 = __fmul_rn((float)q_i4(b[(k + 1) * ldb + n / 2], n & 1), scales[(k + 1) * g + n / 32]);
        } else {
            const float* b = static_cast<const float*>(B);
            w0 = b[k * ldb + n];
            w1 = b[(k + 1) * ldb + n];
        }
        uint32_t hi, lo;
        split2(w0, w1, hi, lo);
        w[e / 2] = q < 4 ? hi : lo;
    }
    *reinterpret_cast<v4u*>(out + i * 16) = v4u{w[0], w[1], w[2], w[3]};
}

// The pre-split copy (W_BS8) of an int8 weight [K][N]: thread i writes
// 16-byte piece i, the 8 codes of k group i & 3 of column n of chunk c as
// bf16 (exact: |q| <= 128).
__global__ __launch_bounds__(256) void split_pack_i8(int K, int N, const signed char* B, int ldb,
                                                     unsigned char* out)
{
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= (long long)(K / KT) * N * 4) return;
    const int q = (int)(i & 3);
    const long long cn = i >> 2;
    const int n = (int)(cn % N), c = (int)(cn / N);
    uint32_t w[4];
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
        const size_t k = (size_t)(KT * c + 8 * q + e);
        w[e / 2] = bits2(to_bf2((float)B[k * ldb + n], (float)B[(k + 1) * ldb + n]));
    }
    *reinterpret_cast<v4u*>(out + i * 16) = v4u{w[0], w[1], w[2], w[3]};
}

// Launch shape.  Where 128 x 128 tiles outnumber the CUs, 256 x 128 tiles
// (8 waves, one workgroup per CU by its LDS) give no CU more rows x columns
// than two 128 x 128 workgroups would, and split each weight for twice the
// rows: the int4 up projection at 1656 rows took 66.7 against 71.7 us.
// Otherwise the largest tile (128 x 128, 128 x 64) whose count still gives
// every CU a workgroup; else 64 x 64 tiles with K split over 4 waves (when
// each wave gets at least two chunks), else 64 x 64 tiles of one wave.
enum SplitShape { SP_4x2, SP_2x2, SP_2x1, SP_K4, SP_1x1 };
constexpr int kKSplit = 4;

// PK_GPU_SPLIT_WIDE=0: 128 x 128 tiles (two workgroups per CU) where 256 x
// 128 tiles would be taken.  A tuning switch, read once.
bool split_wide()
{
    static const bool wide = [] {
        const char* v = getenv("PK_GPU_SPLIT_WIDE");
        return !(v && strcmp(v, "0") == 0);
    }();
    return wide;
}

SplitShape split_shape(int M, int N, int K)
{
    auto tiles = [&](int bm, int bn) { return (long long)((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
    if (tiles(128, 128) > 256) return split_wide() ? SP_4x2 : SP_2x2;
    if (tiles(128, 128) >= 256) return SP_2x2;
    if (tiles(128, 64) >= 256) return SP_2x1;
    if (K / KT >= 2 * kKSplit) return SP_K4;
    return SP_1x1;
}

// K split over workgroups, for shapes with too few 128 x 128 tiles to give
// every CU one (split_shape's SP_2x1, SP_K4, SP_1x1): 256 x 128 tiles, or
// 128 x 128 where 256-row tiles would pad more than 10% more rows, and as
// many segments of at least kMinSegChunks chunks as keep the workgroups
// within one per CU.  The partial tiles then take n_seg x tiles x tile
// floats <= 256 x 256 x 128 x 4 bytes = kSplitWorkBytes.
// The second launch moves every partial through memory (5-10 us at 1656
// rows), so int8 and int4 weights split K only from K = 2048: at 1656 x
// 1024 x 1024 (int8) and 375 x 4096 x 1024 (int4) their 64 x 64 tiles with K
// over 4 waves were faster (26.0 and 30.1 us against 29.9 and 33.4), while
// fp32's, with a third of their loads in flight, lost to split-K at every
// measured shape (46.9 against 31.1 us at 500 x 4096 x 1024).
constexpr int kMinSegChunks = 4;

struct SplitPlan {
    SplitShape shape;
    int n_seg;
};

// PK_GPU_SPLIT_K: 0 never splits K over workgroups, 2 splits every shape the
// plan allows regardless of weight format and K, anything else (the
// default, 1) follows the rule above.  A tuning switch, read once.
int split_k_mode()
{
    static const int mode = [] {
        const char* v = getenv("PK_GPU_SPLIT_K");
        const int m = v ? atoi(v) : 1;
        return m >= 0 && m <= 2 ? m : 1;
    }();
    return mode;
}

SplitPlan split_plan(WeightKind kind, int M, int N, int K, size_t work_bytes)
{
    const SplitShape s = split_shape(M, N, K);
    const int mode = split_k_mode();
    if (s == SP_4x2 || s == SP_2x2 || work_bytes < kSplitWorkBytes || mode == 0) return {s, 1};
    if (mode == 1 && kind != W_F32 && K < 2048) return {s, 1};
    const long long rows256 = (M + 255LL) / 256 * 256, rows128 = (M + 127LL) / 128 * 128;
    const bool wide = rows256 * 10 <= rows128 * 11;
    const int bm = wide ? 256 : 128;
    const long long tiles = (long long)((M + bm - 1) / bm) * ((N + 127) / 128);
    const long long seg = std::min<long long>(256 / tiles, (K / KT) / kMinSegChunks);
    if (seg < 2) return {s, 1};
    return {wide ? SP_4x2 : SP_2x2, (int)seg};
}

unsigned padded_grid(SpArgs& a, int bm, int bn, int n_seg = 1)
{
    a.tiles_n = (a.N + bn - 1) / bn;
    a.n_tiles = ((a.M + bm - 1) / bm) * a.tiles_n;
    a.n_seg = n_seg;
    a.tiles = a.n_tiles * n_seg;
    return (unsigned)(((a.tiles + kXcd - 1) / kXcd) * kXcd);
}

// ln: LayerNorms for the reduce to form (K split over workgroups only), or null.
template <int WK, bool AS>
hipError_t launch_kind(SpArgs a, SplitPlan plan, hipStream_t st, const SpLn* ln)
{
    // Chunks of loads in flight, as many as fit two waves per SIMD without
    // spills: a lane holds 16 A bytes per 64 rows of the tile and chunk, plus
    // its weight units (fp32's take 4 times int8's registers).
    constexpr bool WIDE = WK == W_F32 || WK == W_BS;      // 16-byte weight loads, 2 or 4 per column
    constexpr int PD22 = WIDE ? 2 : 3, PD21 = 2, PDK = WIDE ? 1 : 2, PD42 = 2;
    if (plan.n_seg > 1) {
        const bool wide = plan.shape == SP_4x2;
        const unsigned grid = padded_grid(a, wide ? 256 : 128, 128, plan.n_seg);
        // the fused reduce reads whole rows: partials row-major (the same
        // bytes as the tiles: N is a whole number of column tiles)
        if (ln) a.work_rows = (a.n_tiles / a.tiles_n) * (wide ? 256 : 128);
        if (wide)
            hipLaunchKernelGGL((split_gemm<WK, 4, 2, PD42, true, AS>), dim3(grid), dim3(512), 0, st, a);
        else
            hipLaunchKernelGGL((split_gemm<WK, 2, 2, PD22, true, AS>), dim3(grid), dim3(256), 0, st, a);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        if (ln) {
            hipLaunchKernelGGL((split_reduce_ln<kReduceLnRows>), dim3((unsigned)((a.M + kReduceLnRows - 1) / kReduceLnRows)),
                               dim3(256), 0, st, a, *ln);
            return hipGetLastError();
        }
        const unsigned blocks = (unsigned)a.n_tiles * (wide ? 8 * 4096 / 1024 : 4 * 4096 / 1024);
        if (wide)
            hipLaunchKernelGGL((split_reduce<4, 2>), dim3(blocks), dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((split_reduce<2, 2>), dim3(blocks), dim3(256), 0, st, a);
        return hipGetLastError();
    }
    if (ln) return hipErrorNotSupported;
    switch (plan.shape) {
    case SP_4x2:
        hipLaunchKernelGGL((split_gemm<WK, 4, 2, PD42, false, AS>), dim3(padded_grid(a, 256, 128)), dim3(512), 0, st, a);
        break;
    case SP_2x2:
        hipLaunchKernelGGL((split_gemm<WK, 2, 2, PD22, false, AS>), dim3(padded_grid(a, 128, 128)), dim3(256), 0, st, a);
        break;
    case SP_2x1:
        hipLaunchKernelGGL((split_gemm<WK, 2, 1, PD21, false, AS>), dim3(padded_grid(a, 128, 64)), dim3(128), 0, st, a);
        break;
    case SP_K4:
        hipLaunchKernelGGL((split_gemm_k<WK, kKSplit, PDK, AS>), dim3(padded_grid(a, 64, 64)), dim3(64 * kKSplit),
                           0, st, a);
        break;
    default:
        // K < 256 here: one or two chunks ahead, as many as fit without spills
        hipLaunchKernelGGL((split_gemm<WK, 1, 1, WK == W_I4 ? 1 : 2, false, AS>), dim3(padded_grid(a, 64, 64)), dim3(64), 0, st, a);
        break;
    }
    return hipGetLastError();
}

}  // namespace

bool split_supports(const GemmProblem& p)
{
    if (p.M < 1 || p.N < 1 || p.K < KT || p.K % KT) return false;
    if (p.chain_bias) return false;
    if (p.alpha == 0.0f || (p.kind == W_I8 && p.scale == 0.0f)) return false;   // beta-only step
    if (p.N % 32) return false;
    const uintptr_t pa = reinterpret_cast<uintptr_t>(p.A), pb = reinterpret_cast<uintptr_t>(p.B);
    if (p.lda % 4 || pa % 16) return false;
    switch (p.kind) {
    case W_I8:  return p.ldb % 4 == 0 && pb % 4 == 0;
    case W_I4:  return p.ldb % 4 == 0 && pb % 4 == 0 && reinterpret_cast<uintptr_t>(p.scales) % 4 == 0;
    default:    return p.ldb % 4 == 0 && pb % 16 == 0;
    }
}

hipError_t launch_split(const GemmProblem& p, hipStream_t st)
{
    if (!split_supports(p)) return hipErrorNotSupported;
    SpArgs a = {};
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
    if (a_ext >= lim || b_ext >= lim || s_ext >= lim) return hipErrorNotSupported;
    a.a_bytes = (uint32_t)a_ext;
    a.b_bytes = (uint32_t)b_ext;
    a.s_bytes = (uint32_t)s_ext;
    // 64 x 64 tiles at most: their count must fit the launch's int arithmetic
    if ((long long)((p.M + 63) / 64) * ((p.N + 63) / 64) > (1LL << 30)) return hipErrorNotSupported;
    const SplitPlan plan = split_plan(p.kind, p.M, p.N, p.K, p.work ? p.work_bytes : 0);
    a.work = p.work;
    a.c_vec4 = p.ldc % 4 == 0 && reinterpret_cast<uintptr_t>(p.C) % 16 == 0 &&
               reinterpret_cast<uintptr_t>(p.bias) % 16 == 0;
    SpLn lnv{p.out_ln_gamma, p.out_ln_beta, p.next_ln_gamma, p.next_ln_beta, p.next_ln_out};
    const bool fuse = p.out_ln_gamma || p.next_ln_gamma;
    if (fuse && (!split_fuses_ln(p) || plan.n_seg < 2)) return hipErrorNotSupported;
    const SpLn* ln = fuse ? &lnv : nullptr;
    if (p.b_presplit) {
        // the weight's pre-split copy (split_pack), split_weight_bytes long
        const size_t bytes = split_weight_bytes(p.kind, p.K, p.N);
        if (!bytes || bytes >= lim || reinterpret_cast<uintptr_t>(p.b_presplit) % 16) return hipErrorNotSupported;
        a.B = p.b_presplit;
        a.b_bytes = (uint32_t)bytes;
        if (p.kind == W_I8)
            return p.a_presplit ? launch_kind<W_BS8, true>(a, plan, st, ln) : launch_kind<W_BS8, false>(a, plan, st, ln);
        return p.a_presplit ? launch_kind<W_BS, true>(a, plan, st, ln) : launch_kind<W_BS, false>(a, plan, st, ln);
    }
    if (p.a_presplit) {
        switch (p.kind) {
        case W_I8: return launch_kind<W_I8, true>(a, plan, st, ln);
        case W_I4: return launch_kind<W_I4, true>(a, plan, st, ln);
        default:   return launch_kind<W_F32, true>(a, plan, st, ln);
        }
    }
    switch (p.kind) {
    case W_I8: return launch_kind<W_I8, false>(a, plan, st, ln);
    case W_I4: return launch_kind<W_I4, false>(a, plan, st, ln);
    default:   return launch_kind<W_F32, false>(a, plan, st, ln);
    }
}

bool split_fuses_ln(const GemmProblem& p)
{
    if (!p.out_ln_gamma && !p.next_ln_gamma) return false;
    if (!split_supports(p) || p.ln_gamma || p.N != kSplitLnN || !p.work || p.work_bytes < kSplitWorkBytes)
        return false;
    // put's 16-byte path (split_reduce's c_vec4)
    auto a16 = [](const void* q) { return reinterpret_cast<uintptr_t>(q) % 16 == 0; };
    if (p.ldc % 4 || !a16(p.C) || !a16(p.bias)) return false;
    if (p.out_ln_gamma && (!p.out_ln_beta || !a16(p.out_ln_gamma) || !a16(p.out_ln_beta))) return false;
    if (p.next_ln_gamma && (!p.next_ln_beta || !p.next_ln_out || !a16(p.next_ln_gamma) ||
                            !a16(p.next_ln_beta) || !a16(p.next_ln_out)))
        return false;
    if (!p.next_ln_gamma && p.next_ln_out) return false;
    return split_plan(p.kind, p.M, p.N, p.K, p.work_bytes).n_seg > 1;
}

size_t split_weight_bytes(WeightKind kind, int K, int N)
{
    if (K < KT || K % KT || N < 32 || N % 32) return 0;
    return (size_t)K * N * (kind == W_I8 ? 2 : 4);
}

hipError_t launch_split_pack(WeightKind kind, int K, int N, const void* B, int ldb, const float* scales,
                             void* out, hipStream_t st)
{
    if (!split_weight_bytes(kind, K, N) || (kind == W_I4 && !scales)) return hipErrorInvalidValue;
    const long long pieces = (long long)(K / KT) * N * (kind == W_I8 ? 4 : 8);
    const dim3 grid((unsigned)((pieces + 255) / 256));
    unsigned char* o = static_cast<unsigned char*>(out);
    if (kind == W_I8)
        hipLaunchKernelGGL(split_pack_i8, grid, dim3(256), 0, st, K, N, static_cast<const signed char*>(B), ldb, o);
    else if (kind == W_I4)
        hipLaunchKernelGGL(split_pack<W_I4>, grid, dim3(256), 0, st, K, N, B, ldb, scales, o);
    else
        hipLaunchKernelGGL(split_pack<W_F32>, grid, dim3(256), 0, st, K, N, B, ldb, scales, o);
    return hipGetLastError();
}

int split_k_segments(WeightKind kind, int M, int N, int K, size_t work_bytes)
{
    if (M < 1 || N < 1 || K < KT) return 1;
    return split_plan(kind, M, N, K, work_bytes).n_seg;
}

}  // namespace pkgpu
