// pk_gemm_tiles.h - CDNA4 (gfx950) tile kernels of the quantized weight GEMMs.
//
// Numerics.  The reference computes every output as a sequential fused
// multiply-add chain over k ascending, c = fma(fl(alpha*A[i][k]), w[k][j], c),
// starting from fl(beta*C) (csrc/blas.c:89-99, 187-218, 617-651), with the
// weight dequantised once per element, w = fl((float)q * s) (blas.c:545-553,
// 815-840).  The fp32 MFMA instructions with K = 1,
//     v_mfma_f32_32x32x1_2b_f32, v_mfma_f32_16x16x1_4b_f32,
//     v_mfma_f32_4x4x1_16b_f32,
// perform exactly one multiply-add per output element, so issuing them in
// ascending k on one accumulator reproduces the chain element for element,
// at the full fp32 matrix-core rate.  Nothing here ever splits k across
// waves or reorders a chain; that is the invariant every tile shape keeps.
//
// Data flow per workgroup (BM x BN output tile, KT-deep chunks of k):
//   global A (fp32, row-major) --> fl(alpha*a) --> LDS As[k][m]   (k-major)
//   global W (fp32 | int8 | packed int4 + fp32 scales) --> dequant in
//        registers --> LDS Bs[k][bpos(n)] fp32                    (k-major)
//   then each wave reads its MFMA operands from LDS a block of k steps
//   ahead of the multiplies.
// LDS is double-buffered; raw loads go to one of PD register sets, PD - 1
// chunks ahead of their conversion, and the conversion of chunk c + 1 runs
// while chunk c is multiplied (interleaved in the same waves, or in
// producer waves for family S).
//
// Cost model (measured on MI355X): a dependent 4x4x1 fp32 MFMA step takes
// ~20 cycles, its issue interval is ~8.5 cycles, and VALU instructions share
// the SIMD's issue and datapath with fp32 MFMAs (they do not overlap).  So
// every VALU conversion, address computation and load wait placed between a
// wave's dependent MFMAs lengthens its chains; the kernels minimise them.
//
// This header holds the kernel templates and the tile-configuration table.
// Each weight format's kernels are instantiated in a translation unit of its
// own (pk_gemm_f32.hip, pk_gemm_i8.hip, pk_gemm_i4.hip).
#pragma once

#include "pk_device_math.h"
#include "pk_gemm_kernels.h"

#include <algorithm>
#include <cmath>
#include <type_traits>

namespace pkgpu {
namespace tiles {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));

// Kernel arguments (device pointers).  N is the number of columns this
// launch computes; n_groups is the int4 scale-row length N_full/32
// (blas.c:958).
struct KArgs {
    int M, N, K;
    float alpha, beta;
    const float* A; int lda;
    const void* B;  int ldb;
    float scale;
    const float* scales; int n_groups;
    float* C; int ldc;
    // Exact byte extents the call may read (buffer-descriptor ranges) and
    // whether A / B rows allow 16-byte vector loads.
    uint32_t a_bytes, b_bytes, s_bytes;
    int vec_a, vec_b;
    const float* bias;       // fused epilogue (Epilogue in pk_gemm_kernels.h)
    const float* chain_bias; // chains start from chain_bias[col] (then beta == 0)
    int epi;
    int tile_order;          // TileOrder: which operand an XCD's tiles share
};

// MI355X dispatches workgroups to its 8 XCDs round-robin by linear id, and
// each XCD has its own L2.  With ORDER_ROWS / ORDER_COLS the tiles are
// re-ordered so that each XCD owns one contiguous run of the tile sequence,
// which walks along a row of tiles (sharing A) or down a column (sharing W):
// a block of that operand is then fetched into one L2 instead of all eight.
// The map from the linear id to the position in the sequence is a bijection
// for any grid size.  ORDER_DISPATCH keeps the launch order.
enum TileOrder { ORDER_DISPATCH = 0, ORDER_ROWS = 1, ORDER_COLS = 2 };
constexpr int kXcds = 8;

__device__ inline void tile_origin(const KArgs& p, int BM, int BN, int& m0, int& n0)
{
    int bx = blockIdx.x, by = blockIdx.y;
    if (p.tile_order != ORDER_DISPATCH) {
        const int nbx = gridDim.x, nby = gridDim.y, total = nbx * nby;
        const int lin = blockIdx.y * nbx + blockIdx.x;
        const int xcd = lin % kXcds, local = lin / kXcds;
        const int base = total / kXcds, extra = total % kXcds;
        const int t = xcd * base + min(xcd, extra) + local;   // start of this XCD's run + local
        bx = p.tile_order == ORDER_ROWS ? t % nbx : t / nby;
        by = p.tile_order == ORDER_ROWS ? t / nbx : t % nby;
    }
    m0 = by * BM;
    n0 = bx * BN;
}

// Buffer descriptor word 3 for gfx9-family raw buffers (32-bit data format).
constexpr int kRsrcWord3 = 0x00020000;

__device__ inline __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             kRsrcWord3);
}

// Raw buffer loads: an offset at or past the descriptor's range returns 0,
// so staging needs no bounds predicates and never touches memory outside
// the caller's operand.
__device__ inline float ld_f32(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0));
}
__device__ inline uint32_t ld_u32(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b32(r, (int)off, 0, 0);
}
__device__ inline uint32_t ld_u8(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b8(r, (int)off, 0, 0);
}
typedef uint32_t v4u __attribute__((ext_vector_type(4)));
__device__ inline v4u ld_v4(__amdgpu_buffer_rsrc_t r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, (int)off, 0, 0);
}

// ---- MFMA shapes -----------------------------------------------------------
// Every shape is used with its blocks stacked along M, so one instruction
// covers 64 rows x NCOL columns: A lane l carries row l, B lane l carries
// column l % NCOL.  row()/col() give the output element held by (lane, reg).

template <int MF> struct Mfma;

template <> struct Mfma<32> {
    static constexpr int NCOL = 32, NACC = 32;
    using acc_t = v32f;
    __device__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, 0, 0, 0);
    }
    __device__ static int row(int l, int r) {
        return 32 * (r >> 4) + 8 * ((r & 15) >> 2) + 4 * (l >> 5) + (r & 3);
    }
    __device__ static int col(int l, int) { return l & 31; }
};

template <> struct Mfma<16> {
    static constexpr int NCOL = 16, NACC = 16;
    using acc_t = v16f;
    __device__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, 0, 0, 0);
    }
    __device__ static int row(int l, int r) { return 16 * (r >> 2) + 4 * (l >> 4) + (r & 3); }
    __device__ static int col(int l, int) { return l & 15; }
};

template <> struct Mfma<4> {
    static constexpr int NCOL = 4, NACC = 4;
    using acc_t = v4f;
    __device__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 0, 0, 0);
    }
    __device__ static int row(int l, int r) { return 4 * (l >> 2) + r; }
    __device__ static int col(int l, int) { return l & 3; }
};

// ---- weight staging (dequantisation, bit-exact) ---------------------------
// A "unit" is VB consecutive columns of one row of W, fetched with one
// vector load when rows are 4/16-byte aligned; "elem" is the scalar form.
// load_*() only issues loads into raw registers; dequant_*() runs after the
// current chunk's MFMAs, so the loads' latency overlaps the multiplies, and
// produces fp32 weights exactly as the reference's pack step does.

template <int WK> struct WStage;

template <> struct WStage<W_F32> {
    static constexpr int VB = 4;
    struct Unit { v4u w; };
    struct Elem { float w; };
    __device__ static Unit load_unit(const KArgs& p, __amdgpu_buffer_rsrc_t rb,
                                     __amdgpu_buffer_rsrc_t, int k, int n) {
        return Unit{ld_v4(rb, ((uint32_t)k * p.ldb + n) * 4u)};
    }
    __device__ static void dequant_unit(const KArgs&, const Unit& u, float* out) {
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = __uint_as_float(u.w[j]);
    }
    __device__ static Elem load_elem(const KArgs& p, __amdgpu_buffer_rsrc_t rb,
                                     __amdgpu_buffer_rsrc_t, int k, int n) {
        return Elem{ld_f32(rb, ((uint32_t)k * p.ldb + n) * 4u)};
    }
    __device__ static float dequant_elem(const KArgs&, const Elem& e, int) { return e.w; }
};

// blas.c:545-553: fl((float)q * scale)
template <> struct WStage<W_I8> {
    static constexpr int VB = 4;
    struct Unit { uint32_t w; };
    struct Elem { uint32_t q; };
    __device__ static Unit load_unit(const KArgs& p, __amdgpu_buffer_rsrc_t rb,
                                     __amdgpu_buffer_rsrc_t, int k, int n) {
        return Unit{ld_u32(rb, (uint32_t)k * p.ldb + n)};
    }
    __device__ static void dequant_unit(const KArgs& p, const Unit& u, float* out) {
#pragma unroll
        for (int j = 0; j < 4; ++j) out[j] = __fmul_rn((float)(int8_t)(u.w >> (8 * j)), p.scale);
    }
    __device__ static Elem load_elem(const KArgs& p, __amdgpu_buffer_rsrc_t rb,
                                     __amdgpu_buffer_rsrc_t, int k, int n) {
        return Elem{ld_u8(rb, (uint32_t)k * p.ldb + n)};
    }
    __device__ static float dequant_elem(const KArgs& p, const Elem& e, int) {
        return __fmul_rn((float)(int8_t)e.q, p.scale);
    }
};

// blas.c:834-840 (portable/NEON decode) and blas.c:794 (scale index): byte j
// of row k holds column 2j in the low nibble and 2j+1 in the high nibble,
// both two's complement; scale = scales[k * (N/32) + n/32].
template <> struct WStage<W_I4> {
    static constexpr int VB = 8;
    struct Unit { uint32_t w; float s; };
    struct Elem { uint32_t b; float s; };
    __device__ static Unit load_unit(const KArgs& p, __amdgpu_buffer_rsrc_t rb,
                                     __amdgpu_buffer_rsrc_t rs, int k, int n) {
        return Unit{ld_u32(rb, (uint32_t)k * p.ldb + (n >> 1)),
                    ld_f32(rs, ((uint32_t)k * p.n_groups + (n >> 5)) * 4u)};
    }
    __device__ static void dequant_unit(const KArgs&, const Unit& u, float* out) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int v = (int)(u.w << (28 - 4 * j)) >> 28;     // sign-extend nibble j
            out[j] = __fmul_rn((float)v, u.s);
        }
    }
    __device__ static Elem load_elem(const KArgs& p, __amdgpu_buffer_rsrc_t rb,
                                     __amdgpu_buffer_rsrc_t rs, int k, int n) {
        return Elem{ld_u8(rb, (uint32_t)k * p.ldb + (n >> 1)),
                    ld_f32(rs, ((uint32_t)k * p.n_groups + (n >> 5)) * 4u)};
    }
    __device__ static float dequant_elem(const KArgs&, const Elem& e, int n) {
        const int v = (n & 1) ? ((int)(int8_t)e.b >> 4) : ((int)(int8_t)(e.b << 4) >> 4);
        return __fmul_rn((float)v, e.s);
    }
};

// ---- tile staging ------------------------------------------------------------
// Stages one KT-deep chunk: A rows [m0, m0+BM) -> As[k*AS + m] as fl(alpha*a),
// W columns [n0, n0+BN) -> Bs[k*BN + bpos(n)] as dequantised fp32.  load() only
// issues unconditional buffer loads (out-of-range -> 0) into one Raw register
// set; store() later converts a Raw set and writes it to LDS, and can run in
// pieces (items [lo, hi)) spread between the multiplies of the current chunk.
// Rows of A past M and columns of W past N only feed outputs that are never
// stored, and k past K is never multiplied.

// LDS position of W column n (0 <= n < BN) inside one k row of Bs.  LDS
// has 32 banks of 4 bytes; a b128 access serves 8 lanes per cycle and a b32
// access 32 lanes.  An int4 unit is 8 columns (two b128 halves), so with the
// identity layout 8 lanes' halves land 32 bytes apart (2-way conflicts).  In
// each 64-column block, unit q's halves go to 16-byte slots
//     first half:  q (q < 4) or q + 8 (q >= 4),   second half: q + 4,
// which puts any 8 lanes' halves in 8 distinct 4-bank groups, and keeps
// columns 0..31 and 32..63 each on 32 distinct banks for the multiplies'
// b32 reads.  Other formats and narrow tiles use the identity.
template <int WK, int BN>
__device__ __forceinline__ int bpos(int n)
{
    if constexpr (WK == W_I4 && BN % 64 == 0) {
        const int q = (n >> 3) & 7, r = n & 7;
        const int slot = (r < 4) ? (q < 4 ? q : q + 8) : q + 4;
        return (n & ~63) + 4 * slot + (r & 3);
    } else {
        return n;
    }
}

template <int WK, int BM, int BN, int KT, int NT, int AS, bool VEC, bool A1>
struct Stager {
    using WS = WStage<WK>;
    static constexpr int VB = WS::VB;
    // Items per chunk: 4-float units of A and VB-column units of W (single
    // elements when !VEC), spread over the NT threads; a chunk with fewer
    // items than threads leaves whole waves idle (totals are multiples of 64).
    static constexpr int A_TOTAL = VEC ? BM * KT / 4 : BM * KT;
    static constexpr int B_TOTAL = VEC ? BN * KT / VB : BN * KT;
    static constexpr int A_ITEMS = (A_TOTAL + NT - 1) / NT;
    static constexpr int B_ITEMS = (B_TOTAL + NT - 1) / NT;
    static constexpr int ITEMS = A_ITEMS + B_ITEMS;       // store() work items
    static_assert(A_TOTAL % 64 == 0 && B_TOTAL % 64 == 0, "wave-uniform staging");
    static_assert(BN % VB == 0 && KT % 4 == 0, "units");

    struct Raw {
        v4u a4[VEC ? A_ITEMS : 1];
        float a1[VEC ? 1 : A_ITEMS];
        typename WS::Unit bu[VEC ? B_ITEMS : 1];
        typename WS::Elem be[VEC ? 1 : B_ITEMS];
    };

    __amdgpu_buffer_rsrc_t rsA, rsB, rsS;

    __device__ explicit Stager(const KArgs& p)
        : rsA(make_rsrc(p.A, p.a_bytes)),
          rsB(make_rsrc(p.B, p.b_bytes)),
          rsS(make_rsrc(WK == W_I4 ? (const void*)p.scales : p.B, WK == W_I4 ? p.s_bytes : 0u)) {}

    __device__ void load(Raw& r, const KArgs& p, int tid, int m0, int n0, int k0) const {
#pragma unroll
        for (int i = 0; i < A_ITEMS; ++i) {
            const int e = tid + i * NT;
            if (A_TOTAL % NT != 0 && e >= A_TOTAL) continue;
            const int row = e % BM, kq = e / BM;          // rows fastest: conflict-free LDS writes
            if constexpr (VEC)
                r.a4[i] = ld_v4(rsA, ((uint32_t)(m0 + row) * p.lda + k0 + 4 * kq) * 4u);
            else
                r.a1[i] = ld_f32(rsA, ((uint32_t)(m0 + row) * p.lda + k0 + kq) * 4u);
        }
#pragma unroll
        for (int i = 0; i < B_ITEMS; ++i) {
            const int e = tid + i * NT;
            if (B_TOTAL % NT != 0 && e >= B_TOTAL) continue;
            if constexpr (VEC) {
                const int kk = e / (BN / VB), nq = e % (BN / VB);   // n fastest
                r.bu[i] = WS::load_unit(p, rsB, rsS, k0 + kk, n0 + VB * nq);
            } else {
                const int kk = e / BN, n = e % BN;
                r.be[i] = WS::load_elem(p, rsB, rsS, k0 + kk, n0 + n);
            }
        }
    }

    // fl(alpha*a) (skipped when alpha is exactly 1, where it is the identity)
    // and the weight dequantisation happen here.  lo/hi are compile-time
    // constants at every call site once loops are unrolled.
    __device__ void store(const Raw& r, const KArgs& p, int tid, float* As, float* Bs,
                          int lo = 0, int hi = ITEMS) const {
#pragma unroll
        for (int i = 0; i < A_ITEMS; ++i) {
            if (i < lo || i >= hi) continue;
            const int e = tid + i * NT;
            if (A_TOTAL % NT != 0 && e >= A_TOTAL) continue;
            const int row = e % BM, kq = e / BM;
            if constexpr (VEC) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float a = __uint_as_float(r.a4[i][j]);
                    As[(4 * kq + j) * AS + row] = A1 ? a : __fmul_rn(p.alpha, a);
                }
            } else {
                As[kq * AS + row] = A1 ? r.a1[i] : __fmul_rn(p.alpha, r.a1[i]);
            }
        }
#pragma unroll
        for (int i = 0; i < B_ITEMS; ++i) {
            if (A_ITEMS + i < lo || A_ITEMS + i >= hi) continue;
            const int e = tid + i * NT;
            if (B_TOTAL % NT != 0 && e >= B_TOTAL) continue;
            if constexpr (VEC) {
                const int kk = e / (BN / VB), nq = e % (BN / VB);
                float w[VB];
                WS::dequant_unit(p, r.bu[i], w);
#pragma unroll
                for (int j = 0; j < VB; ++j) Bs[kk * BN + bpos<WK, BN>(VB * nq + j)] = w[j];
            } else {
                const int kk = e / BN, n = e % BN;
                Bs[kk * BN + bpos<WK, BN>(n)] = WS::dequant_elem(p, r.be[i], n);
            }
        }
    }
};

// The chunk loop is unrolled by PD so that each chunk's Raw register set has
// a compile-time index.  Whole groups of PD full chunks run unconditionally
// (so no load is left in flight across the loop's back edge that the next
// iteration would have to drain); the remaining chunks, including a partial
// last one, run through the guarded form.  f(J, full, c) runs chunk c with
// c % PD == J.
template <int J, int PD, typename F>
__device__ __forceinline__ void chunk_group(F& f, int c0)
{
    if constexpr (J < PD) {
        f(std::integral_constant<int, J>{}, std::true_type{}, c0 + J);
        chunk_group<J + 1, PD>(f, c0);
    }
}
template <int J, int PD, typename F>
__device__ __forceinline__ void chunk_tail(F& f, int c0, int nchunks)
{
    if constexpr (J < PD) {
        if (c0 + J < nchunks) {
            f(std::integral_constant<int, J>{}, std::false_type{}, c0 + J);
            chunk_tail<J + 1, PD>(f, c0, nchunks);
        }
    }
}
// FULLK: the launcher guarantees K % (PD * KT) == 0, so no tail exists and
// the guarded form is not compiled.  Its copy of the accumulators costs
// registers: the 32x32 tile with two 32-deep chunks in flight needs 105 VGPRs
// + 64 AGPRs with it (2 waves per SIMD) and 101 + 32 without (3 waves, as
// many as its 48 KB of LDS allows; the int4 GEMMs of a 3312-row encoder pass
// took 27.4 instead of 28.2 ms on one box).  The launcher uses it for tiles
// with 32-deep chunks only: the 16-deep 32x32 tile would go from 3 to 4 waves
// per SIMD, and its int8 GEMMs measured 7% slower there.
template <int PD, bool FULLK = false, typename F>
__device__ __forceinline__ void run_chunks(F& f, int K, int KT)
{
    const int nfull = K / KT, nchunks = (K + KT - 1) / KT;
    int c0 = 0;
    for (; c0 + PD <= nfull; c0 += PD) chunk_group<0, PD>(f, c0);
    if constexpr (!FULLK) chunk_tail<0, PD>(f, c0, nchunks);
}

// The fused output step for C[row][col] (row < M, col < N): bias add, then
// the activation or the (half) residual (encoder.c:193-216, 410-424,
// 473-475).  0.5 * v is exact, so fl(c + 0.5 * v) equals the reference's
// fma(out, 0.5, x).
__device__ inline float epilogue(const KArgs& p, float v, int row, int col)
{
    if (p.bias) v = __fadd_rn(v, p.bias[col]);
    if (p.epi == EPI_SWISH) return swish_f(v);
    if (p.epi == EPI_HALF_RESIDUAL) return __fmaf_rn(v, 0.5f, p.C[(size_t)row * p.ldc + col]);
    if (p.epi == EPI_RESIDUAL) return __fadd_rn(p.C[(size_t)row * p.ldc + col], v);
    // _mm256_max_ps(v, 0) as pk_relu compiles: v unless v > 0 is false, then +0
    if (p.epi == EPI_RELU) return v > 0.0f ? v : 0.0f;
    return v;
}

// Store one output; the plain store is the common case and stays a single
// write (the condition is uniform across the launch).
__device__ inline void store_c(const KArgs& p, float v, int row, int col)
{
    float* c = p.C + (size_t)row * p.ldc + col;
    *c = (p.bias == nullptr && p.epi == EPI_NONE) ? v : epilogue(p, v, row, col);
}

// Chains start from beta*C exactly as scale_c leaves it (blas.c:89-99), or
// from the column's bias when chain_bias is set.
__device__ inline float beta_c(const KArgs& p, int row, int col)
{
    if (row >= p.M || col >= p.N) return 0.0f;
    if (p.chain_bias) return p.chain_bias[col];
    if (p.beta == 0.0f) return 0.0f;
    const float cv = p.C[(size_t)row * p.ldc + col];
    return (p.beta == 1.0f) ? cv : __fmul_rn(cv, p.beta);
}

// ---- family R: rows on lanes ------------------------------------------------
// Each MFMA covers 64 rows x NCOL columns (blocks stacked along M): A lane l
// carries row l, B lane l carries column l % NCOL.  A wave owns CW column
// tiles (CW independent chains); WGM x WGN waves share the staged tiles.

template <int WK, int MF, int CW, int WGM, int WGN, int KT, int PD, bool VEC, bool A1>
__global__ __launch_bounds__(64 * WGM * WGN)
void chain_gemm(KArgs p)
{
    using T = Mfma<MF>;
    constexpr int NT = 64 * WGM * WGN;
    constexpr int BM = 64 * WGM;
    constexpr int AS = BM + 1;              // padded row of As: conflict-free stores
    constexpr int WN = T::NCOL * CW;
    constexpr int BN = WN * WGN;
    constexpr int U = 8;                    // k steps per operand block
    constexpr int NBLK = KT / U;
    static_assert(KT % U == 0 && PD % 2 == 0, "chunking");
    using ST = Stager<WK, BM, BN, KT, NT, AS, VEC, A1>;
    constexpr int PER_BLK = (ST::ITEMS + NBLK - 1) / NBLK;

    __shared__ float As[2][KT * AS];
    __shared__ float Bs[2][KT * BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WGN, wn = wave % WGN;
    int m0, n0;
    tile_origin(p, BM, BN, m0, n0);

    typename T::acc_t acc[CW];
#pragma unroll
    for (int c = 0; c < CW; ++c)
#pragma unroll
        for (int r = 0; r < T::NACC; ++r)
            acc[c][r] = beta_c(p, m0 + wm * 64 + T::row(lane, r),
                               n0 + wn * WN + c * T::NCOL + T::col(lane, r));

    // LDS position of each of the wave's B columns (lane % NCOL of tile cc)
    int bcol[CW];
#pragma unroll
    for (int cc = 0; cc < CW; ++cc) bcol[cc] = bpos<WK, BN>(wn * WN + cc * T::NCOL + (lane % T::NCOL));

    // Chunk c's raw operands live in raw[c % PD]: loads run PD - 1 chunks
    // ahead of the chunk whose multiplies they are converted under.
    const ST st(p);
    typename ST::Raw raw[PD];
    // Sets are loaded one after another, in the order the loop consumes and
    // reissues them, so that wait counts at the loop head stay exact.
#pragma unroll
    for (int j = 0; j < PD; ++j) {
        st.load(raw[j], p, tid, m0, n0, j * KT);
        __builtin_amdgcn_sched_barrier(0);
    }
    st.store(raw[0], p, tid, As[0], Bs[0]);
    __syncthreads();

    auto chunk = [&](auto J, auto FULL, int c) {
        constexpr int j = decltype(J)::value;       // c % PD == j, so c & 1 == j & 1
        constexpr int buf = j & 1;
        st.load(raw[j], p, tid, m0, n0, (c + PD) * KT);     // issued first, as one block
        __builtin_amdgcn_sched_barrier(0);
        const float* as = &As[buf][wm * 64 + lane];
        const float* bs = &Bs[buf][0];
        float* as_n = As[buf ^ 1];
        float* bs_n = Bs[buf ^ 1];
        const int kn = decltype(FULL)::value ? KT : min(KT, p.K - c * KT);
        if (kn == KT) {
            // Operands for block kb+1 are read from LDS while block kb is
            // multiplied; piece kb of the next chunk's conversion sits between.
            float av[2][U], bv[2][U][CW];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                av[0][u] = as[u * AS];
#pragma unroll
                for (int cc = 0; cc < CW; ++cc) bv[0][u][cc] = bs[u * BN + bcol[cc]];
            }
#pragma unroll
            for (int kb = 0; kb < NBLK; ++kb) {
                const int cur = kb & 1;
                if (kb + 1 < NBLK) {
#pragma unroll
                    for (int u = 0; u < U; ++u) {
                        av[cur ^ 1][u] = as[((kb + 1) * U + u) * AS];
#pragma unroll
                        for (int cc = 0; cc < CW; ++cc)
                            bv[cur ^ 1][u][cc] = bs[((kb + 1) * U + u) * BN + bcol[cc]];
                    }
                }
                // Keep the next block's reads here, a block ahead of their use:
                // left alone, the scheduler sinks them next to their MFMAs and
                // the chains wait on LDS latency.
                __builtin_amdgcn_sched_barrier(0);
                st.store(raw[(j + 1) % PD], p, tid, as_n, bs_n, kb * PER_BLK, (kb + 1) * PER_BLK);
#pragma unroll
                for (int u = 0; u < U; ++u)
#pragma unroll
                    for (int cc = 0; cc < CW; ++cc) acc[cc] = T::step(av[cur][u], bv[cur][u][cc], acc[cc]);
            }
        } else {
            for (int kk = 0; kk < kn; ++kk) {
                const float a = as[kk * AS];
#pragma unroll
                for (int cc = 0; cc < CW; ++cc)
                    acc[cc] = T::step(a, bs[kk * BN + bcol[cc]], acc[cc]);
            }
            st.store(raw[(j + 1) % PD], p, tid, as_n, bs_n);
        }
        __syncthreads();
        // Keep the scheduler from hoisting a later chunk's conversion (and
        // with it a wait on loads still in flight) into this one.
        __builtin_amdgcn_sched_barrier(0);
    };
    run_chunks<PD>(chunk, p.K, KT);

#pragma unroll
    for (int c = 0; c < CW; ++c) {
#pragma unroll
        for (int r = 0; r < T::NACC; ++r) {
            const int row = m0 + wm * 64 + T::row(lane, r);
            const int col = n0 + wn * WN + c * T::NCOL + T::col(lane, r);
            if (row < p.M && col < p.N) store_c(p, acc[c][r], row, col);
        }
    }
}

// ---- family X: columns on lanes, A broadcast ---------------------------------
// Each MFMA covers BS rows x 64 columns (blocks side by side along N): B lane
// l carries column l, and A comes from one block only (CBSZ broadcast of
// block ABID to all blocks), so a single A register holds NB = 64/BS
// consecutive k steps (lane BS*t + i = A[row i][k + t]) and ABID = t picks
// the step.  A wave owns R row groups (R independent chains) sharing each B
// register; NWM x NWN waves share the staged tiles.

template <int MF> struct MfmaX;

template <> struct MfmaX<4> {
    static constexpr int BS = 4, NB = 16, CBSZ = 4, NACC = 4;
    using acc_t = v4f;
    template <int T_>
    __device__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, CBSZ, T_, 0);
    }
    __device__ static int row(int, int r) { return r; }
    __device__ static int col(int l, int) { return l; }
};

template <> struct MfmaX<16> {
    static constexpr int BS = 16, NB = 4, CBSZ = 2, NACC = 16;
    using acc_t = v16f;
    template <int T_>
    __device__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, c, CBSZ, T_, 0);
    }
    __device__ static int row(int l, int r) { return 4 * (l >> 4) + (r & 3); }
    __device__ static int col(int l, int r) { return 16 * (r >> 2) + (l & 15); }
};

template <> struct MfmaX<32> {
    static constexpr int BS = 32, NB = 2, CBSZ = 1, NACC = 32;
    using acc_t = v32f;
    template <int T_>
    __device__ static acc_t step(float a, float b, acc_t c) {
        return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, c, CBSZ, T_, 0);
    }
    __device__ static int row(int l, int r) { return 8 * ((r & 15) >> 2) + 4 * (l >> 5) + (r & 3); }
    __device__ static int col(int l, int r) { return 32 * (r >> 4) + (l & 31); }
};

// Steps t = T_..NB-1 of one NB-block: MFMA with ABID = t for every row group
// (ABID is an instruction field, so t must be a compile-time constant).
template <typename T, int R, int T_>
__device__ inline void x_steps(const float (&a)[R], const float* b, typename T::acc_t (&acc)[R])
{
    if constexpr (T_ < T::NB) {
#pragma unroll
        for (int g = 0; g < R; ++g) acc[g] = T::template step<T_>(a[g], b[T_], acc[g]);
        x_steps<T, R, T_ + 1>(a, b, acc);
    }
}

// The first n < NB steps only (partial last chunk).
template <typename T, int R, int T_>
__device__ inline void x_steps_n(const float (&a)[R], const float* b, typename T::acc_t (&acc)[R],
                                 int n)
{
    if constexpr (T_ < T::NB) {
        if (T_ < n) {
#pragma unroll
            for (int g = 0; g < R; ++g) acc[g] = T::template step<T_>(a[g], b[T_], acc[g]);
            x_steps_n<T, R, T_ + 1>(a, b, acc, n);
        }
    }
}

template <int MF> struct XPad;                       // conflict-free A-register reads
template <> struct XPad<4> { static constexpr int v = 4; };
template <> struct XPad<16> { static constexpr int v = 16; };
template <> struct XPad<32> { static constexpr int v = 0; };

template <int WK, int MF, int R, int NWM, int NWN, int KT, int PD, bool VEC, bool A1,
          bool FULLK = false>
__global__ __launch_bounds__(64 * NWM * NWN)
void chain_gemm_x(KArgs p)
{
    using T = MfmaX<MF>;
    constexpr int BS = T::BS, NB = T::NB;
    constexpr int NT = 64 * NWM * NWN;
    constexpr int BM = NWM * R * BS;
    constexpr int BN = NWN * 64;
    constexpr int AS = BM + XPad<MF>::v;
    constexpr int NBLK = KT / NB;
    static_assert(KT % NB == 0 && PD % 2 == 0, "chunk must hold whole A registers");
    using ST = Stager<WK, BM, BN, KT, NT, AS, VEC, A1>;
    constexpr int PER_BLK = (ST::ITEMS + NBLK - 1) / NBLK;

    __shared__ float As[2][KT * AS];
    __shared__ float Bs[2][KT * BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / NWN, wn = wave % NWN;
    int m0, n0;
    tile_origin(p, BM, BN, m0, n0);
    const int wrow = wm * R * BS;                  // wave's first row within the tile

    typename T::acc_t acc[R];
#pragma unroll
    for (int g = 0; g < R; ++g)
#pragma unroll
        for (int r = 0; r < T::NACC; ++r)
            acc[g][r] = beta_c(p, m0 + wrow + g * BS + T::row(lane, r),
                               n0 + wn * 64 + T::col(lane, r));

    // Chunk c's raw operands live in raw[c % PD]: loads run PD - 1 chunks
    // ahead of the chunk whose multiplies they are converted under.
    const ST st(p);
    typename ST::Raw raw[PD];
    // Sets are loaded one after another, in the order the loop consumes and
    // reissues them, so that wait counts at the loop head stay exact.
#pragma unroll
    for (int j = 0; j < PD; ++j) {
        st.load(raw[j], p, tid, m0, n0, j * KT);
        __builtin_amdgcn_sched_barrier(0);
    }
    st.store(raw[0], p, tid, As[0], Bs[0]);
    __syncthreads();

    // lane BS*t + i reads A[row i][k + t]
    const int a_off = (lane / BS) * AS + wrow + (lane % BS);
    auto chunk = [&](auto J, auto FULL, int c) {
        constexpr int j = decltype(J)::value;       // c % PD == j, so c & 1 == j & 1
        constexpr int buf = j & 1;
        st.load(raw[j], p, tid, m0, n0, (c + PD) * KT);     // issued first, as one block
        __builtin_amdgcn_sched_barrier(0);
        const float* as = &As[buf][a_off];
        const float* bs = &Bs[buf][wn * 64 + bpos<WK, BN>(lane)];
        float* as_n = As[buf ^ 1];
        float* bs_n = Bs[buf ^ 1];
        const int kn = decltype(FULL)::value ? KT : min(KT, p.K - c * KT);
        if (kn == KT) {
            // NB-blocks of k: the next block's operands are read while the
            // current block is multiplied; piece kb of the next chunk's
            // conversion sits between.
            float a[2][R], b[2][NB];
#pragma unroll
            for (int g = 0; g < R; ++g) a[0][g] = as[g * BS];
#pragma unroll
            for (int t = 0; t < NB; ++t) b[0][t] = bs[t * BN];
#pragma unroll
            for (int kb = 0; kb < NBLK; ++kb) {
                const int cur = kb & 1;
                if (kb + 1 < NBLK) {
#pragma unroll
                    for (int g = 0; g < R; ++g) a[cur ^ 1][g] = as[(kb + 1) * NB * AS + g * BS];
#pragma unroll
                    for (int t = 0; t < NB; ++t) b[cur ^ 1][t] = bs[((kb + 1) * NB + t) * BN];
                }
                __builtin_amdgcn_sched_barrier(0);    // next block's reads stay a block ahead
                st.store(raw[(j + 1) % PD], p, tid, as_n, bs_n, kb * PER_BLK, (kb + 1) * PER_BLK);
                x_steps<T, R, 0>(a[cur], b[cur], acc);
            }
        } else {
            for (int kb = 0; kb < kn; kb += NB) {
                float a[R], b[NB];
#pragma unroll
                for (int g = 0; g < R; ++g) a[g] = as[kb * AS + g * BS];
#pragma unroll
                for (int t = 0; t < NB; ++t) b[t] = bs[(kb + t) * BN];
                x_steps_n<T, R, 0>(a, b, acc, kn - kb);
            }
            st.store(raw[(j + 1) % PD], p, tid, as_n, bs_n);
        }
        __syncthreads();
        // Keep the scheduler from hoisting a later chunk's conversion (and
        // with it a wait on loads still in flight) into this one.
        __builtin_amdgcn_sched_barrier(0);
    };
    run_chunks<PD, FULLK>(chunk, p.K, KT);

#pragma unroll
    for (int g = 0; g < R; ++g) {
#pragma unroll
        for (int r = 0; r < T::NACC; ++r) {
            const int row = m0 + wrow + g * BS + T::row(lane, r);
            const int col = n0 + wn * 64 + T::col(lane, r);
            if (row < p.M && col < p.N) store_c(p, acc[g][r], row, col);
        }
    }
}

// ---- family S: family X with producer waves -----------------------------------
// The same tiles and arithmetic as family X, but the workgroup holds NC =
// NWM * NWN consumer waves, which only read LDS and issue the chains'
// MFMAs, and NC producer waves, which issue the global loads, dequantise
// and write LDS.  fp32 MFMA and VALU instructions share a SIMD's issue and
// datapath, and a wave issues in order: a wave that does both stalls its own
// dependent MFMAs on every conversion and load wait.  Waves w and w + NC sit
// on the same SIMD, so the producer's conversions fill the cycles the
// consumer's dependent MFMAs leave idle.  Both roles pass the same barriers:
// one after the first chunk is staged and one per chunk.

template <int WK, int MF, int R, int NWM, int NWN, int KT, int PD, bool VEC, bool A1>
__global__ __launch_bounds__(128 * NWM * NWN)
void chain_gemm_xs(KArgs p)
{
    using T = MfmaX<MF>;
    constexpr int BS = T::BS, NB = T::NB;
    constexpr int NC = NWM * NWN;
    constexpr int BM = NWM * R * BS;
    constexpr int BN = NWN * 64;
    constexpr int AS = BM + XPad<MF>::v;
    constexpr int NBLK = KT / NB;
    static_assert(KT % NB == 0 && PD % 2 == 0, "chunk must hold whole A registers");
    using ST = Stager<WK, BM, BN, KT, 64 * NC, AS, VEC, A1>;

    __shared__ float As[2][KT * AS];
    __shared__ float Bs[2][KT * BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    int m0, n0;
    tile_origin(p, BM, BN, m0, n0);

    if (wave >= NC) {
        // Producer: chunk c's raw operands live in raw[c % PD]; while the
        // consumers multiply chunk c, chunk c + 1 is converted into the other
        // LDS buffer and chunk c + PD is loaded.
        const int ptid = tid - 64 * NC;
        const ST st(p);
        typename ST::Raw raw[PD];
#pragma unroll
        for (int j = 0; j < PD; ++j) {
            st.load(raw[j], p, ptid, m0, n0, j * KT);
            __builtin_amdgcn_sched_barrier(0);
        }
        st.store(raw[0], p, ptid, As[0], Bs[0]);
        __syncthreads();
        auto chunk = [&](auto J, auto, int c) {
            constexpr int j = decltype(J)::value;       // c % PD == j, so c & 1 == j & 1
            constexpr int buf = j & 1;
            st.load(raw[j], p, ptid, m0, n0, (c + PD) * KT);
            __builtin_amdgcn_sched_barrier(0);
            st.store(raw[(j + 1) % PD], p, ptid, As[buf ^ 1], Bs[buf ^ 1]);
            __syncthreads();
            __builtin_amdgcn_sched_barrier(0);
        };
        run_chunks<PD>(chunk, p.K, KT);
        return;
    }

    // Consumer.
    const int wm = wave / NWN, wn = wave % NWN;
    const int wrow = wm * R * BS;                  // wave's first row within the tile
    typename T::acc_t acc[R];
#pragma unroll
    for (int g = 0; g < R; ++g)
#pragma unroll
        for (int r = 0; r < T::NACC; ++r)
            acc[g][r] = beta_c(p, m0 + wrow + g * BS + T::row(lane, r),
                               n0 + wn * 64 + T::col(lane, r));
    __syncthreads();                               // chunk 0 staged

    // lane BS*t + i reads A[row i][k + t]
    const int a_off = (lane / BS) * AS + wrow + (lane % BS);
    const int b_off = wn * 64 + bpos<WK, BN>(lane);
    // Whole chunks, then the partial last one (if any) after the loop: a
    // partial-chunk branch inside the loop made the compiler keep the
    // accumulators in two register sets and copy them on every chunk.
    // The MFMAs and their order are the same either way.
    const int nfull = p.K / KT;
    for (int c = 0; c < nfull; ++c) {
        const float* as = &As[c & 1][a_off];
        const float* bs = &Bs[c & 1][b_off];
        float a[2][R], b[2][NB];
#pragma unroll
        for (int g = 0; g < R; ++g) a[0][g] = as[g * BS];
#pragma unroll
        for (int t = 0; t < NB; ++t) b[0][t] = bs[t * BN];
#pragma unroll
        for (int kb = 0; kb < NBLK; ++kb) {
            const int cur = kb & 1;
            if (kb + 1 < NBLK) {
#pragma unroll
                for (int g = 0; g < R; ++g) a[cur ^ 1][g] = as[(kb + 1) * NB * AS + g * BS];
#pragma unroll
                for (int t = 0; t < NB; ++t) b[cur ^ 1][t] = bs[((kb + 1) * NB + t) * BN];
            }
            x_steps<T, R, 0>(a[cur], b[cur], acc);
        }
        __syncthreads();
    }
    if (const int kn = p.K - nfull * KT; kn > 0) {
        const float* as = &As[nfull & 1][a_off];
        const float* bs = &Bs[nfull & 1][b_off];
        for (int kb = 0; kb < kn; kb += NB) {
            float a[R], b[NB];
#pragma unroll
            for (int g = 0; g < R; ++g) a[g] = as[kb * AS + g * BS];
#pragma unroll
            for (int t = 0; t < NB; ++t) b[t] = bs[(kb + t) * BN];
            x_steps_n<T, R, 0>(a, b, acc, kn - kb);
        }
        __syncthreads();
    }

#pragma unroll
    for (int g = 0; g < R; ++g) {
#pragma unroll
        for (int r = 0; r < T::NACC; ++r) {
            const int row = m0 + wrow + g * BS + T::row(lane, r);
            const int col = n0 + wn * 64 + T::col(lane, r);
            if (row < p.M && col < p.N) store_c(p, acc[g][r], row, col);
        }
    }
}

// ---- configurations and dispatch -------------------------------------------

// Tile configurations: family, MFMA shape, chains per wave, waves along M
// and N, k per LDS chunk.  The set covers the encoder's shapes: short-M,
// long-K chains (latency bound: many waves, 4x4 MFMAs, producer waves), mid
// M (4x4 / 16x16 with 2-3 chains per wave) and long M (32x32 / 16x16 tiles,
// MFMA-throughput bound).
#define PK_CONFIGS(X)                                                       \
    X(0, 'R', 32, 2, 2, 2, 32)   /* 128 x 128, wave 64 x 64            */  \
    X(1, 'R', 32, 1, 2, 2, 32)   /* 128 x 64,  wave 64 x 32            */  \
    X(2, 'R', 16, 2, 1, 4, 32)   /*  64 x 128, wave 64 x 32            */  \
    X(3, 'R', 16, 1, 1, 4, 64)   /*  64 x 64,  wave 64 x 16            */  \
    X(4, 'R', 4, 1, 1, 4, 64)    /*  64 x 16,  wave 64 x 4             */  \
    X(5, 'X', 4, 1, 4, 1, 64)    /*  16 x 64,  wave 4 x 64, 1 chain    */  \
    X(6, 'X', 4, 2, 4, 1, 64)    /*  32 x 64,  wave 8 x 64, 2 chains   */  \
    X(7, 'X', 4, 4, 4, 1, 64)    /*  64 x 64,  wave 16 x 64, 4 chains  */  \
    X(8, 'X', 4, 1, 8, 1, 64)    /*  32 x 64,  8 waves, 1 chain        */  \
    X(9, 'X', 16, 1, 4, 1, 64)   /*  64 x 64,  wave 16 x 64            */  \
    X(10, 'X', 16, 2, 2, 2, 32)  /*  64 x 128, wave 32 x 64, 2 chains  */  \
    X(11, 'X', 32, 1, 4, 1, 32)  /* 128 x 64,  wave 32 x 64            */  \
    X(12, 'S', 4, 1, 4, 1, 64)   /*  16 x 64,  4 + 4 waves, 1 chain    */  \
    X(13, 'S', 4, 2, 4, 1, 64)   /*  32 x 64,  4 + 4 waves, 2 chains   */  \
    X(14, 'S', 4, 3, 4, 1, 64)   /*  48 x 64,  4 + 4 waves, 3 chains   */  \
    X(15, 'S', 4, 2, 4, 1, 32)   /*  32 x 64,  4 + 4 waves, 2 chains   */  \
    X(16, 'S', 4, 2, 4, 1, 128)  /*  32 x 64,  4 + 4 waves, 2 chains   */  \
    X(17, 'S', 4, 1, 8, 1, 128)  /*  32 x 64,  8 + 8 waves, 1 chain    */  \
    X(18, 'S', 16, 1, 4, 1, 64)  /*  64 x 64,  4 + 4 waves             */  \
    X(19, 'S', 32, 1, 4, 1, 32)  /* 128 x 64,  4 + 4 waves             */  \
    X(20, 'Y', 32, 1, 4, 1, 32)  /* 128 x 64,  as 11, 2 chunks in flight */ \
    X(21, 'Y', 32, 1, 4, 1, 16)  /* 128 x 64,  k 16, 2 chunks in flight */  \
    X(22, 'X', 32, 1, 4, 1, 16)  /* 128 x 64,  k 16 per chunk          */  \
    X(23, 'Y', 16, 1, 4, 1, 32)  /*  64 x 64,  2 chunks in flight      */

#define PK_CFG_ENTRY(i, fam, mf, c, wm, wn, kt) {fam, mf, c, wm, wn, kt},
static const TileConfig kConfigs[] = {PK_CONFIGS(PK_CFG_ENTRY)};
constexpr int kNumConfigs = sizeof(kConfigs) / sizeof(kConfigs[0]);

template <int WK, bool VEC, bool A1>
hipError_t launch_chain(int cfg, const KArgs& a, hipStream_t s)
{
    const TileConfig& t = kConfigs[cfg];
    dim3 grid((a.N + t.bn() - 1) / t.bn(), (a.M + t.bm() - 1) / t.bm());
    dim3 block(t.threads());
#define PK_CFG_CASE(i, fam, mf, c, wm, wn, kt)                                            \
    case i:                                                                               \
        if constexpr (fam == 'R')                                                         \
            hipLaunchKernelGGL((chain_gemm<WK, mf, c, wm, wn, kt, 2, VEC, A1>), grid, block, 0, s, a); \
        else if constexpr (fam == 'X' || fam == 'Y') {                                    \
            constexpr int pd = (VEC && fam == 'X') ? 4 : 2;                               \
            constexpr bool fk = VEC && A1 && kt == 32;                                    \
            if (fk && a.K % (pd * kt) == 0)                                               \
                hipLaunchKernelGGL((chain_gemm_x<WK, mf, c, wm, wn, kt, pd, VEC, A1, fk>), \
                                   grid, block, 0, s, a);                                 \
            else                                                                          \
                hipLaunchKernelGGL((chain_gemm_x<WK, mf, c, wm, wn, kt, pd, VEC, A1>),    \
                                   grid, block, 0, s, a);                                 \
        }                                                                                 \
        else {                                                                            \
            /* unaligned operands take per-element loads: 128-deep chunks of */           \
            /* them spilled, so those tiles stage 64-deep chunks (same chains) */         \
            constexpr int kts = (!VEC && kt == 128) ? 64 : kt;                            \
            hipLaunchKernelGGL((chain_gemm_xs<WK, mf, c, wm, wn, kts, 2, VEC, A1>), grid, block, 0, s, a); \
        }                                                                                 \
        break;
    switch (cfg) {
        PK_CONFIGS(PK_CFG_CASE)
    default: return hipErrorInvalidValue;
    }
#undef PK_CFG_CASE
    return hipGetLastError();
}

// alpha == 1 (every encoder call) stages A without the multiply.
template <int WK>
hipError_t launch_chain(int cfg, const KArgs& a, hipStream_t s)
{
    const bool vec = a.vec_a && a.vec_b, a1 = a.alpha == 1.0f;
    if (vec) return a1 ? launch_chain<WK, true, true>(cfg, a, s) : launch_chain<WK, true, false>(cfg, a, s);
    return a1 ? launch_chain<WK, false, true>(cfg, a, s) : launch_chain<WK, false, false>(cfg, a, s);
}

// Launchers of one weight format each (defined in pk_gemm_{f32,i8,i4}.hip).
hipError_t launch_chain_f32(int cfg, const KArgs& a, hipStream_t s);
hipError_t launch_chain_i8(int cfg, const KArgs& a, hipStream_t s);
hipError_t launch_chain_i4(int cfg, const KArgs& a, hipStream_t s);

}  // namespace tiles
}  // namespace pkgpu
