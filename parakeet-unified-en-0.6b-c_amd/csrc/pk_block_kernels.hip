// pk_block_kernels.hip - the conformer-block operations between the weight
// GEMMs, for the device-resident encoder: LayerNorm, relative-position
// multi-head attention (scores, relative shift, softmax, scores x V), GLU,
// and the depthwise convolution with its Swish.
//
// Activations are time-major rows of d_model = 1024 floats; several chunks
// of the chunked encoder (encoder.c:514-575) sit one after another in one
// buffer, and the per-chunk operations (attention, depthwise convolution)
// take the chunks' first rows from a small device table.
//
// Numerics follow the compiled reference (x86 AVX2 build), operation by
// operation, with every rounding explicit (__f*_rn, and the library is
// compiled with -ffp-contract=off so no multiply is fused into an add that
// the reference rounds separately): where the reference's
// order of operations is fixed by its source or by how it is compiled, the
// result is bit-identical (attention for T % 8 == 0, depthwise convolution,
// the LayerNorm sums).  Where the reference's build uses CPU-model-specific
// approximations (vrsqrtss for LayerNorm's 1/sqrt, vrcpps for Swish's and
// GLU's reciprocal) the value here is the IEEE operation its source writes
// (1/sqrtf, a division); glibc's vector expf in GLU is replaced by
// expf_ieee (pk_device_math.h).  Every function here is therefore a fixed
// sequence of IEEE operations that a CPU reproduces bit for bit.
#include "pk_block_kernels.h"
#include "pk_gemm_tiles.h"

#include <cstdlib>
#include <cstring>
#include <utility>

namespace pkgpu {
namespace {

using tiles::v4f;

__device__ inline float hsum8(const float (&p)[8])
{
    return __fadd_rn(__fadd_rn(__fadd_rn(p[0], p[4]), __fadd_rn(p[2], p[6])),
                     __fadd_rn(__fadd_rn(p[1], p[5]), __fadd_rn(p[3], p[7])));
}

// ---- LayerNorm (tensor_ops.c:150-185) ---------------------------------------
// One wave per 8 rows, 8 lanes per row; lane l of a row holds the partial
// sums of elements l, l+8, l+16, ... in order, like one AVX2 lane.  The rows
// come in with 16-byte loads into LDS (padded rows: the strided reads of the
// 64 lanes hit distinct banks but for 2-way overlaps), each lane keeps its
// NPL = D/8 elements in registers for the two sequential passes (sum,
// squared deviations) and writes the deviations back.  The outputs
// fl(fl(dev * inv) * gamma + beta) are independent, so they are formed per
// 16-byte group: each lane then needs 4 of gamma's and beta's groups
// (loaded first, with the rows) instead of 2 x NPL scattered values.
// In place (out == x) is safe: every row is read before any is written.

template <int NPL>
__global__ __launch_bounds__(64) void layer_norm_rows(const float* x, int ldx,
                                                      const float* __restrict__ gamma,
                                                      const float* __restrict__ beta,
                                                      float* out, int ldo, int rows)
{
    constexpr int D = 8 * NPL, LD = D + 8, V4 = D / 4, NQ = 8 * V4 / 64;
    static_assert(V4 % 64 == 0, "each lane's 16-byte groups repeat every 64 lanes");
    constexpr int NG = V4 / 64;                     // distinct column groups per lane
    __shared__ float buf[8 * LD];
    __shared__ float inv_row[8];
    const int lane = threadIdx.x;
    const int row0 = blockIdx.x * 8;
    const int nr = min(8, rows - row0);
    // all of a lane's row loads in flight at once (rows past the end read row
    // 0), then its gamma and beta groups: columns 4 * (lane + 64 j)
    float4 in[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int idx = lane + 64 * q, r = idx / V4, c4 = idx % V4;
        in[q] = *reinterpret_cast<const float4*>(x + (size_t)(r < nr ? row0 + r : row0) * ldx + 4 * c4);
    }
    float4 g4[NG], b4[NG];
#pragma unroll
    for (int j = 0; j < NG; ++j) {
        g4[j] = *reinterpret_cast<const float4*>(gamma + 4 * (lane + 64 * j));
        b4[j] = *reinterpret_cast<const float4*>(beta + 4 * (lane + 64 * j));
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int idx = lane + 64 * q;
        *reinterpret_cast<float4*>(buf + (idx / V4) * LD + 4 * (idx % V4)) = in[q];
    }
    __syncthreads();
    const int r = lane >> 3, l = lane & 7;
    float* br = buf + r * LD + l;
    float v[NPL];
#pragma unroll
    for (int i = 0; i < NPL; ++i) v[i] = br[8 * i];
    float p = 0.0f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) p = __fadd_rn(p, v[i]);
    const float mean = __fdiv_rn(hsum8_lanes(p), (float)D);
    float q = 0.0f;
#pragma unroll
    for (int i = 0; i < NPL; ++i) {
        v[i] = __fsub_rn(v[i], mean);
        q = __fmaf_rn(v[i], v[i], q);
    }
    const float var = __fdiv_rn(hsum8_lanes(q), (float)D);
    // sqrtf and '/' are correctly rounded here (HIP's __fsqrt_rn is the
    // native, approximate square root unless OCML_BASIC_ROUNDED_OPERATIONS).
    const float inv = 1.0f / sqrtf(__fadd_rn(var, 1e-5f));
#pragma unroll
    for (int i = 0; i < NPL; ++i) br[8 * i] = v[i];      // the deviations x - mean
    if (l == 0) inv_row[r] = inv;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int idx = lane + 64 * q, rr = idx / V4, c4 = idx % V4, j = q % NG;
        if (rr < nr) {
            const float4 d = *reinterpret_cast<const float4*>(buf + rr * LD + 4 * c4);
            const float s = inv_row[rr];
            float4 o;
            o.x = __fmaf_rn(__fmul_rn(d.x, s), g4[j].x, b4[j].x);
            o.y = __fmaf_rn(__fmul_rn(d.y, s), g4[j].y, b4[j].y);
            o.z = __fmaf_rn(__fmul_rn(d.z, s), g4[j].z, b4[j].z);
            o.w = __fmaf_rn(__fmul_rn(d.w, s), g4[j].w, b4[j].w);
            *reinterpret_cast<float4*>(out + (size_t)(row0 + rr) * ldo + 4 * c4) = o;
        }
    }
}

// LayerNorm with split outputs, the fast numerics mode's input to the split
// GEMMs: one workgroup of 4 waves per 8 rows.  The rows come in with 16-byte
// loads (8 per thread) into LDS, padded 8 floats per row.  Thread c owns
// columns 4c .. 4c + 3 of every row (one 16-byte group of gamma and of
// beta).  The statistics are ln_row_stats_rolled: 8 lanes per row (lanes
// 0-15 of each wave, 2 rows a wave), the same chains as layer_norm_rows.  The outputs
// fl(fl(fl(x - mean) * inv) * gamma + beta) are independent and formed per
// 16-byte group.  In place (out == x) is safe: a workgroup reads its rows
// before it writes them.  Each output o goes out split as the split GEMM
// kernels multiply it (hi = bf16(o), lo = bf16(o - hi), both to nearest: the
// split those kernels would make of the fp32 output), in their pre-split
// layout: per row and group of 8 columns, the 8 hi then the 8 lo, in the
// fp32 row's bytes.  The statistics loops stay rolled (82 VGPRs instead of
// 178): these workgroups run beside the other row group's split GEMMs, on
// the CUs those leave free, and more of them fit there.  Measured on the
// fast encoder pass (A/B on two boxes, two runs each): +0.3% and +1.5%
// against one wave per 8 rows.  The plain LayerNorm keeps that layout: in
// the exact pass the four-wave form measured 0.4% slower.
template <int NPL>
__global__ __launch_bounds__(256) void layer_norm_split_rows(const float* x, int ldx,
                                                             const float* __restrict__ gamma,
                                                             const float* __restrict__ beta,
                                                             float* out, int ldo, int rows)
{
    constexpr int D = 8 * NPL, LD = D + 8, V4 = D / 4, NQ = 8 * V4 / 256;
    static_assert(V4 == 256, "one 16-byte column group per thread");
    __shared__ float buf[8 * LD];
    __shared__ float st[8][2];                      // mean, inv per row
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int row0 = blockIdx.x * 8;
    const int nr = min(8, rows - row0);
    // every load in flight at once: row q of the workgroup, columns 4 tid
    // (rows past the end read row 0 of the workgroup)
    float4 in[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q)
        in[q] = *reinterpret_cast<const float4*>(x + (size_t)(q < nr ? row0 + q : row0) * ldx + 4 * tid);
    const float4 g4 = *reinterpret_cast<const float4*>(gamma + 4 * tid);
    const float4 b4 = *reinterpret_cast<const float4*>(beta + 4 * tid);
#pragma unroll
    for (int q = 0; q < NQ; ++q) *reinterpret_cast<float4*>(buf + q * LD + 4 * tid) = in[q];
    __syncthreads();
    if (lane < 16) {
        const int r = 2 * w + (lane >> 3), l = lane & 7;
        float mean, inv;
        ln_row_stats_rolled<32>(buf + r * LD, D, l, mean, inv);
        if (l == 0) {
            st[r][0] = mean;
            st[r][1] = inv;
        }
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        if (q < nr) {
            const float mean = st[q][0], s = st[q][1];
            const float4 v = in[q];
            float4 o;
            o.x = __fmaf_rn(__fmul_rn(__fsub_rn(v.x, mean), s), g4.x, b4.x);
            o.y = __fmaf_rn(__fmul_rn(__fsub_rn(v.y, mean), s), g4.y, b4.y);
            o.z = __fmaf_rn(__fmul_rn(__fsub_rn(v.z, mean), s), g4.z, b4.z);
            o.w = __fmaf_rn(__fmul_rn(__fsub_rn(v.w, mean), s), g4.w, b4.w);
            uint32_t h0, l0, h1, l1;
            split_bf16x2(o.x, o.y, h0, l0);
            split_bf16x2(o.z, o.w, h1, l1);
            // columns 4 tid .. +3: half (tid & 1) of group tid / 2, whose
            // 16 bf16 values occupy the group's 8 floats
            unsigned short* g8 = reinterpret_cast<unsigned short*>(
                out + (size_t)(row0 + q) * ldo + 8 * (tid >> 1));
            *reinterpret_cast<uint2*>(g8 + 4 * (tid & 1)) = make_uint2(h0, h1);
            *reinterpret_cast<uint2*>(g8 + 8 + 4 * (tid & 1)) = make_uint2(l0, l1);
        }
    }
}

// ---- relative-position attention (encoder.c:300-408) ------------------------
// One workgroup: 32 query rows of one head of one chunk, 4 waves of 8 rows.
// Products use v_mfma_f32_4x4x1_16b_f32 with block 0's A broadcast to all 16
// blocks (CBSZ = 4): one MFMA = 4 rows x 64 columns, lane j holds column j of
// rows 0..3, and the A register lane 4t + i holds row i at k-step t (ABID =
// t).  Each MFMA is one fused multiply-add per output.
//
// Scores (NT dot products, blas.c:221-249): eight accumulators per output,
// step k goes to accumulator k % 8, so accumulator l is the chain over
// k = l, l+8, ... of one AVX2 lane; the eight are reduced as hsum8.
// AC = Q_u K^T per column tile of keys; BD = Q_v P^T per tile of position
// rows m, scattered to the score of column j = m - (T-1-i) (the relative
// shift, encoder.c:230-254).  Softmax per row (tensor_ops.c:336-357), then
// scores x V as one fma chain per output over j ascending (sgemm NN).

constexpr int kDh = 128;                 // PK_HEAD_DIM
constexpr int kTileLd = kDh + 4;         // padded LDS row of a value tile
constexpr float kScoreScale = 0.0883883461356163f;   // 1/sqrtf(128) = 0x3db504f3
static_assert(kTileLd == 132, "attn_short_lds_bytes counts staged rows of 132 floats");

template <int T_>
__device__ inline v4f mfma_bcast(float a, float b, v4f c)
{
    return __builtin_amdgcn_mfma_f32_4x4x1f32(a, b, c, 4, T_, 0);
}

// acc[g][t % 8] += A_g(step t) * b[t] for the 16 steps of one A register.
template <int... Ts>
__device__ inline void score_steps(std::integer_sequence<int, Ts...>, const float (&a)[2],
                                   const float (&b)[16], v4f (&acc)[2][8])
{
    ((acc[0][Ts & 7] = mfma_bcast<Ts>(a[0], b[Ts], acc[0][Ts & 7]),
      acc[1][Ts & 7] = mfma_bcast<Ts>(a[1], b[Ts], acc[1][Ts & 7])), ...);
}

// Tiles staged through LDS, fetched into registers (4 float4 per thread of
// the 256) one tile ahead of their use; source rows outside [0, n) read as 0.
//   half tile:  64 rows x 64 columns (from column c0) of keys or positions,
//               LDS row stride kHalfLd
//   value tile: 32 rows x 128 columns of values, LDS row stride kTileLd
constexpr int kHalfLd = 64 + 4;
constexpr int kTileFloats = 64 * kHalfLd;          // >= 32 * kTileLd
static_assert(32 * kTileLd <= kTileFloats, "one LDS buffer holds either tile");

struct TileRegs {
    float4 v[4];
};

// The rows of one head's keys, values or positions: row r at src + r * ld,
// rows [0, n) valid, 128 columns each.  A tile's loads go through a buffer
// descriptor that starts at the tile's first row and ends after row n - 1,
// so rows past the end read as 0 without a predicate (the hardware's range
// check) and each thread's offsets are the same for every tile.
struct TileSrc {
    const float* src;
    int ld, n;
    __device__ __amdgpu_buffer_rsrc_t at(int r0) const     // r0 >= 0, uniform
    {
        const long long left = ((long long)(n - 1 - r0) * ld + kDh) * 4;
        return tiles::make_rsrc(src + (size_t)r0 * ld, left > 0 ? (uint32_t)left : 0u);
    }
};

__device__ inline float4 as_float4(tiles::v4u u)
{
    return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z),
                       __uint_as_float(u.w));
}

__device__ inline void load_half(TileRegs& t, const TileSrc& s, int r0, int c0)
{
    const __amdgpu_buffer_rsrc_t rs = s.at(r0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int idx = threadIdx.x + 256 * q;
        t.v[q] = as_float4(tiles::ld_v4(rs, (uint32_t)((idx >> 4) * s.ld + c0 + 4 * (idx & 15)) * 4u));
    }
}

__device__ inline void store_half(float* tile, const TileRegs& t)
{
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int idx = threadIdx.x + 256 * q;
        *reinterpret_cast<float4*>(tile + (idx >> 4) * kHalfLd + 4 * (idx & 15)) = t.v[q];
    }
}

__device__ inline void load_vtile(TileRegs& t, const TileSrc& s, int r0)
{
    const __amdgpu_buffer_rsrc_t rs = s.at(r0);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int idx = threadIdx.x + 256 * q;
        t.v[q] = as_float4(tiles::ld_v4(rs, (uint32_t)((idx >> 5) * s.ld + 4 * (idx & 31)) * 4u));
    }
}

__device__ inline void store_vtile(float* tile, const TileRegs& t)
{
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int idx = threadIdx.x + 256 * q;
        *reinterpret_cast<float4*>(tile + (idx >> 5) * kTileLd + 4 * (idx & 31)) = t.v[q];
    }
}

// One 4-row x 64-column tile of NT dot products for two row groups of a wave,
// accumulated over the two 64-column halves of k: a[g][kb] holds rows
// (4g..4g+3) in broadcast layout for k in [16kb, 16kb+16); half H covers
// kb = 4H..4H+3 from the half tile in LDS.  Chain t % 8 of each output takes
// k ascending across both halves.  The B fragments of the next 16 k-steps are
// read from LDS while the current 32 MFMAs issue (the scheduling barrier
// keeps that order).
template <int H>
__device__ inline void score_half(const float* tile, const float (&a)[2][8], v4f (&acc)[2][8])
{
    const int lane = threadIdx.x & 63;
    const float* trow = tile + lane * kHalfLd;
    float b[2][16];
    auto fetch = [&](float (&dst)[16], int kb) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = *reinterpret_cast<const float4*>(trow + kb * 16 + 4 * q);
            dst[4 * q] = v.x; dst[4 * q + 1] = v.y; dst[4 * q + 2] = v.z; dst[4 * q + 3] = v.w;
        }
    };
    fetch(b[0], 0);
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
        if (kb + 1 < 4) fetch(b[(kb + 1) & 1], kb + 1);
        __builtin_amdgcn_sched_barrier(0);
        const float ak[2] = {a[0][4 * H + kb], a[1][4 * H + kb]};
        score_steps(std::make_integer_sequence<int, 16>{}, ak, b[kb & 1], acc);
        __builtin_amdgcn_sched_barrier(0);
    }
}

__device__ inline void score_sums(const v4f (&acc)[2][8], float (&out)[2][4])
{
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float p[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) p[l] = acc[g][l][i];
            out[g][i] = hsum8(p);
        }
}

// The 32 x 64 scores of source rows [c, c + 64) (keys or positions; rows
// past the end read 0), through the two half tiles: pre holds the first half
// on entry and the next tile's first half (rows [c + 64, ...), when next is
// set) on return.  Both barriers of each half are taken by the whole
// workgroup.
__device__ inline void score_block(float* tile, TileRegs& pre, const TileSrc& src, int c, bool next,
                                   const float (&a)[2][8], float (&out)[2][4])
{
    v4f acc[2][8];
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int l = 0; l < 8; ++l) acc[g][l] = v4f{0.f, 0.f, 0.f, 0.f};
    store_half(tile, pre);
    __syncthreads();
    load_half(pre, src, c, 64);
    score_half<0>(tile, a, acc);
    __syncthreads();
    store_half(tile, pre);
    __syncthreads();
    if (next) load_half(pre, src, c + 64, 0);
    score_half<1>(tile, a, acc);
    score_sums(acc, out);
}

// scores x V: acc[g][d] += S[row 4g+i][j0 + t] * V[j0 + t][64d + lane].
// Full blocks of 16 steps read all 32 value fragments first, then issue the
// 64 MFMAs; a partial last block steps with a bound.
template <int... Ts>
__device__ inline void pv_steps_full(std::integer_sequence<int, Ts...>, const float (&a)[2],
                                     const float* vt, v4f (&acc)[2][2])
{
    const int lane = threadIdx.x & 63;
    float b0[16], b1[16];
    ((b0[Ts] = vt[Ts * kTileLd + lane], b1[Ts] = vt[Ts * kTileLd + 64 + lane]), ...);
    ((acc[0][0] = mfma_bcast<Ts>(a[0], b0[Ts], acc[0][0]),
      acc[1][0] = mfma_bcast<Ts>(a[1], b0[Ts], acc[1][0]),
      acc[0][1] = mfma_bcast<Ts>(a[0], b1[Ts], acc[0][1]),
      acc[1][1] = mfma_bcast<Ts>(a[1], b1[Ts], acc[1][1])), ...);
}

template <int... Ts>
__device__ inline void pv_steps(std::integer_sequence<int, Ts...>, const float (&a)[2],
                                const float* vt, int n, v4f (&acc)[2][2])
{
    const int lane = threadIdx.x & 63;
    (((Ts < n) ? (acc[0][0] = mfma_bcast<Ts>(a[0], vt[Ts * kTileLd + lane], acc[0][0]),
                  acc[1][0] = mfma_bcast<Ts>(a[1], vt[Ts * kTileLd + lane], acc[1][0]),
                  acc[0][1] = mfma_bcast<Ts>(a[0], vt[Ts * kTileLd + 64 + lane], acc[0][1]),
                  acc[1][1] = mfma_bcast<Ts>(a[1], vt[Ts * kTileLd + 64 + lane], acc[1][1]), 0)
               : 0), ...);
}

// Workgroups are dispatched to the 8 XCDs round-robin; renumber them so
// each XCD runs a contiguous run of (row block, head, chunk) tasks, row
// block fastest: the row blocks of one head of one chunk then share one
// XCD's L2 for their K, P and V rows.  Returns the task number.
__device__ inline int attn_task(int& rb, int& h, int& z)
{
    const int nrb = gridDim.x, nh = gridDim.y, total = nrb * nh * gridDim.z;
    const int lin = blockIdx.x + nrb * (blockIdx.y + nh * blockIdx.z);
    const int xcd = lin % 8, local = lin / 8;
    const int base = total / 8, extra = total % 8;
    const int task = xcd * base + min(xcd, extra) + local;
    rb = task % nrb;
    h = (task / nrb) % nh;
    z = task / (nrb * nh);
    return task;
}

// Softmax of one score row s[0, T) in place (tensor_ops.c:336-357), by the 8
// lanes of an aligned group (lane q owns j = q, q+8, ...): the row maximum,
// e = exp(s - max) with the partial sums of each lane in order, hsum8; the
// last T % 8 entries by one lane, in order (the reference's scalar tail);
// then s * (1 / sum).  A row past the sequence (live false) is zeroed.
__device__ inline void softmax_row(float* s, int T, bool live)
{
    const int lane = threadIdx.x & 63, q = lane & 7;
    if (live) {
        float mx = s[0];
#pragma unroll 8
        for (int j = q; j < T; j += 8) mx = fmaxf(mx, s[j]);
        mx = fmaxf(mx, __shfl_xor(mx, 4));
        mx = fmaxf(mx, __shfl_xor(mx, 2));
        mx = fmaxf(mx, __shfl_xor(mx, 1));
        const int T8 = T & ~7;
        float part = 0.0f;
#pragma unroll 8
        for (int j = q; j < T8; j += 8) {
            const float e = exp_poly(__fsub_rn(s[j], mx));
            s[j] = e;
            part = __fadd_rn(part, e);
        }
        float sum = hsum8_lanes(part);
        if (T8 < T) {                 // scalar tail, one lane, in order
            if (q == 0)
                for (int j = T8; j < T; ++j) {
                    const float e = expf_ieee(__fsub_rn(s[j], mx));
                    s[j] = e;
                    sum = __fadd_rn(sum, e);
                }
            sum = __shfl(sum, lane & ~7);
        }
        const float inv = __fdiv_rn(1.0f, sum);
#pragma unroll 8
        for (int j = q; j < T; j += 8) s[j] = __fmul_rn(s[j], inv);
    } else {
        for (int j = q; j < T; j += 8) s[j] = 0.0f;
    }
}

// kGlobal: the block's score rows live in its own slice of p.scores (task
// order) instead of LDS, for sequences beyond kAttnMaxT; every operation and
// its order are the same, and __syncthreads orders the workgroup's global
// writes as it does its LDS writes.
template <bool kGlobal>
__global__ __launch_bounds__(256, 2) void rel_pos_attention(AttnArgs p)
{
    // Scores of the block's rows [kAttnRows][sld], then one staging tile.
    extern __shared__ float smem[];
    const int sld = attn_sld(p.T);

    // (row block, head, chunk) in XCD runs
    int rb, h, z;
    const int task = attn_task(rb, h, z);
    float* S = kGlobal ? p.scores + (size_t)task * kAttnRows * sld : smem;
    float* tile = kGlobal ? smem : smem + kAttnRows * sld;
    const int T = p.chunk_T ? p.chunk_T[z] : p.T;           // this chunk's rows
    const int r0 = rb * kAttnRows;
    if (r0 >= T) return;                                     // the whole workgroup
    const int row0 = p.chunk_rows ? p.chunk_rows[z] : 0;   // first row of this chunk
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int D = p.H * kDh;
    const float* qkv = p.qkv + (size_t)row0 * p.ldq;
    const float* K = qkv + D + h * kDh;
    const float* V = qkv + 2 * D + h * kDh;
    const float* P = p.P + (size_t)(p.T - T) * p.ldp + h * kDh;

    // Q_u, Q_v rows of this wave in broadcast layout (encoder.c:319-338).
    float au[2][8], av[2][8];
    {
        const int i = lane & 3, t = lane >> 2;
        // every load is unconditional (rows past T read row T-1 and are
        // zeroed after), so they are all in flight together
        float qv[2][8], bu[8], bv[8];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const int r = min(r0 + 8 * w + 4 * g + i, T - 1);
            const float* q = qkv + (size_t)r * p.ldq + h * kDh;
#pragma unroll
            for (int kb = 0; kb < 8; ++kb) qv[g][kb] = q[16 * kb + t];
        }
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            bu[kb] = p.pos_bias_u[h * kDh + 16 * kb + t];
            bv[kb] = p.pos_bias_v[h * kDh + 16 * kb + t];
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            const bool live = r0 + 8 * w + 4 * g + i < T;
#pragma unroll
            for (int kb = 0; kb < 8; ++kb) {
                au[g][kb] = live ? __fadd_rn(qv[g][kb], bu[kb]) : 0.0f;
                av[g][kb] = live ? __fadd_rn(qv[g][kb], bv[kb]) : 0.0f;
            }
        }
    }

    // AC: S[row][j] = Q_u[row] . K[j]
    TileRegs pre;
    const TileSrc ks{K, p.ldq, T};
    load_half(pre, ks, 0, 0);
    for (int j0 = 0; j0 < T; j0 += 64) {
        float o[2][4];
        score_block(tile, pre, ks, j0, j0 + 64 < T, au, o);
        const int j = j0 + lane;
        if (j < T)
#pragma unroll
            for (int g = 0; g < 2; ++g)
#pragma unroll
                for (int i = 0; i < 4; ++i) S[(8 * w + 4 * g + i) * sld + j] = o[g][i];
        __syncthreads();
    }

    // BD at the shifted positions: m = T-1-row+j for this block's rows.
    const int r_hi = min(r0 + kAttnRows, T) - 1;
    const int L = 2 * T - 1;
    const int m_first = T - 1 - r_hi, m_last = 2 * T - 2 - r0;
    const TileSrc ps{P, p.ldp, L};
    load_half(pre, ps, m_first, 0);
    for (int m0 = m_first; m0 <= m_last; m0 += 64) {
        float o[2][4];
        score_block(tile, pre, ps, m0, m0 + 64 <= m_last, av, o);
        // every (row, j) takes exactly one shifted BD value: row rl of the
        // block takes column j = jb + rl, whose score is at S[jb + rl (sld + 1)].
        // Read the eight scores first, then write them back combined.
        const int jb = m0 + lane - (T - 1) + r0;
        float sc[2][4];
        bool ok[2][4];
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int rl = 8 * w + 4 * g + i;           // uniform in the wave
                ok[g][i] = r0 + rl < T && (unsigned)(jb + rl) < (unsigned)T;
                sc[g][i] = S[ok[g][i] ? jb + rl * (sld + 1) : 0];
            }
#pragma unroll
        for (int g = 0; g < 2; ++g)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (ok[g][i])
                    S[jb + (8 * w + 4 * g + i) * (sld + 1)] =
                        __fmul_rn(__fadd_rn(sc[g][i], o[g][i]), kScoreScale);
        __syncthreads();
    }
    const TileSrc vs{V, p.ldq, T};
    load_vtile(pre, vs, 0);               // the first value tile, during the softmax

    // Softmax of each row: 8 lanes per row
    {
        const int rl = 8 * w + (lane >> 3);
        softmax_row(S + rl * sld, T, r0 + rl < T);
    }
    __syncthreads();

    // out[row][h*128 + d] = sum over j ascending of S[row][j] * V[j][d],
    // through 32-row value tiles: whole blocks of 16 keys in the loop, the
    // last T % 16 keys after it, from the last tile (still in LDS: the loop's
    // last pass takes no closing barrier).
    v4f acc[2][2];
#pragma unroll
    for (int g = 0; g < 2; ++g) acc[g][0] = acc[g][1] = v4f{0.f, 0.f, 0.f, 0.f};
    const int i = lane & 3, t = lane >> 2;
    const float* srow[2] = {S + (8 * w + i) * sld + t, S + (8 * w + 4 + i) * sld + t};
    int j0 = 0;
    for (;; j0 += 32) {
        store_vtile(tile, pre);
        __syncthreads();
        const bool more = j0 + 32 < T;
        if (more) load_vtile(pre, vs, j0 + 32);
#pragma unroll
        for (int jb = 0; jb < 32; jb += 16) {
            if (j0 + jb + 16 <= T) {
                const float a[2] = {srow[0][j0 + jb], srow[1][j0 + jb]};
                pv_steps_full(std::make_integer_sequence<int, 16>{}, a, tile + jb * kTileLd, acc);
            }
        }
        if (!more) break;
        __syncthreads();
    }
    if (T & 15) {
        const int jb = (T & ~15) - j0;                  // 0 or 16 within the last tile
        const int jj = (T & ~15) + t;
        const float a[2] = {jj < T ? srow[0][T & ~15] : 0.0f, jj < T ? srow[1][T & ~15] : 0.0f};
        pv_steps(std::make_integer_sequence<int, 16>{}, a, tile + jb * kTileLd, T & 15, acc);
    }
    float* out = p.out + (size_t)row0 * p.ldo + h * kDh;
#pragma unroll
    for (int g = 0; g < 2; ++g)
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int r = r0 + 8 * w + 4 * g + ii;
            if (r < T) {
                out[(size_t)r * p.ldo + lane] = acc[g][0][ii];
                out[(size_t)r * p.ldo + 64 + lane] = acc[g][1][ii];
            }
        }
}

// ---- fast numerics: attention on split bf16 operands -------------------------
// Under PK_GPU_NUMERICS_FAST the attention of chunks of kAttnShortT < T <=
// kAttnMaxT rows multiplies on v_mfma_f32_16x16x32_bf16 with each operand
// split as the split GEMM kernels split theirs (x = hi + lo + r, hi =
// bf16(x), lo = bf16(x - hi), r below 2^-16 |x|): three products hi hi +
// lo hi + hi lo per pair, within about 1e-5 of the exact kernel.  The
// organisation is rel_pos_attention's: 32 query rows of one head of one
// chunk per workgroup, their score rows in LDS, the content scores, then
// the relative-position term added at the shifted positions, softmax, then
// scores x V.  Fragments of v_mfma_f32_16x16x32_bf16: lane l = i + 16 g
// holds row (A) or column (B) i and k = 8 g .. 8 g + 7 of a 32-deep step;
// the 16 x 16 result gives lane l column i and rows 4 g .. 4 g + 3.
// attn_fast_prep writes every B operand pre-split in fragment order, each
// fragment 2 KB: the 64 lanes' 16-byte hi parts, then their lo parts, so a
// wave's fragment load is 1 KB contiguous:
//   Kf [n][H][KB][4]  keys: fragment (z, h, kb, s) holds key 16 kb + i of
//                     chunk z, columns 32 s + 8 g .. of head h (KB = T/16
//                     rounded up; keys past the chunk's end 0)
//   Pf [H][PB][4]     the launch's position rows: (h, pb, s) holds row
//                     16 pb + i, columns 32 s + 8 g .. of head h
//   Vf [n][H][8][TS]  values: (z, h, db, t) holds column 16 db + i and keys
//                     32 t + 8 g .. of chunk z (TS = T/32 rounded up)
typedef uint32_t fa_v4u __attribute__((ext_vector_type(4)));
typedef __bf16 fa_v8bf __attribute__((ext_vector_type(8)));
constexpr int kFragFloats = 512;                  // one fragment, hi and lo, 2 KB
// Score-row stride of the split kernel, 4 more than a multiple of 32 floats:
// the 4 lane groups of a result store, and the 16 rows of a fragment read,
// start 4 or 16 banks apart (8 apart, rel_pos_attention's stride, put the
// 4 groups of a store on the same banks).
__host__ __device__ constexpr int fa_sld(int T) { return ((T + 31) & ~31) + 4; }

struct FaLayout {
    int KB, PB, TS;                               // key blocks, position blocks, value steps
    size_t kf, pf;                                // Kf, Pf offsets in floats (Vf follows Pf)
    __host__ __device__ FaLayout(int T, int H, int n)
    {
        KB = (T + 15) / 16;
        PB = (2 * T - 1 + 15) / 16;
        TS = (T + 31) / 32;
        kf = 0;
        pf = (size_t)n * H * KB * 4 * kFragFloats;
    }
    __host__ __device__ size_t vf(int H) const { return pf + (size_t)H * PB * 4 * kFragFloats; }
    __host__ __device__ size_t floats(int H, int n) const { return vf(H) + (size_t)n * H * 8 * TS * kFragFloats; }
};

__device__ inline __amdgpu_buffer_rsrc_t fa_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// 8 floats -> their bf16 hi and lo halves, in order
__device__ inline void fa_split8(const float (&x)[8], fa_v4u& hi, fa_v4u& lo)
{
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint32_t h, l;
        split_bf16x2(x[2 * k], x[2 * k + 1], h, l);
        hi[k] = h;
        lo[k] = l;
    }
}

// this lane's part of fragment f (in fragments from the buffer's start);
// past the buffer's extent both read 0
__device__ inline void fa_load(__amdgpu_buffer_rsrc_t r, uint32_t f, fa_v8bf& hi, fa_v8bf& lo)
{
    const uint32_t byte = f * (kFragFloats * 4) + (threadIdx.x & 63) * 16;
    hi = __builtin_bit_cast(fa_v8bf, __builtin_amdgcn_raw_buffer_load_b128(r, (int)byte, 0, 0));
    lo = __builtin_bit_cast(fa_v8bf, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(byte + 1024), 0, 0));
}

__device__ inline v4f fa_mfma3(fa_v8bf ah, fa_v8bf al, fa_v8bf bh, fa_v8bf bl, v4f c)
{
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bh, c, 0, 0, 0);
    c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al, bh, c, 0, 0, 0);
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah, bl, c, 0, 0, 0);
}

// One thread per (fragment, lane): its 8 source values, split, to the
// fragment's hi and lo parts.  Keys, then position rows, then values.
__global__ __launch_bounds__(256) void attn_fast_prep(AttnArgs p, int n_chunks, float* ws)
{
    const FaLayout L(p.T, p.H, n_chunks);
    const int D = p.H * kDh;
    const long long nk = (long long)n_chunks * p.H * L.KB * 4 * 64, np = (long long)p.H * L.PB * 4 * 64;
    const long long nv = (long long)n_chunks * p.H * 8 * L.TS * 64;
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int l = (int)(idx & 63), i = l & 15, g = l >> 4;
    const long long f = idx >> 6;                 // fragment within its operand
    float x[8];
    float* dst;
    if (idx < nk) {
        const int s = (int)(f % 4), kb = (int)(f / 4 % L.KB), h = (int)(f / 4 / L.KB % p.H), z = (int)(f / 4 / L.KB / p.H);
        const int Tz = p.chunk_T ? p.chunk_T[z] : p.T, row0 = p.chunk_rows ? p.chunk_rows[z] : 0;
        const int j = 16 * kb + i;
        if (j < Tz) {
            const float4* src = reinterpret_cast<const float4*>(p.qkv + (size_t)(row0 + j) * p.ldq + D + h * kDh + 32 * s + 8 * g);
            const float4 a = src[0], b = src[1];
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = 0.0f;
        }
        dst = ws + L.kf + (size_t)f * kFragFloats;
    } else if (idx < nk + np) {
        const long long q = f - nk / 64;
        const int s = (int)(q % 4), pb = (int)(q / 4 % L.PB), h = (int)(q / 4 / L.PB);
        const int m = 16 * pb + i;
        if (m < 2 * p.T - 1) {
            const float4* src = reinterpret_cast<const float4*>(p.P + (size_t)m * p.ldp + h * kDh + 32 * s + 8 * g);
            const float4 a = src[0], b = src[1];
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = 0.0f;
        }
        dst = ws + L.pf + (size_t)q * kFragFloats;
    } else if (idx < nk + np + nv) {
        const long long q = f - (nk + np) / 64;
        const int t = (int)(q % L.TS), db = (int)(q / L.TS % 8), h = (int)(q / L.TS / 8 % p.H), z = (int)(q / L.TS / 8 / p.H);
        const int Tz = p.chunk_T ? p.chunk_T[z] : p.T, row0 = p.chunk_rows ? p.chunk_rows[z] : 0;
        const float* v = p.qkv + 2 * D + h * kDh + 16 * db + i;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int j = 32 * t + 8 * g + e;
            x[e] = j < Tz ? v[(size_t)(row0 + j) * p.ldq] : 0.0f;
        }
        dst = ws + L.vf(p.H) + (size_t)q * kFragFloats;
    } else {
        return;
    }
    fa_v4u hi, lo;
    fa_split8(x, hi, lo);
    reinterpret_cast<fa_v4u*>(dst)[l] = hi;
    reinterpret_cast<fa_v4u*>(dst + 256)[l] = lo;
}

// Q + bias of this lane's fragment rows r0 + 16 b + i (rows past T repeat
// row T - 1: their scores are zeroed and their outputs not stored), split.
__device__ inline void fa_qfrags(const AttnArgs& p, const float* bias, int row0, int r0, int T, int h,
                                 fa_v8bf (&qh)[2][4], fa_v8bf (&ql)[2][4])
{
    const int lane = threadIdx.x & 63, i = lane & 15, g = lane >> 4;
#pragma unroll
    for (int b = 0; b < 2; ++b) {
        const int r = min(r0 + 16 * b + i, T - 1);
        const float* q = p.qkv + (size_t)(row0 + r) * p.ldq + h * kDh;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int d = 32 * s + 8 * g;
            const float4 a0 = *reinterpret_cast<const float4*>(q + d), a1 = *reinterpret_cast<const float4*>(q + d + 4);
            const float4 u0 = *reinterpret_cast<const float4*>(bias + h * kDh + d);
            const float4 u1 = *reinterpret_cast<const float4*>(bias + h * kDh + d + 4);
            const float x[8] = {__fadd_rn(a0.x, u0.x), __fadd_rn(a0.y, u0.y), __fadd_rn(a0.z, u0.z),
                                __fadd_rn(a0.w, u0.w), __fadd_rn(a1.x, u1.x), __fadd_rn(a1.y, u1.y),
                                __fadd_rn(a1.z, u1.z), __fadd_rn(a1.w, u1.w)};
            fa_v4u hi, lo;
            fa_split8(x, hi, lo);
            qh[b][s] = __builtin_bit_cast(fa_v8bf, hi);
            ql[b][s] = __builtin_bit_cast(fa_v8bf, lo);
        }
    }
}

// MAXT: the launch's T rounded up to 64 (the unrolled loops' bound)
template <int MAXT>
__global__ __launch_bounds__(256, 2) void rel_pos_attention_fast(AttnArgs p, const float* ws)
{
    extern __shared__ float S[];                     // [kAttnRows][sld] score rows
    const int sld = fa_sld(p.T);
    int rb, h, z;
    attn_task(rb, h, z);
    const int T = p.chunk_T ? p.chunk_T[z] : p.T;
    const int r0 = rb * kAttnRows;
    if (r0 >= T) return;                             // the whole workgroup
    const int row0 = p.chunk_rows ? p.chunk_rows[z] : 0;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6, i = lane & 15, g = lane >> 4;
    const FaLayout L(p.T, p.H, gridDim.z);
    const auto rK = fa_rsrc(ws + L.kf, (uint32_t)((L.pf - L.kf) * 4));
    const auto rP = fa_rsrc(ws + L.pf, (uint32_t)((L.vf(p.H) - L.pf) * 4));
    const auto rV = fa_rsrc(ws + L.vf(p.H), (uint32_t)((L.floats(p.H, gridDim.z) - L.vf(p.H)) * 4));

    // Every operand fragment comes from L2: each phase keeps kRing tiles
    // (steps) of loads in flight in a ring of register sets, refilled right
    // after the set is multiplied.  The loops run to their bounds at T =
    // kAttnMaxT, unrolled, and every tile is multiplied: past the chunk's
    // last tile the loads repeat it and only the stores are skipped (their
    // keys or positions fall outside the chunk).  A loop back edge made the
    // compiler wait for every load in flight at its head, and a multiply
    // under a branch let it sink the tile's loads next to their use.
    constexpr int kRing = 3, kRingV = 6;
    constexpr int kAcTiles = MAXT / 64;                      // content tiles
    constexpr int kBdTiles = (MAXT + 45) / 64 + 1;           // position tiles (span T + 45 at most)
    constexpr int kPvSteps = MAXT / 32;                      // value steps

    // content scores: wave w takes keys 64 t + 16 w .. + 15 of tile t
    {
        fa_v8bf qh[2][4], ql[2][4];
        fa_qfrags(p, p.pos_bias_u, row0, r0, T, h, qh, ql);
        const int nt = (T + 63) / 64;
        fa_v8bf kh[kRing][4], kl[kRing][4];
        const uint32_t kf0 = (uint32_t)((z * p.H + h) * L.KB) * 4;
        auto load = [&](fa_v8bf (&bh)[4], fa_v8bf (&bl)[4], int t) {
            const uint32_t kb = (uint32_t)(4 * min(t, nt - 1) + w);
#pragma unroll
            for (int s = 0; s < 4; ++s) fa_load(rK, kf0 + 4 * kb + s, bh[s], bl[s]);
        };
#pragma unroll
        for (int k = 0; k < kRing; ++k) load(kh[k], kl[k], k);
#pragma unroll
        for (int t0 = 0; t0 < kAcTiles; t0 += kRing) {
#pragma unroll
            for (int k = 0; k < kRing; ++k) {
                const int t = t0 + k;
                v4f acc[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int b = 0; b < 2; ++b) acc[b] = fa_mfma3(qh[b][s], ql[b][s], kh[k][s], kl[k][s], acc[b]);
                const int jj = 64 * t + 16 * w + i;
                if (jj < T)
#pragma unroll
                    for (int b = 0; b < 2; ++b)
#pragma unroll
                        for (int v = 0; v < 4; ++v) S[(16 * b + 4 * g + v) * sld + jj] = acc[b][v];
                load(kh[k], kl[k], t + kRing);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    __syncthreads();

    // position term at the shifted positions m = T - 1 - row + j (each (row,
    // j) takes exactly one m, so no two lanes write one score); wave w takes
    // m_first + 64 t + 16 w .. + 15 of tile t
    {
        fa_v8bf qh[2][4], ql[2][4];
        fa_qfrags(p, p.pos_bias_v, row0, r0, T, h, qh, ql);
        const int r_hi = min(r0 + kAttnRows, T) - 1;
        const int m_first = T - 1 - r_hi, m_last = 2 * T - 2 - r0;
        // tiles of 64 launch rows m' = pbase + m from a multiple of 16; the
        // positions outside [m_first, m_last] give no (row, j) in range
        const int pbase = p.T - T;                   // this chunk's rows within the launch's P
        const int a0 = (pbase + m_first) & ~15;
        const int nt = (pbase + m_last - a0) / 64 + 1;
        const uint32_t pf0 = (uint32_t)(h * L.PB) * 4;
        fa_v8bf ph[kRing][4], pl[kRing][4];
        auto load = [&](fa_v8bf (&bh)[4], fa_v8bf (&bl)[4], int t) {
            const uint32_t pb = (uint32_t)((a0 >> 4) + 4 * min(t, nt - 1) + w);
#pragma unroll
            for (int s = 0; s < 4; ++s) fa_load(rP, pf0 + 4 * pb + s, bh[s], bl[s]);
        };
#pragma unroll
        for (int k = 0; k < kRing; ++k) load(ph[k], pl[k], k);
#pragma unroll
        for (int t0 = 0; t0 < kBdTiles; t0 += kRing) {
#pragma unroll
            for (int k = 0; k < kRing; ++k) {
                const int t = t0 + k;
                v4f acc[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int b = 0; b < 2; ++b) acc[b] = fa_mfma3(qh[b][s], ql[b][s], ph[k][s], pl[k][s], acc[b]);
                // past the last tile every j falls at or past T
                const int mm = a0 + 64 * t + 16 * w + i - pbase;
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int rl = 16 * b + 4 * g + v, j = mm - (T - 1) + r0 + rl;
                        if (r0 + rl < T && (unsigned)j < (unsigned)T) {
                            float* sp = S + rl * sld + j;
                            *sp = __fmul_rn(__fadd_rn(*sp, acc[b][v]), kScoreScale);
                        }
                    }
                load(ph[k], pl[k], t + kRing);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    __syncthreads();

    // softmax of each row, 8 lanes a row, lane q taking the groups of 8
    // scores q, q + 8, ...: max, exp and sum, then each group scaled and
    // written back split in place (its 8 hi, then its 8 lo bf16 values: the
    // A fragment scores x V reads), groups up to T rounded to 32 (zeros past
    // T; a row past the chunk all zeros).
    {
        const int rl = 8 * w + (lane >> 3), q = lane & 7;
        float* sr = S + rl * sld;
        const int ng = (T + 7) / 8, ngp = (T + 31) / 32 * 4;
        const bool live = r0 + rl < T;
        float mx = -INFINITY, sum = 0.0f;
        if (live) {
            for (int gi = q; gi < ng; gi += 8) {
                const float4 a = *reinterpret_cast<const float4*>(sr + 8 * gi);
                const float4 b = *reinterpret_cast<const float4*>(sr + 8 * gi + 4);
                const float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (8 * gi + e < T) mx = fmaxf(mx, x[e]);
            }
        }
        mx = fmaxf(mx, __shfl_xor(mx, 4));
        mx = fmaxf(mx, __shfl_xor(mx, 2));
        mx = fmaxf(mx, __shfl_xor(mx, 1));
        if (live) {
            for (int gi = q; gi < ng; gi += 8) {
                float4 a = *reinterpret_cast<const float4*>(sr + 8 * gi);
                float4 b = *reinterpret_cast<const float4*>(sr + 8 * gi + 4);
                float x[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    x[e] = 8 * gi + e < T ? __expf(x[e] - mx) : 0.0f;
                    sum += x[e];
                }
                *reinterpret_cast<float4*>(sr + 8 * gi) = make_float4(x[0], x[1], x[2], x[3]);
                *reinterpret_cast<float4*>(sr + 8 * gi + 4) = make_float4(x[4], x[5], x[6], x[7]);
            }
        }
        sum += __shfl_xor(sum, 4);
        sum += __shfl_xor(sum, 2);
        sum += __shfl_xor(sum, 1);
        const float inv = live ? 1.0f / sum : 0.0f;
        for (int gi = q; gi < ngp; gi += 8) {
            float x[8];
            if (live && gi < ng) {
                const float4 a = *reinterpret_cast<const float4*>(sr + 8 * gi);
                const float4 b = *reinterpret_cast<const float4*>(sr + 8 * gi + 4);
                x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w; x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] *= inv;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) x[e] = 0.0f;
            }
            fa_v4u hi, lo;
            fa_split8(x, hi, lo);
            *reinterpret_cast<fa_v4u*>(sr + 8 * gi) = hi;
            *reinterpret_cast<fa_v4u*>(sr + 8 * gi + 4) = lo;
        }
    }

    // scores x V: wave w takes columns 32 w .. 32 w + 31 of the head for all
    // 32 rows (each value group read once per workgroup), 32 keys a step.
    // The value ring is filled before the barrier.
    v4f acc[2][2];
#pragma unroll
    for (int b = 0; b < 2; ++b) acc[b][0] = acc[b][1] = v4f{0.f, 0.f, 0.f, 0.f};
    {
        const int ns = (T + 31) / 32;
        const uint32_t vf0 = (uint32_t)(((z * p.H + h) * 8 + 2 * w) * L.TS);
        fa_v8bf vh[kRingV][2], vl[kRingV][2];
        auto load = [&](fa_v8bf (&bh)[2], fa_v8bf (&bl)[2], int t) {
            const uint32_t ts = (uint32_t)min(t, ns - 1);
#pragma unroll
            for (int c = 0; c < 2; ++c) fa_load(rV, vf0 + (uint32_t)(c * L.TS) + ts, bh[c], bl[c]);
        };
#pragma unroll
        for (int k = 0; k < kRingV; ++k) load(vh[k], vl[k], k);
        __syncthreads();
#pragma unroll
        for (int t0 = 0; t0 < kPvSteps; t0 += kRingV) {
#pragma unroll
            for (int k = 0; k < kRingV; ++k) {
                const int t = t0 + k;
                // the probabilities' split groups, as the softmax left them;
                // past the last step zeros (the values repeat the last step)
                const bool live = t < ns;
                const int tc = min(t, ns - 1);
                fa_v8bf ah[2], al[2];
#pragma unroll
                for (int b = 0; b < 2; ++b) {
                    const float* sr = S + (16 * b + i) * sld + 32 * tc + 8 * g;
                    const fa_v4u zero = {0u, 0u, 0u, 0u};
                    ah[b] = __builtin_bit_cast(fa_v8bf, live ? *reinterpret_cast<const fa_v4u*>(sr) : zero);
                    al[b] = __builtin_bit_cast(fa_v8bf, live ? *reinterpret_cast<const fa_v4u*>(sr + 4) : zero);
                }
#pragma unroll
                for (int b = 0; b < 2; ++b)
#pragma unroll
                    for (int c = 0; c < 2; ++c) acc[b][c] = fa_mfma3(ah[b], al[b], vh[k][c], vl[k][c], acc[b][c]);
                load(vh[k], vl[k], t + kRingV);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    }
    float* out = p.out + (size_t)row0 * p.ldo + h * kDh + 32 * w + i;
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
            const int r = r0 + 16 * b + 4 * g + v;
            if (r < T) {
                out[(size_t)r * p.ldo] = acc[b][0][v];
                out[(size_t)r * p.ldo + 16] = acc[b][1][v];
            }
        }
}

// ---- short sequences (T <= kAttnShortT) -------------------------------------
// A workgroup of 4 waves takes kAttnShortRows = 16 query rows, 4 per wave.
// Every key, position and value row it reads is loaded into LDS at once,
// behind one barrier: keys [0, 64), positions [m_first, m_first + 64 nb)
// (nb 64-row blocks cover the block's shifted positions), values [0, T
// rounded up to 16).  Rows past an operand's end read 0.  After the barrier
// each wave runs its own rows without waiting for the others.  It performs
// the operations of rel_pos_attention, each output through the same chain in
// the same order, so the bits are the same:
// - AC, and BD with the shift and the scale;
// - the softmax;
// - scores x V.
// Only the work division differs: 4 rows a wave instead of 8, and one
// staging round trip instead of one per 64-row tile.

// acc[t % 8] += A(step t) * b[t] for the 16 steps of one A register.
template <int... Ts>
__device__ inline void score_steps1(std::integer_sequence<int, Ts...>, float a, const float (&b)[16],
                                    v4f (&acc)[8])
{
    ((acc[Ts & 7] = mfma_bcast<Ts>(a, b[Ts], acc[Ts & 7])), ...);
}

// 4 rows x 64 columns of NT dot products over k = 0..127: a[kb] holds the 4
// rows in broadcast layout for k in [16 kb, 16 kb + 16), lane j's B row is
// brow (128 floats in LDS).  Chain t % 8 of each output takes k ascending;
// the 8 chains are reduced as hsum8 (score_half and score_sums' order).
__device__ inline void score_rows(const float* brow, const float (&a)[8], float (&out)[4])
{
    v4f acc[8];
#pragma unroll
    for (int l = 0; l < 8; ++l) acc[l] = v4f{0.f, 0.f, 0.f, 0.f};
    float b[2][16];
    auto fetch = [&](float (&dst)[16], int kb) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 v = *reinterpret_cast<const float4*>(brow + kb * 16 + 4 * q);
            dst[4 * q] = v.x; dst[4 * q + 1] = v.y; dst[4 * q + 2] = v.z; dst[4 * q + 3] = v.w;
        }
    };
    fetch(b[0], 0);
#pragma unroll
    for (int kb = 0; kb < 8; ++kb) {
        if (kb + 1 < 8) fetch(b[(kb + 1) & 1], kb + 1);
        __builtin_amdgcn_sched_barrier(0);
        score_steps1(std::make_integer_sequence<int, 16>{}, a[kb], b[kb & 1], acc);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float s8[8];
#pragma unroll
        for (int l = 0; l < 8; ++l) s8[l] = acc[l][i];
        out[i] = hsum8(s8);
    }
}

// scores x V for 4 rows: acc[d] += S[row i][j0 + t] * V[j0 + t][64 d + lane].
template <int... Ts>
__device__ inline void pv_steps1_full(std::integer_sequence<int, Ts...>, float a, const float* vt,
                                      v4f (&acc)[2])
{
    const int lane = threadIdx.x & 63;
    float b0[16], b1[16];
    ((b0[Ts] = vt[Ts * kTileLd + lane], b1[Ts] = vt[Ts * kTileLd + 64 + lane]), ...);
    ((acc[0] = mfma_bcast<Ts>(a, b0[Ts], acc[0]), acc[1] = mfma_bcast<Ts>(a, b1[Ts], acc[1])), ...);
}

template <int... Ts>
__device__ inline void pv_steps1(std::integer_sequence<int, Ts...>, float a, const float* vt, int n,
                                 v4f (&acc)[2])
{
    const int lane = threadIdx.x & 63;
    (((Ts < n) ? (acc[0] = mfma_bcast<Ts>(a, vt[Ts * kTileLd + lane], acc[0]),
                  acc[1] = mfma_bcast<Ts>(a, vt[Ts * kTileLd + 64 + lane], acc[1]), 0)
               : 0), ...);
}

__global__ __launch_bounds__(256) void rel_pos_attention_short(AttnArgs p)
{
    // Score rows [kAttnShortRows][sld], then the staged rows [n_rows][kTileLd].
    extern __shared__ float smem[];
    const int sld = attn_sld(p.T);
    int rb, h, z;
    attn_task(rb, h, z);
    const int T = p.chunk_T ? p.chunk_T[z] : p.T;           // this chunk's rows
    const int r0 = rb * kAttnShortRows;
    if (r0 >= T) return;                                     // the whole workgroup
    const int row0 = p.chunk_rows ? p.chunk_rows[z] : 0;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int D = p.H * kDh;
    const float* qkv = p.qkv + (size_t)row0 * p.ldq;
    const float* K = qkv + D + h * kDh;
    const float* V = qkv + 2 * D + h * kDh;
    const float* P = p.P + (size_t)(p.T - T) * p.ldp + h * kDh;
    const int r_hi = min(r0 + kAttnShortRows, T) - 1;
    const int L = 2 * T - 1;
    const int m_first = T - 1 - r_hi, m_last = 2 * T - 2 - r0;
    const int nb = (m_last - m_first + 64) / 64;             // position blocks: 1 or 2
    const int n_rows = 64 + 64 * nb + ((T + 15) & ~15);      // keys, positions, values
    float* S = smem;
    float* kt = smem + kAttnShortRows * sld;                 // staged row s at kt + s kTileLd
    float* pt = kt + 64 * kTileLd;
    float* vt = pt + 64 * nb * kTileLd;

    // This wave's Q rows in broadcast layout (lane 4t + i: row r0 + 4w + i at
    // k = 16 kb + t), loaded with the staged rows; rows past T read row T-1
    // and are zeroed after.
    const int i = lane & 3, t = lane >> 2;
    const int rq = r0 + 4 * w + i;
    float qv[8], bu[8], bv[8];
    {
        const float* q = qkv + (size_t)min(rq, T - 1) * p.ldq + h * kDh;
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            qv[kb] = q[16 * kb + t];
            bu[kb] = p.pos_bias_u[h * kDh + 16 * kb + t];
            bv[kb] = p.pos_bias_v[h * kDh + 16 * kb + t];
        }
    }
    // Staged row s (32 float4 per row, 8 rows per pass of the 256 threads):
    // key s for s < 64, position m_first + s - 64 below 64 + 64 nb, then
    // value s - 64 - 64 nb.  Region bounds are multiples of 16 rows, so each
    // pass reads one region and its branch is uniform.
    {
        constexpr int kPass = (64 + 128 + kAttnShortT) / 8;
        const TileSrc ks{K, p.ldq, T}, ps{P, p.ldp, L}, vs{V, p.ldq, T};
        const __amdgpu_buffer_rsrc_t rk = ks.at(0), rp = ps.at(m_first), rv = vs.at(0);
        const int sr = threadIdx.x >> 5, c = 4 * (threadIdx.x & 31);
        float4 st[kPass];
#pragma unroll
        for (int q = 0; q < kPass; ++q) {
            const int s0 = 8 * q, s = s0 + sr;
            if (s0 < n_rows) {
                tiles::v4u u;
                if (s0 < 64)
                    u = tiles::ld_v4(rk, (uint32_t)(s * p.ldq + c) * 4u);
                else if (s0 < 64 + 64 * nb)
                    u = tiles::ld_v4(rp, (uint32_t)((s - 64) * p.ldp + c) * 4u);
                else
                    u = tiles::ld_v4(rv, (uint32_t)((s - 64 - 64 * nb) * p.ldq + c) * 4u);
                st[q] = as_float4(u);
            }
        }
#pragma unroll
        for (int q = 0; q < kPass; ++q)
            if (8 * q < n_rows) *reinterpret_cast<float4*>(kt + (8 * q + sr) * kTileLd + c) = st[q];
    }
    float au[8], av[8];
    {
        const bool live = rq < T;
#pragma unroll
        for (int kb = 0; kb < 8; ++kb) {
            au[kb] = live ? __fadd_rn(qv[kb], bu[kb]) : 0.0f;
            av[kb] = live ? __fadd_rn(qv[kb], bv[kb]) : 0.0f;
        }
    }
    __syncthreads();

    // From here on a wave reads and writes only its own 4 score rows (LDS
    // accesses of one wave complete in order): no more barriers.
    float* Sw = S + 4 * w * sld;
    {   // AC: S[row][j] = Q_u[row] . K[j], j = lane
        float o[4];
        score_rows(kt + lane * kTileLd, au, o);
        if (lane < T)
#pragma unroll
            for (int ii = 0; ii < 4; ++ii) Sw[ii * sld + lane] = o[ii];
    }
    // BD at the shifted positions m = T-1-row+j, combined and scaled
    for (int b = 0; b < nb; ++b) {
        const int m0 = m_first + 64 * b;
        float o[4];
        score_rows(pt + (64 * b + lane) * kTileLd, av, o);
        const int jb = m0 + lane - (T - 1) + r0;
        float sc[4];
        bool ok[4];
#pragma unroll
        for (int ii = 0; ii < 4; ++ii) {
            const int rl = 4 * w + ii;
            ok[ii] = r0 + rl < T && (unsigned)(jb + rl) < (unsigned)T;
            sc[ii] = S[ok[ii] ? jb + rl * (sld + 1) : 0];
        }
#pragma unroll
        for (int ii = 0; ii < 4; ++ii)
            if (ok[ii])
                S[jb + (4 * w + ii) * (sld + 1)] = __fmul_rn(__fadd_rn(sc[ii], o[ii]), kScoreScale);
    }
    // softmax: lanes 0..31, 8 per row
    if (lane < 32) softmax_row(Sw + (lane >> 3) * sld, T, r0 + 4 * w + (lane >> 3) < T);

    // out[row][h*128 + d] = sum over j ascending of S[row][j] * V[j][d]
    v4f acc[2] = {v4f{0.f, 0.f, 0.f, 0.f}, v4f{0.f, 0.f, 0.f, 0.f}};
    const float* srow = Sw + i * sld + t;
    int j0 = 0;
    for (; j0 + 16 <= T; j0 += 16)
        pv_steps1_full(std::make_integer_sequence<int, 16>{}, srow[j0], vt + j0 * kTileLd, acc);
    if (T & 15) {
        const float a = j0 + t < T ? srow[j0] : 0.0f;
        pv_steps1(std::make_integer_sequence<int, 16>{}, a, vt + j0 * kTileLd, T & 15, acc);
    }
    float* out = p.out + (size_t)row0 * p.ldo + h * kDh;
#pragma unroll
    for (int ii = 0; ii < 4; ++ii) {
        const int r = r0 + 4 * w + ii;
        if (r < T) {
            out[(size_t)r * p.ldo + lane] = acc[0][ii];
            out[(size_t)r * p.ldo + 64 + lane] = acc[1][ii];
        }
    }
}

// ---- GLU (encoder.c:453-461) -------------------------------------------------
// gated[r][d] = va * (1 / (1 + exp(-vb))), va = in[r][d], vb = in[r][D + d].
__device__ inline float glu_value(float va, float vb)
{
    return __fmul_rn(va, __fdiv_rn(1.0f, __fadd_rn(1.0f, expf_ieee(-vb))));
}

__global__ void glu_rows(const float* __restrict__ in, int ldi, float* out, int ldo, int rows, int D)
{
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)rows * D) return;
    const int r = (int)(idx / D), d = (int)(idx % D);
    out[(size_t)r * ldo + d] = glu_value(in[(size_t)r * ldi + d], in[(size_t)r * ldi + D + d]);
}

// ---- depthwise convolution + Swish (tensor_ops.c:476-548, encoder.c:467-469)
// Time-major x [rows][C]; each chunk (first row from the table, T rows) is
// convolved on its own with zero padding at its edges.  Positions in the
// reference's 8-wide interior take the explicit fma chain over the taps; the
// others take the compiled form of its scalar loops: taps 0..7 multiplied,
// out-of-range ones as +0, reduced as hsum8 and added to the bias, then fma
// for the remaining taps.  dw_output is that arithmetic for one output, with
// the input value at window position j given by win(j) (window position 0 is
// input time t - pad).
template <int KK, typename Win, typename Wt>
__device__ inline float dw_output(const DwArgs& p, int T, int t, int k_rt, float bias, Win win, Wt wt)
{
    const int K = KK > 0 ? KK : k_rt;
    const int pad = (K - 1) / 2;
    const int t_hi = T - pad > pad ? T - pad : pad;
    const int t_vec = pad + (t_hi - pad) / 8 * 8;
    float val = bias;
    if (t >= pad && t < t_vec) {
        if constexpr (KK > 0) {
            float xv[KK];
#pragma unroll
            for (int k = 0; k < KK; ++k) xv[k] = win(k);
#pragma unroll
            for (int k = 0; k < KK; ++k) val = __fmaf_rn(xv[k], wt(k), val);
        } else {
            for (int k = 0; k < K; ++k) val = __fmaf_rn(win(k), wt(k), val);
        }
    } else {
        const int K8 = K & ~7;
        for (int k0 = 0; k0 < K8; k0 += 8) {
            float pr[8];
#pragma unroll
            for (int l = 0; l < 8; ++l) {
                const int src = t - pad + k0 + l;
                pr[l] = (src >= 0 && src < T) ? __fmul_rn(win(k0 + l), wt(k0 + l)) : 0.0f;
            }
            val = __fadd_rn(val, hsum8(pr));
        }
        for (int k = K8; k < K; ++k) {
            const int src = t - pad + k;
            if (src >= 0 && src < T) val = __fmaf_rn(win(k), wt(k), val);
        }
    }
    return p.swish ? swish_f(val) : val;
}

// Any tap count: one thread per output, each input read where it is used
// (GLU'd on the fly when p.glu).
__global__ void depthwise_swish(DwArgs p)
{
    const int T = p.chunk_T ? p.chunk_T[blockIdx.y] : p.T;   // this chunk's rows
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)T * p.C) return;
    const int t = (int)(idx / p.C), c = (int)(idx % p.C);
    const int row0 = p.chunk_rows ? p.chunk_rows[blockIdx.y] : 0;
    const int pad = (p.K - 1) / 2;
    const float* x = p.x + (size_t)row0 * p.ldx + c;
    const float* wc = p.w + (size_t)c * p.K;
    // window position j is input time t - pad + j, read only where in range
    auto win = [&](int j) {
        const float* xr = x + (size_t)(t - pad + j) * p.ldx;
        return p.glu ? glu_value(xr[0], xr[p.C]) : xr[0];
    };
    p.out[(size_t)(row0 + t) * p.ldo + c] =
        dw_output<0>(p, T, t, p.K, p.b ? p.b[c] : 0.0f, win, [&](int k) { return wc[k]; });
}

// KK taps fixed at compile time: a workgroup takes TB output times of 64
// channels of one chunk.  Its input window (TB + KK - 1 times) is staged in
// LDS once, gated when p.glu, so each input is read, and its GLU formed,
// once per workgroup rather than once per tap; window times outside the
// chunk hold 0 and are never taken (the edge path checks the range).  All of
// a thread's window loads are issued before the first is used.
template <int KK, int TB>
__global__ __launch_bounds__(256) void depthwise_tiled(DwArgs p)
{
    constexpr int pad = (KK - 1) / 2, W = TB + KK - 1, WQ = (W + 3) / 4;
    __shared__ float win_s[W][64];
    const int z = blockIdx.z;
    const int T = p.chunk_T ? p.chunk_T[z] : p.T;            // this chunk's rows
    const int t0 = blockIdx.x * TB;
    if (t0 >= T) return;                                     // the whole workgroup
    const int row0 = p.chunk_rows ? p.chunk_rows[z] : 0;
    const int lane = threadIdx.x & 63, slot = threadIdx.x >> 6;
    const int c = blockIdx.y * 64 + lane;
    const int cc = min(c, p.C - 1);                          // loads of columns past C: column C - 1
    const float* x = p.x + (size_t)row0 * p.ldx + cc;
    float va[WQ], vb[WQ];
#pragma unroll
    for (int q = 0; q < WQ; ++q) {
        const int u = min(max(t0 - pad + slot + 4 * q, 0), T - 1);
        va[q] = x[(size_t)u * p.ldx];
        vb[q] = p.glu ? x[(size_t)u * p.ldx + p.C] : 0.0f;
    }
#pragma unroll
    for (int q = 0; q < WQ; ++q) {
        const int j = slot + 4 * q, u = t0 - pad + j;
        if (j < W) win_s[j][lane] = (u >= 0 && u < T) ? (p.glu ? glu_value(va[q], vb[q]) : va[q]) : 0.0f;
    }
    __syncthreads();
    if (c >= p.C) return;
    float wc[KK];
#pragma unroll
    for (int k = 0; k < KK; ++k) wc[k] = p.w[(size_t)c * KK + k];
    const float bias = p.b ? p.b[c] : 0.0f;
#pragma unroll
    for (int q = 0; q < TB / 4; ++q) {
        const int t = t0 + slot + 4 * q;
        if (t >= T) break;                                   // uniform per wave
        const int j0 = t - t0;                               // window position of input time t - pad
        p.out[(size_t)(row0 + t) * p.ldo + c] = dw_output<KK>(
            p, T, t, KK, bias, [&](int j) { return win_s[j0 + j][lane]; }, [&](int k) { return wc[k]; });
    }
}

// ---- pre-encode subsampling (encoder.c:103-174) ------------------------------
// Activations channel-last, [H][W][256].  pk_conv2d (tensor_ops.c:436-475)
// computes every output as val = bias, then val = fma(x, w, val) over its
// in-range taps (ic, kh, kw ascending), which the kernels below repeat; the
// 1x1 convolutions are chain GEMMs started from the bias (the GEMM's chain_bias).

constexpr int kSub = 256;          // PK_SUB_CHANNELS

// conv.0: 1 -> 256 channels, 3x3, stride 2, pad 1, over the image whose row
// t is mel frame t (mel [n_mels][T], encoder.c:110-120), then ReLU.  One
// workgroup per output row oh and run of kC0Run output columns, one thread
// per channel: the run's input window (3 frames x 2 kC0Run + 1 mel bins, 0
// outside the image) is staged in LDS by one load per thread, a channel's
// nine weights and bias are read once, and each position stores 256
// consecutive floats.  pk_conv2d skips the taps outside the image; here they
// take part with x = 0.  fma(0, w, v) is v except that a zero v may change
// sign, and the ReLU maps either zero to +0, so the outputs are the same.
constexpr int kC0Run = 16;
constexpr int kC0Win = 2 * kC0Run + 1;

__global__ __launch_bounds__(kSub) void conv0_relu(const float* __restrict__ mel, int T, int n_mels,
                                                   const float* __restrict__ w,
                                                   const float* __restrict__ b, float* out, int H1,
                                                   int W1)
{
    __shared__ float win[3 * kC0Win];
    const int c = threadIdx.x;
    const int oh = blockIdx.x, ow0 = blockIdx.y * kC0Run;
    const int ih0 = 2 * oh - 1, iw0 = 2 * ow0 - 1;
    if (c < 3 * kC0Win) {
        const int ih = ih0 + c / kC0Win, iw = iw0 + c % kC0Win;
        win[c] = ih >= 0 && ih < T && iw >= 0 && iw < n_mels ? mel[(size_t)iw * T + ih] : 0.0f;
    }
    float wv[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) wv[k] = w[c * 9 + k];
    const float bias = b[c];
    __syncthreads();
    const int nr = min(kC0Run, W1 - ow0);
    float* o = out + ((size_t)oh * W1 + ow0) * kSub + c;
#pragma unroll
    for (int r = 0; r < kC0Run; ++r) {
        if (r < nr) {
            float v = bias;
#pragma unroll
            for (int k = 0; k < 9; ++k) v = __fmaf_rn(win[(k / 3) * kC0Win + 2 * r + k % 3], wv[k], v);
            o[(size_t)r * kSub] = v > 0.0f ? v : 0.0f;
        }
    }
}

// Depthwise 3x3, stride 2, pad 1 (conv.2 and conv.5, groups = 256).
__global__ void dwconv3x3s2(const float* __restrict__ in, int H, int W,
                            const float* __restrict__ w, const float* __restrict__ b, float* out,
                            int Ho, int Wo)
{
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)Ho * Wo * kSub) return;
    const int c = (int)(idx % kSub);
    const int pos = (int)(idx / kSub), ow = pos % Wo, oh = pos / Wo;
    float xv[9], wv[9];
    bool ok[9];
#pragma unroll
    for (int k = 0; k < 9; ++k) {
        const int ih = 2 * oh - 1 + k / 3, iw = 2 * ow - 1 + k % 3;
        ok[k] = ih >= 0 && ih < H && iw >= 0 && iw < W;
        xv[k] = in[((size_t)min(max(ih, 0), H - 1) * W + min(max(iw, 0), W - 1)) * kSub + c];
        wv[k] = w[c * 9 + k];
    }
    float v = b[c];
#pragma unroll
    for (int k = 0; k < 9; ++k)
        if (ok[k]) v = __fmaf_rn(xv[k], wv[k], v);
    out[idx] = v;
}

// rows x n of C set to bias[0..n): the starting value of a chain that the
// reference begins at the bias.

// [H][W][256] -> [H][256*W], element (c, w) of row h at c*W + w
// (encoder.c:152-158).
__global__ void flatten_rows(const float* __restrict__ in, float* out, int H, int W)
{
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    const int F = kSub * W;
    if (idx >= (long long)H * F) return;
    const int h = (int)(idx / F), r = (int)(idx % F), c = r / W, w = r % W;
    out[idx] = in[((size_t)h * W + w) * kSub + c];
}

// x *= s in place (s = sqrtf(d_model) = 32, encoder.c:578-592: exact).
__global__ void scale_inplace(float* x, long long n, float s)
{
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx < n) x[idx] = __fmul_rn(x[idx], s);
}

// ---- transpose (weights at upload: [R][C] -> [C][R]) --------------------------
__global__ void transpose(const float* __restrict__ in, float* out, int R, int C)
{
    __shared__ float tl[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    for (int y = threadIdx.y; y < 32; y += blockDim.y) {
        const int r = r0 + y, c = c0 + threadIdx.x;
        if (r < R && c < C) tl[y][threadIdx.x] = in[(size_t)r * C + c];
    }
    __syncthreads();
    for (int y = threadIdx.y; y < 32; y += blockDim.y) {
        const int c = c0 + y, r = r0 + threadIdx.x;
        if (r < R && c < C) out[(size_t)c * R + r] = tl[threadIdx.x][y];
    }
}

}  // namespace

hipError_t launch_layer_norm(const float* x, int ldx, const float* gamma, const float* beta,
                             float* out, int ldo, int rows, int D, hipStream_t s)
{
    if (rows <= 0) return hipSuccess;
    if (D != 1024) return hipErrorInvalidValue;   // d_model (PK_D_MODEL)
    // 16-byte loads and stores of x, out, gamma and beta
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
         reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta)) % 16 ||
        ldx % 4 || ldo % 4)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL((layer_norm_rows<128>), dim3((rows + 7) / 8), dim3(64), 0, s, x, ldx,
                       gamma, beta, out, ldo, rows);
    return hipGetLastError();
}

hipError_t launch_layer_norm_split(const float* x, int ldx, const float* gamma, const float* beta,
                                   float* out, int ldo, int rows, int D, hipStream_t s)
{
    if (rows <= 0) return hipSuccess;
    if (D != 1024) return hipErrorInvalidValue;   // d_model (PK_D_MODEL)
    // 16-byte loads of x, gamma and beta; 8-byte stores into 32-byte groups
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
         reinterpret_cast<uintptr_t>(gamma) | reinterpret_cast<uintptr_t>(beta)) % 16 ||
        ldx % 4 || ldo % 8)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL((layer_norm_split_rows<128>), dim3((rows + 7) / 8), dim3(256), 0, s, x, ldx,
                       gamma, beta, out, ldo, rows);
    return hipGetLastError();
}

// PK_GPU_ATTN_SHORT=0 sends short sequences to rel_pos_attention too (the
// same bits; for comparing the two).
bool attn_short_enabled()
{
    static const bool on = [] {
        const char* v = getenv("PK_GPU_ATTN_SHORT");
        return !(v && strcmp(v, "0") == 0);
    }();
    return on;
}

hipError_t launch_attention(const AttnArgs& a, int n_chunks, hipStream_t s)
{
    if (a.T <= 0 || n_chunks <= 0) return hipSuccess;
    dim3 grid((a.T + kAttnRows - 1) / kAttnRows, a.H, n_chunks);
    if (a.T > kAttnMaxT) {
        // score rows in the caller's workspace; LDS holds the staging tile only
        if (!a.scores) return hipErrorInvalidValue;
        if ((size_t)grid.x * grid.y * grid.z * kAttnRows * attn_sld(a.T) >= ((size_t)1 << 40))
            return hipErrorInvalidValue;
        hipLaunchKernelGGL(rel_pos_attention<true>, grid, dim3(256), 4u * kTileFloats, s, a);
        return hipGetLastError();
    }
    if (a.T <= kAttnShortT && attn_short_enabled()) {
        static const hipError_t attr_s = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&rel_pos_attention_short),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)attn_short_lds_bytes(kAttnShortT));
        if (attr_s != hipSuccess) return attr_s;
        const dim3 gs((a.T + kAttnShortRows - 1) / kAttnShortRows, a.H, n_chunks);
        hipLaunchKernelGGL(rel_pos_attention_short, gs, dim3(256), attn_short_lds_bytes(a.T), s, a);
        return hipGetLastError();
    }
    // LDS above the default dynamic limit is granted once per process.
    static const hipError_t attr = hipFuncSetAttribute(
        reinterpret_cast<const void*>(&rel_pos_attention<false>), hipFuncAttributeMaxDynamicSharedMemorySize,
        (int)attn_lds_bytes(kAttnMaxT));
    if (attr != hipSuccess) return attr;
    hipLaunchKernelGGL(rel_pos_attention<false>, grid, dim3(256), attn_lds_bytes(a.T), s, a);
    return hipGetLastError();
}

size_t attn_fast_ws_floats(int T, int H, int n_chunks)
{
    return FaLayout(T, H, n_chunks).floats(H, n_chunks);
}

hipError_t launch_attention_fast(const AttnArgs& a, int n_chunks, float* ws, size_t ws_floats, hipStream_t s)
{
    if (a.T <= 0 || n_chunks <= 0) return hipSuccess;
    if (a.T > kAttnMaxT || !ws || attn_fast_ws_floats(a.T, a.H, n_chunks) > ws_floats ||
        ws_floats * 4 >= ((size_t)1 << 31) || a.ldq % 4 || a.ldp % 4)
        return hipErrorInvalidValue;
    const FaLayout L(a.T, a.H, n_chunks);
    const long long items = 64LL * ((long long)n_chunks * a.H * L.KB * 4 + (long long)a.H * L.PB * 4 +
                                    (long long)n_chunks * a.H * 8 * L.TS);
    hipLaunchKernelGGL(attn_fast_prep, dim3((unsigned)((items + 255) / 256)), dim3(256), 0, s, a, n_chunks, ws);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const dim3 grid((a.T + kAttnRows - 1) / kAttnRows, a.H, n_chunks);
    const unsigned lds = 4u * kAttnRows * fa_sld(a.T);
    const float* cws = ws;
    auto run = [&](auto kern) {
        // LDS above the default dynamic limit is granted once per instantiation
        static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                           hipFuncAttributeMaxDynamicSharedMemorySize,
                                                           (int)(4u * kAttnRows * fa_sld(kAttnMaxT)));
        if (attr != hipSuccess) return attr;
        hipLaunchKernelGGL(kern, grid, dim3(256), lds, s, a, cws);
        return hipGetLastError();
    };
    switch ((a.T + 63) / 64) {
    case 1:
    case 2: return run(rel_pos_attention_fast<128>);
    case 3: return run(rel_pos_attention_fast<192>);
    case 4: return run(rel_pos_attention_fast<256>);
    case 5: return run(rel_pos_attention_fast<320>);
    case 6: return run(rel_pos_attention_fast<384>);
    case 7: return run(rel_pos_attention_fast<448>);
    default: return run(rel_pos_attention_fast<512>);
    }
}

hipError_t launch_glu(const float* in, int ldi, float* out, int ldo, int rows, int D, hipStream_t s)
{
    const long long n = (long long)rows * D;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(glu_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, in, ldi, out,
                       ldo, rows, D);
    return hipGetLastError();
}

hipError_t launch_depthwise(const DwArgs& a, int n_chunks, hipStream_t s)
{
    const long long n = (long long)a.T * a.C;
    if (n <= 0 || n_chunks <= 0) return hipSuccess;
    if (a.K == 9) {
        // short sequences: 16-time tiles (more workgroups); else 32 (less overlap)
        const unsigned cb = (unsigned)((a.C + 63) / 64);
        if (a.T <= 128)
            hipLaunchKernelGGL((depthwise_tiled<9, 16>), dim3((unsigned)((a.T + 15) / 16), cb, n_chunks), dim3(256),
                               0, s, a);
        else
            hipLaunchKernelGGL((depthwise_tiled<9, 32>), dim3((unsigned)((a.T + 31) / 32), cb, n_chunks), dim3(256),
                               0, s, a);
    } else {
        hipLaunchKernelGGL(depthwise_swish, dim3((unsigned)((n + 255) / 256), n_chunks), dim3(256), 0, s, a);
    }
    return hipGetLastError();
}

hipError_t launch_transpose(const float* in, float* out, int R, int C, hipStream_t s)
{
    if (R <= 0 || C <= 0) return hipSuccess;
    hipLaunchKernelGGL(transpose, dim3((C + 31) / 32, (R + 31) / 32), dim3(32, 8), 0, s, in, out, R, C);
    return hipGetLastError();
}

static unsigned blocks_of(long long n) { return (unsigned)((n + 255) / 256); }

hipError_t launch_conv0_relu(const float* mel, int T, int n_mels, const float* w, const float* b,
                             float* out, int H1, int W1, hipStream_t s)
{
    if (H1 <= 0 || W1 <= 0) return hipSuccess;
    hipLaunchKernelGGL(conv0_relu, dim3(H1, (W1 + kC0Run - 1) / kC0Run), dim3(kSub), 0, s, mel, T,
                       n_mels, w, b, out, H1, W1);
    return hipGetLastError();
}

hipError_t launch_dwconv3x3s2(const float* in, int H, int W, const float* w, const float* b,
                              float* out, int Ho, int Wo, hipStream_t s)
{
    const long long n = (long long)Ho * Wo * kSub;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(dwconv3x3s2, dim3(blocks_of(n)), dim3(256), 0, s, in, H, W, w, b, out, Ho, Wo);
    return hipGetLastError();
}

hipError_t launch_flatten_rows(const float* in, float* out, int H, int W, hipStream_t s)
{
    const long long n = (long long)H * W * kSub;
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(flatten_rows, dim3(blocks_of(n)), dim3(256), 0, s, in, out, H, W);
    return hipGetLastError();
}

hipError_t launch_scale(float* x, long long n, float sc, hipStream_t s)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(scale_inplace, dim3(blocks_of(n)), dim3(256), 0, s, x, n, sc);
    return hipGetLastError();
}

}  // namespace pkgpu
