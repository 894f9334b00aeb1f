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
//   int4: w = fl(q * s[k][n/32]) exactly as blas.c:834-840 dequantises it,
//         split into w_hi + w_lo; C = alpha * (A_hi W_hi + A_lo W_hi +
//         A_hi W_lo) (3 MFMAs; the dropped A_lo W_lo term is below 2^-16).
// The activations are never quantised: they stay fp32-valued to 16 bits.
//
// Work split.  A workgroup of 4 waves owns 128 columns; its waves take
// consecutive 32-deep k steps of one k segment (KS steps each).  A wave's
// lane (i, g) = (lane % 16, lane / 16) loads, per k step, rows k0 + 8g ..
// k0 + 8g + 7 of columns c0 + 8i .. c0 + 8i + 7: 16 lanes read one 128-byte
// run of each row (int8; 64 bytes for int4, with the row's scales), and the
// weights reach the MFMA operand layout (8 k values of one column per lane)
// in registers, with no LDS pass.  MFMA slice j (0..7) multiplies column
// c0 + 8i + j into output slot i.
// The 4 waves' partial tiles are summed in LDS in a fixed order,
// (w0 + w2) + (w1 + w3).  With S > 1 segments per column tile each
// workgroup writes its partial to scratch at device scope; the last to
// arrive (an atomic counter per tile) sums the S partials in segment order,
// applies the epilogue and resets the counter.  Every sum has a fixed order, so results
// are deterministic.  The S segments of a tile go to workgroups on one XCD.
#include "pk_gemm_kernels.h"
#include "pk_device_math.h"

#include <algorithm>
#include <cstdlib>

namespace pkgpu {
namespace {

typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
typedef __bf16 v4bf __attribute__((ext_vector_type(4)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef uint32_t v2u __attribute__((ext_vector_type(2)));
typedef uint32_t v4u __attribute__((ext_vector_type(4)));

constexpr int kCols = 128;     // columns per workgroup
constexpr int kWaves = 4;
constexpr int kXcd = 8;
constexpr int kSc1 = 16;       // buffer-op cache policy: device-scope coherence (sc1)

struct SmArgs {
    int M, N, K;
    float alpha;               // int8: alpha * scale
    float beta;
    const float* A; int lda;
    const void* B; int ldb;    // row pitch in elements (int4: bytes)
    const float* scales; int n_groups;
    float* C; int ldc;
    const float* bias; int epi;
    uint32_t a_bytes, b_bytes, s_bytes;
    int NT, S;                 // column tiles, k segments per tile
    float* part;               // [NT][S][16*RB][128] partial tiles (S > 1)
    uint32_t part_bytes;
    unsigned* cnt;             // [NT] arrival counters, zero between launches
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

// Raw weight bits of one lane's 8 columns in one row.
template <int WK> struct RowBits;
template <> struct RowBits<W_I8> { typedef v2u T; };     // 8 int8
template <> struct RowBits<W_I4> { typedef uint32_t T; }; // 8 nibbles

template <int WK>
__device__ inline typename RowBits<WK>::T load_row(__amdgpu_buffer_rsrc_t r, const SmArgs& p, int k, int c)
{
    if constexpr (WK == W_I8)
        return __builtin_amdgcn_raw_buffer_load_b64(r, (int)((uint32_t)k * (uint32_t)p.ldb + (uint32_t)c), 0, 0);
    else
        return __builtin_amdgcn_raw_buffer_load_b32(r, (int)((uint32_t)k * (uint32_t)p.ldb + (uint32_t)(c >> 1)), 0, 0);
}

// Weight value of column j (0..7) of a lane's row bits.
__device__ inline float w_i8(v2u b, int j)
{
    const uint32_t w = j < 4 ? b[0] : b[1];
    return (float)(signed char)(w >> (8 * (j & 3)));
}
__device__ inline int q_i4(uint32_t b, int j)
{
    return (int)(b << (28 - 4 * j)) >> 28;          // low nibble = even column
}

// SMAX: at least the k segments S (1: one segment, no partials).
template <int WK, int RB, int KS, int SMAX>
__global__ __launch_bounds__(256) void smallm_gemm(SmArgs p)
{
    constexpr int MP = 16 * RB;                     // padded rows
    __shared__ float lds[2][MP][kCols];
    __shared__ int last;

    // workgroup -> (column tile t, k segment s); the S segments of a tile on one XCD
    const int x = blockIdx.x, xcd = x % kXcd, r = x / kXcd;
    const int s = r % p.S, t = (r / p.S) * kXcd + xcd;
    if (t >= p.NT) return;                          // padding workgroups (uniform)
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane & 15, g = lane >> 4;
    const int c0 = t * kCols;
    const int kw = s * (kWaves * KS * 32) + wave * (KS * 32);   // this wave's first k

    const auto rA = rsrc(p.A, p.a_bytes), rB = rsrc(p.B, p.b_bytes);
    const auto rS = rsrc(p.scales, p.s_bytes);

    v4f acc[RB][8];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[rb][j] = v4f{0.f, 0.f, 0.f, 0.f};

    // every weight load of the wave first: the HBM stream is the latency to hide
    typename RowBits<WK>::T wb[KS][8];
    float sc[KS][8];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
            const int k = kw + 32 * ks + 8 * g + rr;        // rows >= K read 0 (past the extent)
            wb[ks][rr] = load_row<WK>(rB, p, k, c0 + 8 * i);
            if constexpr (WK == W_I4)
                sc[ks][rr] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    rS, (int)(((uint32_t)k * (uint32_t)p.n_groups + (uint32_t)((c0 + 8 * i) >> 5)) * 4u), 0, 0));
        }

#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
        const int k0 = kw + 32 * ks;
        if (k0 >= p.K) break;                       // K % 32 == 0: whole steps only (uniform)
        v8bf ahi[RB], alo[RB];
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            // row 16rb + i, k0 + 8g .. +7: rows >= M read 0 (past the extent)
            const uint32_t off = ((uint32_t)(16 * rb + i) * (uint32_t)p.lda + (uint32_t)(k0 + 8 * g)) * 4u;
            const v4u a0 = __builtin_amdgcn_raw_buffer_load_b128(rA, (int)off, 0, 0);
            const v4u a1 = __builtin_amdgcn_raw_buffer_load_b128(rA, (int)(off + 16), 0, 0);
            const float xa[8] = {__uint_as_float(a0[0]), __uint_as_float(a0[1]), __uint_as_float(a0[2]),
                                 __uint_as_float(a0[3]), __uint_as_float(a1[0]), __uint_as_float(a1[1]),
                                 __uint_as_float(a1[2]), __uint_as_float(a1[3])};
            split8(xa, ahi[rb], alo[rb]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if constexpr (WK == W_I8) {
                const v8bf b = cat(to_bf2(w_i8(wb[ks][0], j), w_i8(wb[ks][1], j)),
                                   to_bf2(w_i8(wb[ks][2], j), w_i8(wb[ks][3], j)),
                                   to_bf2(w_i8(wb[ks][4], j), w_i8(wb[ks][5], j)),
                                   to_bf2(w_i8(wb[ks][6], j), w_i8(wb[ks][7], j)));
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    acc[rb][j] = mfma(ahi[rb], b, acc[rb][j]);
                    acc[rb][j] = mfma(alo[rb], b, acc[rb][j]);
                }
            } else {
                float w[8];
#pragma unroll
                for (int rr = 0; rr < 8; ++rr) w[rr] = __fmul_rn((float)q_i4(wb[ks][rr], j), sc[ks][rr]);
                v8bf bhi, blo;
                split8(w, bhi, blo);
#pragma unroll
                for (int rb = 0; rb < RB; ++rb) {
                    acc[rb][j] = mfma(ahi[rb], bhi, acc[rb][j]);
                    acc[rb][j] = mfma(alo[rb], bhi, acc[rb][j]);
                    acc[rb][j] = mfma(ahi[rb], blo, acc[rb][j]);
                }
            }
        }
    }

    // fixed-order sum of the 4 waves' tiles: (w0 + w2) + (w1 + w3), in LDS.
    // Lane (i, g) holds rows 16rb + 4g + v, columns 8i + j.
    auto put = [&](int slot) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                float* row = &lds[slot][16 * rb + 4 * g + v][8 * i];
                *reinterpret_cast<v4f*>(row) = v4f{acc[rb][0][v], acc[rb][1][v], acc[rb][2][v], acc[rb][3][v]};
                *reinterpret_cast<v4f*>(row + 4) = v4f{acc[rb][4][v], acc[rb][5][v], acc[rb][6][v], acc[rb][7][v]};
            }
    };
    auto add = [&](int slot) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const float* row = &lds[slot][16 * rb + 4 * g + v][8 * i];
                const v4f a = *reinterpret_cast<const v4f*>(row), b = *reinterpret_cast<const v4f*>(row + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    acc[rb][j][v] = __fadd_rn(acc[rb][j][v], a[j]);
                    acc[rb][4 + j][v] = __fadd_rn(acc[rb][4 + j][v], b[j]);
                }
            }
    };
    if (wave >= 2) put(wave - 2);
    __syncthreads();
    if (wave < 2) add(wave);
    __syncthreads();
    if (wave == 1) put(0);
    __syncthreads();
    if (wave == 0) {
        add(0);
        put(1);                                     // the workgroup's partial tile
    }
    __syncthreads();

    // all 256 threads: 16*RB rows x 128 columns as float4s, U per thread
    constexpr int kVec = MP * kCols / 4, U = kVec / 256;
    const v4f* tile = reinterpret_cast<const v4f*>(&lds[1][0][0]);
    auto finish = [&](int e, v4f sum) {
        const int m = (4 * e) / kCols, col = c0 + (4 * e) % kCols;
        if (m >= p.M) return;
        float* crow = p.C + (size_t)m * p.ldc;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int n = col + u;
            if (n >= p.N) break;
            float v = __fmul_rn(p.alpha, sum[u]);
            if (p.beta != 0.0f) v = __fadd_rn(p.beta == 1.0f ? crow[n] : __fmul_rn(p.beta, crow[n]), v);
            if (p.bias) v = __fadd_rn(v, p.bias[n]);
            switch (p.epi) {
            case EPI_SWISH:         v = swish_f(v); break;
            case EPI_HALF_RESIDUAL: v = __fmaf_rn(v, 0.5f, crow[n]); break;
            case EPI_RESIDUAL:      v = __fadd_rn(crow[n], v); break;
            case EPI_RELU:          v = v > 0.0f ? v : 0.0f; break;
            default:                break;
            }
            crow[n] = v;
        }
    };
    if constexpr (SMAX == 1) {
#pragma unroll
        for (int u = 0; u < U; ++u) finish(threadIdx.x + 256 * u, tile[threadIdx.x + 256 * u]);
    } else {
        // The partials pass between workgroups that may sit on different XCDs,
        // whose L2s are not coherent with each other: they are stored and
        // loaded at device scope (sc1: written through to, and read from, the
        // device's coherence point), so no L2-wide write-back or invalidate
        // (what a device-scope fence costs) is needed.  The stores complete
        // (vmcnt 0) before the workgroup's arrival is counted.
        const auto rP = rsrc(p.part, p.part_bytes);
        const uint32_t mine = (uint32_t)(((size_t)t * p.S + s) * (MP * kCols) * 4);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const v4f v = tile[threadIdx.x + 256 * u];
            __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, v), rP,
                                                   (int)(mine + 16u * (threadIdx.x + 256 * u)), 0, kSc1);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (threadIdx.x == 0)
            last = __hip_atomic_fetch_add(&p.cnt[t], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM) ==
                   (unsigned)(p.S - 1);
        __syncthreads();
        if (!last) return;
        // every partial load of a batch in flight at once, then the sums in
        // segment order; batches of UB float4s per thread keep <= 32 in flight
        const uint32_t seg0 = (uint32_t)((size_t)t * p.S * (MP * kCols) * 4);
        constexpr int UB = (32 / SMAX) < 1 ? 1 : ((32 / SMAX) > U ? U : (32 / SMAX));
#pragma unroll
        for (int u0 = 0; u0 < U; u0 += UB) {
            v4f q[UB][SMAX];
#pragma unroll
            for (int ub = 0; ub < UB; ++ub)
#pragma unroll
                for (int s2 = 0; s2 < SMAX; ++s2)
                    if (s2 < p.S)
                        q[ub][s2] = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(
                            rP, (int)(seg0 + 16u * ((uint32_t)s2 * kVec + threadIdx.x + 256 * (u0 + ub))),
                            0, kSc1));
#pragma unroll
            for (int ub = 0; ub < UB; ++ub) {
                v4f sum = q[ub][0];
#pragma unroll
                for (int s2 = 1; s2 < SMAX; ++s2)
                    if (s2 < p.S)
                        sum = v4f{__fadd_rn(sum[0], q[ub][s2][0]), __fadd_rn(sum[1], q[ub][s2][1]),
                                  __fadd_rn(sum[2], q[ub][s2][2]), __fadd_rn(sum[3], q[ub][s2][3])};
                finish(threadIdx.x + 256 * (u0 + ub), sum);
            }
        }
        if (threadIdx.x == 0)                       // every segment has arrived
            __hip_atomic_store(&p.cnt[t], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

// ---- narrow tiles: 16 columns and all of K per workgroup, no partials ----
// A workgroup of NW waves owns 16 columns (one MFMA's width) and the whole k
// range: wave w takes k steps [w*ns/NW, (w+1)*ns/NW) of the ns = K/32 steps,
// at most kMaxSteps, every load of them issued before the first MFMA.
// Lane (i, g) reads column c0 + i of rows k0 + 8g .. k0 + 8g + 7 (bytes for
// int8 / int4, words for fp32): the 16 lanes of a row read one 16-byte run,
// and consecutive tiles run on one XCD, so each 128-byte line of a row comes
// through that XCD's L2 once.  The 16 columns of an int4 tile lie in one
// 32-column scale group, so the scale folds into the activations
// (A' = fl(A * s[k][g]), then split) and the codes enter the MFMA exactly.
// The NW partial tiles are summed in LDS in wave order, then the epilogue.
template <int WK, int RB, int NW, int kMaxSteps>
__global__ __launch_bounds__(64 * NW) void smallm_narrow(SmArgs p)
{
    __shared__ v4f red[NW][RB][64];
    // consecutive tiles on one XCD (workgroups reach the XCDs round-robin)
    const int x = blockIdx.x, per = gridDim.x / kXcd;
    const int t = (x % kXcd) * per + x / kXcd;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int i = lane & 15, g = lane >> 4;
    const int c = t * 16 + i;                        // this lane's column (>= N reads 0 or junk, never stored)
    const int ns = p.K / 32, s0 = wave * ns / NW, s1 = (wave + 1) * ns / NW;

    const auto rA = rsrc(p.A, p.a_bytes), rB = rsrc(p.B, p.b_bytes);
    const auto rS = rsrc(p.scales, p.s_bytes);

    float wv[kMaxSteps][8], sv[kMaxSteps][8];
    v4u ar[kMaxSteps][RB][2];
#pragma unroll
    for (int st = 0; st < kMaxSteps; ++st) {
        if (s0 + st >= s1) break;                    // uniform per wave
        const int k0 = 32 * (s0 + st);
#pragma unroll
        for (int rr = 0; rr < 8; ++rr) {
            const uint32_t k = (uint32_t)(k0 + 8 * g + rr);
            if constexpr (WK == W_I8) {
                wv[st][rr] = (float)(signed char)__builtin_amdgcn_raw_buffer_load_b8(
                    rB, (int)(k * (uint32_t)p.ldb + (uint32_t)c), 0, 0);
            } else if constexpr (WK == W_I4) {
                const uint32_t b = __builtin_amdgcn_raw_buffer_load_b8(
                    rB, (int)(k * (uint32_t)p.ldb + (uint32_t)(c >> 1)), 0, 0);
                wv[st][rr] = (float)q_i4(b, c & 1);
                sv[st][rr] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    rS, (int)((k * (uint32_t)p.n_groups + (uint32_t)(c >> 5)) * 4u), 0, 0));
            } else {
                wv[st][rr] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(
                    rB, (int)((k * (uint32_t)p.ldb + (uint32_t)c) * 4u), 0, 0));
            }
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            const uint32_t off = ((uint32_t)(16 * rb + i) * (uint32_t)p.lda + (uint32_t)(k0 + 8 * g)) * 4u;
            ar[st][rb][0] = __builtin_amdgcn_raw_buffer_load_b128(rA, (int)off, 0, 0);
            ar[st][rb][1] = __builtin_amdgcn_raw_buffer_load_b128(rA, (int)(off + 16), 0, 0);
        }
    }

    v4f acc[RB];
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) acc[rb] = v4f{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int st = 0; st < kMaxSteps; ++st) {
        if (s0 + st >= s1) break;
        v8bf bhi, blo;
        if constexpr (WK == W_F32) {
            split8(wv[st], bhi, blo);
        } else {
            bhi = cat(to_bf2(wv[st][0], wv[st][1]), to_bf2(wv[st][2], wv[st][3]),
                      to_bf2(wv[st][4], wv[st][5]), to_bf2(wv[st][6], wv[st][7]));   // exact
        }
#pragma unroll
        for (int rb = 0; rb < RB; ++rb) {
            float xa[8] = {__uint_as_float(ar[st][rb][0][0]), __uint_as_float(ar[st][rb][0][1]),
                           __uint_as_float(ar[st][rb][0][2]), __uint_as_float(ar[st][rb][0][3]),
                           __uint_as_float(ar[st][rb][1][0]), __uint_as_float(ar[st][rb][1][1]),
                           __uint_as_float(ar[st][rb][1][2]), __uint_as_float(ar[st][rb][1][3])};
            if constexpr (WK == W_I4) {
#pragma unroll
                for (int e = 0; e < 8; ++e) xa[e] = __fmul_rn(xa[e], sv[st][e]);
            }
            v8bf ahi, alo;
            split8(xa, ahi, alo);
            acc[rb] = mfma(ahi, bhi, acc[rb]);
            acc[rb] = mfma(alo, bhi, acc[rb]);
            if constexpr (WK == W_F32) acc[rb] = mfma(ahi, blo, acc[rb]);
        }
    }

    // fixed-order sum over the waves, one output per thread
#pragma unroll
    for (int rb = 0; rb < RB; ++rb) red[wave][rb][lane] = acc[rb];
    __syncthreads();
    const int o = threadIdx.x;                       // output (rb, lane l, v)
    if (o >= RB * 256) return;
    const int rb = o >> 8, l = (o >> 2) & 63, v = o & 3;
    float sum = red[0][rb][l][v];
#pragma unroll
    for (int w = 1; w < NW; ++w) sum = __fadd_rn(sum, red[w][rb][l][v]);
    const int m = 16 * rb + 4 * (l >> 4) + v, n = t * 16 + (l & 15);
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

// 16 waves of at most 2 k steps (K <= 1024); 4 steps would spill registers
// at 48 and 64 rows (a wave of a 1024-thread workgroup holds 128).
template <int WK, int RB>
hipError_t launch_narrow_rb(const SmArgs& a, hipStream_t st)
{
    const int tiles = (a.N + 15) / 16;
    const dim3 grid((unsigned)(((tiles + kXcd - 1) / kXcd) * kXcd));
    hipLaunchKernelGGL((smallm_narrow<WK, RB, 16, 2>), grid, dim3(1024), 0, st, a);
    return hipGetLastError();
}

template <int WK>
hipError_t launch_narrow(int RB, const SmArgs& a, hipStream_t st)
{
    switch (RB) {
    case 1: return launch_narrow_rb<WK, 1>(a, st);
    case 2: return launch_narrow_rb<WK, 2>(a, st);
    case 3: return launch_narrow_rb<WK, 3>(a, st);
    default: return launch_narrow_rb<WK, 4>(a, st);
    }
}

template <int WK, int RB, int KS>
hipError_t launch_ks(const SmArgs& a, hipStream_t st)
{
    const dim3 grid((unsigned)(((a.NT + kXcd - 1) / kXcd) * kXcd * a.S)), block(256);
    if (a.S == 1)
        hipLaunchKernelGGL((smallm_gemm<WK, RB, KS, 1>), grid, block, 0, st, a);
    else if (a.S <= 8)
        hipLaunchKernelGGL((smallm_gemm<WK, RB, KS, 8>), grid, block, 0, st, a);
    else
        hipLaunchKernelGGL((smallm_gemm<WK, RB, KS, 16>), grid, block, 0, st, a);
    return hipGetLastError();
}

template <int WK, int RB>
hipError_t launch_rb(int KS, const SmArgs& a, hipStream_t st)
{
    switch (KS) {
    case 1: return launch_ks<WK, RB, 1>(a, st);
    case 2: return launch_ks<WK, RB, 2>(a, st);
    default: return launch_ks<WK, RB, 4>(a, st);
    }
}

template <int WK>
hipError_t launch_kind(int RB, int KS, const SmArgs& a, hipStream_t st)
{
    switch (RB) {
    case 1: return launch_rb<WK, 1>(KS, a, st);
    case 2: return launch_rb<WK, 2>(KS, a, st);
    case 3: return launch_rb<WK, 3>(KS, a, st);
    default: return launch_rb<WK, 4>(KS, a, st);
    }
}

}  // namespace

// K up to 1024 takes the narrow tiles (no partials); longer K the wide ones.
constexpr int kNarrowMaxK = 1024;

bool smallm_supports(const GemmProblem& p)
{
    if (p.M < 1 || p.M > kSmallMaxM || p.N < 1 || p.K < 32 || p.K % 32) return false;
    if (p.chain_bias || (p.kind == W_F32 && p.K > kNarrowMaxK)) return false;
    if (p.alpha == 0.0f || (p.kind == W_I8 && p.scale == 0.0f)) return false;   // beta-only step
    const uintptr_t pa = reinterpret_cast<uintptr_t>(p.A), pb = reinterpret_cast<uintptr_t>(p.B);
    if (p.lda % 4 || pa % 16) return false;
    if (p.kind == W_F32) return pb % 4 == 0;
    if (p.kind == W_I8) return p.N % 8 == 0 && p.ldb % 8 == 0 && pb % 8 == 0;
    return p.N % 32 == 0 && p.ldb % 4 == 0 && pb % 4 == 0 &&
           reinterpret_cast<uintptr_t>(p.scales) % 4 == 0;
}

int smallm_plan(const GemmProblem& p, int* ks_out, int* s_out)
{
    const int RB = (p.M + 15) / 16, NT = (p.N + kCols - 1) / kCols;
    // KS = 1 (one 32-deep step per wave) spreads the weight stream over the
    // most workgroups; deeper steps cut the number of k segments (partials)
    // for long K.  PK_GPU_SMALLM_KS overrides the choice (tuning sweeps).
    static const int forced = [] {
        const char* e = getenv("PK_GPU_SMALLM_KS");
        return e ? atoi(e) : 0;
    }();
    int KS = forced == 1 || forced == 2 || forced == 4 ? forced : 1;
    if (!forced)
        while (KS < 4 && (p.K + kWaves * 32 * KS - 1) / (kWaves * 32 * KS) > 8) KS *= 2;
    (void)RB;
    if (ks_out) *ks_out = KS;
    if (s_out) *s_out = (p.K + kWaves * 32 * KS - 1) / (kWaves * 32 * KS);
    return NT;
}

size_t smallm_scratch_bytes(const GemmProblem& p)
{
    if (p.K <= kNarrowMaxK) return 0;
    int KS = 1, S = 1;
    const int NT = smallm_plan(p, &KS, &S);
    if (S == 1) return 0;
    return (size_t)NT * S * (16 * ((p.M + 15) / 16)) * kCols * sizeof(float);
}

int smallm_counters(const GemmProblem& p) { return p.K <= kNarrowMaxK ? 0 : smallm_plan(p, nullptr, nullptr); }

hipError_t launch_smallm(const GemmProblem& p, hipStream_t st, const SmallmScratch& sc)
{
    if (!smallm_supports(p)) return hipErrorNotSupported;
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
    if (a_ext >= lim || b_ext >= lim || s_ext >= lim) return hipErrorNotSupported;
    a.a_bytes = (uint32_t)a_ext;
    a.b_bytes = (uint32_t)b_ext;
    a.s_bytes = (uint32_t)s_ext;
    const int RB = (p.M + 15) / 16;
    if (p.K <= kNarrowMaxK) {
        switch (p.kind) {
        case W_I8: return launch_narrow<W_I8>(RB, a, st);
        case W_I4: return launch_narrow<W_I4>(RB, a, st);
        default:   return launch_narrow<W_F32>(RB, a, st);
        }
    }
    int KS = 1, S = 1;
    a.NT = smallm_plan(p, &KS, &S);
    if (S > 16) return hipErrorNotSupported;        // K > 8192: the exact kernels
    a.S = S;
    if (S > 1) {
        if (!sc.part || !sc.cnt || smallm_scratch_bytes(p) > sc.part_bytes || a.NT > sc.cnt_n)
            return hipErrorNotSupported;
        a.part = sc.part;
        a.part_bytes = (uint32_t)smallm_scratch_bytes(p);
        a.cnt = sc.cnt;
    }
    return p.kind == W_I8 ? launch_kind<W_I8>(RB, KS, a, st) : launch_kind<W_I4>(RB, KS, a, st);
}

}  // namespace pkgpu
