// pk_gemm_kernels.hip - dispatch of the weight GEMMs and the small kernels
// around them (beta-only pass, int8 edge columns, swish).  The tile kernels
// and their numerics are described in pk_gemm_tiles.h.
#include "pk_gemm_tiles.h"

namespace pkgpu {
namespace {

using tiles::KArgs;

// int8 columns j >= 16*floor(N/16): the compiled reference evaluates
// blas.c:752 (c += ax*bs*(float)b) as c = fma(fl(A*fl(alpha*bs)), (float)q, c)
// after hoisting alpha*bs; one thread per output, k ascending.
__global__ void i8_edge(KArgs p, int n_begin, int n_edge)
{
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)p.M * n_edge) return;
    const int i = (int)(idx / n_edge);
    const int j = n_begin + (int)(idx % n_edge);
    const int8_t* Q = static_cast<const int8_t*>(p.B);
    float c = 0.0f;
    if (p.beta != 0.0f) {
        const float cv = p.C[(size_t)i * p.ldc + j];
        c = (p.beta == 1.0f) ? cv : __fmul_rn(cv, p.beta);
    }
    const float as = __fmul_rn(p.alpha, p.scale);
    for (int k = 0; k < p.K; ++k) {
        const float a = __fmul_rn(p.A[(size_t)i * p.lda + k], as);
        c = __fmaf_rn(a, (float)Q[(size_t)k * p.ldb + j], c);
    }
    tiles::store_c(p, c, i, j);
}

// C <- beta*C alone (alpha == 0, int8 scale == 0, or K == 0): blas.c:89-99,
// followed by the fused epilogue when one is requested.
__global__ void scale_c(KArgs p)
{
    const long long idx = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (long long)p.M * p.N) return;
    const int i = (int)(idx / p.N), j = (int)(idx % p.N);
    float* c = p.C + (size_t)i * p.ldc + j;
    const float v = (p.beta == 0.0f) ? 0.0f : (p.beta == 1.0f ? *c : __fmul_rn(*c, p.beta));
    tiles::store_c(p, v, i, j);
}

// pk_swish over n elements (tensor_ops.c:381-388); x may equal y.
__global__ void swish(const float* x, float* y, long long n)
{
    const long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    y[i] = swish_f(x[i]);
}

}  // namespace

using tiles::kConfigs;
using tiles::kNumConfigs;

int num_configs() { return kNumConfigs; }
TileConfig config_at(int i) { return kConfigs[i]; }

// Every output is a chain of K dependent MFMA steps, so the work that can run
// at once is the number of independent chains (M*N / outputs per MFMA).
// Chosen from a sweep of every configuration over the encoder's GEMM shapes
// on MI355X (hot weights; times in us for the best and the chosen config):
//   M*N < 200K          config 12 (S 4x4, 1 chain)    QKV M=32: 11.6
//   M*N < 1M, K >= 2048 config 17 (S 4x4, 8+8 waves)  FF down M=375: 51.6
//   M*N < 1M            config 13 (S 4x4, 2 chains)   out/pos/conv: 15-26
//   M*N < 1.6M          config 14 (S 4x4, 3 chains)   FF up M=375: 35.1
//   M*N < 3M            config 18 (S 16x16)           FF up M=416/500: 41
//   otherwise, M=1656:  int4 up     config 20 (Y 32x32, full chunks, 3 waves per
//                                   SIMD): beside the other row group's kernels 1.2%
//                                   less encoder time than config 19 (S 32x32), which
//                                   had won while config 20 held 2 waves per SIMD
//   otherwise, M=3312:  int4 up     config 20 (Y 32x32)  242-252 (config 11: 249-257)
//                       int4 down   config 11 (X 32x32)  264-271
//                       int8        config 21 (Y 32x32, k 16)  QKV 180, out 70.0
//                                   (config 11: 183-185, 72.5-72.9)
//                       fp32 2048   config 23 (Y 16x16)  132.6 (config 10: 141-144); also
//                                   at M=1656 (0.4% less encoder time than config 21)
//                       fp32 1024   config 21            68.8 (config 10: 71.6-71.7)
static int choose_index(int M, int N, int K, WeightKind kind = W_I8)
{
    const double outputs = (double)M * (double)N;
    if (outputs < 200e3) return 12;
    if (outputs < 1.0e6) return K >= 2048 ? 17 : 13;
    if (outputs < 1.6e6) return 14;
    if (outputs < 3.0e6) return 18;
    // Long M (the encoder's batched chunks): measured per weight format at
    // M = 3312, and for the int4 projections also at M = 1656 (one of two
    // row groups whose kernels run side by side).  Two LDS chunks in flight
    // (fewer registers, 3 waves per SIMD) win except for the int4 down
    // projection, whose 1656 wave-long chains fill 1024 SIMDs unevenly
    // whatever the occupancy.
    switch (kind) {
    case W_I4:  return N < K ? 11 : 20;
    case W_I8:  return 21;
    default:    return outputs >= 3.0e6 && N >= 2048 ? 23 : 21;
    }
}

int choose_config_index(int M, int N, int K, WeightKind kind) { return choose_index(M, N, K, kind); }

hipError_t launch_gemm(const GemmProblem& p, hipStream_t stream, int cfg_index, Tolerance tol)
{
    if (p.M <= 0 || p.N <= 0) return hipSuccess;
    if ((p.epi == EPI_HALF_RESIDUAL || p.epi == EPI_RESIDUAL) && p.beta != 0.0f)
        return hipErrorInvalidValue;
    if (p.chain_bias && (p.beta != 0.0f || p.bias || p.alpha == 0.0f || p.K <= 0 ||
                         (p.kind == W_I8 && p.scale == 0.0f)))
        return hipErrorInvalidValue;

    KArgs a = {};
    a.M = p.M; a.N = p.N; a.K = p.K;
    a.alpha = p.alpha; a.beta = p.beta;
    a.A = p.A; a.lda = p.lda;
    a.B = p.B; a.ldb = p.ldb;
    a.scale = p.scale;
    a.scales = p.scales; a.n_groups = p.N / 32;
    a.C = p.C; a.ldc = p.ldc;
    a.bias = p.bias; a.epi = p.epi;
    a.chain_bias = p.chain_bias;
    // GEMMs of at least 1.5M outputs (the encoder's row groups of 1656 rows
    // and up) keep the larger operand's blocks within one XCD's L2
    // (tile_origin): 1-3% faster at 3312 rows, 0.5% faster for the encoder's
    // two concurrent 1656-row groups (bench A/B, three runs each), with less
    // HBM traffic.  Smaller shapes keep the dispatch order, where the order
    // cost 1.5-3% (cold weights).
    a.tile_order = tiles::ORDER_DISPATCH;
    if ((double)p.M * p.N >= 1.5e6) {
        const double a_total = 4.0 * p.M * p.K;
        const double w_total = p.kind == W_F32 ? 4.0 * p.K * p.N
                             : p.kind == W_I8  ? 1.0 * p.K * p.N
                                               : 0.5 * p.K * p.N + 4.0 * p.K * (p.N / 32);
        a.tile_order = a_total >= w_total ? tiles::ORDER_ROWS : tiles::ORDER_COLS;
    }

    const bool fused = p.bias != nullptr || p.epi != EPI_NONE;
    const bool early = (p.alpha == 0.0f) || (p.kind == W_I8 && p.scale == 0.0f) || p.K <= 0;
    // the output LayerNorms ride on the panel or split-K reduce
    if ((p.out_ln_gamma || p.next_ln_gamma) && early) return hipErrorInvalidValue;
    if (early) {   // blas.c:764-765, 955-956, 1063-1064: only the beta step runs
        if (p.beta == 1.0f && !fused) return hipSuccess;
        const long long n = (long long)p.M * p.N;
        hipLaunchKernelGGL(scale_c, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a);
        return hipGetLastError();
    }

    if (p.ln_gamma || p.out_ln_gamma || p.next_ln_gamma) {
        // fused LayerNorms: the panel kernels apply input and output ones,
        // the split kernels' reduce output ones and the next GEMM's input
        if (tol == TOL_NONE || cfg_index >= 0) return hipErrorInvalidValue;
        if (!p.next_ln_gamma && panel_supports(p)) return launch_panel(p, stream);
        if (tol == TOL_ALL && split_fuses_ln(p)) return launch_split(p, stream);
        return hipErrorInvalidValue;
    }
    if (p.a_presplit) {
        // A comes pre-split: only the split kernels read it
        if (tol != TOL_ALL || cfg_index >= 0 || !split_supports(p)) return hipErrorInvalidValue;
        return launch_split(p, stream);
    }
    if (tol != TOL_NONE && cfg_index < 0) {
        if (panel_supports(p)) {
            const hipError_t e = launch_panel(p, stream);
            if (e != hipErrorNotSupported) return e;
        }
        if (smallm_supports(p)) {
            const hipError_t e = launch_smallm(p, stream);
            if (e != hipErrorNotSupported) return e;
        }
        if (tol == TOL_ALL && split_supports(p)) {
            const hipError_t e = launch_split(p, stream);
            if (e != hipErrorNotSupported) return e;
        }
    }

    // Exact extents of what the call may read; the kernels address operands
    // through 32-bit buffer offsets, so each must stay below 2 GiB.
    const size_t esz = p.kind == W_F32 ? 4 : 1;
    const size_t b_row = p.kind == W_I4 ? (size_t)p.N / 2 : (size_t)p.N;
    const size_t a_ext = ((size_t)(p.M - 1) * p.lda + p.K) * 4;
    const size_t b_ext = ((size_t)(p.K - 1) * p.ldb + b_row) * esz;
    const size_t s_ext = p.kind == W_I4 ? int4_scale_count(p.K, p.N) * 4 : 0;
    const size_t lim = (size_t)1 << 31;
    if (a_ext >= lim || b_ext >= lim || s_ext >= lim) return hipErrorInvalidValue;
    a.a_bytes = (uint32_t)a_ext;
    a.b_bytes = (uint32_t)b_ext;
    a.s_bytes = (uint32_t)s_ext;
    const uintptr_t pa = reinterpret_cast<uintptr_t>(p.A), pb = reinterpret_cast<uintptr_t>(p.B);
    a.vec_a = (p.lda % 4 == 0) && (pa % 16 == 0);
    a.vec_b = p.kind == W_F32 ? ((p.ldb % 4 == 0) && (pb % 16 == 0))
                              : ((p.ldb % 4 == 0) && (pb % 4 == 0));

    int n_main = p.N;
    if (p.kind == W_I8) n_main = (p.N / 16) * 16;     // blas.c:686, 734
    a.N = n_main;

    const int cfg = (cfg_index >= 0 && cfg_index < kNumConfigs) ? cfg_index
                                                                : choose_index(p.M, n_main, p.K, p.kind);
    hipError_t err = hipSuccess;
    if (n_main > 0) {
        switch (p.kind) {
        case W_F32: err = tiles::launch_chain_f32(cfg, a, stream); break;
        case W_I8:  err = tiles::launch_chain_i8(cfg, a, stream); break;
        case W_I4:  err = tiles::launch_chain_i4(cfg, a, stream); break;
        }
        if (err != hipSuccess) return err;
    }
    if (p.kind == W_I8 && n_main < p.N) {
        const int n_edge = p.N - n_main;
        const long long n = (long long)p.M * n_edge;
        hipLaunchKernelGGL(i8_edge, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                           a, n_main, n_edge);
        err = hipGetLastError();
    }
    return err;
}

// The weights the chain kernels multiply, written to out [K][N] through the
// staging's own loads and conversions (WStage): unit_path takes whole VB-column
// units (the kernels' path when rows allow vector loads), else one element
// at a time (the path of narrow or unaligned rows).
template <int WK>
__global__ __launch_bounds__(256) void dequant_matrix(KArgs p, float* out, int unit_path)
{
    using WS = tiles::WStage<WK>;
    const auto rb = tiles::make_rsrc(p.B, p.b_bytes), rs = tiles::make_rsrc(p.scales, p.s_bytes);
    const long long t = (long long)blockIdx.x * 256 + threadIdx.x;
    if (unit_path) {
        const int per_row = p.N / WS::VB;
        if (t >= (long long)p.K * per_row) return;
        const int k = (int)(t / per_row), n = (int)(t % per_row) * WS::VB;
        float w[WS::VB];
        WS::dequant_unit(p, WS::load_unit(p, rb, rs, k, n), w);
#pragma unroll
        for (int j = 0; j < WS::VB; ++j) out[(size_t)k * p.N + n + j] = w[j];
    } else {
        if (t >= (long long)p.K * p.N) return;
        const int k = (int)(t / p.N), n = (int)(t % p.N);
        out[(size_t)k * p.N + n] = WS::dequant_elem(p, WS::load_elem(p, rb, rs, k, n), n);
    }
}

int dequant_unit_columns(WeightKind kind)
{
    return kind == W_I4 ? tiles::WStage<W_I4>::VB : kind == W_I8 ? tiles::WStage<W_I8>::VB : tiles::WStage<W_F32>::VB;
}

hipError_t launch_dequant(WeightKind kind, int K, int N, const void* B, int ldb, float scale,
                          const float* scales, bool unit_path, float* out, hipStream_t stream)
{
    if (K <= 0 || N <= 0) return hipSuccess;
    if (unit_path && N % dequant_unit_columns(kind)) return hipErrorInvalidValue;
    KArgs a = {};
    a.N = N; a.K = K;
    a.B = B; a.ldb = ldb;
    a.scale = scale;
    a.scales = scales; a.n_groups = N / 32;
    const size_t esz = kind == W_F32 ? 4 : 1;
    const size_t b_row = kind == W_I4 ? (size_t)N / 2 : (size_t)N;
    const size_t b_ext = ((size_t)(K - 1) * ldb + b_row) * esz;
    const size_t s_ext = kind == W_I4 ? int4_scale_count(K, N) * 4 : 0;
    if (b_ext >= ((size_t)1 << 31) || s_ext >= ((size_t)1 << 31)) return hipErrorInvalidValue;
    a.b_bytes = (uint32_t)b_ext;
    a.s_bytes = (uint32_t)s_ext;
    const long long items = unit_path ? (long long)K * (N / dequant_unit_columns(kind)) : (long long)K * N;
    const dim3 grid((unsigned)((items + 255) / 256));
    const int up = unit_path ? 1 : 0;
    switch (kind) {
    case W_F32: hipLaunchKernelGGL(dequant_matrix<W_F32>, grid, dim3(256), 0, stream, a, out, up); break;
    case W_I8:  hipLaunchKernelGGL(dequant_matrix<W_I8>, grid, dim3(256), 0, stream, a, out, up); break;
    case W_I4:  hipLaunchKernelGGL(dequant_matrix<W_I4>, grid, dim3(256), 0, stream, a, out, up); break;
    }
    return hipGetLastError();
}

hipError_t launch_swish(const float* x, float* y, long long n, hipStream_t stream)
{
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(swish, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, x, y, n);
    return hipGetLastError();
}

}  // namespace pkgpu
