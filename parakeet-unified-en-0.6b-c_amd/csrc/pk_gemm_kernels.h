// pk_gemm_kernels.h - device-side entry points of the weight-GEMM library.
//
// Internal C++ interface between the kernels (pk_gemm_kernels.hip) and the
// host runtime (pk_gpu_runtime.hip).  All pointers are device pointers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace pkgpu {

enum WeightKind { W_F32 = 0, W_I8 = 1, W_I4 = 2 };

// Elementwise work fused into the GEMM's output store (encoder.c:193-216):
//   v = chain result; if bias: v = fl(v + bias[j]); then
//   EPI_SWISH:         C[i][j] = swish(v)                  (pk_swish)
//   EPI_HALF_RESIDUAL: C[i][j] = fl(C[i][j] + 0.5 * v)     (macaron residual)
//   EPI_RESIDUAL:      C[i][j] = fl(C[i][j] + v)           (attention / conv residual,
//                                                           encoder.c:410-424, 473-475)
//   EPI_RELU:          C[i][j] = v > 0 ? v : +0               (pk_relu, tensor_ops.c:401-415)
//   EPI_NONE:          C[i][j] = v
enum Epilogue { EPI_NONE = 0, EPI_SWISH = 1, EPI_HALF_RESIDUAL = 2, EPI_RESIDUAL = 3, EPI_RELU = 4 };

// One weight GEMM, C <- beta*C + alpha*A*W, row-major, NoTrans/NoTrans,
// with W given in one of the on-disk formats (weights.c:240-266):
//   W_F32: fp32 [K][ldb]
//   W_I8 : int8 [K][ldb] with one per-tensor scale
//   W_I4 : packed int4 [K][ldb bytes], two's-complement nibbles, low nibble
//          = even column, scales fp32 [K][N/32]
struct GemmProblem {
    WeightKind kind;
    int M, N, K;
    float alpha, beta;
    const float* A; int lda;
    const void* B;  int ldb;
    float scale;              // W_I8
    const float* scales;      // W_I4
    float* C; int ldc;
    const float* bias = nullptr;     // length N, or null
    Epilogue epi = EPI_NONE;         // the residual epilogues require beta == 0
    // Chains start from chain_bias[j] instead of beta*C (beta must be 0 and
    // bias null): a convolution whose sum starts from its bias (pk_conv2d).
    const float* chain_bias = nullptr;
    // Device memory of kSplitWorkBytes or more that the split kernels may
    // use for partial tiles (K split over workgroups), or null.  Calls that
    // overlap on the device must not share it.
    float* work = nullptr;
    size_t work_bytes = 0;
    // A given pre-split (split kernels only, TOL_ALL): per row and group of
    // 8 consecutive k, the 8 values hi = bf16(a) then the 8 lo = bf16(a - hi)
    // (split_bf16x2), so a row keeps the bytes and the pitch lda (in floats)
    // of the fp32 row.  launch_gemm refuses the problem if the split kernels
    // do not take it.
    bool a_presplit = false;
    // The weight's panel copy (launch_pack of this B, scales, K and N), or
    // null.  With it, the small-M path takes the panel kernels.
    const void* panel = nullptr;
    // The weight's pre-split copy (launch_split_pack of this B, scales, K and
    // N), or null.  The split kernels then stage it with plain copies instead
    // of decoding and splitting B (the same bf16 values).
    const void* b_presplit = nullptr;
    // Panel kernels only (panel_supports): A is x, and the GEMM multiplies
    // LayerNorm(x) over its K columns with these gamma, beta [K] (the
    // LayerNorm kernel's arithmetic, bit for bit; K <= 1024).
    const float* ln_gamma = nullptr;
    const float* ln_beta = nullptr;
    // Panel kernels with K split over workgroups (panel_fuses_out_ln), or
    // split kernels with K split over workgroups (split_fuses_ln): after the
    // output step, each output row is replaced by its LayerNorm with these
    // gamma, beta [N].
    const float* out_ln_gamma = nullptr;
    const float* out_ln_beta = nullptr;
    // Split kernels with K split over workgroups only (split_fuses_ln): the
    // LayerNorm with these gamma, beta [N] of the rows C ends with (after
    // out_ln_gamma's, if given) is written to next_ln_out [M][N], pre-split
    // as a_presplit describes, for a split GEMM that reads it next.
    const float* next_ln_gamma = nullptr;
    const float* next_ln_beta = nullptr;
    float* next_ln_out = nullptr;
};

// The row width (N) of a split GEMM whose reduce forms LayerNorms.
constexpr int kSplitLnN = 1024;

// Scales an int4 GEMM reads: the reference takes scale k * (N/32) + n/32 for
// weight (k, n) with N/32 floored (blas.c:794, 958), so when N % 32 != 0 the
// columns past the last whole group of row k read row k + 1's first scale and
// the last row's read one float past K * (N/32).
inline size_t int4_scale_count(int K, int N)
{
    return (size_t)K * (N / 32) + (N % 32 ? 1 : 0);
}

// Partial tiles of one split-K launch: at most 256 workgroups of at most
// 256 x 128 fp32 outputs each (32 MiB).
constexpr size_t kSplitWorkBytes = (size_t)256 * 256 * 128 * 4;

// Kernel tile configuration chosen for a shape (see choose_config_index).
//   family 'R': rows on MFMA lanes, one MFMA = 64 rows x mfma columns,
//               cw column tiles (independent chains) per wave;
//   family 'X': columns on MFMA lanes with A broadcast, one MFMA = mfma rows
//               x 64 columns, cw row groups (independent chains) per wave;
//   family 'S': the 'X' tiles with wgm*wgn additional producer waves that
//               stage the operands while the others only multiply;
//   family 'Y': the 'X' tiles with two LDS chunks of operands in flight
//               instead of four (fewer registers: more waves per SIMD).
struct TileConfig {
    char family;
    int mfma;   // 32, 16 or 4: v_mfma_f32_{32x32x1_2b,16x16x1_4b,4x4x1_16b}_f32
    int cw;     // independent chains (MFMA tiles) per wave
    int wgm;    // waves along M per workgroup
    int wgn;    // waves along N per workgroup
    int kt;     // k per LDS chunk
    int bm() const { return family == 'R' ? 64 * wgm : wgm * cw * mfma; }
    int bn() const { return family == 'R' ? mfma * cw * wgn : 64 * wgn; }
    int threads() const { return (family == 'S' ? 128 : 64) * wgm * wgn; }
};

// Pick the tile configuration with the lowest modelled time on 256 CUs.
int choose_config_index(int M, int N, int K, WeightKind kind);
// Number of configurations and access by index (for tests and sweeps).
int num_configs();
TileConfig config_at(int i);

// ---- small-M kernels (pk_smallm.hip): the tolerance path for M <= 64 -----
constexpr int kSmallMaxM = 64;
// Whether a shape and its operands' alignment suit the small-M kernels
// (M <= 64, K % 32 == 0, 16-byte aligned A rows, dword-aligned weight rows,
// int4: N % 32 == 0, ...).
bool smallm_supports(const GemmProblem& p);
// Tile the small-M kernel takes for a shape: rb 16-row blocks and nct
// 16-column tiles per workgroup.
void smallm_tile(const GemmProblem& p, int* rb, int* nct);
// Force the tile of later launches on the calling thread ((0, 0): the model's
// choice); false for an invalid tile.  fp32 clamps to nct = 1, rb <= 3.
bool smallm_force_tile(int rb, int nct);
// Launch on `stream`; hipErrorNotSupported if the shape is not handled (the
// caller then takes the exact kernels).
hipError_t launch_smallm(const GemmProblem& p, hipStream_t stream);

// ---- panel kernels (pk_panel.hip): small-M GEMMs on repacked weights ------
// Bytes of a weight's panel copy (0 if K is not a multiple of 32): int8
// ceil(N/16)*16*K, int4 half that plus the scales [N/32][K], fp32 4*that
// (bf16 hi and lo halves).
size_t panel_bytes(WeightKind kind, int K, int N);
// Write the panel copy of B [K][ldb] (int4: and its scales [K][N/32]) to
// `panel` (panel_bytes of device memory) on `stream`.
hipError_t launch_pack(WeightKind kind, int K, int N, const void* B, int ldb, const float* scales,
                       void* panel, hipStream_t stream);
// The weights as the panel kernels multiply them, to out [K][N] (int8 with
// `scale`): for tests of the repack.
hipError_t launch_panel_decode(WeightKind kind, int K, int N, const void* panel, float scale, float* out,
                               hipStream_t stream);
// Whether the panel kernels take a problem (p.panel set, M <= 64, K % 32 ==
// 0, 16-byte aligned A rows, int4 N % 32 == 0, alpha and scale nonzero, no
// chain bias).
bool panel_supports(const GemmProblem& p);
// K segments over workgroups a problem takes (> 1 only with p.work: the
// partial tiles are summed by a second launch).
int panel_segments(const GemmProblem& p);
// k of one LDS phase for a workgroup of `rows` rows.
int panel_phase_k(int rows);
// Whether the panel kernels can fuse an output LayerNorm (p.out_ln_gamma)
// into a problem: panel_supports(p) with K split over workgroups.
bool panel_fuses_out_ln(const GemmProblem& p);
// The workgroup tile a problem takes: mb 16-row blocks, nct 16-column tiles.
void panel_tile(const GemmProblem& p, int* mb, int* nct);
// Force the workgroup tile (mb 1..4, nct 1..2) on the calling thread ((0,
// 0): the default); false if out of range.
bool panel_force_tiles(int mb, int nct);
hipError_t launch_panel(const GemmProblem& p, hipStream_t stream);

// Whether a shape and its operands suit the split kernels (pk_split.hip):
// any M, K % 32 == 0, N % 32 == 0, 16-byte aligned A rows, dword-aligned
// weight rows (16-byte for fp32), no chain_bias.
bool split_supports(const GemmProblem& p);
// Launch on `stream`; hipErrorNotSupported if the shape is not handled.
// With p.work, shapes with too few tiles to fill the CUs split K over
// workgroups and sum the partial tiles in a second launch.
hipError_t launch_split(const GemmProblem& p, hipStream_t stream);
// Bytes of a weight's pre-split copy for the split kernels (K and N
// multiples of 32; else 0): int4 and fp32 K N 4, per 32-deep chunk and column
// the 32 bf16 hi halves then the 32 lo halves; int8 K N 2, per chunk and
// column the 32 codes as bf16.
size_t split_weight_bytes(WeightKind kind, int K, int N);
// Write that copy of B [K][ldb] (int4: and its scales [K][N/32]) to `out`.
hipError_t launch_split_pack(WeightKind kind, int K, int N, const void* B, int ldb, const float* scales,
                             void* out, hipStream_t stream);
// Whether the split kernels form the LayerNorms a problem asks for
// (p.out_ln_gamma, p.next_ln_gamma) in its split-K reduce: split_supports(p),
// N = kSplitLnN, K split over workgroups with p.work, 16-byte aligned C
// rows, bias, gammas, betas and next_ln_out, and no input LayerNorm.  The
// results are the same bits as the GEMM followed by the LayerNorm kernels.
bool split_fuses_ln(const GemmProblem& p);
// Segments of K over workgroups that launch_split takes for a shape given
// work_bytes of workspace (1: K is not split over workgroups).
int split_k_segments(WeightKind kind, int M, int N, int K, size_t work_bytes);

// Which shapes may leave the exact chains for a kernel within the 1e-3
// contract: none; those the small-M kernels take (M <= 64); or those and
// every other shape the split kernels take.
enum Tolerance { TOL_NONE = 0, TOL_SMALL_M = 1, TOL_ALL = 2 };

// Launch the whole GEMM (beta pre-pass semantics, early exits, int8 edge
// columns) on `stream`.  Returns hipSuccess or the launch error.
// cfg_index < 0 selects choose_config_index(); a forced configuration
// (cfg_index >= 0) always runs the exact chains.
hipError_t launch_gemm(const GemmProblem& p, hipStream_t stream, int cfg_index,
                       Tolerance tol = TOL_NONE);

// The weights the chain kernels multiply (fl(q*s), or the fp32 weight) into
// out [K][N], through the staging's own load and conversion code: whole
// units of dequant_unit_columns(kind) columns (N a multiple of them) or one
// element at a time.  For tests of the decode.
int dequant_unit_columns(WeightKind kind);
hipError_t launch_dequant(WeightKind kind, int K, int N, const void* B, int ldb, float scale,
                          const float* scales, bool unit_path, float* out, hipStream_t stream);

// Swish y = x * (1 / (1 + exp(-x))) with the reference's polynomial exp
// (tensor_ops.c:98-120, 381-388), n elements, in place allowed.
hipError_t launch_swish(const float* x, float* y, long long n, hipStream_t stream);

}  // namespace pkgpu
