// pk_block_kernels.h - device-side entry points of the conformer-block
// operations (pk_block_kernels.hip).  All pointers are device pointers;
// activations are time-major rows.
#pragma once

#include <hip/hip_runtime.h>

namespace pkgpu {

// Longest chunk whose score rows the attention kernel keeps in LDS.  The
// reference's encoder never attends over more than 500 frames unless
// chunking is forced off (PK_CHUNK_THRESHOLD, parakeet.h; encoder.c:595-610);
// longer sequences keep each workgroup's score rows in a device workspace
// (AttnArgs::scores) and run the same arithmetic.
constexpr int kAttnMaxT = 512;
constexpr int kAttnRows = 32;          // query rows per workgroup
// LDS row stride of a workgroup's score rows for chunks of T rows, and the
// workgroup's LDS: the score rows plus one staging tile of 64 x 68 floats.
// The stride is 8 more than a multiple of 32 floats, so rows 8 apart in
// banks: the softmax's 4 rows x 8 lanes and the value loop's 4 rows x 8
// keys per half wave reach 32 distinct banks.  At T = 416 two workgroups
// fit in a CU's 160 KiB.
__host__ __device__ constexpr int attn_sld(int T) { return ((T + 31) & ~31) + 8; }
__host__ __device__ constexpr unsigned attn_lds_bytes(int T)
{
    return 4u * (unsigned)(kAttnRows * attn_sld(T) + 64 * 68);
}

// Sequences of at most kAttnShortT rows take rel_pos_attention_short:
// kAttnShortRows query rows per workgroup, and every key, position and value
// row it reads staged in LDS at once (the score rows, then 64 key rows, one
// or two blocks of 64 position rows and the value rows, T rounded up to 16,
// each kTileLd = 132 floats apart).
constexpr int kAttnShortT = 64;
constexpr int kAttnShortRows = 16;
__host__ __device__ constexpr unsigned attn_short_lds_bytes(int T)
{
    return 4u * (unsigned)(kAttnShortRows * attn_sld(T) +
                           (64 + 64 * ((T + kAttnShortRows - 1 + 63) / 64) + ((T + 15) & ~15)) * 132);
}

// Relative-position attention of n chunks (encoder.c:300-408); chunk z has
// chunk_T[z] <= T rows (all T when chunk_T is null).
//   qkv  [rows][ldq]: Q | K | V (H*128 columns each, bias added); chunk z
//        starts at row chunk_rows[z]
//   P    [2T-1][ldp]: linear_pos(pe_slice(T)); a chunk of Tz rows uses its
//        rows [T - Tz, T + Tz - 1), which are linear_pos(pe_slice(Tz))
//   out  [rows][ldo]: the concatenated head outputs, chunk z at chunk_rows[z]
struct AttnArgs {
    const float* qkv; int ldq;
    const float* P; int ldp;
    const float* pos_bias_u;   // [H*128]
    const float* pos_bias_v;
    float* out; int ldo;
    const int* chunk_rows;     // device, n entries (null: one chunk at row 0)
    const int* chunk_T;        // device, n entries, each in [1, T] (null: all T)
    int T, H;
    // T > kAttnMaxT: attn_scores_floats(T, H, n) floats of device workspace,
    // one slice of score rows per workgroup (unused otherwise)
    float* scores;
};
// Workspace floats the attention of n chunks of up to T rows needs (0 when
// its score rows fit in LDS).
inline size_t attn_scores_floats(int T, int H, int n_chunks)
{
    if (T <= kAttnMaxT) return 0;
    return (size_t)((T + kAttnRows - 1) / kAttnRows) * H * n_chunks * kAttnRows * attn_sld(T);
}

// Depthwise convolution over time with optional Swish (tensor_ops.c:476-548,
// encoder.c:467-469), channel c of chunk z: x[chunk_rows[z] + t][c] for t in
// [0, chunk_T[z]) (all T when chunk_T is null).
struct DwArgs {
    const float* x; int ldx;
    const float* w;            // [C][K]
    const float* b;            // [C] or null
    float* out; int ldo;
    const int* chunk_rows;     // device, n entries (null: one chunk at row 0)
    const int* chunk_T;        // device, n entries, each in [1, T] (null: all T)
    int T, C, K;
    int swish;
    // x holds the pointwise convolution's 2C-wide rows and each input value
    // is their GLU, gated = x[t][c] * (1 / (1 + exp(-x[t][C + c]))), formed
    // as the GLU kernel forms it (the GLU fused: the same bits)
    int glu;
};

hipError_t launch_layer_norm(const float* x, int ldx, const float* gamma, const float* beta,
                             float* out, int ldo, int rows, int D, hipStream_t s);
// The same LayerNorm with its output pre-split for the split GEMM kernels
// (GemmProblem::a_presplit): the fp32 row's bytes hold, per group of 8
// columns, the 8 bf16 hi then the 8 bf16 lo halves.
hipError_t launch_layer_norm_split(const float* x, int ldx, const float* gamma, const float* beta,
                                   float* out, int ldo, int rows, int D, hipStream_t s);
hipError_t launch_attention(const AttnArgs& a, int n_chunks, hipStream_t s);
// The same attention on split bf16 operands (fast numerics, within about 1e-5
// of launch_attention; not bit-identical), for T <= kAttnMaxT: a first
// launch splits the chunks' keys and values and the launch's position rows
// into ws, in the matrix cores' fragment order, which must hold
// attn_fast_ws_floats(a.T, a.H, n_chunks) floats.
size_t attn_fast_ws_floats(int T, int H, int n_chunks);
hipError_t launch_attention_fast(const AttnArgs& a, int n_chunks, float* ws, size_t ws_floats, hipStream_t s);
hipError_t launch_glu(const float* in, int ldi, float* out, int ldo, int rows, int D, hipStream_t s);
hipError_t launch_depthwise(const DwArgs& a, int n_chunks, hipStream_t s);
hipError_t launch_transpose(const float* in, float* out, int R, int C, hipStream_t s);

// Pre-encode subsampling (encoder.c:103-174), channel-last [H][W][256].
hipError_t launch_conv0_relu(const float* mel, int T, int n_mels, const float* w, const float* b,
                             float* out, int H1, int W1, hipStream_t s);
hipError_t launch_dwconv3x3s2(const float* in, int H, int W, const float* w, const float* b,
                              float* out, int Ho, int Wo, hipStream_t s);
hipError_t launch_flatten_rows(const float* in, float* out, int H, int W, hipStream_t s);
hipError_t launch_scale(float* x, long long n, float sc, hipStream_t s);

}  // namespace pkgpu
