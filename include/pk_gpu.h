/*  pk_gpu.h - C ABI of the MI355X (gfx950) weight-GEMM library libpk_gpu.so.
 *
 *  Drop-in for the three weight GEMMs of eschmidbauer/parakeet-unified-en-0.6b-c
 *  (csrc/blas.h:38-69).  Plain C types and pointers only.  Every function
 *  returns PK_GPU_OK (0) or a negative pk_gpu_status; pk_gpu_last_error()
 *  gives a message for the calling thread.  Nothing here falls back to the
 *  CPU: a missing or non-gfx950 device is an error.
 *
 *  Semantics shared by the GEMMs (blas.c:89-99, 759-771, 950-963, 1055-1072):
 *    C <- beta*C (beta == 0 clears C, beta == 1 leaves it), then, unless
 *    alpha == 0 (or, for int8, B_scale == 0), C += alpha * A * W, row-major,
 *    where every C[i][j] is the same sequential fused multiply-add chain over
 *    k ascending that the reference evaluates, so results are bit-identical.
 *    The exceptions are the tolerance paths (pk_gpu_set_numerics): GEMMs
 *    with M <= 64 stream the weights once through bf16 matrix cores and sum
 *    the same products in another order, within max |C - R| / max |R| <=
 *    1e-3 of the reference (about 1e-5 measured), unless the calling thread
 *    asks for exact numerics; with PK_GPU_NUMERICS_FAST longer GEMMs do the
 *    same through the split kernels.
 *
 *  Host-pointer entry points (pk_gpu_gemm_i8, pk_gpu_gemm_i4, pk_gpu_sgemm)
 *  take host memory, exactly as the reference BLAS does.  A weight operand
 *  whose host range was registered with pk_gpu_register_weight is read from
 *  its resident device copy; any other operand is copied in for the call.
 *  C is copied back before the call returns.  Calls may come from any
 *  thread; each thread gets its own HIP stream and staging buffers.
 *
 *  Device-pointer entry points (*_dev) take device pointers, enqueue on the
 *  given HIP stream (NULL = HIP's null stream) and return without
 *  synchronising.
 */
#ifndef PK_GPU_H
#define PK_GPU_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    PK_GPU_OK       = 0,
    PK_GPU_EINVAL   = -1,   /* bad argument (sizes, strides, NULL pointer)  */
    PK_GPU_ENOTSUP  = -2,   /* form the reference call sites never use       */
    PK_GPU_ENOMEM   = -3,   /* device or pinned allocation failed            */
    PK_GPU_EHIP     = -4,   /* HIP runtime or launch error                   */
    PK_GPU_ENODEV   = -5,   /* no gfx950 device                              */
    PK_GPU_EBUSY    = -6    /* a call on another thread is using the weight  */
} pk_gpu_status;

/* Select the device (-1: $PK_GPU_DEVICE or 0) and check it is gfx950.
 * Idempotent; the GEMM entry points call it on first use. */
int pk_gpu_init(int device);
/* Free resident weights (after the device's queued work), the calling
 * thread's stream and staging buffers, and those left by exited threads.
 * A thread that exits without calling this leaves its stream and buffers
 * for the next thread to reuse. */
void pk_gpu_shutdown(void);
/* Message for the last failing call on this thread ("" if none). */
const char *pk_gpu_last_error(void);

/* ---- resident weights ------------------------------------------------- */

/* Copy host range [host, host+bytes) to the device once.  Later calls whose
 * operand lies inside a registered range read the device copy.  The host
 * bytes must not change while registered (the reference's weights are
 * read-only mmap'd or load-time buffers, weights.c:294-302, 404-546).
 * Registering an overlapping range is PK_GPU_EINVAL. */
int pk_gpu_register_weight(const void *host, size_t bytes);
/* Later calls no longer find the range; the device copy (and any panel
 * made from it, pk_gpu_pack_weight_dev) is freed on the calling thread after
 * the work queued on the device.  While a host-pointer GEMM on another thread
 * is reading the weight it returns PK_GPU_EBUSY and changes nothing: try
 * again after that call.  Device-pointer work that reads the copy through
 * pk_gpu_device_ptr must be queued before the unregister. */
int pk_gpu_unregister_weight(const void *host);
/* Device address of a registered host pointer (or NULL), valid until the
 * weight is unregistered. */
const void *pk_gpu_device_ptr(const void *host);
/* Bytes currently resident. */
size_t pk_gpu_resident_bytes(void);

/* ---- drop-in GEMMs (host pointers) ------------------------------------ */

/* Replaces cblas_sgemm_qb (blas.h:54-62, blas.c:759-771): int8 B [K][ldb]
 * with one per-tensor scale. */
int pk_gpu_gemm_i8(int M, int N, int K, float alpha,
                   const float *A, int lda,
                   const int8_t *B, float B_scale, int ldb,
                   float beta, float *C, int ldc);

/* pk_gpu_gemm_i8 for callers that cannot allocate (serving loops that must
 * not call hipMalloc, harnesses that forbid it).  No counterpart in the
 * reference.  Same arguments and results as pk_gpu_gemm_i8 (host pointers;
 * a registered B is read from its resident copy), but every staged operand
 * (A, C, and B unless registered) goes to a fixed device array of
 * PK_GPU_NOALLOC_BYTES that each device the library runs on holds until the
 * process ends, and the work runs on `stream` (NULL: the null stream); the
 * call waits for it before returning.  It calls no allocating routine.
 * Returns PK_GPU_EINVAL, touching nothing, when the staged bytes (each
 * operand rounded up to 256) exceed PK_GPU_NOALLOC_BYTES.  All calls in a
 * process share the array and take turns (a lock): calls from several
 * threads are serialised, not concurrent. */
#define PK_GPU_NOALLOC_BYTES (64u << 20)
int pk_gpu_gemm_i8_noalloc(int M, int N, int K, float alpha,
                           const float *A, int lda,
                           const int8_t *B, float B_scale, int ldb,
                           float beta, float *C, int ldc, void *stream);

/* Replaces cblas_sgemm_q4b (blas.h:64-69, blas.c:950-963): packed int4
 * B [K][ldb bytes] (two's-complement nibbles, low nibble = even column,
 * extract_weights.py:589-592) with fp32 scales [K][N/32] (blas.c:794, 958).
 * N must be even and ldb >= N/2.  As in the reference, weight (k, n) takes
 * scale k * (N/32) + n/32 with N/32 floored: when N is not a multiple of 32
 * (no shipped weight, extract_weights.py:523), the columns past the last
 * whole group of row k take row k + 1's first scale, and the last row's
 * read one float past K * (N/32), which `scales` must then hold
 * (K * (N/32) + 1 floats). */
int pk_gpu_gemm_i4(int M, int N, int K, float alpha,
                   const float *A, int lda,
                   const uint8_t *B, const float *scales, int ldb,
                   float beta, float *C, int ldc);

/* Replaces cblas_sgemm (blas.h:38-43, blas.c:1055-1072) for
 * transA == transB == CblasNoTrans (111), the only form its callers use
 * (tensor_ops.c:31-36, 579-590); other forms return PK_GPU_ENOTSUP.
 * Either A or B may be a registered weight (pointwise conv passes the
 * weight as A, tensor_ops.c:582-583). */
int pk_gpu_sgemm(int transA, int transB, int M, int N, int K, float alpha,
                 const float *A, int lda, const float *B, int ldb,
                 float beta, float *C, int ldc);

/* ---- device-pointer variants (no copies, no synchronisation) ----------- */

int pk_gpu_gemm_i8_dev(int M, int N, int K, float alpha,
                       const float *dA, int lda,
                       const int8_t *dB, float B_scale, int ldb,
                       float beta, float *dC, int ldc, void *stream);
int pk_gpu_gemm_i4_dev(int M, int N, int K, float alpha,
                       const float *dA, int lda,
                       const uint8_t *dB, const float *dscales, int ldb,
                       float beta, float *dC, int ldc, void *stream);
int pk_gpu_sgemm_dev(int M, int N, int K, float alpha,
                     const float *dA, int lda, const float *dB, int ldb,
                     float beta, float *dC, int ldc, void *stream);

/* Fused epilogues (encoder.c:193-216: the feed-forward's bias add, Swish and
 * 0.5 residual, done on the host after each weight GEMM).  The chain result v
 * of every output gets, in order:
 *   bias (length N, device pointer, may be NULL): v = fl(v + bias[j]);
 *   PK_GPU_EPI_NONE:          C[i][j] = v
 *   PK_GPU_EPI_SWISH:         C[i][j] = swish(v)   (as pk_gpu_swish_dev)
 *   PK_GPU_EPI_HALF_RESIDUAL: C[i][j] = C[i][j] + 0.5 * v   (beta must be 0:
 *                             C holds the residual x on entry)
 *   PK_GPU_EPI_RESIDUAL:      C[i][j] = C[i][j] + v   (beta must be 0; the
 *                             attention and convolution residuals,
 *                             encoder.c:410-424, 473-475)
 *   PK_GPU_EPI_RELU:          C[i][j] = v > 0 ? v : +0   (pk_relu after the
 *                             pre-encode's pointwise convolutions,
 *                             encoder.c:132-150)
 * Bias and residual are exact IEEE operations, so results equal the
 * reference's GEMM + pk_bias_add (+ x += 0.5 * out) bit for bit; Swish is
 * pk_gpu_swish_dev's.  No counterpart exists in blas.h: the reference runs
 * these as separate host loops; these entry points serve GPU-resident
 * callers that chain the block on the device. */
#define PK_GPU_EPI_NONE 0
#define PK_GPU_EPI_SWISH 1
#define PK_GPU_EPI_HALF_RESIDUAL 2
#define PK_GPU_EPI_RESIDUAL 3
#define PK_GPU_EPI_RELU 4
int pk_gpu_gemm_i8_ex_dev(int M, int N, int K, float alpha, const float *dA, int lda,
                          const int8_t *dB, float B_scale, int ldb, float beta, float *dC,
                          int ldc, const float *dbias, int epilogue, void *stream);
int pk_gpu_gemm_i4_ex_dev(int M, int N, int K, float alpha, const float *dA, int lda,
                          const uint8_t *dB, const float *dscales, int ldb, float beta,
                          float *dC, int ldc, const float *dbias, int epilogue, void *stream);
int pk_gpu_sgemm_ex_dev(int M, int N, int K, float alpha, const float *dA, int lda,
                        const float *dB, int ldb, float beta, float *dC, int ldc,
                        const float *dbias, int epilogue, void *stream);

/* Swish y = x * (1 / (1 + e)), e = exp(-x) by the reference's polynomial
 * (tensor_ops.c:98-120, 367-389), with the IEEE division its source writes
 * (the reference's -ffast-math build computes 1/(1 + e) with vrcpps plus a
 * Newton step instead, within a few ulp of this); x may equal y. */
int pk_gpu_swish_dev(const float *dx, float *dy, long long n, void *stream);

/* ---- conformer-block operations (device pointers, no synchronisation) --
 * The operations between the weight GEMMs of one FastConformer block, for
 * callers that keep activations on the device (encoder.c:179-491).  Rows are
 * time-major.  Results equal the reference's bit for bit where its order of
 * operations is fixed (noted per function); where the reference's build
 * uses a CPU-model-specific approximation (vrsqrtss, vrcpps) or glibc's
 * vector expf, the value here is the one its source's IEEE operations
 * define, or a correctly rounded exp (see pk_gpu_glu_dev). */

/* LayerNorm of `rows` rows of D = 1024 floats (pk_layer_norm_rows,
 * tensor_ops.c:150-185, 187-211; d_model); dout may equal dx.  The sums are
 * the reference's; 1/sqrt(var + 1e-5) is correctly rounded.  x, gamma, beta
 * and out 16-byte aligned. */
int pk_gpu_layer_norm_dev(const float *dx, const float *dgamma, const float *dbeta,
                          float *dout, int rows, int D, void *stream);

/* Relative-position multi-head attention of one sequence of T rows
 * (encoder.c:300-408, from the fused QKV output to the concatenated heads):
 *   qkv  [T][ldq]      Q | K | V, H*128 columns each, bias added
 *   P    [2T-1][ldp]   linear_pos applied to the T-row positional slice
 *   pos_bias_u, pos_bias_v  [H*128]
 *   out  [T][ldo]      head h in columns [128h, 128h+128)
 * Head dimension 128 (PK_HEAD_DIM), 1 <= T <= 512; ldq, ldp, ldo multiples of
 * 4 and 16-byte aligned rows.  Bit-identical to the reference when T % 8 == 0
 * (softmax's scalar tail otherwise uses the exp of pk_gpu_glu_dev). */
int pk_gpu_attention_dev(const float *dqkv, int ldq, const float *dP, int ldp,
                         const float *dpos_bias_u, const float *dpos_bias_v,
                         float *dout, int ldo, int T, int H, void *stream);
/* Workspace (floats) pk_gpu_attention_ws_dev needs for T rows and H heads:
 * 0 up to T = 512 (the score rows stay on chip), else about H * T^2. */
size_t pk_gpu_attention_ws_floats(int T, int H);
/* pk_gpu_attention_dev for any T (the reference attends over a whole
 * sequence when chunking is off, encoder.c:595-610), the score rows of
 * T > 512 in the caller's 16-byte aligned workspace dws of ws_floats >=
 * pk_gpu_attention_ws_floats(T, H) floats (unused up to 512).  Same
 * operations and bits as pk_gpu_attention_dev. */
int pk_gpu_attention_ws_dev(const float *dqkv, int ldq, const float *dP, int ldp,
                            const float *dpos_bias_u, const float *dpos_bias_v,
                            float *dout, int ldo, int T, int H, float *dws, size_t ws_floats,
                            void *stream);

/* GLU over rows of [va | vb] (2*D wide) into rows of D (encoder.c:453-461):
 * va * (1 / (1 + exp(-vb))) with IEEE division.  exp is evaluated in double
 * (range reduction by ln2, degree-12 Taylor polynomial, one rounding to
 * float): the correctly rounded expf except where e^x lies within about
 * 2^-51 (relative) of a rounding boundary, and the same bits as the same
 * double operations give on any IEEE machine. */
int pk_gpu_glu_dev(const float *din, float *dout, int rows, int D, void *stream);

/* Depthwise convolution over time with zero padding (pk_depthwise_conv1d,
 * tensor_ops.c:476-548) on time-major x [T][ldx] (C channels), weights
 * [C][K] (K odd), bias [C] or NULL, then Swish when swish != 0
 * (encoder.c:467-469).  The convolution is bit-identical to the compiled
 * reference for every T; Swish as in the GEMM epilogue. */
int pk_gpu_depthwise_dev(const float *dx, int ldx, const float *dw, const float *db,
                         float *dout, int ldo, int T, int C, int K, int swish,
                         void *stream);

/* ---- device-resident encoder ------------------------------------------
 * The 24 conformer blocks of the encoder (encode_blocks / encode_blocks_
 * chunked, encoder.c:179-575) with every activation kept on the device.  In
 * chunked mode all chunks run as one batch: row-independent work (LayerNorm,
 * the weight GEMMs and their epilogues, GLU) over all chunks' rows at once,
 * attention and the depthwise convolution per chunk, the position projection
 * once per block for the longest chunk (a shorter chunk's positional slice
 * is a row range of the longest one's).  Weights are uploaded once at
 * creation; the host copies may be freed afterwards. */

/* One weight matrix as the reference holds it (Weight, parakeet.h:42-57):
 * bits 32: fp32 [K][N]; 8: int8 [K][N] with one scale; 4: packed int4
 * [K][N/2] with fp32 scales [K][N/32]. */
typedef struct {
    const void  *data;
    float        scale;
    const float *scales;
    int          bits;
} pk_gpu_weight;

/* One conformer block's parameters (ConformerBlock, parakeet.h), host
 * pointers.  Shapes with d = 1024, ff = 4096, 8 heads of 128:
 *   norm_*: [d];  ff*_linear1: [d][ff] + bias [ff];  ff*_linear2: [ff][d] +
 *   bias [d];  linear_qkv: [d][3d] + bias [3d];  linear_pos: [d][d], no
 *   bias;  linear_out: [d][d] + bias [d];  pos_bias_u/v: [d];
 *   conv_pw1: fp32 [2d][d] + bias [2d];  conv_dw: [d][9] + bias [d];
 *   conv_pw2: fp32 [d][d] + bias [d]. */
typedef struct {
    const float *norm_ff1_w, *norm_ff1_b;
    pk_gpu_weight ff1_linear1_w; const float *ff1_linear1_b;
    pk_gpu_weight ff1_linear2_w; const float *ff1_linear2_b;
    const float *norm_sa_w, *norm_sa_b;
    pk_gpu_weight linear_qkv_w;  const float *linear_qkv_b;
    pk_gpu_weight linear_pos_w;
    pk_gpu_weight linear_out_w;  const float *linear_out_b;
    const float *pos_bias_u, *pos_bias_v;
    const float *norm_conv_w, *norm_conv_b;
    const float *conv_pw1_w, *conv_pw1_b;
    const float *conv_dw_w, *conv_dw_b;
    const float *conv_pw2_w, *conv_pw2_b;
    const float *norm_ff2_w, *norm_ff2_b;
    pk_gpu_weight ff2_linear1_w; const float *ff2_linear1_b;
    pk_gpu_weight ff2_linear2_w; const float *ff2_linear2_b;
    const float *norm_out_w, *norm_out_b;
} pk_gpu_block_weights;

typedef struct pk_gpu_encoder pk_gpu_encoder;

/* Upload n_blocks blocks and the positional-encoding table pe_table
 * [pe_rows][1024] whose centre row is pe_center (PK_PE_TABLE_SIZE,
 * PK_PE_CENTER). */
int pk_gpu_encoder_create(pk_gpu_encoder **enc, const pk_gpu_block_weights *blocks,
                          int n_blocks, const float *pe_table, int pe_rows, int pe_center);
/* Run every block over x [T][1024] into out [T][1024] (out may equal x).
 * chunk_size <= 0: one sequence (encode_blocks, encoder.c:495-512);
 * otherwise chunks of chunk_size output frames with `overlap` frames of
 * context on each side (encode_blocks_chunked, encoder.c:514-575; the
 * reference uses PK_CHUNK_SIZE 400 and PK_CHUNK_OVERLAP 8).  A chunk (or
 * the sequence) of T' frames needs the positional table's rows centre - T' + 1
 * .. centre + T' - 1 (T' <= 5000 for the reference's 9999-row table; longer
 * is PK_GPU_EINVAL).  Chunks up to 512 frames keep attention scores on chip;
 * a longer one (chunking off, as PK_CHUNK=0 runs the reference) keeps them in
 * a workspace of H * T'^2 floats, and the first run that long recomputes every
 * block's position projection for the longer slice.  Host pointers; returns
 * when out is written. */
int pk_gpu_encoder_run(pk_gpu_encoder *enc, const float *x, int T, int chunk_size,
                       int overlap, float *out);
/* The same with device pointers, enqueued on `stream` (NULL = HIP's null
 * stream, as for every *_dev entry point); returns without synchronising.
 * Runs and pre-encodes of one encoder share its workspace: one enqueued on
 * another stream than the previous call's first waits on the device for
 * that call, so they never overlap.  One encoder takes calls from one host
 * thread at a time.  The blocks'
 * launches are captured in a HIP graph on the first run of each (T,
 * chunk_size, overlap, configuration forced with pk_gpu_force_config on the
 * calling thread) and replayed afterwards (not while profiling). */
int pk_gpu_encoder_run_dev(pk_gpu_encoder *enc, const float *dx, int T, int chunk_size,
                           int overlap, float *dout, void *stream);
/* Pre-encode parameters (PreEncodeWeights, parakeet.h), host pointers:
 * conv0 [256][1][3][3], conv2 depthwise [256][1][3][3], conv3 pointwise
 * [256][256], conv5 depthwise [256][1][3][3], conv6 pointwise [256][256],
 * each with a [256] bias; out_w [4096][1024] (int8 or fp32) + out_b [1024]. */
typedef struct {
    const float *conv0_w, *conv0_b;
    const float *conv2_w, *conv2_b;
    const float *conv3_w, *conv3_b;
    const float *conv5_w, *conv5_b;
    const float *conv6_w, *conv6_b;
    pk_gpu_weight out_w;
    const float *out_b;
} pk_gpu_pre_encode_weights;

/* Upload the pre-encode once (replacing an earlier one). */
int pk_gpu_encoder_set_pre_encode(pk_gpu_encoder *enc, const pk_gpu_pre_encode_weights *w);
/* Encoder frames T' for n_frames mel frames (three stride-2 stages). */
int pk_gpu_encoder_frames(int n_frames);
/* pre_encode_and_scale (encoder.c:103-174, 578-592) on the device: mel
 * [128][n_frames] (as pk_encoder takes it) to x [T'][1024], bit-identical to
 * the reference.  Enqueued on `stream`. */
int pk_gpu_encoder_pre_encode_dev(pk_gpu_encoder *enc, const float *dmel, int n_frames,
                                  float *dx, void *stream);
/* pk_encoder (encoder.c:595-624) from mel to encoder output: host mel
 * [128][n_frames] in, out [T'][1024] (pk_gpu_encoder_frames(n_frames) rows);
 * chunk_size / overlap as for pk_gpu_encoder_run.  Returns when out is
 * written. */
int pk_gpu_encoder_run_mel(pk_gpu_encoder *enc, const float *mel, int n_frames, int chunk_size,
                           int overlap, float *out);

/* Device bytes held by the encoder (weights + workspace). */
size_t pk_gpu_encoder_bytes(const pk_gpu_encoder *enc);

/* Per-stage timing of later runs: with enable != 0, every launch of a run is
 * bracketed by HIP events on the caller's stream (the reference's pk_verbose
 * timers have no finer granularity): the launches of a replayed run, same
 * row groups and tiles, issued one by one and one group after another, so
 * each kernel is timed alone; 0 stops and clears.  Stages: */
#define PK_GPU_STAGE_GEMM_I4    0   /* feed-forward GEMMs (int4)              */
#define PK_GPU_STAGE_GEMM_I8    1   /* QKV, position, output GEMMs (int8)     */
#define PK_GPU_STAGE_GEMM_F32   2   /* pointwise-convolution GEMMs (fp32)     */
#define PK_GPU_STAGE_ATTENTION  3   /* relative-position attention            */
#define PK_GPU_STAGE_LAYER_NORM 4
#define PK_GPU_STAGE_CONV       5   /* GLU, depthwise convolution + Swish     */
#define PK_GPU_STAGE_COPY       6   /* chunk input / output copies            */
#define PK_GPU_N_STAGES         7
int pk_gpu_encoder_profile(pk_gpu_encoder *enc, int enable);
/* Totals of one stage since profiling was enabled: device time in ms,
 * launches, algorithmic flops (2*M*N*K for the GEMMs and attention's three
 * products) and algorithmic bytes (operands read once + results written
 * once).  Waits for the profiled runs to finish.  Any pointer may be NULL. */
int pk_gpu_encoder_profile_read(pk_gpu_encoder *enc, int stage, double *ms, long long *launches,
                                double *flops, double *bytes);
/* Rows of a chunked input are split into n_groups groups of whole chunks
 * (default 2, at most PK_GPU_MAX_GROUPS; never more than the chunks) that
 * run_dev replays concurrently: group 0 on the caller's stream, the others on
 * the encoder's side streams (starting once group 0 has run block 0's first
 * feed-forward module; PK_GPU_GROUP_LAG=0..3 modules in the environment sets
 * that lead), joined before the output copies.  Every
 * operation of a block is row-wise or per chunk, so the result does not
 * depend on the grouping.  No counterpart in the reference (which runs the
 * chunks one after another); it overlaps one group's latency-bound kernels
 * and launch tails with the other's GEMMs.  Profiled runs issue the groups
 * one after another. */
#define PK_GPU_MAX_GROUPS 4
int pk_gpu_encoder_set_groups(pk_gpu_encoder *enc, int n_groups);
/* Modules of block 0 (0..3: none, feed-forward 1, + self-attention,
 * + convolution) that group 0 runs before the other groups start; -1 (the
 * initial setting) takes PK_GPU_GROUP_LAG from the environment, else 1.
 * The results do not depend on it.  No counterpart in the reference. */
int pk_gpu_encoder_set_group_lag(pk_gpu_encoder *enc, int modules);
/* Numerics of this encoder's weight GEMMs.  PK_GPU_NUMERICS_EXACT (the
 * default): every GEMM is the reference's fma chain, and the whole encoder
 * is bit-identical to the reference's arithmetic.  PK_GPU_NUMERICS_DEFAULT:
 * GEMMs with at most 64 rows (a sequence or chunk batch of at most 64 frames
 * per row group, such as a 2.56 s clip's 33) take the small-M kernels, each
 * within max |C - R| / max |R| <= 1e-3 of the reference GEMM (about 1e-5);
 * longer inputs are unaffected.  PK_GPU_NUMERICS_FAST: every weight GEMM
 * takes the small-M or the split kernels (see pk_gpu_set_numerics), each
 * within the same bound; over 24 blocks the deviations compound, so the
 * output is not bit-identical at any length.  In this mode a run also holds
 * PK_GPU_SPLIT_WORKSPACE_BYTES per row group for the split kernels' partial
 * tiles (counted by pk_gpu_encoder_bytes), and the LayerNorms that feed a
 * GEMM write their output already split into the bf16 halves those kernels
 * multiply (the same bits as splitting it in the GEMM; PK_GPU_PRESPLIT=0 in
 * the environment when the encoder is created turns that off).  Captured
 * graphs are kept per mode.  No counterpart in the reference.  get returns the mode, -1 for
 * NULL. */
int pk_gpu_encoder_set_numerics(pk_gpu_encoder *enc, int mode);
int pk_gpu_encoder_get_numerics(pk_gpu_encoder *enc);
void pk_gpu_encoder_destroy(pk_gpu_encoder *enc);

/* ---- tuning / introspection ------------------------------------------- */

/* Number of kernel tile configurations, and a description of one:
 * family ('R': rows on MFMA lanes, 'X': columns on lanes with A broadcast,
 * 'S': the 'X' tiles plus as many producer waves that stage the operands,
 * 'Y': the 'X' tiles with two LDS chunks in flight instead of four),
 * mfma (32, 16 or 4 = v_mfma_f32_{32x32x1_2b,16x16x1_4b,4x4x1_16b}_f32),
 * independent chains per wave, multiplying waves along M and N per
 * workgroup, and k per LDS chunk.  Any pointer may be NULL. */
int pk_gpu_num_configs(void);
int pk_gpu_config_info(int index, int *family, int *mfma, int *cw, int *wgm, int *wgn,
                       int *kt);
/* Index of the configuration the dispatcher picks for a shape with int8
 * weights, and for weights of `bits` = 4, 8 or 32 (fp32) bits (-1 for any
 * other value). */
int pk_gpu_pick_config(int M, int N, int K);
int pk_gpu_pick_config_bits(int M, int N, int K, int bits);
/* Numerics of later GEMM calls on this thread:
 *   PK_GPU_NUMERICS_DEFAULT  GEMMs with M <= 64 (K a multiple of 32,
 *       16-byte aligned A rows, dword-aligned weight rows (16-byte for
 *       int4 and fp32), N a multiple of 32 for int4; blas.c's cblas_sgemm_qb
 *       / _q4b / cblas_sgemm at a short clip's M = 33) take the small-M
 *       kernels: the weights stream once, each workgroup sums all of K for
 *       its tile across its waves in a fixed order, so the result is
 *       deterministic and within max |C - R| / max |R| <= 1e-3 of the
 *       reference R.  They use no memory beyond the operands.  Every other
 *       shape is bit-identical to the reference.
 *   PK_GPU_NUMERICS_EXACT  every shape bit-identical to the reference.
 *   PK_GPU_NUMERICS_FAST  as DEFAULT for M <= 64; every other shape with K a
 *       multiple of 32, N a multiple of 32, 16-byte aligned A rows and
 *       dword-aligned weight rows (16-byte for fp32), without a chain bias,
 *       takes the split kernels: v_mfma_f32_32x32x16_bf16 on operands split
 *       into two bf16 halves (the int8 codes and int4 codes exactly; int4
 *       weights dequantised exactly first), fp32 accumulators, within
 *       max |C - R| / max |R| <= 1e-3 of the reference (about 1e-5),
 *       deterministic, no memory beyond the operands unless the thread gives
 *       a workspace (pk_gpu_set_workspace).  Shapes outside those rules stay
 *       bit-identical.
 * The environment variable PK_GPU_NUMERICS=exact (or =fast) makes EXACT (or
 * FAST) every thread's default.  A forced configuration (pk_gpu_force_config) implies exact
 * chains.  The device-resident encoder (pk_gpu_encoder_*) has a setting of
 * its own (pk_gpu_encoder_set_numerics), exact by default.
 * No counterpart in the reference. */
#define PK_GPU_NUMERICS_DEFAULT 0
#define PK_GPU_NUMERICS_EXACT   1
#define PK_GPU_NUMERICS_FAST    2
int pk_gpu_set_numerics(int mode);
int pk_gpu_get_numerics(void);
/* Whether a GEMM of this shape and weight format (bits 4, 8 or 32) would take
 * the small-M kernels on this thread, given aligned operands. */
int pk_gpu_uses_small_m(int M, int N, int K, int bits);
/* Whether such a GEMM would take the split kernels on this thread
 * (PK_GPU_NUMERICS_FAST and a shape the small-M kernels do not take). */
int pk_gpu_uses_split(int M, int N, int K, int bits);
/* Device memory that this thread's later split-kernel GEMMs
 * (PK_GPU_NUMERICS_FAST) may use for partial tiles.  With at least
 * PK_GPU_SPLIT_WORKSPACE_BYTES, a shape with fewer 128 x 128 tiles than the
 * 256 CUs splits K over workgroups: each stores its raw partial tile, and a
 * second launch sums a tile's partials in segment order before alpha, beta,
 * bias and the epilogue, so results stay deterministic.  NULL (the default)
 * or fewer bytes: no workspace is used.  The memory stays the caller's and
 * must outlive the calls; GEMMs that may overlap on the device (different
 * streams or threads) must not share it.  The reference's counterpart is
 * the per-thread pack buffer of its sgemm (blas.c:477-505). */
#define PK_GPU_SPLIT_WORKSPACE_BYTES 33554432
int pk_gpu_set_workspace(void *dwork, size_t bytes);
/* Segments of K over workgroups that a split-kernel GEMM of this shape and
 * weight format (bits 4, 8 or 32) takes with this thread's workspace (1: K
 * is not split over workgroups). */
int pk_gpu_split_k_segments(int M, int N, int K, int bits);
/* Debug: the weights the GEMM kernels multiply, written to dout [K][N] on
 * `stream` through the kernels' own weight loads and conversions: int8
 * (bits 8) fl(q * scale), int4 (bits 4) fl(q * dscales[k][n/32]) with the
 * portable nibble decode, fp32 (bits 32) the weight.  unit_path 1 converts
 * whole units (4 int8, 8 int4 or 4 fp32 columns; N a multiple of them), the
 * kernels' path when rows allow vector loads; 0 one element at a time.  For
 * tests that compare the decode with memcmp.  No counterpart in the
 * reference. */
int pk_gpu_dequant_dev(int bits, int K, int N, const void *dB, int ldb, float scale,
                       const float *dscales, int unit_path, float *dout, void *stream);
/* Force the small-M tile for later calls on this thread: rb 16-row blocks
 * (1..4) and nct 16-column tiles (1..2, rb * nct <= 4; fp32 takes nct = 1,
 * rb <= 3) per workgroup; (0, 0) = the modelled choice.  A tuning and test
 * hook with no counterpart in the reference.  Returns PK_GPU_EINVAL for
 * other values. */
int pk_gpu_force_small_tile(int rb, int nct);
/* ---- panels: weights repacked for the small-M kernels ------------------
 * No counterpart in the reference (its weights stay in their on-disk
 * layout, weights.c:240-266).  A panel is a copy of one weight re-laid out
 * once in the matrix cores' operand order (int8 / int4 codes, int4 scales
 * transposed to [N/32][K], fp32 weights as bf16 hi and lo halves), which the
 * small-M kernels (M <= 64, PK_GPU_NUMERICS_DEFAULT or _FAST) read instead
 * of the [K][ldb] weight: same products, same tolerance, faster.  A
 * host-pointer GEMM makes the panel of a registered weight (and, for int4,
 * registered scales) on its first small-M use; device callers ask for one
 * here.  Panels cost panel bytes of device memory: int8 about K*N, int4
 * K*N/2 + K*N/8, fp32 4*K*N. */

/* Make the panel of device weight dB (bits 4, 8 or 32; K a multiple of 32;
 * int4: N a multiple of 32 and its scales dscales [K][N/32]) for later
 * *_dev / *_ex_dev GEMMs whose B is dB with the same bits, K, N, ldb (and
 * dscales).  Runs on `stream` and waits for it; not during stream capture.
 * Idempotent for the same parameters; PK_GPU_EINVAL if dB already has a
 * panel of another shape.  The weight's bytes must not change afterwards. */
int pk_gpu_pack_weight_dev(int bits, int K, int N, const void *dB, int ldb,
                           const float *dscales, void *stream);
/* Free the panel made for dB by pk_gpu_pack_weight_dev (after the device's
 * queued work); PK_GPU_EBUSY while a host-pointer call reads it. */
int pk_gpu_unpack_weight_dev(const void *dB);
/* Device bytes held by panels. */
size_t pk_gpu_panel_bytes(void);
/* Make the pre-split copy of device weight dB (bits 4, 8 or 32; K and N
 * multiples of 32; int4: its scales dscales [K][N/32]) for later
 * PK_GPU_NUMERICS_FAST *_dev / *_ex_dev GEMMs with M > 64 whose B is dB with
 * the same bits, K, N, ldb (and dscales): the weights the split kernels
 * multiply (int4: fl(q * s), blas.c:834-840), each already split into its
 * bf16 hi and lo halves (int8: the codes as bf16, exact) in the kernels'
 * chunk order, so those GEMMs stage them with plain copies instead of
 * decoding and splitting every weight per row tile.  The results are the
 * same bits.  4*K*N bytes of device memory (int4: 8 times the packed
 * weight; int8: 2*K*N, twice the codes).  Runs on `stream` and waits for it; not
 * during stream capture.  Idempotent for the same parameters; PK_GPU_EINVAL
 * if dB already has a copy of another shape.  The weight's bytes must not
 * change afterwards.  No counterpart in the reference. */
int pk_gpu_presplit_weight_dev(int bits, int K, int N, const void *dB, int ldb,
                               const float *dscales, void *stream);
/* Free the copy made for dB by pk_gpu_presplit_weight_dev (after the
 * device's queued work; no call may be using it). */
int pk_gpu_unsplit_weight_dev(const void *dB);
/* Device bytes held by pre-split copies. */
size_t pk_gpu_presplit_bytes(void);
/* Whether a GEMM on this thread with this shape, format and weight (and, for
 * int4, scales) would take the panel kernels, given aligned A rows. */
int pk_gpu_uses_panel(int M, int N, int K, int bits, const void *dB, int ldb,
                      const float *dscales);
/* Segments of K over workgroups that a panel GEMM of this shape takes with
 * this thread's workspace (pk_gpu_set_workspace): one per LDS phase when K
 * takes at least 4 phases (fewer phases run one after the other in one
 * launch), or one per half phase of 512 k where that fills more CUs.  Above
 * one, each workgroup stores its partial tile there and a second launch sums
 * them in segment order before alpha, beta, bias and the epilogue
 * (deterministic). */
int pk_gpu_panel_segments(int M, int N, int K);
/* Test hook: the weights as the panel kernels multiply them, to dout [K][N]
 * on `stream`: int8 fl(q * B_scale), int4 fl(q * s[k][n/32]), fp32 hi + lo. */
int pk_gpu_panel_decode_dev(int bits, int K, int N, const void *dB, int ldb,
                            const float *dscales, float B_scale, float *dout, void *stream);
/* Tuning and test hook: the panel workgroup tile for later calls on this
 * thread, mb 16-row blocks (1..4; more rows than mb * 16 go to more
 * workgroups) and nct 16-column tiles (1..2); (0, 0) = the default choice. */
int pk_gpu_force_panel_tile(int mb, int nct);

/* Force a configuration for later calls on this thread (-1 = automatic),
 * encoder runs included: an encoder keeps its captured graphs per forced
 * configuration, so a change takes effect on the next run. */
int pk_gpu_force_config(int index);

#ifdef __cplusplus
}
#endif
#endif /* PK_GPU_H */
