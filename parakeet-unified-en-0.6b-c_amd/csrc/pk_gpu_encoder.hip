// pk_gpu_encoder.hip - host side of the device-resident conformer encoder and
// of the block-operation entry points (include/pk_gpu.h).
//
// The reference runs each conformer block as host loops around its BLAS
// (encoder.c:179-491) and the chunks of a long input one after another
// (encoder.c:514-575).  Here the whole block stays on the device, every
// weight GEMM carries its bias / Swish / residual in its output store, and
// all chunks run as one batch of rows: row-independent work (LayerNorm,
// the weight GEMMs, GLU) sees M = sum of the chunks' rows, while attention
// and the depthwise convolution run per chunk, one launch per distinct chunk
// length.  The position projection (linear_pos of the positional slice)
// runs once per block for the longest chunk: the slice of a chunk of T rows
// is pe_table[center-T+1, center+T) (encoder.c:220-228), a row range of the
// longest chunk's slice, and GEMM rows are independent, so a shorter chunk
// reads its P rows from the same result.
#include "pk_block_kernels.h"
#include "pk_gemm_kernels.h"
#include "pk_gpu.h"
#include "pk_gpu_internal.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <map>
#include <tuple>
#include <vector>

using pkgpu::Epilogue;
using pkgpu::GemmProblem;
using pkgpu::WeightKind;

namespace {

constexpr int kD = 1024;          // PK_D_MODEL
constexpr int kFF = 4096;         // PK_FF_DIM
constexpr int kHeads = 8;         // PK_N_HEADS
constexpr int kConvK = 9;         // PK_CONV_KERNEL
constexpr size_t kMaxGraphs = 64; // captured block graphs kept per encoder

struct DevWeight {
    WeightKind kind = pkgpu::W_F32;
    const void* data = nullptr;
    float scale = 0.0f;
    const float* scales = nullptr;
    int K = 0, N = 0;
    // its panel copy for the small-M kernels (pk_panel.hip), made on the
    // first run with a row group of at most 64 rows outside exact numerics
    const void* panel = nullptr;
    // int4 and fp32: its pre-split copy for the split kernels (pk_split.hip),
    // made on the first fast-numerics run with a row group of more than 64 rows
    const void* split = nullptr;
};

struct DevBlock {
    const float *ln_ff1_w, *ln_ff1_b, *ln_sa_w, *ln_sa_b, *ln_conv_w, *ln_conv_b;
    const float *ln_ff2_w, *ln_ff2_b, *ln_out_w, *ln_out_b;
    DevWeight ff1_w1, ff1_w2, ff2_w1, ff2_w2, qkv, pos, out, pw1t, pw2t;
    const float *ff1_b1, *ff1_b2, *ff2_b1, *ff2_b2, *qkv_b, *out_b, *pu, *pv;
    const float *pw1_b, *dw_w, *dw_b, *pw2_b;
    // linear_pos(pe_slice(p_T)) [2 p_T - 1][kD], computed once at creation: a
    // chunk of T <= p_T rows reads its rows [p_T - T, p_T + T - 1)
    const float* P = nullptr;
};

struct Chunk {
    int in_start, in_len, out_start, out_len, left_ov, row;   // row: first row in the batch
};

// Whole chunks occupying batch rows [r0, r0 + R), run as one unit: its
// chunks are entries [tab, tab + n) of the device chunk table, with rows
// relative to r0, ordered by length; by_len maps a length to (first entry,
// count).  Every workspace buffer is partitioned by rows, so groups do not
// share memory and may run concurrently.
struct RowGroup {
    int r0 = 0, R = 0, Tmax = 0, tab = 0, n = 0;
    std::map<int, std::pair<int, int>> by_len;
    size_t scores_off = 0;      // its attention's score rows (Tmax > kAttnMaxT) in e->scores
    float* part = nullptr;      // its split-K partial tiles (fast numerics), or null
};

constexpr int kMels = 128;        // PK_N_MELS
constexpr int kSub = 256;         // PK_SUB_CHANNELS

struct DevPreEncode {
    bool set = false;
    const float *w0, *b0, *w2, *b2, *b3, *w5, *b5, *b6, *out_b;
    DevWeight w3t, w6t, out;
    std::vector<void*> allocs;
};

// Output size of a 3x3 stride-2 pad-1 stage (encoder.c:116, 125, 137).
inline int half_up(int n) { return (n + 2 - 3) / 2 + 1; }

// One profiled launch: events on its stream and its algorithmic work.
struct ProfRec {
    int stage;
    hipEvent_t a, b;
    double flops, bytes;
};

}  // namespace

struct pk_gpu_encoder {
    std::vector<DevBlock> blocks;
    std::vector<void*> allocs;          // weights, tables
    size_t weight_bytes = 0;
    const float* pe = nullptr;          // [pe_rows][kD]
    int pe_rows = 0, pe_center = 0;
    int p_T = 0;                        // longest chunk the blocks' projections cover
    std::vector<void*> pos_allocs;      // the blocks' projections (replaced when p_T grows)
    hipStream_t stream = nullptr;
    // workspace, grown on demand
    size_t ws_rows = 0;
    float *x = nullptr, *ln = nullptr, *h = nullptr, *att = nullptr;
    int* rows_tab = nullptr;            // device: chunk rows [rows_cap], then chunk lengths [rows_cap]
    float* scores = nullptr;            // attention score rows of sequences beyond kAttnMaxT
    size_t scores_n = 0;                // floats
    size_t rows_cap = 0;
    std::vector<int> tab_host;          // what rows_tab was last given (kept alive for the copy)
    size_t ws_bytes = 0;
    // per-stage timing (pk_gpu_encoder_profile)
    bool prof = false;
    std::vector<ProfRec> pending;
    std::vector<hipEvent_t> event_pool;
    double ms[PK_GPU_N_STAGES] = {}, flops[PK_GPU_N_STAGES] = {}, bytes[PK_GPU_N_STAGES] = {};
    long long launches[PK_GPU_N_STAGES] = {};
    // the 24 blocks' launches captured once per (T, chunk, overlap) and
    // replayed; their device pointers are the workspace's, so a workspace
    // change drops them
    // (T, chunk, overlap, group, forced tile config): a graph freezes the
    // tiles its GEMMs were launched with, so a pk_gpu_force_config in force
    // at capture is part of what the graph is
    // and the encoder's numerics (which kernels its GEMMs take)
    std::map<std::tuple<int, int, int, int, int, int>, hipGraphExec_t> graphs;
    int numerics = PK_GPU_NUMERICS_EXACT;     // pk_gpu_encoder_set_numerics
    // Row groups replayed concurrently: group 0 on the caller's stream, group
    // g > 0 on side[g - 1], joined through events around the replay.
    int n_groups = 2;
    int lag = -1;                  // pk_gpu_encoder_set_group_lag (-1: group_lag())
    // fast numerics: LayerNorms feeding a GEMM write pre-split output
    // (PK_GPU_PRESPLIT=0 at creation turns it off; the results are the same)
    bool presplit = true;
    // small row groups on the panel kernels: LayerNorms fused into the GEMMs;
    // fast numerics in larger row groups: LayerNorms formed by the split-K
    // reduces that finish their rows
    // (PK_GPU_FUSE_LN=0 at creation turns both off; the results are the same)
    bool fuse_ln = true;
    // fast numerics: the int4 and fp32 block weights' pre-split copies
    // (PK_GPU_PRESPLIT_W=0 at creation turns them off; the results are the same)
    bool presplit_w = true;
    // fast numerics: attention of row groups above 64 rows on split bf16
    // operands (PK_GPU_FAST_ATTN=0 at creation keeps the exact kernel)
    bool fast_attn = true;
    std::vector<hipStream_t> side;
    std::vector<hipEvent_t> side_done;
    hipEvent_t inputs_ready = nullptr;
    // Runs and pre-encodes share the workspace.  Each records last_done on
    // its stream when it is enqueued; a call on another stream waits for it
    // on the device first (follow_last), so calls on different streams never
    // overlap, and host-side waits on the current stream cover the previous
    // call too.
    hipEvent_t last_done = nullptr;
    hipStream_t last_stream = nullptr;
    // pre-encode: weights and two ping-pong buffers, grown on demand
    DevPreEncode pre;
    float *pre_a = nullptr, *pre_b = nullptr, *pre_x = nullptr;
    size_t pre_a_n = 0, pre_b_n = 0, pre_x_n = 0;
    // fast numerics: kSplitWorkBytes of split-K partial tiles per row group
    // (groups replay concurrently, so each has its own), grown on demand
    float* part = nullptr;
    size_t part_groups = 0;
    // the block weights' panels (made once, see DevWeight::panel)
    std::vector<void*> panel_allocs;
    size_t panel_bytes = 0;
    // the block weights' pre-split copies (made once, see DevWeight::split)
    std::vector<void*> split_allocs;
    size_t split_bytes = 0;
};

namespace {

using pkgpu::rt::error;
using pkgpu::rt::hip_error;

int dev_alloc(pk_gpu_encoder* e, size_t bytes, void** out)
{
    *out = nullptr;
    hipError_t r = hipMalloc(out, bytes ? bytes : 4);
    if (r != hipSuccess) return error(PK_GPU_ENOMEM, "device allocation of %zu bytes failed", bytes);
    e->allocs.push_back(*out);
    e->weight_bytes += bytes;
    return PK_GPU_OK;
}

int upload(pk_gpu_encoder* e, const void* host, size_t bytes, const char* what, const void** out)
{
    if (!host) return error(PK_GPU_EINVAL, "%s is NULL", what);
    void* d = nullptr;
    int rc = dev_alloc(e, bytes, &d);
    if (rc) return rc;
    hipError_t r = hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, e->stream);
    if (r != hipSuccess) return hip_error(r, what);
    *out = d;
    return PK_GPU_OK;
}

int upload_f(pk_gpu_encoder* e, const float* host, size_t n, const char* what, const float** out)
{
    const void* d = nullptr;
    int rc = upload(e, host, n * sizeof(float), what, &d);
    *out = static_cast<const float*>(d);
    return rc;
}

int upload_weight(pk_gpu_encoder* e, const pk_gpu_weight& w, int K, int N, const char* what,
                  DevWeight* out)
{
    out->K = K;
    out->N = N;
    out->scale = w.scale;
    switch (w.bits) {
    case 32:
        out->kind = pkgpu::W_F32;
        return upload(e, w.data, (size_t)K * N * 4, what, &out->data);
    case 8:
        out->kind = pkgpu::W_I8;
        return upload(e, w.data, (size_t)K * N, what, &out->data);
    case 4: {
        out->kind = pkgpu::W_I4;
        int rc = upload(e, w.data, (size_t)K * N / 2, what, &out->data);
        if (rc) return rc;
        return upload_f(e, w.scales, (size_t)K * (N / 32), what, &out->scales);
    }
    default:
        return error(PK_GPU_EINVAL, "%s: bits = %d (expected 32, 8 or 4)", what, w.bits);
    }
}

// A pointwise-convolution weight [Cout][Cin] (the A operand of the
// reference's sgemm, tensor_ops.c:579-590) stored transposed, [Cin][Cout]:
// out^T[t][c] = sum_k ln[t][k] * W[c][k] is then an NN GEMM with the weight
// as B and the time-major activations as A, with the same fma chain per
// output (the two factors of each product just swap places).
int upload_pointwise(pk_gpu_encoder* e, const float* host, int Cout, int Cin, const char* what,
                     DevWeight* out)
{
    if (!host) return error(PK_GPU_EINVAL, "%s is NULL", what);
    const size_t bytes = (size_t)Cout * Cin * 4;
    void* t = nullptr;
    int rc = dev_alloc(e, bytes, &t);
    if (rc) return rc;
    void* tmp = nullptr;
    if (hipMalloc(&tmp, bytes) != hipSuccess) return error(PK_GPU_ENOMEM, "%s staging", what);
    hipError_t r = hipMemcpyAsync(tmp, host, bytes, hipMemcpyHostToDevice, e->stream);
    if (r == hipSuccess)
        r = pkgpu::launch_transpose(static_cast<const float*>(tmp), static_cast<float*>(t), Cout, Cin,
                                    e->stream);
    if (r == hipSuccess) r = hipStreamSynchronize(e->stream);
    (void)hipFree(tmp);
    if (r != hipSuccess) return hip_error(r, what);
    out->kind = pkgpu::W_F32;
    out->data = t;
    out->K = Cin;
    out->N = Cout;
    return PK_GPU_OK;
}

int upload_block(pk_gpu_encoder* e, const pk_gpu_block_weights& b, DevBlock* d)
{
    int rc = 0;
#define UP(field, src, n) if (!rc) rc = upload_f(e, b.src, (n), #src, &d->field)
    UP(ln_ff1_w, norm_ff1_w, kD); UP(ln_ff1_b, norm_ff1_b, kD);
    UP(ln_sa_w, norm_sa_w, kD);   UP(ln_sa_b, norm_sa_b, kD);
    UP(ln_conv_w, norm_conv_w, kD); UP(ln_conv_b, norm_conv_b, kD);
    UP(ln_ff2_w, norm_ff2_w, kD); UP(ln_ff2_b, norm_ff2_b, kD);
    UP(ln_out_w, norm_out_w, kD); UP(ln_out_b, norm_out_b, kD);
    UP(ff1_b1, ff1_linear1_b, kFF); UP(ff1_b2, ff1_linear2_b, kD);
    UP(ff2_b1, ff2_linear1_b, kFF); UP(ff2_b2, ff2_linear2_b, kD);
    UP(qkv_b, linear_qkv_b, 3 * kD); UP(out_b, linear_out_b, kD);
    UP(pu, pos_bias_u, kD); UP(pv, pos_bias_v, kD);
    UP(pw1_b, conv_pw1_b, 2 * kD); UP(pw2_b, conv_pw2_b, kD);
    UP(dw_w, conv_dw_w, kD * kConvK); UP(dw_b, conv_dw_b, kD);
#undef UP
    if (!rc) rc = upload_weight(e, b.ff1_linear1_w, kD, kFF, "ff1.linear1", &d->ff1_w1);
    if (!rc) rc = upload_weight(e, b.ff1_linear2_w, kFF, kD, "ff1.linear2", &d->ff1_w2);
    if (!rc) rc = upload_weight(e, b.ff2_linear1_w, kD, kFF, "ff2.linear1", &d->ff2_w1);
    if (!rc) rc = upload_weight(e, b.ff2_linear2_w, kFF, kD, "ff2.linear2", &d->ff2_w2);
    if (!rc) rc = upload_weight(e, b.linear_qkv_w, kD, 3 * kD, "linear_qkv", &d->qkv);
    if (!rc) rc = upload_weight(e, b.linear_pos_w, kD, kD, "linear_pos", &d->pos);
    if (!rc) rc = upload_weight(e, b.linear_out_w, kD, kD, "linear_out", &d->out);
    if (!rc) rc = upload_pointwise(e, b.conv_pw1_w, 2 * kD, kD, "conv.pw1", &d->pw1t);
    if (!rc) rc = upload_pointwise(e, b.conv_pw2_w, kD, kD, "conv.pw2", &d->pw2t);
    return rc;
}

void drop_graphs(pk_gpu_encoder* e)
{
    for (auto& g : e->graphs) (void)hipGraphExecDestroy(g.second);
    e->graphs.clear();
}

void free_workspace(pk_gpu_encoder* e)
{
    drop_graphs(e);
    for (float* p : {e->x, e->ln, e->h, e->att})
        if (p) (void)hipFree(p);
    if (e->rows_tab) (void)hipFree(e->rows_tab);
    if (e->scores) (void)hipFree(e->scores);
    e->x = e->ln = e->h = e->att = nullptr;
    e->rows_tab = nullptr;
    e->scores = nullptr;
    e->scores_n = 0;
    e->tab_host.clear();
    e->ws_rows = e->rows_cap = e->ws_bytes = 0;
}

// Grows the workspace; the old one may still be read by work queued on `s`
// (which already waits for the previous call, whatever its stream).
int workspace(pk_gpu_encoder* e, size_t rows, size_t n_chunks, size_t scores_n, hipStream_t s)
{
    if (rows <= e->ws_rows && n_chunks <= e->rows_cap && scores_n <= e->scores_n) return PK_GPU_OK;
    hipError_t r = hipStreamSynchronize(s);
    if (r != hipSuccess) return hip_error(r, "encoder stream");
    rows = std::max(rows, e->ws_rows);
    n_chunks = std::max(n_chunks, e->rows_cap);
    scores_n = std::max(scores_n, e->scores_n);
    free_workspace(e);
    const size_t bytes[4] = {rows * kD * 4, rows * kD * 4, rows * kFF * 4, rows * kD * 4};
    float** dst[4] = {&e->x, &e->ln, &e->h, &e->att};
    for (int i = 0; i < 4; ++i) {
        if (hipMalloc(reinterpret_cast<void**>(dst[i]), bytes[i]) != hipSuccess) {
            free_workspace(e);
            return error(PK_GPU_ENOMEM, "encoder workspace of %zu bytes failed", bytes[i]);
        }
        e->ws_bytes += bytes[i];
    }
    if (hipMalloc(reinterpret_cast<void**>(&e->rows_tab), 2 * n_chunks * sizeof(int)) != hipSuccess) {
        free_workspace(e);
        return error(PK_GPU_ENOMEM, "encoder chunk table failed");
    }
    if (scores_n) {
        if (hipMalloc(reinterpret_cast<void**>(&e->scores), scores_n * sizeof(float)) != hipSuccess) {
            free_workspace(e);
            return error(PK_GPU_ENOMEM, "attention score workspace of %zu bytes failed",
                         scores_n * sizeof(float));
        }
        e->ws_bytes += scores_n * sizeof(float);
        e->scores_n = scores_n;
    }
    e->ws_rows = rows;
    e->rows_cap = n_chunks;
    return PK_GPU_OK;
}

// LayerNorms fused into a small-M GEMM (panel kernels only): `in` normalises
// its input rows, `out` its output rows after the epilogue.
struct FusedLn {
    const float *in_g = nullptr, *in_b = nullptr, *out_g = nullptr, *out_b = nullptr;
    // the split-K reduce's LayerNorm of its rows into next_out, pre-split
    const float *next_g = nullptr, *next_b = nullptr;
    float* next_out = nullptr;
};

// The GEMM problem of a block weight; presplit: A holds a split-output
// LayerNorm's rows (GemmProblem::a_presplit), for the split kernels only.
GemmProblem block_problem(const DevWeight& w, const float* A, int M, float* C, const float* bias,
                          Epilogue epi, pkgpu::Tolerance tol, float* work, bool presplit,
                          const FusedLn& ln)
{
    GemmProblem p{};
    p.kind = w.kind;
    p.M = M;
    p.N = w.N;
    p.K = w.K;
    p.alpha = 1.0f;
    p.beta = 0.0f;
    p.A = A;
    p.lda = w.K;
    p.B = w.data;
    p.ldb = w.kind == pkgpu::W_I4 ? w.N / 2 : w.N;
    p.scale = w.scale;
    p.scales = w.scales;
    p.C = C;
    p.ldc = w.N;
    p.bias = bias;
    p.epi = epi;
    if (work) {
        p.work = work;
        p.work_bytes = pkgpu::kSplitWorkBytes;
    }
    p.a_presplit = presplit;
    if (tol != pkgpu::TOL_NONE) p.panel = w.panel;      // read only where the small-M path may run
    if (tol == pkgpu::TOL_ALL) p.b_presplit = w.split;  // read only by the split kernels
    p.ln_gamma = ln.in_g;
    p.ln_beta = ln.in_b;
    p.out_ln_gamma = ln.out_g;
    p.out_ln_beta = ln.out_b;
    p.next_ln_gamma = ln.next_g;
    p.next_ln_beta = ln.next_b;
    p.next_ln_out = ln.next_out;
    return p;
}

int gemm_launch(const DevWeight& w, const float* A, int M, float* C, const float* bias,
                Epilogue epi, hipStream_t s, pkgpu::Tolerance tol = pkgpu::TOL_NONE,
                float* work = nullptr, bool presplit = false, const FusedLn& ln = FusedLn())
{
    return pkgpu::rt::gemm(block_problem(w, A, M, C, bias, epi, tol, work, presplit, ln), s, tol);
}

int check(hipError_t r, const char* what) { return r == hipSuccess ? PK_GPU_OK : hip_error(r, what); }

// Order a call on `s` after the previous call of this encoder (see last_done).
int follow_last(pk_gpu_encoder* e, hipStream_t s)
{
    if (!e->last_done || e->last_stream == s) return PK_GPU_OK;
    return check(hipStreamWaitEvent(s, e->last_done, 0), "encoder event");
}

int mark_last(pk_gpu_encoder* e, hipStream_t s)
{
    if (!e->last_done) {
        const hipError_t r = hipEventCreateWithFlags(&e->last_done, hipEventDisableTiming);
        if (r != hipSuccess) return hip_error(r, "hipEventCreate");
    }
    e->last_stream = s;
    return check(hipEventRecord(e->last_done, s), "encoder event");
}

// Host wait for every queued call of this encoder, whatever its stream.
void wait_all(pk_gpu_encoder* e)
{
    if (e->stream) (void)hipStreamSynchronize(e->stream);
    for (hipStream_t st : e->side) (void)hipStreamSynchronize(st);
    if (e->last_done) (void)hipEventSynchronize(e->last_done);
}

hipEvent_t take_event(pk_gpu_encoder* e)
{
    if (!e->event_pool.empty()) {
        hipEvent_t ev = e->event_pool.back();
        e->event_pool.pop_back();
        return ev;
    }
    hipEvent_t ev = nullptr;
    return hipEventCreate(&ev) == hipSuccess ? ev : nullptr;
}

// Run launch(), bracketed by events on s when profiling is on.
template <class F>
int timed(pk_gpu_encoder* e, int stage, double flops, double bytes, hipStream_t s, F&& launch)
{
    if (!e->prof) return launch();
    hipEvent_t a = take_event(e), b = take_event(e);
    int rc = (a && b) ? check(hipEventRecord(a, s), "profiling event")
                      : error(PK_GPU_EHIP, "profiling events");
    if (!rc) rc = launch();
    if (!rc) rc = check(hipEventRecord(b, s), "profiling event");
    if (rc) {                                   // the pair is not pending: back to the pool
        if (a) e->event_pool.push_back(a);
        if (b) e->event_pool.push_back(b);
        return rc;
    }
    e->pending.push_back({stage, a, b, flops, bytes});
    return PK_GPU_OK;
}

// Fold finished events into the totals.
int collect(pk_gpu_encoder* e)
{
    for (const ProfRec& r : e->pending) {
        hipError_t err = hipEventSynchronize(r.b);
        if (err != hipSuccess) return hip_error(err, "profiling");
        float ms = 0.0f;
        (void)hipEventElapsedTime(&ms, r.a, r.b);
        e->ms[r.stage] += ms;
        e->flops[r.stage] += r.flops;
        e->bytes[r.stage] += r.bytes;
        e->launches[r.stage] += 1;
        e->event_pool.push_back(r.a);
        e->event_pool.push_back(r.b);
    }
    e->pending.clear();
    return PK_GPU_OK;
}

double weight_bytes_of(const DevWeight& w)
{
    switch (w.kind) {
    case pkgpu::W_I4: return 0.5 * w.K * w.N + 4.0 * w.K * (w.N / 32);
    case pkgpu::W_I8: return 1.0 * w.K * w.N + 4.0;
    default: return 4.0 * w.K * w.N;
    }
}

int stage_of(const DevWeight& w)
{
    return w.kind == pkgpu::W_I4 ? PK_GPU_STAGE_GEMM_I4
         : w.kind == pkgpu::W_I8 ? PK_GPU_STAGE_GEMM_I8 : PK_GPU_STAGE_GEMM_F32;
}

// encoder.c:514-575: output frames [c*C, c*C + C), input with `ov` frames of
// context each side, clipped to [0, T).  chunk_size <= 0: one sequence.
std::vector<Chunk> plan_chunks(int T, int C, int ov)
{
    std::vector<Chunk> v;
    if (C <= 0) {
        v.push_back({0, T, 0, T, 0, 0});
        return v;
    }
    const int n = (T + C - 1) / C;
    int row = 0;
    for (int ci = 0; ci < n; ++ci) {
        const int out_start = ci * C, out_end = std::min(out_start + C, T);
        const int in_start = std::max(out_start - ov, 0), in_end = std::min(out_end + ov, T);
        v.push_back({in_start, in_end - in_start, out_start, out_end - out_start,
                     out_start - in_start, row});
        row += in_end - in_start;
    }
    return v;
}

// A weight GEMM of the block: M rows of A through w, with its epilogue;
// `work`: the row group's split-K partial tiles, or null; `presplit`: A holds
// a split-output LayerNorm's rows (layer_norm with split); `exact`: the
// exact chains whatever the encoder's numerics; `ln`: LayerNorms fused into
// it (fusable() said the panel kernels take them).
int gemm(pk_gpu_encoder* e, const DevWeight& w, const float* A, int M, float* C,
         const float* bias, Epilogue epi, hipStream_t s, float* work = nullptr,
         bool presplit = false, bool exact = false, const FusedLn& ln = FusedLn())
{
    const double flops = 2.0 * M * w.N * w.K;
    double bytes = weight_bytes_of(w) + 4.0 * M * w.K + 4.0 * M * w.N;
    if (bias) bytes += 4.0 * w.N;
    if (epi == pkgpu::EPI_HALF_RESIDUAL || epi == pkgpu::EPI_RESIDUAL) bytes += 4.0 * M * w.N;
    if (ln.in_g) bytes += 8.0 * w.K;
    if (ln.out_g) bytes += 8.0 * w.N;
    if (ln.next_g) bytes += 8.0 * w.N + 4.0 * M * w.N;
    const pkgpu::Tolerance tol = exact ? pkgpu::TOL_NONE : pkgpu::rt::tolerance_of(e->numerics);
    return timed(e, stage_of(w), flops, bytes, s,
                 [&] {
                     return gemm_launch(w, A, M, C, bias, epi, s, tol, work, presplit, ln);
                 });
}

// Whether the panel kernels take this block GEMM with these LayerNorms
// fused (the encoder's numerics allow the small-M path, no forced tile, the
// weight has its panel, and the shape and LDS allow it).
bool fusable(pk_gpu_encoder* e, const DevWeight& w, const float* A, int M, float* C, const float* bias,
             Epilogue epi, float* work, const FusedLn& ln)
{
    if (!e->fuse_ln || e->numerics == PK_GPU_NUMERICS_EXACT || pkgpu::rt::forced_config() >= 0 || !w.panel)
        return false;
    const GemmProblem p = block_problem(w, A, M, C, bias, epi, pkgpu::rt::tolerance_of(e->numerics), work,
                                        false, ln);
    return ln.out_g ? pkgpu::panel_fuses_out_ln(p) : pkgpu::panel_supports(p);
}

// Whether the split kernels form these LayerNorms (ln.out_g, ln.next_g)
// in this block GEMM's split-K reduce (fused LayerNorms on, fast numerics,
// no forced tile).
bool split_fusable(pk_gpu_encoder* e, const DevWeight& w, const float* A, int M, float* C, const float* bias,
                   Epilogue epi, float* work, const FusedLn& ln)
{
    if (!e->fuse_ln || e->numerics != PK_GPU_NUMERICS_FAST || pkgpu::rt::forced_config() >= 0) return false;
    return pkgpu::split_fuses_ln(block_problem(w, A, M, C, bias, epi, pkgpu::TOL_ALL, work, false, ln));
}

// split: the output pre-split for the split GEMM kernels, for a GEMM that
// then reads it with presplit.
int layer_norm(pk_gpu_encoder* e, const float* x, const float* g, const float* b, float* out, int R,
               hipStream_t s, bool split = false)
{
    return timed(e, PK_GPU_STAGE_LAYER_NORM, 0.0, 8.0 * R * kD + 8.0 * kD, s, [&] {
        if (split)
            return check(pkgpu::launch_layer_norm_split(x, kD, g, b, out, kD, R, kD, s), "layer norm");
        return check(pkgpu::launch_layer_norm(x, kD, g, b, out, kD, R, kD, s), "layer norm");
    });
}

// One conformer block (encoder.c:479-491) over one row group.
// Modules [from, to) of one block: 0 feed-forward 1, 1 self-attention,
// 2 convolution, 3 feed-forward 2 and the output LayerNorm.
int run_block(pk_gpu_encoder* e, const DevBlock& b, const RowGroup& g, hipStream_t s,
              int from = 0, int to = 4)
{
    const int R = g.R, Tmax = g.Tmax;
    // h holds [R][4096], [R][3072] or [R][2048] rows: a group's part is sized
    // for the widest
    float* x = e->x + (size_t)g.r0 * kD;
    float* ln = e->ln + (size_t)g.r0 * kD;
    float* h = e->h + (size_t)g.r0 * kFF;
    float* att = e->att + (size_t)g.r0 * kD;
    const int* rows = e->rows_tab + g.tab;
    const int* lens = e->rows_tab + e->rows_cap + g.tab;
    // Fast numerics beyond the small-M rows: the LayerNorms that feed a GEMM
    // (feed-forward up, QKV, pointwise 1) write their outputs pre-split, so
    // those GEMMs stage A without splitting it again per column tile (fast
    // pass +0.8-1.8%).  The GEMMs' inputs, and so every result, are the same
    // bits.  The up projection's Swish output pre-split for the down
    // projection measured no faster: its scattered 2-byte stores cost what
    // the down projection saved.
    const bool ps = e->presplit && e->numerics == PK_GPU_NUMERICS_FAST &&
                    pkgpu::rt::forced_config() < 0 && R > 64;
    // Small row groups on the panel kernels: each LayerNorm that feeds a GEMM
    // is fused into that GEMM (its rows normalised as they are staged), and
    // the block's output LayerNorm into the second feed-forward's split-K
    // reduce; the results are the same bits as the separate launches give
    // those kernels.
    auto fused_in = [&](const DevWeight& w, const float* gm, const float* be, float* C, const float* bias,
                        Epilogue epi) {
        FusedLn f;
        f.in_g = gm;
        f.in_b = be;
        return fusable(e, w, x, R, C, bias, epi, g.part, f) ? f : FusedLn();
    };
    // The LayerNorms that a GEMM writing x forms in its split-K reduce:
    // `want` if the split kernels take them (pre-split row groups), else its
    // output LayerNorm alone if the panel kernels take that, else none.  Each
    // consumer asks the same question of its producer, so both agree.
    enum XWriter { FF1_DOWN, PW2, FF2_DOWN };
    auto reduce_ln = [&](const DevBlock& bb, XWriter which, const DevBlock* next_block) {
        FusedLn want;
        const DevWeight* w = nullptr;
        const float *A = h, *bias = nullptr;
        Epilogue epi = pkgpu::EPI_HALF_RESIDUAL;
        switch (which) {
        case FF1_DOWN:          // x after feed-forward 1: self-attention's input
            w = &bb.ff1_w2;
            bias = bb.ff1_b2;
            want.next_g = bb.ln_sa_w;
            want.next_b = bb.ln_sa_b;
            break;
        case PW2:               // after the convolution: feed-forward 2's input
            w = &bb.pw2t;
            A = ln;
            bias = bb.pw2_b;
            epi = pkgpu::EPI_RESIDUAL;
            want.next_g = bb.ln_ff2_w;
            want.next_b = bb.ln_ff2_b;
            break;
        case FF2_DOWN:          // the block's output, and the next block's input
            w = &bb.ff2_w2;
            bias = bb.ff2_b2;
            want.out_g = bb.ln_out_w;
            want.out_b = bb.ln_out_b;
            if (next_block) {
                want.next_g = next_block->ln_ff1_w;
                want.next_b = next_block->ln_ff1_b;
            }
            break;
        }
        if (want.next_g) want.next_out = ln;
        if (ps && split_fusable(e, *w, A, R, x, bias, epi, g.part, want)) return want;
        FusedLn o;
        o.out_g = want.out_g;
        o.out_b = want.out_b;
        if (o.out_g && fusable(e, *w, A, R, x, bias, epi, g.part, o)) return o;
        return FusedLn();
    };
    const size_t bi = (size_t)(&b - e->blocks.data());
    const DevBlock* next = bi + 1 < e->blocks.size() ? &e->blocks[bi + 1] : nullptr;
    const FusedLn ff1_o = reduce_ln(b, FF1_DOWN, nullptr);
    const FusedLn pw2_o = reduce_ln(b, PW2, nullptr);
    const FusedLn ff2_o = reduce_ln(b, FF2_DOWN, next);
    // whether the previous block's last reduce wrote this block's first input
    const bool ff1_ready = bi > 0 && reduce_ln(e->blocks[bi - 1], FF2_DOWN, &b).next_g != nullptr;
    // the normalised input of a GEMM: fused into it, already in `ln` (ready:
    // the reduce before wrote it), or a LayerNorm launch into `ln`
    auto norm_in = [&](const FusedLn& f, const float* gm, const float* be, const float** A, bool ready) {
        *A = f.in_g ? x : ln;
        return f.in_g || ready ? PK_GPU_OK : layer_norm(e, x, gm, be, ln, R, s, ps);
    };
    // o: the LayerNorms the down projection's reduce forms
    auto ffn = [&](const float* gm, const float* be, const DevWeight& w1, const float* b1,
                   const DevWeight& w2, const float* b2, bool ready, const FusedLn& o) {
        const FusedLn f = fused_in(w1, gm, be, h, b1, pkgpu::EPI_SWISH);
        const float* A = nullptr;
        int r = norm_in(f, gm, be, &A, ready);
        if (!r) r = gemm(e, w1, A, R, h, b1, pkgpu::EPI_SWISH, s, g.part, ps && !f.in_g, false, f);   // encoder.c:193-196
        if (!r) r = gemm(e, w2, h, R, x, b2, pkgpu::EPI_HALF_RESIDUAL, s, g.part, false, false, o);   // encoder.c:198-216
        return r;
    };
    // self-attention (encoder.c:300-424)
    auto self_attention = [&]() {
        const FusedLn f = fused_in(b.qkv, b.ln_sa_w, b.ln_sa_b, h, b.qkv_b, pkgpu::EPI_NONE);
        const float* A = nullptr;
        int rc = norm_in(f, b.ln_sa_w, b.ln_sa_b, &A, ff1_o.next_g != nullptr);
        if (!rc) rc = gemm(e, b.qkv, A, R, h, b.qkv_b, pkgpu::EPI_NONE, s, g.part, ps && !f.in_g, false, f);
        if (rc) return rc;
        // every chunk of the group in one launch, each with its own length
        double flops = 0.0, bytes = 4.0 * (2 * Tmax - 1) * kD;   // the P rows read
        for (const auto& l : g.by_len) {
            const double T = l.first, c = l.second.second;
            flops += 6.0 * T * T * kD * c;     // Q_u K^T, shifted Q_v P^T, scores x V
            bytes += (4.0 * T * 3 * kD + 4.0 * T * kD) * c;
        }
        pkgpu::AttnArgs a{};
        a.qkv = h; a.ldq = 3 * kD;
        a.P = b.P + (size_t)(e->p_T - Tmax) * kD; a.ldp = kD;
        a.pos_bias_u = b.pu; a.pos_bias_v = b.pv;
        a.out = att; a.ldo = kD;
        a.chunk_rows = rows;
        a.chunk_T = lens;
        a.T = Tmax; a.H = kHeads;
        a.scores = Tmax > pkgpu::kAttnMaxT ? e->scores + g.scores_off : nullptr;
        // Fast numerics: split bf16 operands, prepared in the row group's
        // split-K workspace, which nothing holds between the QKV GEMM (K is
        // not split for it) and the output projection.
        const size_t ws_floats = pkgpu::kSplitWorkBytes / sizeof(float);
        const bool fast = e->fast_attn && e->numerics == PK_GPU_NUMERICS_FAST && R > pkgpu::kSmallMaxM &&
                          Tmax > pkgpu::kAttnShortT && Tmax <= pkgpu::kAttnMaxT && g.part &&
                          pkgpu::attn_fast_ws_floats(Tmax, kHeads, g.n) <= ws_floats;
        rc = timed(e, PK_GPU_STAGE_ATTENTION, flops, bytes, s, [&] {
            return check(fast ? pkgpu::launch_attention_fast(a, g.n, g.part, ws_floats, s)
                              : pkgpu::launch_attention(a, g.n, s),
                         "attention");
        });
        if (!rc) rc = gemm(e, b.out, att, R, x, b.out_b, pkgpu::EPI_RESIDUAL, s, g.part);
        return rc;
    };
    // convolution module (encoder.c:430-476), time-major throughout
    auto convolution = [&]() {
        const FusedLn f = fused_in(b.pw1t, b.ln_conv_w, b.ln_conv_b, h, b.pw1_b, pkgpu::EPI_NONE);
        const float* A = nullptr;
        int rc = norm_in(f, b.ln_conv_w, b.ln_conv_b, &A, false);
        if (!rc) rc = gemm(e, b.pw1t, A, R, h, b.pw1_b, pkgpu::EPI_NONE, s, g.part, ps && !f.in_g, false, f);
        // The GLU is formed inside the depthwise convolution, as the kernel
        // stages its input window (each value gated once per workgroup, the
        // window's 8 extra times aside): one launch, and one write and read
        // of the gated rows, fewer.  The same bits (PK_GPU_FUSE_LN=0 keeps
        // the separate GLU launch).
        const bool glu_in_dw = e->fuse_ln;
        if (!rc && !glu_in_dw)
            rc = timed(e, PK_GPU_STAGE_CONV, 0.0, 12.0 * R * kD, s, [&] {
                return check(pkgpu::launch_glu(h, 2 * kD, att, kD, R, kD, s), "glu");
            });
        if (rc) return rc;
        // every chunk of the group in one launch, each with its own length
        pkgpu::DwArgs d{};
        d.x = glu_in_dw ? h : att;
        d.ldx = glu_in_dw ? 2 * kD : kD;
        d.glu = glu_in_dw ? 1 : 0;
        d.w = b.dw_w; d.b = b.dw_b;
        d.out = ln; d.ldo = kD;
        d.chunk_rows = rows;
        d.chunk_T = lens;
        d.T = Tmax; d.C = kD; d.K = kConvK; d.swish = 1;
        rc = timed(e, PK_GPU_STAGE_CONV, 0.0, (glu_in_dw ? 12.0 : 8.0) * R * kD, s, [&] {
            return check(pkgpu::launch_depthwise(d, g.n, s), "depthwise conv");
        });
        if (!rc) rc = gemm(e, b.pw2t, ln, R, x, b.pw2_b, pkgpu::EPI_RESIDUAL, s, g.part, false, false, pw2_o);
        return rc;
    };
    for (int m = from; m < to; ++m) {
        int rc = PK_GPU_OK;
        switch (m) {
        case 0:     // feed-forward 1 (encoder.c:483)
            rc = ffn(b.ln_ff1_w, b.ln_ff1_b, b.ff1_w1, b.ff1_b1, b.ff1_w2, b.ff1_b2, ff1_ready, ff1_o);
            break;
        case 1: rc = self_attention(); break;
        case 2: rc = convolution(); break;
        default:    // feed-forward 2 and the block's output LayerNorm (encoder.c:486-487)
            rc = ffn(b.ln_ff2_w, b.ln_ff2_b, b.ff2_w1, b.ff2_b1, b.ff2_w2, b.ff2_b2, pw2_o.next_g != nullptr,
                     ff2_o);
            if (!rc && !ff2_o.out_g) rc = layer_norm(e, x, b.ln_out_w, b.ln_out_b, x, R, s);
            break;
        }
        if (rc) return rc;
    }
    return PK_GPU_OK;
}

// At least n side streams and their completion events, plus the event that
// marks the inputs copied (created on first use, kept until destroy).
int side_streams(pk_gpu_encoder* e, int n)
{
    if (n > 0 && !e->inputs_ready) {
        hipError_t r = hipEventCreateWithFlags(&e->inputs_ready, hipEventDisableTiming);
        if (r != hipSuccess) return hip_error(r, "hipEventCreate");
    }
    while ((int)e->side.size() < n) {
        hipStream_t st = nullptr;
        hipEvent_t ev = nullptr;
        hipError_t r = hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
        if (r != hipSuccess) return hip_error(r, "hipStreamCreate");
        r = hipEventCreateWithFlags(&ev, hipEventDisableTiming);
        if (r != hipSuccess) {
            (void)hipStreamDestroy(st);
            return hip_error(r, "hipEventCreate");
        }
        e->side.push_back(st);
        e->side_done.push_back(ev);
    }
    return PK_GPU_OK;
}

// Consecutive chunks split into at most n groups of about equal rows (every
// group at least one chunk).
std::vector<RowGroup> plan_groups(const std::vector<Chunk>& chunks, int n)
{
    const int nc = (int)chunks.size();
    n = std::max(1, std::min(n, nc));
    int R = 0;
    for (const Chunk& c : chunks) R += c.in_len;
    std::vector<RowGroup> groups(n);
    int i = 0;
    for (int g = 0; g < n; ++g) {
        RowGroup& rg = groups[g];
        rg.r0 = chunks[i].row;
        const long long target = (long long)R * (g + 1) / n;   // rows groups 0..g cover
        do {
            rg.R += chunks[i].in_len;
            rg.Tmax = std::max(rg.Tmax, chunks[i].in_len);
            ++i;
        } while (i < nc - (n - 1 - g) &&
                 (g == n - 1 || chunks[i].row + chunks[i].in_len / 2 <= target));
    }
    return groups;
}

int project_positions(pk_gpu_encoder* e, int T);

// Modules of block 0 that group 0 runs before the other row groups start:
// its first feed-forward module, so that from then on one group's GEMMs
// overlap the other's attention and row kernels rather than its own twin
// GEMMs.  Measured with two groups of 1656 rows (three boxes, 2-3 runs
// each): 0.3-1.1% less time per pass than starting together; starting after
// 2 or 3 modules gave the same.  PK_GPU_GROUP_LAG (0-3) overrides it.
int group_lag()
{
    static const int lag = [] {
        const char* v = getenv("PK_GPU_GROUP_LAG");
        const int n = v ? atoi(v) : 1;
        return n >= 0 && n <= 3 ? n : 1;
    }();
    return lag;
}

// The panels of every block weight the small-M kernels read (pk_panel.hip),
// made once on the encoder's stream and waited for (never under capture).
int make_panels(pk_gpu_encoder* e)
{
    if (!e->panel_allocs.empty()) return PK_GPU_OK;
    std::vector<void*> fresh;
    size_t total = 0;
    int rc = PK_GPU_OK;
    for (DevBlock& b : e->blocks) {
        for (DevWeight* w : {&b.ff1_w1, &b.ff1_w2, &b.ff2_w1, &b.ff2_w2, &b.qkv, &b.out, &b.pw1t, &b.pw2t}) {
            const size_t bytes = pkgpu::panel_bytes(w->kind, w->K, w->N);
            void* d = nullptr;
            if (!bytes || hipMalloc(&d, bytes) != hipSuccess) {
                rc = error(PK_GPU_ENOMEM, "weight panels: device allocation of %zu bytes failed", bytes);
                break;
            }
            fresh.push_back(d);
            total += bytes;
            const hipError_t r = pkgpu::launch_pack(w->kind, w->K, w->N, w->data,
                                                    w->kind == pkgpu::W_I4 ? w->N / 2 : w->N, w->scales, d,
                                                    e->stream);
            if (r != hipSuccess) {
                rc = hip_error(r, "weight panels");
                break;
            }
        }
        if (rc) break;
    }
    if (!rc) rc = check(hipStreamSynchronize(e->stream), "weight panels");
    if (rc) {
        (void)hipStreamSynchronize(e->stream);
        for (void* d : fresh) (void)hipFree(d);
        return rc;
    }
    size_t i = 0;
    for (DevBlock& b : e->blocks)
        for (DevWeight* w : {&b.ff1_w1, &b.ff1_w2, &b.ff2_w1, &b.ff2_w2, &b.qkv, &b.out, &b.pw1t, &b.pw2t})
            w->panel = fresh[i++];
    e->panel_allocs.swap(fresh);
    e->panel_bytes = total;
    return PK_GPU_OK;
}

// The block weights' pre-split copies (DevWeight::split; int8: the codes as
// bf16), made once on the encoder's stream.
int make_splits(pk_gpu_encoder* e)
{
    if (!e->split_allocs.empty()) return PK_GPU_OK;
    std::vector<void*> fresh;
    std::vector<DevWeight*> made;
    size_t total = 0;
    int rc = PK_GPU_OK;
    for (DevBlock& b : e->blocks) {
        for (DevWeight* w : {&b.ff1_w1, &b.ff1_w2, &b.ff2_w1, &b.ff2_w2, &b.qkv, &b.out, &b.pw1t, &b.pw2t}) {
            const size_t bytes = pkgpu::split_weight_bytes(w->kind, w->K, w->N);
            if (!bytes) continue;
            void* d = nullptr;
            if (hipMalloc(&d, bytes) != hipSuccess) {
                rc = error(PK_GPU_ENOMEM, "pre-split weights: device allocation of %zu bytes failed", bytes);
                break;
            }
            fresh.push_back(d);
            made.push_back(w);
            total += bytes;
            const hipError_t r = pkgpu::launch_split_pack(w->kind, w->K, w->N, w->data,
                                                          w->kind == pkgpu::W_I4 ? w->N / 2 : w->N, w->scales, d,
                                                          e->stream);
            if (r != hipSuccess) {
                rc = hip_error(r, "pre-split weights");
                break;
            }
        }
        if (rc) break;
    }
    if (!rc) rc = check(hipStreamSynchronize(e->stream), "pre-split weights");
    if (rc) {
        (void)hipStreamSynchronize(e->stream);
        for (void* d : fresh) (void)hipFree(d);
        return rc;
    }
    for (size_t i = 0; i < made.size(); ++i) made[i]->split = fresh[i];
    e->split_allocs.swap(fresh);
    e->split_bytes = total;
    return PK_GPU_OK;
}

int run_queued(pk_gpu_encoder* e, const float* x, int T, int chunk, int ov, float* out,
               hipStream_t s, hipMemcpyKind in_kind, hipMemcpyKind out_kind)
{
    if (T <= 0) return error(PK_GPU_EINVAL, "T = %d", T);
    if (!x || !out) return error(PK_GPU_EINVAL, "x or out is NULL");
    if (chunk > 0 && ov < 0) return error(PK_GPU_EINVAL, "overlap = %d", ov);
    const std::vector<Chunk> chunks = plan_chunks(T, chunk, ov);
    int R = 0, Tmax = 0;
    for (const Chunk& c : chunks) {
        R += c.in_len;
        Tmax = std::max(Tmax, c.in_len);
    }
    const int pe_limit = std::min(e->pe_center + 1, e->pe_rows - e->pe_center);
    if (Tmax > pe_limit)
        return error(PK_GPU_EINVAL, "positional table too small for %d frames (at most %d)", Tmax,
                     pe_limit);
    if (Tmax > e->p_T) {
        // longer than every earlier chunk: each block's projection over the
        // longer slice (the graphs read the old ones)
        wait_all(e);
        drop_graphs(e);
        const int rc = project_positions(e, std::min(pe_limit, (Tmax + 63) & ~63));
        if (rc) return rc;
    }

    // Row groups; each group's chunks are table entries [tab, tab + n), by
    // length, with rows relative to the group; the lengths follow at entry
    // rows_cap.
    std::vector<RowGroup> groups = plan_groups(chunks, e->n_groups);
    std::vector<int> table, lens;
    {
        size_t ci = 0;
        for (RowGroup& g : groups) {
            std::map<int, std::vector<int>> by_len;
            for (int got = 0; got < g.R; ++ci) {
                by_len[chunks[ci].in_len].push_back(chunks[ci].row - g.r0);
                got += chunks[ci].in_len;
            }
            g.tab = (int)table.size();
            for (const auto& l : by_len) {
                g.by_len[l.first] = {(int)table.size() - g.tab, (int)l.second.size()};
                table.insert(table.end(), l.second.begin(), l.second.end());
                lens.insert(lens.end(), l.second.size(), l.first);
            }
            g.n = (int)table.size() - g.tab;
        }
    }
    // attention score rows of groups beyond the LDS limit, one region per group
    size_t scores_n = 0;
    for (RowGroup& g : groups) {
        g.scores_off = scores_n;
        scores_n += pkgpu::attn_scores_floats(g.Tmax, kHeads, g.n);
    }
    int rc = workspace(e, (size_t)R, table.size(), scores_n, s);
    if (rc) return rc;
    // Row groups of at most 64 rows take the small-M kernels outside exact
    // numerics: they read the weights' panels, and split K over workgroups
    // in their group's partial tiles.
    bool small = false;
    for (const RowGroup& g : groups) small = small || g.R <= pkgpu::kSmallMaxM;
    small = small && e->numerics != PK_GPU_NUMERICS_EXACT;
    if (small && e->panel_allocs.empty()) {
        if ((rc = check(hipStreamSynchronize(s), "encoder stream"))) return rc;
        if ((rc = make_panels(e))) return rc;
    }
    // Fast numerics on row groups above 64 rows: the split kernels read the
    // int4 and fp32 weights' pre-split copies.
    bool big = false;
    for (const RowGroup& g : groups) big = big || g.R > pkgpu::kSmallMaxM;
    if (big && e->numerics == PK_GPU_NUMERICS_FAST && e->presplit_w && e->split_allocs.empty()) {
        if ((rc = check(hipStreamSynchronize(s), "encoder stream"))) return rc;
        if ((rc = make_splits(e))) return rc;
    }
    if (e->numerics == PK_GPU_NUMERICS_FAST || small) {
        if (groups.size() > e->part_groups) {
            // the graphs hold the old partial-tile pointers
            wait_all(e);
            drop_graphs(e);
            if (e->part) (void)hipFree(e->part);
            e->part = nullptr;
            e->part_groups = 0;
            if (hipMalloc(reinterpret_cast<void**>(&e->part), groups.size() * pkgpu::kSplitWorkBytes) !=
                hipSuccess) {
                e->part = nullptr;
                return error(PK_GPU_ENOMEM, "split-K workspace of %zu bytes failed",
                             groups.size() * pkgpu::kSplitWorkBytes);
            }
            e->part_groups = groups.size();
        }
        for (size_t gi = 0; gi < groups.size(); ++gi)
            groups[gi].part = e->part + gi * (pkgpu::kSplitWorkBytes / sizeof(float));
    }
    std::vector<int> want(2 * e->rows_cap, 0);
    std::copy(table.begin(), table.end(), want.begin());
    std::copy(lens.begin(), lens.end(), want.begin() + e->rows_cap);
    if (want != e->tab_host) {
        // A previous copy may still be queued: wait for it before the host
        // table it reads is rewritten.
        if ((rc = check(hipStreamSynchronize(s), "encoder stream"))) return rc;
        e->tab_host.swap(want);
        if ((rc = check(hipMemcpyAsync(e->rows_tab, e->tab_host.data(),
                                       e->tab_host.size() * sizeof(int), hipMemcpyHostToDevice, s),
                        "chunk table")))
            return rc;
    }
    // every chunk's input rows (encoder.c:552-553)
    for (const Chunk& c : chunks) {
        const size_t n = (size_t)c.in_len * kD * 4;
        rc = timed(e, PK_GPU_STAGE_COPY, 0.0, 2.0 * n, s, [&] {
            return check(hipMemcpyAsync(e->x + (size_t)c.row * kD, x + (size_t)c.in_start * kD, n,
                                        in_kind, s), "input copy");
        });
        if (rc) return rc;
    }
    if (e->prof) {
        // eager, with an event pair around every launch: the replay's own
        // kernels (same groups, same tiles), one group after another on s
        for (const RowGroup& g : groups)
            for (const DevBlock& b : e->blocks)
                if ((rc = run_block(e, b, g, s))) return rc;
    } else {
        if ((rc = side_streams(e, (int)groups.size() - 1))) return rc;
        // One graph per chunking of the input and group: captured on the
        // encoder's own stream (the null stream cannot capture).  A caller
        // that sees many input lengths would keep adding graphs; past
        // kMaxGraphs they are all dropped and recaptured on demand.
        const int forced = pkgpu::rt::forced_config();
        // The other groups start when group 0 has run the first `lag` modules
        // of block 0 (its lead graph), so that the groups' GEMMs and their
        // row kernels fall at different times.
        const int lag = groups.size() < 2 ? 0 : e->lag >= 0 ? e->lag : group_lag();
        if (e->graphs.size() + groups.size() + (lag > 0) > kMaxGraphs &&
            !e->graphs.count(std::make_tuple(T, chunk, ov, lag > 0 ? 100 + lag : 0, forced,
                                             e->numerics))) {
            if ((rc = check(hipStreamSynchronize(s), "encoder stream"))) return rc;
            for (hipStream_t st : e->side)
                if ((rc = check(hipStreamSynchronize(st), "encoder stream"))) return rc;
            drop_graphs(e);
        }
        auto graph = [&](int id, int gi, int b_from, int m_from, int b_to, int m_to,
                         hipGraphExec_t* out) -> int {
            const auto key = std::make_tuple(T, chunk, ov, id, forced, e->numerics);
            auto it = e->graphs.find(key);
            if (it == e->graphs.end()) {
                int r = check(hipStreamBeginCapture(e->stream, hipStreamCaptureModeThreadLocal),
                              "graph capture");
                if (r) return r;
                // modules m_from.. of block b_from through modules ..m_to of block b_to
                for (int bi = b_from; bi <= b_to && !r; ++bi)
                    r = run_block(e, e->blocks[bi], groups[gi], e->stream, bi == b_from ? m_from : 0,
                                  bi == b_to ? m_to : 4);
                hipGraph_t g = nullptr;
                const hipError_t end = hipStreamEndCapture(e->stream, &g);
                if (!r && end != hipSuccess) r = hip_error(end, "graph capture");
                hipGraphExec_t x_ = nullptr;
                if (!r) r = check(hipGraphInstantiate(&x_, g, nullptr, nullptr, 0), "graph instantiate");
                if (g) (void)hipGraphDestroy(g);
                if (r) return r;
                it = e->graphs.emplace(key, x_).first;
            }
            *out = it->second;
            return PK_GPU_OK;
        };
        const int nb = (int)e->blocks.size();
        std::vector<hipGraphExec_t> ex(groups.size(), nullptr);
        hipGraphExec_t lead = nullptr;
        for (size_t gi = 0; gi < groups.size(); ++gi) {
            if (gi == 0 && lag > 0) {
                if ((rc = graph(-lag, 0, 0, 0, 0, lag, &lead)) ||
                    (rc = graph(100 + lag, 0, 0, lag, nb - 1, 4, &ex[0])))
                    return rc;
            } else if ((rc = graph((int)gi, (int)gi, 0, 0, nb - 1, 4, &ex[gi]))) {
                return rc;
            }
        }
        // group 0 on `s`; the others on side streams that start after the
        // input copies (and group 0's lead graph) and that `s` waits for
        // before the output copies
        if (lead && (rc = check(hipGraphLaunch(lead, s), "graph launch"))) return rc;
        if (groups.size() > 1 &&
            (rc = check(hipEventRecord(e->inputs_ready, s), "encoder event")))
            return rc;
        for (size_t gi = 1; gi < groups.size(); ++gi) {
            hipStream_t ss = e->side[gi - 1];
            if ((rc = check(hipStreamWaitEvent(ss, e->inputs_ready, 0), "encoder event")) ||
                (rc = check(hipGraphLaunch(ex[gi], ss), "graph launch")) ||
                (rc = check(hipEventRecord(e->side_done[gi - 1], ss), "encoder event")))
                return rc;
        }
        if ((rc = check(hipGraphLaunch(ex[0], s), "graph launch"))) return rc;
        for (size_t gi = 1; gi < groups.size(); ++gi)
            if ((rc = check(hipStreamWaitEvent(s, e->side_done[gi - 1], 0), "encoder event")))
                return rc;
    }
    // the centre rows of every chunk (encoder.c:567-569)
    for (const Chunk& c : chunks) {
        const size_t n = (size_t)c.out_len * kD * 4;
        rc = timed(e, PK_GPU_STAGE_COPY, 0.0, 2.0 * n, s, [&] {
            return check(hipMemcpyAsync(out + (size_t)c.out_start * kD,
                                        e->x + (size_t)(c.row + c.left_ov) * kD, n, out_kind, s),
                         "output copy");
        });
        if (rc) return rc;
    }
    return PK_GPU_OK;
}

int run(pk_gpu_encoder* e, const float* x, int T, int chunk, int ov, float* out, hipStream_t s,
        hipMemcpyKind in_kind, hipMemcpyKind out_kind)
{
    if (!e) return error(PK_GPU_EINVAL, "encoder is NULL");
    int rc = follow_last(e, s);
    if (rc) return rc;
    rc = run_queued(e, x, T, chunk, ov, out, s, in_kind, out_kind);
    const int m = mark_last(e, s);          // also after a failure: work may be queued
    return rc ? rc : m;
}

// Upload into the pre-encode's own allocations (freed when it is replaced).
int pre_upload(pk_gpu_encoder* e, const void* host, size_t bytes, const char* what, const void** out)
{
    if (!host) return error(PK_GPU_EINVAL, "%s is NULL", what);
    void* d = nullptr;
    if (hipMalloc(&d, bytes) != hipSuccess) return error(PK_GPU_ENOMEM, "%s: device allocation", what);
    e->pre.allocs.push_back(d);
    hipError_t r = hipMemcpyAsync(d, host, bytes, hipMemcpyHostToDevice, e->stream);
    if (r != hipSuccess) return hip_error(r, what);
    *out = d;
    return PK_GPU_OK;
}

void free_pre(pk_gpu_encoder* e)
{
    for (void* p : e->pre.allocs) (void)hipFree(p);
    e->pre = DevPreEncode{};
    for (float* p : {e->pre_a, e->pre_b, e->pre_x})
        if (p) (void)hipFree(p);
    e->pre_a = e->pre_b = e->pre_x = nullptr;
    e->pre_a_n = e->pre_b_n = e->pre_x_n = 0;
}

int grow(float** buf, size_t* cap, size_t n, hipStream_t s)
{
    if (n <= *cap) return PK_GPU_OK;
    hipError_t r = hipStreamSynchronize(s);
    if (r != hipSuccess) return hip_error(r, "pre-encode stream");
    if (*buf) (void)hipFree(*buf);
    *buf = nullptr;
    *cap = 0;
    if (hipMalloc(reinterpret_cast<void**>(buf), n * sizeof(float)) != hipSuccess)
        return error(PK_GPU_ENOMEM, "pre-encode workspace of %zu floats", n);
    *cap = n;
    return PK_GPU_OK;
}

// pre_encode_and_scale (encoder.c:103-174, 578-592): mel [128][T] to
// x [T'][1024].  Channel-last throughout; the 1x1 convolutions and the output
// linear are chain GEMMs (the convolutions started from their bias).
int pre_encode_queued(pk_gpu_encoder* e, const float* mel, int T, float* x, hipStream_t s)
{
    const DevPreEncode& w = e->pre;
    const int H1 = half_up(T), W1 = half_up(kMels);
    const int H2 = half_up(H1), W2 = half_up(W1);
    const int H3 = half_up(H2), W3 = half_up(W2);
    int rc = grow(&e->pre_a, &e->pre_a_n, (size_t)H1 * W1 * kSub, s);
    if (!rc) rc = grow(&e->pre_b, &e->pre_b_n, (size_t)H2 * W2 * kSub, s);
    if (rc) return rc;
    float *A = e->pre_a, *B = e->pre_b;
    // conv.0 + ReLU -> A [H1][W1][256]
    if ((rc = check(pkgpu::launch_conv0_relu(mel, T, kMels, w.w0, w.b0, A, H1, W1, s), "conv.0"))) return rc;
    // conv.2 (depthwise) -> B; conv.3 (pointwise) + ReLU -> A
    if ((rc = check(pkgpu::launch_dwconv3x3s2(A, H1, W1, w.w2, w.b2, B, H2, W2, s), "conv.2"))) return rc;
    // Rows are independent, so long inputs run in slabs whose operands stay
    // under the chain kernels' 2 GiB extent.
    auto pointwise = [&](const DevWeight& wt, const float* bias, const float* in, float* out, int rows) {
        const int slab = (1 << 28) / kSub;          // 1 GiB of A per launch
        for (int r0 = 0; r0 < rows; r0 += slab) {
            GemmProblem p{};
            p.kind = pkgpu::W_F32;
            p.M = std::min(slab, rows - r0); p.N = kSub; p.K = kSub;
            p.alpha = 1.0f; p.beta = 0.0f;
            p.chain_bias = bias;                    // the chain starts from the bias
            p.A = in + (size_t)r0 * kSub; p.lda = kSub;
            p.B = wt.data; p.ldb = kSub;
            p.C = out + (size_t)r0 * kSub; p.ldc = kSub;
            p.epi = pkgpu::EPI_RELU;
            const int r = pkgpu::rt::gemm(p, s);
            if (r) return r;
        }
        return (int)PK_GPU_OK;
    };
    if ((rc = pointwise(w.w3t, w.b3, B, A, H2 * W2))) return rc;
    // conv.5 (depthwise) -> B; conv.6 (pointwise) + ReLU -> A
    if ((rc = check(pkgpu::launch_dwconv3x3s2(A, H2, W2, w.w5, w.b5, B, H3, W3, s), "conv.5"))) return rc;
    if ((rc = pointwise(w.w6t, w.b6, B, A, H3 * W3))) return rc;
    // flatten -> B [T'][256*W3]; out linear + bias -> x; times sqrt(1024)
    if ((rc = check(pkgpu::launch_flatten_rows(A, B, H3, W3, s), "flatten"))) return rc;
    const int slab = (1 << 28) / (kSub * W3);        // 1 GiB of A per launch
    for (int r0 = 0; r0 < H3; r0 += slab)
        if ((rc = gemm_launch(w.out, B + (size_t)r0 * kSub * W3, std::min(slab, H3 - r0),
                              x + (size_t)r0 * kD, w.out_b, pkgpu::EPI_NONE, s)))
            return rc;
    return check(pkgpu::launch_scale(x, (long long)H3 * kD, 32.0f, s), "scale");
}

int pre_encode(pk_gpu_encoder* e, const float* mel, int T, float* x, hipStream_t s)
{
    int rc = follow_last(e, s);
    if (rc) return rc;
    rc = pre_encode_queued(e, mel, T, x, s);
    const int m = mark_last(e, s);
    return rc ? rc : m;
}

int dev_stream(void* stream, hipStream_t* s)
{
    hipStream_t own = nullptr;
    int rc = pkgpu::rt::bind(&own);
    *s = static_cast<hipStream_t>(stream);
    return rc;
}

// Every block's linear_pos over the positional slice of chunks of up to T
// rows.  A chunk of T' <= T rows uses the slice pe[centre - T' + 1,
// centre + T' - 1], rows T - T' onwards of this one, and each projected row
// depends only on its own input row, so the rows are the ones the reference
// computes per chunk (encoder.c:319-338).  Replaces the previous projections
// (the caller has drained every stream and dropped the graphs that read them).
int project_positions(pk_gpu_encoder* e, int T)
{
    const int L = 2 * T - 1;
    const size_t bytes = (size_t)L * kD * 4;
    const float* slice = e->pe + (size_t)(e->pe_center - T + 1) * kD;
    std::vector<void*> fresh;
    int rc = PK_GPU_OK;
    for (DevBlock& b : e->blocks) {
        void* d = nullptr;
        if (hipMalloc(&d, bytes) != hipSuccess) {
            rc = error(PK_GPU_ENOMEM, "position projections of %zu bytes failed", bytes);
            break;
        }
        fresh.push_back(d);
        // exact chains in every numerics mode: the projections are constants
        // that later runs in any mode read (encoder.c:319-338)
        rc = gemm(e, b.pos, slice, L, static_cast<float*>(d), nullptr, pkgpu::EPI_NONE, e->stream,
                  nullptr, false, true);
        if (rc) break;
    }
    if (!rc) rc = check(hipStreamSynchronize(e->stream), "position projections");
    if (rc) {
        (void)hipStreamSynchronize(e->stream);
        for (void* d : fresh) (void)hipFree(d);
        return rc;
    }
    for (void* d : e->pos_allocs) (void)hipFree(d);
    e->weight_bytes = e->weight_bytes - e->pos_allocs.size() * (size_t)(2 * e->p_T - 1) * kD * 4 +
                      fresh.size() * bytes;
    e->pos_allocs.swap(fresh);
    for (size_t i = 0; i < e->blocks.size(); ++i) e->blocks[i].P = static_cast<const float*>(e->pos_allocs[i]);
    e->p_T = T;
    return PK_GPU_OK;
}

}  // namespace

extern "C" {

int pk_gpu_encoder_create(pk_gpu_encoder** out, const pk_gpu_block_weights* blocks, int n_blocks,
                          const float* pe_table, int pe_rows, int pe_center)
{
    if (!out) return error(PK_GPU_EINVAL, "enc is NULL");
    *out = nullptr;
    if (!blocks || n_blocks <= 0) return error(PK_GPU_EINVAL, "no blocks");
    if (!pe_table || pe_rows <= 0 || pe_center < 0 || pe_center >= pe_rows)
        return error(PK_GPU_EINVAL, "bad positional table (%d rows, centre %d)", pe_rows, pe_center);
    int rc = pkgpu::rt::bind(nullptr);
    if (rc) return rc;
    pk_gpu_encoder* e = new pk_gpu_encoder;
    if (const char* v = getenv("PK_GPU_PRESPLIT")) e->presplit = strcmp(v, "0") != 0;
    if (const char* v = getenv("PK_GPU_FUSE_LN")) e->fuse_ln = strcmp(v, "0") != 0;
    if (const char* v = getenv("PK_GPU_FAST_ATTN")) e->fast_attn = strcmp(v, "0") != 0;
    if (const char* v = getenv("PK_GPU_PRESPLIT_W")) e->presplit_w = strcmp(v, "0") != 0;
    hipError_t r = hipStreamCreateWithFlags(&e->stream, hipStreamNonBlocking);
    if (r != hipSuccess) {
        delete e;
        return hip_error(r, "hipStreamCreate");
    }
    e->blocks.resize(n_blocks);
    for (int i = 0; i < n_blocks && !rc; ++i) rc = upload_block(e, blocks[i], &e->blocks[i]);
    if (!rc) rc = upload_f(e, pe_table, (size_t)pe_rows * kD, "pe_table", &e->pe);
    e->pe_rows = pe_rows;
    e->pe_center = pe_center;
    if (!rc) rc = project_positions(e, std::min({pkgpu::kAttnMaxT, pe_center + 1, pe_rows - pe_center}));
    if (!rc) rc = check(hipStreamSynchronize(e->stream), "weight upload");
    if (rc) {
        pk_gpu_encoder_destroy(e);
        return rc;
    }
    *out = e;
    return PK_GPU_OK;
}

int pk_gpu_encoder_run(pk_gpu_encoder* enc, const float* x, int T, int chunk_size, int overlap,
                       float* out)
{
    int rc = pkgpu::rt::bind(nullptr);
    if (rc) return rc;
    // x may equal out: the input is copied into the workspace first
    rc = run(enc, x, T, chunk_size, overlap, out, enc ? enc->stream : nullptr,
             hipMemcpyHostToDevice, hipMemcpyDeviceToHost);
    if (rc) return rc;
    return check(hipStreamSynchronize(enc->stream), "encoder run");
}

int pk_gpu_encoder_run_dev(pk_gpu_encoder* enc, const float* dx, int T, int chunk_size, int overlap,
                           float* dout, void* stream)
{
    hipStream_t s = nullptr;
    int rc = dev_stream(stream, &s);
    if (rc) return rc;
    return run(enc, dx, T, chunk_size, overlap, dout, s, hipMemcpyDeviceToDevice,
               hipMemcpyDeviceToDevice);
}

size_t pk_gpu_encoder_bytes(const pk_gpu_encoder* enc)
{
    return enc ? enc->weight_bytes + enc->ws_bytes + enc->part_groups * pkgpu::kSplitWorkBytes +
                     enc->panel_bytes + enc->split_bytes
               : 0;
}

int pk_gpu_encoder_profile(pk_gpu_encoder* enc, int enable)
{
    if (!enc) return error(PK_GPU_EINVAL, "encoder is NULL");
    int rc = collect(enc);
    if (rc) return rc;
    enc->prof = enable != 0;
    for (int i = 0; i < PK_GPU_N_STAGES; ++i) {
        enc->ms[i] = enc->flops[i] = enc->bytes[i] = 0.0;
        enc->launches[i] = 0;
    }
    return PK_GPU_OK;
}

int pk_gpu_encoder_profile_read(pk_gpu_encoder* enc, int stage, double* ms, long long* launches,
                                double* flops, double* bytes)
{
    if (!enc) return error(PK_GPU_EINVAL, "encoder is NULL");
    if (stage < 0 || stage >= PK_GPU_N_STAGES) return error(PK_GPU_EINVAL, "stage %d", stage);
    int rc = collect(enc);
    if (rc) return rc;
    if (ms) *ms = enc->ms[stage];
    if (launches) *launches = enc->launches[stage];
    if (flops) *flops = enc->flops[stage];
    if (bytes) *bytes = enc->bytes[stage];
    return PK_GPU_OK;
}

void pk_gpu_encoder_destroy(pk_gpu_encoder* enc)
{
    if (!enc) return;
    wait_all(enc);
    (void)collect(enc);
    for (hipEvent_t ev : enc->event_pool) (void)hipEventDestroy(ev);
    free_workspace(enc);
    free_pre(enc);
    if (enc->part) (void)hipFree(enc->part);
    for (void* p : enc->allocs) (void)hipFree(p);
    for (void* p : enc->pos_allocs) (void)hipFree(p);
    for (void* p : enc->panel_allocs) (void)hipFree(p);
    for (void* p : enc->split_allocs) (void)hipFree(p);
    for (hipEvent_t ev : enc->side_done) (void)hipEventDestroy(ev);
    if (enc->inputs_ready) (void)hipEventDestroy(enc->inputs_ready);
    if (enc->last_done) (void)hipEventDestroy(enc->last_done);
    for (hipStream_t st : enc->side) (void)hipStreamDestroy(st);
    if (enc->stream) (void)hipStreamDestroy(enc->stream);
    delete enc;
}

int pk_gpu_encoder_set_numerics(pk_gpu_encoder* enc, int mode)
{
    if (!enc) return error(PK_GPU_EINVAL, "encoder is NULL");
    if (mode != PK_GPU_NUMERICS_DEFAULT && mode != PK_GPU_NUMERICS_EXACT &&
        mode != PK_GPU_NUMERICS_FAST)
        return error(PK_GPU_EINVAL, "numerics mode %d", mode);
    enc->numerics = mode;          // graphs are kept per mode
    return PK_GPU_OK;
}

int pk_gpu_encoder_get_numerics(pk_gpu_encoder* enc)
{
    return enc ? enc->numerics : -1;
}

int pk_gpu_encoder_set_group_lag(pk_gpu_encoder* enc, int modules)
{
    if (!enc) return error(PK_GPU_EINVAL, "encoder is NULL");
    if (modules < -1 || modules > 3) return error(PK_GPU_EINVAL, "group lag %d (-1..3)", modules);
    enc->lag = modules;            // graphs are kept per lead
    return PK_GPU_OK;
}

int pk_gpu_encoder_set_groups(pk_gpu_encoder* enc, int n_groups)
{
    if (!enc) return error(PK_GPU_EINVAL, "encoder is NULL");
    if (n_groups < 1 || n_groups > PK_GPU_MAX_GROUPS)
        return error(PK_GPU_EINVAL, "n_groups = %d (1..%d)", n_groups, PK_GPU_MAX_GROUPS);
    int rc = pkgpu::rt::bind(nullptr);
    if (rc) return rc;
    if (n_groups != enc->n_groups) {
        wait_all(enc);
        drop_graphs(enc);
        enc->n_groups = n_groups;
    }
    return PK_GPU_OK;
}

int pk_gpu_encoder_set_pre_encode(pk_gpu_encoder* enc, const pk_gpu_pre_encode_weights* w)
{
    if (!enc || !w) return error(PK_GPU_EINVAL, "encoder or weights is NULL");
    int rc = pkgpu::rt::bind(nullptr);
    if (rc) return rc;
    wait_all(enc);
    free_pre(enc);
    DevPreEncode& d = enc->pre;
    const void* v = nullptr;
    auto up = [&](const float* host, size_t n, const char* what, const float** out) {
        int r = pre_upload(enc, host, n * sizeof(float), what, &v);
        *out = static_cast<const float*>(v);
        return r;
    };
    if (!rc) rc = up(w->conv0_w, kSub * 9, "conv0_w", &d.w0);
    if (!rc) rc = up(w->conv0_b, kSub, "conv0_b", &d.b0);
    if (!rc) rc = up(w->conv2_w, kSub * 9, "conv2_w", &d.w2);
    if (!rc) rc = up(w->conv2_b, kSub, "conv2_b", &d.b2);
    if (!rc) rc = up(w->conv3_b, kSub, "conv3_b", &d.b3);
    if (!rc) rc = up(w->conv5_w, kSub * 9, "conv5_w", &d.w5);
    if (!rc) rc = up(w->conv5_b, kSub, "conv5_b", &d.b5);
    if (!rc) rc = up(w->conv6_b, kSub, "conv6_b", &d.b6);
    if (!rc) rc = up(w->out_b, kD, "out_b", &d.out_b);
    // 1x1 convolution weights [Cout][Cin] stored transposed, [Cin][Cout]:
    // the weight becomes the GEMM's B operand (upload_pointwise).
    for (int k = 0; k < 2 && !rc; ++k) {
        const float* host = k ? w->conv6_w : w->conv3_w;
        DevWeight* dw = k ? &d.w6t : &d.w3t;
        const float* raw = nullptr;
        rc = up(host, kSub * kSub, k ? "conv6_w" : "conv3_w", &raw);
        void* t = nullptr;
        if (!rc && hipMalloc(&t, kSub * kSub * 4) != hipSuccess) rc = error(PK_GPU_ENOMEM, "pointwise");
        if (!rc) {
            d.allocs.push_back(t);
            rc = check(pkgpu::launch_transpose(raw, static_cast<float*>(t), kSub, kSub, enc->stream),
                       "transpose");
            dw->kind = pkgpu::W_F32;
            dw->data = t;
            dw->K = dw->N = kSub;
        }
    }
    if (!rc) {
        const pk_gpu_weight& o = w->out_w;
        const int K = kSub * 16, N = kD;          // 256 channels x 16 mel bins after three stages
        d.out.K = K;
        d.out.N = N;
        d.out.scale = o.scale;
        if (o.bits == 8) {
            d.out.kind = pkgpu::W_I8;
            rc = pre_upload(enc, o.data, (size_t)K * N, "out_w", &d.out.data);
        } else if (o.bits == 32) {
            d.out.kind = pkgpu::W_F32;
            rc = pre_upload(enc, o.data, (size_t)K * N * 4, "out_w", &d.out.data);
        } else if (o.bits == 4) {
            d.out.kind = pkgpu::W_I4;
            rc = pre_upload(enc, o.data, (size_t)K * N / 2, "out_w", &d.out.data);
            if (!rc) rc = pre_upload(enc, o.scales, (size_t)K * (N / 32) * 4, "out_w scales", &v);
            d.out.scales = static_cast<const float*>(v);
        } else {
            rc = error(PK_GPU_EINVAL, "out_w: bits = %d", o.bits);
        }
    }
    if (!rc) rc = check(hipStreamSynchronize(enc->stream), "pre-encode upload");
    if (rc) {
        free_pre(enc);
        return rc;
    }
    d.set = true;
    return PK_GPU_OK;
}

int pk_gpu_encoder_frames(int n_frames)
{
    return n_frames > 0 ? half_up(half_up(half_up(n_frames))) : 0;
}

int pk_gpu_encoder_pre_encode_dev(pk_gpu_encoder* enc, const float* dmel, int n_frames, float* dx,
                                  void* stream)
{
    if (!enc || !dmel || !dx) return error(PK_GPU_EINVAL, "NULL argument");
    if (!enc->pre.set) return error(PK_GPU_EINVAL, "no pre-encode weights (pk_gpu_encoder_set_pre_encode)");
    if (n_frames <= 0) return error(PK_GPU_EINVAL, "n_frames = %d", n_frames);
    hipStream_t s;
    int rc = dev_stream(stream, &s);
    if (rc) return rc;
    return pre_encode(enc, dmel, n_frames, dx, s);
}

int pk_gpu_encoder_run_mel(pk_gpu_encoder* enc, const float* mel, int n_frames, int chunk_size,
                           int overlap, float* out)
{
    if (!enc || !mel || !out) return error(PK_GPU_EINVAL, "NULL argument");
    if (!enc->pre.set) return error(PK_GPU_EINVAL, "no pre-encode weights (pk_gpu_encoder_set_pre_encode)");
    if (n_frames <= 0) return error(PK_GPU_EINVAL, "n_frames = %d", n_frames);
    int rc = pkgpu::rt::bind(nullptr);
    if (rc) return rc;
    hipStream_t s = enc->stream;
    const int Tp = pk_gpu_encoder_frames(n_frames);
    if ((rc = grow(&enc->pre_x, &enc->pre_x_n, (size_t)Tp * kD, s))) return rc;
    float* dmel = nullptr;
    if (hipMalloc(reinterpret_cast<void**>(&dmel), (size_t)kMels * n_frames * 4) != hipSuccess)
        return error(PK_GPU_ENOMEM, "mel buffer");
    rc = check(hipMemcpyAsync(dmel, mel, (size_t)kMels * n_frames * 4, hipMemcpyHostToDevice, s),
               "mel upload");
    if (!rc) rc = pre_encode(enc, dmel, n_frames, enc->pre_x, s);
    if (!rc) rc = run(enc, enc->pre_x, Tp, chunk_size, overlap, out, s, hipMemcpyDeviceToDevice,
                      hipMemcpyDeviceToHost);
    if (!rc) rc = check(hipStreamSynchronize(s), "encoder run");
    else (void)hipStreamSynchronize(s);
    (void)hipFree(dmel);
    return rc;
}

int pk_gpu_layer_norm_dev(const float* dx, const float* dgamma, const float* dbeta, float* dout,
                          int rows, int D, void* stream)
{
    if (rows < 0 || D != kD) return error(PK_GPU_EINVAL, "rows = %d, D = %d (D must be %d)", rows, D, kD);
    if (rows && (!dx || !dgamma || !dbeta || !dout)) return error(PK_GPU_EINVAL, "NULL operand");
    if ((reinterpret_cast<uintptr_t>(dx) | reinterpret_cast<uintptr_t>(dout) |
         reinterpret_cast<uintptr_t>(dgamma) | reinterpret_cast<uintptr_t>(dbeta)) % 16)
        return error(PK_GPU_EINVAL, "x, gamma, beta and out must be 16-byte aligned");
    hipStream_t s;
    int rc = dev_stream(stream, &s);
    if (rc) return rc;
    return check(pkgpu::launch_layer_norm(dx, D, dgamma, dbeta, dout, D, rows, D, s), "layer norm");
}

namespace {
int attention_call(const float* dqkv, int ldq, const float* dP, int ldp, const float* dpu,
                   const float* dpv, float* dout, int ldo, int T, int H, float* dws,
                   size_t ws_floats, void* stream)
{
    if (T < 1) return error(PK_GPU_EINVAL, "T = %d", T);
    if (H < 1) return error(PK_GPU_EINVAL, "H = %d", H);
    const int D = 128 * H;
    if (ldq < 3 * D || ldp < D || ldo < D || ldq % 4 || ldp % 4)
        return error(PK_GPU_EINVAL, "leading dimensions %d/%d/%d too small or not multiples of 4",
                     ldq, ldp, ldo);
    if (!dqkv || !dP || !dpu || !dpv || !dout) return error(PK_GPU_EINVAL, "NULL operand");
    if ((reinterpret_cast<uintptr_t>(dqkv) | reinterpret_cast<uintptr_t>(dP)) % 16)
        return error(PK_GPU_EINVAL, "qkv and P must be 16-byte aligned");
    const size_t need = pkgpu::attn_scores_floats(T, H, 1);
    if (need && (!dws || ws_floats < need || reinterpret_cast<uintptr_t>(dws) % 16))
        return error(PK_GPU_EINVAL, "T = %d needs a 16-byte aligned workspace of %zu floats "
                     "(pk_gpu_attention_ws_floats)", T, need);
    hipStream_t s;
    int rc = dev_stream(stream, &s);
    if (rc) return rc;
    pkgpu::AttnArgs a{};
    a.qkv = dqkv; a.ldq = ldq; a.P = dP; a.ldp = ldp;
    a.pos_bias_u = dpu; a.pos_bias_v = dpv;
    a.out = dout; a.ldo = ldo;
    a.chunk_rows = nullptr;
    a.T = T; a.H = H;
    a.scores = need ? dws : nullptr;
    return check(pkgpu::launch_attention(a, 1, s), "attention");
}
}  // namespace

int pk_gpu_attention_dev(const float* dqkv, int ldq, const float* dP, int ldp, const float* dpu,
                         const float* dpv, float* dout, int ldo, int T, int H, void* stream)
{
    if (T > pkgpu::kAttnMaxT)
        return error(PK_GPU_EINVAL, "T = %d (1..%d; longer sequences: pk_gpu_attention_ws_dev)", T,
                     pkgpu::kAttnMaxT);
    return attention_call(dqkv, ldq, dP, ldp, dpu, dpv, dout, ldo, T, H, nullptr, 0, stream);
}

size_t pk_gpu_attention_ws_floats(int T, int H)
{
    return T < 1 || H < 1 ? 0 : pkgpu::attn_scores_floats(T, H, 1);
}

int pk_gpu_attention_ws_dev(const float* dqkv, int ldq, const float* dP, int ldp, const float* dpu,
                            const float* dpv, float* dout, int ldo, int T, int H, float* dws,
                            size_t ws_floats, void* stream)
{
    return attention_call(dqkv, ldq, dP, ldp, dpu, dpv, dout, ldo, T, H, dws, ws_floats, stream);
}

int pk_gpu_glu_dev(const float* din, float* dout, int rows, int D, void* stream)
{
    if (rows < 0 || D <= 0) return error(PK_GPU_EINVAL, "rows = %d, D = %d", rows, D);
    if (rows && (!din || !dout)) return error(PK_GPU_EINVAL, "NULL operand");
    hipStream_t s;
    int rc = dev_stream(stream, &s);
    if (rc) return rc;
    return check(pkgpu::launch_glu(din, 2 * D, dout, D, rows, D, s), "glu");
}

int pk_gpu_depthwise_dev(const float* dx, int ldx, const float* dw, const float* db, float* dout,
                         int ldo, int T, int C, int K, int swish, void* stream)
{
    if (T < 0 || C <= 0 || K <= 0 || K % 2 == 0 || ldx < C || ldo < C)
        return error(PK_GPU_EINVAL, "T = %d, C = %d, K = %d, ldx = %d, ldo = %d", T, C, K, ldx, ldo);
    if (T && (!dx || !dw || !dout)) return error(PK_GPU_EINVAL, "NULL operand");
    hipStream_t s;
    int rc = dev_stream(stream, &s);
    if (rc) return rc;
    pkgpu::DwArgs d{};
    d.x = dx; d.ldx = ldx; d.w = dw; d.b = db; d.out = dout; d.ldo = ldo;
    d.chunk_rows = nullptr;
    d.T = T; d.C = C; d.K = K; d.swish = swish != 0;
    return check(pkgpu::launch_depthwise(d, 1, s), "depthwise conv");
}

}  // extern "C"
