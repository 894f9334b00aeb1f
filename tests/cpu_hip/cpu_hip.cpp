// CPU implementation of the HIP stand-in (hip/hip_runtime.h) and of the
// kernel launchers pk_gpu_runtime.hip calls, for the registry stress test.
// Streams hold queues of work that run, in order, when the stream or the
// device is synchronised; hipFree synchronises the device first, as HIP's
// does.  The launchers queue work that reads every operand the real kernels
// read and writes the output, so ThreadSanitizer sees a device copy freed
// while queued work still needs it.
#include <hip/hip_runtime.h>

#include "pk_gemm_kernels.h"

#include <atomic>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <deque>
#include <mutex>
#include <set>

struct ihipStream_t {
    std::mutex mu;      // guards q
    std::mutex run;     // held while draining, so items run in order, one at a time
    std::deque<std::function<void()>> q;
};

namespace {

ihipStream_t g_null;
std::mutex g_streams_mu;
std::set<ihipStream_t*>& streams()
{
    static std::set<ihipStream_t*>* s = new std::set<ihipStream_t*>{&g_null};
    return *s;
}

void drain(ihipStream_t* s)
{
    std::lock_guard<std::mutex> r(s->run);
    for (;;) {
        std::function<void()> w;
        {
            std::lock_guard<std::mutex> lk(s->mu);
            if (s->q.empty()) return;
            w = std::move(s->q.front());
            s->q.pop_front();
        }
        w();
    }
}

ihipStream_t* of(hipStream_t s) { return s ? s : &g_null; }

thread_local int t_role = 0;
std::atomic<long> g_syncs[4];

void drain_all()
{
    std::set<ihipStream_t*> all;
    {
        std::lock_guard<std::mutex> lk(g_streams_mu);
        all = streams();
    }
    for (ihipStream_t* s : all) drain(s);
}

// Reads of an operand's first and last bytes stand for the kernel's reads.
thread_local volatile unsigned char g_sink;
void touch(const void* p, size_t bytes)
{
    if (!p || !bytes) return;
    const unsigned char* b = static_cast<const unsigned char*>(p);
    g_sink = b[0];
    g_sink = b[bytes - 1];
}

}  // namespace

void cpu_hip_set_role(int role) { t_role = role; }
long cpu_hip_device_syncs(int role) { return g_syncs[role & 3].load(); }

void cpu_hip_enqueue(hipStream_t s, std::function<void()> work)
{
    ihipStream_t* st = of(s);
    std::lock_guard<std::mutex> lk(st->mu);
    st->q.push_back(std::move(work));
}

hipError_t hipGetDeviceCount(int* n) { *n = 1; return hipSuccess; }
hipError_t hipGetDeviceProperties(hipDeviceProp_t* p, int)
{
    std::memset(p, 0, sizeof *p);
    std::strcpy(p->name, "cpu stand-in");
    std::strcpy(p->gcnArchName, "gfx950:sramecc+:xnack-");
    p->multiProcessorCount = 256;
    return hipSuccess;
}
hipError_t hipSetDevice(int) { return hipSuccess; }
hipError_t hipGetDevice(int* d) { *d = 0; return hipSuccess; }
hipError_t hipGetSymbolAddress(void** out, const void* symbol) { *out = const_cast<void*>(symbol); return hipSuccess; }
hipError_t hipMalloc(void** p, size_t bytes)
{
    *p = std::calloc(bytes ? bytes : 1, 1);
    return *p ? hipSuccess : hipErrorOutOfMemory;
}
hipError_t hipFree(void* p)
{
    drain_all();                // hipFree waits for the device's queued work
    std::free(p);
    return hipSuccess;
}
hipError_t hipMemcpy(void* dst, const void* src, size_t bytes, hipMemcpyKind)
{
    drain(&g_null);
    std::memcpy(dst, src, bytes);
    return hipSuccess;
}
hipError_t hipMemcpyAsync(void* dst, const void* src, size_t bytes, hipMemcpyKind, hipStream_t s)
{
    cpu_hip_enqueue(s, [=] { std::memcpy(dst, src, bytes); });
    return hipSuccess;
}
hipError_t hipMemcpy2DAsync(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width,
                            size_t rows, hipMemcpyKind, hipStream_t s)
{
    cpu_hip_enqueue(s, [=] {
        for (size_t r = 0; r < rows; ++r)
            std::memcpy(static_cast<char*>(dst) + r * dpitch, static_cast<const char*>(src) + r * spitch, width);
    });
    return hipSuccess;
}
hipError_t hipMemsetAsync(void* dst, int value, size_t bytes, hipStream_t s)
{
    cpu_hip_enqueue(s, [=] { std::memset(dst, value, bytes); });
    return hipSuccess;
}
hipError_t hipStreamCreate(hipStream_t* s) { return hipStreamCreateWithFlags(s, 0); }
hipError_t hipStreamCreateWithFlags(hipStream_t* s, unsigned)
{
    *s = new ihipStream_t;
    std::lock_guard<std::mutex> lk(g_streams_mu);
    streams().insert(*s);
    return hipSuccess;
}
hipError_t hipStreamDestroy(hipStream_t s)
{
    drain(s);
    {
        std::lock_guard<std::mutex> lk(g_streams_mu);
        streams().erase(s);
    }
    delete s;
    return hipSuccess;
}
hipError_t hipStreamSynchronize(hipStream_t s) { drain(of(s)); return hipSuccess; }
hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus* st)
{
    *st = hipStreamCaptureStatusNone;
    return hipSuccess;
}
hipError_t hipDeviceSynchronize()
{
    ++g_syncs[t_role & 3];
    drain_all();
    return hipSuccess;
}
hipError_t hipGetLastError() { return hipSuccess; }
const char* hipGetErrorString(hipError_t) { return "cpu stand-in error"; }

// ---- the kernel launchers (pk_gemm_kernels.h), as queued reads and writes ----
namespace pkgpu {

int choose_config_index(int, int, int, WeightKind) { return 0; }
int num_configs() { return 1; }
TileConfig config_at(int) { return TileConfig{'X', 32, 1, 1, 1, 32}; }
bool smallm_supports(const GemmProblem&) { return false; }
void smallm_tile(const GemmProblem&, int* rb, int* nct) { *rb = 1; *nct = 1; }
bool smallm_force_tile(int, int) { return true; }
hipError_t launch_smallm(const GemmProblem&, hipStream_t) { return hipErrorNotSupported; }
size_t panel_bytes(WeightKind kind, int K, int N)
{
    if (K <= 0 || N <= 0 || K % 32) return 0;
    const size_t n = (size_t)(N + 15) / 16 * 16 * K;
    return kind == W_I8 ? n : kind == W_I4 ? n / 2 + (size_t)K * (N / 32) * 4 + 256 : 4 * n;
}
hipError_t launch_pack(WeightKind kind, int K, int N, const void* B, int ldb, const float* scales, void* panel,
                       hipStream_t s)
{
    const size_t bb = (size_t)(K - 1) * ldb + (kind == W_I4 ? N / 2 : N) * (kind == W_F32 ? 4 : 1);
    const size_t pb = panel_bytes(kind, K, N);
    cpu_hip_enqueue(s, [=] {
        touch(B, bb);
        if (scales) touch(scales, (size_t)K * (N / 32) * 4);
        std::memset(panel, 1, pb);
    });
    return hipSuccess;
}
hipError_t launch_panel_decode(WeightKind kind, int K, int N, const void* panel, float, float* out, hipStream_t s)
{
    const size_t pb = panel_bytes(kind, K, N);
    cpu_hip_enqueue(s, [=] { touch(panel, pb); std::memset(out, 0, (size_t)K * N * 4); });
    return hipSuccess;
}
bool panel_supports(const GemmProblem& p) { return p.panel && p.M >= 1 && p.M <= kSmallMaxM && p.K % 32 == 0; }
int panel_segments(const GemmProblem&) { return 1; }
int panel_phase_k(int) { return 1024; }
bool panel_fuses_out_ln(const GemmProblem&) { return false; }
void panel_tile(const GemmProblem&, int* mb, int* nct) { *mb = 1; *nct = 1; }
bool panel_force_tiles(int, int) { return true; }
bool split_supports(const GemmProblem&) { return false; }
int split_k_segments(WeightKind, int, int, int, size_t) { return 1; }
size_t split_weight_bytes(WeightKind kind, int K, int N)
{
    return kind == W_I8 || K % 32 || N % 32 ? 0 : (size_t)K * N * 4;
}
hipError_t launch_split_pack(WeightKind kind, int K, int N, const void* B, int ldb, const float* scales, void* out,
                             hipStream_t s)
{
    const size_t bb = (size_t)(K - 1) * ldb + (kind == W_I4 ? N / 2 : N * 4);
    cpu_hip_enqueue(s, [=] {
        touch(B, bb);
        if (scales) touch(scales, (size_t)K * (N / 32) * 4);
        std::memset(out, 0, (size_t)K * N * 4);
    });
    return hipSuccess;
}
int dequant_unit_columns(WeightKind kind) { return kind == W_I4 ? 8 : 4; }
hipError_t launch_dequant(WeightKind, int K, int N, const void* B, int ldb, float, const float* scales, bool,
                          float* out, hipStream_t s)
{
    cpu_hip_enqueue(s, [=] {
        touch(B, (size_t)(K - 1) * ldb + 1);
        if (scales) touch(scales, 4);
        std::memset(out, 0, (size_t)K * N * 4);
    });
    return hipSuccess;
}
hipError_t launch_swish(const float* x, float* y, long long n, hipStream_t s)
{
    cpu_hip_enqueue(s, [=] { for (long long i = 0; i < n; ++i) y[i] = x[i]; });
    return hipSuccess;
}

// The GEMM: reads A, the weight (or its panel), the scales and (beta != 0) C,
// then writes C.
hipError_t launch_gemm(const GemmProblem& p, hipStream_t s, int, Tolerance)
{
    if (p.M <= 0 || p.N <= 0) return hipSuccess;
    const GemmProblem q = p;
    cpu_hip_enqueue(s, [q] {
        if (q.K > 0 && q.alpha != 0.0f) {
            touch(q.A, ((size_t)(q.M - 1) * q.lda + q.K) * 4);
            const size_t elem = q.kind == W_F32 ? 4 : 1;
            const size_t cols = q.kind == W_I4 ? (size_t)(q.N + 1) / 2 : (size_t)q.N;
            touch(q.B, ((size_t)(q.K - 1) * q.ldb + cols) * elem);
            if (q.panel) touch(q.panel, panel_bytes(q.kind, q.K, q.N));
            if (q.kind == W_I4) touch(q.scales, int4_scale_count(q.K, q.N) * 4);
        }
        for (int m = 0; m < q.M; ++m)
            for (int n = 0; n < q.N; ++n) {
                float* c = q.C + (size_t)m * q.ldc + n;
                *c = q.beta * *c;
            }
    });
    return hipSuccess;
}

}  // namespace pkgpu
