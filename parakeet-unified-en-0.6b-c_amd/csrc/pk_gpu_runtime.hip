// pk_gpu_runtime.hip - host side of libpk_gpu.so: device selection,
// resident-weight registry, per-thread streams and staging, and the C ABI
// declared in include/pk_gpu.h.
//
// The reference BLAS is called with host pointers from whatever thread runs
// the encoder (csrc/tensor_ops.c:31-61, 579-590; main.c:167-188 runs one
// thread per file).  Here each calling thread owns a HIP stream and a set of
// staging buffers, so concurrent callers never share mutable state except
// the weight registry, which is guarded by a mutex.
#include "pk_gpu.h"
#include "pk_gemm_kernels.h"
#include "pk_gpu_internal.h"

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

using pkgpu::GemmProblem;
using pkgpu::WeightKind;

namespace {

std::mutex g_mu;                 // guards everything below
bool g_inited = false;
int g_device = -1;

// Staging of pk_gpu_gemm_i8_noalloc: a fixed device array that every device
// the library runs on holds until the process ends.  Host code reaches it
// only through its device address, looked up per device at initialisation
// (g_noalloc_base); the array's name is a host-side stand-in.  Calls that use
// it take g_noalloc_mu, one at a time.
constexpr size_t kNoallocBytes = PK_GPU_NOALLOC_BYTES;
static __device__ __align__(256) unsigned char scratch[kNoallocBytes];
constexpr int kMaxDevices = 64;
void* g_noalloc_base[kMaxDevices] = {};  // written at initialisation, under g_mu
std::mutex g_noalloc_mu;

// A registered weight's device copy.  Host-pointer GEMMs hold a reference
// from the lookup (taken under g_mu) until their stream has finished; while
// one does, pk_gpu_unregister_weight refuses (PK_GPU_EBUSY), so the copy is
// freed on the unregistering thread (or at shutdown), after the device's
// queued work.
struct Resident {
    size_t bytes = 0;
    void* dev = nullptr;
    Resident(size_t b, void* d) : bytes(b), dev(d) {}
    Resident(const Resident&) = delete;
    Resident& operator=(const Resident&) = delete;
    ~Resident()
    {
        (void)hipDeviceSynchronize();     // queued device-pointer work may still read it
        (void)hipFree(dev);
    }
};
// host begin -> device copy; never destroyed, so no HIP call runs from a
// static destructor after the runtime has gone
std::map<uintptr_t, std::shared_ptr<Resident>>& g_weights =
    *new std::map<uintptr_t, std::shared_ptr<Resident>>;
size_t g_resident_bytes = 0;

// A weight's panel copy (pk_panel.hip): the layout the small-M kernels read,
// made once from the weight at a device address with the shape and format it
// is multiplied with.  Made by pk_gpu_pack_weight_dev, or by a host-pointer
// GEMM from a registered weight's resident copy (owner: that copy's base;
// unregistering the weight frees its panels).
struct Panel {
    pkgpu::WeightKind kind = pkgpu::W_F32;
    int K = 0, N = 0, ldb = 0;
    const void* scales = nullptr;   // int4: the device scales it was made from
    uintptr_t owner = 0;            // resident copy it was made from (0: a device weight)
    void* dev = nullptr;
    size_t bytes = 0;
    Panel() = default;
    Panel(const Panel&) = delete;
    Panel& operator=(const Panel&) = delete;
    ~Panel() { (void)hipFree(dev); }   // hipFree waits for the device's queued work
};
// weight device address -> its panel; never destroyed (see g_weights)
std::map<uintptr_t, std::shared_ptr<Panel>>& g_panels = *new std::map<uintptr_t, std::shared_ptr<Panel>>;
size_t g_panel_bytes = 0;
// weight device address -> its pre-split copy for the split kernels
// (pk_gpu_presplit_weight_dev; the same record, owner always 0)
std::map<uintptr_t, std::shared_ptr<Panel>>& g_splits = *new std::map<uintptr_t, std::shared_ptr<Panel>>;
size_t g_split_bytes = 0;
std::mutex g_pack_mu;           // one panel made at a time (host-pointer GEMMs)

thread_local std::string t_err;
thread_local int t_force_cfg = -1;
// PK_GPU_NUMERICS_DEFAULT, _EXACT or _FAST for this thread's later calls;
// the environment's PK_GPU_NUMERICS=exact or =fast sets every thread's
// default.
int default_numerics()
{
    const char* e = getenv("PK_GPU_NUMERICS");
    if (e && strcmp(e, "exact") == 0) return PK_GPU_NUMERICS_EXACT;
    if (e && strcmp(e, "fast") == 0) return PK_GPU_NUMERICS_FAST;
    return PK_GPU_NUMERICS_DEFAULT;
}
thread_local int t_numerics = default_numerics();
// pk_gpu_set_workspace: partial tiles of this thread's split-K GEMMs
thread_local float* t_work = nullptr;
thread_local size_t t_work_bytes = 0;

// Per-thread stream and staging buffers (slot 0: A, 1: B, 2: C, 3: scales).
struct ThreadCtx {
    hipStream_t stream = nullptr;
    void* buf[4] = {nullptr, nullptr, nullptr, nullptr};
    size_t cap[4] = {0, 0, 0, 0};
};
// A thread's context goes back to g_free_ctx when the thread exits (no HIP
// call at exit: the stream is idle, since every host-pointer call waits for
// it) and is reused by the next thread that needs one, so threads that come
// and go (one per input file) hold at most as many contexts as ran at once.
std::vector<ThreadCtx*> g_free_ctx;        // guarded by g_mu
struct CtxHolder {
    ThreadCtx* c = nullptr;
    ~CtxHolder()
    {
        if (!c) return;
        std::lock_guard<std::mutex> lk(g_mu);
        g_free_ctx.push_back(c);
    }
};
thread_local CtxHolder t_holder;

void free_ctx(ThreadCtx* c)
{
    (void)hipStreamSynchronize(c->stream);
    for (int i = 0; i < 4; ++i)
        if (c->buf[i]) (void)hipFree(c->buf[i]);
    (void)hipStreamDestroy(c->stream);
    delete c;
}

int fail(int code, const char* fmt, ...)
{
    char msg[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    t_err = msg;
    return code;
}

int hip_fail(hipError_t e, const char* what)
{
    return fail(PK_GPU_EHIP, "%s: %s", what, hipGetErrorString(e));
}

int init_locked(int device)
{
    if (g_inited) return PK_GPU_OK;
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) return fail(PK_GPU_ENODEV, "no HIP device visible");
    if (device < 0) {
        const char* env = getenv("PK_GPU_DEVICE");
        device = env ? atoi(env) : 0;
    }
    if (device >= n) return fail(PK_GPU_ENODEV, "device %d out of range (%d visible)", device, n);
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(PK_GPU_ENODEV, "device %d is %s; this library is built for gfx950 only",
                    device, prop.gcnArchName);
    if (device >= kMaxDevices)
        return fail(PK_GPU_ENODEV, "device %d above the library's %d", device, kMaxDevices);
    // the no-allocation staging array of this device, at its own address
    e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    void* base = nullptr;
    e = hipGetSymbolAddress(&base, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return hip_fail(e, "staging array address");
    g_noalloc_base[device] = base;
    g_device = device;
    g_inited = true;
    return PK_GPU_OK;
}

int ensure_init()
{
    std::lock_guard<std::mutex> lk(g_mu);
    return init_locked(-1);
}

// The calling thread's context; creates it (and binds the device) on first use.
int thread_ctx(ThreadCtx** out)
{
    int rc = ensure_init();
    if (rc) return rc;
    if (!t_holder.c) {
        hipError_t e = hipSetDevice(g_device);
        if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
        ThreadCtx* c = nullptr;
        {
            std::lock_guard<std::mutex> lk(g_mu);
            if (!g_free_ctx.empty()) {
                c = g_free_ctx.back();
                g_free_ctx.pop_back();
            }
        }
        if (!c) {
            c = new ThreadCtx;
            e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
            if (e != hipSuccess) {
                delete c;
                return hip_fail(e, "hipStreamCreate");
            }
        }
        t_holder.c = c;
    }
    *out = t_holder.c;
    return PK_GPU_OK;
}

int staging(ThreadCtx* c, int slot, size_t bytes, void** out)
{
    if (bytes == 0) bytes = 4;
    if (c->cap[slot] < bytes) {
        if (c->buf[slot]) (void)hipFree(c->buf[slot]);
        c->buf[slot] = nullptr;
        c->cap[slot] = 0;
        size_t want = bytes + bytes / 4;                 // grow with headroom
        hipError_t e = hipMalloc(&c->buf[slot], want);
        if (e != hipSuccess) return fail(PK_GPU_ENOMEM, "staging alloc of %zu bytes failed", want);
        c->cap[slot] = want;
    }
    *out = c->buf[slot];
    return PK_GPU_OK;
}

// Device copy of [host, host+need) if the whole range lies in one registered
// weight, else nullptr; *hold (if given) then keeps that copy alive.
const void* resident(const void* host, size_t need, std::shared_ptr<Resident>* hold = nullptr)
{
    if (!host) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    const uintptr_t h = reinterpret_cast<uintptr_t>(host);
    auto it = g_weights.upper_bound(h);
    if (it == g_weights.begin()) return nullptr;
    --it;
    if (h >= it->first && h + need <= it->first + it->second->bytes) {
        if (hold) *hold = it->second;
        return static_cast<const char*>(it->second->dev) + (h - it->first);
    }
    return nullptr;
}

// Host <-> device copy of `rows` rows of `width` bytes at the given pitches.
// From pageable host memory hipMemcpy2DAsync runs at 0.4-2.2 GB/s on MI355X,
// against 18-38 GB/s for one hipMemcpyAsync of the same bytes (1.7-13.6 MB
// operands), so rows that lie back to back on both sides (the reference's
// lda = K, ldc = N) go as one linear copy; strided rows keep the 2D form.
hipError_t copy_rows(void* dst, size_t dpitch, const void* src, size_t spitch, size_t width,
                     int rows, hipMemcpyKind kind, hipStream_t stream)
{
    if (rows <= 0 || width == 0) return hipSuccess;
    if (rows == 1 || (dpitch == width && spitch == width))
        return hipMemcpyAsync(dst, src, width * (size_t)rows, kind, stream);
    return hipMemcpy2DAsync(dst, dpitch, src, spitch, width, (size_t)rows, kind, stream);
}

// Operand rows x cols elements of elem bytes with row pitch ld: either its
// resident copy (keeps pitch ld; *hold keeps it alive) or a packed staged
// copy (pitch cols).
int operand(ThreadCtx* c, int slot, const void* host, int rows, int cols, int ld, size_t elem,
            const void** dev, int* dev_ld, std::shared_ptr<Resident>* hold)
{
    const size_t extent = rows > 0 ? ((size_t)(rows - 1) * ld + cols) * elem : 0;
    if (const void* r = resident(host, extent, hold)) {
        *dev = r;
        *dev_ld = ld;
        return PK_GPU_OK;
    }
    void* d = nullptr;
    int rc = staging(c, slot, (size_t)rows * cols * elem, &d);
    if (rc) return rc;
    if (rows > 0 && cols > 0) {
        hipError_t e = copy_rows(d, (size_t)cols * elem, host, (size_t)ld * elem,
                                 (size_t)cols * elem, rows, hipMemcpyHostToDevice, c->stream);
        if (e != hipSuccess) return hip_fail(e, "operand upload");
    }
    *dev = d;
    *dev_ld = cols;
    return PK_GPU_OK;
}

int check_gemm(int M, int N, int K, int lda, int ldb_min, int ldb, int ldc)
{
    if (M < 0 || N < 0 || K < 0) return fail(PK_GPU_EINVAL, "negative size M=%d N=%d K=%d", M, N, K);
    if (lda < (K > 1 ? K : 1)) return fail(PK_GPU_EINVAL, "lda=%d < K=%d", lda, K);
    if (ldb < (ldb_min > 1 ? ldb_min : 1)) return fail(PK_GPU_EINVAL, "ldb=%d < %d", ldb, ldb_min);
    if (ldc < (N > 1 ? N : 1)) return fail(PK_GPU_EINVAL, "ldc=%d < N=%d", ldc, N);
    return PK_GPU_OK;
}

bool does_multiply(const GemmProblem& p)
{
    return p.M > 0 && p.N > 0 && p.K > 0 && p.alpha != 0.0f &&
           !(p.kind == pkgpu::W_I8 && p.scale == 0.0f);
}

// The panel made from weight p.B with p's format and shape, or null; *hold
// (if given) keeps it alive.
const void* panel_for(const GemmProblem& p, std::shared_ptr<Panel>* hold = nullptr)
{
    if (!p.B) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_panels.find(reinterpret_cast<uintptr_t>(p.B));
    if (it == g_panels.end()) return nullptr;
    const Panel& q = *it->second;
    if (q.kind != p.kind || q.K != p.K || q.N != p.N || q.ldb != p.ldb ||
        (p.kind == pkgpu::W_I4 && q.scales != p.scales))
        return nullptr;
    if (hold) *hold = it->second;
    return q.dev;
}

// The pre-split copy made from weight p.B with p's format and shape, or null.
const void* split_for(const GemmProblem& p)
{
    if (!p.B) return nullptr;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_splits.find(reinterpret_cast<uintptr_t>(p.B));
    if (it == g_splits.end()) return nullptr;
    const Panel& q = *it->second;
    if (q.kind != p.kind || q.K != p.K || q.N != p.N || q.ldb != p.ldb ||
        (p.kind == pkgpu::W_I4 && q.scales != p.scales))
        return nullptr;
    return q.dev;
}

// Whether a call may leave the exact chains (this thread's numerics, no
// forced tile) and has the small-M kernels' shape.
bool small_m_call(const GemmProblem& p, bool tol_ok)
{
    return tol_ok && t_force_cfg < 0 && t_numerics != PK_GPU_NUMERICS_EXACT &&
           p.M > 0 && p.M <= pkgpu::kSmallMaxM;
}

// tol_ok: the call may leave the exact chains as this thread's numerics
// allow (the public GEMM entry points, unless a tile is forced).  The small-M
// kernels read the weight's panel when one was made for it.
int launch(const GemmProblem& p, hipStream_t s, bool tol_ok, std::shared_ptr<Panel>* hold = nullptr)
{
    const pkgpu::Tolerance tol =
        tol_ok && t_force_cfg < 0 ? pkgpu::rt::tolerance_of(t_numerics) : pkgpu::TOL_NONE;
    GemmProblem q = p;
    if (tol != pkgpu::TOL_NONE) {
        q.work = t_work;
        q.work_bytes = t_work_bytes;
    }
    if (small_m_call(p, tol_ok)) q.panel = panel_for(p, hold);
    if (tol == pkgpu::TOL_ALL && p.M > pkgpu::kSmallMaxM) q.b_presplit = split_for(p);
    const hipError_t e = pkgpu::launch_gemm(q, s, t_force_cfg, tol);
    if (e == hipErrorInvalidValue)
        return fail(PK_GPU_EINVAL, "%dx%dx%d GEMM not launched: an operand extent exceeds 2 GiB",
                    p.M, p.N, p.K);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return PK_GPU_OK;
}

// Make the panel of device weight p.B (format, K, N, ldb, scales of p) on
// stream s and register it; owner: the resident copy it lies in (0: none).
// A panel already made for p.B with the same parameters is kept.  The panel
// is complete when this returns (the stream is synchronised).
int make_panel(const GemmProblem& p, uintptr_t owner, hipStream_t s)
{
    const size_t bytes = pkgpu::panel_bytes(p.kind, p.K, p.N);
    if (!bytes) return fail(PK_GPU_EINVAL, "panel: K = %d is not a multiple of 32", p.K);
    auto pn = std::make_shared<Panel>();
    pn->kind = p.kind;
    pn->K = p.K;
    pn->N = p.N;
    pn->ldb = p.ldb;
    pn->scales = p.kind == pkgpu::W_I4 ? p.scales : nullptr;
    pn->owner = owner;
    pn->bytes = bytes;
    hipError_t e = hipMalloc(&pn->dev, bytes);
    if (e != hipSuccess) {
        pn->dev = nullptr;
        return fail(PK_GPU_ENOMEM, "panel: device alloc of %zu bytes failed", bytes);
    }
    e = pkgpu::launch_pack(p.kind, p.K, p.N, p.B, p.ldb, p.scales, pn->dev, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "panel: repack");
    std::lock_guard<std::mutex> lk(g_mu);
    auto& slot = g_panels[reinterpret_cast<uintptr_t>(p.B)];
    if (slot) return fail(PK_GPU_EINVAL, "panel: weight %p already has a panel of another shape", p.B);
    slot = pn;
    g_panel_bytes += bytes;
    return PK_GPU_OK;
}

// The panel of a resident weight, made on first use by a small-M call.
int make_resident_panel(const GemmProblem& p, uintptr_t owner, hipStream_t s)
{
    if (panel_for(p) || !pkgpu::panel_bytes(p.kind, p.K, p.N) || (p.kind == pkgpu::W_I4 && p.N % 32))
        return PK_GPU_OK;
    std::lock_guard<std::mutex> lk(g_pack_mu);
    if (panel_for(p)) return PK_GPU_OK;             // another thread made it meanwhile
    {
        std::lock_guard<std::mutex> lk2(g_mu);
        if (g_panels.count(reinterpret_cast<uintptr_t>(p.B)))
            return PK_GPU_OK;                       // made for another shape: keep the narrow kernels
    }
    return make_panel(p, owner, s);
}

// Host-pointer GEMM: stage what is not resident, run, copy C back, wait.
int host_gemm(GemmProblem p, const float* hA, const void* hB, const float* hScales, float* hC,
              size_t b_elem, int b_cols)
{
    if (p.M == 0 || p.N == 0) return PK_GPU_OK;              // scale_c loops are empty
    const bool mul = does_multiply(p);
    if (!mul && p.beta == 1.0f) return PK_GPU_OK;            // C unchanged
    if (!hC) return fail(PK_GPU_EINVAL, "C is NULL");
    if (mul && (!hA || !hB)) return fail(PK_GPU_EINVAL, "A or B is NULL");
    if (mul && p.kind == pkgpu::W_I4 && !hScales) return fail(PK_GPU_EINVAL, "scales is NULL");

    ThreadCtx* c = nullptr;
    int rc = thread_ctx(&c);
    if (rc) return rc;

    // resident operands stay registered until this call's stream is done
    // (or, on an error return, until the device's queued work is)
    std::shared_ptr<Resident> hold[3];
    if (mul) {
        const void* dA = nullptr;
        int lda = 0;
        rc = operand(c, 0, hA, p.M, p.K, p.lda, sizeof(float), &dA, &lda, &hold[0]);
        if (rc) return rc;
        p.A = static_cast<const float*>(dA);
        p.lda = lda;
        const void* dB = nullptr;
        int ldb = 0;
        rc = operand(c, 1, hB, p.K, b_cols, p.ldb, b_elem, &dB, &ldb, &hold[1]);
        if (rc) return rc;
        p.B = dB;
        p.ldb = ldb;
        if (p.kind == pkgpu::W_I4) {
            const void* dS = nullptr;
            int lds = 0;
            const int ns = (int)pkgpu::int4_scale_count(p.K, p.N);   // one flat run of floats
            rc = operand(c, 3, hScales, 1, ns, ns, sizeof(float), &dS, &lds, &hold[2]);
            if (rc) return rc;
            p.scales = static_cast<const float*>(dS);
        }
    }
    void* dC = nullptr;
    rc = staging(c, 2, (size_t)p.M * p.N * sizeof(float), &dC);
    if (rc) return rc;
    hipError_t e;
    if (p.beta != 0.0f) {
        e = copy_rows(dC, (size_t)p.N * 4, hC, (size_t)p.ldc * 4, (size_t)p.N * 4, p.M,
                      hipMemcpyHostToDevice, c->stream);
        if (e != hipSuccess) return hip_fail(e, "C upload");
    }
    const int ldc_host = p.ldc;
    p.C = static_cast<float*>(dC);
    p.ldc = p.N;
    // a registered weight (and, for int4, registered scales) that the small-M
    // kernels will read gets its panel on first use
    if (mul && hold[1] && (p.kind != pkgpu::W_I4 || hold[2]) && small_m_call(p, true)) {
        rc = make_resident_panel(p, reinterpret_cast<uintptr_t>(hold[1]->dev), c->stream);
        if (rc) return rc;
    }
    std::shared_ptr<Panel> panel_hold;
    rc = launch(p, c->stream, true, &panel_hold);
    if (rc) return rc;
    e = copy_rows(hC, (size_t)ldc_host * 4, dC, (size_t)p.N * 4, (size_t)p.N * 4, p.M,
                  hipMemcpyDeviceToHost, c->stream);
    if (e != hipSuccess) return hip_fail(e, "C download");
    e = hipStreamSynchronize(c->stream);
    if (e != hipSuccess) return hip_fail(e, "stream synchronize");
    return PK_GPU_OK;
}

// host_gemm with every staged operand in the fixed array (no allocation):
// A and C, and B unless its host range is registered, at 256-byte aligned
// offsets, on the caller's stream.  Nothing in the array needs clearing:
// each call uploads what it reads and the GEMM writes all of C.
int noalloc_gemm(GemmProblem p, const float* hA, const void* hB, float* hC, size_t b_elem,
                 int b_cols, hipStream_t s)
{
    if (p.M == 0 || p.N == 0) return PK_GPU_OK;
    const bool mul = does_multiply(p);
    if (!mul && p.beta == 1.0f) return PK_GPU_OK;
    if (!hC) return fail(PK_GPU_EINVAL, "C is NULL");
    if (mul && (!hA || !hB)) return fail(PK_GPU_EINVAL, "A or B is NULL");
    int rc = ensure_init();
    if (rc) return rc;
    unsigned char* base = static_cast<unsigned char*>(g_noalloc_base[g_device]);
    if (!base) return fail(PK_GPU_ENODEV, "no staging array on device %d", g_device);
    int cur = -1;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
    if (cur != g_device && (e = hipSetDevice(g_device)) != hipSuccess) return hip_fail(e, "hipSetDevice");

    // the plan: which operands are staged, and at which offsets
    auto round_up = [](size_t b) { return (b + 255) & ~size_t(255); };
    std::shared_ptr<Resident> hold[2];
    const void* rA = nullptr;
    const void* rB = nullptr;
    if (mul) {
        rA = resident(hA, ((size_t)(p.M - 1) * p.lda + p.K) * sizeof(float), &hold[0]);
        rB = resident(hB, ((size_t)(p.K - 1) * p.ldb + b_cols) * b_elem, &hold[1]);
    }
    const size_t a_bytes = mul && !rA ? (size_t)p.M * p.K * sizeof(float) : 0;
    const size_t b_bytes = mul && !rB ? (size_t)p.K * b_cols * b_elem : 0;
    const size_t c_bytes = (size_t)p.M * p.N * sizeof(float);
    const size_t need = round_up(a_bytes) + round_up(b_bytes) + round_up(c_bytes);
    if (need > kNoallocBytes)
        return fail(PK_GPU_EINVAL, "%dx%dx%d GEMM needs %zu bytes of staging, above the fixed "
                    "array's %zu (PK_GPU_NOALLOC_BYTES)", p.M, p.N, p.K, need, kNoallocBytes);
    unsigned char* dA = base;
    unsigned char* dB = dA + round_up(a_bytes);
    float* dC = reinterpret_cast<float*>(dB + round_up(b_bytes));

    std::lock_guard<std::mutex> lk(g_noalloc_mu);
    if (mul) {
        if (rA) {
            p.A = static_cast<const float*>(rA);
        } else {
            e = copy_rows(dA, (size_t)p.K * 4, hA, (size_t)p.lda * 4, (size_t)p.K * 4, p.M,
                          hipMemcpyHostToDevice, s);
            if (e != hipSuccess) {
                (void)hipStreamSynchronize(s);      // the array is free again when the lock is
                return hip_fail(e, "A upload");
            }
            p.A = reinterpret_cast<const float*>(dA);
            p.lda = p.K;
        }
        if (rB) {
            p.B = rB;
        } else {
            e = copy_rows(dB, (size_t)b_cols * b_elem, hB, (size_t)p.ldb * b_elem,
                          (size_t)b_cols * b_elem, p.K, hipMemcpyHostToDevice, s);
            if (e != hipSuccess) {
                (void)hipStreamSynchronize(s);
                return hip_fail(e, "B upload");
            }
            p.B = dB;
            p.ldb = b_cols;
        }
    }
    if (p.beta != 0.0f) {
        e = copy_rows(dC, (size_t)p.N * 4, hC, (size_t)p.ldc * 4, (size_t)p.N * 4, p.M,
                      hipMemcpyHostToDevice, s);
        if (e != hipSuccess) {
            (void)hipStreamSynchronize(s);
            return hip_fail(e, "C upload");
        }
    }
    const int ldc_host = p.ldc;
    p.C = dC;
    p.ldc = p.N;
    rc = launch(p, s, true);
    if (rc) {
        (void)hipStreamSynchronize(s);              // the array is free again when the lock is
        return rc;
    }
    e = copy_rows(hC, (size_t)ldc_host * 4, dC, (size_t)p.N * 4, (size_t)p.N * 4, p.M,
                  hipMemcpyDeviceToHost, s);
    if (e != hipSuccess) {
        (void)hipStreamSynchronize(s);
        return hip_fail(e, "C download");
    }
    e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "stream synchronize");
    return PK_GPU_OK;
}

// Device-pointer calls enqueue on the caller's stream; NULL is HIP's null
// stream, as in every HIP API.  The calling thread is bound to the device.
hipStream_t pick_stream(void* stream, int* rc)
{
    ThreadCtx* c = nullptr;
    *rc = thread_ctx(&c);
    return static_cast<hipStream_t>(stream);
}

}  // namespace

extern "C" {

int pk_gpu_init(int device)
{
    std::lock_guard<std::mutex> lk(g_mu);
    if (g_inited && device >= 0 && device != g_device)
        return fail(PK_GPU_EINVAL, "already initialised on device %d", g_device);
    return init_locked(device);
}

void pk_gpu_shutdown(void)
{
    std::vector<ThreadCtx*> idle;
    std::map<uintptr_t, std::shared_ptr<Resident>> weights;
    std::map<uintptr_t, std::shared_ptr<Panel>> panels, splits;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        weights.swap(g_weights);
        g_resident_bytes = 0;
        panels.swap(g_panels);
        g_panel_bytes = 0;
        splits.swap(g_splits);
        g_split_bytes = 0;
        idle.swap(g_free_ctx);
    }
    panels.clear();           // each freed after queued work, or by its last holder
    splits.clear();
    weights.clear();
    for (ThreadCtx* c : idle) free_ctx(c);
    if (t_holder.c) {
        free_ctx(t_holder.c);
        t_holder.c = nullptr;
    }
}

const char* pk_gpu_last_error(void) { return t_err.c_str(); }

// Caller holds g_mu.
static bool overlaps_registered(uintptr_t h, size_t bytes)
{
    auto it = g_weights.upper_bound(h);
    if (it != g_weights.end() && it->first < h + bytes) return true;
    if (it != g_weights.begin()) {
        --it;
        if (it->first + it->second->bytes > h) return true;
    }
    return false;
}

int pk_gpu_register_weight(const void* host, size_t bytes)
{
    if (!host || bytes == 0) return fail(PK_GPU_EINVAL, "register: NULL or empty range");
    ThreadCtx* c = nullptr;
    int rc = thread_ctx(&c);
    if (rc) return rc;
    const uintptr_t h = reinterpret_cast<uintptr_t>(host);
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (overlaps_registered(h, bytes))
            return fail(PK_GPU_EINVAL, "register: range overlaps a registered weight");
    }
    // The upload runs unlocked; the overlap test is repeated before insertion
    // in case another thread registered an overlapping range meanwhile.
    void* d = nullptr;
    hipError_t e = hipMalloc(&d, bytes);
    if (e != hipSuccess) return fail(PK_GPU_ENOMEM, "register: device alloc of %zu bytes failed", bytes);
    e = hipMemcpy(d, host, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return hip_fail(e, "register: upload");
    }
    {
        std::lock_guard<std::mutex> lk(g_mu);
        if (!overlaps_registered(h, bytes)) {
            g_weights[h] = std::make_shared<Resident>(bytes, d);
            g_resident_bytes += bytes;
            return PK_GPU_OK;
        }
    }
    (void)hipFree(d);
    return fail(PK_GPU_EINVAL, "register: range overlaps a registered weight");
}

int pk_gpu_unregister_weight(const void* host)
{
    std::shared_ptr<Resident> r;
    std::vector<std::shared_ptr<Panel>> panels;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_weights.find(reinterpret_cast<uintptr_t>(host));
        if (it == g_weights.end()) return fail(PK_GPU_EINVAL, "unregister: not registered");
        // Lookups take their references under g_mu, so no call can start
        // holding it after this test.
        if (it->second.use_count() > 1)
            return fail(PK_GPU_EBUSY, "unregister: a GEMM call on another thread is reading the weight");
        const uintptr_t lo = reinterpret_cast<uintptr_t>(it->second->dev), hi = lo + it->second->bytes;
        for (auto pit = g_panels.lower_bound(lo); pit != g_panels.end() && pit->first < hi;) {
            if (pit->second->owner == lo) {
                g_panel_bytes -= pit->second->bytes;
                panels.push_back(std::move(pit->second));
                pit = g_panels.erase(pit);
            } else {
                ++pit;
            }
        }
        r = std::move(it->second);
        g_resident_bytes -= r->bytes;
        g_weights.erase(it);
    }
    // freed here, after the device's queued work
    panels.clear();
    r.reset();
    return PK_GPU_OK;
}

const void* pk_gpu_device_ptr(const void* host) { return resident(host, 1); }

size_t pk_gpu_resident_bytes(void)
{
    std::lock_guard<std::mutex> lk(g_mu);
    return g_resident_bytes;
}

int pk_gpu_gemm_i8(int M, int N, int K, float alpha, const float* A, int lda,
                   const int8_t* B, float B_scale, int ldb, float beta, float* C, int ldc)
{
    int rc = check_gemm(M, N, K, lda, N, ldb, ldc);
    if (rc) return rc;
    GemmProblem p{pkgpu::W_I8, M, N, K, alpha, beta, nullptr, lda, nullptr, ldb,
                  B_scale, nullptr, nullptr, ldc};
    return host_gemm(p, A, B, nullptr, C, 1, N);
}

int pk_gpu_gemm_i8_noalloc(int M, int N, int K, float alpha, const float* A, int lda,
                           const int8_t* B, float B_scale, int ldb, float beta, float* C, int ldc,
                           void* stream)
{
    int rc = check_gemm(M, N, K, lda, N, ldb, ldc);
    if (rc) return rc;
    GemmProblem p{pkgpu::W_I8, M, N, K, alpha, beta, nullptr, lda, nullptr, ldb,
                  B_scale, nullptr, nullptr, ldc};
    return noalloc_gemm(p, A, B, C, 1, N, static_cast<hipStream_t>(stream));
}

int pk_gpu_gemm_i4(int M, int N, int K, float alpha, const float* A, int lda,
                   const uint8_t* B, const float* scales, int ldb, float beta, float* C, int ldc)
{
    if (N % 2 != 0) return fail(PK_GPU_EINVAL, "int4: N=%d is odd (rows hold N/2 bytes)", N);
    int rc = check_gemm(M, N, K, lda, N / 2, ldb, ldc);
    if (rc) return rc;
    GemmProblem p{pkgpu::W_I4, M, N, K, alpha, beta, nullptr, lda, nullptr, ldb,
                  0.0f, nullptr, nullptr, ldc};
    return host_gemm(p, A, B, scales, C, 1, N / 2);
}

int pk_gpu_sgemm(int transA, int transB, int M, int N, int K, float alpha, const float* A,
                 int lda, const float* B, int ldb, float beta, float* C, int ldc)
{
    if (transA != 111 || transB != 111)
        return fail(PK_GPU_ENOTSUP, "sgemm: only NoTrans/NoTrans (111/111), got %d/%d", transA,
                    transB);
    int rc = check_gemm(M, N, K, lda, N, ldb, ldc);
    if (rc) return rc;
    GemmProblem p{pkgpu::W_F32, M, N, K, alpha, beta, nullptr, lda, nullptr, ldb,
                  0.0f, nullptr, nullptr, ldc};
    return host_gemm(p, A, B, nullptr, C, sizeof(float), N);
}

// Device-pointer entry points; the *_ex forms add the fused epilogue.
static int check_epilogue(const float* bias, int epi, float beta)
{
    if (epi < PK_GPU_EPI_NONE || epi > PK_GPU_EPI_RELU)
        return fail(PK_GPU_EINVAL, "epilogue %d is not one of PK_GPU_EPI_*", epi);
    if ((epi == PK_GPU_EPI_HALF_RESIDUAL || epi == PK_GPU_EPI_RESIDUAL) && beta != 0.0f)
        return fail(PK_GPU_EINVAL, "residual epilogues need beta == 0 (C is the residual)");
    (void)bias;
    return PK_GPU_OK;
}

static int dev_gemm(GemmProblem p, const float* dbias, int epi, void* stream)
{
    int rc = check_epilogue(dbias, epi, p.beta);
    if (rc) return rc;
    // A NULL device operand would become a buffer descriptor at address 0.
    if (p.M > 0 && p.N > 0 && !p.C) return fail(PK_GPU_EINVAL, "C is NULL");
    if (does_multiply(p) &&
        (!p.A || !p.B || (p.kind == pkgpu::W_I4 && !p.scales)))
        return fail(PK_GPU_EINVAL, "A, B or scales is NULL");
    hipStream_t s = pick_stream(stream, &rc);
    if (rc) return rc;
    p.bias = dbias;
    p.epi = static_cast<pkgpu::Epilogue>(epi);
    return launch(p, s, true);
}

int pk_gpu_gemm_i8_ex_dev(int M, int N, int K, float alpha, const float* dA, int lda,
                          const int8_t* dB, float B_scale, int ldb, float beta, float* dC, int ldc,
                          const float* dbias, int epilogue, void* stream)
{
    int rc = check_gemm(M, N, K, lda, N, ldb, ldc);
    if (rc) return rc;
    GemmProblem p{pkgpu::W_I8, M, N, K, alpha, beta, dA, lda, dB, ldb, B_scale, nullptr, dC, ldc};
    return dev_gemm(p, dbias, epilogue, stream);
}

int pk_gpu_gemm_i4_ex_dev(int M, int N, int K, float alpha, const float* dA, int lda,
                          const uint8_t* dB, const float* dscales, int ldb, float beta, float* dC,
                          int ldc, const float* dbias, int epilogue, void* stream)
{
    if (N % 2 != 0) return fail(PK_GPU_EINVAL, "int4: N=%d is odd (rows hold N/2 bytes)", N);
    int rc = check_gemm(M, N, K, lda, N / 2, ldb, ldc);
    if (rc) return rc;
    GemmProblem p{pkgpu::W_I4, M, N, K, alpha, beta, dA, lda, dB, ldb, 0.0f, dscales, dC, ldc};
    return dev_gemm(p, dbias, epilogue, stream);
}

int pk_gpu_sgemm_ex_dev(int M, int N, int K, float alpha, const float* dA, int lda,
                        const float* dB, int ldb, float beta, float* dC, int ldc,
                        const float* dbias, int epilogue, void* stream)
{
    int rc = check_gemm(M, N, K, lda, N, ldb, ldc);
    if (rc) return rc;
    GemmProblem p{pkgpu::W_F32, M, N, K, alpha, beta, dA, lda, dB, ldb, 0.0f, nullptr, dC, ldc};
    return dev_gemm(p, dbias, epilogue, stream);
}

int pk_gpu_gemm_i8_dev(int M, int N, int K, float alpha, const float* dA, int lda,
                       const int8_t* dB, float B_scale, int ldb, float beta, float* dC, int ldc,
                       void* stream)
{
    return pk_gpu_gemm_i8_ex_dev(M, N, K, alpha, dA, lda, dB, B_scale, ldb, beta, dC, ldc,
                                 nullptr, PK_GPU_EPI_NONE, stream);
}

int pk_gpu_gemm_i4_dev(int M, int N, int K, float alpha, const float* dA, int lda,
                       const uint8_t* dB, const float* dscales, int ldb, float beta, float* dC,
                       int ldc, void* stream)
{
    return pk_gpu_gemm_i4_ex_dev(M, N, K, alpha, dA, lda, dB, dscales, ldb, beta, dC, ldc,
                                 nullptr, PK_GPU_EPI_NONE, stream);
}

int pk_gpu_sgemm_dev(int M, int N, int K, float alpha, const float* dA, int lda, const float* dB,
                     int ldb, float beta, float* dC, int ldc, void* stream)
{
    return pk_gpu_sgemm_ex_dev(M, N, K, alpha, dA, lda, dB, ldb, beta, dC, ldc, nullptr,
                               PK_GPU_EPI_NONE, stream);
}

int pk_gpu_swish_dev(const float* dx, float* dy, long long n, void* stream)
{
    if (n < 0 || (n > 0 && (!dx || !dy))) return fail(PK_GPU_EINVAL, "swish: bad arguments");
    int rc = 0;
    hipStream_t s = pick_stream(stream, &rc);
    if (rc) return rc;
    hipError_t e = pkgpu::launch_swish(dx, dy, n, s);
    return e == hipSuccess ? PK_GPU_OK : hip_fail(e, "swish launch");
}

static pkgpu::WeightKind kind_of_bits(int bits)
{
    return bits == 4 ? pkgpu::W_I4 : bits == 8 ? pkgpu::W_I8 : pkgpu::W_F32;
}

int pk_gpu_pack_weight_dev(int bits, int K, int N, const void* dB, int ldb, const float* dscales,
                           void* stream)
{
    if (bits != 4 && bits != 8 && bits != 32) return fail(PK_GPU_EINVAL, "pack: bits = %d (4, 8 or 32)", bits);
    if (K <= 0 || N <= 0 || K % 32) return fail(PK_GPU_EINVAL, "pack: K = %d (a positive multiple of 32), N = %d", K, N);
    if (bits == 4 && N % 32) return fail(PK_GPU_EINVAL, "pack: int4 N = %d is not a multiple of 32", N);
    if (ldb < (bits == 4 ? N / 2 : N)) return fail(PK_GPU_EINVAL, "pack: ldb = %d too small for N = %d", ldb, N);
    if (!dB || (bits == 4 && !dscales)) return fail(PK_GPU_EINVAL, "pack: NULL operand");
    int rc = 0;
    hipStream_t s = pick_stream(stream, &rc);
    if (rc) return rc;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
        return fail(PK_GPU_EINVAL, "pack: not during stream capture (it allocates and waits)");
    GemmProblem p{};
    p.kind = kind_of_bits(bits);
    p.K = K; p.N = N; p.B = dB; p.ldb = ldb;
    p.scales = bits == 4 ? dscales : nullptr;
    if (panel_for(p)) return PK_GPU_OK;              // already made with these parameters
    std::lock_guard<std::mutex> lk(g_pack_mu);
    return make_panel(p, 0, s);
}

int pk_gpu_unpack_weight_dev(const void* dB)
{
    std::shared_ptr<Panel> pn;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_panels.find(reinterpret_cast<uintptr_t>(dB));
        if (it == g_panels.end()) return fail(PK_GPU_EINVAL, "unpack: no panel for %p", dB);
        if (it->second->owner)
            return fail(PK_GPU_EINVAL, "unpack: the panel of a registered weight goes with pk_gpu_unregister_weight");
        if (it->second.use_count() > 1)
            return fail(PK_GPU_EBUSY, "unpack: a GEMM call on another thread is reading the panel");
        pn = std::move(it->second);
        g_panel_bytes -= pn->bytes;
        g_panels.erase(it);
    }
    pn.reset();                                      // freed after the device's queued work
    return PK_GPU_OK;
}

int pk_gpu_presplit_weight_dev(int bits, int K, int N, const void* dB, int ldb, const float* dscales,
                               void* stream)
{
    if (bits != 4 && bits != 8 && bits != 32) return fail(PK_GPU_EINVAL, "presplit: bits = %d (4, 8 or 32)", bits);
    if (K <= 0 || N <= 0 || K % 32 || N % 32)
        return fail(PK_GPU_EINVAL, "presplit: K = %d and N = %d must be positive multiples of 32", K, N);
    if (ldb < (bits == 4 ? N / 2 : N)) return fail(PK_GPU_EINVAL, "presplit: ldb = %d too small for N = %d", ldb, N);
    if (!dB || (bits == 4 && !dscales)) return fail(PK_GPU_EINVAL, "presplit: NULL operand");
    int rc = 0;
    hipStream_t s = pick_stream(stream, &rc);
    if (rc) return rc;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cap) == hipSuccess && cap != hipStreamCaptureStatusNone)
        return fail(PK_GPU_EINVAL, "presplit: not during stream capture (it allocates and waits)");
    GemmProblem p{};
    p.kind = kind_of_bits(bits);
    p.K = K; p.N = N; p.B = dB; p.ldb = ldb;
    p.scales = bits == 4 ? dscales : nullptr;
    if (split_for(p)) return PK_GPU_OK;              // already made with these parameters
    std::lock_guard<std::mutex> lk(g_pack_mu);
    if (split_for(p)) return PK_GPU_OK;
    const size_t bytes = pkgpu::split_weight_bytes(p.kind, K, N);
    if (bytes >= ((size_t)1 << 31)) return fail(PK_GPU_EINVAL, "presplit: %zu bytes exceed 2 GiB", bytes);
    auto pn = std::make_shared<Panel>();
    pn->kind = p.kind;
    pn->K = K;
    pn->N = N;
    pn->ldb = ldb;
    pn->scales = p.scales;
    pn->bytes = bytes;
    hipError_t e = hipMalloc(&pn->dev, bytes);
    if (e != hipSuccess) {
        pn->dev = nullptr;
        return fail(PK_GPU_ENOMEM, "presplit: device alloc of %zu bytes failed", bytes);
    }
    e = pkgpu::launch_split_pack(p.kind, K, N, dB, ldb, p.scales, pn->dev, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "presplit: pack");
    std::lock_guard<std::mutex> lk2(g_mu);
    auto& slot = g_splits[reinterpret_cast<uintptr_t>(dB)];
    if (slot) return fail(PK_GPU_EINVAL, "presplit: weight %p already has a copy of another shape", dB);
    slot = pn;
    g_split_bytes += bytes;
    return PK_GPU_OK;
}

int pk_gpu_unsplit_weight_dev(const void* dB)
{
    std::shared_ptr<Panel> pn;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        auto it = g_splits.find(reinterpret_cast<uintptr_t>(dB));
        if (it == g_splits.end()) return fail(PK_GPU_EINVAL, "unsplit: no pre-split copy of %p", dB);
        pn = std::move(it->second);
        g_split_bytes -= pn->bytes;
        g_splits.erase(it);
    }
    pn.reset();                                      // freed after the device's queued work
    return PK_GPU_OK;
}

size_t pk_gpu_presplit_bytes(void)
{
    std::lock_guard<std::mutex> lk(g_mu);
    return g_split_bytes;
}

size_t pk_gpu_panel_bytes(void)
{
    std::lock_guard<std::mutex> lk(g_mu);
    return g_panel_bytes;
}

int pk_gpu_uses_panel(int M, int N, int K, int bits, const void* dB, int ldb, const float* dscales)
{
    GemmProblem p{};
    p.kind = kind_of_bits(bits);
    p.M = M; p.N = N; p.K = K;
    p.alpha = 1.0f; p.scale = 1.0f;
    p.A = reinterpret_cast<const float*>(uintptr_t(256));
    p.lda = K;
    p.B = dB; p.ldb = ldb;
    p.scales = dscales;
    p.ldc = N;
    if (!small_m_call(p, true)) return 0;
    p.panel = panel_for(p);
    return pkgpu::panel_supports(p);
}

int pk_gpu_panel_segments(int M, int N, int K)
{
    GemmProblem p{};
    p.M = M; p.N = N; p.K = K;
    p.work = t_work;
    p.work_bytes = t_work_bytes;
    return pkgpu::panel_segments(p);
}

int pk_gpu_panel_decode_dev(int bits, int K, int N, const void* dB, int ldb, const float* dscales,
                            float B_scale, float* dout, void* stream)
{
    GemmProblem p{};
    p.kind = kind_of_bits(bits);
    p.K = K; p.N = N; p.B = dB; p.ldb = ldb;
    p.scales = bits == 4 ? dscales : nullptr;
    const void* pn = panel_for(p);
    if (!pn) return fail(PK_GPU_EINVAL, "decode: no panel for %p with these parameters", dB);
    if (!dout) return fail(PK_GPU_EINVAL, "decode: NULL output");
    int rc = 0;
    hipStream_t s = pick_stream(stream, &rc);
    if (rc) return rc;
    const hipError_t e = pkgpu::launch_panel_decode(p.kind, K, N, pn, B_scale, dout, s);
    return e == hipSuccess ? PK_GPU_OK : hip_fail(e, "panel decode launch");
}

int pk_gpu_force_panel_tile(int mb, int nct)
{
    if (!pkgpu::panel_force_tiles(mb, nct))
        return fail(PK_GPU_EINVAL, "panel tile mb = %d, nct = %d (mb 1..4, nct 1..2; (0, 0) = default)", mb, nct);
    return PK_GPU_OK;
}

int pk_gpu_num_configs(void) { return pkgpu::num_configs(); }

int pk_gpu_config_info(int index, int* family, int* mfma, int* cw, int* wgm, int* wgn, int* kt)
{
    if (index < 0 || index >= pkgpu::num_configs()) return fail(PK_GPU_EINVAL, "no config %d", index);
    pkgpu::TileConfig t = pkgpu::config_at(index);
    if (family) *family = t.family;
    if (kt) *kt = t.kt;
    if (mfma) *mfma = t.mfma;
    if (cw) *cw = t.cw;
    if (wgm) *wgm = t.wgm;
    if (wgn) *wgn = t.wgn;
    return PK_GPU_OK;
}

int pk_gpu_pick_config(int M, int N, int K) { return pkgpu::choose_config_index(M, N, K, pkgpu::W_I8); }

int pk_gpu_pick_config_bits(int M, int N, int K, int bits)
{
    switch (bits) {
    case 4: return pkgpu::choose_config_index(M, N, K, pkgpu::W_I4);
    case 8: return pkgpu::choose_config_index(M, N, K, pkgpu::W_I8);
    case 32: return pkgpu::choose_config_index(M, N, K, pkgpu::W_F32);
    default: return -1;
    }
}

int pk_gpu_force_config(int index)
{
    if (index >= pkgpu::num_configs()) return fail(PK_GPU_EINVAL, "no config %d", index);
    t_force_cfg = index < 0 ? -1 : index;
    return PK_GPU_OK;
}

int pk_gpu_set_numerics(int mode)
{
    if (mode != PK_GPU_NUMERICS_DEFAULT && mode != PK_GPU_NUMERICS_EXACT &&
        mode != PK_GPU_NUMERICS_FAST)
        return fail(PK_GPU_EINVAL, "numerics mode %d is not one of PK_GPU_NUMERICS_*", mode);
    t_numerics = mode;
    return PK_GPU_OK;
}

int pk_gpu_get_numerics(void) { return t_numerics; }

int pk_gpu_set_workspace(void* dwork, size_t bytes)
{
    if (dwork && reinterpret_cast<uintptr_t>(dwork) % 16)
        return fail(PK_GPU_EINVAL, "workspace %p is not 16-byte aligned", dwork);
    t_work = dwork ? static_cast<float*>(dwork) : nullptr;
    t_work_bytes = dwork ? bytes : 0;
    return PK_GPU_OK;
}

int pk_gpu_split_k_segments(int M, int N, int K, int bits)
{
    const pkgpu::WeightKind kind = bits == 4 ? pkgpu::W_I4 : bits == 8 ? pkgpu::W_I8 : pkgpu::W_F32;
    return pkgpu::split_k_segments(kind, M, N, K, t_work ? t_work_bytes : 0);
}

int pk_gpu_dequant_dev(int bits, int K, int N, const void* dB, int ldb, float scale,
                       const float* dscales, int unit_path, float* dout, void* stream)
{
    if (bits != 4 && bits != 8 && bits != 32) return fail(PK_GPU_EINVAL, "bits = %d (4, 8 or 32)", bits);
    if (K < 0 || N < 0) return fail(PK_GPU_EINVAL, "K = %d, N = %d", K, N);
    if (K == 0 || N == 0) return PK_GPU_OK;
    const pkgpu::WeightKind kind = bits == 4 ? pkgpu::W_I4 : bits == 8 ? pkgpu::W_I8 : pkgpu::W_F32;
    if (bits == 4 && N % 2) return fail(PK_GPU_EINVAL, "int4: N = %d is odd", N);
    if (ldb < (bits == 4 ? N / 2 : N)) return fail(PK_GPU_EINVAL, "ldb = %d too small for N = %d", ldb, N);
    if (unit_path && N % pkgpu::dequant_unit_columns(kind))
        return fail(PK_GPU_EINVAL, "unit path: N = %d is not a multiple of %d", N,
                    pkgpu::dequant_unit_columns(kind));
    if (!dB || !dout || (bits == 4 && !dscales)) return fail(PK_GPU_EINVAL, "NULL operand");
    // the unit path's vector loads need what the kernels require before taking it
    const uintptr_t pb = reinterpret_cast<uintptr_t>(dB);
    if (unit_path && (ldb % 4 || pb % (bits == 32 ? 16 : 4)))
        return fail(PK_GPU_EINVAL, "unit path: weight rows not aligned for vector loads");
    int rc = 0;
    hipStream_t s = pick_stream(stream, &rc);
    if (rc) return rc;
    const hipError_t e = pkgpu::launch_dequant(kind, K, N, dB, ldb, scale, dscales, unit_path != 0,
                                               dout, s);
    if (e == hipErrorInvalidValue) return fail(PK_GPU_EINVAL, "weight extent exceeds 2 GiB");
    if (e != hipSuccess) return hip_fail(e, "dequant launch");
    return PK_GPU_OK;
}

int pk_gpu_force_small_tile(int rb, int nct)
{
    if (!pkgpu::smallm_force_tile(rb, nct))
        return fail(PK_GPU_EINVAL, "small-M tile rb = %d, nct = %d (rb 1..4, nct 1..2, rb * nct <= 4)", rb, nct);
    return PK_GPU_OK;
}

int pk_gpu_uses_small_m(int M, int N, int K, int bits)
{
    GemmProblem p{};
    p.kind = bits == 4 ? pkgpu::W_I4 : bits == 8 ? pkgpu::W_I8 : pkgpu::W_F32;
    p.M = M; p.N = N; p.K = K;
    p.alpha = 1.0f; p.scale = 1.0f;
    p.A = reinterpret_cast<const float*>(uintptr_t(256));
    p.B = reinterpret_cast<const void*>(uintptr_t(256));
    p.scales = reinterpret_cast<const float*>(uintptr_t(256));
    p.lda = K; p.ldb = bits == 4 ? N / 2 : N; p.ldc = N;
    return t_numerics != PK_GPU_NUMERICS_EXACT && t_force_cfg < 0 && pkgpu::smallm_supports(p);
}

int pk_gpu_uses_split(int M, int N, int K, int bits)
{
    GemmProblem p{};
    p.kind = bits == 4 ? pkgpu::W_I4 : bits == 8 ? pkgpu::W_I8 : pkgpu::W_F32;
    p.M = M; p.N = N; p.K = K;
    p.alpha = 1.0f; p.scale = 1.0f;
    p.A = reinterpret_cast<const float*>(uintptr_t(256));
    p.B = reinterpret_cast<const void*>(uintptr_t(256));
    p.scales = reinterpret_cast<const float*>(uintptr_t(256));
    p.lda = K; p.ldb = bits == 4 ? N / 2 : N; p.ldc = N;
    return t_numerics == PK_GPU_NUMERICS_FAST && t_force_cfg < 0 && !pkgpu::smallm_supports(p) &&
           pkgpu::split_supports(p);
}

}  // extern "C"

// Hooks for the other host translation units (pk_gpu_internal.h).
namespace pkgpu {
namespace rt {

int error(int code, const char* fmt, ...)
{
    char msg[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(msg, sizeof msg, fmt, ap);
    va_end(ap);
    t_err = msg;
    return code;
}

int hip_error(hipError_t e, const char* what) { return hip_fail(e, what); }

int bind(hipStream_t* thread_stream)
{
    ThreadCtx* c = nullptr;
    int rc = thread_ctx(&c);
    if (rc) return rc;
    if (thread_stream) *thread_stream = c->stream;
    return PK_GPU_OK;
}

Tolerance tolerance_of(int numerics)
{
    return numerics == PK_GPU_NUMERICS_DEFAULT ? TOL_SMALL_M
         : numerics == PK_GPU_NUMERICS_FAST    ? TOL_ALL
                                               : TOL_NONE;
}

int gemm(const GemmProblem& p, hipStream_t s, Tolerance tol)
{
    // the caller's choice of numerics; a forced tile still implies exact chains
    const hipError_t e = pkgpu::launch_gemm(p, s, t_force_cfg, t_force_cfg < 0 ? tol : TOL_NONE);
    if (e == hipErrorInvalidValue)
        return fail(PK_GPU_EINVAL, "%dx%dx%d GEMM not launched: an operand extent exceeds 2 GiB",
                    p.M, p.N, p.K);
    if (e != hipSuccess) return hip_fail(e, "kernel launch");
    return PK_GPU_OK;
}

int forced_config() { return t_force_cfg; }

}  // namespace rt
}  // namespace pkgpu
