"""GPU: the split kernels (pk_split.hip), which GEMMs with M > 64 take under
PK_GPU_NUMERICS_FAST (pk_gpu_set_numerics).

The reference computes every output as one fp32 fma chain over k
(blas.c:187-218, 759-771, 950-963).  These kernels take the same products
(activations split into two bf16 halves; int8 and int4 codes exact, int4
weights dequantised exactly as blas.c:834-840 does and then split, fp32
weights split) through v_mfma_f32_32x32x16_bf16 with fp32 accumulators, in
another, fixed order.  The contract is max |C - R| / max |R| <= 1e-3 against
the oracle R (bit-identical to the reference, test_oracle.py); the tests
also hold the measured error below 1e-4, so a lost term, a wrong scale
group, nibble or output position fails them.  Each of the five launch shapes
(workgroup tiles of 256 x 128, 128 x 128 and 128 x 64; 64 x 64 with K split over 4
waves and summed in LDS, also with chunk counts that do not divide by 4;
64 x 64 on one wave) is taken by some of the shapes below; rows and columns
past M and N, alpha, beta and the fused epilogues are covered, and results
are deterministic.

With a workspace (pk_gpu_set_workspace), shapes with fewer 128 x 128 tiles
than CUs split K over workgroups: 256 x 128 or 128 x 128 tiles, partial tiles
summed in segment order by a second launch.  The same bounds hold there, on
shapes with 2 to 16 segments, with chunk counts that do not divide evenly, and
with partial row and column tiles."""
import numpy as np
import pytest

import pyoracle as po
from pkgpu import Dev, bits_equal, gpu_available, pk
from test_gpu_gemm import make, oracle

pytestmark = pytest.mark.gpu

CONTRACT, MEASURED = 1e-3, 1e-4
#                      launch shape the shape takes (256 x 128 when tiles of
#                      128 x 128 > 256; 128 x 128 at exactly 256; else 128 x 64
#                      when >= 256 of them; else 64 x 64 with K over 4 waves
#                      when K >= 256, else 64 x 64 on one wave)
SHAPES = [("i4", 1656, 4096, 96),     # 256 x 128 (more than 256 tiles of 128 x 128)
          ("i8", 1600, 3072, 64),     # partial last row tile
          ("f32", 1100, 4160, 64),    # partial last column tile
          ("i8", 1024, 4096, 256),    # 128 x 128: 8 x 32 tiles
          ("i4", 1024, 4096, 256),
          ("f32", 1024, 4096, 128),
          ("i8", 1024, 2048, 128),    # 128 x 64: 8 x 32 tiles
          ("i4", 1000, 2048, 160),    # partial last row tile
          ("f32", 1024, 2048, 96),
          ("i8", 416, 3072, 1024),    # K over 4 waves: the QKV of one 416-row chunk
          ("i4", 416, 4096, 1024),    # feed-forward up and down of one chunk
          ("i4", 375, 1024, 4096),
          ("f32", 416, 2048, 1024),   # pointwise 1
          ("i8", 300, 512, 1056),     # 33 chunks: waves take 8, 8, 8 and 9
          ("f32", 130, 256, 320),     # 10 chunks: 2, 3, 2, 3
          ("i4", 97, 96, 288),
          ("i8", 65, 96, 64), ("i4", 130, 160, 224), ("f32", 77, 32, 32), ("i8", 200, 1056, 32)]


@pytest.fixture(scope="module")
def dev():
    if not gpu_available():
        pytest.skip("no GPU")
    return Dev()


def bits_of(kind):
    return {"i4": 4, "i8": 8, "f32": 32}[kind]


def rel_err(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


def fast(dev, kind, A, W, extra, C0, alpha=1.0, beta=0.0, bias=None, epi=None):
    kw = {"scales": extra} if kind == "i4" else {"scale": extra} if kind == "i8" else {}
    return dev.gemm(kind, A, W, C0, alpha, beta, bias=bias, epi=epi, numerics=pk.NUMERICS_FAST, **kw)


def uses_split(M, N, K, bits):
    lib = pk.load()
    prev = lib.pk_gpu_get_numerics()
    pk.call("pk_gpu_set_numerics", pk.NUMERICS_FAST)
    try:
        return lib.pk_gpu_uses_split(M, N, K, bits)
    finally:
        pk.call("pk_gpu_set_numerics", prev)


@pytest.mark.parametrize("kind,M,N,K", SHAPES)
def test_split_within_tolerance(dev, kind, M, N, K):
    assert uses_split(M, N, K, bits_of(kind)) == 1
    A, W, extra, _ = make(kind, M, N, K, f"sp.{kind}.{M}.{N}.{K}")
    Z = np.zeros((M, N), np.float32)
    want = oracle(kind, A, W, extra, Z)
    got = fast(dev, kind, A, W, extra, Z)
    e = rel_err(got, want)
    print(f"{kind} {M}x{N}x{K}: max|C - R| / max|R| = {e:.3g}", flush=True)
    assert e <= CONTRACT and e <= MEASURED, e
    assert bits_equal(fast(dev, kind, A, W, extra, Z), got), "not deterministic"


@pytest.mark.parametrize("kind", ["i8", "i4", "f32"])
def test_split_alpha_beta_and_epilogues(dev, kind):
    M, N, K = 200, 256, 512
    A, W, extra, C0 = make(kind, M, N, K, f"spepi.{kind}")
    bias = po.normal((N,), 0.0, 0.02, po.seed(0x5EED3000, f"spepi.{kind}.b"))
    Z = np.zeros((M, N), np.float32)
    plain = oracle(kind, A, W, extra, Z)
    for alpha, beta in [(0.75, 0.5), (1.0, 1.0), (-2.0, 0.0)]:
        want = oracle(kind, A, W, extra, C0, alpha, beta)
        assert rel_err(fast(dev, kind, A, W, extra, C0, alpha, beta), want) <= MEASURED, (alpha, beta)
    biased = (plain + bias[None, :]).astype(np.float32)
    cases = {
        pk.EPI_NONE: biased,
        pk.EPI_SWISH: po.swish(biased),
        pk.EPI_HALF_RESIDUAL: (C0 + np.float32(0.5) * biased).astype(np.float32),
        pk.EPI_RESIDUAL: (C0 + biased).astype(np.float32),
        4: np.maximum(biased, 0.0),                                   # EPI_RELU
    }
    for epi, want in cases.items():
        C_in = C0 if epi in (pk.EPI_HALF_RESIDUAL, pk.EPI_RESIDUAL) else Z
        got = fast(dev, kind, A, W, extra, C_in, 1.0, 0.0, bias=bias, epi=epi)
        assert rel_err(got, want) <= MEASURED, f"epilogue {epi}"


def test_split_dispatch_rules(dev):
    """FAST sends M <= 64 to the small-M kernels and other suitable shapes
    here; DEFAULT and EXACT never take these kernels, a forced tile
    configuration means exact chains, and shapes outside the rules (N or K
    not a multiple of 32) stay exact."""
    lib = pk.load()
    assert uses_split(33, 3072, 1024, 8) == 0 and uses_split(65, 3072, 1024, 8) == 1
    assert uses_split(1656, 1000, 1024, 8) == 0          # N % 32
    assert uses_split(1656, 1024, 1000, 32) == 0          # K % 32
    for mode in (pk.NUMERICS_DEFAULT, pk.NUMERICS_EXACT):
        prev = lib.pk_gpu_get_numerics()
        pk.call("pk_gpu_set_numerics", mode)
        try:
            assert lib.pk_gpu_uses_split(1656, 4096, 1024, 4) == 0
        finally:
            pk.call("pk_gpu_set_numerics", prev)
    pk.call("pk_gpu_force_config", 20)
    try:
        assert uses_split(1656, 4096, 1024, 4) == 0
    finally:
        pk.call("pk_gpu_force_config", -1)
    assert lib.pk_gpu_set_numerics(3) == -1


def test_split_shapes_outside_rules_stay_exact(dev):
    """N not a multiple of 32 under FAST: the exact chains, bit for bit."""
    M, N, K = 200, 1000, 256
    A, W, extra, _ = make("i8", M, N, K, "spx")
    Z = np.zeros((M, N), np.float32)
    assert bits_equal(fast(dev, "i8", A, W, extra, Z), oracle("i8", A, W, extra, Z))


#                          segments of K with a 32 MiB workspace
SPLIT_K = [("i4", 1656, 1024, 4096, 4),    # feed-forward down of a 1656-row group
           ("i8", 1656, 1024, 2048, 4),
           ("f32", 1656, 2048, 1024, 2),   # pointwise 1
           ("f32", 1656, 1024, 1024, 4),   # pointwise 2
           ("i4", 375, 1024, 4096, 10),    # 128 x 128 tiles (256-row tiles pad too much)
           ("i4", 300, 2048, 2048, 5),
           ("f32", 500, 1024, 4096, 16),
           ("f32", 500, 4096, 1024, 4),
           ("i8", 300, 512, 2080, 16),     # 65 chunks over 16 segments
           ("i4", 97, 96, 2336, 18),       # one partial tile, 73 chunks
           ("f32", 130, 256, 320, 2)]


class Workspace:
    """pk_gpu_set_workspace on this thread for the duration of a with-block."""

    def __init__(self, dev, nbytes=pk.SPLIT_WORKSPACE_BYTES):
        import torch
        self.buf = torch.empty(nbytes // 4, dtype=torch.float32, device=dev.dev)
        self.nbytes = nbytes

    def __enter__(self):
        pk.call("pk_gpu_set_workspace", self.buf.data_ptr(), self.nbytes)
        return self

    def __exit__(self, *exc):
        pk.call("pk_gpu_set_workspace", None, 0)


@pytest.mark.parametrize("kind,M,N,K,segs", SPLIT_K)
def test_split_k_within_tolerance(dev, kind, M, N, K, segs):
    lib = pk.load()
    A, W, extra, _ = make(kind, M, N, K, f"spk.{kind}.{M}.{N}.{K}")
    Z = np.zeros((M, N), np.float32)
    want = oracle(kind, A, W, extra, Z)
    assert lib.pk_gpu_split_k_segments(M, N, K, bits_of(kind)) == 1
    with Workspace(dev):
        assert lib.pk_gpu_split_k_segments(M, N, K, bits_of(kind)) == segs
        got = fast(dev, kind, A, W, extra, Z)
        again = fast(dev, kind, A, W, extra, Z)
    e = rel_err(got, want)
    print(f"{kind} {M}x{N}x{K}, {segs} segments: max|C - R| / max|R| = {e:.3g}", flush=True)
    assert e <= CONTRACT and e <= MEASURED, e
    assert bits_equal(again, got), "not deterministic"


@pytest.mark.parametrize("kind", ["i8", "i4", "f32"])
def test_split_k_alpha_beta_and_epilogues(dev, kind):
    """alpha, beta, bias and every epilogue are applied once, after the
    partial tiles are summed (16 segments of 256 x 128 tiles here)."""
    lib = pk.load()
    M, N, K = 200, 256, 2048
    A, W, extra, C0 = make(kind, M, N, K, f"spkepi.{kind}")
    bias = po.normal((N,), 0.0, 0.02, po.seed(0x5EED3000, f"spkepi.{kind}.b"))
    Z = np.zeros((M, N), np.float32)
    plain = oracle(kind, A, W, extra, Z)
    biased = (plain + bias[None, :]).astype(np.float32)
    cases = {
        pk.EPI_NONE: biased,
        pk.EPI_SWISH: po.swish(biased),
        pk.EPI_HALF_RESIDUAL: (C0 + np.float32(0.5) * biased).astype(np.float32),
        pk.EPI_RESIDUAL: (C0 + biased).astype(np.float32),
        4: np.maximum(biased, 0.0),                                   # EPI_RELU
    }
    with Workspace(dev):
        assert lib.pk_gpu_split_k_segments(M, N, K, bits_of(kind)) == 16
        for alpha, beta in [(0.75, 0.5), (1.0, 1.0), (-2.0, 0.0)]:
            want = oracle(kind, A, W, extra, C0, alpha, beta)
            assert rel_err(fast(dev, kind, A, W, extra, C0, alpha, beta), want) <= MEASURED, (alpha, beta)
        for epi, want in cases.items():
            C_in = C0 if epi in (pk.EPI_HALF_RESIDUAL, pk.EPI_RESIDUAL) else Z
            got = fast(dev, kind, A, W, extra, C_in, 1.0, 0.0, bias=bias, epi=epi)
            assert rel_err(got, want) <= MEASURED, f"epilogue {epi}"


def test_split_k_workspace_rules(dev):
    """A workspace smaller than PK_GPU_SPLIT_WORKSPACE_BYTES is not used (the
    GEMM still runs, without split-K), a misaligned one is refused, and
    DEFAULT numerics never touch it."""
    lib = pk.load()
    M, N, K = 375, 1024, 4096
    A, W, extra, _ = make("i4", M, N, K, "spkrule")
    Z = np.zeros((M, N), np.float32)
    want = oracle("i4", A, W, extra, Z)
    with Workspace(dev, pk.SPLIT_WORKSPACE_BYTES - 4096) as ws:
        assert lib.pk_gpu_split_k_segments(M, N, K, 4) == 1
        assert rel_err(fast(dev, "i4", A, W, extra, Z), want) <= MEASURED
        assert lib.pk_gpu_set_workspace(ws.buf.data_ptr() + 4, pk.SPLIT_WORKSPACE_BYTES) == -1
    with Workspace(dev) as ws:
        ws.buf.fill_(float("nan"))
        got = dev.gemm("i4", A, W, Z, scales=extra, exact=False)
        assert bits_equal(got, want)                 # M > 64: exact chains
        assert bool(ws.buf.isnan().all())            # untouched


def test_split_swish_epilogue_against_its_input(dev):
    """The split kernels' Swish epilogue against the oracle's pk_swish
    applied to the same GEMM's un-activated output (the same sums, so the
    difference is the epilogue's alone).  The kernels use the reference's
    own form (its exp polynomial and the IEEE division), so the two agree to
    rounding; the bound would still hold for any Swish within 5e-6 relative
    (a hardware exp2 / reciprocal form measured about 3e-7), and a wrong sign
    or scale in the exponent fails it by orders of magnitude."""
    M, N, K = 300, 512, 256
    A, W, extra, _ = make("i4", M, N, K, "spswish")
    A = (A * np.float32(4.0)).astype(np.float32)                 # outputs over about +-30
    bias = po.normal((N,), 0.0, 0.5, po.seed(0x5EED3000, "spswish.b"))
    Z = np.zeros((M, N), np.float32)
    plain = fast(dev, "i4", A, W, extra, Z, 1.0, 0.0, bias=bias, epi=pk.EPI_NONE)
    act = fast(dev, "i4", A, W, extra, Z, 1.0, 0.0, bias=bias, epi=pk.EPI_SWISH)
    want = po.swish(plain).astype(np.float64)
    err = np.abs(act.astype(np.float64) - want)
    assert float(np.abs(plain).max()) > 8.0                      # both tails exercised
    assert float((err / np.maximum(np.abs(want), 1e-30)).max()) <= 5e-6, float(err.max())


def test_split_k_workspaces_per_thread(dev):
    """Four threads at once, each with its own workspace (thread-local, as
    pk_gpu_set_workspace documents) and its own stream, run split-K GEMMs of
    two shapes twice: every result equals the single-thread run bit for bit
    (the sums have a fixed order)."""
    import threading
    import torch
    lib = pk.load()
    shapes = [("i4", 375, 1024, 4096), ("f32", 500, 1024, 2048)]
    cases = [make(kind, M, N, K, f"spkthr.{kind}.{M}") for kind, M, N, K in shapes]
    with Workspace(dev):
        want = [fast(dev, kind, A, W, extra, np.zeros((M, N), np.float32))
                for (kind, M, N, K), (A, W, extra, _) in zip(shapes, cases)]
        assert all(lib.pk_gpu_split_k_segments(M, N, K, bits_of(kind)) > 1 for kind, M, N, K in shapes)
    n_thr = 4
    spaces = [torch.empty(pk.SPLIT_WORKSPACE_BYTES // 4, device=dev.dev) for _ in range(n_thr)]
    streams = [torch.cuda.Stream(device=dev.dev) for _ in range(n_thr)]
    dev_in = []
    for (kind, M, N, K), (A, W, extra, _) in zip(shapes, cases):
        dev_in.append((dev.put(A), dev.put(W), dev.put(extra) if kind == "i4" else None))
    outs = [[torch.empty((M, N), device=dev.dev) for kind, M, N, K in shapes] for _ in range(n_thr)]
    torch.cuda.synchronize(dev.dev)
    errs = []

    def work(t):
        try:
            pk.call("pk_gpu_set_numerics", pk.NUMERICS_FAST)
            pk.call("pk_gpu_set_workspace", spaces[t].data_ptr(), pk.SPLIT_WORKSPACE_BYTES)
            st = streams[t].cuda_stream
            for _ in range(2):
                for s, ((kind, M, N, K), (dA, dW, dS)) in enumerate(zip(shapes, dev_in)):
                    C = outs[t][s]
                    if kind == "i4":
                        pk.call("pk_gpu_gemm_i4_dev", M, N, K, 1.0, dA.data_ptr(), K, dW.data_ptr(),
                                dS.data_ptr(), N // 2, 0.0, C.data_ptr(), N, st)
                    else:
                        pk.call("pk_gpu_sgemm_dev", M, N, K, 1.0, dA.data_ptr(), K, dW.data_ptr(), N,
                                0.0, C.data_ptr(), N, st)
            streams[t].synchronize()
            pk.call("pk_gpu_set_workspace", None, 0)
        except Exception as e:                       # reported on the main thread
            errs.append(f"thread {t}: {e}")

    threads = [threading.Thread(target=work, args=(t,)) for t in range(n_thr)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errs, errs
    for t in range(n_thr):
        for s in range(len(shapes)):
            assert bits_equal(outs[t][s].cpu().numpy(), want[s]), (t, shapes[s])


def test_split_k_unaligned_output_rows(dev):
    """The split-K reduce writes C with 16-byte accesses where its rows allow
    it; with ldc = N + 1 it takes the per-element path: the same sums, the
    column past N untouched."""
    import torch
    M, N, K = 500, 1024, 2048
    A, W, _, C0 = make("f32", M, N, K, "spkldc")
    want = oracle("f32", A, W, None, C0, 1.0, 1.0)
    lib = pk.load()
    with Workspace(dev):
        assert lib.pk_gpu_split_k_segments(M, N, K, 32) > 1
        big = np.full((M, N + 1), 7.0, np.float32)
        big[:, :N] = C0
        dA, dW, dC = dev.put(A), dev.put(W), dev.put(big)
        prev = lib.pk_gpu_get_numerics()
        pk.call("pk_gpu_set_numerics", pk.NUMERICS_FAST)
        try:
            pk.call("pk_gpu_sgemm_dev", M, N, K, 1.0, dA.data_ptr(), K, dW.data_ptr(), N, 1.0,
                    dC.data_ptr(), N + 1, dev.stream())
        finally:
            pk.call("pk_gpu_set_numerics", prev)
        dev.sync()
        got = dC.cpu().numpy()
    assert rel_err(got[:, :N], want) <= MEASURED
    assert bool((got[:, N] == 7.0).all())


# ---- weights pre-split once (pk_gpu_presplit_weight_dev) ---------------------

def fast_dev(dev, kind, dA, dW, dS, extra, M, N, K, dC, bias=None, epi=None):
    """One FAST GEMM on device operands (no upload), into dC."""
    lib = pk.load()
    ex = bias is not None or epi is not None
    tail = (bias.data_ptr() if bias is not None else None, epi or 0) if ex else ()
    s = dev.stream()
    if kind == "i4":
        rc = getattr(lib, "pk_gpu_gemm_i4_ex_dev" if ex else "pk_gpu_gemm_i4_dev")(
            M, N, K, 1.0, dA.data_ptr(), K, dW.data_ptr(), dS.data_ptr(), N // 2, 0.0, dC.data_ptr(), N, *tail, s)
    elif kind == "i8":
        rc = getattr(lib, "pk_gpu_gemm_i8_ex_dev" if ex else "pk_gpu_gemm_i8_dev")(
            M, N, K, 1.0, dA.data_ptr(), K, dW.data_ptr(), extra, N, 0.0, dC.data_ptr(), N, *tail, s)
    else:
        rc = getattr(lib, "pk_gpu_sgemm_ex_dev" if ex else "pk_gpu_sgemm_dev")(
            M, N, K, 1.0, dA.data_ptr(), K, dW.data_ptr(), N, 0.0, dC.data_ptr(), N, *tail, s)
    assert rc == 0, lib.pk_gpu_last_error()
    dev.sync()
    return dC.cpu().numpy()


# Every launch shape the pre-split copy meets, split-K included (a workspace).
PRESPLIT_SHAPES = [("i4", 1656, 4096, 1024), ("f32", 1656, 2048, 1024), ("i4", 1024, 4096, 256),
                   ("f32", 1024, 2048, 96), ("i4", 416, 4096, 1024), ("i4", 375, 1024, 4096),
                   ("f32", 130, 256, 320), ("i4", 97, 96, 288), ("f32", 77, 32, 32), ("i4", 1656, 1024, 4096),
                   ("i8", 1656, 3072, 1024), ("i8", 1656, 1024, 1024), ("i8", 416, 3072, 1024),
                   ("i8", 375, 1024, 4096), ("i8", 130, 256, 320), ("i8", 97, 96, 288), ("i8", 77, 32, 32)]


@pytest.mark.parametrize("kind,M,N,K", PRESPLIT_SHAPES)
@pytest.mark.parametrize("work", [False, True])
def test_presplit_weights_give_the_same_bits(dev, kind, M, N, K, work):
    """The split kernels read a weight's pre-split copy (the staging's own
    decode and split, done once; int8: the codes as bf16) instead of the
    weight: the same products in the same order, so the same bits, with and
    without split-K."""
    torch = dev.torch
    A, W, extra, C0 = make(kind, M, N, K, f"sps.{kind}.{M}.{N}.{K}")
    bias = po.normal((N,), 0.0, 0.02, po.seed(0x5EED3300, f"sps.{kind}.b"))
    dA, dW = dev.put(A), dev.put(W)
    dS = dev.put(extra) if kind == "i4" else None
    dC, dB = torch.zeros((M, N), device=dev.dev), dev.put(bias)
    lib = pk.load()
    prev = lib.pk_gpu_get_numerics()
    pk.call("pk_gpu_set_numerics", pk.NUMERICS_FAST)
    try:
        with Workspace(dev, pk.SPLIT_WORKSPACE_BYTES if work else 0):
            presplit_case(dev, kind, A, W, extra, M, N, K, dA, dW, dS, dC, dB)
    finally:
        pk.call("pk_gpu_set_numerics", prev)


def presplit_case(dev, kind, A, W, extra, M, N, K, dA, dW, dS, dC, dB):
    lib = pk.load()
    bits = bits_of(kind)
    assert uses_split(M, N, K, bits) == 1
    plain = fast_dev(dev, kind, dA, dW, dS, extra, M, N, K, dC)
    epi = fast_dev(dev, kind, dA, dW, dS, extra, M, N, K, dC, bias=dB, epi=pk.EPI_SWISH)
    before = lib.pk_gpu_presplit_bytes()
    pk.call("pk_gpu_presplit_weight_dev", bits, K, N, dW.data_ptr(), N // 2 if kind == "i4" else N,
            dS.data_ptr() if dS is not None else None, dev.stream())
    try:
        assert lib.pk_gpu_presplit_bytes() == before + (2 if kind == "i8" else 4) * K * N
        # idempotent for the same parameters
        pk.call("pk_gpu_presplit_weight_dev", bits, K, N, dW.data_ptr(), N // 2 if kind == "i4" else N,
                dS.data_ptr() if dS is not None else None, dev.stream())
        dW_orig = dW.clone()
        dW.zero_()                 # the kernels must not read the weight itself any more
        got = fast_dev(dev, kind, dA, dW, dS, extra, M, N, K, dC)
        dW.copy_(dW_orig)
        assert bits_equal(got, plain), describe(got, plain)
        assert bits_equal(fast_dev(dev, kind, dA, dW, dS, extra, M, N, K, dC, bias=dB, epi=pk.EPI_SWISH), epi)
        want = oracle(kind, A, W, extra, np.zeros((M, N), np.float32))
        assert rel_err(got, want) <= MEASURED
    finally:
        pk.call("pk_gpu_unsplit_weight_dev", dW.data_ptr())
    assert lib.pk_gpu_presplit_bytes() == before


def describe(got, want):
    d = got.view(np.uint32) != want.view(np.uint32)
    return f"{int(d.sum())} of {d.size} outputs differ"


def test_presplit_argument_checks(dev):
    lib = pk.load()
    W = dev.torch.zeros((64, 64), device=dev.dev)
    s = dev.stream()
    assert lib.pk_gpu_presplit_weight_dev(16, 64, 64, W.data_ptr(), 64, None, s) == -1    # no such format
    assert lib.pk_gpu_presplit_weight_dev(32, 48, 64, W.data_ptr(), 64, None, s) == -1    # K % 32
    assert lib.pk_gpu_presplit_weight_dev(32, 64, 40, W.data_ptr(), 64, None, s) == -1    # N % 32
    assert lib.pk_gpu_presplit_weight_dev(4, 64, 64, W.data_ptr(), 32, None, s) == -1     # no scales
    assert lib.pk_gpu_presplit_weight_dev(32, 64, 64, W.data_ptr(), 32, None, s) == -1    # ldb < N
    assert lib.pk_gpu_unsplit_weight_dev(W.data_ptr()) == -1                             # none made
