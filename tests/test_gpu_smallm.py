"""GPU: the small-M kernels (pk_smallm.hip), which GEMMs with M <= 64 take
under the default numerics (pk_gpu_set_numerics).

The reference computes every output as one fp32 fma chain over k
(blas.c:187-218, 759-771, 950-963); these kernels take the same products
(fp32 activations split into two bf16 parts, the weights dequantised as the
reference does) through bf16 matrix cores and add them in another, fixed
order.  The contract is max |C - R| / max |R| <= 1e-3 against the oracle R
(which is bit-identical to the reference, test_oracle.py); the tests also
hold the measured error below 1e-4, so a lost term or a wrong scale (errors
of 1e-3 and up) fails them.  Results must be deterministic: the same call
twice, on two streams, from several threads or replayed from a graph gives
the same bits, and every workgroup tile (rows x columns per workgroup) meets
the same bound.  The shapes include the int8 fused QKV of a 2.56 s clip
(M = 32 and 33, K = 1024, N = 3072, encoder.c:312), the int4 feed-forward
pair at M = 33 (encoder.c:193-198), ragged N, rows that are dword- but not
16-byte aligned, and K not a multiple of the 16 waves' 32-row steps."""
import threading

import numpy as np
import pytest

import pyoracle as po
from pkgpu import Dev, bits_equal, gpu_available, pk
from test_gpu_gemm import make, oracle

pytestmark = pytest.mark.gpu

CONTRACT, MEASURED = 1e-3, 1e-4
SHAPES = [("i8", 32, 3072, 1024), ("i8", 33, 3072, 1024), ("i8", 33, 1024, 1024),
          ("i8", 1, 1024, 1024), ("i8", 64, 256, 64), ("i8", 17, 136, 96), ("i8", 5, 40, 32),
          ("i8", 33, 1024, 4096), ("i8", 48, 3072, 1024),
          ("i4", 33, 4096, 1024), ("i4", 33, 1024, 4096), ("i4", 1, 128, 64),
          ("i4", 64, 96, 32), ("i4", 40, 160, 224), ("i4", 32, 4096, 1024),
          ("f32", 33, 1024, 1024), ("f32", 64, 200, 96), ("f32", 7, 3072, 1024),
          ("f32", 33, 1024, 4096), ("i8", 33, 1000, 1056), ("i8", 3, 3068, 4096),
          ("i4", 33, 1024, 8192), ("i8", 64, 4104, 2080)]
TILES = [(1, 1), (2, 1), (3, 1), (4, 1), (1, 2), (2, 2)]


@pytest.fixture(scope="module")
def dev():
    if not gpu_available():
        pytest.skip("no GPU")
    return Dev()


def rel_err(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


def bits_of(kind):
    return {"i4": 4, "i8": 8, "f32": 32}[kind]


def small(dev, kind, A, W, extra, C0, alpha=1.0, beta=0.0, bias=None, epi=None):
    if kind == "i4":
        return dev.gemm(kind, A, W, C0, alpha, beta, scales=extra, bias=bias, epi=epi, exact=False)
    if kind == "i8":
        return dev.gemm(kind, A, W, C0, alpha, beta, scale=extra, bias=bias, epi=epi, exact=False)
    return dev.gemm(kind, A, W, C0, alpha, beta, bias=bias, epi=epi, exact=False)


@pytest.mark.parametrize("kind,M,N,K", SHAPES)
def test_small_m_within_tolerance(dev, kind, M, N, K):
    assert pk.load().pk_gpu_uses_small_m(M, N, K, bits_of(kind)) == 1
    A, W, extra, _ = make(kind, M, N, K, f"sm.{kind}.{M}.{N}.{K}")
    Z = np.zeros((M, N), np.float32)
    want = oracle(kind, A, W, extra, Z)
    got = small(dev, kind, A, W, extra, Z)
    e = rel_err(got, want)
    print(f"{kind} {M}x{N}x{K}: max|C - R| / max|R| = {e:.3g}")
    assert e <= CONTRACT and e <= MEASURED, e
    assert bits_equal(small(dev, kind, A, W, extra, Z), got), "not deterministic"
    # the exact chains for the same shape, on request
    assert bits_equal(dev.gemm(kind, A, W, Z, scale=extra if kind == "i8" else None,
                               scales=extra if kind == "i4" else None, exact=True), want)


@pytest.mark.parametrize("kind", ["i8", "i4", "f32"])
def test_small_m_alpha_beta_and_epilogues(dev, kind):
    for M, N, K in [(33, 256, 512), (33, 256, 2048)] if kind != "f32" else [(33, 256, 512)]:
        alpha_beta_epilogues(dev, kind, M, N, K)


def alpha_beta_epilogues(dev, kind, M, N, K):
    A, W, extra, C0 = make(kind, M, N, K, f"smepi.{kind}.{K}")
    bias = po.normal((N,), 0.0, 0.02, po.seed(0x5EED3000, f"smepi.{kind}.b"))
    Z = np.zeros((M, N), np.float32)
    plain = oracle(kind, A, W, extra, Z)
    for alpha, beta in [(0.75, 0.5), (1.0, 1.0), (-2.0, 0.0)]:
        want = oracle(kind, A, W, extra, C0, alpha, beta)
        got = small(dev, kind, A, W, extra, C0, alpha, beta)
        assert rel_err(got, want) <= MEASURED, (alpha, beta)
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
        got = small(dev, kind, A, W, extra, C_in, 1.0, 0.0, bias=bias, epi=epi)
        assert rel_err(got, want) <= MEASURED, f"epilogue {epi}"


@pytest.mark.parametrize("rb,nct", TILES)
def test_small_m_every_tile(dev, rb, nct):
    """Every workgroup tile the model can pick, forced on each weight format
    (fp32 clamps to one column tile and three row blocks): M = 50 spans four
    16-row blocks with a partial last one, N is ragged for int8 and fp32,
    and K = 1056 gives the 16 waves 2 or 3 steps each."""
    lib = pk.load()
    pk.call("pk_gpu_force_small_tile", rb, nct)
    try:
        for kind, M, N, K in [("i8", 50, 1000, 1056), ("i4", 50, 1024, 2048), ("f32", 50, 520, 1056)]:
            assert lib.pk_gpu_uses_small_m(M, N, K, bits_of(kind)) == 1
            A, W, extra, _ = make(kind, M, N, K, f"smt.{kind}.{rb}.{nct}")
            Z = np.zeros((M, N), np.float32)
            e = rel_err(small(dev, kind, A, W, extra, Z), oracle(kind, A, W, extra, Z))
            print(f"tile {rb}x{nct} {kind} {M}x{N}x{K}: {e:.3g}")
            assert e <= MEASURED, (kind, e)
    finally:
        pk.call("pk_gpu_force_small_tile", 0, 0)
    assert lib.pk_gpu_force_small_tile(3, 2) == -1 and lib.pk_gpu_force_small_tile(5, 1) == -1


def test_small_m_two_streams(dev):
    """One thread, two streams, no host sync in between: the launches share
    no state, so each result equals its single-stream one bit for bit."""
    torch = dev.torch
    lib = pk.load()
    M, N, K = 33, 3072, 1024
    A1, Q1, _, _ = make("i8", M, N, K, "sm2s.1")
    A2, Q2, _, _ = make("i8", M, N, K, "sm2s.2")
    Z = np.zeros((M, N), np.float32)
    want = [small(dev, "i8", A1, Q1, 0.01, Z), small(dev, "i8", A2, Q2, 0.01, Z)]
    s1, s2 = torch.cuda.Stream(dev.dev), torch.cuda.Stream(dev.dev)
    ops = [(dev.put(A1), dev.put(Q1)), (dev.put(A2), dev.put(Q2))]
    outs = [torch.empty((M, N), device=dev.dev) for _ in range(2)]
    dev.sync()
    for rep in range(3):
        for (dA, dQ), dC, st in zip(ops, outs, (s1, s2)):
            pk.check("pk_gpu_gemm_i8_dev", lib.pk_gpu_gemm_i8_dev(
                M, N, K, 1.0, dA.data_ptr(), K, dQ.data_ptr(), 0.01, N, 0.0, dC.data_ptr(), N,
                st.cuda_stream))
        dev.sync()
        for o, w in zip(outs, want):
            assert bits_equal(o.cpu().numpy(), w), f"repeat {rep}"


def test_small_m_graph_replays_equal_eager(dev):
    """Captured into a graph, every replay equals the eager result bit for
    bit, with eager work between the replays."""
    torch = dev.torch
    lib = pk.load()
    shapes = [("i8", 33, 3072, 1024), ("i4", 33, 4096, 1024), ("i4", 33, 1024, 4096)]
    bufs, want = [], []
    for kind, M, N, K in shapes:
        A, W, extra, _ = make(kind, M, N, K, f"smg.{kind}.{N}")
        want.append(small(dev, kind, A, W, extra, np.zeros((M, N), np.float32)))
        bufs.append((kind, M, N, K, dev.put(A), dev.put(W),
                     dev.put(extra) if kind == "i4" else extra, torch.zeros((M, N), device=dev.dev)))

    def launch_all():
        s = torch.cuda.current_stream(dev.dev).cuda_stream
        for kind, M, N, K, dA, dW, ex, dC in bufs:
            if kind == "i8":
                rc = lib.pk_gpu_gemm_i8_dev(M, N, K, 1.0, dA.data_ptr(), K, dW.data_ptr(), ex, N, 0.0,
                                            dC.data_ptr(), N, s)
            else:
                rc = lib.pk_gpu_gemm_i4_dev(M, N, K, 1.0, dA.data_ptr(), K, dW.data_ptr(),
                                            ex.data_ptr(), N // 2, 0.0, dC.data_ptr(), N, s)
            pk.check("small-M launch", rc)

    launch_all()                                    # eager warm-up
    dev.sync()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        launch_all()
    for rep in range(3):
        for *_, dC in bufs:
            dC.fill_(float("nan"))
        g.replay()
        dev.sync()
        for (*_, dC), w in zip(bufs, want):
            assert bits_equal(dC.cpu().numpy(), w), f"replay {rep}"
        launch_all()                                # eager work between replays
        dev.sync()


def test_small_m_host_pointer_from_threads(dev):
    """The drop-in host-pointer entry at the clip's M = 33 from four threads at
    once (each with its own stream): every result equals the single-threaded
    one bit for bit."""
    lib = pk.load()
    M, N, K = 33, 3072, 1024
    cases = [make("i8", M, N, K, f"smt.{t}") for t in range(4)]
    want = []
    for A, Q, s, _ in cases:
        C = np.zeros((M, N), np.float32)
        pk.check("pk_gpu_gemm_i8", lib.pk_gpu_gemm_i8(M, N, K, 1.0, A.ctypes.data, K, Q.ctypes.data,
                                                       s, N, 0.0, C.ctypes.data, N))
        assert rel_err(C, oracle("i8", A, Q, s, np.zeros((M, N), np.float32))) <= MEASURED
        want.append(C)
    got, errs = [None] * 4, []

    def work(t):
        try:
            A, Q, s, _ = cases[t]
            for _ in range(5):
                C = np.zeros((M, N), np.float32)
                rc = lib.pk_gpu_gemm_i8(M, N, K, 1.0, A.ctypes.data, K, Q.ctypes.data, s, N, 0.0,
                                        C.ctypes.data, N)
                if rc:
                    errs.append(f"thread {t}: rc {rc}")
                    return
                if not bits_equal(C, want[t]):
                    errs.append(f"thread {t}: differs")
                    return
            got[t] = C
        except Exception as e:                       # reported on the main thread
            errs.append(f"thread {t}: {e}")

    threads = [threading.Thread(target=work, args=(t,)) for t in range(4)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errs, errs


def test_small_m_dispatch_rules(dev):
    """Which shapes take the small-M kernels: M <= 64 and K % 32 == 0; int8
    rows dword aligned, int4 N % 32 == 0, fp32 rows 16-byte aligned; under the
    default numerics only."""
    lib = pk.load()
    assert lib.pk_gpu_get_numerics() == pk.NUMERICS_DEFAULT
    assert lib.pk_gpu_uses_small_m(33, 3072, 1024, 8) == 1
    assert lib.pk_gpu_uses_small_m(64, 4096, 1024, 4) == 1
    assert lib.pk_gpu_uses_small_m(65, 3072, 1024, 8) == 0          # M > 64: exact chains
    assert lib.pk_gpu_uses_small_m(33, 3072, 1000, 8) == 0          # K % 32 != 0
    assert lib.pk_gpu_uses_small_m(33, 3070, 1024, 8) == 0          # int8 rows not dword aligned
    assert lib.pk_gpu_uses_small_m(33, 3068, 1024, 8) == 1          # dword aligned: 4-byte loads
    assert lib.pk_gpu_uses_small_m(33, 1008, 1024, 4) == 0          # int4 N % 32 != 0
    assert lib.pk_gpu_uses_small_m(33, 1024, 4096, 32) == 1         # fp32
    assert lib.pk_gpu_uses_small_m(33, 1022, 1024, 32) == 0         # fp32 rows not 16-byte aligned
    pk.call("pk_gpu_set_numerics", pk.NUMERICS_EXACT)
    try:
        assert lib.pk_gpu_uses_small_m(33, 3072, 1024, 8) == 0
    finally:
        pk.call("pk_gpu_set_numerics", pk.NUMERICS_DEFAULT)
    pk.call("pk_gpu_force_config", 12)
    try:
        assert lib.pk_gpu_uses_small_m(33, 3072, 1024, 8) == 0      # forced tile: exact
    finally:
        pk.call("pk_gpu_force_config", -1)
    assert lib.pk_gpu_set_numerics(7) == -1
