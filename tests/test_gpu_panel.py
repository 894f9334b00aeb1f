"""GPU: the panel kernels (pk_panel.hip), the small-M GEMMs (M <= 64) on
weights repacked once into the matrix cores' operand order.

They are the tolerance path of the other small-M kernels: the reference's
products (blas.c:187-218, 759-771, 950-963, 1055-1072) summed in another,
fixed order, within max |C - R| / max |R| <= 1e-3 of the oracle R (which is
bit-identical to the reference, test_oracle.py).  The tests hold the measured
error below 1e-4, so a lost term, a wrong scale or a wrong k permutation
(errors of 1e-3 and up) fails them.

The repack itself is pinned byte for byte: the panel's decode (the weights
exactly as the panel kernels multiply them) equals the oracle's decode of the
on-disk layout (memcmp): int8 fl(q * s), int4 fl(q * s[k][n/32]) with the
signed low-nibble-first decode (blas.c:834-840, extract_weights.py:589-592);
fp32 hi + lo with hi = bf16(w) and lo = bf16(w - hi), both rounded to
nearest even, computed here in numpy.

Shapes: the clip's QKV (M = 32, 33), the feed-forward pair at M = 33, the
pointwise convolutions, M across the LDS phase boundaries (35/36, 48/49,
64), K not a multiple of 256, ragged N, split-K with a workspace (K = 4096),
every tile width, alpha / beta, every epilogue, graph replays, and the
registered-weight drop-in path that makes panels on first use."""
import numpy as np
import pytest

import pyoracle as po
from pkgpu import Dev, bits_equal, describe_mismatch, gpu_available, pk
from test_gpu_gemm import make, oracle

pytestmark = pytest.mark.gpu

MEASURED = 1e-4
BITS = {"i4": 4, "i8": 8, "f32": 32}
SHAPES = [("i8", 32, 3072, 1024), ("i8", 33, 3072, 1024), ("i8", 33, 1024, 1024),
          ("i4", 33, 4096, 1024), ("i4", 33, 1024, 4096), ("f32", 33, 2048, 1024),
          ("f32", 33, 1024, 1024), ("i8", 1, 3072, 1024), ("i8", 16, 256, 96),
          ("i8", 17, 136, 224), ("i8", 35, 1000, 1056), ("i8", 36, 520, 1056),
          ("i4", 36, 256, 2048), ("f32", 48, 200, 800), ("i8", 49, 3068, 1024),
          ("i4", 49, 96, 512), ("i8", 64, 3072, 1024), ("f32", 64, 96, 1088),
          ("i4", 64, 4096, 1024), ("i8", 5, 40, 32), ("i4", 1, 128, 64), ("f32", 7, 3072, 1024)]


@pytest.fixture(scope="module")
def dev():
    if not gpu_available():
        pytest.skip("no GPU")
    return Dev()


def rel_err(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / max(np.abs(want).max(), 1e-30))


class Packed:
    """Device copies of A, W (and int4 scales) with W's panel made."""

    def __init__(self, dev, kind, A, W, extra):
        self.dev, self.kind = dev, kind
        self.M, self.K = A.shape
        self.N = W.shape[1] * 2 if kind == "i4" else W.shape[1]
        self.ldb = W.shape[1]
        self.extra = extra
        self.dA, self.dW = dev.put(A), dev.put(W)
        self.dS = dev.put(extra) if kind == "i4" else None
        self.sp = self.dS.data_ptr() if self.dS is not None else None
        pk.call("pk_gpu_pack_weight_dev", BITS[kind], self.K, self.N, self.dW.data_ptr(), self.ldb,
                self.sp, dev.stream())

    def uses_panel(self):
        return pk.load().pk_gpu_uses_panel(self.M, self.N, self.K, BITS[self.kind], self.dW.data_ptr(),
                                           self.ldb, self.sp)

    def run(self, C0, alpha=1.0, beta=0.0, bias=None, epi=None, stream=None, out=None):
        """One GEMM on the default numerics; returns numpy C (or leaves it in out)."""
        dev = self.dev
        dC = out if out is not None else dev.put(C0)
        dbias = dev.put(bias) if bias is not None else None
        ex = bias is not None or epi is not None
        tail = ((dbias.data_ptr() if dbias is not None else None, epi or 0) if ex else ())
        s = stream if stream is not None else dev.stream()
        M, N, K = self.M, self.N, self.K
        if self.kind == "i4":
            pk.call("pk_gpu_gemm_i4_ex_dev" if ex else "pk_gpu_gemm_i4_dev", M, N, K, alpha,
                    self.dA.data_ptr(), K, self.dW.data_ptr(), self.sp, self.ldb, beta,
                    dC.data_ptr(), N, *tail, s)
        elif self.kind == "i8":
            pk.call("pk_gpu_gemm_i8_ex_dev" if ex else "pk_gpu_gemm_i8_dev", M, N, K, alpha,
                    self.dA.data_ptr(), K, self.dW.data_ptr(), self.extra, self.ldb, beta,
                    dC.data_ptr(), N, *tail, s)
        else:
            pk.call("pk_gpu_sgemm_ex_dev" if ex else "pk_gpu_sgemm_dev", M, N, K, alpha,
                    self.dA.data_ptr(), K, self.dW.data_ptr(), self.ldb, beta, dC.data_ptr(), N,
                    *tail, s)
        if out is not None:
            return None
        dev.sync()
        return dC.cpu().numpy()

    def close(self):
        pk.call("pk_gpu_unpack_weight_dev", self.dW.data_ptr())


@pytest.fixture()
def default_numerics():
    lib = pk.load()
    prev = lib.pk_gpu_get_numerics()
    pk.call("pk_gpu_set_numerics", pk.NUMERICS_DEFAULT)
    yield
    pk.call("pk_gpu_set_numerics", prev)


@pytest.fixture()
def workspace(dev):
    work = dev.torch.empty(pk.SPLIT_WORKSPACE_BYTES // 4, device=dev.dev)
    pk.call("pk_gpu_set_workspace", work.data_ptr(), pk.SPLIT_WORKSPACE_BYTES)
    yield work
    pk.call("pk_gpu_set_workspace", None, 0)


# ---- the repack, byte for byte ------------------------------------------------

def bf16_rne(x):
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000).astype(np.uint32)
    return r.view(np.float32)


def decode(dev, kind, K, N, dW, ldb, dS, scale=0.0):
    out = dev.torch.full((K, N), float("nan"), device=dev.dev)
    pk.call("pk_gpu_panel_decode_dev", BITS[kind], K, N, dW.data_ptr(), ldb,
            dS.data_ptr() if dS is not None else None, scale, out.data_ptr(), dev.stream())
    dev.sync()
    return out.cpu().numpy()


@pytest.mark.parametrize("scale", [0.01, -0.5, 2.5e36])
def test_int8_panel_decode_is_the_oracles(dev, scale):
    K, N = 96, 272                         # N ragged: 17 tiles of 16
    k = np.arange(K)[:, None]
    Q = ((np.arange(N)[None, :] + 7 * k) % 256).astype(np.uint8).view(np.int8)   # every byte value
    dW = dev.put(Q)
    pk.call("pk_gpu_pack_weight_dev", 8, K, N, dW.data_ptr(), N, None, dev.stream())
    try:
        got = decode(dev, "i8", K, N, dW, N, None, scale)
    finally:
        pk.call("pk_gpu_unpack_weight_dev", dW.data_ptr())
    want = po.dequant_i8(np.ascontiguousarray(Q), scale)
    assert bits_equal(got, want), describe_mismatch(got, want)


def test_int4_panel_decode_is_the_oracles(dev):
    K, N = 64, 512
    k = np.arange(K)[:, None]
    P = ((np.arange(N // 2)[None, :] + 5 * k) % 256).astype(np.uint8)               # every byte value
    S = po.uniform((K, N // 32), 0.005, 0.02, po.seed(0x5EED7100, "p4.S"))
    S[0, :4] = [-0.75, 3.0e-39, 2.0e37, 1.0]                  # negative, subnormal product, huge
    dW, dS = dev.put(P), dev.put(S)
    pk.call("pk_gpu_pack_weight_dev", 4, K, N, dW.data_ptr(), N // 2, dS.data_ptr(), dev.stream())
    try:
        got = decode(dev, "i4", K, N, dW, N // 2, dS)
    finally:
        pk.call("pk_gpu_unpack_weight_dev", dW.data_ptr())
    want = po.dequant_i4(np.ascontiguousarray(P), np.ascontiguousarray(S))
    assert bits_equal(got, want), describe_mismatch(got, want)


def test_fp32_panel_decode_is_hi_plus_lo(dev):
    K, N = 64, 48
    W = po.normal((K, N), 0.0, 0.02, po.seed(0x5EED7100, "p32.W"))
    W[0, :6] = [0.0, -0.0, 1.0 + 2.0 ** -9, 3.0e30, -1.5e-30, 1.0 + 2.0 ** -8 + 2.0 ** -17]
    hi = bf16_rne(W)
    lo = bf16_rne((W - hi).astype(np.float32))
    want = (hi + lo).astype(np.float32)
    dW = dev.put(W)
    pk.call("pk_gpu_pack_weight_dev", 32, K, N, dW.data_ptr(), N, None, dev.stream())
    try:
        got = decode(dev, "f32", K, N, dW, N, None)
    finally:
        pk.call("pk_gpu_unpack_weight_dev", dW.data_ptr())
    assert bits_equal(got, want), describe_mismatch(got, want)
    assert np.abs(want.astype(np.float64) - W).max() <= 2.0 ** -16 * np.abs(W).max()


# ---- GEMMs ----------------------------------------------------------------------

@pytest.mark.parametrize("kind,M,N,K", SHAPES)
def test_panel_within_tolerance(dev, default_numerics, kind, M, N, K):
    A, W, extra, _ = make(kind, M, N, K, f"pn.{kind}.{M}.{N}.{K}")
    Z = np.zeros((M, N), np.float32)
    want = oracle(kind, A, W, extra, Z)
    pw = Packed(dev, kind, A, W, extra)
    try:
        assert pw.uses_panel() == 1
        got = pw.run(Z)
        e = rel_err(got, want)
        print(f"panel {kind} {M}x{N}x{K}: max|C - R| / max|R| = {e:.3g}")
        assert e <= MEASURED, e
        assert bits_equal(pw.run(Z), got), "not deterministic"
    finally:
        pw.close()
    assert pw.uses_panel() == 0


@pytest.mark.parametrize("kind", ["i8", "i4", "f32"])
def test_panel_alpha_beta_and_epilogues(dev, default_numerics, kind):
    M, N, K = 33, 256, 512
    A, W, extra, C0 = make(kind, M, N, K, f"pnepi.{kind}")
    bias = po.normal((N,), 0.0, 0.02, po.seed(0x5EED7100, f"pnepi.{kind}.b"))
    Z = np.zeros((M, N), np.float32)
    plain = oracle(kind, A, W, extra, Z)
    pw = Packed(dev, kind, A, W, extra)
    try:
        for alpha, beta in [(0.75, 0.5), (1.0, 1.0), (-2.0, 0.0)]:
            want = oracle(kind, A, W, extra, C0, alpha, beta)
            assert rel_err(pw.run(C0, alpha, beta), want) <= MEASURED, (alpha, beta)
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
            assert rel_err(pw.run(C_in, bias=bias, epi=epi), want) <= MEASURED, f"epilogue {epi}"
    finally:
        pw.close()


@pytest.mark.parametrize("kind,M,N,K", [("i8", 40, 136, 2080), ("f32", 33, 1024, 2048),
                                        ("i4", 33, 1024, 3072)])
def test_panel_two_or_three_phases_stay_in_one_launch(dev, default_numerics, workspace, kind, M, N, K):
    """K of 2 or 3 LDS phases runs them one after the other in one launch even
    with a workspace (measured faster than splitting them); the result is the
    same as without a workspace, bit for bit."""
    assert pk.load().pk_gpu_panel_segments(M, N, K) == 1
    A, W, extra, C0 = make(kind, M, N, K, f"pn1l.{kind}.{M}.{K}")
    pw = Packed(dev, kind, A, W, extra)
    try:
        got = pw.run(C0, 0.75, 0.5)
        assert rel_err(got, oracle(kind, A, W, extra, C0, 0.75, 0.5)) <= MEASURED
        pk.call("pk_gpu_set_workspace", None, 0)
        try:
            assert bits_equal(pw.run(C0, 0.75, 0.5), got)
        finally:
            pk.call("pk_gpu_set_workspace", workspace.data_ptr(), pk.SPLIT_WORKSPACE_BYTES)
    finally:
        pw.close()


@pytest.mark.parametrize("kind,M,N,K", [("i4", 33, 1024, 4096), ("i8", 33, 1024, 4096),
                                        ("f32", 33, 1024, 4096), ("i8", 64, 3072, 4096),
                                        ("i4", 17, 512, 3104), ("i8", 40, 136, 3104)])
def test_panel_split_k(dev, default_numerics, workspace, kind, M, N, K):
    """With a workspace, K beyond one LDS phase splits over workgroups: the
    partial tiles are summed in segment order by a second launch, then alpha,
    beta, bias and the epilogue."""
    segs = pk.load().pk_gpu_panel_segments(M, N, K)
    assert segs > 1, segs
    A, W, extra, C0 = make(kind, M, N, K, f"pnsk.{kind}.{M}.{K}")
    bias = po.normal((N,), 0.0, 0.02, po.seed(0x5EED7100, f"pnsk.{kind}.b"))
    Z = np.zeros((M, N), np.float32)
    pw = Packed(dev, kind, A, W, extra)
    try:
        got = pw.run(Z)
        want = oracle(kind, A, W, extra, Z)
        e = rel_err(got, want)
        print(f"split-K {segs} segments {kind} {M}x{N}x{K}: {e:.3g}")
        assert e <= MEASURED, e
        assert bits_equal(pw.run(Z), got), "not deterministic"
        want = oracle(kind, A, W, extra, C0, 0.75, 0.5)
        assert rel_err(pw.run(C0, 0.75, 0.5), want) <= MEASURED
        biased = (oracle(kind, A, W, extra, Z) + bias[None, :]).astype(np.float32)
        want = (C0 + np.float32(0.5) * biased).astype(np.float32)
        assert rel_err(pw.run(C0, bias=bias, epi=pk.EPI_HALF_RESIDUAL), want) <= MEASURED
        # other activations on the same workspace: each call reads back the
        # partials it wrote, none left from the call before (caches included)
        for t in range(2):
            A2 = make(kind, M, N, K, f"pnsk{t}.{kind}.{M}.{K}")[0]
            pw.dA.copy_(dev.put(A2))
            e2 = rel_err(pw.run(Z), oracle(kind, A2, W, extra, Z))
            assert e2 <= MEASURED, (t, e2)
    finally:
        pw.close()


@pytest.mark.parametrize("mb,nct", [(1, 1), (2, 1), (3, 1), (4, 1), (1, 2), (2, 2), (4, 2)])
def test_panel_every_tile(dev, default_numerics, mb, nct):
    """Every workgroup tile, forced: M = 50 gives row groups with a partial
    last block (and, for mb = 4, a 50-row group with LDS phases of 512 k)."""
    pk.call("pk_gpu_force_panel_tile", mb, nct)
    try:
        for kind, M, N, K in [("i8", 50, 1000, 1056), ("i4", 50, 1024, 2048), ("f32", 50, 520, 1056),
                              ("i8", 33, 3072, 1024), ("i4", 20, 96, 352)]:
            A, W, extra, _ = make(kind, M, N, K, f"pnt.{kind}.{nct}")
            Z = np.zeros((M, N), np.float32)
            pw = Packed(dev, kind, A, W, extra)
            try:
                e = rel_err(pw.run(Z), oracle(kind, A, W, extra, Z))
            finally:
                pw.close()
            print(f"tile {mb}x{nct} {kind} {M}x{N}x{K}: {e:.3g}")
            assert e <= MEASURED, (kind, e)
    finally:
        pk.call("pk_gpu_force_panel_tile", 0, 0)
    lib = pk.load()
    assert lib.pk_gpu_force_panel_tile(5, 1) == -1 and lib.pk_gpu_force_panel_tile(1, 3) == -1


def test_panel_graph_replays_equal_eager(dev, default_numerics, workspace):
    """Captured into a graph (split-K reduce launch included), every replay
    equals the eager result bit for bit, with eager work between replays."""
    torch = dev.torch
    cases = []
    for kind, M, N, K in [("i8", 33, 3072, 1024), ("i4", 33, 4096, 1024), ("i4", 33, 1024, 4096)]:
        A, W, extra, _ = make(kind, M, N, K, f"png.{kind}.{N}")
        pw = Packed(dev, kind, A, W, extra)
        cases.append((pw, pw.run(np.zeros((M, N), np.float32)), torch.zeros((M, N), device=dev.dev)))
    try:
        def launch_all():
            for pw, _, dC in cases:
                pw.run(None, out=dC)

        launch_all()
        dev.sync()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            launch_all()
        for rep in range(3):
            for _, _, dC in cases:
                dC.fill_(float("nan"))
            g.replay()
            dev.sync()
            for pw, want, dC in cases:
                assert bits_equal(dC.cpu().numpy(), want), f"replay {rep} {pw.kind}"
            launch_all()
            dev.sync()
    finally:
        for pw, _, _ in cases:
            pw.close()


def test_panel_registry(dev, default_numerics):
    lib = pk.load()
    M, N, K = 33, 512, 256
    A, W, extra, _ = make("i8", M, N, K, "pnreg")
    before = lib.pk_gpu_panel_bytes()
    pw = Packed(dev, "i8", A, W, extra)
    assert lib.pk_gpu_panel_bytes() - before == N * K          # 32 tiles x 8 steps x 512 bytes
    try:
        # idempotent for the same parameters; another shape for the same weight is refused
        pk.call("pk_gpu_pack_weight_dev", 8, K, N, pw.dW.data_ptr(), N, None, dev.stream())
        assert lib.pk_gpu_pack_weight_dev(8, K, N // 2, pw.dW.data_ptr(), N, None, dev.stream()) == -1
        # another shape, or exact numerics, does not take the panel
        assert lib.pk_gpu_uses_panel(M, N // 2, K, 8, pw.dW.data_ptr(), N, None) == 0
        assert lib.pk_gpu_uses_panel(65, N, K, 8, pw.dW.data_ptr(), N, None) == 0
        pk.call("pk_gpu_set_numerics", pk.NUMERICS_EXACT)
        assert pw.uses_panel() == 0
        pk.call("pk_gpu_set_numerics", pk.NUMERICS_DEFAULT)
        assert pw.uses_panel() == 1
        # bad arguments
        assert lib.pk_gpu_pack_weight_dev(8, 100, N, pw.dW.data_ptr(), N, None, dev.stream()) == -1
        assert lib.pk_gpu_pack_weight_dev(4, K, 48, pw.dW.data_ptr(), 24, pw.dW.data_ptr(), dev.stream()) == -1
        assert lib.pk_gpu_pack_weight_dev(16, K, N, pw.dW.data_ptr(), N, None, dev.stream()) == -1
    finally:
        pw.close()
    assert lib.pk_gpu_panel_bytes() == before
    assert lib.pk_gpu_unpack_weight_dev(pw.dW.data_ptr()) == -1


@pytest.mark.parametrize("kind", ["i8", "i4", "f32"])
def test_registered_weight_gets_a_panel(dev, default_numerics, kind):
    """The drop-in path: a host-pointer GEMM at M = 33 on a registered weight
    (int4: and registered scales) makes its panel on first use and reads it
    from then on; unregistering frees it.  Results within the tolerance."""
    lib = pk.load()
    M, N, K = 33, 1024, 1024
    A, W, extra, C0 = make(kind, M, N, K, f"pnhost.{kind}")
    W = np.ascontiguousarray(W)
    regs = [W] + ([np.ascontiguousarray(extra)] if kind == "i4" else [])
    for r in regs:
        pk.call("pk_gpu_register_weight", r.ctypes.data, r.nbytes)
    before = lib.pk_gpu_panel_bytes()
    try:
        want = oracle(kind, A, W, extra, C0, 0.75, 0.5)
        for rep in range(2):
            C = C0.copy()
            if kind == "i8":
                pk.call("pk_gpu_gemm_i8", M, N, K, 0.75, A.ctypes.data, K, W.ctypes.data, extra, N,
                        0.5, C.ctypes.data, N)
            elif kind == "i4":
                pk.call("pk_gpu_gemm_i4", M, N, K, 0.75, A.ctypes.data, K, W.ctypes.data,
                        regs[1].ctypes.data, N // 2, 0.5, C.ctypes.data, N)
            else:
                pk.call("pk_gpu_sgemm", pk.NOTRANS, pk.NOTRANS, M, N, K, 0.75, A.ctypes.data, K,
                        W.ctypes.data, N, 0.5, C.ctypes.data, N)
            assert rel_err(C, want) <= MEASURED, rep
            assert lib.pk_gpu_panel_bytes() > before
    finally:
        for r in regs:
            pk.call("pk_gpu_unregister_weight", r.ctypes.data)
    assert lib.pk_gpu_panel_bytes() == before
