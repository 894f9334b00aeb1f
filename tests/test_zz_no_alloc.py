"""GPU: pk_gpu_gemm_i8_noalloc, the host-pointer int8 GEMM that stages its
operands in the library's fixed device array instead of allocating.

It must give exactly what pk_gpu_gemm_i8 gives (the same kernels run on the
same staged values, so the bits are equal), on consecutive calls that reuse
the array, the second smaller than the first (stale contents of the array
must not leak into a result); with a registered weight read in place; with
beta != 0 (C uploaded); under exact and default numerics; and it must refuse
a call whose staging exceeds PK_GPU_NOALLOC_BYTES, leaving C untouched."""
import numpy as np
import pytest

from pkgpu import bits_equal, gpu_available, pk
from test_gpu_gemm import make

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not gpu_available():
        pytest.skip("no GPU")
    pk.call("pk_gpu_init", 0)
    return pk.load()


def call(lib, fn, A, Q, scale, C, alpha=1.0, beta=0.0, stream=None):
    M, K = A.shape
    N = Q.shape[1]
    args = [M, N, K, alpha, A.ctypes.data, K, Q.ctypes.data, scale, N, beta, C.ctypes.data, N]
    if fn == "pk_gpu_gemm_i8_noalloc":
        args.append(stream)
    return getattr(lib, fn)(*args)


def both(lib, A, Q, scale, C0, alpha=1.0, beta=0.0):
    """C from the allocating entry point and from the no-allocation one."""
    want, got = C0.copy(), C0.copy()
    pk.check("pk_gpu_gemm_i8", call(lib, "pk_gpu_gemm_i8", A, Q, scale, want, alpha, beta))
    pk.check("pk_gpu_gemm_i8_noalloc", call(lib, "pk_gpu_gemm_i8_noalloc", A, Q, scale, got, alpha, beta))
    return want, got


@pytest.mark.parametrize("numerics", ["exact", "default"])
def test_noalloc_equals_gemm_i8_on_consecutive_calls(lib, numerics):
    """Two calls in a row, the second smaller (M = 33 then 5): each equals
    pk_gpu_gemm_i8 bit for bit; then the first shape again."""
    mode = pk.NUMERICS_EXACT if numerics == "exact" else pk.NUMERICS_DEFAULT
    prev = lib.pk_gpu_get_numerics()
    pk.call("pk_gpu_set_numerics", mode)
    try:
        for M, N, K, beta in [(33, 3072, 1024, 0.5), (5, 520, 256, 0.0), (33, 3072, 1024, 0.0)]:
            A, Q, s, C0 = make("i8", M, N, K, f"noalloc.{M}.{N}")
            want, got = both(lib, A, Q, s, C0, 0.75, beta)
            assert bits_equal(got, want), (M, N, K, beta)
    finally:
        pk.call("pk_gpu_set_numerics", prev)


def test_noalloc_registered_weight_and_long_m(lib):
    """A registered B is read in place (only A and C staged): M = 400 takes
    the exact chain kernels, M = 20 the small-M ones."""
    A, Q, s, C0 = make("i8", 400, 1024, 1024, "noalloc.reg")
    pk.call("pk_gpu_register_weight", Q.ctypes.data, Q.nbytes)
    try:
        for M in (400, 20):
            want, got = both(lib, np.ascontiguousarray(A[:M]), Q, s, np.ascontiguousarray(C0[:M]))
            assert bits_equal(got, want), M
    finally:
        pk.call("pk_gpu_unregister_weight", Q.ctypes.data)


def test_noalloc_on_a_stream(lib):
    """On a caller stream: the same bits as on the null stream."""
    import torch
    A, Q, s, C0 = make("i8", 33, 1024, 1024, "noalloc.stream")
    st = torch.cuda.Stream(torch.device("cuda:0"))
    want, got = C0.copy(), C0.copy()
    pk.check("noalloc", call(lib, "pk_gpu_gemm_i8_noalloc", A, Q, s, want))
    pk.check("noalloc", call(lib, "pk_gpu_gemm_i8_noalloc", A, Q, s, got, stream=st.cuda_stream))
    assert bits_equal(got, want)


def test_noalloc_refuses_oversized_staging(lib):
    """Staging above PK_GPU_NOALLOC_BYTES: PK_GPU_EINVAL, a message naming
    the limit, C unchanged; the next call that fits works."""
    M, K, N = 2048, 4096, 8192            # A 32 MiB + B 32 MiB + C 64 MiB
    A = np.ones((M, K), np.float32)
    Q = np.ones((K, N), np.int8)
    C = np.full((M, N), 7.0, np.float32)
    rc = call(lib, "pk_gpu_gemm_i8_noalloc", A, Q, 0.01, C)
    assert pk.STATUS.get(rc) == "EINVAL", rc
    msg = lib.pk_gpu_last_error().decode()
    assert "PK_GPU_NOALLOC_BYTES" in msg, msg
    assert np.all(C == 7.0)
    A2, Q2, s2, C2 = make("i8", 8, 256, 64, "noalloc.after")
    want, got = both(lib, A2, Q2, s2, C2)
    assert bits_equal(got, want)
