"""GPU: the weight decode of the GEMM kernels, compared directly.

pk_gpu_dequant_dev writes the weights the chain kernels multiply through the
kernels' own staging code (WStage's loads and conversions, the unit path
that vector-aligned rows take and the element path of the others).  Each
result must equal the oracle's decode byte for byte (a memcmp):
  int8  fl((float)q * scale)                        blas.c:545-553
  int4  fl(q * scales[k][n/32]), q the signed nibble  blas.c:794, 834-840
        (low nibble = even column, the portable decode)
  fp32  the weight itself.
Every byte value occurs in every row, and the scales include subnormal
products, values near the fp32 maximum and negative scales, so a wrong
sign extension, nibble order, scale index or rounding shows."""
import numpy as np
import pytest

import pyoracle as po
from pkgpu import bits_equal, describe_mismatch, gpu_available, pk

pytestmark = pytest.mark.gpu
SEED = 0x5EED7000


@pytest.fixture(scope="module")
def dev():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    pk.call("pk_gpu_init", 0)
    return torch


def all_bytes(K, width, shift):
    """[K][width] bytes, row k a rotation of 0..255 (every value in every row)."""
    k = np.arange(K)[:, None]
    j = np.arange(width)[None, :]
    return ((j + shift * k) % 256).astype(np.uint8)


def run(torch, bits, B, N, ldb, unit_path, scale=0.0, scales=None):
    dB = torch.from_numpy(np.ascontiguousarray(B)).cuda()
    dS = torch.from_numpy(np.ascontiguousarray(scales)).cuda() if scales is not None else None
    K = B.shape[0]
    out = torch.full((K, N), float("nan"), device="cuda")
    pk.check("pk_gpu_dequant_dev", pk.load().pk_gpu_dequant_dev(
        bits, K, N, dB.data_ptr(), ldb, scale, dS.data_ptr() if dS is not None else None,
        unit_path, out.data_ptr(), None))
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("unit_path", [1, 0])
@pytest.mark.parametrize("scale", [0.01, 0.0118, 1.0, -0.5, 3.0e-39, 2.5e36])
def test_int8_decode_is_the_oracles(dev, unit_path, scale):
    K, N = 64, 512
    Q = all_bytes(K, N, 7).view(np.int8)
    got = run(dev, 8, Q, N, N, unit_path, scale=scale)
    want = po.dequant_i8(np.ascontiguousarray(Q), scale)
    assert bits_equal(got, want), describe_mismatch(got, want)


@pytest.mark.parametrize("unit_path", [1, 0])
def test_int4_decode_is_the_oracles(dev, unit_path):
    K, N = 96, 512                                   # 256 bytes per row: every byte value
    P = all_bytes(K, N // 2, 11)
    rng = np.random.Generator(np.random.PCG64(SEED))
    S = rng.uniform(0.005, 0.02, (K, N // 32)).astype(np.float32)
    S[0, :] = [3.0e-39, -0.0117, 1.0, 2.0e37, -1.0e-3, 0.5, 7.0e-42, 1.5] * (N // 32 // 8)
    S[1, ::2] = -S[1, ::2]
    got = run(dev, 4, P, N, N // 2, unit_path, scales=S)
    want = po.dequant_i4(P, S)
    assert bits_equal(got, want), describe_mismatch(got, want)


def test_padded_rows_and_fp32(dev):
    """Row pitch above the width (the element path reads inside each row
    only) and fp32 weights (the identity)."""
    K, N = 40, 96
    Q = all_bytes(K, N + 32, 3).view(np.int8)        # ldb = 128 > N
    got = run(dev, 8, Q, N, N + 32, 1, scale=0.0123)
    want = po.dequant_i8(np.ascontiguousarray(Q[:, :N]), 0.0123)
    assert bits_equal(got, want), describe_mismatch(got, want)
    W = np.random.Generator(np.random.PCG64(SEED + 1)).standard_normal((K, N)).astype(np.float32)
    for up in (1, 0):
        assert bits_equal(run(dev, 32, W, N, N, up), W)


def test_decode_argument_checks(dev):
    lib = pk.load()
    ok = dev.zeros(64, device="cuda")
    assert pk.STATUS[lib.pk_gpu_dequant_dev(16, 4, 4, ok.data_ptr(), 4, 1.0, None, 0, ok.data_ptr(), None)] == "EINVAL"
    # int4 rows hold N/2 bytes: odd N is refused before anything is launched
    assert pk.STATUS[lib.pk_gpu_dequant_dev(4, 4, 47, ok.data_ptr(), 24, 1.0, ok.data_ptr(), 0, ok.data_ptr(), None)] == "EINVAL"
    assert pk.STATUS[lib.pk_gpu_dequant_dev(8, 4, 6, ok.data_ptr(), 6, 1.0, None, 1, ok.data_ptr(), None)] == "EINVAL"
    assert pk.STATUS[lib.pk_gpu_dequant_dev(8, 4, 8, ok.data_ptr(), 4, 1.0, None, 0, ok.data_ptr(), None)] == "EINVAL"
