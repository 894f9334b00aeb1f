"""GPU parity of the fused epilogues (the feed-forward's bias add, Swish and
0.5 residual, encoder.c:193-216) against the unfused computation.

Bias and the half residual are exact IEEE operations, so the fused result
must equal the oracle GEMM followed by the same float32 operations in numpy
bit for bit; Swish must equal the device swish kernel applied to the
bias-added GEMM result bit for bit (the device swish's own agreement with the
reference is tested in test_gpu_gemm.test_swish_matches_reference_within_tolerance).
Covers every tile family, the int8 N%16 edge columns, and the alpha == 0
early exit.
"""
import numpy as np
import pytest

import pyoracle as po
from pkgpu import Dev, bits_equal, describe_mismatch, pk
from test_gpu_gemm import make, oracle

pytestmark = pytest.mark.gpu

SEED = 0x5EED2000
NONE, SWISH, HALF = pk.EPI_NONE, pk.EPI_SWISH, pk.EPI_HALF_RESIDUAL


@pytest.fixture(scope="module")
def dev():
    return Dev()


def same(got, want, what):
    assert bits_equal(got, want), f"{what}: {describe_mismatch(got, want)}"


def family_configs():
    """One configuration of each tile family (R, X, S), plus automatic choice."""
    seen, out = set(), [-1]
    for i, (fam, *_rest) in enumerate(pk.configs()):
        if fam not in seen:
            seen.add(fam)
            out.append(i)
    return out


@pytest.mark.parametrize("kind", ["f32", "i8", "i4"])
@pytest.mark.parametrize("cfg", family_configs())
def test_bias_swish_and_half_residual(dev, kind, cfg):
    M, N, K = 45, 160, 96
    A, W, extra, X = make(kind, M, N, K, f"epi.{kind}")
    bias = po.normal((N,), 0.0, 0.1, po.seed(SEED, f"bias.{kind}"))
    zeros = np.zeros((M, N), np.float32)
    ref = oracle(kind, A, W, extra, zeros)
    kw = {"scales": extra} if kind == "i4" else ({"scale": extra} if kind == "i8" else {})
    biased = ref + bias[None, :]                                   # fl(v + b), row-wise
    same(dev.gemm(kind, A, W, zeros, cfg=cfg, bias=bias, **kw), biased, f"bias cfg{cfg}")
    same(dev.gemm(kind, A, W, zeros, cfg=cfg, epi=NONE, **kw), ref, f"plain ex cfg{cfg}")
    fused = dev.gemm(kind, A, W, zeros, cfg=cfg, bias=bias, epi=SWISH, **kw)
    same(fused, dev.swish(biased), f"swish cfg{cfg}")
    # half residual: C holds x on entry; x + 0.5 * (v + b), 0.5 * (.) exact
    got = dev.gemm(kind, A, W, X, cfg=cfg, bias=bias, epi=HALF, **kw)
    same(got, X + np.float32(0.5) * biased, f"half residual cfg{cfg}")


@pytest.mark.parametrize("N", [40, 1000])
def test_int8_edge_columns_get_the_epilogue(dev, N):
    M, K = 19, 70
    A, Q, s, X = make("i8", M, N, K, f"epi.edge.{N}")
    bias = po.normal((N,), 0.0, 0.1, po.seed(SEED, f"edge.bias.{N}"))
    ref = oracle("i8", A, Q, s, np.zeros((M, N), np.float32)) + bias[None, :]
    got = dev.gemm("i8", A, Q, X, scale=s, bias=bias, epi=HALF)
    same(got, X + np.float32(0.5) * ref, f"int8 N={N}")


def test_alpha_zero_runs_the_epilogue_on_beta_c(dev):
    """alpha == 0 skips the multiply (blas.c:1063-1064); the epilogue still
    runs on the beta step's result."""
    M, N, K = 7, 64, 16
    A, W, _, C0 = make("f32", M, N, K, "epi.alpha0")
    bias = po.normal((N,), 0.0, 1.0, po.seed(SEED, "alpha0.bias"))
    got = dev.gemm("f32", A, W, C0, alpha=0.0, beta=0.5, bias=bias, epi=SWISH)
    want = dev.swish(np.float32(0.5) * C0 + bias[None, :])
    same(got, want, "alpha 0")


def test_ffn_pair_fused_matches_unfused(dev):
    """The bench step's fused up-projection (int4, Swish epilogue) equals GEMM +
    swish kernel at the FFN shape M=375."""
    M, D, FF = 375, 1024, 4096
    A, W, S, _ = make("i4", M, FF, D, "epi.ffn")
    zeros = np.zeros((M, FF), np.float32)
    plain = dev.gemm("i4", A, W, zeros, scales=S)
    same(plain, oracle("i4", A, W, S, zeros), "up GEMM")
    same(dev.gemm("i4", A, W, zeros, scales=S, epi=SWISH), dev.swish(plain), "fused swish")
