"""Pins the CPU oracle (oracle/pk_oracle.c) before anything is checked
against it.

  * bit-for-bit against the reference compiled from its own sources
    (oracle/_ref/libpkref.so = x86 AVX2 path; libpkref_portable.so = blas.c's
    portable path, which is the NEON path's arithmetic) on ragged shapes and
    alpha/beta variants.  The int4 GEMM is pinned on the portable path only:
    the AVX2 int4 unpack (blas.c:815-833) mis-decodes nibbles, and
    test_x86_int4_unpack_defect characterises that exactly;
  * dequantisation exhaustively against the two's-complement closed form;
  * an fp64 brute-force bound on every output (catches a dropped term, a
    transposed operand or a wrong scale index independently of the
    reference build);
  * special cases with exact integer answers.
"""
import itertools

import numpy as np
import pytest

import pyoracle as po

needs_ref = pytest.mark.skipif(not po.have_ref(), reason="oracle/_ref not built")
needs_portable = pytest.mark.skipif(not po.have_ref("portable"),
                                    reason="oracle/_ref portable build missing")

SEED = 0x5EED0000


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def rand_case(M, N, K, tag):
    A = po.normal((M, K), 0.0, 1.0, po.seed(SEED, f"{tag}.A"))
    C0 = po.normal((M, N), 0.0, 1.0, po.seed(SEED, f"{tag}.C"))
    return A, C0


# ---- dequantisation: closed forms, exhaustive -------------------------------

def test_int8_dequant_exhaustive():
    lib = po.oracle()
    for s in (0.01, 1.0, 3.0517578125e-05, 0.0123, 7.5):
        s32 = np.float32(s)
        for q in range(-128, 128):
            want = np.float32(np.float32(q) * s32)  # one IEEE product
            got = np.float32(lib.pkor_dequant_i8(q, s32))
            assert got.view(np.uint32) == want.view(np.uint32), (q, s)


def test_int4_nibbles_exhaustive():
    lib = po.oracle()
    for b in range(256):
        lo, hi = b & 0xF, b >> 4
        # two's complement of a 4-bit field
        want_lo = lo - 16 if lo >= 8 else lo
        want_hi = hi - 16 if hi >= 8 else hi
        assert lib.pkor_nibble_lo(b) == want_lo
        assert lib.pkor_nibble_hi(b) == want_hi


def test_int4_matrix_layout():
    """Low nibble is the even column, scale index is k*(N/32) + n/32."""
    K, N = 3, 64
    P = po.bytes_((K, N // 2), po.seed(SEED, "i4layout.P"))
    S = po.uniform((K, N // 32), 0.005, 0.02, po.seed(SEED, "i4layout.S"))
    W = po.dequant_i4(P, S)
    for k in range(K):
        for n in range(N):
            byte = int(P[k, n // 2])
            nib = (byte >> 4) if n % 2 else (byte & 0xF)
            v = nib - 16 if nib >= 8 else nib
            want = np.float32(np.float32(v) * S[k, n // 32])
            assert W[k, n].view(np.uint32) == want.view(np.uint32)


# ---- GEMMs against the compiled reference -----------------------------------

SHAPES_F32 = [(1, 16, 1), (2, 8, 3), (3, 17, 255), (4, 24, 256), (5, 48, 257),
              (33, 1024, 64), (7, 408, 130), (5, 31, 300), (33, 40, 1024)]
SHAPES_I8 = [(1, 16, 1), (3, 17, 255), (4, 32, 256), (5, 48, 257),
             (33, 1024, 64), (2, 9, 40), (6, 31, 100), (5, 3072, 16)]
SHAPES_I4 = [(1, 32, 1), (3, 64, 255), (4, 32, 256), (5, 96, 257),
             (33, 1024, 64), (2, 4096, 8), (9, 128, 1024)]
AB = [(1.0, 0.0), (1.0, 1.0), (0.75, 0.5), (0.0, 0.5), (1.0, -2.0)]


@needs_ref
@needs_portable
@pytest.mark.parametrize("impl", ["ref", "portable"])
@pytest.mark.parametrize("M,N,K", SHAPES_F32)
def test_sgemm_matches_reference(M, N, K, impl):
    B = po.normal((K, N), 0.0, 0.02, po.seed(SEED, f"f32.{M}.{N}.{K}.B"))
    A, C0 = rand_case(M, N, K, f"f32.{M}.{N}.{K}")
    for alpha, beta in AB:
        got = po.sgemm(A, B, C0.copy(), alpha, beta, impl="oracle")
        want = po.sgemm(A, B, C0.copy(), alpha, beta, impl=impl)
        assert bits_equal(got, want), (M, N, K, alpha, beta)


@needs_ref
@pytest.mark.parametrize("M,N,K", SHAPES_I8)
def test_sgemm_qb_matches_reference(M, N, K):
    """int8, AVX2 path, including the N % 16 edge columns (blas.c:733-755)."""
    Q = po.int8s((K, N), -127, 127, po.seed(SEED, f"i8.{M}.{N}.{K}.Q"))
    A, C0 = rand_case(M, N, K, f"i8.{M}.{N}.{K}")
    for (alpha, beta), s in itertools.product(AB, (0.01, 0.0123, 0.0)):
        got = po.sgemm_qb(A, Q, s, C0.copy(), alpha, beta, impl="oracle")
        want = po.sgemm_qb(A, Q, s, C0.copy(), alpha, beta, impl="ref")
        assert bits_equal(got, want), (M, N, K, alpha, beta, s)


@needs_portable
@pytest.mark.parametrize("M,N,K", [s for s in SHAPES_I8 if s[1] % 16 == 0])
def test_sgemm_qb_matches_portable_reference(M, N, K):
    """The portable edge loop differs from the AVX2 build's only in N%16 columns."""
    Q = po.int8s((K, N), -127, 127, po.seed(SEED, f"i8.{M}.{N}.{K}.Q"))
    A, C0 = rand_case(M, N, K, f"i8.{M}.{N}.{K}")
    for alpha, beta in AB:
        got = po.sgemm_qb(A, Q, 0.0123, C0.copy(), alpha, beta, impl="oracle")
        want = po.sgemm_qb(A, Q, 0.0123, C0.copy(), alpha, beta, impl="portable")
        assert bits_equal(got, want), (M, N, K, alpha, beta)


@needs_portable
@pytest.mark.parametrize("M,N,K", SHAPES_I4)
def test_sgemm_q4b_matches_reference(M, N, K):
    P = po.bytes_((K, N // 2), po.seed(SEED, f"i4.{M}.{N}.{K}.P"))
    S = po.uniform((K, N // 32), 0.005, 0.02, po.seed(SEED, f"i4.{M}.{N}.{K}.S"))
    A, C0 = rand_case(M, N, K, f"i4.{M}.{N}.{K}")
    for alpha, beta in AB:
        got = po.sgemm_q4b(A, P, S, C0.copy(), alpha, beta, impl="oracle")
        want = po.sgemm_q4b(A, P, S, C0.copy(), alpha, beta, impl="portable")
        assert bits_equal(got, want), (M, N, K, alpha, beta)


def ragged_int4_case(M, N, K, tag):
    """Packed codes [K][N/2] and the K * floor(N/32) + 1 scales the
    reference reads when N % 32 != 0 (blas.c:794, 958)."""
    P = po.bytes_((K, N // 2), po.seed(SEED, f"{tag}.P"))
    n_s = K * (N // 32) + (1 if N % 32 else 0)
    S = po.uniform((n_s,), 0.005, 0.02, po.seed(SEED, f"{tag}.S"))
    A, C0 = rand_case(M, N, K, tag)
    return A, P, S, C0


@needs_portable
@pytest.mark.parametrize("N", [16, 40, 48, 50, 80, 82, 114])
def test_sgemm_q4b_ragged_n_matches_portable_reference(N):
    """int4 GEMMs whose N is not a multiple of 32 (no shipped weight): the
    reference floors n_groups = N/32 (blas.c:958) and still indexes scale
    k * n_groups + n/32 (blas.c:794, 896, 938), and its N % 16 edge columns
    take the scalar loop of blas.c:925-946.  The oracle (the same dequant
    fl(q * s) and fma chain for every column) equals the compiled portable
    build bit for bit, edge columns included (N = 50, 82, 114)."""
    M, K = 5, 96
    A, P, S, C0 = ragged_int4_case(M, N, K, f"i4r.{N}")
    for alpha, beta in AB:
        got = po.sgemm_q4b(A, P, S, C0.copy(), alpha, beta, impl="oracle")
        want = po.sgemm_q4b(A, P, S, C0.copy(), alpha, beta, impl="portable")
        assert bits_equal(got, want), (N, alpha, beta)


def test_int4_ragged_n_scale_index():
    """Independent of the reference: at N = 48 (one whole group), a code at
    column 40 of row k takes scale k * 1 + 40 // 32 = k + 1, row k + 1's
    first scale; at N = 16 (no whole group) every row takes scale 0.  A
    scale index that did not floor n_groups, or that kept rows apart, fails
    the fp64 bound."""
    for N, col in ((48, 40), (16, 7), (80, 70)):
        M, K = 3, 40
        ng = N // 32
        P = np.zeros((K, N // 2), np.uint8)
        P[:, col // 2] = 1 if col % 2 == 0 else 0x10          # code +1 at column `col`
        S = (np.arange(K * ng + 1, dtype=np.float32) + 1.0) / 64.0
        A = po.normal((M, K), 0.0, 1.0, po.seed(SEED, f"i4idx.{N}"))
        C = po.sgemm_q4b(A, P, S, np.zeros((M, N), np.float32))
        idx = np.arange(K) * ng + col // 32
        exact = A.astype(np.float64) @ S[idx].astype(np.float64)
        mag = np.abs(A.astype(np.float64)) @ np.abs(S[idx].astype(np.float64))
        assert np.all(np.abs(C[:, col] - exact) <= (K + 2) * 2.0 ** -23 * mag), N
        assert not np.any(np.delete(C, col, axis=1)), N


def x86_avx2_int4_weights(P, S):
    """What blas.c:815-833 produces on x86: _mm_slli/_mm_srai_epi16 work on
    16-bit lanes, so within each 8-byte (16-column) panel, column 2w gets the
    low nibble of byte 2w, column 2w+1 gets (byte 2w >> 4) | (byte 2w+1 << 4)
    as a signed byte, and columns 8..15 get 0."""
    K, half = P.shape
    N = half * 2
    W = np.zeros((K, N), np.float32)
    b = P.astype(np.int32)
    for p in range(N // 16):
        for w in range(4):
            lo = b[:, p * 8 + 2 * w] & 0xF
            v0 = np.where(lo >= 8, lo - 16, lo)
            h = ((b[:, p * 8 + 2 * w] >> 4) & 0xF) | ((b[:, p * 8 + 2 * w + 1] & 0xF) << 4)
            v1 = np.where(h >= 128, h - 256, h)
            for j, v in ((2 * w, v0), (2 * w + 1, v1)):
                col = p * 16 + j
                W[:, col] = v.astype(np.float32) * S[:, col // 32]
    return W


@needs_ref
def test_x86_int4_unpack_defect():
    """The x86 AVX2 build's int4 GEMM equals an fp32 GEMM on the mis-decoded
    weights above, bit for bit; the portable/NEON decode is the format's
    (extract_weights.py:589-592) and is what the GPU path implements."""
    M, N, K = 3, 64, 37
    P = po.bytes_((K, N // 2), po.seed(SEED, "x86.P"))
    S = po.uniform((K, N // 32), 0.005, 0.02, po.seed(SEED, "x86.S"))
    A, _ = rand_case(M, N, K, "x86")
    got_x86 = po.sgemm_q4b(A, P, S, np.zeros((M, N), np.float32), impl="ref")
    model = po.sgemm(A, x86_avx2_int4_weights(P, S), np.zeros((M, N), np.float32))
    assert bits_equal(got_x86, model)
    correct = po.sgemm_q4b(A, P, S, np.zeros((M, N), np.float32))
    assert not bits_equal(got_x86, correct)


# ---- reference-independent checks ------------------------------------------

def _bound_check(C, A, W, alpha=1.0):
    """|C - fp64 dot| <= K * 2^-23 * sum|a||w| + tiny (fp32 chain bound)."""
    exact = (np.float64(alpha) * A.astype(np.float64)) @ W.astype(np.float64)
    mag = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64))
    K = A.shape[1]
    tol = (K + 2) * 2.0 ** -23 * np.abs(alpha) * mag + 1e-30
    assert np.all(np.abs(C.astype(np.float64) - exact) <= tol)


def test_bruteforce_bound_all_kinds():
    M, N, K = 5, 96, 300
    A = po.normal((M, K), 0.0, 1.0, po.seed(SEED, "bf.A"))
    Bf = po.normal((K, N), 0.0, 0.02, po.seed(SEED, "bf.B"))
    Q = po.int8s((K, N), -127, 127, po.seed(SEED, "bf.Q"))
    P = po.bytes_((K, N // 2), po.seed(SEED, "bf.P"))
    S = po.uniform((K, N // 32), 0.005, 0.02, po.seed(SEED, "bf.S"))
    z = np.zeros((M, N), np.float32)
    _bound_check(po.sgemm(A, Bf, z.copy()), A, Bf)
    _bound_check(po.sgemm_qb(A, Q, 0.0123, z.copy()), A, po.dequant_i8(Q, np.float32(0.0123)))
    _bound_check(po.sgemm_q4b(A, P, S, z.copy()), A, po.dequant_i4(P, S))
    _bound_check(po.sgemm_q4b(A, P, S, z.copy(), alpha=0.75), A, po.dequant_i4(P, S), 0.75)


def test_exact_integer_results():
    """Integer A, unit scale and |sum| < 2^24: every rounding is exact."""
    M, N, K = 4, 64, 200
    A = po.int8s((M, K), -50, 50, po.seed(SEED, "int.A")).astype(np.float32)
    Q = po.int8s((K, N), -127, 127, po.seed(SEED, "int.Q"))
    got = po.sgemm_qb(A, Q, 1.0, np.zeros((M, N), np.float32))
    want = (A.astype(np.int64) @ Q.astype(np.int64)).astype(np.float32)
    assert bits_equal(got, want)
    P = po.bytes_((K, N // 2), po.seed(SEED, "int.P"))
    S = np.ones((K, N // 32), np.float32)
    got4 = po.sgemm_q4b(A, P, S, np.zeros((M, N), np.float32))
    W = po.dequant_i4(P, S).astype(np.int64)
    assert bits_equal(got4, (A.astype(np.int64) @ W).astype(np.float32))


def test_beta_alpha_semantics():
    M, N, K = 3, 48, 20
    A, C0 = rand_case(M, N, K, "ab")
    C0[0, 0] = np.nan
    Q = po.int8s((K, N), -127, 127, po.seed(SEED, "ab.Q"))
    # beta=0 clears NaN in C; alpha=0 leaves beta*C
    out = po.sgemm_qb(A, Q, 0.01, C0.copy(), alpha=0.0, beta=0.0)
    assert np.all(out == 0)
    out = po.sgemm_qb(A, Q, 0.01, C0.copy(), alpha=0.0, beta=0.5)
    assert bits_equal(out[:, 1:], (C0 * np.float32(0.5))[:, 1:])
    # scale 0 returns after the beta step (blas.c:765)
    out = po.sgemm_qb(A, Q, 0.0, C0.copy(), alpha=1.0, beta=1.0)
    assert bits_equal(out[:, 1:], C0[:, 1:])


def test_row_independence():
    """A row subset of A gives the same rows of C (enables sampled checks)."""
    M, N, K = 12, 64, 77
    A, _ = rand_case(M, N, K, "rows")
    P = po.bytes_((K, N // 2), po.seed(SEED, "rows.P"))
    S = po.uniform((K, N // 32), 0.005, 0.02, po.seed(SEED, "rows.S"))
    full = po.sgemm_q4b(A, P, S, np.zeros((M, N), np.float32))
    rows = [0, 5, 11]
    sub = po.sgemm_q4b(np.ascontiguousarray(A[rows]), P, S, np.zeros((3, N), np.float32))
    assert bits_equal(full[rows], sub)


def _splitmix64(state):
    state = (state + 0x9E3779B97F4A7C15) & (2**64 - 1)
    z = state
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & (2**64 - 1)
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & (2**64 - 1)
    return state, z ^ (z >> 31)


def test_seeded_generators_match_published_algorithms():
    """splitmix64 (Steele et al. 2014), FNV-1a 64 and Box-Muller restated in
    Python; the C generators feed both hosts, so their bytes must match."""
    import math
    h = 0xCBF29CE484222325
    for ch in b"stable":
        h = ((h ^ ch) * 0x100000001B3) & (2**64 - 1)
    st, seed = _splitmix64(0x5EED0000 ^ h)
    assert po.seed(0x5EED0000, "stable") == seed
    x = po.normal((4,), 0.0, 1.0, seed)
    st = seed
    want = []
    for _ in range(2):
        st, a = _splitmix64(st)
        st, b = _splitmix64(st)
        u1 = (a >> 11) * (1.0 / 9007199254740992.0)
        u2 = (b >> 11) * (1.0 / 9007199254740992.0)
        r = math.sqrt(-2.0 * math.log(u1))
        want += [r * math.cos(6.283185307179586 * u2), r * math.sin(6.283185307179586 * u2)]
    assert bits_equal(x, np.array(want, np.float32))
    q = po.int8s((4096,), -127, 127, seed)
    assert q.min() == -127 and q.max() == 127
