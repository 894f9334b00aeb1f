"""CPU: the oracle's conformer-block operations (oracle/pk_oracle_block.c)
pinned against the reference compiled from its own sources
(oracle/_ref/libpkref.so, the x86 AVX2 build), and against closed forms.

Bit-exact pins: LayerNorm (with the compiled vrsqrtss form restated),
softmax for row lengths that are multiples of 8, the NT dot products of
the attention scores, the whole attention core for T % 8 == 0, and the
depthwise convolution for every T.  Tolerance pins (the reference uses
CPU-model-specific approximations there): LayerNorm with a correctly
rounded 1/sqrt, softmax tails, GLU, Swish with the source's IEEE division.
Closed-form pins: the double-evaluated expf against the correctly rounded
e^x, Swish against its polynomial evaluated in double, GLU.  The whole
encoder composed of these operations is pinned against the reference's own
conformer blocks within tolerance, and is independent of the thread count."""
import numpy as np
import pytest

import pyoracle as po

needs_ref = pytest.mark.skipif(not po.have_ref(), reason="reference build missing (oracle/Makefile ref)")
RNG = np.random.default_rng(0x5EEDB10C)


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def ulps(a, b):
    a = np.asarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.asarray(b, np.float32).view(np.int32).astype(np.int64)
    return np.abs(a - b)


def rows(n, d, scale=1.0, shift=0.0):
    return (RNG.standard_normal((n, d)) * scale + shift).astype(np.float32)


@needs_ref
@pytest.mark.parametrize("D", [1024, 64, 1000])
def test_layer_norm_x86_form_is_bit_exact(D):
    x = rows(48, D, 3.0, 0.7)
    g, b = rows(1, D)[0], rows(1, D)[0]
    assert bits_equal(po.layer_norm(x, g, b, x86_rsqrt=True), po.ref_layer_norm(x, g, b))


@needs_ref
def test_layer_norm_correctly_rounded_form_within_tolerance():
    """mode 0 differs from the reference only through 1/sqrt: a few ulp of
    the normalised value, relative to the row's scale."""
    x = rows(256, 1024, 2.0, -0.3)
    g, b = rows(1, 1024)[0], rows(1, 1024)[0]
    ref, ora = po.ref_layer_norm(x, g, b), po.layer_norm(x, g, b)
    rel = np.abs(ref - ora) / np.maximum(np.abs(ref), 1.0)
    assert rel.max() < 1e-6
    # the sums are shared: rows where 1/sqrt agrees are identical
    assert np.mean([bits_equal(ref[i], ora[i]) for i in range(256)]) > 0.2


def test_layer_norm_closed_form():
    """Against fp64 LayerNorm: mean/var/affine within fp32 rounding."""
    x = rows(8, 1024, 5.0, 2.0)
    g, b = rows(1, 1024)[0], rows(1, 1024)[0]
    x64 = x.astype(np.float64)
    m = x64.mean(1, keepdims=True)
    v = ((x64 - m) ** 2).mean(1, keepdims=True)
    want = (x64 - m) / np.sqrt(v + 1e-5) * g + b
    assert np.abs(po.layer_norm(x, g, b) - want).max() < 2e-5


@needs_ref
@pytest.mark.parametrize("T", [416, 408, 104, 8, 832])
def test_softmax_bit_exact_multiple_of_8(T):
    s = rows(24, T, 4.0)
    assert bits_equal(po.softmax(s), po.ref_softmax(s))


@needs_ref
@pytest.mark.parametrize("T", [300, 108, 7, 1, 13])
def test_softmax_tail_within_tolerance(T):
    s = rows(24, T, 4.0)
    a, b = po.softmax(s), po.ref_softmax(s)
    assert np.abs(a - b).max() <= 4e-7
    assert np.allclose(a.sum(1), 1.0, atol=1e-5)


def test_exp_poly_accuracy():
    """The reference's polynomial exp: the 5-term Taylor remainder r^6/720 at
    |r| <= ln2/2 bounds it near 3e-6 relative on [-87, 0] ("~1e-6 relative",
    tensor_ops.c:7-9); exact at 0."""
    x = np.linspace(-87.0, 0.0, 20001, dtype=np.float32)
    got = np.array([po.oracle().pkor_exp_poly(float(v)) for v in x], np.float32)
    want = np.exp(x.astype(np.float64))
    assert np.max(np.abs(got - want) / want) < 4e-6
    assert po.oracle().pkor_exp_poly(0.0) == 1.0


@needs_ref
@pytest.mark.parametrize("K", [128, 64, 8])
def test_nt_dot_bit_exact(K):
    """K % 8 == 0 (the head dimension is 128); the scalar tail for other K is
    compiled differently and is never used by the encoder."""
    A, B = rows(19, K), rows(37, K)
    want = po.ref_sgemm_st(A, B, transB=True)
    got = np.empty_like(want)
    for i in range(A.shape[0]):
        a = np.ascontiguousarray(A[i])
        for j in range(B.shape[0]):
            b = np.ascontiguousarray(B[j])
            got[i, j] = po.oracle().pkor_dot8(po._ptr(a), po._ptr(b), K)
    assert bits_equal(got, want)


def relative_shift_padded(bd, T):
    """encoder.c:230-254 as written: pad a zero column, view the flat buffer
    from offset T with row stride 2T-1."""
    L = 2 * T - 1
    padded = np.zeros((T, 2 * T), np.float32)
    padded[:, 1:] = bd
    flat = padded.reshape(-1)
    return flat[T + np.arange(T)[:, None] * L + np.arange(T)[None, :]]


def test_relative_shift_closed_form():
    T = 9
    bd = rows(T, 2 * T - 1)
    closed = np.array([[bd[i, T - 1 - i + j] for j in range(T)] for i in range(T)], np.float32)
    assert bits_equal(relative_shift_padded(bd, T), closed)


def reference_attention(qkv, P, pu, pv, H=8, Dh=128):
    """The reference's attention core composed from its compiled exported
    functions: cblas_sgemm_st (NT for AC/BD, NN for scores x V) and
    pk_softmax_rows, with the head gather, the relative shift and the score
    combine of encoder.c:315-406 done in numpy (exact fp32 adds/multiplies)."""
    T, D = qkv.shape[0], H * Dh
    scale = np.float32(1.0) / np.sqrt(np.float32(Dh))
    out = np.empty((T, D), np.float32)
    scores = np.empty((H, T, T), np.float32)
    for h in range(H):
        q = qkv[:, h * Dh:(h + 1) * Dh]
        k = np.ascontiguousarray(qkv[:, D + h * Dh:D + (h + 1) * Dh])
        qu = np.ascontiguousarray(q + pu[h * Dh:(h + 1) * Dh])
        qv = np.ascontiguousarray(q + pv[h * Dh:(h + 1) * Dh])
        ac = po.ref_sgemm_st(qu, k, transB=True)
        bd = po.ref_sgemm_st(qv, np.ascontiguousarray(P[:, h * Dh:(h + 1) * Dh]), transB=True)
        scores[h] = (ac + relative_shift_padded(bd, T)) * scale
    flat = np.ascontiguousarray(scores.reshape(H * T, T))
    po.ref().pk_softmax_rows(po._ptr(flat), H * T, T)
    scores = flat.reshape(H, T, T)
    for h in range(H):
        v = np.ascontiguousarray(qkv[:, 2 * D + h * Dh:2 * D + (h + 1) * Dh])
        out[:, h * Dh:(h + 1) * Dh] = po.ref_sgemm_st(np.ascontiguousarray(scores[h]), v, transB=False)
    return out


def attention_inputs(T, H=8, Dh=128):
    D = H * Dh
    qkv = rows(T, 3 * D, 0.5)
    P = rows(2 * T - 1, D, 0.5)
    return qkv, P, rows(1, D, 0.1)[0], rows(1, D, 0.1)[0]


@needs_ref
@pytest.mark.parametrize("T", [24, 64])
def test_attention_core_bit_exact(T):
    qkv, P, pu, pv = attention_inputs(T)
    assert bits_equal(po.attention_core(qkv, P, pu, pv), reference_attention(qkv, P, pu, pv))


@needs_ref
def test_attention_core_tail_within_tolerance():
    qkv, P, pu, pv = attention_inputs(21)
    a, b = po.attention_core(qkv, P, pu, pv), reference_attention(qkv, P, pu, pv)
    assert np.abs(a - b).max() / np.abs(b).max() < 1e-6


@needs_ref
@pytest.mark.parametrize("T", [416, 408, 108, 20, 13, 12, 9, 8, 5, 1])
def test_depthwise_bit_exact(T):
    x = rows(16, T)
    w, b = rows(16, 9), rows(1, 16)[0]
    assert bits_equal(po.depthwise(x, w, b), po.ref_depthwise(x, w, b))


def test_glu_closed_form():
    x = rows(32, 2 * 256, 3.0)
    va, vb = x[:, :256].astype(np.float64), x[:, 256:].astype(np.float64)
    want = va / (1.0 + np.exp(-vb))
    got = po.glu(x)
    assert np.all(ulps(got, want.astype(np.float32)) <= 2)


@pytest.mark.skipif(not po.have_ref_block(), reason="reference block harness missing")
@pytest.mark.parametrize("attn_scale,lo,hi", [(0.01, 1e-2, None), (0.0005, None, 1e-4)])
def test_reference_sensitivity(attn_scale, lo, hi):
    """How the reference's own conformer blocks amplify a 1-ulp change of one
    input element over six blocks.  With the workloads' int8 attention
    statistics (codes uniform in [-127, 127], scale 0.01) the attention
    logits reach several hundred and the difference grows about tenfold per
    block, to more than 1e-2 relative: on that model only arithmetic that is
    bit-identical to the host's (the GEMM drop-in) can reproduce its outputs,
    and the reference would itself give different results on a CPU with
    other vrcpps / vrsqrtss tables.  With trained-like projections (scale
    0.0005) it stays below 1e-4."""
    import blockgen as bg
    blocks = [bg.Block(0xB10C0 + i, attn_scale=attn_scale) for i in range(6)]
    arr = bg.block_array(blocks)
    pe = bg.pe_slice(bg.pe_table(), 64)
    x = rows(64, 1024)
    x2 = x.copy()
    x2[3, 7] = np.nextafter(x2[3, 7], np.float32(10))
    a, b = po.ref_blocks(arr, 6, pe, x), po.ref_blocks(arr, 6, pe, x2)
    rel = np.abs(a - b).max() / np.abs(a).max()
    if lo is not None:
        assert rel > lo
    if hi is not None:
        assert rel < hi


def expl_rounded(x):
    """e^x with a 64-bit significand (x87 expl), rounded once to float: the
    correctly rounded expf except within 2^-39 of a rounding boundary."""
    return np.exp(x.astype(np.longdouble)).astype(np.float32)


def test_expf_ieee_correctly_rounded():
    """pkor_expf_ieee against the correctly rounded e^x: every 61st float bit
    pattern of [-104, 89] (about 35 M inputs), the overflow and underflow
    boundaries, and special values.  (The same comparison over all 2^32
    inputs found no difference.)"""
    assert np.finfo(np.longdouble).nmant >= 63
    lo = np.float32(-104.0).view(np.uint32)              # negative floats: descending bits
    hi = np.float32(89.0).view(np.uint32)
    for bits in (np.arange(0x80000000, lo + 1, 61, dtype=np.uint64),
                 np.arange(0, hi + 1, 61, dtype=np.uint64)):
        for part in np.array_split(bits.astype(np.uint32), 16):
            x = part.view(np.float32)
            got = po.expf_ieee(x)
            want = expl_rounded(x)
            bad = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
            assert bad.size == 0, f"x={x[bad[:4]]!r} got {got[bad[:4]]!r} want {want[bad[:4]]!r}"
    edge = np.array([0.0, -0.0, 1e-30, -1e-30, 88.72283, 88.72284, 88.7229, 89.0, 89.5,
                     -87.33654, -87.33655, -103.27893, -103.97207, -103.97208, -104.0, -120.0,
                     1e30, -1e30, np.inf, -np.inf], np.float32)
    with np.errstate(over="ignore"):
        want = np.exp(edge.astype(np.longdouble)).astype(np.float32)
    assert np.array_equal(po.expf_ieee(edge).view(np.uint32), want.view(np.uint32))
    assert np.isnan(po.expf_ieee(np.array([np.nan], np.float32))[0])


def swish_closed_form(v):
    """pk_swish's polynomial evaluated in double: the same k and the float
    constants of tensor_ops.c:98-120, every other step exact."""
    v = np.asarray(v, np.float32)
    t = np.clip(-v, np.float32(-87.0), np.float32(87.0)).astype(np.float32)
    k = np.rint(t * np.float32(1.44269504088896341)).astype(np.float64)
    r = t.astype(np.float64) - k * np.float64(np.float32(0.69314718055994529))
    c = [np.float64(np.float32(1.0 / n)) for n in (120, 24, 6)] + [0.5, 1.0, 1.0]
    y = np.zeros_like(r) + c[0]
    for ci in c[1:]:
        y = y * r + ci
    return v.astype(np.float64) / (1.0 + y * np.exp2(k))


def test_swish_closed_form():
    """Each float step of the oracle's Swish rounds once (fmas, the product
    with 2^k, the division, the multiply): within 4 ulp of the closed form.
    A wrong or missing polynomial term would be off by hundreds of ulp."""
    x = (RNG.standard_normal(2_000_000) * 6.0).astype(np.float32)
    x[:8] = [0.0, -0.0, 87.0, -87.0, 90.0, -90.0, 1e-30, -3.5]
    got = po.swish(x).astype(np.float64)
    want = swish_closed_form(x)
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(got - want) <= 4 * ulp + 1e-44)


@needs_ref
def test_swish_within_tolerance_of_reference():
    """The reference build's rcpps + Newton step against the source's IEEE
    division: a few ulp."""
    x = (RNG.standard_normal(1_000_000) * 4.0).astype(np.float32)
    got, want = po.swish(x), po.ref_swish(x)
    ulp = np.spacing(np.abs(want).astype(np.float32))
    assert np.all(np.abs(got.astype(np.float64) - want) <= 4 * ulp + 1e-37)
    assert np.mean(got == want) > 0.3


@pytest.mark.skipif(not po.have_ref_block(), reason="reference block harness missing")
@pytest.mark.parametrize("T,chunk", [(72, 0), (150, 64)])
def test_encoder_oracle_matches_reference_blocks(T, chunk):
    """The oracle's whole encoder against the reference's own conformer
    blocks (ref_block_harness.c) chunk by chunk, trained-like attention
    weights: they differ only where the reference build uses vrsqrtss,
    vrcpps and libmvec's expf, well below 1e-4 after four blocks."""
    import blockgen as bg
    blocks = [bg.Block(0xB10D0 + i, attn_scale=0.0005) for i in range(4)]
    arr = bg.block_array(blocks)
    pe = bg.pe_table()
    x = rows(T, 1024)
    got = po.encoder(arr, 4, pe, 4999, x, chunk, 8)
    want = np.empty_like(x)
    C = chunk if chunk > 0 else T
    for o0 in range(0, T, C):
        o1 = min(o0 + C, T)
        i0, i1 = max(o0 - 8, 0) if chunk > 0 else 0, min(o1 + 8, T) if chunk > 0 else T
        y = po.ref_blocks(arr, 4, bg.pe_slice(pe, i1 - i0), x[i0:i1])
        want[o0:o1] = y[o0 - i0:o1 - i0]
    rel = np.abs(got - want).max() / np.abs(want).max()
    assert rel < 1e-4, rel


def test_encoder_oracle_thread_count_invariant():
    """Rows and chunks are spread over threads; no chain or sum is split, so
    one thread and all threads give the same bits."""
    import subprocess
    import sys
    code = ("import sys, hashlib, numpy as np; sys.path[:0] = {paths!r}; import blockgen as bg, "
            "pyoracle as po; blocks = [bg.Block(0xB10C0)]; arr = bg.block_array(blocks); "
            "x = np.random.default_rng(7).standard_normal((100, 1024)).astype(np.float32); "
            "print(hashlib.sha256(po.encoder(arr, 1, bg.pe_table(), 4999, x, 40, 8).tobytes())"
            ".hexdigest())")
    import os
    here = os.path.dirname(os.path.abspath(__file__))
    paths = [here, os.path.join(os.path.dirname(here), "oracle")]
    digests = set()
    for threads in ("1", "5"):
        out = subprocess.run([sys.executable, "-c", code.format(paths=paths)], capture_output=True,
                             text=True, env=dict(os.environ, OMP_NUM_THREADS=threads), timeout=300)
        assert out.returncode == 0, out.stderr[-2000:]
        digests.add(out.stdout.strip())
    assert len(digests) == 1
