"""ctypes view of the CPU oracle and of the compiled reference.

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() and
by bench.py's cpu_baseline leg, always to check results or as the CPU
baseline, never as the thing measured on the GPU.

  Oracle      oracle/_build/liboracle.so   (pk_oracle.c, scalar restatement)
  Reference   oracle/_ref/libpkref.so      (csrc/*.c of the reference, built
                                            by oracle/Makefile, unmodified;
                                            x86 AVX2 code path)
              oracle/_ref/libpkref_portable.so  (same sources, blas.c on its
                                            portable code path, which matches
                                            the NEON path)
              oracle/_ref/libpkref_block.so     (the reference's static
                                            conformer_block, callable;
                                            ref_block_harness.c)
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "_build", "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libpkref.so")
REF_PORTABLE_SO = os.path.join(HERE, "_ref", "libpkref_portable.so")
REF_BLOCK_SO = {"portable": os.path.join(HERE, "_ref", "libpkref_block.so"),
                "x86": os.path.join(HERE, "_ref", "libpkref_block_x86.so")}

_f = ctypes.c_float
_i = ctypes.c_int
_p = ctypes.c_void_p
_u64 = ctypes.c_uint64
_sz = ctypes.c_size_t

_oracle = None
_refs = {}


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def oracle():
    """Load oracle/_build/liboracle.so (built by `make -C oracle restatement`)."""
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_SO):
            raise RuntimeError(f"oracle library missing: {ORACLE_SO} (run __graft_entry__.build())")
        lib = ctypes.CDLL(ORACLE_SO)
        gemm = [_i, _i, _i, _f, _p, _i]
        lib.pkor_sgemm_nn.argtypes = gemm + [_p, _i, _f, _p, _i]
        lib.pkor_sgemm_qb.argtypes = gemm + [_p, _f, _i, _f, _p, _i]
        lib.pkor_sgemm_q4b.argtypes = gemm + [_p, _p, _i, _f, _p, _i]
        for fn in (lib.pkor_sgemm_nn, lib.pkor_sgemm_qb, lib.pkor_sgemm_q4b):
            fn.restype = None
        lib.pkor_dequant_i8.argtypes = [ctypes.c_int8, _f]
        lib.pkor_dequant_i8.restype = _f
        lib.pkor_nibble_lo.argtypes = [ctypes.c_uint8]
        lib.pkor_nibble_lo.restype = _i
        lib.pkor_nibble_hi.argtypes = [ctypes.c_uint8]
        lib.pkor_nibble_hi.restype = _i
        lib.pkor_dequant_i8_matrix.argtypes = [_p, _i, _i, _i, _f, _p]
        lib.pkor_dequant_i4_matrix.argtypes = [_p, _i, _i, _i, _p, _p]
        lib.pkor_seed.argtypes = [_u64, ctypes.c_char_p]
        lib.pkor_seed.restype = _u64
        lib.pkor_fill_normal.argtypes = [_p, _sz, _f, _f, _u64]
        lib.pkor_fill_uniform.argtypes = [_p, _sz, _f, _f, _u64]
        lib.pkor_fill_int8.argtypes = [_p, _sz, _i, _i, _u64]
        lib.pkor_fill_bytes.argtypes = [_p, _sz, _u64]
        lib.pkor_layer_norm_rows.argtypes = [_p, _p, _p, _p, _i, _i, _i]
        lib.pkor_exp_poly.argtypes = [_f]
        lib.pkor_exp_poly.restype = _f
        lib.pkor_expf_ieee.argtypes = [_f]
        lib.pkor_expf_ieee.restype = _f
        lib.pkor_expf_ieee_rows.argtypes = [_p, _p, _sz]
        lib.pkor_expf_ieee_rows.restype = None
        lib.pkor_swish.argtypes = [_f]
        lib.pkor_swish.restype = _f
        lib.pkor_swish_rows.argtypes = [_p, _p, _sz]
        lib.pkor_swish_rows.restype = None
        lib.pkor_softmax_rows.argtypes = [_p, _i, _i]
        lib.pkor_dot8.argtypes = [_p, _p, _i]
        lib.pkor_dot8.restype = _f
        lib.pkor_attention_core.argtypes = [_p, _i, _p, _i, _p, _p, _p, _i, _i, _i, _i]
        lib.pkor_glu_rows.argtypes = [_p, _p, _i, _i]
        lib.pkor_depthwise_conv1d.argtypes = [_p, _p, _p, _p, _i, _i, _i]
        lib.pkor_encoder_run.argtypes = [_p, _i, _p, _i, _i, _p, _i, _i, _i, _p, _p]
        lib.pkor_encoder_run.restype = _i
        for fn in (lib.pkor_layer_norm_rows, lib.pkor_softmax_rows, lib.pkor_attention_core,
                   lib.pkor_glu_rows, lib.pkor_depthwise_conv1d):
            fn.restype = None
        _oracle = lib
    return _oracle


def have_ref(variant="ref"):
    return os.path.exists(REF_SO if variant == "ref" else REF_PORTABLE_SO)


def ref(variant="ref"):
    """Load a compiled reference: "ref" = AVX2 build, "portable" = blas.c's
    portable path."""
    if variant not in _refs:
        path = REF_SO if variant == "ref" else REF_PORTABLE_SO
        if not os.path.exists(path):
            raise RuntimeError(f"reference build missing: {path}")
        lib = ctypes.CDLL(path)
        gemm = [_i, _i, _i, _f, _p, _i]
        lib.cblas_sgemm.argtypes = [_i, _i, _i] + gemm + [_p, _i, _f, _p, _i]
        lib.cblas_sgemm_qb.argtypes = gemm + [_p, _f, _i, _f, _p, _i]
        lib.cblas_sgemm_q4b.argtypes = gemm + [_p, _p, _i, _f, _p, _i]
        for fn in (lib.cblas_sgemm, lib.cblas_sgemm_qb, lib.cblas_sgemm_q4b):
            fn.restype = None
        lib.pk_swish.argtypes = [_p, _i]
        lib.pk_swish.restype = None
        lib.pk_pool.restype = _p
        lib.pk_pool_nthreads.argtypes = [_p]
        lib.pk_pool_nthreads.restype = _i
        lib.pk_layer_norm_rows.argtypes = [_p, _p, _p, _p, _i, _i]
        lib.pk_softmax_rows.argtypes = [_p, _i, _i]
        lib.pk_depthwise_conv1d.argtypes = [_p, _p, _p, _p, _i, _i, _i]
        lib.cblas_sgemm_st.argtypes = [_i, _i, _i] + gemm + [_p, _i, _f, _p, _i]
        for fn in (lib.pk_layer_norm_rows, lib.pk_softmax_rows, lib.pk_depthwise_conv1d,
                   lib.cblas_sgemm_st):
            fn.restype = None
        _refs[variant] = lib
    return _refs[variant]


# ---- seeded data ---------------------------------------------------------

def seed(base, name):
    return int(oracle().pkor_seed(base, name.encode()))


def normal(shape, mean, std, s):
    out = np.empty(shape, np.float32)
    oracle().pkor_fill_normal(_ptr(out), out.size, mean, std, s)
    return out


def uniform(shape, lo, hi, s):
    out = np.empty(shape, np.float32)
    oracle().pkor_fill_uniform(_ptr(out), out.size, lo, hi, s)
    return out


def int8s(shape, lo, hi, s):
    out = np.empty(shape, np.int8)
    oracle().pkor_fill_int8(_ptr(out), out.size, lo, hi, s)
    return out


def bytes_(shape, s):
    out = np.empty(shape, np.uint8)
    oracle().pkor_fill_bytes(_ptr(out), out.size, s)
    return out


# ---- GEMM wrappers (row-major numpy arrays; C is updated in place) --------

def _check(A, C, M, N, K):
    assert A.dtype == np.float32 and C.dtype == np.float32
    assert A.flags.c_contiguous and C.flags.c_contiguous


def sgemm(A, B, C, alpha=1.0, beta=0.0, impl="oracle"):
    M, K = A.shape
    N = B.shape[1]
    _check(A, C, M, N, K)
    if impl == "oracle":
        oracle().pkor_sgemm_nn(M, N, K, alpha, _ptr(A), K, _ptr(B), N, beta, _ptr(C), N)
    else:
        ref(impl).cblas_sgemm(101, 111, 111, M, N, K, alpha, _ptr(A), K, _ptr(B), N, beta, _ptr(C), N)
    return C


def sgemm_qb(A, Q, scale, C, alpha=1.0, beta=0.0, impl="oracle"):
    M, K = A.shape
    N = Q.shape[1]
    _check(A, C, M, N, K)
    assert Q.dtype == np.int8
    fn = oracle().pkor_sgemm_qb if impl == "oracle" else ref(impl).cblas_sgemm_qb
    fn(M, N, K, alpha, _ptr(A), K, _ptr(Q), scale, N, beta, _ptr(C), N)
    return C


def sgemm_q4b(A, P, scales, C, alpha=1.0, beta=0.0, impl="oracle"):
    """P: packed int4 [K][N/2] uint8; scales: fp32 [K][N/32]."""
    M, K = A.shape
    N = P.shape[1] * 2
    _check(A, C, M, N, K)
    assert P.dtype == np.uint8 and scales.dtype == np.float32
    fn = oracle().pkor_sgemm_q4b if impl == "oracle" else ref(impl).cblas_sgemm_q4b
    fn(M, N, K, alpha, _ptr(A), K, _ptr(P), _ptr(scales), N // 2, beta, _ptr(C), N)
    return C


def dequant_i4(P, scales):
    K, half = P.shape
    N = half * 2
    out = np.empty((K, N), np.float32)
    oracle().pkor_dequant_i4_matrix(_ptr(P), K, N, half, _ptr(scales), _ptr(out))
    return out


def dequant_i8(Q, scale):
    K, N = Q.shape
    out = np.empty((K, N), np.float32)
    oracle().pkor_dequant_i8_matrix(_ptr(Q), K, N, N, scale, _ptr(out))
    return out


def swish(x):
    """Oracle Swish (the source's IEEE division) of every element of x."""
    x = _f32(x)
    y = np.empty_like(x)
    oracle().pkor_swish_rows(_ptr(x), _ptr(y), x.size)
    return y


def expf_ieee(x):
    """The oracle's expf (double evaluation, one rounding) of every element."""
    x = _f32(x)
    y = np.empty_like(x)
    oracle().pkor_expf_ieee_rows(_ptr(x), _ptr(y), x.size)
    return y


def ref_swish(x):
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    ref().pk_swish(_ptr(y), y.size)
    return y


# ---- conformer-block operations (pk_oracle_block.c) ------------------------

def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def layer_norm(x, gamma, beta, x86_rsqrt=False):
    """Oracle LayerNorm of the rows of x (correctly rounded 1/sqrt unless
    x86_rsqrt, which restates the compiled vrsqrtss form)."""
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    out = np.empty_like(x)
    oracle().pkor_layer_norm_rows(_ptr(x), _ptr(gamma), _ptr(beta), _ptr(out),
                                  x.shape[0], x.shape[1], int(x86_rsqrt))
    return out


def ref_layer_norm(x, gamma, beta):
    x, gamma, beta = _f32(x), _f32(gamma), _f32(beta)
    out = np.empty_like(x)
    ref().pk_layer_norm_rows(_ptr(x), _ptr(gamma), _ptr(beta), _ptr(out), x.shape[0], x.shape[1])
    return out


def softmax(x):
    x = _f32(x).copy()
    oracle().pkor_softmax_rows(_ptr(x), x.shape[0], x.shape[1])
    return x


def ref_softmax(x):
    x = _f32(x).copy()
    ref().pk_softmax_rows(_ptr(x), x.shape[0], x.shape[1])
    return x


def attention_core(qkv, P, pu, pv, H=8, Dh=128):
    """Oracle relative-position attention: qkv [T][3*H*Dh] (bias added),
    P [2T-1][H*Dh] -> [T][H*Dh]."""
    qkv, P, pu, pv = _f32(qkv), _f32(P), _f32(pu), _f32(pv)
    T = qkv.shape[0]
    out = np.empty((T, H * Dh), np.float32)
    oracle().pkor_attention_core(_ptr(qkv), qkv.shape[1], _ptr(P), P.shape[1], _ptr(pu), _ptr(pv),
                                 _ptr(out), H * Dh, T, H, Dh)
    return out


def glu(x):
    x = _f32(x)
    D = x.shape[1] // 2
    out = np.empty((x.shape[0], D), np.float32)
    oracle().pkor_glu_rows(_ptr(x), _ptr(out), x.shape[0], D)
    return out


def depthwise(x, w, b):
    """Oracle depthwise conv, channel-major x [C][T], w [C][K]."""
    x, w, b = _f32(x), _f32(w), _f32(b)
    out = np.empty_like(x)
    oracle().pkor_depthwise_conv1d(_ptr(x), _ptr(w), _ptr(b), _ptr(out), x.shape[0], x.shape[1],
                                   w.shape[1])
    return out


def ref_depthwise(x, w, b):
    x, w, b = _f32(x), _f32(w), _f32(b)
    out = np.empty_like(x)
    ref().pk_depthwise_conv1d(_ptr(x), _ptr(w), _ptr(b), _ptr(out), x.shape[0], x.shape[1],
                              w.shape[1])
    return out


def ref_sgemm_st(A, B, transB, C=None):
    """The reference's single-threaded cblas_sgemm_st, NoTrans x (NoTrans | Trans)."""
    A, B = _f32(A), _f32(B)
    M, K = A.shape
    N = B.shape[0] if transB else B.shape[1]
    C = np.zeros((M, N), np.float32) if C is None else C
    ref().cblas_sgemm_st(101, 111, 112 if transB else 111, M, N, K, 1.0, _ptr(A), K, _ptr(B),
                         B.shape[1], 0.0, _ptr(C), N)
    return C


_ref_block = {}


def have_ref_block(variant="portable"):
    return os.path.exists(REF_BLOCK_SO[variant])


def ref_blocks(blocks, n_blocks, pe_slice, x, variant="portable"):
    """Run the reference's conformer_block n_blocks times on x [T][1024] (in a
    copy), blocks being a ctypes array of pk_gpu_block_weights.  variant
    "portable": weight GEMMs from blas.c's portable path (decodes int4 as the
    format defines); "x86": the reference's x86 build throughout (its AVX2
    int4 unpack mis-decodes nibbles; used for timing only)."""
    if variant not in _ref_block:
        if not have_ref_block(variant):
            raise RuntimeError(f"reference block harness missing: {REF_BLOCK_SO[variant]}")
        lib = ctypes.CDLL(REF_BLOCK_SO[variant])
        lib.pkref_conformer_blocks.argtypes = [_p, _i, _p, _p, _i]
        lib.pkref_conformer_blocks.restype = _i
        _ref_block[variant] = lib
    x = _f32(x).copy()
    pe_slice = _f32(pe_slice)
    rc = _ref_block[variant].pkref_conformer_blocks(ctypes.cast(blocks, _p), n_blocks,
                                                    _ptr(pe_slice), _ptr(x), x.shape[0])
    if rc:
        raise RuntimeError("pkref_conformer_blocks failed")
    return x


def ref_block_threads(variant="portable"):
    """Threads of the block harness's own reference thread pool."""
    lib = _ref_block[variant]          # loaded by a previous ref_blocks call
    lib.pk_pool.restype = _p
    lib.pk_pool_nthreads.argtypes = [_p]
    lib.pk_pool_nthreads.restype = _i
    return lib.pk_pool_nthreads(lib.pk_pool())


def ref_pre_encode(w, mel, variant="portable"):
    """The reference's pre_encode_and_scale on mel [128][n_frames] with the
    ctypes pk_gpu_pre_encode_weights w; returns x [T'][1024]."""
    if variant not in _ref_block:
        if not have_ref_block(variant):
            raise RuntimeError(f"reference block harness missing: {REF_BLOCK_SO[variant]}")
        lib = ctypes.CDLL(REF_BLOCK_SO[variant])
        lib.pkref_conformer_blocks.argtypes = [_p, _i, _p, _p, _i]
        lib.pkref_conformer_blocks.restype = _i
        _ref_block[variant] = lib
    lib = _ref_block[variant]
    lib.pkref_pre_encode.argtypes = [_p, _p, _i, _p]
    lib.pkref_pre_encode.restype = _i
    mel = _f32(mel)
    n = mel.shape[1]
    tp = (((n - 1) // 2 + 1 - 1) // 2 + 1 - 1) // 2 + 1
    out = np.empty((tp, 1024), np.float32)
    got = lib.pkref_pre_encode(ctypes.byref(w), _ptr(mel), n, _ptr(out))
    if got != tp:
        raise RuntimeError(f"pkref_pre_encode returned {got}, expected {tp}")
    return out


def encoder(blocks, n_blocks, pe_table, pe_center, x, chunk, overlap, snapshots=False):
    """The oracle's whole encoder (pk_oracle_encoder.c): n_blocks conformer
    blocks (a ctypes array of pk_gpu_block_weights) over x [T][1024], chunked
    as the reference chunks.  Returns the output, or (output, [n_blocks][T][1024]
    outputs after every block) with snapshots."""
    x = _f32(x)
    pe_table = _f32(pe_table)
    T = x.shape[0]
    out = np.empty_like(x)
    snap = np.empty((n_blocks, T, x.shape[1]), np.float32) if snapshots else None
    rc = oracle().pkor_encoder_run(ctypes.cast(blocks, _p), n_blocks, _ptr(pe_table),
                                   pe_table.shape[0], pe_center, _ptr(x), T, chunk, overlap,
                                   _ptr(out), _ptr(snap))
    if rc:
        raise RuntimeError("pkor_encoder_run failed")
    return (out, snap) if snapshots else out
