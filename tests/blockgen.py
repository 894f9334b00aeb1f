"""Synthetic conformer-block parameters in the reference's formats, shared by
the block tests: numpy arrays kept alive together with the ctypes
pk_gpu_block_weights that points at them.

Statistics follow the workloads: int4 feed-forward weights (nibble codes
uniform 0..15, decoded signed, scales ~U(0.005, 0.02) per 32 columns), int8
attention projections (uniform -127..127, per-tensor scale 0.01), fp32
pointwise convolutions ~N(0, 0.02), depthwise taps ~N(0, 1/9), biases
~N(0, 0.02), LayerNorm gain 1 + N(0, 0.1) and bias N(0, 0.1).

attn_scale sets the int8 attention projections' scale.  The workloads'
0.01 (weights of standard deviation ~0.73) makes attention logits of several
hundred, and the reference itself then amplifies a 1-ulp difference about
tenfold per block (test_oracle_block.test_reference_sensitivity); 0.0005
(~0.037, about 1/sqrt(1024), like trained projections) keeps it flat."""
import ctypes

import numpy as np

from pkgpu import pk

D, FF, H, DH, KCONV = 1024, 4096, 8, 128, 9


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data)


# int8 codes uniform in [-127, 127] have standard deviation 127/sqrt(3)
I8_CODE_STD = 73.32


class Block:
    """One conformer block's parameters with random values.  mode picks the
    weight directory whose formats the linears take (download_weights.py:20):
    "mixed" (int4 FF linears, int8 attention projections), "int8" (every
    linear int8, FF scale 0.0008) or "fp32" (every linear fp32, with the
    int8 weights' spread).  The mixed model's values do not depend on the
    other modes' code paths (same draws in the same order)."""

    def __init__(self, seed, qkv_bits=8, attn_scale=0.01, mode="mixed"):
        assert mode in ("mixed", "int8", "fp32")
        rng = np.random.default_rng(seed)
        self.keep = []
        f32 = lambda a: self._keep(np.ascontiguousarray(a, dtype=np.float32))
        normal = lambda shape, s: f32(rng.standard_normal(shape) * s)
        w = pk.BlockWeights()

        def ff(K, N):
            if mode == "int8":
                return i8(K, N, 0.0008)
            if mode == "fp32":
                return fp(K, N, 0.06)
            return i4(K, N)

        def proj(K, N, scale):
            return fp(K, N, scale * I8_CODE_STD) if mode == "fp32" else i8(K, N, scale)

        def i4(K, N):
            data = self._keep(rng.integers(0, 256, (K, N // 2), dtype=np.uint8))
            scales = f32(rng.uniform(0.005, 0.02, (K, N // 32)))
            return pk.Weight(data.ctypes.data, 0.0, scales.ctypes.data, 4)

        def i8(K, N, scale=0.01):
            data = self._keep(rng.integers(-127, 128, (K, N), dtype=np.int8))
            return pk.Weight(data.ctypes.data, scale, None, 8)

        def fp(K, N, s=0.02):
            data = normal((K, N), s)
            return pk.Weight(data.ctypes.data, 0.0, None, 32)

        def ln():
            return f32(1.0 + rng.standard_normal(D) * 0.1).ctypes.data, normal(D, 0.1).ctypes.data

        w.norm_ff1_w, w.norm_ff1_b = ln()
        w.ff1_linear1_w, w.ff1_linear1_b = ff(D, FF), normal(FF, 0.02).ctypes.data
        w.ff1_linear2_w, w.ff1_linear2_b = ff(FF, D), normal(D, 0.02).ctypes.data
        w.norm_sa_w, w.norm_sa_b = ln()
        w.linear_qkv_w = proj(D, 3 * D, attn_scale) if qkv_bits == 8 else fp(D, 3 * D)
        w.linear_qkv_b = normal(3 * D, 0.02).ctypes.data
        w.linear_pos_w = proj(D, D, attn_scale)
        w.linear_out_w, w.linear_out_b = proj(D, D, attn_scale), normal(D, 0.02).ctypes.data
        w.pos_bias_u, w.pos_bias_v = normal(D, 0.02).ctypes.data, normal(D, 0.02).ctypes.data
        w.norm_conv_w, w.norm_conv_b = ln()
        w.conv_pw1_w, w.conv_pw1_b = normal((2 * D, D), 0.02).ctypes.data, normal(2 * D, 0.02).ctypes.data
        w.conv_dw_w, w.conv_dw_b = normal((D, KCONV), 1.0 / 3.0).ctypes.data, normal(D, 0.02).ctypes.data
        w.conv_pw2_w, w.conv_pw2_b = normal((D, D), 0.02).ctypes.data, normal(D, 0.02).ctypes.data
        w.norm_ff2_w, w.norm_ff2_b = ln()
        w.ff2_linear1_w, w.ff2_linear1_b = ff(D, FF), normal(FF, 0.02).ctypes.data
        w.ff2_linear2_w, w.ff2_linear2_b = ff(FF, D), normal(D, 0.02).ctypes.data
        w.norm_out_w, w.norm_out_b = ln()
        self.w = w

    def _keep(self, a):
        self.keep.append(a)
        return a


def block_array(blocks):
    arr = (pk.BlockWeights * len(blocks))()
    for i, b in enumerate(blocks):
        arr[i] = b.w
    return arr


def pe_table(rows=9999, center=4999):
    """Sinusoidal relative-position table, row p holding position center - p
    (the layout pos_encoding.pe_table has in the reference's weights)."""
    pos = (center - np.arange(rows, dtype=np.float64))[:, None]
    div = np.exp(-(2.0 * np.arange(D // 2)) * np.log(10000.0) / D)[None, :]
    pe = np.empty((rows, D), np.float32)
    pe[:, 0::2] = np.sin(pos * div)
    pe[:, 1::2] = np.cos(pos * div)
    return pe


def pe_slice(pe, T, center=4999):
    """encoder.c:220-228: rows [center - T + 1, center + T)."""
    return np.ascontiguousarray(pe[center - T + 1:center + T])


class PreEncode:
    """pre_encode parameters (PreEncodeWeights, parakeet.h): 3x3 convolutions
    ~N(0, 0.1) (pointwise ~N(0, 1/16)), biases ~N(0, 0.02), int8 out_w codes
    uniform in [-127, 127] with scale 0.01 / 64 (or fp32 ~N(0, 0.02))."""

    def __init__(self, seed, out_bits=8):
        rng = np.random.default_rng(seed)
        self.keep = []

        def f32(a):
            a = np.ascontiguousarray(a, dtype=np.float32)
            self.keep.append(a)
            return a.ctypes.data

        normal = lambda shape, sd: f32(rng.standard_normal(shape) * sd)
        w = pk.PreEncodeWeights()
        w.conv0_w, w.conv0_b = normal((256, 9), 0.3), normal(256, 0.02)
        w.conv2_w, w.conv2_b = normal((256, 9), 0.3), normal(256, 0.02)
        w.conv3_w, w.conv3_b = normal((256, 256), 1.0 / 16), normal(256, 0.02)
        w.conv5_w, w.conv5_b = normal((256, 9), 0.3), normal(256, 0.02)
        w.conv6_w, w.conv6_b = normal((256, 256), 1.0 / 16), normal(256, 0.02)
        if out_bits == 8:
            q = rng.integers(-127, 128, (4096, 1024), dtype=np.int8)
            self.keep.append(q)
            w.out_w = pk.Weight(q.ctypes.data, 0.01 / 64, None, 8)
        else:
            w.out_w = pk.Weight(normal((4096, 1024), 0.02), 0.0, None, 32)
        w.out_b = normal(1024, 0.02)
        self.w = w
