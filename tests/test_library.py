"""CPU-side checks of the C-ABI libraries (no GPU needed): they load, export
every entry point the headers declare, the drop-in shim exports the
reference's three symbols, and without a gfx950 device every entry point
fails loudly instead of computing on the CPU."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from pkgpu import ROOT, gpu_available, pk


def test_libpk_gpu_exports_every_header_function():
    lib = pk.load()
    names = pk.header_functions()
    assert len(names) >= 15
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_shim_exports_reference_blas_symbols():
    """libpk_gpu_cblas.so provides csrc/blas.h:38-69's weight GEMMs."""
    out = subprocess.run(["nm", "-D", "--defined-only", pk.SHIM_PATH], capture_output=True,
                         text=True, check=True).stdout
    defined = set(re.findall(r" T (\w+)", out))
    assert {"cblas_sgemm", "cblas_sgemm_qb", "cblas_sgemm_q4b"} <= defined
    # the shim must not carry a CPU GEMM of its own: it only forwards
    assert not {"cblas_sgemv", "cblas_sgemm_st"} & defined
    hdr = open(os.path.join(ROOT, "include", "pk_gpu_cblas.h")).read()
    for sym in ("cblas_sgemm", "cblas_sgemm_qb", "cblas_sgemm_q4b"):
        assert re.search(rf"\b{sym}\s*\(", hdr), sym


def test_library_has_no_cpu_gemm_fallback():
    """libpk_gpu.so links HIP and does not import the reference BLAS."""
    out = subprocess.run(["nm", "-D", "--undefined-only", pk.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    assert "cblas_" not in out
    deps = subprocess.run(["ldd", pk.LIB_PATH], capture_output=True, text=True).stdout
    assert "libamdhip64" in deps


@pytest.mark.skipif(gpu_available(), reason="checks the no-device error path")
def test_no_device_is_an_error_not_a_fallback():
    lib = pk.load()
    assert lib.pk_gpu_init(0) == -5          # PK_GPU_ENODEV
    assert b"device" in lib.pk_gpu_last_error().lower() or lib.pk_gpu_last_error()
    A = np.ones((2, 4), np.float32)
    Q = np.ones((4, 16), np.int8)
    C = np.full((2, 16), 7.0, np.float32)
    rc = lib.pk_gpu_gemm_i8(2, 16, 4, 1.0, A.ctypes.data, 4, Q.ctypes.data, 0.5, 16, 0.0,
                            C.ctypes.data, 16)
    assert rc == -5
    assert np.all(C == 7.0)                   # nothing was computed on the host


def test_argument_validation_precedes_device_use():
    lib = pk.load()
    A = np.ones((2, 4), np.float32)
    C = np.zeros((2, 64), np.float32)
    P = np.zeros((4, 24), np.uint8)
    S = np.ones((4, 2), np.float32)
    # int4 rows hold N/2 bytes: N must be even
    assert lib.pk_gpu_gemm_i4(2, 47, 4, 1.0, A.ctypes.data, 4, P.ctypes.data, S.ctypes.data,
                              24, 0.0, C.ctypes.data, 64) == -1
    assert b"odd" in lib.pk_gpu_last_error()
    # transposed forms are not used by the reference call sites
    assert lib.pk_gpu_sgemm(112, 111, 2, 4, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 4, 0.0,
                            C.ctypes.data, 64) == -2
    # strides shorter than a row
    assert lib.pk_gpu_sgemm(111, 111, 2, 8, 4, 1.0, A.ctypes.data, 3, A.ctypes.data, 8, 0.0,
                            C.ctypes.data, 64) == -1
    assert lib.pk_gpu_gemm_i8(-1, 8, 4, 1.0, None, 4, None, 1.0, 8, 0.0, None, 8) == -1


def test_tile_configs_are_well_formed():
    cfgs = pk.configs()
    assert len(cfgs) >= 3
    for fam, mf, cw, wgm, wgn, kt in cfgs:
        assert fam in "RXSY" and mf in (4, 16, 32) and cw >= 1 and wgm >= 1 and wgn >= 1
        assert (128 if fam == "S" else 64) * wgm * wgn <= 1024 and kt % 16 == 0
    lib = pk.load()
    for shape in [(32, 3072, 1024), (375, 4096, 1024), (375, 1024, 4096), (3312, 4096, 1024)]:
        assert 0 <= lib.pk_gpu_pick_config(*shape) < len(cfgs)


# The encoder's GEMMs at 3200 frames: one row group (M = 3312) and each of two
# row groups (M = 1656).  These picks were measured on the encoder itself;
# a change to the dispatcher that moves one of them needs a new measurement.
ENCODER_PICKS = [
    # bits, M, N, K, config
    (4, 3312, 4096, 1024, 20), (4, 3312, 1024, 4096, 11),
    (4, 1656, 4096, 1024, 20), (4, 1656, 1024, 4096, 18),
    (8, 3312, 3072, 1024, 21), (8, 3312, 1024, 1024, 21),
    (8, 1656, 3072, 1024, 21), (8, 1656, 1024, 1024, 18),
    (32, 3312, 2048, 1024, 23), (32, 3312, 1024, 1024, 21),
    (32, 1656, 2048, 1024, 23), (32, 1656, 1024, 1024, 18),
    (8, 32, 3072, 1024, 12), (4, 375, 1024, 4096, 17), (4, 375, 4096, 1024, 14),
]


@pytest.mark.parametrize("bits,M,N,K,cfg", ENCODER_PICKS)
def test_dispatcher_picks_for_encoder_shapes(bits, M, N, K, cfg):
    assert pk.load().pk_gpu_pick_config_bits(M, N, K, bits) == cfg


def test_epilogue_validation_precedes_device_use():
    lib = pk.load()
    A = np.ones((2, 4), np.float32)
    C = np.zeros((2, 16), np.float32)
    # unknown epilogue
    assert lib.pk_gpu_sgemm_ex_dev(2, 16, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 16, 0.0,
                                   C.ctypes.data, 16, None, 7, None) == -1
    assert b"epilogue" in lib.pk_gpu_last_error()
    # the half residual reads C as the residual, so beta must be 0
    assert lib.pk_gpu_sgemm_ex_dev(2, 16, 4, 1.0, A.ctypes.data, 4, A.ctypes.data, 16, 1.0,
                                   C.ctypes.data, 16, None, pk.EPI_HALF_RESIDUAL, None) == -1
    assert b"beta" in lib.pk_gpu_last_error()


def test_null_device_operands_are_rejected():
    """A NULL device pointer must be an error, never a descriptor at address 0."""
    lib = pk.load()
    assert lib.pk_gpu_sgemm_dev(4, 16, 8, 1.0, None, 8, None, 16, 0.0, None, 16, None) == -1
    assert b"NULL" in lib.pk_gpu_last_error()
    C = np.zeros((4, 32), np.float32)
    assert lib.pk_gpu_gemm_i4_dev(4, 32, 8, 1.0, C.ctypes.data, 8, C.ctypes.data, None, 16, 0.0,
                                  C.ctypes.data, 32, None) == -1
    assert b"NULL" in lib.pk_gpu_last_error()


# K segments over workgroups that the split kernels take (fast numerics) with
# a PK_GPU_SPLIT_WORKSPACE_BYTES workspace: shapes with fewer 128 x 128 tiles
# than the 256 CUs, int8 and int4 weights from K = 2048 only, 256 x 128 tiles
# unless 256-row tiles pad more than 10% more rows, as many segments of at
# least 4 chunks as keep the workgroups within 256.
SPLIT_K_PLANS = [
    (4, 1656, 1024, 4096, 4),      # 7 x 8 tiles of 256 x 128
    (8, 1656, 1024, 1024, 1),      # int8 below K = 2048
    (8, 1656, 1024, 2048, 4),
    (32, 1656, 1024, 1024, 4),     # fp32 at any K
    (32, 1656, 2048, 1024, 2),     # 7 x 16
    (8, 1656, 3072, 4096, 1),      # 13 x 24 tiles of 128 x 128: no split
    (4, 1656, 4096, 4096, 1),
    (4, 375, 1024, 4096, 10),      # 3 x 8 tiles of 128 x 128
    (4, 375, 4096, 1024, 1),       # int4 below K = 2048
    (32, 375, 4096, 1024, 2),      # 3 x 32 tiles of 128 x 128 (256-row tiles would pad 36%)
    (32, 500, 1024, 4096, 16),     # 2 x 8 tiles of 256 x 128
    (4, 3312, 1024, 4096, 2),      # 26 x 8 = 208 tiles of 128 x 128; 13 x 8 of 256 x 128
    (32, 200, 256, 2048, 16),
    (32, 97, 96, 96, 1),           # 3 chunks: fewer than two segments of 4
]


@pytest.mark.parametrize("bits,M,N,K,segs", SPLIT_K_PLANS)
def test_split_k_plans(bits, M, N, K, segs):
    """Host-side planning only: the pointer is never dereferenced."""
    lib = pk.load()
    assert lib.pk_gpu_split_k_segments(M, N, K, bits) == 1     # no workspace yet
    fake = 1 << 20
    assert lib.pk_gpu_set_workspace(fake, pk.SPLIT_WORKSPACE_BYTES) == 0
    try:
        assert lib.pk_gpu_split_k_segments(M, N, K, bits) == segs
        assert lib.pk_gpu_set_workspace(fake, pk.SPLIT_WORKSPACE_BYTES - 1) == 0
        assert lib.pk_gpu_split_k_segments(M, N, K, bits) == 1     # too small: unused
        assert lib.pk_gpu_set_workspace(fake + 4, pk.SPLIT_WORKSPACE_BYTES) == -1
    finally:
        assert lib.pk_gpu_set_workspace(None, 0) == 0
