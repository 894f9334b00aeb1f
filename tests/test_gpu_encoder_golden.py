"""GPU: the device-resident encoder bit for bit against the oracle's whole
encoder (oracle/pk_oracle_encoder.c), on the model and input bench.py times.

The benchmark runs pk_gpu_encoder_run_dev on 3200 frames (chunks of 408,
6 x 416 and 408 rows) with the library's default two row groups, on device
memory, with bench.EncoderModel's weights (the workloads' quantization
statistics).  At those statistics the encoder amplifies a 1-ulp difference
about tenfold per block (test_oracle_block.test_reference_sensitivity), so
only identical arithmetic gives an identical output: a digest match here
means every GEMM chain, epilogue, LayerNorm, attention, softmax, GLU,
depthwise convolution and Swish of all 24 blocks agreed bit for bit.

Digests come from tests/golden/make_encoder_golden.py (the oracle on the
CPU).  A mismatch reports the first block after which the outputs differ,
from encoders holding the first b blocks (the same model's prefix).  The
900-frame workload's last chunk has 108 rows, so softmax's scalar tail runs
there; the smallest cases run the oracle live."""
import ctypes
import hashlib
import json
import os

import numpy as np
import pytest

import bench
import pyoracle as po
from pkgpu import bits_equal, describe_mismatch, gpu_available, pk

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))
GOLD = json.load(open(os.path.join(HERE, "golden", "encoder_golden.json")))


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


@pytest.fixture(scope="module")
def model():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    pk.call("pk_gpu_init", 0)
    torch.cuda.set_device(0)
    m = bench.EncoderModel(pk)
    assert sha(m.pe) == GOLD["pe_sha256"]
    return m


def resident(m, n_blocks, x, chunk, overlap, groups=None, lag=None):
    """pk_gpu_encoder_run_dev over device copies of x, as bench.py calls it."""
    import torch
    enc = ctypes.c_void_p()
    pk.call("pk_gpu_encoder_create", ctypes.byref(enc), ctypes.cast(m.blocks, ctypes.c_void_p),
            n_blocks, m.pe.ctypes.data, bench.PE_ROWS, bench.PE_CENTER)
    try:
        if groups:
            pk.call("pk_gpu_encoder_set_groups", enc, groups)
        if lag is not None:
            pk.call("pk_gpu_encoder_set_group_lag", enc, lag)
        dev = torch.device("cuda:0")
        dx = torch.from_numpy(x).to(dev)
        dout = torch.full_like(dx, float("nan"))
        s = torch.cuda.current_stream(dev).cuda_stream
        for _ in range(2):          # the first run captures the graphs, the second replays them
            pk.call("pk_gpu_encoder_run_dev", enc, dx.data_ptr(), x.shape[0], chunk, overlap,
                    dout.data_ptr(), s)
            torch.cuda.synchronize(dev)
            got = dout.cpu().numpy()
            yield got
    finally:
        pk.load().pk_gpu_encoder_destroy(enc)


def first_diverging_block(m, wl, x):
    """Smallest b whose b-block encoder output differs from the oracle's
    output after b blocks (bisection; called after the full encoder's
    output differed)."""
    want = wl["after_block_sha256"]
    lo, hi = 0, len(want)           # blocks [1, lo] agree; block hi differs
    while hi - lo > 1:
        mid = (lo + hi) // 2
        got = list(resident(m, mid, x, wl["chunk"], wl["overlap"]))[0]
        if sha(got) == want[mid - 1]:
            lo = mid
        else:
            hi = mid
    return hi


@pytest.mark.parametrize("wl_index", [0, 1], ids=["3200_frames", "900_frames"])
def test_resident_encoder_matches_oracle_digest(model, wl_index):
    wl = GOLD["workloads"][wl_index]
    x = bench.encoder_features(wl["frames"])
    assert sha(x) == wl["input_sha256"]
    outs = list(resident(model, bench.N_BLOCKS, x, wl["chunk"], wl["overlap"]))
    print(f"{wl['frames']} frames: max |out| {np.abs(outs[-1]).max():.6g} "
          f"(oracle {wl['output_max_abs']:.6g})", flush=True)
    for run, got in enumerate(outs):
        if sha(got) != wl["output_sha256"]:
            b = first_diverging_block(model, wl, x)
            pytest.fail(f"run {run}: output digest differs from the oracle's; the first block "
                        f"after which the outputs differ is block {b}")


@pytest.mark.parametrize("groups", [1, 3])
def test_resident_encoder_digest_any_grouping(model, groups):
    """The 900-frame workload with one and three row groups (every grouping
    computes the same rows the same way)."""
    wl = GOLD["workloads"][1]
    x = bench.encoder_features(wl["frames"])
    for got in resident(model, bench.N_BLOCKS, x, wl["chunk"], wl["overlap"], groups):
        assert sha(got) == wl["output_sha256"]


@pytest.mark.parametrize("groups,lag", [(2, 0), (2, 2), (2, 3), (3, 3)])
def test_resident_encoder_digest_any_group_lead(model, groups, lag):
    """The 900-frame workload with the other row groups starting after 0, 2 or
    3 modules of group 0's block 0 (the default is 1): the order in which the
    groups' kernels run changes, the digest does not."""
    wl = GOLD["workloads"][1]
    x = bench.encoder_features(wl["frames"])
    for got in resident(model, bench.N_BLOCKS, x, wl["chunk"], wl["overlap"], groups, lag):
        assert sha(got) == wl["output_sha256"]
    lib = pk.load()
    assert lib.pk_gpu_encoder_set_group_lag(None, 1) == -1


@pytest.mark.parametrize("T,chunk,n_blocks", [(300, 0, 3), (132, 64, 2)])
def test_resident_encoder_bit_exact_to_live_oracle(model, T, chunk, n_blocks):
    """The oracle run here on the same input: an unchunked 300-frame sequence
    (T % 8 = 4: softmax's scalar tail) and 64-frame chunks of 72, 76 and 12 rows."""
    x = bench.encoder_features(T)
    want = po.encoder(model.blocks, n_blocks, model.pe, bench.PE_CENTER, x, chunk, 8)
    for got in resident(model, n_blocks, x, chunk, 8):
        assert bits_equal(got, want), describe_mismatch(got, want)
