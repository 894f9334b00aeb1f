"""GPU: the resident encoder on sequences longer than 512 frames, unchunked.

The reference attends over the whole sequence when chunking is off
(PK_CHUNK=0, encoder.c:595-610; T up to the positional table's 5000 rows,
workspace encoder.c:49-85).  The attention kernel keeps score rows in LDS up
to 512 frames; beyond that each workgroup's score rows live in a device
workspace and the same operations run in the same order, and every block's
position projection is recomputed once for the longer positional slice.
Each output must equal the oracle's whole encoder (pk_oracle_encoder.c, the
reference's order of operations) bit for bit:
  600 frames, 2 blocks   T % 8 == 0, just past the LDS limit
  1100 frames, 1 block   T % 8 == 4: softmax's scalar tail
  5000 frames, 1 block   the longest sequence the table allows
and after a long run, shorter and chunked runs on the same encoder still
match (the projections and graphs were replaced, not mixed)."""
import ctypes

import numpy as np
import pytest

import bench
import pyoracle as po
from pkgpu import bits_equal, describe_mismatch, gpu_available, pk

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def model():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    pk.call("pk_gpu_init", 0)
    torch.cuda.set_device(0)
    return bench.EncoderModel(pk, n_blocks=2)


class Encoder:
    """One resident encoder over the first n_blocks of the model."""

    def __init__(self, m, n_blocks):
        import torch
        self.torch = torch
        self.enc = ctypes.c_void_p()
        pk.call("pk_gpu_encoder_create", ctypes.byref(self.enc), ctypes.cast(m.blocks, ctypes.c_void_p),
                n_blocks, m.pe.ctypes.data, bench.PE_ROWS, bench.PE_CENTER)

    def run(self, x, chunk, overlap, reps=2):
        """Outputs of `reps` runs (the first captures the graphs, later ones replay)."""
        torch = self.torch
        dev = torch.device("cuda:0")
        dx = torch.from_numpy(x).to(dev)
        dout = torch.full_like(dx, float("nan"))
        s = torch.cuda.current_stream(dev).cuda_stream
        outs = []
        for _ in range(reps):
            pk.call("pk_gpu_encoder_run_dev", self.enc, dx.data_ptr(), x.shape[0], chunk, overlap,
                    dout.data_ptr(), s)
            torch.cuda.synchronize(dev)
            outs.append(dout.cpu().numpy())
        return outs

    def close(self):
        pk.load().pk_gpu_encoder_destroy(self.enc)


def features(T, tag):
    return bench.enc_rng(0xFEA7, tag).standard_normal((T, bench.D)).astype(np.float32)


@pytest.mark.parametrize("T,n_blocks", [(600, 2), (1100, 1), (5000, 1)])
def test_unchunked_long_sequence_bit_exact(model, T, n_blocks):
    x = features(T, 7)
    want = po.encoder(model.blocks, n_blocks, model.pe, bench.PE_CENTER, x, 0, 0)
    enc = Encoder(model, n_blocks)
    try:
        for i, got in enumerate(enc.run(x, 0, 0)):
            assert bits_equal(got, want), f"run {i}: {describe_mismatch(got, want)}"
    finally:
        enc.close()


def test_long_then_short_and_chunked(model):
    """One encoder: 700 frames, then 1300 (the projections grow again), then
    700, 300 and 900 frames in chunks of 400: every run equals the oracle."""
    enc = Encoder(model, 1)
    try:
        for T, chunk, ov in [(700, 0, 0), (1300, 0, 0), (700, 0, 0), (300, 0, 0), (900, 400, 8)]:
            x = features(T, T + chunk)
            want = po.encoder(model.blocks, 1, model.pe, bench.PE_CENTER, x, chunk, ov)
            for got in enc.run(x, chunk, ov, reps=1):
                assert bits_equal(got, want), f"T {T} chunk {chunk}: {describe_mismatch(got, want)}"
    finally:
        enc.close()


@pytest.fixture(scope="module")
def trained_like():
    """The model with the int8 attention projections' scales x 0.05 (as the
    numerics tests and oracle/ref_encode_main.c's PK_SYNTH_ATTN_GAIN do): at
    the workloads' statistics one block's softmax amplifies a 1e-5 GEMM
    difference to about 2e-3."""
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    pk.call("pk_gpu_init", 0)
    torch.cuda.set_device(0)
    m = bench.EncoderModel(pk, n_blocks=2)
    for b in range(2):
        w = m.blocks[b]
        for name in ("linear_qkv_w", "linear_pos_w", "linear_out_w"):
            wt = getattr(w, name)
            wt.scale = wt.scale * 0.05
            setattr(w, name, wt)
    return m


@pytest.mark.parametrize("T,n_blocks", [(1100, 1), (640, 2)])
def test_unchunked_long_sequence_fast_numerics(trained_like, T, n_blocks):
    """PK_GPU_NUMERICS_FAST on sequences past the LDS attention limit: the
    weight GEMMs (M = T) take the split kernels, attention keeps its exact
    workspace path.  With trained-like attention weights the output stays
    within 1e-3 of the oracle's exact encoder (the split GEMMs are within
    about 1e-5 each), and a replay repeats the first run bit for bit."""
    model = trained_like
    x = features(T, 11)
    want = po.encoder(model.blocks, n_blocks, model.pe, bench.PE_CENTER, x, 0, 0)
    enc = Encoder(model, n_blocks)
    try:
        pk.call("pk_gpu_encoder_set_numerics", enc.enc, pk.NUMERICS_FAST)
        got = enc.run(x, 0, 0)
    finally:
        enc.close()
    e = float(np.abs(got[0].astype(np.float64) - want).max() / np.abs(want).max())
    print(f"T {T}, {n_blocks} block(s): fast max |out - oracle| / max |oracle| = {e:.3g}", flush=True)
    assert e <= 1e-3, e
    assert bits_equal(got[1], got[0]), "fast replay differs from its capture run"


def test_longer_than_the_table_is_refused(model):
    enc = Encoder(model, 1)
    try:
        import torch
        x = torch.zeros((5001, bench.D), device="cuda")
        rc = pk.load().pk_gpu_encoder_run_dev(enc.enc, x.data_ptr(), 5001, 0, 0, x.data_ptr(), None)
        assert pk.STATUS[rc] == "EINVAL"
        assert b"positional table" in pk.load().pk_gpu_last_error()
    finally:
        enc.close()
