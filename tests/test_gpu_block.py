"""GPU: the conformer-block operations and the device-resident encoder
through the C ABI (libpk_gpu.so), against the oracle (oracle/pk_oracle_block.c,
itself pinned to the compiled reference in test_oracle_block.py) and against
the reference's own conformer_block (oracle/ref_block_harness.c).

Bit-exact: LayerNorm (against the oracle's correctly rounded 1/sqrt form),
the attention core for every T (T % 8 == 0 also equals the compiled
reference itself), GLU, the depthwise convolution, and chunk batching (a
batch of chunks equals each chunk run alone).  Tolerance: whole blocks
against the reference, whose LayerNorm, Swish and GLU use CPU-model-specific
approximations (vrsqrtss, vrcpps, glibc's vector expf, which is off the
correctly rounded value in about half of its results): with trained-like
attention weights, max |gpu - ref| / max |ref| <= 1e-4 after four blocks;
with the workloads' int8 statistics, where the reference itself amplifies a
1-ulp difference about tenfold per block (test_oracle_block.
test_reference_sensitivity), <= 1e-3 after one block."""
import ctypes

import numpy as np
import pytest

import blockgen as bg
import pyoracle as po
from pkgpu import Dev, bits_equal, describe_mismatch, gpu_available, pk

pytestmark = pytest.mark.gpu
RNG = np.random.default_rng(0x5EEDB10D)


@pytest.fixture(scope="module")
def dev():
    if not gpu_available():
        pytest.skip("no GPU")
    return Dev()


def rows(n, d, scale=1.0, shift=0.0):
    return (RNG.standard_normal((n, d)) * scale + shift).astype(np.float32)


def sync(dev):
    dev.torch.cuda.synchronize(dev.dev)


@pytest.mark.parametrize("n", [1, 7, 100, 3312])
def test_layer_norm_bit_exact(dev, n):
    x = rows(n, 1024, 2.0, 0.5)
    g, b = 1.0 + rows(1, 1024, 0.1)[0], rows(1, 1024, 0.1)[0]
    dx, dg, db = dev.put(x), dev.put(g), dev.put(b)
    dout = dev.torch.empty_like(dx)
    pk.call("pk_gpu_layer_norm_dev", dx.data_ptr(), dg.data_ptr(), db.data_ptr(), dout.data_ptr(),
            n, 1024, dev.stream())
    want = po.layer_norm(x, g, b)
    got = dout.cpu().numpy()
    assert bits_equal(got, want), describe_mismatch(got, want)
    # in place (the block's output LayerNorm)
    pk.call("pk_gpu_layer_norm_dev", dx.data_ptr(), dg.data_ptr(), db.data_ptr(), dx.data_ptr(),
            n, 1024, dev.stream())
    assert bits_equal(dx.cpu().numpy(), want)


def attention_inputs(T):
    D = bg.H * bg.DH
    return rows(T, 3 * D, 0.5), rows(2 * T - 1, D, 0.5), rows(1, D, 0.1)[0], rows(1, D, 0.1)[0]


def gpu_attention(dev, qkv, P, pu, pv):
    T = qkv.shape[0]
    D = bg.H * bg.DH
    dq, dP, du, dv = dev.put(qkv), dev.put(P), dev.put(pu), dev.put(pv)
    dout = dev.torch.full((T, D), float("nan"), device=dev.dev)
    pk.call("pk_gpu_attention_dev", dq.data_ptr(), 3 * D, dP.data_ptr(), D, du.data_ptr(),
            dv.data_ptr(), dout.data_ptr(), D, T, bg.H, dev.stream())
    return dout.cpu().numpy()


@pytest.mark.parametrize("T", [416, 408, 64, 24, 8, 1, 21, 108, 300, 512, 33, 17, 49, 50, 63, 65])
def test_attention_bit_exact_to_oracle(dev, T):
    """T <= 64 takes the short-sequence kernel (every row staged in LDS at
    once; one or two blocks of positions: T = 49 / 50), longer T the tiled one."""
    qkv, P, pu, pv = attention_inputs(T)
    got = gpu_attention(dev, qkv, P, pu, pv)
    want = po.attention_core(qkv, P, pu, pv)
    assert bits_equal(got, want), describe_mismatch(got, want)


@pytest.mark.skipif(not po.have_ref(), reason="reference build missing")
@pytest.mark.parametrize("T", [64, 416])
def test_attention_bit_exact_to_reference(dev, T):
    """The compiled reference's own functions (cblas_sgemm_st NT/NN,
    pk_softmax_rows) with the encoder.c glue, against the GPU kernel."""
    from test_oracle_block import reference_attention
    qkv, P, pu, pv = attention_inputs(T)
    got = gpu_attention(dev, qkv, P, pu, pv)
    want = reference_attention(qkv, P, pu, pv)
    assert bits_equal(got, want), describe_mismatch(got, want)


@pytest.mark.parametrize("T", [513, 640, 1000])
def test_attention_long_sequence_bit_exact_to_oracle(dev, T):
    """Past 512 rows the score rows live in the caller's workspace: the same
    bits as the oracle (T = 1000: softmax's scalar tail)."""
    lib = pk.load()
    qkv, P, pu, pv = attention_inputs(T)
    D = bg.H * bg.DH
    n = lib.pk_gpu_attention_ws_floats(T, bg.H)
    assert n >= bg.H * T * T
    dq, dP, du, dv = dev.put(qkv), dev.put(P), dev.put(pu), dev.put(pv)
    dout = dev.torch.full((T, D), float("nan"), device=dev.dev)
    ws = dev.torch.empty(n, device=dev.dev)
    assert lib.pk_gpu_attention_ws_dev(dq.data_ptr(), 3 * D, dP.data_ptr(), D, du.data_ptr(),
                                       dv.data_ptr(), dout.data_ptr(), D, T, bg.H, ws.data_ptr(),
                                       n - 1, dev.stream()) == -1          # too small
    pk.call("pk_gpu_attention_ws_dev", dq.data_ptr(), 3 * D, dP.data_ptr(), D, du.data_ptr(),
            dv.data_ptr(), dout.data_ptr(), D, T, bg.H, ws.data_ptr(), n, dev.stream())
    got = dout.cpu().numpy()
    want = po.attention_core(qkv, P, pu, pv)
    assert bits_equal(got, want), describe_mismatch(got, want)


def test_attention_rejects_bad_sizes(dev):
    lib = pk.load()
    assert lib.pk_gpu_attention_dev(None, 3072, None, 1024, None, None, None, 1024, 513, 8, None) == -1
    assert lib.pk_gpu_attention_dev(None, 3072, None, 1024, None, None, None, 1024, 0, 8, None) == -1
    assert lib.pk_gpu_attention_ws_floats(512, 8) == 0


@pytest.mark.parametrize("n", [1, 416, 3312])
def test_glu_bit_exact(dev, n):
    x = rows(n, 2048, 3.0)
    dx = dev.put(x)
    dout = dev.torch.empty((n, 1024), device=dev.dev)
    pk.call("pk_gpu_glu_dev", dx.data_ptr(), dout.data_ptr(), n, 1024, dev.stream())
    got, want = dout.cpu().numpy(), po.glu(x)
    assert bits_equal(got, want), describe_mismatch(got, want)


@pytest.mark.parametrize("T", [416, 408, 108, 20, 13, 9, 8, 5, 1])
def test_depthwise_bit_exact(dev, T):
    C = 1024
    x = rows(T, C)                          # time-major, as the encoder keeps it
    w, b = rows(C, 9, 1.0 / 3.0), rows(1, C, 0.02)[0]
    dx, dw, db = dev.put(x), dev.put(w), dev.put(b)
    dout = dev.torch.empty((T, C), device=dev.dev)
    pk.call("pk_gpu_depthwise_dev", dx.data_ptr(), C, dw.data_ptr(), db.data_ptr(),
            dout.data_ptr(), C, T, C, 9, 0, dev.stream())
    got = dout.cpu().numpy()
    want = po.depthwise(x.T.copy(), w, b).T
    assert bits_equal(got, want), describe_mismatch(got, np.ascontiguousarray(want))
    if po.have_ref():
        assert bits_equal(got, po.ref_depthwise(x.T.copy(), w, b).T)
    # with the fused Swish: the device swish of the same values
    pk.call("pk_gpu_depthwise_dev", dx.data_ptr(), C, dw.data_ptr(), db.data_ptr(),
            dout.data_ptr(), C, T, C, 9, 1, dev.stream())
    dsw = dev.put(got)
    pk.call("pk_gpu_swish_dev", dsw.data_ptr(), dsw.data_ptr(), T * C, dev.stream())
    assert bits_equal(dout.cpu().numpy(), dsw.cpu().numpy())


class Encoder:
    def __init__(self, dev, blocks, pe):
        self.dev = dev
        self.arr = bg.block_array(blocks)
        self.blocks = blocks
        self.pe = pe
        self.h = ctypes.c_void_p()
        pk.call("pk_gpu_encoder_create", ctypes.byref(self.h), ctypes.cast(self.arr, ctypes.c_void_p),
                len(blocks), self.pe.ctypes.data, self.pe.shape[0], 4999)

    def run(self, x, chunk=0, overlap=8):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        pk.call("pk_gpu_encoder_run", self.h, x.ctypes.data, x.shape[0], chunk, overlap,
                out.ctypes.data)
        return out

    def close(self):
        pk.load().pk_gpu_encoder_destroy(self.h)


@pytest.fixture(scope="module")
def enc2(dev):
    """Two blocks with the workloads' int8 statistics."""
    blocks = [bg.Block(0xB10C0), bg.Block(0xB10C1)]
    e = Encoder(dev, blocks, bg.pe_table())
    yield e
    e.close()


@pytest.fixture(scope="module")
def enc4(dev):
    """Four blocks with trained-like attention weights."""
    blocks = [bg.Block(0xB10D0 + i, attn_scale=0.0005) for i in range(4)]
    e = Encoder(dev, blocks, bg.pe_table())
    yield e
    e.close()


def compare_to_reference(enc, n_blocks, T, tol):
    x = rows(T, 1024)
    got = enc.run(x)
    want = po.ref_blocks(enc.arr, n_blocks, bg.pe_slice(enc.pe, T), x)
    err = np.abs(got - want).max() / np.abs(want).max()
    print(f"{n_blocks} blocks, T={T}: max |gpu - ref| / max |ref| = {err:.3g}, "
          f"identical elements {np.mean(got == want):.4f}")
    assert np.isfinite(got).all()
    assert err <= tol


@pytest.mark.skipif(not po.have_ref_block(), reason="reference block harness missing")
@pytest.mark.parametrize("T", [416, 108, 33])
def test_encoder_blocks_match_reference(dev, enc4, T):
    """Four blocks, one sequence: every GEMM, attention and the depthwise
    convolution are bit-exact, so what remains is LayerNorm's 1/sqrt,
    Swish's and GLU's reciprocal and GLU's exp."""
    compare_to_reference(enc4, 4, T, 1e-4)


@pytest.mark.skipif(not po.have_ref_block(), reason="reference block harness missing")
def test_encoder_block_workload_stats_within_tolerance(dev):
    blocks = [bg.Block(0xB10C0)]
    e = Encoder(dev, blocks, bg.pe_table())
    try:
        compare_to_reference(e, 1, 416, 1e-3)
    finally:
        e.close()


@pytest.mark.parametrize("mode", ["int8", "fp32"])
@pytest.mark.parametrize("T,chunk", [(300, 0), (132, 64), (100, 40)])
def test_encoder_weight_directories_bit_exact_to_oracle(dev, mode, T, chunk):
    """The resident encoder with the int8 weight directory's formats (every
    linear int8, the FF linears included) and the fp32 one's (every linear
    fp32: QKV, position and output projections on the fp32 chains), two
    blocks, bit for bit against the oracle's encoder on the same blocks: an
    unchunked 300-frame sequence (softmax's scalar tail), 64-frame chunks
    of 72, 76 and 12 rows, and 40-frame chunks of 48, 56 and 28 rows (the
    short-sequence attention over a batch of chunks)."""
    blocks = [bg.Block(0xD1500 + i, attn_scale=0.0005, mode=mode) for i in range(2)]
    assert {blocks[0].w.ff1_linear1_w.bits, blocks[0].w.linear_out_w.bits} == \
        {8 if mode == "int8" else 32}
    e = Encoder(dev, blocks, bg.pe_table())
    try:
        x = rows(T, 1024)
        want = po.encoder(e.arr, 2, e.pe, 4999, x, chunk, 8)
        got = e.run(x, chunk=chunk)
        assert bits_equal(got, want), describe_mismatch(got, want)
    finally:
        e.close()


def test_encoder_chunk_batch_equals_chunks_alone(dev, enc2):
    """Chunked mode runs all chunks as one batch (GEMMs over every chunk's
    rows, attention and depthwise per chunk length); each chunk's rows must
    come out exactly as when that chunk's input runs alone."""
    T, C, ov = 900, 400, 8
    x = rows(T, 1024)
    batched = enc2.run(x, chunk=C, overlap=ov)
    for ci in range(-(-T // C)):
        o0, o1 = ci * C, min(ci * C + C, T)
        i0, i1 = max(o0 - ov, 0), min(o1 + ov, T)
        alone = enc2.run(x[i0:i1])
        assert bits_equal(batched[o0:o1], alone[o0 - i0:o0 - i0 + (o1 - o0)]), f"chunk {ci}"


def test_encoder_dev_entry_and_in_place(dev, enc2):
    T = 408
    x = rows(T, 1024)
    want = enc2.run(x)
    dx = dev.put(x)
    dout = dev.torch.empty_like(dx)
    pk.call("pk_gpu_encoder_run_dev", enc2.h, dx.data_ptr(), T, 0, 8, dout.data_ptr(), dev.stream())
    sync(dev)
    assert bits_equal(dout.cpu().numpy(), want)
    xi = x.copy()
    pk.call("pk_gpu_encoder_run", enc2.h, xi.ctypes.data, T, 0, 8, xi.ctypes.data)
    assert bits_equal(xi, want)


def test_encoder_runs_on_two_streams_are_ordered(dev, enc2):
    """Runs share the encoder's workspace and chunk table.  A run enqueued on
    another stream than the previous run's waits for that run on the device,
    so two runs issued back to back on two streams, with no host wait between
    them, each give what they give alone.  The second input is longer: its
    chunk table is rewritten while the first run may still be queued."""
    torch = dev.torch
    xa, xb = rows(900, 1024), rows(1300, 1024)
    want_a, want_b = enc2.run(xa, chunk=400), enc2.run(xb, chunk=400)
    for _ in range(2):
        da, db = dev.put(xa), dev.put(xb)
        oa, ob = torch.empty_like(da), torch.empty_like(db)
        sync(dev)
        sa, sb = torch.cuda.Stream(), torch.cuda.Stream()
        pk.call("pk_gpu_encoder_run_dev", enc2.h, da.data_ptr(), 900, 400, 8, oa.data_ptr(),
                sa.cuda_stream)
        pk.call("pk_gpu_encoder_run_dev", enc2.h, db.data_ptr(), 1300, 400, 8, ob.data_ptr(),
                sb.cuda_stream)
        torch.cuda.synchronize()
        assert bits_equal(oa.cpu().numpy(), want_a)
        assert bits_equal(ob.cpu().numpy(), want_b)


def test_encoder_graph_replays_match_eager(dev, enc2):
    """Without profiling the blocks run as a HIP graph captured on the first
    run of a chunking and replayed after; with profiling they launch one by
    one.  Replays on alternating inputs, with eager runs in between, must each
    equal the eager result bit for bit."""
    T = 900
    xs = [rows(T, 1024), rows(T, 1024)]
    pk.call("pk_gpu_encoder_profile", enc2.h, 1)
    want = [enc2.run(x, chunk=400) for x in xs]
    pk.call("pk_gpu_encoder_profile", enc2.h, 0)
    for rep in range(4):
        got = enc2.run(xs[rep % 2], chunk=400)
        assert bits_equal(got, want[rep % 2]), f"replay {rep}"
        pk.call("pk_gpu_encoder_profile", enc2.h, 1)
        assert bits_equal(enc2.run(xs[(rep + 1) % 2], chunk=400), want[(rep + 1) % 2])
        pk.call("pk_gpu_encoder_profile", enc2.h, 0)
    ms = ctypes.c_double()
    pk.call("pk_gpu_encoder_profile_read", enc2.h, 0, ctypes.byref(ms), None, None, None)


def test_encoder_forced_config_is_part_of_the_graph(dev, enc2):
    """A pk_gpu_force_config in force when a run's graphs are captured is
    frozen into them, so graphs are kept per forced configuration: forcing,
    then resetting, takes effect on the next run (each run captures or finds
    its own graph), and every configuration gives the same bits."""
    T = 900
    x = rows(T, 1024)
    want = enc2.run(x, chunk=400)
    for cfg in (13, 20, -1, 13):
        pk.call("pk_gpu_force_config", cfg)
        try:
            for _ in range(2):                  # capture (or reuse), then replay
                assert bits_equal(enc2.run(x, chunk=400), want), f"forced config {cfg}"
        finally:
            pk.call("pk_gpu_force_config", -1)


@pytest.mark.parametrize("n_groups", [1, 2, 3, 4])
def test_encoder_row_groups_are_bit_identical(dev, enc2, n_groups):
    """Replays split the chunks into row groups replayed concurrently (group 0
    on the caller's stream, the others on side streams); eager profiled runs
    issue the groups one after another.  The output must not depend on the
    grouping, through both
    the host and the device-pointer entry points."""
    for T in (3200, 900):              # 8 chunks; 3 chunks (4 groups clamp to 3)
        x = rows(T, 1024)
        pk.call("pk_gpu_encoder_profile", enc2.h, 1)
        want = enc2.run(x, chunk=400)
        pk.call("pk_gpu_encoder_profile", enc2.h, 0)
        pk.call("pk_gpu_encoder_set_groups", enc2.h, n_groups)
        try:
            for rep in range(3):
                assert bits_equal(enc2.run(x, chunk=400), want), f"T {T} replay {rep}"
            dx = dev.put(x)
            dout = dev.torch.empty_like(dx)
            for rep in range(2):
                dout.fill_(float("nan"))
                pk.call("pk_gpu_encoder_run_dev", enc2.h, dx.data_ptr(), T, 400, 8, dout.data_ptr(),
                        dev.stream())
                sync(dev)
                assert bits_equal(dout.cpu().numpy(), want), f"T {T} dev replay {rep}"
        finally:
            pk.call("pk_gpu_encoder_set_groups", enc2.h, 2)


def test_encoder_long_input(dev, enc2):
    """12000 frames: 30 chunks, two row groups of 15, a workspace four times the
    bench's; the replay equals the eager one-group run bit for bit."""
    T = 12000
    x = rows(T, 1024)
    pk.call("pk_gpu_encoder_profile", enc2.h, 1)
    want = enc2.run(x, chunk=400)
    pk.call("pk_gpu_encoder_profile", enc2.h, 0)
    for rep in range(2):
        assert bits_equal(enc2.run(x, chunk=400), want), f"replay {rep}"
    assert np.isfinite(want).all()


def test_encoder_many_chunkings(dev, enc2):
    """Each chunking of the input keeps captured graphs (one per row group);
    past the encoder's limit they are dropped and recaptured.  Forty input
    lengths, each compared with its eager run, cross that limit twice over."""
    x = rows(840, 1024)
    for T in range(801, 841):
        pk.call("pk_gpu_encoder_profile", enc2.h, 1)
        want = enc2.run(x[:T], chunk=400)
        pk.call("pk_gpu_encoder_profile", enc2.h, 0)
        assert bits_equal(enc2.run(x[:T], chunk=400), want), f"T {T}"


def test_encoder_group_count_is_checked(dev, enc2):
    lib = pk.load()
    assert lib.pk_gpu_encoder_set_groups(enc2.h, 0) == -1
    assert lib.pk_gpu_encoder_set_groups(enc2.h, 5) == -1
    assert lib.pk_gpu_encoder_set_groups(None, 2) == -1


def test_encoder_rejects_sequence_beyond_the_table(dev, enc2):
    """An unchunked sequence longer than the positional table covers (5000
    frames for a 9999-row table) is refused before any work is queued;
    test_gpu_long_sequence.py runs the lengths up to it."""
    x = np.zeros((5001, 1024), np.float32)
    out = np.empty_like(x)
    rc = pk.load().pk_gpu_encoder_run(enc2.h, x.ctypes.data, 5001, 0, 8, out.ctypes.data)
    assert rc == -1                               # PK_GPU_EINVAL


@pytest.mark.skipif(not po.have_ref_block(), reason="reference block harness missing")
@pytest.mark.parametrize("out_bits", [8, 32])
def test_pre_encode_bit_exact(dev, enc2, out_bits):
    """pre_encode_and_scale: 3x3 convolutions, depthwise and pointwise
    convolutions (chains started from the bias), ReLUs, flatten, the output
    linear and the sqrt(d_model) scale, bit-identical to the reference for
    odd and even frame counts."""
    pre = bg.PreEncode(0xB10CE + out_bits, out_bits)
    pk.call("pk_gpu_encoder_set_pre_encode", enc2.h, ctypes.byref(pre.w))
    lib = pk.load()
    for n in (1, 8, 33, 100, 801, 2400):
        mel = rows(128, n, 2.0)
        want = po.ref_pre_encode(pre.w, mel)
        tp = lib.pk_gpu_encoder_frames(n)
        assert tp == want.shape[0]
        dmel = dev.put(mel)
        dx = dev.torch.full((tp, 1024), float("nan"), device=dev.dev)
        pk.call("pk_gpu_encoder_pre_encode_dev", enc2.h, dmel.data_ptr(), n, dx.data_ptr(),
                dev.stream())
        got = dx.cpu().numpy()
        assert bits_equal(got, want), f"n_frames={n}: " + describe_mismatch(got, want)


@pytest.mark.skipif(not po.have_ref_block(), reason="reference block harness missing")
def test_run_mel_equals_pre_encode_then_blocks(dev, enc2):
    """pk_gpu_encoder_run_mel = pre-encode on the device, then the blocks
    (chunked), against the same two steps through their own entry points."""
    pre = bg.PreEncode(0xB10CF)
    pk.call("pk_gpu_encoder_set_pre_encode", enc2.h, ctypes.byref(pre.w))
    n = 4100                                        # T' = 513 -> two chunks
    mel = rows(128, n, 2.0)
    tp = pk.load().pk_gpu_encoder_frames(n)
    out = np.empty((tp, 1024), np.float32)
    pk.call("pk_gpu_encoder_run_mel", enc2.h, mel.ctypes.data, n, 400, 8, out.ctypes.data)
    x = po.ref_pre_encode(pre.w, mel)
    assert bits_equal(out, enc2.run(x, chunk=400))
