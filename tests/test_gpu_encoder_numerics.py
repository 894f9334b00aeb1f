"""GPU: the resident encoder's numerics setting (pk_gpu_encoder_set_numerics).

Under PK_GPU_NUMERICS_EXACT (the default) every operation is the
reference's, and the output equals the oracle's whole encoder
(pk_oracle_encoder.c) bit for bit.  Under PK_GPU_NUMERICS_DEFAULT the weight
GEMMs of a row group of at most 64 rows (a 2.56 s clip's 33 frames) take the
small-M kernels, and under PK_GPU_NUMERICS_FAST every weight GEMM takes the
small-M or the split kernels, each within 1e-3 of the reference GEMM (about
1e-5); over
24 blocks the deviations compound, so the model here has trained-like
attention weights (the int8 attention projections' scales x 0.05, as
oracle/ref_encode_main.c's PK_SYNTH_ATTN_GAIN does for the end-to-end token
checks): with the workloads' statistics a 1-ulp difference grows about
tenfold per block (test_oracle_block.test_reference_sensitivity).  Inputs
longer than 64 rows per group are unaffected by the setting."""
import ctypes

import numpy as np
import pytest

import bench
import pyoracle as po
from pkgpu import bits_equal, describe_mismatch, gpu_available, pk

pytestmark = pytest.mark.gpu
TOL = 1e-3


@pytest.fixture(scope="module")
def model():
    if not gpu_available():
        pytest.skip("no GPU")
    import torch
    pk.call("pk_gpu_init", 0)
    torch.cuda.set_device(0)
    m = bench.EncoderModel(pk)
    for b in range(bench.N_BLOCKS):
        w = m.blocks[b]
        for name in ("linear_qkv_w", "linear_pos_w", "linear_out_w"):
            wt = getattr(w, name)
            wt.scale = wt.scale * 0.05
            setattr(w, name, wt)
    return m


def run(m, x, chunk, mode, overlap=8):
    return run_blocks(m.blocks, bench.N_BLOCKS, m.pe, x, chunk, mode, overlap)


def run_blocks(blocks, n_blocks, pe, x, chunk, mode, overlap=8):
    """Two runs (graph capture, then replay) of an encoder over n_blocks of
    the ctypes block array `blocks` under numerics `mode`."""
    import torch
    enc = ctypes.c_void_p()
    pk.call("pk_gpu_encoder_create", ctypes.byref(enc), ctypes.cast(blocks, ctypes.c_void_p),
            n_blocks, pe.ctypes.data, pe.shape[0], bench.PE_CENTER)
    try:
        pk.call("pk_gpu_encoder_set_numerics", enc, mode)
        assert pk.load().pk_gpu_encoder_get_numerics(enc) == mode
        dev = torch.device("cuda:0")
        dx = torch.from_numpy(x).to(dev)
        dout = torch.full_like(dx, float("nan"))
        outs = []
        for _ in range(2):               # capture, then replay
            pk.call("pk_gpu_encoder_run_dev", enc, dx.data_ptr(), x.shape[0], chunk, overlap,
                    dout.data_ptr(), torch.cuda.current_stream(dev).cuda_stream)
            torch.cuda.synchronize(dev)
            outs.append(dout.cpu().numpy())
        return outs
    finally:
        pk.load().pk_gpu_encoder_destroy(enc)


def rel_dev(got, want):
    return float(np.abs(got.astype(np.float64) - want).max() / np.abs(want).max())


@pytest.mark.parametrize("T", [33, 64, 1])
def test_short_clip_small_m_within_tolerance(model, T):
    x = bench.enc_rng(0xFEA7, 33).standard_normal((T, bench.D)).astype(np.float32)
    want = po.encoder(model.blocks, bench.N_BLOCKS, model.pe, bench.PE_CENTER, x, 0, 0)
    small = run(model, x, 0, pk.NUMERICS_DEFAULT)
    exact = run(model, x, 0, pk.NUMERICS_EXACT)
    e = rel_dev(small[0], want)
    print(f"T {T}: small-M max |out - oracle| / max |oracle| = {e:.3g}", flush=True)
    assert e <= TOL, e
    assert bits_equal(small[1], small[0]), "small-M replay differs from its capture run"
    for got in exact:
        assert bits_equal(got, want), describe_mismatch(got, want)


@pytest.mark.parametrize("T,chunk", [(200, 0), (300, 140)])
def test_fast_mode_within_tolerance(model, T, chunk):
    """PK_GPU_NUMERICS_FAST: every weight GEMM of every length on the
    tolerance kernels (the split kernels above 64 rows per group; 300 frames
    in chunks of 140 run as two row groups).  Over 24 blocks the output stays
    within 1e-3 of the oracle's exact encoder, and replays repeat the first
    run bit for bit."""
    x = bench.enc_rng(0xFEA7, T + 1).standard_normal((T, bench.D)).astype(np.float32)
    ov = 8 if chunk else 0
    want = po.encoder(model.blocks, bench.N_BLOCKS, model.pe, bench.PE_CENTER, x, chunk, ov)
    got = run(model, x, chunk, pk.NUMERICS_FAST, overlap=ov)
    e = rel_dev(got[0], want)
    print(f"T {T} chunk {chunk}: fast max |out - oracle| / max |oracle| = {e:.3g}", flush=True)
    assert e <= TOL, e
    assert bits_equal(got[1], got[0]), "fast replay differs from its capture run"


@pytest.mark.parametrize("fmt", ["int8", "fp32"])
@pytest.mark.parametrize("T,chunk,mode", [(33, 0, "default"), (300, 140, "fast")])
def test_weight_directories_tolerance_modes(model, fmt, T, chunk, mode):
    """Four blocks in the int8 weight directory's formats (every linear int8,
    the FF linears included) or the fp32 one's (every linear fp32), trained-
    like attention weights: a 33-frame clip under the default setting (small-M
    kernels) and 300 frames in chunks of 140 under the fast one (split
    kernels, two row groups), within 1e-3 of the oracle's exact encoder;
    replays repeat the first run bit for bit."""
    import blockgen as bg
    blocks = [bg.Block(0xD1600 + i, attn_scale=0.0005, mode=fmt) for i in range(4)]
    arr, pe = bg.block_array(blocks), bg.pe_table()
    numerics = pk.NUMERICS_DEFAULT if mode == "default" else pk.NUMERICS_FAST
    x = bench.enc_rng(0xFEA8, T).standard_normal((T, bench.D)).astype(np.float32)
    ov = 8 if chunk else 0
    want = po.encoder(arr, 4, pe, bench.PE_CENTER, x, chunk, ov)
    got = run_blocks(arr, 4, pe, x, chunk, numerics, ov)
    e = rel_dev(got[0], want)
    print(f"{fmt} T {T} chunk {chunk} {mode}: max |out - oracle| / max |oracle| = {e:.3g}", flush=True)
    assert e <= TOL, e
    assert bits_equal(got[1], got[0]), "replay differs from its capture run"


@pytest.mark.parametrize("T", [33, 64, 20])
def test_fused_layer_norms_are_bit_identical(model, T, monkeypatch):
    """Row groups of at most 64 rows on the panel kernels take each LayerNorm
    that feeds a GEMM inside that GEMM (rows normalised as they are staged)
    and the block's output LayerNorm inside the second feed-forward's split-K
    reduce.  Those compute the LayerNorm kernel's arithmetic operation for
    operation, so the encoder with them (the default) equals the encoder with
    separate LayerNorm launches (PK_GPU_FUSE_LN=0 at creation) bit for bit."""
    x = bench.enc_rng(0xFEAA, T).standard_normal((T, bench.D)).astype(np.float32)
    fused = run(model, x, 0, pk.NUMERICS_DEFAULT)
    monkeypatch.setenv("PK_GPU_FUSE_LN", "0")
    apart = run(model, x, 0, pk.NUMERICS_DEFAULT)
    assert bits_equal(fused[0], apart[0]), describe_mismatch(fused[0], apart[0])
    assert bits_equal(fused[1], fused[0]), "replay differs from its capture run"


def test_exact_after_fast_regrow(model):
    """The blocks' position projections are constants that runs in every
    mode read.  A fast run that first sees a sequence longer than the
    projections cover (600 frames, one sequence) recomputes them, on the
    exact chains, so a later exact run (300 frames) is still bit-identical to
    the oracle's encoder."""
    import torch
    x6 = bench.enc_rng(0xFEA9, 600).standard_normal((600, bench.D)).astype(np.float32)
    x3 = bench.enc_rng(0xFEA9, 300).standard_normal((300, bench.D)).astype(np.float32)
    want = po.encoder(model.blocks, bench.N_BLOCKS, model.pe, bench.PE_CENTER, x3, 0, 0)
    enc = ctypes.c_void_p()
    pk.call("pk_gpu_encoder_create", ctypes.byref(enc), ctypes.cast(model.blocks, ctypes.c_void_p),
            bench.N_BLOCKS, model.pe.ctypes.data, model.pe.shape[0], bench.PE_CENTER)
    try:
        dev = torch.device("cuda:0")
        s = torch.cuda.current_stream(dev).cuda_stream
        d6, d3 = torch.from_numpy(x6).to(dev), torch.from_numpy(x3).to(dev)
        o6, o3 = torch.empty_like(d6), torch.full_like(d3, float("nan"))
        pk.call("pk_gpu_encoder_set_numerics", enc, pk.NUMERICS_FAST)
        pk.call("pk_gpu_encoder_run_dev", enc, d6.data_ptr(), 600, 0, 0, o6.data_ptr(), s)
        torch.cuda.synchronize(dev)
        pk.call("pk_gpu_encoder_set_numerics", enc, pk.NUMERICS_EXACT)
        pk.call("pk_gpu_encoder_run_dev", enc, d3.data_ptr(), 300, 0, 0, o3.data_ptr(), s)
        torch.cuda.synchronize(dev)
        got = o3.cpu().numpy()
    finally:
        pk.load().pk_gpu_encoder_destroy(enc)
    assert bits_equal(got, want), describe_mismatch(got, want)


def test_long_input_unaffected(model):
    """200 frames unchunked (one group of 200 rows): the setting changes nothing."""
    x = bench.enc_rng(0xFEA7, 200).standard_normal((200, bench.D)).astype(np.float32)
    want = po.encoder(model.blocks, bench.N_BLOCKS, model.pe, bench.PE_CENTER, x, 0, 0)
    for got in run(model, x, 0, pk.NUMERICS_DEFAULT):
        assert bits_equal(got, want), describe_mismatch(got, want)


def test_numerics_argument_checks(model):
    lib = pk.load()
    assert lib.pk_gpu_encoder_set_numerics(None, 0) == -1
    assert lib.pk_gpu_encoder_get_numerics(None) == -1
    enc = ctypes.c_void_p()
    pk.call("pk_gpu_encoder_create", ctypes.byref(enc), ctypes.cast(model.blocks, ctypes.c_void_p),
            1, model.pe.ctypes.data, bench.PE_ROWS, bench.PE_CENTER)
    try:
        assert lib.pk_gpu_encoder_get_numerics(enc) == pk.NUMERICS_EXACT
        assert lib.pk_gpu_encoder_set_numerics(enc, 5) == -1
        assert lib.pk_gpu_encoder_set_numerics(enc, pk.NUMERICS_FAST) == 0
    finally:
        lib.pk_gpu_encoder_destroy(enc)


def test_fast_mode_row_group_changes(model):
    """PK_GPU_NUMERICS_FAST with split-K: the encoder holds a partial-tile
    workspace per row group.  Going from two groups to three grows it (the
    captured graphs, which hold its addresses, are dropped and recaptured)
    and going back reuses it: every run stays within 1e-3 of the oracle, and
    the two-group runs before and after are bit-identical."""
    import torch
    T, chunk, ov = 300, 64, 8                     # 5 chunks of up to 80 rows
    x = bench.enc_rng(0xFEA7, 301).standard_normal((T, bench.D)).astype(np.float32)
    want = po.encoder(model.blocks, bench.N_BLOCKS, model.pe, bench.PE_CENTER, x, chunk, ov)
    enc = ctypes.c_void_p()
    pk.call("pk_gpu_encoder_create", ctypes.byref(enc), ctypes.cast(model.blocks, ctypes.c_void_p),
            bench.N_BLOCKS, model.pe.ctypes.data, bench.PE_ROWS, bench.PE_CENTER)
    try:
        lib = pk.load()
        pk.call("pk_gpu_encoder_set_numerics", enc, pk.NUMERICS_FAST)
        dev = torch.device("cuda:0")
        dx = torch.from_numpy(x).to(dev)
        outs = {}
        for step, groups in enumerate((2, 3, 2)):
            pk.call("pk_gpu_encoder_set_groups", enc, groups)
            dout = torch.full_like(dx, float("nan"))
            for _ in range(2):                    # capture, then replay
                pk.call("pk_gpu_encoder_run_dev", enc, dx.data_ptr(), T, chunk, ov, dout.data_ptr(),
                        torch.cuda.current_stream(dev).cuda_stream)
            torch.cuda.synchronize(dev)
            got = dout.cpu().numpy()
            e = rel_dev(got, want)
            print(f"groups {groups}: fast max |out - oracle| / max |oracle| = {e:.3g}, "
                  f"device bytes {lib.pk_gpu_encoder_bytes(enc)}", flush=True)
            assert e <= TOL, (groups, e)
            outs[step] = got
        assert bits_equal(outs[2], outs[0]), describe_mismatch(outs[2], outs[0])
    finally:
        pk.load().pk_gpu_encoder_destroy(enc)


def test_fast_mode_presplit_layer_norm_is_bit_identical(model, monkeypatch):
    """Under PK_GPU_NUMERICS_FAST the LayerNorms that feed a GEMM write their
    output already split into the bf16 halves the split kernels multiply.
    That moves the split, not the arithmetic: an encoder created with
    PK_GPU_PRESPLIT=0 (the GEMMs split the fp32 LayerNorm output themselves)
    gives the same bits, over two row groups and 24 blocks."""
    T, chunk, ov = 300, 140, 8
    x = bench.enc_rng(0xFEA7, 302).standard_normal((T, bench.D)).astype(np.float32)
    monkeypatch.delenv("PK_GPU_PRESPLIT", raising=False)
    pre = run(model, x, chunk, pk.NUMERICS_FAST, overlap=ov)
    monkeypatch.setenv("PK_GPU_PRESPLIT", "0")
    plain = run(model, x, chunk, pk.NUMERICS_FAST, overlap=ov)
    for a, b in zip(pre, plain):
        assert bits_equal(a, b), describe_mismatch(a, b)


def test_fast_mode_presplit_weights_are_bit_identical(model, monkeypatch):
    """Under PK_GPU_NUMERICS_FAST the row groups above 64 rows read the int4
    and fp32 block weights' pre-split copies (made once, with the split
    kernels' own decode and split).  An encoder created with
    PK_GPU_PRESPLIT_W=0 (the kernels decode and split every weight per row
    tile) gives the same bits, over two row groups and 24 blocks, split-K
    GEMMs included."""
    T, chunk, ov = 300, 140, 8
    x = bench.enc_rng(0xFEA7, 303).standard_normal((T, bench.D)).astype(np.float32)
    monkeypatch.delenv("PK_GPU_PRESPLIT_W", raising=False)
    pre = run(model, x, chunk, pk.NUMERICS_FAST, overlap=ov)
    monkeypatch.setenv("PK_GPU_PRESPLIT_W", "0")
    plain = run(model, x, chunk, pk.NUMERICS_FAST, overlap=ov)
    for a, b in zip(pre, plain):
        assert bits_equal(a, b), describe_mismatch(a, b)


def layer_norm_launches(m, x, chunk, mode):
    """LayerNorm launches of one profiled run (eager, the replay's kernels)."""
    import torch
    enc = ctypes.c_void_p()
    pk.call("pk_gpu_encoder_create", ctypes.byref(enc), ctypes.cast(m.blocks, ctypes.c_void_p),
            bench.N_BLOCKS, m.pe.ctypes.data, m.pe.shape[0], bench.PE_CENTER)
    try:
        pk.call("pk_gpu_encoder_set_numerics", enc, mode)
        dev = torch.device("cuda:0")
        dx = torch.from_numpy(x).to(dev)
        dout = torch.empty_like(dx)
        pk.call("pk_gpu_encoder_profile", enc, 1)
        pk.call("pk_gpu_encoder_run_dev", enc, dx.data_ptr(), x.shape[0], chunk, 8, dout.data_ptr(),
                torch.cuda.current_stream(dev).cuda_stream)
        n = ctypes.c_longlong()
        pk.call("pk_gpu_encoder_profile_read", enc, pk.STAGE_LAYER_NORM, None, ctypes.byref(n), None, None)
        pk.call("pk_gpu_encoder_profile", enc, 0)
        return n.value
    finally:
        pk.load().pk_gpu_encoder_destroy(enc)


@pytest.mark.parametrize("T, chunk", [(300, 140), (1000, 400)])
def test_fast_mode_reduce_layer_norms_are_bit_identical(model, T, chunk, monkeypatch):
    """Under PK_GPU_NUMERICS_FAST, in row groups above 64 rows, the split-K
    reduces that finish x form the LayerNorms of the rows they write:
    feed-forward 1's down projection self-attention's input, pointwise 2
    feed-forward 2's input, and feed-forward 2's down projection the block's
    output LayerNorm and the next block's input (pre-split).  They use the
    LayerNorm kernels' arithmetic, so the encoder with them equals the
    encoder with separate LayerNorm launches (PK_GPU_FUSE_LN=0 at creation)
    bit for bit.  Two row groups (300 frames: about 150 rows each, 1000
    frames: about 830 and 410, the 128- and 256-row tiles' reduces); the
    profiled run shows the launches gone: per group the convolution
    module's LayerNorm and the first block's input one are left."""
    x = bench.enc_rng(0xFEAB, T).standard_normal((T, bench.D)).astype(np.float32)
    monkeypatch.delenv("PK_GPU_FUSE_LN", raising=False)
    fused = run(model, x, chunk, pk.NUMERICS_FAST)
    n_fused = layer_norm_launches(model, x, chunk, pk.NUMERICS_FAST)
    monkeypatch.setenv("PK_GPU_FUSE_LN", "0")
    apart = run(model, x, chunk, pk.NUMERICS_FAST)
    n_apart = layer_norm_launches(model, x, chunk, pk.NUMERICS_FAST)
    print(f"T {T} chunk {chunk}: LayerNorm launches {n_fused} fused, {n_apart} apart", flush=True)
    assert n_apart == 2 * 5 * bench.N_BLOCKS, n_apart
    assert n_fused == 2 * (bench.N_BLOCKS + 1), n_fused
    for a, b in zip(fused, apart):
        assert bits_equal(a, b), describe_mismatch(a, b)


@pytest.mark.parametrize("T, chunk", [(300, 140), (1000, 400), (200, 0)])
def test_fast_mode_split_attention(model, T, chunk, monkeypatch):
    """Under PK_GPU_NUMERICS_FAST, row groups above 64 rows with chunks of
    65-512 rows take the attention on split bf16 operands
    (rel_pos_attention_fast: three bf16 products per pair, fast softmax).
    Over 24 blocks on trained-like weights the encoder with it stays within
    the 1e-3 contract of the same encoder with the exact attention
    (PK_GPU_FAST_ATTN=0 at creation); the two differ, so the split kernel
    ran; and replays repeat the first run bit for bit."""
    x = bench.enc_rng(0xFEAC, T).standard_normal((T, bench.D)).astype(np.float32)
    monkeypatch.delenv("PK_GPU_FAST_ATTN", raising=False)
    fast = run(model, x, chunk, pk.NUMERICS_FAST)
    monkeypatch.setenv("PK_GPU_FAST_ATTN", "0")
    exact_attn = run(model, x, chunk, pk.NUMERICS_FAST)
    e = rel_dev(fast[0], exact_attn[0].astype(np.float64))
    print(f"T {T} chunk {chunk}: split attention against exact attention, max rel {e:.3g}", flush=True)
    assert np.isfinite(fast[0]).all()
    assert 0.0 < e <= TOL, e
    assert bits_equal(fast[1], fast[0]), "replay differs from its capture run"
