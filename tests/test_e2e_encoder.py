"""End to end: the reference's own encoder and greedy decoder (encoder.c,
decoder.c, weights.c, compiled from its sources by oracle/Makefile) with
the weight GEMMs taken from the GPU drop-in, against the same host code
with blas.c's portable weight GEMMs.  Both load the same synthetic mixed
int4/int8/fp32 model through pk_load_weights (fused-QKV requantisation
included); every other object is shared, so equal encoder-output and
token hashes mean the GPU GEMMs changed nothing.  The reference's other two
weight directories (c_weights_int8: every matmul weight int8; c_weights_fp32:
every weight fp32) are imitated the same way (PK_SYNTH_MODE) and checked by
the *_weight_directories tests.

The x86 AVX2 build of the reference decodes int4 weights wrongly
(blas.c:815-833, see test_oracle.test_x86_int4_unpack_defect); its output
is compared too, to show the effect on a whole encoder.

The reference decoder reads uninitialised memory: pk_lstm_step mallocs its
gate buffer and fills it with cblas_sgemv(NoTrans, beta = 0)
(tensor_ops.c:601-605), whose NoTrans branch computes beta * Y
(blas.c:67).  When the recycled heap block holds NaN or Inf bits the LSTM
state becomes NaN for good, the -ffast-math ReLU of the joint maps NaN to
0, and the decoder emits only blanks; which run that happens in depends
on heap history.  Every driver here therefore runs with glibc's
MALLOC_PERTURB_ set, which fills fresh allocations with a finite pattern,
so 0 * Y is 0 as beta = 0 intends and the token ids are reproducible."""
import json
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REF = os.path.join(os.path.dirname(HERE), "oracle", "_ref")
THREADS = str(min(os.cpu_count() or 1, 16))


def run(binary, frames, tmp_path, dump=None, attn_gain=None, from_mel=False, extra_env=None,
        mode=None, model_dir=None):
    """mode: the weight directory the synthetic model imitates (mixed, int8,
    fp32; PK_SYNTH_MODE); model_dir: where the model is kept and reused by
    later runs of the same mode and gain (PK_MODEL_DIR)."""
    path = os.path.join(REF, binary)
    if not os.path.exists(path):
        pytest.skip(f"{binary} not built (oracle/Makefile ref)")
    env = dict(os.environ, PK_THREADS=THREADS, MALLOC_PERTURB_="192")  # 0x3f3f3f3f fill
    env.pop("PK_SYNTH_MODE", None)
    env.pop("PK_MODEL_DIR", None)
    if mode:
        env["PK_SYNTH_MODE"] = mode
    if model_dir:
        env["PK_MODEL_DIR"] = str(model_dir)
    if dump:
        env["PK_DUMP_ENC"] = str(dump)
    if attn_gain is not None:
        env["PK_SYNTH_ATTN_GAIN"] = str(attn_gain)
    if from_mel:
        env["PK_FROM_MEL"] = "1"
    if extra_env:
        env.update(extra_env)
    out = subprocess.run([path, str(frames), str(tmp_path)], capture_output=True, text=True,
                         env=env, timeout=400)
    assert out.returncode == 0, out.stderr[-2000:]
    line = [l for l in out.stdout.splitlines() if l.startswith("{")][-1]
    print(binary, line, flush=True)
    return json.loads(line)


def margin(ref):
    """The reference decode's smallest gap between the winning logit and the
    best other one over all argmax decisions (decoder.c:107-114; a token can
    change only where a perturbation of the logits exceeds it), with the
    frame where it occurs; the driver's replay of the decode must reproduce
    the reference's tokens."""
    assert ref["margin_replay_equal"] == 1, "the margin replay diverged from pk_greedy_decode"
    return {"min_logit_margin_reference": ref["min_logit_margin"], "margin_frame": ref["margin_frame"],
            "decisions": ref["decisions"]}


def test_reference_drivers_cpu(tmp_path):
    """CPU only: the portable-path and x86 builds run, agree on shape and
    differ in value (the x86 int4 unpack)."""
    ref = run("pk_encode_ref", 48, tmp_path)
    x86 = run("pk_encode_ref_x86", 48, tmp_path)
    assert ref["finite"] == 1 and x86["finite"] == 1 and ref["frames"] == 48
    assert ref["enc_fnv"] != x86["enc_fnv"]


@pytest.fixture
def model_dir(tmp_path):
    """A directory that keeps one written model for the runs of a test (the
    fp32 model is 2.3 GB), removed when the test ends."""
    import shutil
    d = tmp_path / "model"
    yield d
    shutil.rmtree(d, ignore_errors=True)


# the formats pk_load_weights builds from each weight directory
MODE_BITS = {
    "mixed": {"ff_linear1": 4, "ff_linear2": 4, "qkv": 8, "pos": 8, "out": 8, "pre_encode_out": 8},
    "int8": {"ff_linear1": 8, "ff_linear2": 8, "qkv": 8, "pos": 8, "out": 8, "pre_encode_out": 8},
    "fp32": {"ff_linear1": 32, "ff_linear2": 32, "qkv": 32, "pos": 32, "out": 32, "pre_encode_out": 32},
}


def test_reference_driver_int8_model_cpu(tmp_path, model_dir):
    """CPU only: the int8 weight directory's model (every matmul weight int8,
    FF linears included) loads through pk_load_weights with the formats the
    reference builds, and the portable and x86 builds agree bit for bit (the
    x86 build differs only in its int4 unpack, which this model does not
    use)."""
    ref = run("pk_encode_ref", 48, tmp_path, mode="int8", model_dir=model_dir)
    x86 = run("pk_encode_ref_x86", 48, tmp_path, mode="int8", model_dir=model_dir)
    assert ref["bits"] == MODE_BITS["int8"] and x86["bits"] == MODE_BITS["int8"]
    assert ref["finite"] == 1 and ref["enc_fnv"] == x86["enc_fnv"]
    assert ref["tokens_fnv"] == x86["tokens_fnv"]


@pytest.mark.gpu
@pytest.mark.timeout(900)
@pytest.mark.parametrize("mode", ["int8", "fp32"])
def test_gpu_dropin_weight_directories(mode, tmp_path, model_dir):
    """The reference's other two weight directories through the GEMM drop-in,
    900 frames (chunks of 408/416/108 rows): int8 (every matmul weight int8,
    so the FF linears take cblas_sgemm_qb at K = 1024 and 4096) and fp32
    (every matmul cblas_sgemm, the fused QKV the fp32 interleave of
    weights.c:421-436).  Neither uses int4, so the reference exactly as its
    Makefile builds it on x86 (AVX2 weight GEMMs) must agree bit for bit
    too: encoder output and greedy token ids."""
    frames = 900
    gpu = run("pk_encode_gpu", frames, tmp_path, mode=mode, model_dir=model_dir)
    ref = run("pk_encode_ref", frames, tmp_path, mode=mode, model_dir=model_dir)
    x86 = run("pk_encode_ref_x86", frames, tmp_path, mode=mode, model_dir=model_dir)
    assert gpu["bits"] == ref["bits"] == MODE_BITS[mode]
    assert gpu["finite"] == 1 and gpu["chunked"] == ref["chunked"] == 1
    assert gpu["enc_fnv"] == ref["enc_fnv"] == x86["enc_fnv"], "encoder outputs differ"
    assert gpu["n_tokens"] == ref["n_tokens"] == x86["n_tokens"]
    assert gpu["tokens_fnv"] == ref["tokens_fnv"] == x86["tokens_fnv"]
    print(json.dumps({"mode": mode, "frames": frames, "threads": THREADS,
                      "encoder_frames_per_s_gpu_dropin": round(frames / gpu["encoder_s"], 1),
                      "encoder_frames_per_s_cpu_reference_x86": round(frames / x86["encoder_s"], 1),
                      **margin(ref)}),
          flush=True)


@pytest.mark.gpu
@pytest.mark.timeout(600)
@pytest.mark.parametrize("frames", [300, 900, 3200])
def test_gpu_dropin_matches_reference_bit_for_bit(frames, tmp_path):
    """300 frames: full-sequence path (M = 300, pos M = 599); 900 frames:
    chunked path, chunks of 408/416/108 rows (pos 815/831/215); 3200 frames:
    the 256 s encoder (eight chunks of 408/416 rows).  Prints both encoder
    times (the drop-in's includes every host operation and its PCIe copies)."""
    gpu = run("pk_encode_gpu", frames, tmp_path)
    ref = run("pk_encode_ref", frames, tmp_path)
    assert gpu["finite"] == 1
    assert gpu["chunked"] == ref["chunked"] == (1 if frames > 500 else 0)
    assert gpu["enc_fnv"] == ref["enc_fnv"], "encoder outputs differ"
    assert gpu["n_tokens"] == ref["n_tokens"] and gpu["tokens_fnv"] == ref["tokens_fnv"]
    assert gpu["first_tokens"] == ref["first_tokens"]
    print(json.dumps({"frames": frames, "threads": THREADS, **margin(ref),
                      "encoder_frames_per_s_gpu_dropin": round(frames / gpu["encoder_s"], 1),
                      "encoder_frames_per_s_cpu_reference": round(frames / ref["encoder_s"], 1),
                      **margin(ref)}),
          flush=True)
    if frames < 3200:
        x86 = run("pk_encode_ref_x86", frames, tmp_path)
        assert x86["enc_fnv"] != ref["enc_fnv"]


@pytest.mark.gpu
@pytest.mark.timeout(600)
@pytest.mark.parametrize("attn_gain", [0.05, None], ids=["trained_like", "workload_stats"])
def test_gpu_dropin_short_clip_small_m(attn_gain, tmp_path):
    """A 2.56 s clip, T' = 33 encoder frames, through the GEMM drop-in: its
    int8 QKV / output and int4 feed-forward GEMMs have M = 33 and take the
    small-M kernels (the tolerance path); the position projection (M = 65)
    and the fp32 pointwise convolutions keep the exact chains.  With
    trained-like attention weights the encoder output stays within 1e-3 of
    the reference's and the greedy token ids are equal; at the workloads'
    int8 statistics, where the reference amplifies any difference tenfold per
    block, both are reported.  With PK_GPU_NUMERICS=exact the same run is
    bit-identical to the reference."""
    import numpy as np
    frames = 33
    gpu = run("pk_encode_gpu", frames, tmp_path, dump=tmp_path / "gpu.f32", attn_gain=attn_gain)
    ref = run("pk_encode_ref", frames, tmp_path, dump=tmp_path / "ref.f32", attn_gain=attn_gain)
    exact = run("pk_encode_gpu", frames, tmp_path, attn_gain=attn_gain,
                extra_env={"PK_GPU_NUMERICS": "exact"})
    a = np.fromfile(tmp_path / "gpu.f32", dtype=np.float32)
    b = np.fromfile(tmp_path / "ref.f32", dtype=np.float32)
    dev = float(np.abs(a - b).max() / np.abs(b).max())
    print(json.dumps({"frames": frames, "attn_gain": attn_gain, "max_rel_deviation_small_m": dev,
                      "tokens_small_m": gpu["n_tokens"], "tokens_reference": ref["n_tokens"],
                      "tokens_equal": gpu["tokens_fnv"] == ref["tokens_fnv"],
                      "exact_mode_bit_identical": exact["enc_fnv"] == ref["enc_fnv"], **margin(ref)}),
          flush=True)
    assert gpu["finite"] == 1 and gpu["chunked"] == ref["chunked"] == 0
    assert exact["enc_fnv"] == ref["enc_fnv"] and exact["tokens_fnv"] == ref["tokens_fnv"]
    if attn_gain is not None:
        assert dev <= 1e-3
        assert gpu["n_tokens"] == ref["n_tokens"] and gpu["tokens_fnv"] == ref["tokens_fnv"], margin(ref)


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_gpu_dropin_fast_numerics(tmp_path):
    """600 frames (two chunks of about 316 rows) through the GEMM drop-in with
    PK_GPU_NUMERICS=fast: every weight GEMM of the reference's encoder.c takes
    the split kernels (rows > 64), each within 1e-3 of the reference GEMM.
    With trained-like attention weights the encoder output stays within 1e-3
    of the reference's and the greedy token ids are equal."""
    import numpy as np
    frames = 600
    gpu = run("pk_encode_gpu", frames, tmp_path, dump=tmp_path / "gpu.f32", attn_gain=0.05,
              extra_env={"PK_GPU_NUMERICS": "fast"})
    ref = run("pk_encode_ref", frames, tmp_path, dump=tmp_path / "ref.f32", attn_gain=0.05)
    a = np.fromfile(tmp_path / "gpu.f32", dtype=np.float32)
    b = np.fromfile(tmp_path / "ref.f32", dtype=np.float32)
    dev = float(np.abs(a - b).max() / np.abs(b).max())
    print(json.dumps({"frames": frames, "max_rel_deviation_fast": dev, "tokens_fast": gpu["n_tokens"],
                      "tokens_reference": ref["n_tokens"],
                      "tokens_equal": gpu["tokens_fnv"] == ref["tokens_fnv"], **margin(ref)}), flush=True)
    assert gpu["finite"] == 1 and gpu["chunked"] == ref["chunked"]
    assert dev <= 1e-3
    assert gpu["n_tokens"] == ref["n_tokens"] and gpu["tokens_fnv"] == ref["tokens_fnv"], margin(ref)


def resident_vs_reference(frames, tmp_path, attn_gain, from_mel=False, mode=None):
    import shutil

    mdir = tmp_path / "model"
    try:
        return _resident_vs_reference(frames, tmp_path, attn_gain, from_mel, mode, mdir)
    finally:
        shutil.rmtree(mdir, ignore_errors=True)


def _resident_vs_reference(frames, tmp_path, attn_gain, from_mel, mode, mdir):
    import numpy as np
    gres = run("pk_encode_gpures", frames, tmp_path, dump=tmp_path / "gpures.f32", attn_gain=attn_gain,
               from_mel=from_mel, mode=mode, model_dir=mdir)
    ref = run("pk_encode_ref", frames, tmp_path, dump=tmp_path / "ref.f32", attn_gain=attn_gain,
              from_mel=from_mel, mode=mode, model_dir=mdir)
    assert gres["bits"] == ref["bits"] == MODE_BITS[mode or "mixed"]
    a = np.fromfile(tmp_path / "gpures.f32", dtype=np.float32).reshape(frames, 1024)
    b = np.fromfile(tmp_path / "ref.f32", dtype=np.float32).reshape(frames, 1024)
    dev = float(np.abs(a - b).max() / np.abs(b).max())
    print(json.dumps({"frames": frames, "mode": mode or "mixed", "from_mel": from_mel, "attn_gain": attn_gain,
                      "threads": THREADS,
                      "max_rel_deviation": dev, "identical_fraction": float(np.mean(a == b)),
                      "tokens_gpu_resident": gres["n_tokens"], "tokens_reference": ref["n_tokens"],
                      "tokens_equal": gres["tokens_fnv"] == ref["tokens_fnv"],
                      "encoder_frames_per_s_gpu_resident": round(frames / gres["encoder_s"], 1),
                      "encoder_s_gpu_resident_first_call": gres["encoder_first_s"],
                      "encoder_frames_per_s_cpu_reference": round(frames / ref["encoder_s"], 1)}),
          flush=True)
    assert gres["finite"] == 1
    assert gres["chunked"] == ref["chunked"]
    return gres, ref, dev


@pytest.mark.gpu
@pytest.mark.timeout(600)
@pytest.mark.parametrize("frames", [300, 900, 3200])
def test_gpu_resident_encoder_matches_reference(frames, tmp_path):
    """The 24 blocks run by the device-resident encoder (pk_gpu_encoder_run:
    one batch of all chunks, every activation on the device) in place of
    encode_blocks / encode_blocks_chunked, the reference's greedy decoder on
    its output, on the synthetic model with trained-like attention weights
    (PK_SYNTH_ATTN_GAIN = 0.05).  The weight GEMMs, attention and the
    depthwise convolution are bit-exact; LayerNorm's 1/sqrt, Swish's and
    GLU's reciprocal and GLU's exp are correctly rounded where the reference
    uses CPU-model-specific approximations, so the encoder output is
    compared within max |gpu - ref| / max |ref| <= 1e-3 and the token ids
    exactly."""
    gres, ref, dev = resident_vs_reference(frames, tmp_path, 0.05)
    assert dev <= 1e-3
    assert gres["n_tokens"] == ref["n_tokens"] and gres["tokens_fnv"] == ref["tokens_fnv"], margin(ref)


@pytest.mark.gpu
@pytest.mark.timeout(600)
def test_gpu_resident_encoder_workload_stats(tmp_path):
    """The same at the workloads' int8 statistics (gain 1), where the
    reference amplifies any 1-ulp difference about tenfold per block
    (test_oracle_block.test_reference_sensitivity): after 24 blocks its
    output is set by its own rounding, so only a bit-identical host
    computation (the GEMM drop-in above) reproduces it.  Reported, with the
    encoder speed; the output must be finite and of the reference's
    magnitude.  (Against the oracle, which takes the source's IEEE operations
    where the reference build takes CPU-specific approximations, the
    resident encoder is bit-identical at these statistics:
    test_gpu_encoder_golden.)"""
    import numpy as np
    gres, ref, dev = resident_vs_reference(3200, tmp_path, None)
    a = np.fromfile(tmp_path / "gpures.f32", dtype=np.float32)
    b = np.fromfile(tmp_path / "ref.f32", dtype=np.float32)
    assert 0.5 < np.abs(a).max() / np.abs(b).max() < 2.0


@pytest.mark.gpu
@pytest.mark.timeout(600)
@pytest.mark.parametrize("frames", [300, 900])
def test_gpu_resident_encoder_from_mel(frames, tmp_path):
    """pk_encoder from a mel spectrogram ([128][8 x frames] ~N(0,1)): the
    reference's pre-encode + blocks on the CPU, against
    pk_gpu_encoder_run_mel (pre-encode on the device, bit-identical, then the
    resident blocks), trained-like attention weights; token ids equal."""
    gres, ref, dev = resident_vs_reference(frames, tmp_path, 0.05, from_mel=True)
    assert dev <= 1e-3
    assert gres["n_tokens"] == ref["n_tokens"] and gres["tokens_fnv"] == ref["tokens_fnv"], margin(ref)


@pytest.mark.gpu
@pytest.mark.timeout(900)
@pytest.mark.parametrize("mode", ["int8", "fp32"])
def test_gpu_resident_encoder_weight_directories(mode, tmp_path):
    """The device-resident encoder on the int8 and fp32 weight directories'
    models (every block linear int8, or every one fp32, including the fused
    QKV and the position projection), 900 frames from mel, trained-like
    attention weights: pre-encode's int8 or fp32 output projection, then the
    blocks; within 1e-3 of the reference and token ids equal, as for the
    mixed model."""
    gres, ref, dev = resident_vs_reference(900, tmp_path, 0.05, from_mel=True, mode=mode)
    assert dev <= 1e-3
    assert gres["n_tokens"] == ref["n_tokens"] and gres["tokens_fnv"] == ref["tokens_fnv"], margin(ref)
