"""Benchmark: the GPTQ int4 FastConformer FFN pair on one MI355X.

Workload (one "step"): X fp32 [375, 1024] ~ N(0,1)  ->  int4 GEMM up
(1024 -> 4096, packed nibbles [1024][2048] with fp32 scales [1024][128])
with Swish fused into its output store  ->  int4 GEMM down (4096 -> 1024,
[4096][512] + [4096][32]),
i.e. the feed-forward of 30 s of audio (375 encoder frames,
encoder.c:179-217 without the host bias/residual adds), through the C ABI
of libpk_gpu.so with every input already resident in HBM.  Weight nibbles
are uniform 0..15 (decoded signed, as the format defines) and scales
~U(0.005, 0.02); the steps rotate over enough weight replicas (> 256 MB)
that weights stream from HBM rather than from the 256 MB Infinity Cache.

Prints one JSON line: encoder frames/s through the pair, plus
  roofline      the int4 GEMM kernel: algorithmic flops / HIP-event time,
                against the fp32 dense MFMA peak (the instruction it issues)
  cpu_baseline  the reference's own cblas_sgemm_q4b + pk_swish (compiled
                from its sources, oracle/_ref/libpkref.so) on a bounded
                sample of the same workload, PK_THREADS=16 host threads.
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "tests"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

METRIC = "encoder frames/sec + GEMM GB/s & TFLOP/s vs MI355X roofline (int4/int8)"
M, D, FF = 375, 1024, 4096
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
CPU_THREADS = 16            # the reference clamps PK_THREADS to 16 (threadpool.c:10)
SEED = 0x5EED0001           # workload 1


def int4_bytes(K, N):
    """Algorithmic bytes of one int4 GEMM: packed weights + scales + A + C."""
    return K * N // 2 + 4 * K * (N // 32) + 4 * M * K + 4 * M * N


def make_inputs(po):
    X = po.normal((M, D), 0.0, 1.0, po.seed(SEED, "X"))
    P1 = po.bytes_((D, FF // 2), po.seed(SEED, "up.P"))
    S1 = po.uniform((D, FF // 32), 0.005, 0.02, po.seed(SEED, "up.S"))
    P2 = po.bytes_((FF, D // 2), po.seed(SEED, "down.P"))
    S2 = po.uniform((FF, D // 32), 0.005, 0.02, po.seed(SEED, "down.S"))
    return X, P1, S1, P2, S2


def cpu_baseline(po, X, P1, S1, P2, S2, budget_s):
    """The reference's CPU path on the same inputs, timed for ~budget_s."""
    os.environ["PK_THREADS"] = str(CPU_THREADS)
    ref = po.ref("ref")
    threads = ref.pk_pool_nthreads(ref.pk_pool())
    h = np.empty((M, FF), np.float32)
    out = np.empty((M, D), np.float32)

    def step():
        po.sgemm_q4b(X, P1, S1, h, impl="ref")
        ref.pk_swish(h.ctypes.data, h.size)
        po.sgemm_q4b(h, P2, S2, out, impl="ref")

    step()                                  # allocates the per-thread pack buffers
    n, t0 = 0, time.perf_counter()
    while True:
        step()
        n += 1
        el = time.perf_counter() - t0
        if el >= budget_s or n >= 2000:
            break
    return {"value": round(M * n / el, 1), "unit": "frames/s", "cores": threads,
            "kind": "reference",
            "sample": f"{n} FFN-pair steps (M=375, 1024->4096->1024) in {el:.1f} s; "
                      f"cblas_sgemm_q4b x2 + pk_swish, x86 AVX2 build, {threads} threads",
            "ms_per_step": round(1000 * el / n, 3)}


def copy_calibration():
    """10 torch device copies of 256 MiB: each reads and writes exactly
    268,435,456 bytes, which scales the traffic counters."""
    import torch
    src = torch.ones(64 * 1024 * 1024, dtype=torch.float32, device="cuda:0")
    dst = torch.empty_like(src)
    for _ in range(10):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": src.numel() * 4, "copies": 10}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--replicas", type=int, default=64)
    ap.add_argument("--cpu-seconds", type=float, default=15.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run 10 plain 256 MiB device-to-device copies (the reference "
                         "reading for FETCH_SIZE / WRITE_SIZE counters) and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (single-GPU hot path; "
              "multi-GPU sharding is a design note, not built)", file=sys.stderr)
        sys.exit(2)

    import torch
    from pkgpu import pk
    import pyoracle as po

    pk.call("pk_gpu_init", 0)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    s = stream.cuda_stream

    X, P1, S1, P2, S2 = make_inputs(po)
    R = args.replicas
    dX = torch.from_numpy(X).to(dev)
    # rotating weight replicas: R copies of (P1, S1, P2, S2), 5.2 MB each
    reps = []
    for r in range(R):
        reps.append(tuple(torch.from_numpy(a).to(dev) for a in (P1, S1, P2, S2)))
    dH = torch.empty((M, FF), dtype=torch.float32, device=dev)
    dO = torch.empty((M, D), dtype=torch.float32, device=dev)
    lib = pk.load()

    def up(i):
        # up-projection with Swish fused into its output store (encoder.c:193-196)
        p, sc = reps[i % R][0], reps[i % R][1]
        return lib.pk_gpu_gemm_i4_ex_dev(M, FF, D, 1.0, dX.data_ptr(), D, p.data_ptr(),
                                         sc.data_ptr(), FF // 2, 0.0, dH.data_ptr(), FF, None,
                                         pk.EPI_SWISH, s)

    def down(i):
        p, sc = reps[i % R][2], reps[i % R][3]
        return lib.pk_gpu_gemm_i4_dev(M, D, FF, 1.0, dH.data_ptr(), FF, p.data_ptr(), sc.data_ptr(),
                                      D // 2, 0.0, dO.data_ptr(), D, s)

    for i in range(args.warmup):
        assert up(i) == 0 and down(i) == 0, pk.load().pk_gpu_last_error()
    torch.cuda.synchronize(dev)

    # timed region: K steps; events bracket each GEMM launch on the same stream
    K = args.steps
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(K)]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    wall0 = time.perf_counter()
    t_start.record(stream)
    rc = 0
    for i in range(K):
        e = ev[i]
        e[0].record(stream)
        rc |= up(i)
        e[1].record(stream)
        rc |= down(i)
        e[2].record(stream)
    t_end.record(stream)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - wall0
    if rc:
        raise RuntimeError(pk.load().pk_gpu_last_error())

    elapsed_ms = t_start.elapsed_time(t_end)
    ms_per_step = elapsed_ms / K
    up_ms = sum(e[0].elapsed_time(e[1]) for e in ev) / K
    dn_ms = sum(e[1].elapsed_time(e[2]) for e in ev) / K

    flops_up = 2.0 * M * FF * D
    flops_dn = 2.0 * M * D * FF
    gemm_s = (up_ms + dn_ms) / 1e3
    tflops = (flops_up + flops_dn) / gemm_s / 1e12
    gbytes = (int4_bytes(D, FF) + int4_bytes(FF, D)) / gemm_s / 1e9
    frames_per_s = M * K / (elapsed_ms / 1e3)

    cfg_up = lib.pk_gpu_pick_config(M, FF, D)
    cfg_dn = lib.pk_gpu_pick_config(M, D, FF)
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "int4_ffn_pair_m375_traffic.json")
    if os.path.exists(tpath):
        traffic = json.load(open(tpath)).get("hbm_bytes_per_launch")

    out = {
        "metric": METRIC,
        "value": round(frames_per_s, 1),
        "unit": "frames/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "int4 FFN pair, M=375 frames (30 s audio), 1024->4096 swish 4096->1024, "
                               "packed int4 weights, 32-column fp32 scales",
                   "M": M, "d_model": D, "d_ff": FF, "weight_replicas": R,
                   "tile_configs": [cfg_up, cfg_dn]},
        "gemm_tflops": round(tflops, 2),
        "gemm_gbps": round(gbytes, 1),
        "kernel_us": {"int4_up_swish": round(up_ms * 1e3, 2), "int4_down": round(dn_ms * 1e3, 2)},
        "wall_ms_per_step": round(1e3 * wall / K, 4),
        "roofline": {"bound": "mfma", "kernel": "int4 chain GEMM (up with fused Swish, and down)",
                     "achieved": round(tflops, 2), "peak": PEAK_FP32_MFMA_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_FP32_MFMA_TFLOPS, 4),
                     "traffic": traffic},
    }
    if not args.no_cpu and po.have_ref():
        out["cpu_baseline"] = cpu_baseline(po, X, P1, S1, P2, S2, args.cpu_seconds)
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
