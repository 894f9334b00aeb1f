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
PKG = os.path.join(ROOT, "parakeet-unified-en-0.6b-c_amd")

METRIC = "encoder frames/sec + GEMM GB/s & TFLOP/s vs MI355X roofline (int4/int8)"
M, D, FF = 375, 1024, 4096
PEAK_FP32_MFMA_TFLOPS = 157.3
PEAK_HBM_GBS = 8000.0
CPU_THREADS = 16            # the reference clamps PK_THREADS to 16 (threadpool.c:10)
SEED = 0x5EED0001           # workload 1


def int4_bytes(K, N):
    """Algorithmic bytes of one int4 GEMM: packed weights + scales + A + C."""
    return K * N // 2 + 4 * K * (N // 32) + 4 * M * K + 4 * M * N


def rng(tensor):
    """numpy PCG64 stream of one named tensor of the workload (platform-independent)."""
    return np.random.Generator(np.random.PCG64([SEED, tensor]))


def make_inputs():
    """Seeded synthetic inputs: X ~ N(0,1); packed int4 bytes uniform 0..255 (each
    nibble uniform 0..15, decoded signed); scales ~U(0.005, 0.02)."""
    X = rng(0).standard_normal((M, D)).astype(np.float32)
    P1 = rng(1).integers(0, 256, (D, FF // 2), dtype=np.uint8)
    S1 = rng(2).uniform(0.005, 0.02, (D, FF // 32)).astype(np.float32)
    P2 = rng(3).integers(0, 256, (FF, D // 2), dtype=np.uint8)
    S2 = rng(4).uniform(0.005, 0.02, (FF, D // 32)).astype(np.float32)
    return X, P1, S1, P2, S2


def cpu_baseline(X, P1, S1, P2, S2, budget_s):
    """The reference's CPU path on the same inputs, timed for ~budget_s: its own
    cblas_sgemm_q4b and pk_swish, compiled from its sources into oracle/_ref."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as po
    if not po.have_ref():
        return None
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


def load_binding():
    """The ctypes binding of libpk_gpu.so (raises if the library was not built)."""
    import importlib.util
    spec = importlib.util.spec_from_file_location("pk_gpu_ctypes", os.path.join(PKG, "pk_gpu_ctypes.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


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


def alg_bytes(kind, m, n, k):
    """Algorithmic bytes of one GEMM call: weights (+ int4 scales) + A + C."""
    w = {"i4": k * n // 2 + 4 * k * (n // 32), "i8": k * n + 4, "f32": 4 * k * n}[kind]
    return w + 4 * m * k + 4 * m * n


def gemm_mode(specs, steps, warmup, min_weight_bytes=512 << 20):
    """One JSON line per GEMM shape ("kind:MxNxK"): resident inputs, weights
    rotating over enough replicas to exceed the Infinity Cache, average launch
    time from HIP events around a graph replay of `steps` launches."""
    import torch
    pk = load_binding()
    pk.call("pk_gpu_init", 0)
    lib = pk.load()
    dev = torch.device("cuda:0")
    cur = lambda: torch.cuda.current_stream(dev).cuda_stream   # the capture stream inside a graph
    g = torch.Generator(device=dev)
    for spec in specs:
        kind, dims = spec.split(":")
        m, n, k = (int(v) for v in dims.lower().split("x"))
        g.manual_seed(SEED)
        A = torch.randn((m, k), generator=g, device=dev)
        C = torch.zeros((m, n), device=dev)
        wbytes = alg_bytes(kind, m, n, k) - 4 * m * k - 4 * m * n
        reps = max(2, min(256, -(-min_weight_bytes // wbytes)))
        if kind == "i4":
            W = [torch.randint(0, 256, (k, n // 2), dtype=torch.uint8, device=dev, generator=g)
                 for _ in range(reps)]
            S = [torch.rand((k, n // 32), device=dev, generator=g) * 0.015 + 0.005 for _ in range(reps)]
            call = lambda i: lib.pk_gpu_gemm_i4_dev(m, n, k, 1.0, A.data_ptr(), k, W[i % reps].data_ptr(),
                                                    S[i % reps].data_ptr(), n // 2, 0.0, C.data_ptr(), n,
                                                    cur())
        elif kind == "i8":
            W = [torch.randint(-127, 128, (k, n), dtype=torch.int8, device=dev, generator=g)
                 for _ in range(reps)]
            call = lambda i: lib.pk_gpu_gemm_i8_dev(m, n, k, 1.0, A.data_ptr(), k, W[i % reps].data_ptr(),
                                                    0.01, n, 0.0, C.data_ptr(), n, cur())
        else:
            W = [torch.randn((k, n), device=dev, generator=g) * 0.02 for _ in range(reps)]
            call = lambda i: lib.pk_gpu_sgemm_dev(m, n, k, 1.0, A.data_ptr(), k, W[i % reps].data_ptr(),
                                                  n, 0.0, C.data_ptr(), n, cur())
        for i in range(warmup):
            assert call(i) == 0, lib.pk_gpu_last_error()
        torch.cuda.synchronize(dev)
        # The launches are captured into one HIP graph and replayed, so they run
        # back to back: a host loop of ctypes launches cannot keep a queue of
        # ~10 us kernels full, and per-launch events would time its gaps.
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for i in range(steps):
                call(i)
        graph.replay()
        torch.cuda.synchronize(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        graph.replay()
        e1.record()
        torch.cuda.synchronize(dev)
        us = e0.elapsed_time(e1) / steps * 1e3
        del graph
        tf = 2.0 * m * n * k / us / 1e6
        gbs = alg_bytes(kind, m, n, k) / us / 1e3
        print(json.dumps({"gemm": f"{kind} {m}x{n}x{k}", "config": lib.pk_gpu_pick_config(m, n, k),
                          "avg_us": round(us, 2), "tflops": round(tf, 2), "gbps": round(gbs, 1),
                          "frac_mfma_fp32": round(tf / PEAK_FP32_MFMA_TFLOPS, 4),
                          "frac_hbm": round(gbs / PEAK_HBM_GBS, 4), "weight_replicas": reps,
                          "steps": steps}), flush=True)
        del W, A, C
        torch.cuda.empty_cache()


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
    ap.add_argument("--gemm", action="append", default=[], metavar="KIND:MxNxK",
                    help="instead of the FFN pair, time single GEMMs (kind i4, i8 or f32); "
                         "one JSON line each")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gemm:
        gemm_mode(args.gemm, args.steps, args.warmup)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py: this build runs on one GPU only (single-GPU hot path; "
              "multi-GPU sharding is a design note, not built)", file=sys.stderr)
        sys.exit(2)

    import torch
    pk = load_binding()

    pk.call("pk_gpu_init", 0)
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    stream = torch.cuda.current_stream(dev)
    s = stream.cuda_stream

    X, P1, S1, P2, S2 = make_inputs()
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
    out["cpu_baseline"] = None if args.no_cpu else cpu_baseline(X, P1, S1, P2, S2, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
