"""Writes tests/golden/encoder_golden.json: SHA-256 digests of the oracle's
whole encoder (oracle/pk_oracle_encoder.c) on bench.py's own encoder workload,
the model and features the benchmark times: 24 conformer blocks with the
workloads' quantization statistics (EncoderModel), 3200 frames of N(0,1)
features (encoder_features), chunks of 400 frames with 8 frames of overlap.

Recorded per workload: the digest of the [T][1024] fp32 output, the digests
of the output after every block (the same input through the first b blocks,
which is what an encoder created with b blocks returns), and the digests of
the inputs, so a mismatch can be traced to its first block.  A second,
smaller workload (900 frames: chunks of 408, 416 and 108 rows, the last one
exercising softmax's scalar tail) is recorded the same way.

Run from the repository root:  python tests/golden/make_encoder_golden.py
(about a minute on 8 cores).
"""
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import bench  # noqa: E402
import pyoracle as po  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "encoder_golden.json")
WORKLOADS = [(bench.ENC_FRAMES, bench.ENC_CHUNK, bench.ENC_OVERLAP), (900, 400, 8)]


def sha(a):
    return hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()


def main():
    pk = bench.load_binding()
    model = bench.EncoderModel(pk)
    res = {"model": "bench.EncoderModel (24 blocks, seed 0x5EED0004), pe table 9999 x 1024 "
                    "centre 4999", "pe_sha256": sha(model.pe), "workloads": []}
    for T, C, ov in WORKLOADS:
        x = bench.encoder_features(T)
        t0 = time.time()
        out, snaps = po.encoder(model.blocks, bench.N_BLOCKS, model.pe, bench.PE_CENTER, x, C, ov,
                                snapshots=True)
        el = time.time() - t0
        assert np.isfinite(out).all()
        res["workloads"].append({
            "frames": T, "chunk": C, "overlap": ov, "blocks": bench.N_BLOCKS,
            "chunk_rows": bench.chunk_rows(T, C, ov),
            "input_sha256": sha(x),
            "output_sha256": sha(out),
            "after_block_sha256": [sha(s) for s in snaps],
            "output_max_abs": float(np.abs(out).max()),
            "output_mean_abs": float(np.abs(out).mean()),
            "oracle_seconds": round(el, 1),
        })
        print(f"{T} frames: {sha(out)} ({el:.1f} s)", flush=True)
    with open(OUT, "w") as f:
        json.dump(res, f, indent=1)
        f.write("\n")
    print("wrote", OUT)


if __name__ == "__main__":
    main()
