"""Writes tests/golden/gemm_cases.npz: small GEMM cases computed by the
reference compiled from its own sources (oracle/_ref, built by
oracle/Makefile), and tests/golden/digests.json: SHA-256 of the seeded
inputs of each benchmark workload.

int8 and fp32 outputs come from the x86 AVX2 build (libpkref.so); int4
outputs from the portable-path build (libpkref_portable.so), because the
AVX2 int4 unpack mis-decodes nibbles (blas.c:815-833).

Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import pyoracle as po  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
SEED = 0x601D0000

CASES = [  # kind, M, N, K, alpha, beta
    ("f32", 3, 40, 70, 1.0, 0.0), ("f32", 5, 17, 33, 0.75, 0.5), ("f32", 33, 64, 130, 1.0, 1.0),
    ("i8", 4, 48, 100, 1.0, 0.0), ("i8", 6, 31, 77, 0.75, 0.5), ("i8", 33, 64, 130, 1.0, -2.0),
    ("i4", 2, 64, 90, 1.0, 0.0), ("i4", 7, 96, 64, 0.75, 0.5), ("i4", 33, 128, 130, 1.0, 1.0),
]


def main():
    os.environ.setdefault("PK_THREADS", "4")
    arrays = {}
    for idx, (kind, M, N, K, alpha, beta) in enumerate(CASES):
        tag = f"c{idx}"
        A = po.normal((M, K), 0.0, 1.0, po.seed(SEED, tag + ".A"))
        C0 = po.normal((M, N), 0.0, 1.0, po.seed(SEED, tag + ".C"))
        C = C0.copy()
        if kind == "f32":
            W = po.normal((K, N), 0.0, 0.02, po.seed(SEED, tag + ".W"))
            po.sgemm(A, W, C, alpha, beta, impl="ref")
        elif kind == "i8":
            W = po.int8s((K, N), -127, 127, po.seed(SEED, tag + ".W"))
            arrays[tag + "_scale"] = np.float32(0.0123)
            po.sgemm_qb(A, W, 0.0123, C, alpha, beta, impl="ref")
        else:
            W = po.bytes_((K, N // 2), po.seed(SEED, tag + ".W"))
            S = po.uniform((K, N // 32), 0.005, 0.02, po.seed(SEED, tag + ".S"))
            arrays[tag + "_scales"] = S
            po.sgemm_q4b(A, W, S, C, alpha, beta, impl="portable")
        arrays[tag + "_meta"] = np.array([M, N, K], np.int64)
        arrays[tag + "_ab"] = np.array([alpha, beta], np.float32)
        arrays[tag + "_kind"] = np.array(["f32", "i8", "i4"].index(kind), np.int64)
        arrays[tag + "_A"], arrays[tag + "_W"], arrays[tag + "_C0"] = A, W, C0
        arrays[tag + "_C"] = C
    np.savez_compressed(os.path.join(OUT, "gemm_cases.npz"), **arrays)

    # digests of the seeded benchmark inputs (the bytes both hosts must share)
    sys.path.insert(0, ROOT)
    import bench
    X, P1, S1, P2, S2 = bench.make_inputs()
    dig = {name: hashlib.sha256(a.tobytes()).hexdigest()
           for name, a in (("ffn_X", X), ("ffn_up_P", P1), ("ffn_up_S", S1),
                           ("ffn_down_P", P2), ("ffn_down_S", S2))}
    json.dump(dig, open(os.path.join(OUT, "digests.json"), "w"), indent=1)
    print(f"wrote {len(CASES)} cases and {len(dig)} digests")


if __name__ == "__main__":
    main()
