"""Committed golden vectors (tests/golden/, written by make_golden.py from
the reference compiled from its own sources): the oracle must reproduce
them bit for bit on the CPU, the GPU path on the GPU, and the seeded
benchmark inputs must hash to the committed digests on every host."""
import hashlib
import json
import os

import numpy as np
import pytest

import pyoracle as po

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
KINDS = ["f32", "i8", "i4"]


def cases():
    z = np.load(os.path.join(GOLD, "gemm_cases.npz"))
    n = len([k for k in z.files if k.endswith("_meta")])
    for i in range(n):
        t = f"c{i}"
        kind = KINDS[int(z[t + "_kind"])]
        extra = (float(z[t + "_scale"]) if kind == "i8" else
                 z[t + "_scales"] if kind == "i4" else None)
        alpha, beta = (float(v) for v in z[t + "_ab"])
        yield t, kind, z[t + "_A"], z[t + "_W"], extra, z[t + "_C0"], alpha, beta, z[t + "_C"]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_oracle_reproduces_golden_vectors():
    for t, kind, A, W, extra, C0, alpha, beta, want in cases():
        C = C0.copy()
        if kind == "f32":
            po.sgemm(A, W, C, alpha, beta)
        elif kind == "i8":
            po.sgemm_qb(A, W, extra, C, alpha, beta)
        else:
            po.sgemm_q4b(A, W, extra, C, alpha, beta)
        assert np.array_equal(bits(C), bits(want)), t


def test_bench_inputs_match_committed_digests():
    import sys
    sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
    import bench
    X, P1, S1, P2, S2 = bench.make_inputs()
    want = json.load(open(os.path.join(GOLD, "digests.json")))
    got = {name: hashlib.sha256(a.tobytes()).hexdigest()
           for name, a in (("ffn_X", X), ("ffn_up_P", P1), ("ffn_up_S", S1),
                           ("ffn_down_P", P2), ("ffn_down_S", S2))}
    assert got == want


@pytest.mark.gpu
def test_gpu_reproduces_golden_vectors():
    from pkgpu import Dev
    dev = Dev()
    for t, kind, A, W, extra, C0, alpha, beta, want in cases():
        if kind == "i4":
            got = dev.gemm(kind, A, W, C0, alpha, beta, scales=extra)
        elif kind == "i8":
            got = dev.gemm(kind, A, W, C0, alpha, beta, scale=extra)
        else:
            got = dev.gemm(kind, A, W, C0, alpha, beta)
        assert np.array_equal(bits(got), bits(want)), t
