"""Test helpers: load the ctypes binding of libpk_gpu.so and run GEMMs
through its C ABI on device buffers, plus bit-level comparison helpers."""
import importlib.util
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "parakeet-unified-en-0.6b-c_amd")

_spec = importlib.util.spec_from_file_location("pk_gpu_ctypes", os.path.join(PKG, "pk_gpu_ctypes.py"))
pk = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(pk)


def gpu_available():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def bits_equal(a, b):
    return np.array_equal(np.asarray(a, np.float32).view(np.uint32),
                          np.asarray(b, np.float32).view(np.uint32))


def describe_mismatch(got, want):
    """Where GPU and oracle differ: count, worst ulp distance, first index,
    and whether the first wrong value sits elsewhere in `want` (a layout
    permutation) or is off by a few ulp (an arithmetic difference)."""
    g = got.view(np.int32).astype(np.int64)
    w = want.view(np.int32).astype(np.int64)
    bad = np.argwhere(g != w)
    if bad.size == 0:
        return "identical"
    i, j = bad[0]
    ulp = np.abs(g - w).max()
    where = np.argwhere(want == got[i, j])
    loc = where[0].tolist() if where.size else None
    return (f"{len(bad)} of {got.size} differ; max ulp {ulp}; first ({i},{j}) "
            f"got {got[i, j]!r} want {want[i, j]!r}; got value found in want at {loc}")


class Dev:
    """Device buffers from numpy via torch, and GEMMs through the C ABI."""

    def __init__(self):
        import torch
        self.torch = torch
        self.dev = torch.device("cuda:0")
        pk.call("pk_gpu_init", 0)

    def put(self, a):
        return self.torch.from_numpy(np.ascontiguousarray(a)).to(self.dev)

    def stream(self):
        return self.torch.cuda.current_stream(self.dev).cuda_stream

    def sync(self):
        self.torch.cuda.synchronize(self.dev)

    def gemm(self, kind, A, W, C0, alpha=1.0, beta=0.0, scale=None, scales=None, cfg=-1,
             bias=None, epi=None, exact=True, numerics=None):
        """Run C = beta*C0 + alpha*A*W through the *_dev entry points (the *_ex_dev
        ones when a bias or an epilogue is given); returns numpy C.  exact: with
        PK_GPU_NUMERICS_EXACT on this thread (bit-identical chains for every
        shape); otherwise the default numerics (the small-M kernels for M <= 64).
        numerics, when given, is the PK_GPU_NUMERICS_* mode instead."""
        lib = pk.load()
        prev = lib.pk_gpu_get_numerics()
        mode = numerics if numerics is not None else (pk.NUMERICS_EXACT if exact else pk.NUMERICS_DEFAULT)
        pk.call("pk_gpu_set_numerics", mode)
        try:
            return self._gemm(kind, A, W, C0, alpha, beta, scale, scales, cfg, bias, epi)
        finally:
            pk.call("pk_gpu_set_numerics", prev)

    def _gemm(self, kind, A, W, C0, alpha, beta, scale, scales, cfg, bias, epi):
        M, K = A.shape
        dA, dC = self.put(A), self.put(C0)
        ex = bias is not None or epi is not None
        dbias = self.put(bias) if bias is not None else None
        tail = ((dbias.data_ptr() if dbias is not None else None, epi or 0, self.stream())
                if ex else (self.stream(),))
        pk.call("pk_gpu_force_config", cfg)
        try:
            if kind == "i4":
                N = W.shape[1] * 2
                dW, dS = self.put(W), self.put(scales)
                pk.call("pk_gpu_gemm_i4_ex_dev" if ex else "pk_gpu_gemm_i4_dev", M, N, K, alpha,
                        dA.data_ptr(), K, dW.data_ptr(), dS.data_ptr(), N // 2, beta,
                        dC.data_ptr(), N, *tail)
            elif kind == "i8":
                N = W.shape[1]
                dW = self.put(W)
                pk.call("pk_gpu_gemm_i8_ex_dev" if ex else "pk_gpu_gemm_i8_dev", M, N, K, alpha,
                        dA.data_ptr(), K, dW.data_ptr(), scale, N, beta, dC.data_ptr(), N, *tail)
            else:
                N = W.shape[1]
                dW = self.put(W)
                pk.call("pk_gpu_sgemm_ex_dev" if ex else "pk_gpu_sgemm_dev", M, N, K, alpha,
                        dA.data_ptr(), K, dW.data_ptr(), N, beta, dC.data_ptr(), N, *tail)
        finally:
            pk.call("pk_gpu_force_config", -1)
        self.sync()
        return dC.cpu().numpy()

    def swish(self, X):
        """pk_gpu_swish_dev on a copy of X; returns numpy."""
        dX = self.put(X)
        pk.call("pk_gpu_swish_dev", dX.data_ptr(), dX.data_ptr(), dX.numel(), self.stream())
        self.sync()
        return dX.cpu().numpy()
