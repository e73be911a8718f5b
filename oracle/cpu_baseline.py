"""ctypes driver of oracle/build/libcpu_kern_port.so, the C++ restatement of the reference CPU kernel
(cpu_ext/cpu_kern.cpp gather_qmm) used as the timed CPU baseline.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py): bench.py's cpu_baseline leg and the tests load it; the product
path never does.
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "build" / "libcpu_kern_port.so"
_LIB = None

_P, _I, _LL = ctypes.c_void_p, ctypes.c_int, ctypes.c_longlong


def lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            subprocess.run(["make", "-C", str(HERE)], check=True, capture_output=True)
        L = ctypes.CDLL(str(LIB_PATH))
        L.ckp_set_threads.argtypes = [_I]
        L.ckp_has_avx512.argtypes = []
        L.ckp_gather_qmm.argtypes = [_P, _I, _I, _P, _P, _P, _I, _I, _I, _P, _P]
        L.ckp_q4_0_to_affine.argtypes = [_P, _LL, _I, _P, _P, _P]
        L.ckp_q4_k_to_affine.argtypes = [_P, _LL, _I, _P, _P, _P]
        L.ckp_moe_layer.argtypes = [_P, _I, _I, _P, _I, _I, _I, _I] + [_P] * 9 + [_P, _P]
        _LIB = L
    return _LIB


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def usable_cores():
    """Host cores this process may run on (the GPU box gives a share of its cores)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(n, cap) if cap > 0 else n)


def cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


class Affine:
    """One expert matrix set in the affine 4-bit layout cpu_kern reads: w uint8 [E, N, K / 2], sc / bi f32
    [E, N, K / 32] (group size 32), converted losslessly from GGUF Q4_0 or Q4_K blocks [E, N, row bytes]."""

    def __init__(self, blocks, t, K):
        blocks = np.ascontiguousarray(blocks, np.uint8)
        E, N = blocks.shape[0], blocks.shape[1]
        self.E, self.N, self.K = E, N, K
        self.w = np.empty((E, N, K // 2), np.uint8)
        self.sc = np.empty((E, N, K // 32), np.float32)
        self.bi = np.empty((E, N, K // 32), np.float32)
        fn = lib().ckp_q4_0_to_affine if t == "Q4_0" else lib().ckp_q4_k_to_affine
        if fn(_p(blocks), E * N, K, _p(self.w), _p(self.sc), _p(self.bi)) != 0:
            raise ValueError(f"{t}: row length {K} does not convert")


def gather_qmm(x, A, idx):
    """y[r] = x[r] . W[idx[r]]^T over the affine experts A, f32 (idx >= E gives zero rows)."""
    x = np.ascontiguousarray(x, np.float32)
    idx = np.ascontiguousarray(idx, np.uint32)
    y = np.empty((x.shape[0], A.N), np.float32)
    lib().ckp_gather_qmm(_p(x), x.shape[0], A.K, _p(A.w), _p(A.sc), _p(A.bi), A.E, A.N, 32, _p(idx), _p(y))
    return y


def moe_layer(x, wr_f16, k, norm, G, U, D, residual=None):
    """One MoE layer on the CPU end to end (router, top-k, gate/up, SwiGLU, down, combine, residual)."""
    x = np.ascontiguousarray(x, np.float32)
    T, H = x.shape
    wr = np.ascontiguousarray(wr_f16, np.float16).view(np.uint16)
    out = np.empty((T, H), np.float32)
    res = np.ascontiguousarray(residual, np.float32) if residual is not None else None
    lib().ckp_moe_layer(_p(x), T, H, _p(wr), G.E, k, int(norm), G.N, _p(G.w), _p(G.sc), _p(G.bi), _p(U.w), _p(U.sc),
                        _p(U.bi), _p(D.w), _p(D.sc), _p(D.bi), _p(res), _p(out))
    return out
