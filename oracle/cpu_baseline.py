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
    """Logical cores this process may run on (the GPU box gives a share of its cores)."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    cap = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return max(1, min(n, cap) if cap > 0 else n)


def _cpuinfo():
    """/proc/cpuinfo as a list of {field: value} dicts, one a logical core (empty when unreadable)."""
    cores, cur = [], {}
    try:
        for ln in open("/proc/cpuinfo"):
            if not ln.strip():
                if cur:
                    cores.append(cur)
                cur = {}
                continue
            if ":" in ln:
                k, v = ln.split(":", 1)
                cur[k.strip()] = v.strip()
    except OSError:
        return []
    if cur:
        cores.append(cur)
    return cores


def host():
    """The host as the CPU baseline reports it: model, sockets, physical cores (distinct (physical id, core id)
    pairs), physical cores a socket (the "cpu cores" field), logical cores, the cores this process may use, and the
    ISA path the restated kernel takes."""
    info = _cpuinfo()
    model = info[0].get("model name", "unknown") if info else "unknown"
    sockets = len({c.get("physical id", "0") for c in info}) or 1
    physical = len({(c.get("physical id", "0"), c.get("core id", str(i))) for i, c in enumerate(info)}) or 1
    per_socket = int(info[0].get("cpu cores", physical)) if info else physical
    return {"model": model, "sockets": sockets, "physical_cores": physical, "cores_per_socket": per_socket,
            "logical_cores": os.cpu_count() or len(info) or 1, "usable_logical_cores": usable_cores(),
            "isa": "AVX-512 F/BW f32 FMA (group size 32 takes the f32 path)" if lib().ckp_has_avx512()
                   else "scalar f32"}


def threads():
    """Threads the baseline runs, by the reference's rule (cpu_kernels.py:14-22, 91): MOE_CPU_THREADS when set,
    else physical_cores(), which reads /proc/cpuinfo's "cpu cores" (the cores of one socket); capped at the cores
    this process may run on."""
    want = int(os.environ.get("MOE_CPU_THREADS", "0") or 0) or host()["cores_per_socket"]
    return max(1, min(want, usable_cores()))


def cpu_model():
    return host()["model"]


def synthetic(E, N, K, seed=0):
    """An Affine-shaped expert set of E experts [N, K] with fixed pseudo-random nibbles and small scales, for timing
    shapes whose experts are not on the host (the kernel's time does not depend on the values)."""
    a = Affine.__new__(Affine)
    a.E, a.N, a.K = E, N, K
    rng = np.random.default_rng(seed)
    a.w = np.empty((E, N, K // 2), np.uint8)
    a.w.reshape(-1, K // 2)[:] = rng.integers(0, 256, K // 2, dtype=np.uint8)
    a.sc = np.empty((E, N, K // 32), np.float32)
    a.sc.reshape(-1).fill(1e-3)
    a.bi = np.empty((E, N, K // 32), np.float32)
    a.bi.reshape(-1).fill(-8e-3)
    return a


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
