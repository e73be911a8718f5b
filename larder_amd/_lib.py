"""ctypes binding of liblarder_moe.so (include/larder_moe.h) and torch-tensor helpers.

The library is built in-tree by ``python3 -m larder_amd.build`` (or ``__graft_entry__.build()``). Loading fails
loudly when it is missing: there is no CPU or eager fallback anywhere in this package. Errors follow the
reference's native C-ABI convention (native/moe_pipe_cuda.py:95-97): every call returns an int and the reason is
read from ``lmoe_error()``; a refused ggml type raises ValueError (the reference's load-time refusal,
stream_fast.py:8058-8061), any other refusal or HIP failure raises RuntimeError.
"""
import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "liblarder_moe.so"

F32, F16, BF16 = 0, 1, 2
Q4_0, Q4_K = 2, 12
EINVAL, ETYPE, ESHAPE, EALIGN, EWORKSPACE = -1, -2, -3, -4, -5
ABI_VERSION = 1

DTYPE_CODE = {torch.float32: F32, torch.float16: F16, torch.bfloat16: BF16}
# ggml type name -> (ggml type id, weights a block, bytes a block) (gguf_ref.py:8-15)
TYPES = {"Q4_0": (2, 32, 18), "Q4_K": (12, 256, 144), "Q4_1": (3, 32, 20), "Q8_0": (8, 32, 34),
         "Q5_K": (13, 256, 176), "Q6_K": (14, 256, 210)}
# the two types every kernel (prepared rows, fused top-k, nibble-decoding grouped GEMMs) takes; the others run on
# the general decode chain and on the grouped path over f16-dequantized experts
Q4_TYPES = ("Q4_0", "Q4_K")

_P, _I, _SZ, _LL, _F = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_longlong, ctypes.c_float
# name -> (restype, argtypes): every symbol include/larder_moe.h declares
SIGNATURES = {
    "lmoe_error": (ctypes.c_char_p, []),
    "lmoe_abi_version": (_I, []),
    "lmoe_profile_arm": (_I, [_I]),
    "lmoe_profile_read": (_I, [_P, _I, _P]),
    "lmoe_timeline_arm": (_I, [_P, _LL]),
    "lmoe_timeline_disarm": (_I, [_P]),
    "lmoe_timeline_launch": (_I, [_I, _P, _P, _P]),
    "lmoe_timeline_clock_khz": (_I, [_P]),
    "lmoe_router_topk": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "lmoe_router_topk_shared": (_I, [_P, _I, _I, _I, _I, _P, _I, _P, _P, _P]),
    "lmoe_prep_x": (_I, [_P, _I, _I, _I, _I, _P, _P]),
    "lmoe_router_gemv": (_I, [_P, _I, _P, _P, _I, _I, _I, _I, _P, _P, _I, _P]),
    "lmoe_router_gemv_topk": (_I, [_P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P]),
    "lmoe_router_gemv_rank": (_I, [_P, _I, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _I, _P, _P]),
    "lmoe_route_bias": (_I, [_P, _I, _I, _I, _I, _P, _P, _I, _F, _F, _I, _I, _P, _P, _P, _P, _P]),
    "lmoe_gemv_gate_up": (_I, [_P, _I, _P, _I, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "lmoe_gemv_gate_up_prepped": (_I, [_P, _P, _P, _I, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P, _I, _P]),
    "lmoe_moe_gate_up": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _P]),
    "lmoe_moe_gate_up_ext": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _I, _P]),
    "lmoe_moe_gate_up_h": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _I, _P]),
    "lmoe_gemv_down_combine": (_I, [_P, _P, _P, _I, _I, _P, _I, _I, _I, _I, _P, _P, _I, _P, _I, _P, _I, _P]),
    "lmoe_gemv_down_combine_prepped": (_I, [_P, _I, _P, _P, _I, _I, _P, _I, _I, _I, _I, _P, _P, _I, _P, _I, _P, _I,
                                            _P]),
    "lmoe_topk_and_gemm_f16": (_I, [_P, _I, _I, _I, _I, _I, _P, _P, _P, _I, _LL, _P, _P]),
    "lmoe_gemv_gate_up_runs": (_I, [_P, _I, _P, _I, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "lmoe_gemv_down_runs": (_I, [_P, _P, _I, _I, _P, _I, _I, _I, _I, _P, _I, _P]),
    "lmoe_gemv_chain_gate_up": (_I, [_P, _I, _P, _I, _I, _P, _P, _I, _I, _I, _I, _P, _P, _I, _P]),
    "lmoe_gemv_chain_down": (_I, [_P, _P, _I, _P, _I, _I, _I, _I, _P, _I, _P]),
    "lmoe_gemv_gate_up_runs_prepped": (_I, [_P, _P, _I, _I, _P, _P, _I, _I, _I, _I, _P, _P, _I, _P]),
    "lmoe_gemv_down_runs_prepped": (_I, [_P, _P, _I, _I, _P, _I, _I, _I, _I, _P, _I, _P]),
    "lmoe_group_workspace_bytes": (_SZ, [_I, _I]),
    "lmoe_group_rows": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P]),
    "lmoe_group_rows_noalloc": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P]),
    "lmoe_max_tiles": (_I, [_I, _I, _I]),
    "lmoe_grouped_tile_rows": (_I, []),
    "lmoe_grouped_pick_tile_rows": (_I, [_I, _I, _I, _I, _I]),
    "lmoe_grouped_pick_ksplit": (_I, [_I, _I, _I, _I]),
    "lmoe_grouped_workspace_bytes": (_SZ, [_I, _I, _I, _I, _I]),
    "lmoe_to_f16": (_I, [_P, _I, _LL, _P, _P]),
    "lmoe_to_gemm_f16": (_I, [_P, _I, _LL, _P, _P]),
    "lmoe_router_gemm_ksplit": (_I, [_I, _I, _I]),
    "lmoe_router_gemm_workspace_bytes": (_SZ, [_I, _I, _I]),
    "lmoe_router_gemm": (_I, [_P, _I, _I, _P, _I, _I, _P, _P, _P, _P]),
    "lmoe_router_gemm_topk": (_I, [_P, _I, _I, _P, _I, _I, _P, _P, _P, _I, _I, _I, _P, _P, _P]),
    "lmoe_router_norms": (_I, [_P, _P, _I, _I, _I, _P, _P]),
    "lmoe_router_refine": (_I, [_P, _I, _I, _P, _I, _I, _I, _P, _P, _I, _I, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P]),
    "lmoe_router_gemm_refine": (_I, [_P, _I, _I, _P, _I, _I, _P, _P, _I, _P, _P, _I, _P, _I, _I, _I, _P, _P, _P, _P,
                                     _P, _P]),
    "lmoe_grouped_gate_up": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I, _P, _P]),
    "lmoe_grouped_down": (_I, [_P, _P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _I, _P]),
    "lmoe_grouped_gate_up_bm": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _I, _I, _I, _I, _I, _P,
                                     _P]),
    "lmoe_grouped_down_bm": (_I, [_P, _I, _P, _P, _P, _I, _I, _I, _P, _P, _I, _I, _I, _I, _P, _I, _P]),
    "lmoe_grouped_gate_up_sl": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _I, _I, _I, _I, _I, _P,
                                     _P]),
    "lmoe_grouped_down_sl": (_I, [_P, _I, _P, _P, _P, _I, _I, _I, _P, _P, _I, _I, _I, _I, _P, _I, _P]),
    "lmoe_stream_bytes": (_SZ, [_I, _I, _I, _I]),
    "lmoe_stream_repack": (_I, [_P, _I, _I, _I, _I, _P, _P]),
    "lmoe_combine_sorted": (_I, [_P, _I, _P, _P, _I, _I, _I, _P, _P, _I, _P, _I, _P, _I, _P]),
    "lmoe_dequant": (_I, [_P, _I, _I, _I, _I, _P, _I, _P, _I, _P]),
    "lmoe_dequant_gemm_f16": (_I, [_P, _I, _I, _I, _I, _P, _P]),
    "lmoe_qmv_rows": (_I, [_P, _I, _P, _P, _P, _I, _I, _I, _P, _P]),
    "lmoe_swiglu_bf16": (_I, [_P, _P, _LL, _P, _P]),
    "lmoe_grouped_gate_up_f16w": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _I, _I, _P, _P, _I, _I, _I, _P, _P]),
    "lmoe_grouped_down_f16w": (_I, [_P, _P, _P, _P, _I, _I, _P, _I, _I, _I, _P, _I, _P]),
    "lmoe_quantize_q4_0": (_I, [_P, _I, _LL, _I, _P, _P]),
    "lmoe_quantize_q4_k": (_I, [_P, _I, _LL, _I, _P, _P]),
}

_LIB = None


def lib():
    """The loaded library (loaded once); raises RuntimeError when it is not built."""
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"{LIB_PATH} is not built: run `python3 -m larder_amd.build` (hipcc, gfx950)")
        L = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        if L.lmoe_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH}: ABI {L.lmoe_abi_version()} but this package speaks {ABI_VERSION}")
        _LIB = L
    return _LIB


def call(name, *args):
    """Call an entry point; raise on a nonzero return with the library's reason."""
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        why = lib().lmoe_error().decode()
        if rc == ETYPE:
            raise ValueError(why)
        raise RuntimeError(f"{name} returned {rc}: {why}")
    return rc


def ptr(t):
    """Device pointer of a CUDA tensor (None -> NULL)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise ValueError("larder_amd: tensors must live on the GPU")
    if not t.is_contiguous():
        raise ValueError("larder_amd: tensors must be contiguous")
    return ctypes.c_void_p(t.data_ptr())


def dcode(dtype):
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"larder_amd: dtype {dtype} is not float32, float16 or bfloat16") from None


def qcode(t):
    """ggml type name -> ggml type id; ValueError for any type this path does not implement."""
    if t not in TYPES:
        raise ValueError(f"larder_amd: ggml type {t} is not supported ({', '.join(TYPES)} are)")
    return TYPES[t][0]


# device index -> True once the known-answer self-check (larder_amd.selfcheck) passed there; False while it runs
_CHECKED = {}


def stream():
    """The current torch stream as a hipStream_t, for a call that launches work. The first such call on a device
    first runs the library's known-answer self-check there (and raises if it fails), unless LMOE_SELF_CHECK=0 or a
    graph is being captured (then the next eager call checks)."""
    dev = torch.cuda.current_device()
    if dev not in _CHECKED:
        _self_check(dev)
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _self_check(dev):
    if os.environ.get("LMOE_SELF_CHECK", "1") == "0" or torch.cuda.is_current_stream_capturing():
        return
    _CHECKED[dev] = False  # the check's own calls pass through
    try:
        from . import selfcheck
        selfcheck.run(dev)
    except BaseException:
        del _CHECKED[dev]
        raise
    _CHECKED[dev] = True


def row_bytes(t, n):
    _, be, bb = TYPES[t]
    if n % be:
        raise ValueError(f"{t}: a row of {n} weights is not a whole number of {be}-weight blocks")
    return n // be * bb
