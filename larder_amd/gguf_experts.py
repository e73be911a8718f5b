"""Routed experts in llama.cpp's GGUF block formats (Q4_0, Q4_K, Q4_1, Q8_0, Q5_K, Q6_K) on MI355X: the call
surface of the reference's gguf_experts module (gguf_experts.py:573-819) over torch tensors, backed by
liblarder_moe.so.

    experts(x, bufs, rhs, types, host=None)    gguf_experts.py:803-819
    gemv(x, w, slots, topk, types, out_dtype)  gguf_experts.py:600-607  (the decode chain)
    dense(x, w, host, types, out_dtype)        gguf_experts.py:698-722  (the grouped path)
    dequant(buf, slots, t, dtype), dims(buf, t) gguf_experts.py:573-586
    calibrate(hid, inter, types), dense_pays(u, p) gguf_experts.py:771-800

Argument meanings are the reference's: expert buffers are uint8 [S, rows, row bytes] (arena slots), slots are
expert ids (uint32 / int32 / int64 tensors), types are ggml type names ("Q4_0/Q4_0/Q4_0" or a tuple), outputs
come back unweighted in the requested dtype. Unsupported types raise ValueError.
"""
import hashlib
import json
import os
import time
from pathlib import Path

import torch

from . import _lib
from ._lib import TYPES, call, dcode, ptr, qcode, stream

__all__ = ["TYPES", "dims", "dequant", "gemv", "dense", "experts", "calibrate", "dense_pays", "CALIB_DIR"]


def _types(types):
    if isinstance(types, str):
        types = tuple(types.split("/"))
    types = tuple(types)
    if len(types) != 3:
        raise ValueError(f"three ggml types (gate, up, down) expected, got {types}")
    for t in types:
        qcode(t)
    return types


def dims(buf, t):
    """(rows, row length) of an expert buffer [S, rows, row bytes] in ggml type t (gguf_experts.py:573-576)."""
    _, be, bb = TYPES[t] if t in TYPES else (None, None, None)
    if be is None:
        qcode(t)
    return buf.shape[1], buf.shape[2] // bb * be


def _slots_u32(slots):
    s = slots.reshape(-1)
    if s.dtype != torch.int32:
        s = s.to(torch.int32)
    return s.contiguous()


def dequant(buf, slots, t, dtype):
    """Q [len(slots), rows, row length] in dtype of the experts at ``slots`` of buf [S, rows, row bytes]
    (gguf_experts.py:579-586)."""
    rows, cols = dims(buf, t)
    s = _slots_u32(slots)
    q = torch.empty((s.numel(), rows, cols), dtype=dtype, device=buf.device)
    call("lmoe_dequant", ptr(buf), qcode(t), buf.shape[0], rows, cols, ptr(s), s.numel(), ptr(q), dcode(dtype),
         stream())
    return q


def _chain(x, w, slots, topk, types, out_dtype):
    """gemv() through the decode chain: (h float32 [n, I], y [n, H] in out_dtype)."""
    bg, bu, bd = w
    tg, tu, td = types
    inter, hid = dims(bg, tg)
    s = _slots_u32(slots)
    n = s.numel()
    x = x.contiguous()
    h = torch.empty((n, inter), dtype=torch.float32, device=x.device)
    y = torch.empty((n, hid), dtype=out_dtype, device=x.device)
    call("lmoe_gemv_gate_up", ptr(x), dcode(x.dtype), ptr(s), n, topk, ptr(bg), ptr(bu), qcode(tg), qcode(tu),
         bg.shape[0], hid, inter, ptr(h), stream())
    call("lmoe_gemv_down_combine", ptr(h), ptr(s), None, n, 1, ptr(bd), qcode(td), bd.shape[0], inter, hid, None,
         None, 0, None, 0, ptr(y), dcode(out_dtype), stream())
    return h, y


def gemv(x, w, slots, topk, types, out_dtype):
    """Every slot's expert output, unweighted: x (rows, hidden), slots (rows * topk,) with slot s on row s // topk,
    w the gate, up and down buffers [S, rows, row bytes] in ``types``; returns (rows * topk, hidden) in out_dtype
    (gguf_experts.py:600-607)."""
    return _chain(x, w, slots, topk, _types(types), out_dtype)[1]


def dense(x, w, host, types, out_dtype):
    """Every row's expert output, unweighted, one slot a row (``host``: the slots, any order), through the device
    grouping and the grouped MFMA GEMMs (gguf_experts.py:698-722)."""
    from . import grouped
    types = _types(types)
    host = torch.as_tensor(host).reshape(-1).to(device=x.device, dtype=torch.int32)
    return grouped.expert_rows(x.contiguous(), w, host, types, out_dtype)


# Per-device costs of the two paths as calibrate() measures them: chain fixed s, chain s a row, dense fixed s,
# dense s an expert, dense s a row (gguf_experts.py:725-729); until then every pass takes the decode chain.
_COST = None
CALIB_DIR = Path(os.environ.get("LMOE_CACHE", Path.home() / ".cache" / "larder-amd"))


def _measure(hid, inter, types):
    """The cost model's five terms, timed on random Q4 experts at these shapes (best of 5), fitted by least
    squares: the chain over three row counts and the dense path over five (experts, rows) points
    (gguf_experts.py:731-768)."""
    dev = torch.device("cuda")
    E = 32
    g = torch.Generator(device=dev).manual_seed(0)
    w = tuple(_random_q4(E, r, c, t, g) for (r, c), t in zip(((inter, hid), (inter, hid), (hid, inter)), types))
    x = torch.randn((80 * E, hid), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)

    def secs(u, p, dense_path):
        host = (torch.arange(p, device=dev) % u).to(torch.int32)
        f = (lambda: dense(x[:p], w, host, types, x.dtype)) if dense_path else \
            (lambda: _chain(x[:p], w, host, 1, types, x.dtype)[1])
        f()
        torch.cuda.synchronize()
        best = float("inf")
        for _ in range(5):
            t0 = time.perf_counter()
            f()
            torch.cuda.synchronize()
            best = min(best, time.perf_counter() - t0)
        return best

    def fit(rows, ts):
        a = torch.tensor(rows, dtype=torch.float64)
        b = torch.tensor(ts, dtype=torch.float64).reshape(-1, 1)
        return torch.linalg.lstsq(a, b).solution.reshape(-1).tolist()

    chain = [(p, secs(E, p, False)) for p in (10, 10 * E, 80 * E)]
    cg = fit([[1.0, p] for p, _ in chain], [t for _, t in chain])
    pts = [(u, p, secs(u, p, True)) for u, p in ((1, 10), (10, 100), (10, 800), (E, 10 * E), (E, 80 * E))]
    cd = fit([[1.0, u, p] for u, p, _ in pts], [t for *_, t in pts])
    return [max(float(v), 0.0) for v in (*cg, *cd)]


# byte offsets of each block type's f16 scale fields
_SCALE_AT = {"Q4_0": (0,), "Q4_K": (0, 2), "Q4_1": (0, 2), "Q8_0": (0,), "Q5_K": (0, 2), "Q6_K": (208,)}


def _random_q4(n, rows, cols, t, gen):
    """n random experts [n, rows, row bytes] of type t with finite scales, made on the device (Q4_0 through the
    device quantizer, the other types as random blocks with small f16 scales)."""
    if t == "Q4_0":
        wf = torch.randn((n * rows, cols), generator=gen, device="cuda", dtype=torch.float32) * 0.02
        out = torch.empty((n, rows, _lib.row_bytes(t, cols)), dtype=torch.uint8, device="cuda")
        call("lmoe_quantize_q4_0", ptr(wf), _lib.F32, n * rows, cols, ptr(out), stream())
        return out
    _, be, bb = TYPES[t]
    nb = cols // be
    b = torch.randint(0, 256, (n, rows, nb, bb), generator=gen, device="cuda", dtype=torch.uint8)
    for at in _SCALE_AT[t]:
        d = (torch.rand((n, rows, nb, 1), generator=gen, device="cuda") * 1e-3).to(torch.float16)
        b[..., at:at + 2] = d.view(torch.uint8).reshape(n, rows, nb, 2)
    return b.reshape(n, rows, -1).contiguous()


def _source_hash():
    h = hashlib.sha1()
    for p in sorted((Path(__file__).parent / "csrc").glob("*")):
        h.update(p.read_bytes())
    return h.hexdigest()


def calibrate(hid, inter, types):
    """This device's cost model at these shapes and types, measured once (a few seconds) and cached on disk
    keyed by the GPU architecture, the HIP runtime version, the kernels' source hash and the shapes
    (gguf_experts.py:771-794)."""
    global _COST
    types = _types(types)
    props = torch.cuda.get_device_properties(0)
    key = json.dumps([getattr(props, "gcnArchName", props.name), torch.version.hip, _source_hash(), hid, inter,
                      list(types)])
    path = CALIB_DIR / f"gguf-{hashlib.sha1(key.encode()).hexdigest()[:16]}.json"
    try:
        _COST = json.loads(path.read_text())["cost"]
    except (OSError, ValueError, KeyError):
        _COST = _measure(hid, inter, types)
        try:
            path.parent.mkdir(parents=True, exist_ok=True)
            tmp = path.with_suffix(".tmp")
            tmp.write_text(json.dumps({"cost": _COST}))
            tmp.replace(path)
        except OSError as e:
            print(f"  gguf: could not save the prefill switch to {path}: {e}", flush=True)
    return _COST


def dense_pays(u, p):
    """Whether dense() beats gemv() on p rows of u experts, by this device's cost model (gguf_experts.py:797-800)."""
    c = _COST
    return c is not None and c[2] + c[3] * u + c[4] * p < c[0] + c[1] * p


def experts(x, bufs, rhs, types, host=None):
    """The routed experts' outputs, x (..., 1, hidden) broadcast against rhs (...) slot ids, bufs the
    (gguf part, [pad part]) buffers of gate, up and down, types their ggml types; returns rhs.shape + (1, hidden)
    in x's dtype. With ``host`` (the slots, one row of x a slot) dense_pays() may pick the grouped path
    (gguf_experts.py:803-819)."""
    types = _types(types)
    hid = x.shape[-1]
    x2 = x.reshape(-1, hid)
    w = tuple(b[0] for b in bufs)
    if host is not None:
        host = torch.as_tensor(host).reshape(-1)
        if not (host.numel() == x2.shape[0] == rhs.numel()):
            raise ValueError("dense: one row of x per slot")
        if dense_pays(int(torch.unique(host).numel()), host.numel()):
            return dense(x2, w, host, types, x.dtype).reshape(tuple(rhs.shape) + (1, hid))
    y = gemv(x2, w, rhs.reshape(-1), rhs.numel() // x2.shape[0], types, x.dtype)
    return y.reshape(tuple(rhs.shape) + (1, hid))
