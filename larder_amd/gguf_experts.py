"""Routed experts in llama.cpp's GGUF block formats (Q4_0, Q4_K, Q4_1, Q8_0, Q5_K, Q6_K) on MI355X: the call
surface of the reference's gguf_experts module (gguf_experts.py:573-819) over torch tensors, backed by
liblarder_moe.so.

    experts(x, bufs, rhs, types, host=None)    gguf_experts.py:803-819
    gemv(x, w, slots, topk, types, out_dtype)  gguf_experts.py:600-607  (the decode chain, or the run kernels)
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
import tempfile
from pathlib import Path

import numpy as np
import torch

from . import _lib
from ._lib import TYPES, call, dcode, ptr, qcode, stream

__all__ = ["TYPES", "dims", "dequant", "gemv", "dense", "experts", "calibrate", "dense_pays", "calib_dir", "runs_on",
           "run_rows"]


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


def fast_form(hid, inter, types):
    """Whether gemv() at these shapes and types runs the register-resident kernels (lmoe_gemv_chain_gate_up: x
    prepared inside the launch, h kept as f16 prepared rows; lmoe_gemv_chain_down). They take one Q4 type for gate and
    up, a Q4 down, hidden 2048 or 4096 and a width that is a multiple of 128 up to 8192; everything else runs the
    raw-activation kernels with fp32 h between them."""
    tg, tu, td = types
    return (tg == tu and tg in _lib.Q4_TYPES and td in _lib.Q4_TYPES and hid in (2048, 4096)
            and inter % 128 == 0 and inter // 64 <= 128)


def _prepared(x, t):
    """x's rows as prepared units for block type t (lmoe_prep_x): int32 [rows, hidden / 64 * 36]."""
    rows, hid = x.shape
    xp = torch.empty((rows, hid // 64 * 36), dtype=torch.int32, device=x.device)
    call("lmoe_prep_x", ptr(x), dcode(x.dtype), rows, hid, qcode(t), ptr(xp), stream())
    return xp


def _chain(x, w, slots, topk, types, out_dtype, want_h=True):
    """gemv() through the decode chain, a workgroup row a slot: (h float32 [n, I] or None when not wanted,
    y [n, H] in out_dtype) (gguf_experts.py:610-629)."""
    bg, bu, bd = w
    tg, tu, td = types
    inter, hid = dims(bg, tg)
    s = _slots_u32(slots)
    n = s.numel()
    x = x.contiguous()
    h = torch.empty((n, inter), dtype=torch.float32, device=x.device) if want_h or not fast_form(hid, inter, types) \
        else None
    y = torch.empty((n, hid), dtype=out_dtype, device=x.device)
    if fast_form(hid, inter, types):
        hp = torch.empty((n, inter // 64 * 36), dtype=torch.int32, device=x.device)
        call("lmoe_gemv_chain_gate_up", ptr(x), dcode(x.dtype), ptr(s), n, topk, ptr(bg), ptr(bu), qcode(tg),
             bg.shape[0], hid, inter, ptr(h), ptr(hp), qcode(td), stream())
        call("lmoe_gemv_chain_down", ptr(hp), ptr(s), n, ptr(bd), qcode(td), bd.shape[0], inter, hid, ptr(y),
             dcode(out_dtype), stream())
        return h, y
    call("lmoe_gemv_gate_up", ptr(x), dcode(x.dtype), ptr(s), n, topk, ptr(bg), ptr(bu), qcode(tg), qcode(tu),
         bg.shape[0], hid, inter, ptr(h), stream())
    call("lmoe_gemv_down_combine", ptr(h), ptr(s), None, n, 1, ptr(bd), qcode(td), bd.shape[0], inter, hid, None,
         None, 0, None, 0, ptr(y), dcode(out_dtype), stream())
    return h, y


def runs_on():
    """LMOE_GGUF_RUNS, read on every call (the reference's MOE_GGUF_RUNS, gguf_experts.py:590-596): on unless "0".
    When on, gemv() on rows of one slot each goes through the run kernels, once _runs_ok() has found them bit-equal
    to the chain at that shape."""
    return os.environ.get("LMOE_GGUF_RUNS", "1") != "0"


def run_rows():
    """LMOE_GGUF_RUN_ROWS: rows a window of the run kernels (the reference's MOE_GGUF_RUN_TILE window, default 4, the
    fastest measured on sorted and unsorted rows; the library lowers it to fit LDS). No bit depends on it."""
    return max(1, int(os.environ.get("LMOE_GGUF_RUN_ROWS", "4")))


def _gemv_runs(x, w, slots, types, out_dtype, want_h=True):
    """gemv() on rows of one slot each (best sorted by slot) through the run kernels: a window of rows reads a weight
    row once a run of equal slots; returns (h float32 [n, I] or None, y [n, H] in out_dtype), the kernels matching
    the chain's form at these shapes (gguf_experts.py:632-658)."""
    bg, bu, bd = w
    tg, tu, td = types
    inter, hid = dims(bg, tg)
    s = _slots_u32(slots)
    n = s.numel()
    x = x.contiguous()
    fast = fast_form(hid, inter, types)
    h = torch.empty((n, inter), dtype=torch.float32, device=x.device) if want_h or not fast else None
    y = torch.empty((n, hid), dtype=out_dtype, device=x.device)
    tr = run_rows()
    if fast:
        xp = _prepared(x, tg)
        hp = torch.empty((n, inter // 64 * 36), dtype=torch.int32, device=x.device)
        call("lmoe_gemv_gate_up_runs_prepped", ptr(xp), ptr(s), n, tr, ptr(bg), ptr(bu), qcode(tg), bg.shape[0], hid,
             inter, ptr(h), ptr(hp), qcode(td), stream())
        call("lmoe_gemv_down_runs_prepped", ptr(hp), ptr(s), n, tr, ptr(bd), qcode(td), bd.shape[0], inter, hid,
             ptr(y), dcode(out_dtype), stream())
        return h, y
    call("lmoe_gemv_gate_up_runs", ptr(x), dcode(x.dtype), ptr(s), n, tr, ptr(bg), ptr(bu), qcode(tg), qcode(tu),
         bg.shape[0], hid, inter, ptr(h), stream())
    call("lmoe_gemv_down_runs", ptr(h), ptr(s), n, tr, ptr(bd), qcode(td), bd.shape[0], inter, hid, ptr(y),
         dcode(out_dtype), stream())
    return h, y


def _bits(t):
    """t's raw bits as an integer tensor of its element size (so -0 / +0 and NaN payloads compare as bits)."""
    return t.contiguous().view({4: torch.int32, 2: torch.int16}[t.element_size()])


def _identical(a, b):
    return a.dtype == b.dtype and a.shape == b.shape and bool(torch.equal(_bits(a), _bits(b)))


# (hid, inter, types, x dtype, out dtype) -> whether the run kernels stand in for the chain there. An entry is
# written False before its check runs, so anything gemv() is asked during the check takes the chain.
_RUNS_OK = {}


def _run_check_case(hid, inter, types, x_dtype):
    """The check's input: six random experts of these types, 16 runs of distinct lengths 1..16 (120 rows) over
    slots 0..6 (slot 6 is past the experts: zero rows), and x random in x_dtype; seeded by the shape."""
    g = torch.Generator(device="cuda").manual_seed(7 * hid + inter)
    shapes = ((inter, hid), (inter, hid), (hid, inter))
    w = tuple(_random_q4(6, r, c, t, g) for (r, c), t in zip(shapes, types))
    run_len = torch.randperm(16, generator=g, device="cuda") + 1
    run_id = torch.randint(0, 7, (16,), generator=g, device="cuda")
    slots = torch.repeat_interleave(run_id.cpu(), run_len.cpu()).to(device="cuda", dtype=torch.int32)
    x = torch.randn((slots.numel(), hid), generator=g, device="cuda").to(x_dtype)
    return x, w, slots


def _check_runs(hid, inter, types, x_dtype, out_dtype):
    """(verdict, reason): the run kernels against the chain on _run_check_case, both outputs bit for bit."""
    if not all(t in _lib.Q4_TYPES for t in types):
        return False, f"no run kernels for {'/'.join(types)} (Q4_0 and Q4_K only)"
    try:
        x, w, slots = _run_check_case(hid, inter, types, x_dtype)
        chain = _chain(x, w, slots, 1, types, out_dtype)
        runs = _gemv_runs(x, w, slots, types, out_dtype)
    except (RuntimeError, ValueError) as e:  # refused at this shape
        return False, f"refused: {type(e).__name__}: {str(e)[:200]}"
    for name, a, b in zip(("h", "output"), chain, runs):
        if not _identical(a, b):
            return False, f"their {name} is not bit-identical to the chain's"
    return True, "bit-identical to the chain"


def _runs_ok(hid, inter, types, x_dtype, out_dtype):
    """Whether gemv() may take the run kernels at these shapes and dtypes (the reference's _runs_ok contract,
    gguf_experts.py:661-680): decided once a key by _check_runs, logged once, False on any difference or refusal."""
    key = (hid, inter, tuple(types), x_dtype, out_dtype)
    if key not in _RUNS_OK:
        _RUNS_OK[key] = False
        ok, reason = _check_runs(hid, inter, tuple(types), x_dtype, out_dtype)
        _RUNS_OK[key] = ok
        state = "in use" if ok else "not used"
        print(f"larder_amd: run kernels {state} at {hid}x{inter} {'/'.join(types)} "
              f"({str(x_dtype).split('.')[-1]} -> {str(out_dtype).split('.')[-1]}): {reason}", flush=True)
    return _RUNS_OK[key]


def gemv(x, w, slots, topk, types, out_dtype):
    """Every slot's expert output, unweighted: x (rows, hidden), slots (rows * topk,) with slot s on row s // topk,
    w the gate, up and down buffers [S, rows, row bytes] in ``types``; returns (rows * topk, hidden) in out_dtype,
    through the run kernels at one slot a row when runs_on() and they passed their check (gguf_experts.py:600-607)."""
    types = _types(types)
    n = slots.numel()
    if topk == 1 and n > 1 and runs_on():
        inter, hid = dims(w[0], types[0])
        if _runs_ok(hid, inter, types, x.dtype, out_dtype):
            return _gemv_runs(x, w, slots, types, out_dtype, want_h=False)[1]
    return _chain(x, w, slots, topk, types, out_dtype, want_h=False)[1]


def dense(x, w, host, types, out_dtype):
    """Every row's expert output, unweighted, one slot a row (``host``: the slots, any order), through the device
    grouping and the grouped MFMA GEMMs (gguf_experts.py:698-722)."""
    from . import grouped
    types = _types(types)
    host = torch.as_tensor(host).reshape(-1).to(device=x.device, dtype=torch.int32)
    return grouped.expert_rows(x.contiguous(), w, host, types, out_dtype)


# This device's cost model of the two paths, as calibrate() fits it: five non-negative terms (chain fixed, chain per
# row, dense fixed, dense per expert, dense per row), the form the reference's callers rely on (gguf_experts.py:725-800,
# read through dense_pays). None until calibrate() runs: every pass then takes the decode chain.
_COST = None
_CAL_E = 64  # experts in the calibration pool


def calib_dir():
    """Where calibrate() caches its fits: $LMOE_CACHE, else ~/.cache/larder-amd (read on every call)."""
    return Path(os.environ.get("LMOE_CACHE") or (Path.home() / ".cache" / "larder-amd"))


def _sample_points(rows_a_tile):
    """(chain row counts, dense (experts, rows) points) for the fit. The chain's cost grows with its rows (one
    workgroup row a slot): 1 token, a decode batch, and past the crossing. The grouped path's cost has a part per
    m-tile (one at least per expert used) and a part per row: points at one tile, at a dozen experts, at ~2 tiles an
    expert over the whole pool, and two between, so that the expert and row terms are separable."""
    bm = rows_a_tile
    chain = (1, 16, 128, 512)
    dense = ((1, bm), (12, 12 * bm // 4), (12, 24 * bm), (_CAL_E, 2 * _CAL_E * bm), (_CAL_E // 2, 4 * bm),
             (_CAL_E, _CAL_E * bm // 8))
    return chain, dense


def _time_call(fn, batches=3, reps=5):
    """Median over batches of the mean time of ``reps`` calls of fn, in seconds, from events on the current
    stream."""
    fn()
    fn()
    torch.cuda.current_stream().synchronize()
    means = []
    for _ in range(batches):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(reps):
            fn()
        b.record()
        b.synchronize()
        means.append(a.elapsed_time(b) / reps * 1e-3)
    return sorted(means)[len(means) // 2]


def _measure(hid, inter, types):
    """The five cost terms at these shapes, fitted by least squares to timings of both paths on a pool of random
    experts of these types (made on the device)."""
    from . import grouped
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(1234)
    w = tuple(_random_q4(_CAL_E, r, c, t, g) for (r, c), t in zip(((inter, hid), (inter, hid), (hid, inter)), types))
    chain_rows, dense_pts = _sample_points(grouped.pick_tile_rows(4 * _CAL_E, _CAL_E, types))
    most = max(max(chain_rows), max(p for _, p in dense_pts))
    x = torch.randn((most, hid), generator=g, device=dev).to(torch.bfloat16)

    def slots(u, p):  # p rows over u experts, spread evenly
        return (torch.arange(p, device=dev, dtype=torch.int32) * 7919) % u

    t_chain = [_time_call(lambda p=p: _chain(x[:p], w, slots(_CAL_E, p), 1, types, x.dtype)) for p in chain_rows]
    t_dense = [_time_call(lambda u=u, p=p: dense(x[:p], w, slots(u, p), types, x.dtype)) for u, p in dense_pts]
    a_chain = np.array([[1.0, p] for p in chain_rows])
    a_dense = np.array([[1.0, u, p] for u, p in dense_pts], dtype=np.float64)
    fit_chain = np.linalg.lstsq(a_chain, np.array(t_chain), rcond=None)[0]
    fit_dense = np.linalg.lstsq(a_dense, np.array(t_dense), rcond=None)[0]
    return [max(float(v), 0.0) for v in np.concatenate([fit_chain, fit_dense])]


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


def _source_digest():
    h = hashlib.sha256()
    for p in sorted((Path(__file__).parent / "csrc").glob("*")):
        h.update(p.name.encode())
        h.update(p.read_bytes())
    return h.hexdigest()[:20]


def _device_key():
    """What a fit depends on besides the shapes: the GPU, the HIP runtime and the kernels' sources."""
    props = torch.cuda.get_device_properties(torch.cuda.current_device())
    return [getattr(props, "gcnArchName", props.name), props.multi_processor_count, torch.version.hip,
            _source_digest()]


def calibrate(hid, inter, types):
    """This device's cost model at these shapes and types (the reference's calibrate, gguf_experts.py:771-794):
    read from the cache under calib_dir() when a fit for this device, runtime, kernel source and shape is there,
    else measured (a few seconds) and stored. Returns the five terms and makes them the ones dense_pays() uses."""
    global _COST
    types = _types(types)
    ident = json.dumps({"device": _device_key(), "hid": hid, "inter": inter, "types": list(types)}, sort_keys=True)
    path = calib_dir() / f"dense-switch-{hashlib.sha256(ident.encode()).hexdigest()[:24]}.json"
    cost = None
    if path.is_file():
        try:
            got = json.loads(path.read_text())
            if got.get("ident") == ident and len(got.get("cost", ())) == 5:
                cost = [float(v) for v in got["cost"]]
        except (OSError, ValueError):
            cost = None
    if cost is None:
        cost = _measure(hid, inter, types)
        try:
            path.parent.mkdir(parents=True, exist_ok=True)
            fd, tmp = tempfile.mkstemp(dir=path.parent, prefix=path.name, suffix=".part")
            with os.fdopen(fd, "w") as f:
                json.dump({"ident": ident, "cost": cost}, f)
            os.replace(tmp, path)
        except OSError as e:
            print(f"larder_amd: the dense-path fit for {hid}x{inter} {'/'.join(types)} was measured but not cached "
                  f"({e})", flush=True)
    _COST = cost
    if runs_on():  # the run kernels are checked here, at load, not in the middle of the first prompt
        _runs_ok(hid, inter, types, torch.bfloat16, torch.bfloat16)
    return cost


def dense_pays(u, p):
    """Whether dense() beats gemv() on p rows of u experts, by this device's cost model (gguf_experts.py:797-800)."""
    c = _COST
    return c is not None and c[2] + c[3] * u + c[4] * p < c[0] + c[1] * p


def _dense_knob(rule):
    """LMOE_DENSE, read on every call: "1" sends every call with ``host`` to dense(), "0" none, unset (or anything
    else) leaves it to rule() (dense_pays)."""
    v = os.environ.get("LMOE_DENSE", "")
    return True if v == "1" else False if v == "0" else rule()


def experts(x, bufs, rhs, types, host=None):
    """The routed experts' outputs, x (..., 1, hidden) broadcast against rhs (...) slot ids, bufs the
    (gguf part, [pad part]) buffers of gate, up and down, types their ggml types; returns rhs.shape + (1, hidden)
    in x's dtype. With ``host`` (the slots, one row of x a slot) dense_pays() may pick the grouped path, or
    LMOE_DENSE forces the choice (gguf_experts.py:803-819)."""
    types = _types(types)
    hid = x.shape[-1]
    x2 = x.reshape(-1, hid)
    w = tuple(b[0] for b in bufs)
    if host is not None:
        host = torch.as_tensor(host).reshape(-1)
        if not (host.numel() == x2.shape[0] == rhs.numel()):
            raise ValueError("dense: one row of x per slot")
        if _dense_knob(lambda: dense_pays(int(torch.unique(host).numel()), host.numel())):
            return dense(x2, w, host, types, x.dtype).reshape(tuple(rhs.shape) + (1, hid))
    y = gemv(x2, w, rhs.reshape(-1), rhs.numel() // x2.shape[0], types, x.dtype)
    return y.reshape(tuple(rhs.shape) + (1, hid))
