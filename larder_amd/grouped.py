"""The grouped (prefill / batched decode) expert path: device grouping, grouped MFMA GEMMs, weighted combine.

The reference's dense path (gguf_experts.py:698-722) sorts rows by slot on the host (np.argsort / np.unique /
searchsorted), dequantizes DENSE_CHUNK experts at a time to f16 and runs MLX gather_mm twice, syncing between
chunks. Here every step stays on the device with no host round trip:

    lmoe_group_rows        ids -> counts, offsets, order, inv, work list (expert, m-tile), its length
    lmoe_grouped_gate_up   h [R, I] f16 = silu(x . wg) * (x . wu), rows gathered through `order`
    lmoe_grouped_down      y [R, H] = h . wd, grouped order
    lmoe_combine_sorted    out [T, H] = sum_j scores[t, j] y[inv[t k + j]] (+ shared) (+ residual)

`expert_rows` mirrors gguf_experts.dense (one slot a row, unweighted rows in the caller's order); `prefill` is a
whole layer over T tokens from router logits.
"""
import ctypes
import os

import torch

from . import _lib
from ._lib import call, dcode, ptr, qcode, stream


def tile_rows():
    """Rows of one grouped-GEMM m-tile (the grouping's bm)."""
    return _lib.lib().lmoe_grouped_tile_rows()


def pick_tile_rows(R, E, types):
    """The GEMMs' tile rows for R rows over E experts (lmoe_grouped_pick_tile_rows, the measured rule): 32 when
    every projection is Q4_0 and the average expert has fewer than 16 rows (batched decode: few tiles have work,
    each streams its expert's weights, and 32-row tiles keep five K steps in flight and allow split-K; cfg4 116.6 ->
    108.8 us a step); 64 when gate/up runs on dequantized f16 weights (a type beyond Q4_0 / Q4_K, or gate and up of
    two types: the f16-weight GEMM then fits two workgroups a CU, 2,048 x 8 rows 405 -> 377 us) and for Q4_K (the
    direct-copy kernel: cfg5's gate/up 545 -> 387 us); otherwise 128. LMOE_TILE_ROWS (32, 64 or 128, read on every
    call) overrides the rule where the types' GEMMs take that height."""
    return _lib.lib().lmoe_grouped_pick_tile_rows(int(R), int(E), *(qcode(t) for t in types))


def pick_ksplit(R, E, bm, K):
    """Split-K slices for a GEMM over K of R rows in E experts (lmoe_grouped_pick_ksplit): with 32-row tiles and
    fewer than 16 rows an expert on average, few tiles have work and each would walk every K step alone, so each
    tile is split over 4, 3 or 2 workgroups (at least 4 K steps each); otherwise 1. LMOE_KSPLIT (1-8, read on every
    call) overrides the rule on 32-row tiles when it divides the K steps."""
    return _lib.lib().lmoe_grouped_pick_ksplit(int(R), int(E), int(bm), int(K))


def splitk_floats(R, E, bm, H, I):
    """Floats of the split-K workspace that gate_up and down over this grouping need (0 without a split):
    lmoe_grouped_workspace_bytes / 4."""
    return _lib.lib().lmoe_grouped_workspace_bytes(int(R), int(E), int(bm), int(H), int(I)) // 4


class Grouping:
    """Device buffers of one grouping of R rows over E experts (allocated once, reusable for any ids of R rows),
    in m-tiles of bm rows (128 by default; see pick_tile_rows)."""

    def __init__(self, R, E, device="cuda", bm=None):
        self.R, self.E, self.bm = int(R), int(E), int(bm) if bm else tile_rows()
        self.max_tiles = _lib.lib().lmoe_max_tiles(self.R, self.E, self.bm)
        i32 = dict(dtype=torch.int32, device=device)
        self.counts = torch.empty(E, **i32)
        self.offsets = torch.empty(E + 1, **i32)
        self.order = torch.empty(max(R, 1), **i32)
        self.inv = torch.empty(max(R, 1), **i32)
        self.tiles = torch.empty(max(self.max_tiles, 1), **i32)
        self.n_tiles = torch.empty(1, **i32)
        nws = _lib.lib().lmoe_group_workspace_bytes(self.R, self.E)
        self.ws = torch.empty(max(nws // 4, 1), **i32)

    def run(self, ids):
        """Group the flat expert ids [R] (int32 / uint32 on the device); ids >= E go after every expert."""
        if ids.numel() != self.R:
            raise ValueError(f"grouping holds {self.R} rows, got {ids.numel()} ids")
        call("lmoe_group_rows", ptr(ids), self.R, self.E, self.bm, ptr(self.counts), ptr(self.offsets),
             ptr(self.order), ptr(self.inv), ptr(self.tiles), ptr(self.n_tiles), ptr(self.ws), stream())
        return self

    @classmethod
    def identity(cls, R, device="cuda", bm=None):
        """All R rows on expert 0 in their own order (a dense FFN, such as the shared expert, on the same kernels),
        in m-tiles of bm rows (128 by default); built on the host once."""
        g = cls.__new__(cls)
        g.R, g.E, g.bm = int(R), 1, int(bm) if bm else tile_rows()
        nt = -(-g.R // g.bm)
        g.max_tiles = nt
        i32 = dict(dtype=torch.int32)
        g.counts = torch.tensor([g.R], **i32).to(device)
        g.offsets = torch.tensor([0, g.R], **i32).to(device)
        g.order = torch.arange(max(g.R, 1), **i32).to(device)
        g.inv = g.order
        g.tiles = torch.arange(max(nt, 1), **i32).to(device)
        g.n_tiles = torch.tensor([nt], **i32).to(device)
        g.ws = None
        return g


def kperm_index(n, device="cuda"):
    """Position of natural column j (0..n-1) in the grouped GEMMs' K order: within each 32-wide block the columns
    run 0-3, 16-19, 4-7, 20-23, 8-11, 24-27, 12-15, 28-31."""
    j = torch.arange(n, device=device)
    g4 = (j % 32) // 4
    return j - j % 32 + torch.where(g4 < 4, 8 * g4, 8 * (g4 - 4) + 4) + j % 4


def as_gemm_f16(x, out=None):
    """x [rows, K] as float16 in the grouped GEMMs' K order (lmoe_to_gemm_f16), into ``out`` when given."""
    x = x.contiguous()
    if out is None:
        out = torch.empty(x.shape, dtype=torch.float16, device=x.device)
    call("lmoe_to_gemm_f16", ptr(x), dcode(x.dtype), x.numel(), ptr(out), stream())
    return out


def from_kperm(h):
    """h [rows, K] in the grouped GEMMs' K order (as gate_up leaves it) back in natural column order."""
    return h[:, kperm_index(h.shape[1], h.device)]


def gemm_weights(w, t):
    """Every expert of w [E, rows, row bytes] in ggml type t as f16 [E, rows, cols] in the GEMMs' K order
    (lmoe_dequant_gemm_f16): the weight operand of the grouped path for the types beyond Q4_0 / Q4_K."""
    E, rows = w.shape[0], w.shape[1]
    _, be, bb = _lib.TYPES[t]
    cols = w.shape[2] // bb * be
    out = torch.empty((E, rows, cols), dtype=torch.float16, device=w.device)
    call("lmoe_dequant_gemm_f16", ptr(w), qcode(t), E, rows, cols, ptr(out), stream())
    return out


def _ws(n, ws, device):
    if n == 0:
        return None
    if ws is not None and ws.numel() >= n:
        return ws
    return torch.empty(n, dtype=torch.float32, device=device)


def stream_copy(w, t):
    """The stream-layout copy of a Q4_0 / Q4_K expert matrix w uint8 [E, rows, row bytes] (lmoe_stream_repack): the
    same bytes, ordered so that each grouped-GEMM step reads one contiguous run for a block of 128 features instead
    of a 32- or 36-byte piece of every row. rows must be a multiple of 128. For resident layers (MoELayer.keep_stream);
    the decode kernels keep reading the GGUF copy."""
    E, rows = w.shape[0], w.shape[1]
    cols = w.shape[2] // _lib.TYPES[t][2] * _lib.TYPES[t][1]
    if t not in _lib.Q4_TYPES or _lib.lib().lmoe_stream_bytes(qcode(t), E, rows, cols) == 0:
        raise ValueError(f"{t} experts of {rows} x {cols} have no stream layout (Q4_0 / Q4_K, rows a multiple of 128)")
    out = torch.empty_like(w)
    call("lmoe_stream_repack", ptr(w.contiguous()), qcode(t), E, rows, cols, ptr(out), stream())
    return out


def gate_up(x, G, topk, wg, wu, types, h, xh=None, prepped=False, ws=None, ksplit=None, w16=None, sl=None):
    """h [R, I] f16 (grouped order, columns in the GEMMs' K order: from_kperm undoes it) = silu(x . wg) * (x . wu)
    over the grouping G of x's rows (row p reads x[order[p] // topk]); x [T, H] in natural order, any float dtype,
    meets the weights as f16 in the K order (converted into ``xh``; prepped: x already is that form). Q4_0 / Q4_K
    weights are decoded inside the GEMM; the other types are dequantized to f16 first (gemm_weights). ksplit
    (None: pick_ksplit) and ws (the split-K workspace, allocated when not given) drive split-K. sl: (gate, up) in the
    stream layout (stream_copy) to read instead of wg / wu, same results bit for bit."""
    tg, tu = qcode(types[0]), qcode(types[1])
    if not prepped:
        x = as_gemm_f16(x, xh)
    T, H = x.shape
    E, I = wg.shape[0], wg.shape[1]
    if types[0] in _lib.Q4_TYPES and types[1] == types[0]:
        # split-K pays on the GGUF layout only: on stream copies cfg4 took 120.6 us a step without it, 124.1 with
        ks = ksplit or (pick_ksplit(G.R, G.E, G.bm, H) if types[0] == "Q4_0" and sl is None else 1)
        w = _ws(ks * G.R * 2 * I if ks > 1 else 0, ws, x.device)
        entry, (wg_, wu_) = ("lmoe_grouped_gate_up_sl", sl) if sl is not None else ("lmoe_grouped_gate_up_bm", (wg, wu))
        call(entry, ptr(x), _lib.F16, T, topk, ptr(G.order), ptr(G.offsets), ptr(G.tiles), ptr(G.n_tiles),
             G.max_tiles, G.bm, ks, ptr(w), ptr(wg_), ptr(wu_), tg, tu, E, H, I, ptr(h), stream())
    else:
        if G.bm not in (64, tile_rows()):
            raise ValueError(f"the f16-weight GEMMs take 64- or {tile_rows()}-row tiles, not {G.bm}")
        wg16, wu16 = w16 if w16 is not None else (gemm_weights(wg, types[0]), gemm_weights(wu, types[1]))
        call("lmoe_grouped_gate_up_f16w", ptr(x), _lib.F16, T, topk, ptr(G.order), ptr(G.offsets), ptr(G.tiles),
             ptr(G.n_tiles), G.max_tiles, G.bm, ptr(wg16), ptr(wu16), E, H, I, ptr(h), stream())
    return h


def down(h, G, wd, t, y, ws=None, ksplit=None, w16=None, sl=None):
    """y [R, H] (f16 / f32, grouped order, natural columns) = h . wd over the grouping G; h as gate_up leaves it.
    sl: wd in the stream layout (stream_copy) to read instead, same results bit for bit."""
    E, H = wd.shape[0], wd.shape[1]
    I = h.shape[1]
    if t in _lib.Q4_TYPES:
        ks = ksplit or (pick_ksplit(G.R, G.E, G.bm, I) if t == "Q4_0" and sl is None else 1)
        w = _ws(ks * G.R * H if ks > 1 else 0, ws, h.device)
        call("lmoe_grouped_down_sl" if sl is not None else "lmoe_grouped_down_bm", ptr(h), G.R, ptr(G.offsets),
             ptr(G.tiles), ptr(G.n_tiles), G.max_tiles, G.bm, ks, ptr(w), ptr(sl if sl is not None else wd), qcode(t),
             E, I, H, ptr(y), dcode(y.dtype), stream())
    else:
        if G.bm not in (64, tile_rows()):
            raise ValueError(f"the f16-weight GEMMs take 64- or {tile_rows()}-row tiles, not {G.bm}")
        wd16 = w16 if w16 is not None else gemm_weights(wd, t)
        call("lmoe_grouped_down_f16w", ptr(h), ptr(G.offsets), ptr(G.tiles), ptr(G.n_tiles), G.max_tiles, G.bm,
             ptr(wd16), E, I, H, ptr(y), dcode(y.dtype), stream())
    return y


def expert_rows(x, w, host, types, out_dtype):
    """Every row's expert output, unweighted, in the caller's row order: x [R, H], host [R] slot a row (device or
    host ints), w = (wg, wu, wd) uint8 experts [S, rows, row bytes]. Rows whose slot is outside 0..S-1 come out
    zero. The device form of gguf_experts.dense (gguf_experts.py:698-722)."""
    wg, wu, wd = w
    R, H = x.shape
    E, I = wg.shape[0], wg.shape[1]
    dev = x.device
    ids = torch.as_tensor(host).reshape(-1).to(device=dev, dtype=torch.int32)
    G = Grouping(R, E, dev, bm=pick_tile_rows(R, E, types)).run(ids)
    h = torch.empty((R, I), dtype=torch.float16, device=dev)
    # the down GEMM's f32 result goes to out_dtype with one rounding: an f16 y only when out is f16 itself
    y = torch.empty((R, H), dtype=torch.float16 if out_dtype == torch.float16 else torch.float32, device=dev)
    gate_up(x.contiguous(), G, 1, wg, wu, types, h)
    down(h, G, wd, types[2], y)
    out = torch.empty((R, H), dtype=out_dtype, device=dev)
    call("lmoe_combine_sorted", ptr(y), dcode(y.dtype), ptr(G.inv), None, R, 1, H, None, None, 0, None, 0, ptr(out),
         dcode(out_dtype), stream())
    bad = (ids < 0) | (ids >= E)
    return out.masked_fill_(bad[:, None], 0)


class PrefillBuffers:
    """Every intermediate of a prefill pass of T tokens through layers of one shape, allocated once. y_dtype is the
    dtype of the routed experts' unweighted outputs between the down GEMM and the combine: float16 (the default,
    half the traffic; an output row entry above 65504 in magnitude becomes inf) or float32 (finite wherever the
    layer's output is, the reference dense path's f32 until the output dtype, gguf_experts.py:698-722)."""

    def __init__(self, layer, T, device="cuda", y_dtype=torch.float16):
        if y_dtype not in (torch.float16, torch.float32):
            raise ValueError(f"y_dtype must be float16 or float32, not {y_dtype}")
        L = layer
        self.T = T
        f32 = dict(dtype=torch.float32, device=device)
        self.logits = torch.empty((T, L.E), **f32)
        self.gate = torch.empty(T, **f32) if L.shared is not None else None   # the shared expert's gate logit
        # candidates a token the exact pick recomputed in the decode router's order (lmoe_router_gemm_refine)
        self.n_cand = torch.zeros(T, dtype=torch.int32, device=device)
        self.rws = None
        if L.wr is not None:
            nrw = _lib.lib().lmoe_router_gemm_workspace_bytes(T, L.H, L.E + (1 if L.shared is not None else 0))
            self.rws = torch.empty(max(nrw // 4, 1), **f32)
        # a folded shared expert (MoELayer.folded, m slices) rides in the routed GEMMs as experts E .. E + m - 1,
        # slots k .. k + m - 1 of every token, when the router weight gives its gate logit
        self.fold = L.folded is not None and L.wr is not None
        ks, ne = (L.k + L.n_shared, L.E + L.n_shared) if self.fold else (L.k, L.E)
        R = T * ks
        self.ids_ext = torch.empty((T, ks), dtype=torch.int32, device=device)
        self.scores_ext = torch.empty((T, ks), **f32)
        self.ids, self.scores = self.ids_ext[:, :L.k], self.scores_ext[:, :L.k]  # the routed picks
        self.G = Grouping(R, ne, device, bm=pick_tile_rows(R, ne, L.types))
        nws = splitk_floats(R, ne, self.G.bm, L.H, L.I)
        self.ws = torch.empty(nws, **f32) if nws else None
        self.xh = torch.empty((T, L.H), dtype=torch.float16, device=device)
        self.h = torch.empty((R, L.I), dtype=torch.float16, device=device)
        self.y = torch.empty((R, L.H), dtype=y_dtype, device=device)
        if L.shared is not None and not self.fold:
            self.Gs = Grouping.identity(T, device, bm=pick_tile_rows(T, 1, L.types))
            self.hs = torch.empty((T, L.Is), dtype=torch.float16, device=device)
            self.ys = torch.empty((T, L.H), **f32)
            # the shared expert runs on a second stream (default priority) beside the routed experts: its dense
            # GEMMs fill the units the routed, weight-streaming ones leave idle
            self.side = torch.cuda.Stream(device=device)
            self.x_ready = torch.cuda.Event()
            self.shared_done = torch.cuda.Event()


def prefill(layer, x, bufs, out, residual=None, logits=None):
    """out [T, H] = layer(x) (+ residual) for x [T, H] through the grouped path: x once to f16 in the GEMM K order,
    router logits (given, or lmoe_router_gemm on that x), top-k, device grouping, grouped gate/up + SwiGLU, grouped
    down, [the shared expert on the same kernels, on a side stream that joins before the combine], weighted
    combine (+ sigmoid-gated shared) (+ residual). No host synchronisation and no allocation."""
    L, B = layer, bufs
    T, H = x.shape
    st = stream()
    x = x.contiguous()
    # with the logits given and no shared expert, the top-k and x's conversion go out as one launch
    # (LMOE_FUSED_TOPK=0: two)
    fused = logits is not None and L.shared is None and os.environ.get("LMOE_FUSED_TOPK", "1") != "0"
    ranked = fused  # ids / scores already out of the launch that made them
    if not fused:
        call("lmoe_to_gemm_f16", ptr(x), dcode(x.dtype), x.numel(), ptr(B.xh), st)
    if logits is None:
        if L.wr is None:
            raise ValueError("this layer has no router weight: pass logits")
        ng = 1 if L.shared is not None else 0
        # the router GEMM, then its picks made exact: the candidates its error bound leaves are recomputed in the
        # decode router's fixed order, so the ids are the top-k of the decode router's logits on the same x
        norms = L.router_norms()
        call("lmoe_router_gemm_refine", ptr(B.xh), T, H, ptr(L.router_gemm_weight()), L.E, ng, ptr(B.rws), ptr(x),
             dcode(x.dtype), ptr(L.wr), ptr(L._router_wsg), dcode(L.wr.dtype), ptr(norms), L.k, int(L.norm),
             L.n_shared if B.fold else 0, ptr(B.ids_ext), ptr(B.scores_ext), ptr(B.logits),
             ptr(B.gate) if ng else None, ptr(B.n_cand), st)
        ranked = True
        lg = B.logits
    else:
        if L.shared is not None:
            raise ValueError("a shared expert's gate logit comes from the router: use the router weight")
        if logits.dtype != torch.float32 or not logits.is_contiguous() or tuple(logits.shape) != (T, L.E):
            raise ValueError(f"logits must be float32 [{T}, {L.E}] and contiguous")
        lg = logits
    if B.fold:  # the shared expert's slices as experts E .. E + m - 1 in the routed GEMMs: no side stream
        m = L.n_shared
        ks = L.k + m
        if not ranked:
            call("lmoe_router_topk_shared", ptr(lg), T, L.E, L.k, int(L.norm), ptr(B.gate), m, ptr(B.ids_ext),
                 ptr(B.scores_ext), st)
        B.G.run(B.ids_ext.reshape(-1))
        fs = L.folded_stream or (None, None, None)
        sl_ok = lambda t: t == "Q4_0" or B.G.bm == 64  # noqa: E731
        fg, fu, fd = L.folded
        gate_up(B.xh, B.G, ks, fg, fu, L.types, B.h, prepped=True, ws=B.ws,
                sl=fs[:2] if fs[0] is not None and sl_ok(L.types[0]) else None)
        down(B.h, B.G, fd, L.types[2], B.y, ws=B.ws, sl=fs[2] if sl_ok(L.types[2]) else None)
        call("lmoe_combine_sorted", ptr(B.y), dcode(B.y.dtype), ptr(B.G.inv), ptr(B.scores_ext), T, ks, H, None,
             None, 0, ptr(residual), dcode(residual.dtype) if residual is not None else 0, ptr(out), dcode(out.dtype),
             st)
        return out
    shared = gate = None
    if L.shared is not None:  # x is ready: the shared expert starts on the side stream
        main = torch.cuda.current_stream()
        B.x_ready.record(main)
        B.side.wait_event(B.x_ready)
        with torch.cuda.stream(B.side):
            sg, su, sd = L.shared
            ss = L.shared_stream or (None, None, None)
            s_ok = lambda t: t == "Q4_0" or B.Gs.bm == 64  # noqa: E731
            gate_up(B.xh, B.Gs, 1, sg, su, L.types, B.hs, prepped=True,
                    sl=ss[:2] if ss[0] is not None and s_ok(L.types[0]) else None)
            down(B.hs, B.Gs, sd, L.types[2], B.ys, sl=ss[2] if s_ok(L.types[2]) else None)
            B.shared_done.record(B.side)
        shared, gate = ptr(B.ys), ptr(B.gate)
    if fused:
        call("lmoe_topk_and_gemm_f16", ptr(lg), _lib.F32, T, L.E, L.k, int(L.norm), ptr(B.ids_ext), ptr(B.scores_ext),
             ptr(x), dcode(x.dtype), x.numel(), ptr(B.xh), st)
    elif not ranked:
        call("lmoe_router_topk", ptr(lg), _lib.F32, T, L.E, L.k, int(L.norm), ptr(B.ids_ext), ptr(B.scores_ext),
             st)
    B.G.run(B.ids_ext.reshape(-1))
    f16, sl = L.prefill_f16, L.stream_w or (None, None, None)
    sl_ok = lambda t: t == "Q4_0" or B.G.bm == 64  # noqa: E731  (stream-layout Q4_K: the 64-row kernel)
    gate_up(B.xh, B.G, L.k, L.wg, L.wu, L.types, B.h, prepped=True, ws=B.ws,
            w16=f16[:2] if f16 and f16[0] is not None else None,
            sl=sl[:2] if sl[0] is not None and sl_ok(L.types[0]) else None)
    down(B.h, B.G, L.wd, L.types[2], B.y, ws=B.ws, w16=f16[2] if f16 else None,
         sl=sl[2] if sl_ok(L.types[2]) else None)
    if L.shared is not None:
        torch.cuda.current_stream().wait_event(B.shared_done)
    call("lmoe_combine_sorted", ptr(B.y), dcode(B.y.dtype), ptr(B.G.inv), ptr(B.scores_ext), T, L.k, H, shared, gate,
         1 if shared is not None else 0, ptr(residual), dcode(residual.dtype) if residual is not None else 0,
         ptr(out), dcode(out.dtype), st)
    return out



class PrefillStack:
    """A chunk of T tokens through a stack of MoE layers of one shape, layer-major: x -> x + layer_l(x) for l = 0 ..
    L-1, each layer's whole chunk on the device (router GEMM, top-k, grouping, grouped GEMMs, combine with the
    residual fused) and no host synchronisation between layers.

    The reference's layer-major prefill (stream_fast.py:5058-5210, _call_resident) schedules each layer's experts as
    units through a ring of GPU slots, on the host, because its experts stream from SSD into a small arena. With
    the model's experts resident in HBM (288 GB holds the 48-layer stack's 16 GB many times over) a layer is one
    pass over its grouped rows, and the host only queues launches."""

    def __init__(self, layers, T, dtype=torch.bfloat16, device="cuda"):
        if any(L.wr is None for L in layers):
            raise ValueError("PrefillStack: every layer needs its router weight")
        self.layers = layers
        self.T = T
        self.bufs = PrefillBuffers(layers[0], T, device)
        H = layers[0].H
        self.ping = torch.empty((T, H), dtype=dtype, device=device)
        self.pong = torch.empty((T, H), dtype=dtype, device=device)

    def run(self, x, keep=False):
        """The stack's output for x [T, H] (a view of ping or pong). keep: also return every layer's input and router
        logits (copies), for checking a layer at a time."""
        cur = x
        trace = []
        for i, L in enumerate(self.layers):
            nxt = self.ping if i % 2 == 0 else self.pong
            prefill(L, cur, self.bufs, nxt, residual=cur)
            if keep:
                trace.append((cur.clone(), self.bufs.logits.clone()))
            cur = nxt
        return (cur, trace) if keep else cur
