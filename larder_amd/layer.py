"""One routed-expert MoE layer on MI355X, and a stack of them for batch-1 decode.

The layer is the reference block's sequence (stream_fast.py:4352-4377 over gguf_experts.experts,
gguf_experts.py:803-819): router logits x . Wr, softmax top-k, the k experts' SwiGLU chains read straight from
GGUF blocks, the weighted combine, and a sigmoid-gated shared expert when the model has one. Two drivers:

  * decode (T <= 16 tokens): lmoe_router_gemv_topk -> lmoe_gemv_gate_up [-> shared expert gate/up + down]
    -> lmoe_gemv_down_combine (down, weighted combine, shared expert, residual in one kernel); 3 launches a layer
    without a shared expert, no host synchronisation, every buffer preallocated so a whole step can be captured
    in a HIP graph;
  * prefill / batched decode (any T): the device grouping and the grouped MFMA GEMMs (larder_amd.grouped).
"""
import ctypes

import torch

from . import _lib
from ._lib import call, dcode, ptr, qcode, stream


class MoELayer:
    """A layer's weights (all on the GPU):

    wg, wu   uint8 [E, I, H / bw * bb]      routed experts' gate and up, ggml type types[0] / types[1]
    wd       uint8 [E, H, I / bw * bb]      routed experts' down, ggml type types[2]
    wr       [E, H] float16 / bfloat16 / float32 router weight (None: logits are given to the call)
    shared   (sg, su, sd) uint8 [1, Is, .], [1, Is, .], [1, H, .] shared expert, same types, or None
    wsg      [H] shared-expert gate weight, wr's dtype, or None
    """

    def __init__(self, wg, wu, wd, types, top_k, norm, wr=None, shared=None, wsg=None):
        self.types = tuple(types)
        for t in self.types:
            qcode(t)
        self.wg, self.wu, self.wd = wg, wu, wd
        self.E, self.I = wg.shape[0], wg.shape[1]
        self.H = wd.shape[1]
        self.k, self.norm = int(top_k), bool(norm)
        self.wr, self.wsg = wr, wsg
        self.shared = shared
        self.Is = shared[0].shape[1] if shared is not None else 0
        if shared is not None and wsg is None:
            raise ValueError("a shared expert needs its gate weight wsg")

    def nbytes_touched(self, n_unique):
        """Algorithmic HBM bytes of one decode pass touching n_unique routed experts (weights only)."""
        per = self.wg[0].numel() + self.wu[0].numel() + self.wd[0].numel()
        sh = sum(s.numel() for s in self.shared) if self.shared is not None else 0
        rw = self.wr.numel() * self.wr.element_size() if self.wr is not None else 0
        sg = self.wsg.numel() * self.wsg.element_size() if self.wsg is not None else 0
        return n_unique * per + sh + rw + sg


class DecodeBuffers:
    """Every intermediate of a decode pass of T tokens through layers of one shape, allocated once."""

    def __init__(self, layer, T, device="cuda"):
        if T > 16:
            raise ValueError("the decode driver takes at most 16 tokens a pass; use the grouped path")
        L = layer
        self.T = T
        rows = L.E + (1 if L.shared is not None else 0)
        f32 = dict(dtype=torch.float32, device=device)
        self.ws = torch.zeros(max(64, _lib.lib().lmoe_router_workspace_bytes() // 4), dtype=torch.int32,
                              device=device)
        self.logits = torch.empty((T, rows), **f32)
        self.ids = torch.empty((T, L.k), dtype=torch.int32, device=device)
        self.scores = torch.empty((T, L.k), **f32)
        self.h = torch.empty((T * L.k, L.I), **f32)
        if L.shared is not None:
            self.zero_slots = torch.zeros(T, dtype=torch.int32, device=device)
            self.hs = torch.empty((T, L.Is), **f32)
            self.shared_y = torch.empty((T, L.H), **f32)


def decode(layer, x, bufs, out, residual=None, logits=None):
    """out [T, H] = layer(x) (+ residual) for x [T, H] (float16 / bfloat16 / float32) through the decode chain.
    ``logits`` [T, E] replaces the router GEMV when the layer has no router weight."""
    L, B = layer, bufs
    T = x.shape[0]
    st = stream()
    tg, tu, td = (qcode(t) for t in L.types)
    if logits is None:
        if L.wr is None:
            raise ValueError("this layer has no router weight: pass logits")
        call("lmoe_router_gemv_topk", ptr(x), dcode(x.dtype), ptr(L.wr), ptr(L.wsg), dcode(L.wr.dtype), T, L.H,
             L.E, L.k, int(L.norm), ptr(B.logits), ptr(B.ids), ptr(B.scores), ptr(B.ws), st)
        gate, gate_stride = (B.logits[:, L.E:], L.E + 1) if L.shared is not None else (None, 0)
    else:
        lg = logits.contiguous()
        call("lmoe_router_topk", ptr(lg), dcode(lg.dtype), T, L.E, L.k, int(L.norm), ptr(B.ids), ptr(B.scores), st)
        gate, gate_stride = None, 0
        if L.shared is not None:
            raise ValueError("a shared expert's gate logit comes from the router GEMV: use the router weight")
    call("lmoe_gemv_gate_up", ptr(x), dcode(x.dtype), ptr(B.ids), T * L.k, L.k, ptr(L.wg), ptr(L.wu), tg, tu, L.E,
         L.H, L.I, ptr(B.h), st)
    shared_y = None
    if L.shared is not None:
        sg, su, sd = L.shared
        call("lmoe_gemv_gate_up", ptr(x), dcode(x.dtype), ptr(B.zero_slots), T, 1, ptr(sg), ptr(su), tg, tu, 1, L.H,
             L.Is, ptr(B.hs), st)
        call("lmoe_gemv_down_combine", ptr(B.hs), ptr(B.zero_slots), None, T, 1, ptr(sd), td, 1, L.Is, L.H, None,
             None, 0, None, 0, ptr(B.shared_y), _lib.F32, st)
        shared_y = B.shared_y
    gptr = _ptr_offset(B.logits, L.E) if gate is not None else None
    call("lmoe_gemv_down_combine", ptr(B.h), ptr(B.ids), ptr(B.scores), T, L.k, ptr(L.wd), td, L.E, L.I, L.H,
         ptr(shared_y), gptr, gate_stride, ptr(residual), dcode(residual.dtype) if residual is not None else 0,
         ptr(out), dcode(out.dtype), st)
    return out


def _ptr_offset(t, elems):
    """Device pointer ``elems`` elements into tensor t."""
    return ctypes.c_void_p(t.data_ptr() + elems * t.element_size())


class DecodeStack:
    """A stack of MoE layers of one shape driven at batch T: x -> x + layer_l(x) for l = 0..L-1, the residual add
    fused into each layer's combine. ``step`` runs eagerly; ``capture`` records one step as a HIP graph reading
    ``self.x_in`` and leaving the result in ``self.x_out``."""

    def __init__(self, layers, T, dtype=torch.float16, device="cuda"):
        self.layers = layers
        self.T = T
        self.bufs = DecodeBuffers(layers[0], T, device)
        H = layers[0].H
        self.x_in = torch.zeros((T, H), dtype=dtype, device=device)
        self.ping = torch.empty((T, H), dtype=dtype, device=device)
        self.pong = torch.empty((T, H), dtype=dtype, device=device)
        self.graph = None

    def step(self):
        cur = self.x_in
        for i, L in enumerate(self.layers):
            nxt = self.ping if i % 2 == 0 else self.pong
            decode(L, cur, self.bufs, nxt, residual=cur)
            cur = nxt
        self.x_out = cur
        return cur

    def capture(self):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            self.step()  # warm the allocator-free path once on the capture stream
        torch.cuda.current_stream().wait_stream(s)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self.step()
        self.graph = g
        return g
