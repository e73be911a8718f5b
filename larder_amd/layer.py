"""One routed-expert MoE layer on MI355X, and a stack of them for batch-1 decode.

The layer is the reference block's sequence (stream_fast.py:4352-4377 over gguf_experts.experts,
gguf_experts.py:803-819): router logits x . Wr, softmax top-k, the k experts' SwiGLU chains read straight from
GGUF blocks, the weighted combine, and a sigmoid-gated shared expert when the model has one. Two drivers:

  * decode (T <= 16 tokens): router GEMV (which also writes x prepared for the expert kernels) -> top-k fused
    into gate/up + SwiGLU on the picked experts (writing h prepared for down) [-> the shared expert's gate/up and
    down] -> down + weighted combine + shared expert + residual in one kernel; 3 launches a layer without a shared
    expert, no host synchronisation, every buffer preallocated so a whole step can be captured in a HIP graph. A
    layer with a projection beyond Q4_0 / Q4_K passes h as fp32 to the general down (decode_general);
  * prefill / batched decode (any T): the device grouping and the grouped MFMA GEMMs (larder_amd.grouped).
"""
import ctypes
import os

import torch

from . import _lib
from ._lib import call, dcode, ptr, qcode, stream

# Where a decode layer ranks its router logits. False (the default): inside gate/up, one rank a workgroup (the router
# GEMV keeps one router row a workgroup, its widest form). True: in the router kernel's last workgroup
# (lmoe_router_gemv_rank), which needs fewer, wider router workgroups; measured on cfg2 in a HIP graph it is the
# slower of the two (17.1 against 15.7 us a layer), so it stays off.
RANKED_ROUTER = False
RANK_MAX_E, RANK_MAX_K = 512, 16  # the router-and-rank kernel's limits


class MoELayer:
    """A layer's weights (all on the GPU):

    wg, wu   uint8 [E, I, H / bw * bb]      routed experts' gate and up, ggml type types[0] / types[1]
    wd       uint8 [E, H, I / bw * bb]      routed experts' down, ggml type types[2]
    wr       [E, H] float16 / bfloat16 / float32 router weight (None: logits are given to the call)
    shared   (sg, su, sd) uint8 [1, Is, .], [1, Is, .], [1, H, .] shared expert, same types, or None
    wsg      [H] shared-expert gate weight, wr's dtype, or None
    """

    def __init__(self, wg, wu, wd, types, top_k, norm, wr=None, shared=None, wsg=None, fold_shared=True):
        self.types = tuple(types)
        for t in self.types:
            qcode(t)
        self.E, self.I = wg.shape[0], wg.shape[1]
        self.H = wd.shape[1]
        self.k, self.norm = int(top_k), bool(norm)
        self.wr, self.wsg = wr, wsg
        self.shared = shared
        self.Is = shared[0].shape[1] if shared is not None else 0
        if shared is not None and wsg is None:
            raise ValueError("a shared expert needs its gate weight wsg")
        # A shared expert m times the routed width (m >= 1), with a router weight, rides in the decode kernels as m
        # experts E .. E + m - 1 of extended buffers [E + m, ...] (lmoe_moe_gate_up_ext): slice j is its intermediate
        # features [j I, (j + 1) I), i.e. gate / up rows j I .. and down columns j I .. (whole GGUF blocks, since I is
        # a multiple of the block length), and the m slices' down outputs, each weighted by the gate's sigmoid, add
        # up to the gated shared row. Three launches a layer instead of five. The routed buffers are then views of
        # the extended ones (no second copy of them).
        self.folded, self.n_shared = None, 0
        m = self.Is // self.I if shared is not None and self.Is % self.I == 0 else 0
        if (fold_shared and m >= 1 and wr is not None and self.k + m <= 64
                and self.types[0] == self.types[1] and self.H in (2048, 4096) and self.I % 2 == 0
                and shared[2].shape[1] == wd.shape[1] and shared[2].shape[2] == m * wd.shape[2]):
            sg, su, sd = shared
            slices = (sg.reshape(m, self.I, sg.shape[2]), su.reshape(m, self.I, su.shape[2]),
                      sd.reshape(self.H, m, wd.shape[2]).permute(1, 0, 2))
            self.folded = tuple(torch.cat([w, sw], 0).contiguous() for w, sw in zip((wg, wu, wd), slices))
            self.n_shared = m
            wg, wu, wd = (f[:self.E] for f in self.folded)
        self.wg, self.wu, self.wd = wg, wu, wd
        self.prefill_f16 = None
        self.stream_w = None
        self.shared_stream = None
        self.folded_stream = None
        self._router_k = None
        self._router_norms = None
        self._router_wsg = None

    def router_gemm_weight(self):
        """The router weight, with the shared expert's gate row after it when there is a shared expert, as float16
        [E (+ 1), H] in the grouped GEMMs' K order: the weight operand of the prefill router (lmoe_router_gemm),
        converted on the first call and kept (f16 and bf16 weights convert exactly)."""
        if self._router_k is None:
            if self.wr is None:
                raise ValueError("this layer has no router weight")
            n = self.E + (1 if self.shared is not None else 0)
            w = torch.empty((n, self.H), dtype=torch.float16, device=self.wr.device)
            wr = self.wr.contiguous()
            call("lmoe_to_gemm_f16", ptr(wr), dcode(wr.dtype), self.E * self.H, ptr(w), stream())
            if self.shared is not None:
                sg = self.wsg.contiguous()
                call("lmoe_to_gemm_f16", ptr(sg), dcode(sg.dtype), self.H, ptr(w[self.E]), stream())
            self._router_k = w
        return self._router_k

    def router_norms(self):
        """float32 [E (+ 1)][4] norms of the router rows (and the shared gate row) as the prefill router's exact picks
        need them (lmoe_router_norms: |f16(w)|, |w|, |f16(w) - w|, |f16(w) restricted to f16 subnormals|), computed
        on the first call and kept."""
        if self._router_norms is None:
            if self.wr is None:
                raise ValueError("this layer has no router weight")
            n = self.E + (1 if self.shared is not None else 0)
            out = torch.empty((n, 4), dtype=torch.float32, device=self.wr.device)
            wr = self.wr.contiguous()
            wsg = self.wsg.contiguous() if self.shared is not None else None
            if wsg is not None and wsg.dtype != wr.dtype:
                wsg = wsg.to(wr.dtype)
            self._router_wsg = wsg
            call("lmoe_router_norms", ptr(wr), ptr(wsg), dcode(wr.dtype), self.E, self.H, ptr(out), stream())
            self._router_norms = out
        return self._router_norms

    def keep_prefill_f16(self):
        """Hold the f16 K-order weights the grouped path needs for projections beyond Q4_0 / Q4_K (gate/up together,
        down alone) resident, so prefill does not dequantize them each call: 2 bytes a weight beside the packed
        ones, a trade the 288 GB of HBM affords. Returns the bytes held."""
        from . import grouped
        gu = None
        if not (self.types[0] in _lib.Q4_TYPES and self.types[1] == self.types[0]):
            gu = (grouped.gemm_weights(self.wg, self.types[0]), grouped.gemm_weights(self.wu, self.types[1]))
        dn = grouped.gemm_weights(self.wd, self.types[2]) if self.types[2] not in _lib.Q4_TYPES else None
        self.prefill_f16 = (gu[0] if gu else None, gu[1] if gu else None, dn)
        return sum(t.numel() * 2 for t in self.prefill_f16 if t is not None)

    def keep_stream(self):
        """Hold stream-layout copies (grouped.stream_copy) of the Q4_0 / Q4_K projections for the grouped path: each
        GEMM step then reads one contiguous run a block of 128 features (cfg5 prefill's gate/up 434 -> 342 us in a
        probe with that access pattern). The copies double those projections' bytes in HBM; the decode kernels keep
        the GGUF copies. Gate/up get theirs together (the kernels take one type for both), down alone, and the shared
        expert's likewise; a projection that has no stream layout keeps None. Returns the bytes held."""
        from . import grouped
        tg, tu, td = self.types
        # a folded layer's copies cover its extended buffers (the shared slices too); the routed ones are prefixes
        src = self.folded if self.folded is not None else (self.wg, self.wu, self.wd)
        gu = None
        if tg == tu and tg in _lib.Q4_TYPES and self.I % 128 == 0:
            gu = (grouped.stream_copy(src[0], tg), grouped.stream_copy(src[1], tu))
        dn = grouped.stream_copy(src[2], td) if td in _lib.Q4_TYPES and self.H % 128 == 0 else None
        full = (gu[0] if gu else None, gu[1] if gu else None, dn)
        held = [t for t in full if t is not None]
        if self.folded is not None:
            self.folded_stream = full
            full = tuple(t[:self.E] if t is not None else None for t in full)
        self.stream_w = full
        if self.shared is not None and self.folded is None:  # the shared expert's GEMMs on the same kernels
            sg, su, sd = self.shared
            sgu = ((grouped.stream_copy(sg, tg), grouped.stream_copy(su, tu))
                   if tg == tu and tg in _lib.Q4_TYPES and self.Is % 128 == 0 else None)
            sdn = grouped.stream_copy(sd, td) if td in _lib.Q4_TYPES and self.H % 128 == 0 else None
            self.shared_stream = (sgu[0] if sgu else None, sgu[1] if sgu else None, sdn)
            held += [t for t in self.shared_stream if t is not None]
        return sum(t.numel() for t in held)

    def drop_stream(self):
        """Release the stream-layout copies: the grouped path reads the GGUF blocks as stored again."""
        self.stream_w = self.folded_stream = self.shared_stream = None

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
        u32 = dict(dtype=torch.int32, device=device)
        self.logits = torch.empty((T, rows), **f32)
        ks = L.k + L.n_shared  # slots a token (the folded shared expert's slices last)
        self.ids_ext = torch.empty((T, ks), **u32)
        self.scores_ext = torch.empty((T, ks), **f32)
        self.ids, self.scores = self.ids_ext[:, :L.k], self.scores_ext[:, :L.k]
        # the router-and-rank kernel's arrival counter (zero between launches; one a stream)
        self.sync = torch.zeros(1, **u32)
        # prepared rows (36 dwords a 64-value unit): x for the gate / up type, h for the down type
        self.xprep = torch.empty((T, L.H // 64 * 36), **u32)
        self.xprep_u = torch.empty((T, L.H // 64 * 36), **u32) if L.types[1] != L.types[0] else None
        self.hprep = torch.empty((T * ks, L.I // 64 * 36), **u32)
        if L.shared is not None and L.folded is None:
            self.zero_slots = torch.zeros(T, **u32)
            self.hprep_s = torch.empty((T, L.Is // 64 * 36), **u32)
            self.shared_y = torch.empty((T, L.H), **f32)
        # a layer off the prepared chain (a projection beyond Q4_0 / Q4_K) passes h between gate/up and down as fp32
        self.h32 = self.h32_s = None
        if not prepared_chain(L):
            self.h32 = torch.empty((T * ks, L.I), **f32)
            if L.shared is not None and L.folded is None:
                self.h32_s = torch.empty((T, L.Is), **f32)


def prepared_chain(layer):
    """Whether ``layer`` decodes on the prepared chain (h passed prepared from gate/up to down): every projection
    Q4_0 / Q4_K, or a Q6_K down (the 35B's mix) or a Q8_0 down under gate and up of one Q4 type in the
    register-resident form (hidden 2048 or 4096), whose kernels read h prepared in the Q4_K / Q4_0 order. Other
    layers take decode_general."""
    t = layer.types
    if all(x in _lib.Q4_TYPES for x in t):
        return True
    return (t[2] in ("Q6_K", "Q8_0") and t[0] == t[1] and t[0] in _lib.Q4_TYPES and layer.H in (2048, 4096)
            and layer.I % 64 == 0)


def decode_general(layer, x, bufs, out, residual=None, logits=None):
    """decode() for a layer with a projection beyond Q4_0 / Q4_K, such as the 35B's Q4_K / Q4_K / Q6_K (the
    reference runs every type through gguf_experts.gemv's chain, gguf_experts.py:600-653, with f32 h):
      * when gate and up share one Q4 type at hidden 2048 or 4096: the router GEMV (x prepared), then gate/up +
        SwiGLU with the top-k fused in (lmoe_moe_gate_up_h: ids / scores with a folded shared expert's slots, h as
        fp32), as the prepared chain does;
      * otherwise the router GEMV ranks in its last workgroup (lmoe_router_gemv_rank), or lmoe_router_topk takes
        given logits, and gate/up + SwiGLU run from raw x (lmoe_gemv_gate_up) into fp32 h;
      * [an unfolded shared expert's gate/up and down into an fp32 row;]
      * the general down + weighted combine + shared + residual (lmoe_gemv_down_combine; Q6_K on its packed-f16
        kernel).
    Three launches a layer (five with an unfolded shared expert), all preallocated, so a stack still captures as
    one HIP graph."""
    L, B = layer, bufs
    T = x.shape[0]
    st = stream()
    tg, tu, td = (qcode(t) for t in L.types)
    xd = dcode(x.dtype)
    ks = L.k + L.n_shared
    xr = L.types[0] == L.types[1] and L.types[0] in _lib.Q4_TYPES and L.H in (2048, 4096) and L.I % 2 == 0
    if logits is not None and L.shared is not None:
        raise ValueError("a shared expert's gate logit comes from the router GEMV: use the router weight")
    if logits is None and L.wr is None:
        raise ValueError("this layer has no router weight: pass logits")
    wg, wu, wd = L.folded if L.folded is not None else (L.wg, L.wu, L.wd)
    ne = L.E + L.n_shared
    if xr:  # the prepared chain's router and fused top-k, h out as fp32
        if logits is None:
            call("lmoe_router_gemv", ptr(x), xd, ptr(L.wr), ptr(L.wsg), dcode(L.wr.dtype), T, L.H, L.E,
                 ptr(B.logits), ptr(B.xprep), tg, st)
            lg, stride = B.logits, B.logits.shape[1]
        else:
            lg, stride = logits.to(torch.float32).contiguous(), L.E
            call("lmoe_prep_x", ptr(x), xd, T, L.H, tg, ptr(B.xprep), st)
        call("lmoe_moe_gate_up_h", ptr(lg), stride, T, L.k, int(L.norm), ptr(B.xprep), ptr(wg), ptr(wu), tg, L.E,
             L.H, L.I, ptr(B.ids_ext), ptr(B.scores_ext), ptr(B.h32), L.n_shared, st)
    elif logits is None:
        if L.E > RANK_MAX_E or L.k > RANK_MAX_K:
            raise ValueError(f"decode takes at most {RANK_MAX_E} experts and top-{RANK_MAX_K} when gate/up are "
                             f"beyond Q4_0 / Q4_K (got {L.E}, top-{L.k})")
        call("lmoe_router_gemv_rank", ptr(x), xd, ptr(L.wr), ptr(L.wsg), dcode(L.wr.dtype), T, L.H, L.E, L.k,
             int(L.norm), ks, ptr(B.logits), ptr(B.ids_ext), ptr(B.scores_ext), None, tg, ptr(B.sync), st)
    else:
        lg = logits.to(torch.float32).contiguous()
        call("lmoe_router_topk", ptr(lg), _lib.F32, T, L.E, L.k, int(L.norm), ptr(B.ids_ext), ptr(B.scores_ext), st)

    def gate_up(slots, n, topk, g, u, n_exp, width, h):
        if xr:
            call("lmoe_gemv_gate_up_prepped", ptr(B.xprep), ptr(B.xprep), ptr(slots), n, topk, ptr(g), ptr(u), tg,
                 tu, n_exp, L.H, width, ptr(h), None, 0, st)
        else:
            call("lmoe_gemv_gate_up", ptr(x), xd, ptr(slots), n, topk, ptr(g), ptr(u), tg, tu, n_exp, L.H, width,
                 ptr(h), st)

    if not xr:
        gate_up(B.ids_ext, T * ks, ks, wg, wu, ne, L.I, B.h32)
    shared_y = gptr = None
    gate_stride = 0
    if L.shared is not None and L.folded is None:
        sg, su, sd = L.shared
        gate_up(B.zero_slots, T, 1, sg, su, 1, L.Is, B.h32_s)
        call("lmoe_gemv_down_combine", ptr(B.h32_s), ptr(B.zero_slots), None, T, 1, ptr(sd), td, 1, L.Is, L.H, None,
             None, 0, None, 0, ptr(B.shared_y), _lib.F32, st)
        shared_y = B.shared_y
        gptr, gate_stride = _ptr_offset(B.logits, L.E), L.E + 1
    call("lmoe_gemv_down_combine", ptr(B.h32), ptr(B.ids_ext), ptr(B.scores_ext), T, ks, ptr(wd), td, ne, L.I, L.H,
         ptr(shared_y), gptr, gate_stride, ptr(residual), dcode(residual.dtype) if residual is not None else 0,
         ptr(out), dcode(out.dtype), st)
    return out


def decode(layer, x, bufs, out, residual=None, logits=None):
    """out [T, H] = layer(x) (+ residual) for x [T, H] (float16 / bfloat16 / float32) through the decode chain:
    router GEMV (+ x prepared for the experts) and top-k, gate/up + SwiGLU (writing h prepared for down),
    [the shared expert's gate/up and down], then down + weighted combine + shared + residual. ``logits`` [T, E]
    replaces the router GEMV when the layer has no router weight. A layer with a projection beyond Q4_0 / Q4_K
    goes through decode_general."""
    L, B = layer, bufs
    if not prepared_chain(L):
        return decode_general(L, x, B, out, residual, logits)
    T = x.shape[0]
    st = stream()
    tg, tu, td = (qcode(t) for t in L.types)
    xd = dcode(x.dtype)
    ranked = False
    if logits is None:
        if L.wr is None:
            raise ValueError("this layer has no router weight: pass logits")
        if RANKED_ROUTER and L.E <= RANK_MAX_E and L.k <= RANK_MAX_K:
            # router GEMV and top-k in one launch: ids / scores (with the folded shared expert's slot) come out of it
            call("lmoe_router_gemv_rank", ptr(x), xd, ptr(L.wr), ptr(L.wsg), dcode(L.wr.dtype), T, L.H, L.E, L.k,
                 int(L.norm), B.ids_ext.shape[1], ptr(B.logits), ptr(B.ids_ext), ptr(B.scores_ext), ptr(B.xprep), tg,
                 ptr(B.sync), st)
            ranked = True
        else:
            call("lmoe_router_gemv", ptr(x), xd, ptr(L.wr), ptr(L.wsg), dcode(L.wr.dtype), T, L.H, L.E,
                 ptr(B.logits), ptr(B.xprep), tg, st)
        lg, stride = B.logits, B.logits.shape[1]
    else:
        if L.shared is not None:
            raise ValueError("a shared expert's gate logit comes from the router GEMV: use the router weight")
        lg, stride = logits.to(torch.float32).contiguous(), L.E
        call("lmoe_prep_x", ptr(x), xd, T, L.H, tg, ptr(B.xprep), st)
    xu = B.xprep
    if B.xprep_u is not None:
        call("lmoe_prep_x", ptr(x), xd, T, L.H, tu, ptr(B.xprep_u), st)
        xu = B.xprep_u
    if L.folded is not None:  # the shared expert's m slices as slots k .. k + m - 1: gate/up, then down + combine
        fg, fu, fd = L.folded
        ks = L.k + L.n_shared
        if ranked:
            call("lmoe_gemv_gate_up_prepped", ptr(B.xprep), ptr(xu), ptr(B.ids_ext), T * ks, ks,
                 ptr(fg), ptr(fu), tg, tu, L.E + L.n_shared, L.H, L.I, None, ptr(B.hprep), td, st)
        else:
            call("lmoe_moe_gate_up_ext", ptr(lg), stride, T, L.k, int(L.norm), ptr(B.xprep), ptr(xu), ptr(fg),
                 ptr(fu), tg, tu, L.E, L.H, L.I, ptr(B.ids_ext), ptr(B.scores_ext), ptr(B.hprep), td, L.n_shared,
                 st)
        call("lmoe_gemv_down_combine_prepped", ptr(B.hprep), 0, ptr(B.ids_ext), ptr(B.scores_ext), T, ks,
             ptr(fd), td, L.E + L.n_shared, L.I, L.H, None, None, 0, ptr(residual),
             dcode(residual.dtype) if residual is not None else 0, ptr(out), dcode(out.dtype), st)
        return out
    if ranked:
        call("lmoe_gemv_gate_up_prepped", ptr(B.xprep), ptr(xu), ptr(B.ids_ext), T * L.k, L.k, ptr(L.wg),
             ptr(L.wu), tg, tu, L.E, L.H, L.I, None, ptr(B.hprep), td, st)
    else:
        call("lmoe_moe_gate_up", ptr(lg), stride, T, L.k, int(L.norm), ptr(B.xprep), ptr(xu), ptr(L.wg), ptr(L.wu),
             tg, tu, L.E, L.H, L.I, ptr(B.ids), ptr(B.scores), ptr(B.hprep), td, st)
    shared_y = gptr = None
    gate_stride = 0
    if L.shared is not None:
        sg, su, sd = L.shared
        call("lmoe_gemv_gate_up_prepped", ptr(B.xprep), ptr(xu), ptr(B.zero_slots), T, 1, ptr(sg), ptr(su), tg, tu,
             1, L.H, L.Is, None, ptr(B.hprep_s), td, st)
        call("lmoe_gemv_down_combine_prepped", ptr(B.hprep_s), 0, ptr(B.zero_slots), None, T, 1, ptr(sd), td, 1,
             L.Is, L.H, None, None, 0, None, 0, ptr(B.shared_y), _lib.F32, st)
        shared_y = B.shared_y
        gptr, gate_stride = _ptr_offset(B.logits, L.E), L.E + 1
    call("lmoe_gemv_down_combine_prepped", ptr(B.hprep), 0, ptr(B.ids), ptr(B.scores), T, L.k, ptr(L.wd), td, L.E,
         L.I, L.H, ptr(shared_y), gptr, gate_stride, ptr(residual),
         dcode(residual.dtype) if residual is not None else 0, ptr(out), dcode(out.dtype), st)
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
